"""Host-side logic of the drop-in (CPU only): argument checks, layouts, the module and its gate."""

import numpy as np
import pytest
import torch

import golden_io
from mlx_tree_spec_amd import QuantizedLinear, dequantize, eligible, install, pack_nax, quantized_matmul, unpack_nax
from oracle import qmm4_oracle as O


def tensors(m=4, k=256, n=64, seed=0):
    x, w, s, b = O.make_inputs(m, k, n, seed=seed)
    t = lambda a: torch.from_numpy(a.astype(np.int16) if a.dtype == np.uint16 else a.view(np.int32))
    return (t(x).view(torch.bfloat16), t(w), t(s).view(torch.bfloat16), t(b).view(torch.bfloat16))


def test_no_cpu_path():
    x, w, s, b = tensors()
    with pytest.raises(ValueError, match="HIP device"):
        quantized_matmul(x, w, s, b)
    with pytest.raises(ValueError, match="HIP device"):
        dequantize(w, s, b)


@pytest.mark.parametrize("kw,exc", [(dict(bits=3), NotImplementedError), (dict(bits=6), NotImplementedError),
                                    (dict(group_size=16), NotImplementedError),
                                    (dict(transpose=False), NotImplementedError), (dict(mode="mxfp4"), NotImplementedError)])
def test_format_errors(kw, exc):
    x, w, s, b = tensors()
    with pytest.raises(exc):
        quantized_matmul(x, w, s, b, **kw)


@pytest.mark.parametrize("bits,group_size", [(8, 64), (2, 32), (4, 128)])
def test_general_formats_are_accepted(bits, group_size):
    """2-, 4- and 8-bit codes in groups of 32, 64 or 128 pass the format checks (the general path:
    HIP dequantize, then a bf16 GEMM); on CPU tensors the call then stops at the device check."""
    n, k = 64, 256
    x = torch.zeros((2, k), dtype=torch.bfloat16)
    w = torch.zeros((n, k * bits // 32), dtype=torch.int32)
    s = torch.zeros((n, k // group_size), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        quantized_matmul(x, w, s, s, group_size=group_size, bits=bits)
    with pytest.raises(ValueError, match="HIP device"):
        dequantize(w, s, s, group_size=group_size, bits=bits)
    with pytest.raises(ValueError, match="does not match"):  # weights of another width
        quantized_matmul(x, w, s, s, group_size=group_size, bits=8 if bits == 4 else 4)


def test_shape_and_dtype_errors():
    x, w, s, b = tensors()
    with pytest.raises(ValueError, match="does not match"):
        quantized_matmul(x[:, :128], w, s, b)
    with pytest.raises(ValueError, match="bfloat16"):
        quantized_matmul(x.float(), w, s, b)
    with pytest.raises(ValueError, match="scales shape"):
        quantized_matmul(x, w, s[:, :2], b)
    with pytest.raises(ValueError, match="int32/uint32"):
        quantized_matmul(x, w.float(), s, b)
    with pytest.raises(ValueError, match="both scales and biases"):
        quantized_matmul(x, w, s, None)
    # K must be whole groups (x of 96 against weights of 96 codes per row: 12 words, one scale)
    x96 = torch.zeros((2, 96), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="multiple of group_size"):
        quantized_matmul(x96, torch.zeros((16, 12), dtype=torch.int32), s[:16, :1], b[:16, :1])


def test_pack_nax_torch_matches_fixture_and_inverts():
    z = golden_io.load("pack_nax.npz")
    w = torch.from_numpy(z["w"].view(np.int32))
    s = torch.from_numpy(z["s"].astype(np.int16)).view(torch.bfloat16)
    wq2, sp2, bp2 = pack_nax(w, s, s)
    assert np.array_equal(wq2.numpy().view(np.uint32), z["wq2"])
    assert np.array_equal(sp2.view(torch.int16).numpy().view(np.uint16), z["sp2"])
    w2, s2, b2 = unpack_nax(wq2, sp2, bp2, w.shape[0])
    assert torch.equal(w2, w) and torch.equal(s2.view(torch.int16), s.view(torch.int16))
    wu = w.view(torch.uint32)
    wq2u, _, _ = pack_nax(wu, s, s)
    assert wq2u.dtype == torch.uint32 and np.array_equal(wq2u.view(torch.int32).numpy().view(np.uint32), z["wq2"])


def test_quantized_linear_module_and_gate():
    m = QuantizedLinear(256, 64)
    assert m.weight.shape == (64, 32) and m.scales.shape == (64, 4) and m.biases.shape == (64, 4)
    assert m.input_dims == 256 and m.output_dims == 64
    assert eligible(m)
    assert not eligible(QuantizedLinear(256, 48))           # N % 32 != 0
    assert not eligible(QuantizedLinear(192, 64))           # K % 128 != 0
    assert not eligible(QuantizedLinear(256, 64, bias=True))
    assert not eligible(QuantizedLinear(256, 64, group_size=32))  # the kernels implement group 64 only
    b8 = QuantizedLinear(256, 64)
    b8.bits = 8
    assert not eligible(b8)
    assert not eligible(torch.nn.Linear(256, 64))
    x, w, s, b = tensors()
    q = QuantizedLinear.from_quantized(w.view(torch.uint32), s, b)
    assert q.weight.dtype == torch.int32 and eligible(q)


def test_install_requires_device():
    model = torch.nn.Sequential(QuantizedLinear(256, 64), QuantizedLinear(128, 48))
    with pytest.raises(ValueError, match="HIP device"):
        install(model, verbose=False)


@pytest.mark.parametrize("m,k,n,sigma,seed", [(4, 5120, 96, 1.0, 1), (64, 17408, 32, 0.5, 2), (3, 128, 16, 1.0, 0)])
def test_bench_inputs_are_the_pinned_generator(m, k, n, sigma, seed):
    """bench.py draws its workloads with its own generator (the oracle serves only its CPU baseline);
    it must produce the same bits as the oracle's make_inputs, the generator the parity tests and
    the committed fixtures use."""
    import bench

    got = bench.synthetic_inputs(m, k, n, sigma=sigma, seed=seed)
    want = O.make_inputs(m, k, n, sigma=sigma, seed=seed)
    for g, w in zip(got, want):
        assert g.dtype == w.dtype and g.shape == w.shape
        assert np.array_equal(g, w)
