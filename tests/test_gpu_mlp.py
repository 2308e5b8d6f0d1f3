"""The fused gate+up projection with its SiLU·mul epilogue, and the MLP drop-in (needs an MI355X).

Bars:
  * against the GPU's own unfused projection (quantized_matmul of the stacked weight, halves g and u)
    through the oracle's silu_mul: at least 99.9% of outputs bit-equal, every one within one bf16
    ulp (the fp32 exp of the kernel and of numpy may differ in their last bit);
  * against the CPU fp32-accumulated reference composition: max_rel <= 1e-2 and mean_rel <= 2e-3.
"""

import numpy as np
import pytest
import torch

from mlx_tree_spec_amd import STATS, QuantizedLinear, QuantizedMLP, gate_up_silu, quantized_matmul
from oracle import cpu
from oracle import qmm4_oracle as O
from route_cases import GATE_UP_CASES, RANDOM_GATE_UP

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def bf16_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)


def u32_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(DEV)


def host_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def within_one_ulp(a_bits, b_bits):
    a = O.bf16_bits_to_f32(a_bits).astype(np.float64)
    b = O.bf16_bits_to_f32(b_bits).astype(np.float64)
    mag = np.maximum(np.maximum(np.abs(a), np.abs(b)), 2.0 ** -126)
    return np.abs(a - b) <= 2.0 ** (np.floor(np.log2(mag)) - 7)


def check_gate_up(x, w, s, b):
    m, n = x.shape[0], w.shape[0]
    h = n // 2
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(gate_up_silu(xd, wd, sd, bd))
    assert y.shape == (m, h)
    t = host_bits(quantized_matmul(xd, wd, sd, bd))
    ref = O.silu_mul(t[:, :h], t[:, h:])
    eq = float(np.mean(y == ref))
    print(f"  gate_up {m}x{x.shape[1]}x{n}: bit-equal to the unfused composition {eq:.5f}", flush=True)
    assert eq >= 0.999
    assert within_one_ulp(y, ref).all()
    tf = O.f32_to_bf16_bits(cpu.qmm_f32(x, w, s, b))
    cref = O.bf16_bits_to_f32(O.silu_mul(tf[:, :h], tf[:, h:])).astype(np.float64)
    yf = O.bf16_bits_to_f32(y).astype(np.float64)
    assert O.max_rel(yf, cref) <= O.MAX_REL_TOL and O.mean_rel(yf, cref) <= O.MEAN_REL_TOL
    # deterministic
    assert np.array_equal(host_bits(gate_up_silu(xd, wd, sd, bd)), y)
    return y


# One row-split launch with the epilogue fused (up to 16 rows; N = 34848 leaves the last workgroup a
# partial range, K = 4096 gives units of 4 super-steps, 5120 of 5, 9 to 16 rows take 16-row
# fragments with K in slices), or the projection into the library's scratch buffer followed by the
# epilogue pass (x slices too large for LDS at up to 16 rows; the row-phase and GEMM kernels
# underneath at 64 and 100 rows), or one row-phase launch with the epilogue fused (5-96 rows over
# N that gives every CU its own blocks; 33024 leaves the last range 2 + 2 blocks).
# tests/test_plans.py checks each case's route against the planner.
@pytest.mark.parametrize("m,k,n,route", GATE_UP_CASES)
def test_gate_up_silu(m, k, n, route):
    print(f"  gate_up M={m} K={k} N={n} ({route})", flush=True)
    x, w, s, b = O.make_inputs(m, k, n, seed=m + 31 * k + n)
    check_gate_up(x, w, s, b)


@pytest.mark.parametrize("m,k,n", RANDOM_GATE_UP)
def test_gate_up_silu_random_shapes(m, k, n):
    print(f"  gate_up random M={m} K={k} N={n}", flush=True)
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 7919 + k * 31 + n)
    check_gate_up(x, w, s, b)


def test_gate_up_silu_rejects_odd_halves():
    x, w, s, b = O.make_inputs(2, 256, 48, seed=1)
    with pytest.raises(ValueError):
        gate_up_silu(bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b))


def test_gate_up_silu_saturated_and_zero_gates():
    """Gate sums far past the sigmoid's range (+-60: silu = g and 0) and exactly zero (silu = 0):
    scale 1 and bias 0 with codes 15 or 0 make the gate sum an exact multiple of sum(x)."""
    m, k, n = 2, 512, 64
    h = n // 2
    rng = np.random.default_rng(5)
    q = np.zeros((n, k), np.uint8)
    q[:h // 2] = 15              # gate columns 0..15: 15 * sum(x)
    q[h:] = rng.integers(0, 16, size=(h, k))
    w = O.pack_codes(q)
    s = np.full((n, k // 64), O.f32_to_bf16_bits(np.float32(1.0)), np.uint16)
    b = np.zeros((n, k // 64), np.uint16)
    x = np.zeros((m, k), np.uint16)
    x[0, :4] = O.f32_to_bf16_bits(np.float32(1.0))    # row 0: sum 4 -> gate 60
    x[1, :4] = O.f32_to_bf16_bits(np.float32(-1.0))   # row 1: sum -4 -> gate -60
    y = check_gate_up(x, w, s, b)
    yf = O.bf16_bits_to_f32(y)
    assert np.all(yf[:, h // 2:] == 0)  # zero gate (codes 0, bias 0)


def test_quantized_mlp_matches_composition():
    d, hdim, m = 512, 1024, 3
    rng = np.random.default_rng(7)

    def lin(n, k, seed):
        _, w, s, b = O.make_inputs(1, k, n, seed=seed)
        return QuantizedLinear.from_quantized(u32_dev(w), bf16_dev(s), bf16_dev(b)), (w, s, b)

    gate, gw = lin(hdim, d, 1)
    up, uw = lin(hdim, d, 2)
    down, dw = lin(d, hdim, 3)
    mlp = QuantizedMLP(gate, up, down)
    x = O.f32_to_bf16_bits(rng.standard_normal((m, d)).astype(np.float32))
    before = STATS["gate_up_silu"]
    y = host_bits(mlp(bf16_dev(x)))
    assert STATS["gate_up_silu"] == before + 1
    # the same kernels called one by one
    wgu = np.concatenate([gw[0], uw[0]]), np.concatenate([gw[1], uw[1]]), np.concatenate([gw[2], uw[2]])
    hb = gate_up_silu(bf16_dev(x), u32_dev(wgu[0]), bf16_dev(wgu[1]), bf16_dev(wgu[2]))
    y2 = host_bits(quantized_matmul(hb, down.weight, down.scales, down.biases))
    assert np.array_equal(y, y2)
    # against the CPU composition: fp32-accumulated projections, the oracle's epilogue
    t = O.f32_to_bf16_bits(cpu.qmm_f32(x, *wgu))
    hh = O.silu_mul(t[:, :hdim], t[:, hdim:])
    ref = cpu.qmm_f32(hh, *dw).astype(np.float64)
    yf = O.bf16_bits_to_f32(y).astype(np.float64)
    assert O.max_rel(yf, ref) <= O.MAX_REL_TOL and O.mean_rel(yf, ref) <= O.MEAN_REL_TOL
