"""The fused residual add + RMS norm on the GPU (needs an MI355X).

Bars: h bit-exact (one bf16 rounding of x + r); n against the oracle at least 99.9% bit-equal and
every value within two bf16 ulps: the kernel's fp32 row sum may differ from the oracle's in its
last bit, which can move inv, then bf16(h * inv) by one ulp, and the product with the weight,
rounded again, by up to two.
"""

import numpy as np
import pytest
import torch

from mlx_tree_spec_amd import add_rms_norm, add_rms_norm_
from oracle import qmm4_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def bf16_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)


def host_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def within_ulps(a_bits, b_bits, ulps):
    a = O.bf16_bits_to_f32(a_bits).astype(np.float64)
    b = O.bf16_bits_to_f32(b_bits).astype(np.float64)
    mag = np.maximum(np.maximum(np.abs(a), np.abs(b)), 2.0 ** -126)
    return np.abs(a - b) <= ulps * 2.0 ** (np.floor(np.log2(mag)) - 7)


def inputs(rows, d, seed):
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16_bits(rng.standard_normal((rows, d)).astype(np.float32))
    r = O.f32_to_bf16_bits((rng.standard_normal((rows, d)) * 0.5).astype(np.float32))
    w = O.f32_to_bf16_bits((1 + 0.2 * rng.standard_normal(d)).astype(np.float32))
    return x, r, w


# Decode and verify rows at the model width (K = 5120), a prefill chunk, the smallest and largest
# widths, and widths that leave threads without a chunk or with a partial last one.
@pytest.mark.parametrize("rows,d", [(1, 5120), (4, 5120), (64, 5120), (4096, 5120), (3, 8), (5, 2056),
                                    (2, 16384), (9, 17408 // 2)])
def test_add_rms_norm_matches_oracle(rows, d):
    eps = 1e-6
    x, r, w = inputs(rows, d, rows * 7 + d)
    h, n = add_rms_norm_(bf16_dev(x), bf16_dev(r), bf16_dev(w), eps)
    hb, nb = host_bits(h), host_bits(n)
    ho, no = O.add_rms_norm(x, r, w, eps)
    assert np.array_equal(hb, ho)
    eq = float(np.mean(nb == no))
    print(f"  add_rms_norm {rows}x{d}: n bit-equal {eq:.5f}", flush=True)
    assert eq >= 0.999
    assert within_ulps(nb, no, 2).all()
    # deterministic
    h2, n2 = add_rms_norm_(bf16_dev(x), bf16_dev(r), bf16_dev(w), eps)
    assert np.array_equal(host_bits(n2), nb) and np.array_equal(host_bits(h2), hb)


def test_add_rms_norm_zero_rows_and_module_call():
    d = 256
    x, r, w = inputs(3, d, 5)
    r[1] = x[1] ^ np.uint16(0x8000)  # row 1: x + r = 0 exactly, so n = 0 (inv = 1/sqrt(eps))
    norm = torch.nn.RMSNorm(d, eps=1e-5, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(bf16_dev(w))
    h, n = add_rms_norm(bf16_dev(x).reshape(1, 3, d), bf16_dev(r).reshape(1, 3, d), norm)
    assert h.shape == (1, 3, d) and n.shape == (1, 3, d)
    hb, nb = host_bits(h).reshape(3, d), host_bits(n).reshape(3, d)
    assert np.all(O.bf16_bits_to_f32(hb[1]) == 0) and np.all(O.bf16_bits_to_f32(nb[1]) == 0)
    ho, no = O.add_rms_norm(x, r, w, 1e-5)
    assert np.array_equal(hb, ho) and within_ulps(nb, no, 2).all()
    # torch's own RMSNorm module applied to h: mostly within two ulps of n (its roundings differ)
    ref = norm(h.float().reshape(3, d).to(torch.bfloat16))
    assert within_ulps(nb, host_bits(ref), 2).mean() > 0.99


def test_add_rms_norm_rejects_mismatched_shapes():
    x, r, w = inputs(2, 64, 1)
    with pytest.raises(ValueError):
        add_rms_norm_(bf16_dev(x), bf16_dev(r[:1]), bf16_dev(w), 1e-6)
    with pytest.raises(ValueError):
        add_rms_norm_(bf16_dev(x), bf16_dev(r), bf16_dev(w[:32]), 1e-6)
    with pytest.raises(ValueError):  # width not a multiple of 8
        add_rms_norm_(bf16_dev(x[:, :60]), bf16_dev(r[:, :60]), bf16_dev(w[:60]), 1e-6)
