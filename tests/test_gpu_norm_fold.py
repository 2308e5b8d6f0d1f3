"""The residual add + RMS norm folded into the projection that consumes its output (needs an MI355X).

qmm4_add_rms_norm_qmm_bf16 replaces the pair add_rms_norm + projection of tree_verify.py:444-446
(fused_ops.py:107-160 then packed_linear.py:97 / the MLP's gate+up). Bars:
  - against the unfused pair (add_rms_norm_, then quantized_matmul / gate_up_silu on its n): h, n
    and y bit-equal. The fold performs the norm's arithmetic over the same partition of each row
    (the same chunks per thread, the butterfly, the waves in order) and stages the n it forms into
    the row-split kernel that the plain call runs, so any difference is a bug;
  - against the oracle: h bit-exact; n at least 99.9% bit-equal and every value within two bf16
    ulps (the fp32 row sum's order is the kernel's own); y to max_rel <= 1e-2, mean_rel <= 2e-3
    of the oracle's fp32-accumulated projection (and SiLU·mul) of the GPU's n.
The shapes (route_cases.FOLD_CASES, whose routes tests/test_plans.py checks against the planner)
cover each form of the folded kernel (whole K, K in 2 slices for the plain and the gate+up
epilogue, units of 4 and 5 super-steps, K from 512 to the largest folded 8192) and the shapes that
run as two launches (5 rows, K > 8192, 16 rows, and 24-64 rows over the row-phase kernel, fused
gate+up or K split).
"""

import numpy as np
import pytest
import torch

from mlx_tree_spec_amd import add_rms_norm_, add_rms_norm_qmm_, gate_up_silu, quantized_matmul
from mlx_tree_spec_amd import _lib
from oracle import cpu
from oracle import qmm4_oracle as O
from route_cases import FOLD_CASES

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-6


def bf16_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)


def u32_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(DEV)


def host_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def within_ulps(a_bits, b_bits, ulps):
    a = O.bf16_bits_to_f32(a_bits).astype(np.float64)
    b = O.bf16_bits_to_f32(b_bits).astype(np.float64)
    mag = np.maximum(np.maximum(np.abs(a), np.abs(b)), 2.0 ** -126)
    return np.abs(a - b) <= ulps * 2.0 ** (np.floor(np.log2(mag)) - 7)


def make_case(m, n, k, seed):
    x, w, s, b = O.make_inputs(m, k, n, seed=seed)
    rng = np.random.default_rng(seed + 1)
    r = O.f32_to_bf16_bits((0.5 * rng.standard_normal((m, k))).astype(np.float32))
    nw = O.f32_to_bf16_bits((1 + 0.2 * rng.standard_normal(k)).astype(np.float32))
    return x, r, nw, w, s, b


CASES = [c[:4] for c in FOLD_CASES]


@pytest.mark.parametrize("m,n,k,silu_mul", CASES)
def test_fold_equals_unfused_pair_and_oracle(m, n, k, silu_mul):
    print(f"  fold M={m} N={n} K={k} silu_mul={silu_mul}", flush=True)
    x, r, nw, w, s, b = make_case(m, n, k, seed=m * 131 + n + k)
    xd, rd, nwd, wd, sd, bd = bf16_dev(x), bf16_dev(r), bf16_dev(nw), u32_dev(w), bf16_dev(s), bf16_dev(b)
    h, nrm, y = add_rms_norm_qmm_(xd, rd, nwd, EPS, wd, sd, bd, silu_mul=silu_mul)
    # The unfused pair on the same inputs.
    h2, n2 = add_rms_norm_(xd, rd, nwd, EPS)
    y2 = gate_up_silu(n2, wd, sd, bd) if silu_mul else quantized_matmul(n2, wd, sd, bd)
    hb, nb, yb = host_bits(h), host_bits(nrm), host_bits(y)
    assert np.array_equal(hb, host_bits(h2)), "h differs from add_rms_norm"
    assert np.array_equal(nb, host_bits(n2)), "n differs from add_rms_norm"
    assert np.array_equal(yb, host_bits(y2)), "y differs from the projection of add_rms_norm's n"
    # The oracle.
    ho, no = O.add_rms_norm(x, r, nw, EPS)
    assert np.array_equal(hb, ho)
    assert float(np.mean(nb == no)) >= 0.999 and within_ulps(nb, no, 2).all()
    t = cpu.qmm_f32(nb, w, s, b)
    if silu_mul:
        tb = O.f32_to_bf16_bits(t)
        want = O.bf16_bits_to_f32(O.silu_mul(tb[:, : n // 2], tb[:, n // 2:])).astype(np.float64)
    else:
        want = t.astype(np.float64)
    got = O.bf16_bits_to_f32(yb).astype(np.float64)
    print(f"    y max_rel={O.max_rel(got, want):.2e} mean_rel={O.mean_rel(got, want):.2e}", flush=True)
    assert O.max_rel(got, want) <= O.MAX_REL_TOL and O.mean_rel(got, want) <= O.MEAN_REL_TOL
    # Deterministic.
    h3, n3, y3 = add_rms_norm_qmm_(xd, rd, nwd, EPS, wd, sd, bd, silu_mul=silu_mul)
    assert np.array_equal(host_bits(y3), yb) and np.array_equal(host_bits(n3), nb)


def test_fold_zero_rows_of_r_and_large_eps():
    """r = 0 (h = x) and a large eps (inv far from 1/rms): still the unfused pair's bits."""
    m, n, k = 2, 34816, 5120
    x, _, nw, w, s, b = make_case(m, n, k, seed=5)
    r = np.zeros_like(x)
    for eps in (0.0, 4.0):
        xd, rd, nwd = bf16_dev(x), bf16_dev(r), bf16_dev(nw)
        wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
        h, nrm, y = add_rms_norm_qmm_(xd, rd, nwd, eps, wd, sd, bd, silu_mul=True)
        h2, n2 = add_rms_norm_(xd, rd, nwd, eps)
        y2 = gate_up_silu(n2, wd, sd, bd)
        assert np.array_equal(host_bits(h), x)
        assert np.array_equal(host_bits(nrm), host_bits(n2))
        assert np.array_equal(host_bits(y), host_bits(y2))


def test_fold_no_projection_columns_runs_the_norm():
    m, k = 3, 5120
    x, r, nw, _, _, _ = make_case(m, 16, k, seed=9)
    xd, rd, nwd = bf16_dev(x), bf16_dev(r), bf16_dev(nw)
    w0 = torch.zeros((0, k // 8), dtype=torch.int32, device=DEV)
    s0 = torch.zeros((0, k // 64), dtype=torch.bfloat16, device=DEV)
    h, nrm, y = add_rms_norm_qmm_(xd, rd, nwd, EPS, w0, s0, s0)
    h2, n2 = add_rms_norm_(xd, rd, nwd, EPS)
    assert y.shape == (m, 0)
    assert np.array_equal(host_bits(h), host_bits(h2)) and np.array_equal(host_bits(nrm), host_bits(n2))


def test_fold_rejects_overlapping_outputs():
    """h_out may not alias x: every workgroup of the folded kernel reads x while the first writes h."""
    m, n, k = 1, 34816, 5120
    x, r, nw, w, s, b = make_case(m, n, k, seed=3)
    xd, rd, nwd, wd, sd, bd = bf16_dev(x), bf16_dev(r), bf16_dev(nw), u32_dev(w), bf16_dev(s), bf16_dev(b)
    nbuf = torch.empty_like(xd)
    y = torch.empty((m, n // 2), dtype=torch.bfloat16, device=DEV)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.qmm4_add_rms_norm_qmm_bf16(xd.data_ptr(), rd.data_ptr(), nwd.data_ptr(), EPS, xd.data_ptr(),
                                        nbuf.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), y.data_ptr(),
                                        m, n, k, 64, 4, 1, _lib.QMM4_EPILOGUE_SILU_MUL, stream)
    assert rc == _lib.QMM4_ERR_INVALID and "overlap" in _lib.last_error()
