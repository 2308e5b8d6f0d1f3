"""The oracle, pinned before it is trusted (CPU only).

How each oracle function is pinned:
  unpack_codes / pack_codes  bytes-view decode of qmm_packed.py:115-116 (independent of shifts);
                             brute-force fixture; round trip; for the general path's 2- and 8-bit
                             words, the rows' little-endian bit strings cut into fields (8 bits:
                             the bytes themselves); parity unpinned beyond that shared formula
                             (MLX's own packing of other widths is not in the reference)
  f32_to_bf16_bits           torch's own fp32 -> bf16 conversion (round to nearest even)
  dequantize                 exact-rational brute-force fixture (incl. 257 double-rounding
                             entries); closed forms s=1,b=0 -> q; q=0 -> b; s=0 -> b;
                             group mapping with distinct per-group scales; 2/4/8-bit codes in
                             groups of 32/64/128 against the exact-rational dequant
  quantized_matmul(_exact)   brute-force fixture (exact rational sums); one-hot x picks single
                             dequantized weights; integer codes with s=1, b=0 against integer
                             arithmetic; linearity and power-of-two scaling
  pack_nax / unpack_nax      index-loop fixture of qmm_packed.py:224-231; round trip
  metrics, byte/flop counts  closed forms (the workload table's published byte counts)
  C restatement (cpu.py)     against the numpy oracle (bit-exact dequant, tolerance on y)
  silu_mul                   closed forms (g = 0, u = 0, saturated g); every bf16 g in [-30, 30]
                             against g * sigmoid(g) * u in float64 (three roundings: 3 ulps);
                             torch's own bf16 silu and multiply (within 3 ulps, mostly equal)
  gate_up_silu               halves of quantized_matmul, gate first, through silu_mul
A planted mistake in the oracle (reversed nibble order, raw-code accumulation, a sigmoid of the
wrong sign) must fail.
"""

import numpy as np
import pytest
import torch

import golden_io
from oracle import cpu
from oracle import qmm4_oracle as O


def bytes_view_codes(w):
    """Codes from the little-endian bytes: byte j of word c -> k = 8c+2j (low), 8c+2j+1 (high)."""
    b = np.ascontiguousarray(w, dtype="<u4").view(np.uint8).reshape(w.shape[0], -1)
    out = np.empty((w.shape[0], b.shape[1] * 2), dtype=np.uint8)
    out[:, 0::2] = b & 0xF
    out[:, 1::2] = b >> 4
    return out


def test_unpack_codes_matches_bytes_view():
    rng = np.random.default_rng(1)
    w = rng.integers(0, 2**32, size=(37, 24), dtype=np.uint32)
    assert np.array_equal(O.unpack_codes(w), bytes_view_codes(w))
    assert np.array_equal(O.pack_codes(O.unpack_codes(w)), w)


def test_unpack_codes_single_word():
    w = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    assert O.unpack_codes(w).tolist() == [list(range(16))]


def row_bit_string_codes(w, bits):
    """Codes of each row read from the row's whole little-endian bit string (one Python integer per
    row): code k is bits [bits k, bits k + bits) of it. Independent of per-word shifts."""
    w = np.ascontiguousarray(w, dtype="<u4")
    out = []
    for row in w:
        v = int.from_bytes(row.tobytes(), "little")
        out.append([(v >> (bits * k)) & ((1 << bits) - 1) for k in range(row.size * 32 // bits)])
    return np.array(out, dtype=np.uint8)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_unpack_codes_general_bits_against_row_bit_string(bits):
    """The general path's whole-word formats: code k = (32 / bits) c + i in bits [bits i, bits i +
    bits) of word c is the row's little-endian bit string cut into bits-wide fields (4 bits: the
    byte view above, qmm_packed.py:115-116)."""
    rng = np.random.default_rng(bits)
    w = rng.integers(0, 2**32, size=(5, 12), dtype=np.uint32)
    q = O.unpack_codes(w, bits)
    assert np.array_equal(q, row_bit_string_codes(w, bits))
    assert np.array_equal(O.pack_codes(q, bits), w)
    if bits == 8:  # the codes are the words' little-endian bytes
        assert np.array_equal(q, np.ascontiguousarray(w, dtype="<u4").view(np.uint8).reshape(5, -1))
    # A planted mistake: fields taken from the top of each word down.
    per = 32 // bits
    rev = q.reshape(5, -1, per)[:, :, ::-1].reshape(5, -1)
    assert not np.array_equal(rev, row_bit_string_codes(w, bits))


@pytest.mark.parametrize("bits,group_size", [(2, 32), (2, 128), (8, 32), (8, 64), (8, 128), (4, 32), (4, 128)])
def test_dequantize_general_formats_exact_rational(bits, group_size):
    """dequantize for the general path's formats against the exact-rational dequant of
    tests/golden/make_golden.py (bf16_rne(fp32_rne(s * q + b)) computed with Fractions), codes
    read from the row bit strings, each group's own scale and bias (distinct per group)."""
    import sys
    import os
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import make_golden as G

    rng = np.random.default_rng(100 * bits + group_size)
    n, k = 3, 256
    w = rng.integers(0, 2**32, size=(n, k * bits // 32), dtype=np.uint32)
    sf = (np.abs(rng.standard_normal((n, k // group_size))) * 0.01 + 1e-3).astype(np.float32)
    s = O.f32_to_bf16_bits(sf)
    b = O.f32_to_bf16_bits((-(2 ** (bits - 1)) * O.bf16_bits_to_f32(s)
                            + rng.standard_normal((n, k // group_size)).astype(np.float32) * 1e-3).astype(np.float32))
    got = O.dequantize(w, s, b, group_size, bits)
    q = row_bit_string_codes(w, bits)
    want = np.array([[G.dequant_one(int(s[i, j // group_size]), int(b[i, j // group_size]), int(q[i, j]))
                      for j in range(k)] for i in range(n)], dtype=np.uint16)
    assert np.array_equal(got, want)
    # A planted mistake: the neighbouring group's scale.
    s2 = np.roll(s, 1, axis=1)
    assert not np.array_equal(O.dequantize(w, s2, b, group_size, bits), want)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, size=200000, dtype=np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    ties = (rng.integers(0, 2**16, size=5000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    ties = ties[np.isfinite(ties)]
    for arr in (f, ties, np.array([0.0, -0.0, 1e-40, -1e-40, 3.4e38, -3.4e38], np.float32)):
        ref = torch.from_numpy(arr.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(O.f32_to_bf16_bits(arr), ref)
    nan = O.f32_to_bf16_bits(np.array([np.nan], np.float32))
    assert np.isnan(O.bf16_bits_to_f32(nan)).all()


def test_dequant_matches_bruteforce_table():
    w, s, b, expected, single = golden_io.dequant_table_weights()
    got = O.dequantize(w, s, b)
    assert np.array_equal(got, expected)
    # The table holds entries where rounding s*q+b straight to bf16 would differ: the oracle must
    # follow the reference's fp32-then-bf16 rounding there.
    assert (expected != single).sum() > 100
    assert not np.array_equal(got, single)


def test_dequant_closed_forms():
    rng = np.random.default_rng(3)
    n, k = 8, 256
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    q = O.unpack_codes(w).astype(np.float32)
    one = np.full((n, k // 64), 0x3F80, np.uint16)
    zero = np.zeros((n, k // 64), np.uint16)
    assert np.array_equal(O.bf16_bits_to_f32(O.dequantize(w, one, zero)), q)
    b = O.f32_to_bf16_bits(rng.standard_normal((n, k // 64)).astype(np.float32))
    assert np.array_equal(O.dequantize(w, zero, b), np.repeat(b, 64, axis=1))
    assert np.array_equal(O.dequantize(np.zeros_like(w), one, b), np.repeat(b, 64, axis=1))


def test_dequant_group_mapping():
    n, k = 4, 512
    w = O.pack_codes(np.ones((n, k), np.uint8))
    s = O.f32_to_bf16_bits(2.0 ** -np.arange(k // 64, dtype=np.float32))[None, :].repeat(n, 0)
    got = O.bf16_bits_to_f32(O.dequantize(w, s, np.zeros_like(s)))
    for kk in range(k):
        assert (got[:, kk] == 2.0 ** -(kk // 64)).all()


@pytest.mark.parametrize("case", golden_io.qmm_cases(), ids=lambda c: f"{c['m']}x{c['k']}x{c['n']}")
def test_qmm_matches_bruteforce(case):
    deq = O.dequantize(case["w"], case["s"], case["b"])
    assert np.array_equal(deq, case["deq"])
    exact = O.quantized_matmul_exact(case["x"], case["w"], case["s"], case["b"])
    np.testing.assert_allclose(exact, case["exact"], rtol=1e-12, atol=1e-12)
    y = O.quantized_matmul(case["x"], case["w"], case["s"], case["b"])
    assert np.array_equal(y, case["y"])


def test_qmm_one_hot_picks_weights():
    x0, w, s, b = O.make_inputs(1, 256, 32, seed=5)
    deq = O.bf16_bits_to_f32(O.dequantize(w, s, b))
    for kk in (0, 7, 8, 63, 64, 200, 255):
        x = np.zeros((1, 256), np.uint16)
        x[0, kk] = 0x3F80  # 1.0
        y = O.quantized_matmul_exact(x, w, s, b)
        assert np.array_equal(y[0], deq[:, kk].astype(np.float64))


def test_qmm_integer_codes():
    rng = np.random.default_rng(6)
    m, k, n = 5, 384, 48
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    xi = rng.integers(-8, 8, size=(m, k))
    x = O.f32_to_bf16_bits(xi.astype(np.float32))
    one = np.full((n, k // 64), 0x3F80, np.uint16)
    y = O.quantized_matmul_exact(x, w, one, np.zeros_like(one))
    assert np.array_equal(y, (xi @ bytes_view_codes(w).astype(np.int64).T).astype(np.float64))


def test_qmm_linearity_and_pow2_scaling():
    x, w, s, b = O.make_inputs(4, 256, 64, seed=7)
    y = O.quantized_matmul_exact(x, w, s, b)
    x2 = O.f32_to_bf16_bits(O.bf16_bits_to_f32(x) * 2)
    assert np.array_equal(O.quantized_matmul_exact(x2, w, s, b), 2 * y)
    xa, _, _, _ = O.make_inputs(4, 256, 64, seed=8)
    xs = O.bf16_bits_to_f32(x).astype(np.float64) + O.bf16_bits_to_f32(xa)
    wd = O.bf16_bits_to_f32(O.dequantize(w, s, b)).astype(np.float64)
    np.testing.assert_allclose(y + O.quantized_matmul_exact(xa, w, s, b), xs @ wd.T, rtol=1e-12, atol=1e-12)


def test_planted_mistakes_fail():
    """A plausible mistake in the oracle must be caught by the pins above."""
    case = golden_io.qmm_cases()[3]
    # Reversed nibble order inside each word.
    q = O.unpack_codes(case["w"]).reshape(case["n"], -1, 8)[:, :, ::-1].reshape(case["n"], -1)
    assert not np.array_equal(O.dequantize(O.pack_codes(q), case["s"], case["b"]), case["deq"])
    # Raw-code accumulation s*sum(qx) + b*sum(x), skipping the bf16 rounding of the weights: out
    # of the mean-relative tolerance at a model-sized K.
    x, w, s, b = O.make_inputs(16, 5120, 512, seed=0)
    ref = O.quantized_matmul_exact(x, w, s, b)
    q = O.unpack_codes(w).astype(np.float64)
    raw = O.bf16_bits_to_f32(x).astype(np.float64) @ (q * np.repeat(O.bf16_bits_to_f32(s), 64, 1)
                                                     + np.repeat(O.bf16_bits_to_f32(b), 64, 1)).T
    raw_bf16 = O.bf16_bits_to_f32(O.f32_to_bf16_bits(raw.astype(np.float32)))
    assert O.mean_rel(raw_bf16, ref) > O.MEAN_REL_TOL
    good = O.bf16_bits_to_f32(O.quantized_matmul(x, w, s, b))
    assert O.mean_rel(good, ref) < O.MEAN_REL_TOL and O.max_rel(good, ref) < O.MAX_REL_TOL


def bf16_grid(lo: float, hi: float) -> np.ndarray:
    """Every finite bf16 bit pattern whose value lies in [lo, hi]."""
    u = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    v = O.bf16_bits_to_f32(u)
    return u[np.isfinite(v) & (v >= lo) & (v <= hi)]


def silu_f64(g, u):
    gf = O.bf16_bits_to_f32(g).astype(np.float64)
    return gf / (1.0 + np.exp(-gf)) * O.bf16_bits_to_f32(u).astype(np.float64)


def within_ulps(out_bits, exact, ulps):
    """|out - exact| <= ulps bf16 ulps of exact (or of the smallest normal, near zero)."""
    out = O.bf16_bits_to_f32(out_bits).astype(np.float64)
    mag = np.maximum(np.abs(exact), 2.0 ** -126)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 7)
    return np.abs(out - exact) <= ulps * ulp


def test_silu_mul_closed_forms():
    one, half = O.f32_to_bf16_bits(np.float32(1.0)), O.f32_to_bf16_bits(np.float32(0.5))
    g = bf16_grid(-30, 30)
    assert np.all(O.bf16_bits_to_f32(O.silu_mul(np.zeros(5, np.uint16), g[:5])) == 0)  # silu(0) = 0
    assert np.all(O.bf16_bits_to_f32(O.silu_mul(g, np.zeros_like(g))) == 0)
    big = O.f32_to_bf16_bits(np.array([20.0, 64.0, 1000.0], np.float32))  # sigmoid = 1 in fp32
    assert np.array_equal(O.silu_mul(big, np.full(3, one)), big)
    assert np.array_equal(O.silu_mul(big, np.full(3, half)), O.f32_to_bf16_bits(O.bf16_bits_to_f32(big) * 0.5))
    # silu(g) - silu(-g) = g (sigmoid(g) + sigmoid(-g) = 1)
    gp = bf16_grid(0.5, 8)
    sp = O.bf16_bits_to_f32(O.silu_mul(gp, np.full(gp.shape, one))).astype(np.float64)
    sn = O.bf16_bits_to_f32(O.silu_mul(gp ^ np.uint16(0x8000), np.full(gp.shape, one))).astype(np.float64)
    np.testing.assert_allclose(sp - sn, O.bf16_bits_to_f32(gp), rtol=2 ** -6, atol=2 ** -6)


def test_silu_mul_matches_float64_and_torch():
    g = bf16_grid(-30, 30)
    for uval in (1.0, -0.75, 3.5):
        u = np.full(g.shape, O.f32_to_bf16_bits(np.float32(uval)))
        out = O.silu_mul(g, u)
        assert within_ulps(out, silu_f64(g, u), 3).all()
        # torch: silu in fp32 rounded once to bf16, then the bf16 product (one rounding fewer than
        # the op-by-op composition, which rounds the sigmoid first)
        tg = torch.from_numpy(g.astype(np.int16)).view(torch.bfloat16)
        tu = torch.from_numpy(u.astype(np.int16)).view(torch.bfloat16)
        tref = (torch.nn.functional.silu(tg) * tu).view(torch.int16).numpy().view(np.uint16)
        assert within_ulps(out, O.bf16_bits_to_f32(tref).astype(np.float64), 3).all()
        assert np.mean(out == tref) > 0.9
    # planted mistake: the sigmoid of the wrong sign
    gf = O.bf16_bits_to_f32(g)
    wrong = O.f32_to_bf16_bits(gf * (1.0 / (1.0 + np.exp(gf))))
    assert not within_ulps(wrong, silu_f64(g, np.full(g.shape, O.f32_to_bf16_bits(np.float32(1.0)))), 3).all()


def test_add_rms_norm_closed_forms():
    d = 64
    one = O.f32_to_bf16_bits(np.float32(1.0))
    w = O.f32_to_bf16_bits(np.linspace(-2, 2, d).astype(np.float32))
    # a constant power-of-two row with eps = 0: h = c, inv = 1/|c| exactly, n = sign(c) * w
    for c in (4.0, -0.5):
        x = np.full((1, d), O.f32_to_bf16_bits(np.float32(c)))
        h, n = O.add_rms_norm(x, np.zeros_like(x), w, 0.0)
        assert np.array_equal(h, x)
        assert np.array_equal(O.bf16_bits_to_f32(n), np.sign(c) * O.bf16_bits_to_f32(w)[None, :])
    # h = x + r exactly where it is representable; a zero row gives n = 0 (inv = 1/sqrt(eps))
    x = np.full((2, d), one)
    r = np.full((2, d), O.f32_to_bf16_bits(np.float32(-1.0)))
    h, n = O.add_rms_norm(x, r, w, 1e-6)
    assert np.all(O.bf16_bits_to_f32(h) == 0) and np.all(O.bf16_bits_to_f32(n) == 0)
    # eps enters the mean: a row of ones with eps = 3 has inv = 1/2
    h, n = O.add_rms_norm(np.full((1, d), one), np.zeros((1, d), np.uint16), np.full(d, one), 3.0)
    assert np.all(O.bf16_bits_to_f32(n) == 0.5)


def test_add_rms_norm_matches_torch():
    rng = np.random.default_rng(3)
    rows, d, eps = 7, 5120, 1e-6
    x = O.f32_to_bf16_bits(rng.standard_normal((rows, d)).astype(np.float32))
    r = O.f32_to_bf16_bits(rng.standard_normal((rows, d)).astype(np.float32) * 0.3)
    w = O.f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(d)).astype(np.float32))
    h, n = O.add_rms_norm(x, r, w, eps)
    tb = lambda a: torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16)
    th = tb(x) + tb(r)  # torch adds bf16 in fp32 and rounds once
    assert np.array_equal(h, th.view(torch.int16).numpy().view(np.uint16))
    hf = th.float()
    normed = (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
    tn = (tb(w) * normed).view(torch.int16).numpy().view(np.uint16)
    assert within_ulps(n, O.bf16_bits_to_f32(tn).astype(np.float64), 1).all()
    assert np.mean(n == tn) >= 0.999
    # planted mistake: the mean over D + 1 values (inv off by 1e-4 relative) moves ~1% of outputs
    hf64 = O.bf16_bits_to_f32(h).astype(np.float64)
    inv = 1.0 / np.sqrt((hf64 ** 2).sum(-1) / (d + 1) + eps)
    wrong = O.f32_to_bf16_bits((O.bf16_bits_to_f32(w)[None] * O.bf16_bits_to_f32(
        O.f32_to_bf16_bits((hf64 * inv[:, None]).astype(np.float32)))).astype(np.float32))
    assert np.mean(wrong == tn) < 0.999


def test_gate_up_silu_is_halves_of_the_projection():
    x, w, s, b = O.make_inputs(3, 256, 64, seed=9)
    y = O.quantized_matmul(x, w, s, b)
    h = O.gate_up_silu(x, w, s, b)
    assert h.shape == (3, 32)
    assert np.array_equal(h, O.silu_mul(y[:, :32], y[:, 32:]))
    # gate first: swapping the halves changes the result
    assert not np.array_equal(h, O.silu_mul(y[:, 32:], y[:, :32]))


def test_pack_nax_matches_index_loops():
    z = golden_io.load("pack_nax.npz")
    wq2, sp2, _ = O.pack_nax(z["w"], z["s"], z["s"])
    assert np.array_equal(wq2, z["wq2"]) and np.array_equal(sp2, z["sp2"])
    w, s, b = O.unpack_nax(wq2, sp2, sp2, z["w"].shape[0])
    assert np.array_equal(w, z["w"]) and np.array_equal(s, z["s"]) and np.array_equal(b, z["s"])


def test_metrics_closed_forms():
    ref = np.array([1.0, -2.0, 4.0])
    y = np.array([1.5, -2.0, 4.0])
    assert O.max_rel(y, ref) == pytest.approx(0.5 / 4)
    assert O.mean_rel(y, ref) == pytest.approx((0.5 / 3) / (7 / 3))
    assert O.rel_l2(y, ref) == pytest.approx(0.5 / np.sqrt(21))


def test_workload_bytes_and_flops():
    # The workload table's byte counts: c0 15.07 MB, c1 100.35/100.43/100.59, c2 53.02, c3 447.63, c4 234.68.
    expect = {(16, 5120, 5120): 15.07, (1, 5120, 34816): 100.35, (2, 5120, 34816): 100.43,
              (4, 5120, 34816): 100.59, (64, 17408, 5120): 53.02, (32, 5120, 151936): 447.63,
              (4096, 5120, 17408): 234.68}
    for (m, k, n), mb in expect.items():
        assert O.bytes_per_call(m, k, n) / 1e6 == pytest.approx(mb, abs=0.006)
    assert O.flops_per_call(4096, 5120, 17408) / 1e9 == pytest.approx(730.14, abs=0.01)


def test_make_inputs_deterministic_and_distributed():
    a = O.make_inputs(4, 512, 64, seed=1)
    b = O.make_inputs(4, 512, 64, seed=1)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    x, w, s, bb = O.make_inputs(8, 5120, 256, sigma=0.5, seed=2)
    q = O.unpack_codes(w)
    counts = np.bincount(q.ravel(), minlength=16) / q.size
    assert np.abs(counts - 1 / 16).max() < 0.002
    sf = O.bf16_bits_to_f32(s)
    assert sf.min() >= 1e-4 * 0.99 and abs(O.bf16_bits_to_f32(x).std() - 0.5) < 0.01
    bf = O.bf16_bits_to_f32(bb)
    assert np.abs(bf + 8 * sf).max() < 0.01
    x1, *_ = O.config_inputs(1, m=1)
    x4, *_ = O.config_inputs(1)
    assert x4.shape == (4, 5120) and np.array_equal(x1, x4[:1])


def test_c_restatement_matches_numpy_oracle():
    x, w, s, b = O.make_inputs(9, 1024, 96, seed=4)
    assert np.array_equal(cpu.dequant(w, s, b), O.dequantize(w, s, b))
    ref = O.quantized_matmul_exact(x, w, s, b)
    y = O.bf16_bits_to_f32(cpu.qmm(x, w, s, b))
    assert O.max_rel(y, ref) < O.MAX_REL_TOL and O.mean_rel(y, ref) < O.MEAN_REL_TOL
    yf = cpu.qmm_f32(x, w, s, b)
    np.testing.assert_allclose(yf, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    assert np.array_equal(O.f32_to_bf16_bits(yf), cpu.qmm(x, w, s, b))
    w2, s2, b2, expected, _ = golden_io.dequant_table_weights()
    assert np.array_equal(cpu.dequant(w2, s2, b2), expected)
