"""Parity of the gfx950 kernels with the oracle, through the C ABI (needs an MI355X).

Bars:
  * dequantize: bit-exact against the exact-rational brute-force table, and against the oracle
    over every finite bf16 scale and random model-sized weights;
  * quantized_matmul: the parity tolerance against the fp32-accumulated reference
    (max|y-ref|/max|ref| <= 1e-2, mean|y-ref|/mean|ref| <= 2e-3), and, much tighter, per element:
    at least 99% of outputs equal bf16_rne(ref) and every other output is within one bf16 ulp of
    ref plus 2^-17 * sum_k |x||w| (only the fp32 accumulation order differs from the oracle);
  * size-independent properties at the full workload sizes: determinism, y(2x) == 2 y(x).
"""

import os
import sys
import warnings

import numpy as np
import pytest
import torch

import golden_io
from mlx_tree_spec_amd import STATS, QuantizedLinear, dequantize, install, quantized_matmul
from oracle import cpu
from oracle import qmm4_oracle as O
from route_cases import (MID_ROW_CASES, ROWPHASE_ONE_HOT, ROWPHASE_SHAPES, ROWPHASE_WIDE_CASES,
                         ROWPHASE_WINDOW_CASES)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bf16_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)


def u32_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(DEV)


def host_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def gpu_qmm(x, w, s, b):
    y = quantized_matmul(bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b))
    return host_bits(y)


def abs_dot(x, w, s, b, rows, cols):
    """S[i] = sum_k |x[rows[i], k]| * |dequant(w)[cols[i], k]|: the scale of fp32 rounding error
    in output (rows[i], cols[i])."""
    ucols, inv = np.unique(cols, return_inverse=True)
    wd = np.abs(O.bf16_bits_to_f32(O.dequantize(w[ucols], s[ucols], b[ucols])).astype(np.float64))
    xa = np.abs(O.bf16_bits_to_f32(x).astype(np.float64))
    return np.einsum("ik,ik->i", xa[rows], wd[inv])


def check_qmm(y_bits, ref, what="", inputs=None):
    """max_rel <= 1e-2 and mean_rel <= 2e-3, plus per element: at least 99% of outputs equal bf16_rne(ref), and
    every other one is within one bf16 ulp of ref plus 2^-17 * sum_k |x||w| (fp32 accumulation
    in another order can move a result near zero by many of its own ulps, never by more)."""
    ref = np.asarray(ref, dtype=np.float64)
    y = O.bf16_bits_to_f32(y_bits).astype(np.float64)
    mx, mn = O.max_rel(y, ref), O.mean_rel(y, ref)
    rne = O.f32_to_bf16_bits(ref.astype(np.float32))
    mism = y_bits != rne
    nm = int(mism.sum())
    far = 0
    if nm and inputs is not None:
        x, w, s, b = inputs
        rows, cols = np.nonzero(mism.reshape(-1, mism.shape[-1]))
        sel = np.arange(rows.size)
        if sel.size > 4096:
            sel = np.random.default_rng(0).choice(sel, 4096, replace=False)
        rows, cols = rows[sel], cols[sel]
        yy = y.reshape(-1, y.shape[-1])[rows, cols]
        rr = ref.reshape(-1, ref.shape[-1])[rows, cols]
        ulp = np.spacing(np.abs(O.bf16_bits_to_f32(rne.reshape(-1, rne.shape[-1])[rows, cols])).astype(np.float32)) * 65536.0
        bound = ulp + 2.0 ** -17 * abs_dot(np.asarray(x).reshape(-1, np.asarray(x).shape[-1]), w, s, b, rows, cols)
        far = int((np.abs(yy - rr) > bound).sum())
    note(f"  {what} max_rel={mx:.2e} mean_rel={mn:.2e} mismatches={nm}/{mism.size} far={far}")
    assert mx <= O.MAX_REL_TOL and mn <= O.MEAN_REL_TOL
    assert nm <= max(2, mism.size // 100)
    assert far == 0


def test_native_library_is_loaded():
    x, w, s, b = O.make_inputs(1, 128, 16, seed=0)
    gpu_qmm(x, w, s, b)
    maps = open("/proc/self/maps").read()
    assert "libqmm4.so" in maps


# ----------------------------------------------------------------------------- dequant
def test_dequant_bruteforce_table():
    w, s, b, expected, _ = golden_io.dequant_table_weights()
    got = host_bits(dequantize(u32_dev(w), bf16_dev(s), bf16_dev(b)))
    assert np.array_equal(got, expected)


@pytest.mark.parametrize("bias_kind", ["model", "random"])
def test_dequant_every_finite_bf16_scale(bias_kind):
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    s = allbits[((allbits >> 7) & 0xFF) != 0xFF]
    n = s.size
    rng = np.random.default_rng(11)
    if bias_kind == "model":
        with np.errstate(over="ignore"):  # -8 s overflows for the largest scales; those become 0 below
            b = O.f32_to_bf16_bits(-8 * O.bf16_bits_to_f32(s) + rng.standard_normal(n).astype(np.float32) * 1e-3)
        b = np.where(((b >> 7) & 0xFF) == 0xFF, np.uint16(0), b)
    else:
        b = rng.integers(0, 65536, n).astype(np.uint16)
        b = np.where(((b >> 7) & 0xFF) == 0xFF, np.uint16(0x3F80), b)
    codes = np.tile(np.arange(16, dtype=np.uint8), (n, 4))
    w = O.pack_codes(codes)
    s2, b2 = s.reshape(n, 1), b.reshape(n, 1)
    got = host_bits(dequantize(u32_dev(w), bf16_dev(s2), bf16_dev(b2)))
    assert np.array_equal(got, O.dequantize(w, s2, b2))


@pytest.mark.parametrize("n,k", [(16, 64), (48, 192), (512, 5120), (1000, 17408)])
def test_dequant_random(n, k):
    _, w, s, b = O.make_inputs(1, k, n, seed=n)
    got = host_bits(dequantize(u32_dev(w), bf16_dev(s), bf16_dev(b)))
    assert np.array_equal(got, O.dequantize(w, s, b))


# ----------------------------------------------------------------------------- dequant inside qmm
def scale_bias_pairs(kind, n, rng):
    """bf16 (s, b) bit patterns for n groups. 'fast': scale exponent field in [0, 230], the
    range the kernels dequantize with v_fma_mix_f32 (zero and subnormal scales included), with
    biases of any exponent up to 60 fields away; 'slow': scales in [2^104, 2^124), which the kernels
    send to the general form; 'mixed': one group in eight slow. Every dequantized value is finite."""
    def bits(sign, e, m):
        return ((sign << 15) | (e << 7) | m).astype(np.uint16)
    sgn = lambda: rng.integers(0, 2, n, dtype=np.uint32)
    man = lambda: rng.integers(0, 128, n, dtype=np.uint32)
    if kind in ("fast", "slow"):
        lo, hi = (0, 231) if kind == "fast" else (231, 251)
        es = rng.integers(lo, hi, n, dtype=np.uint32)
        es[:2] = [lo, hi - 1]
        eb = np.clip(es.astype(np.int64) + rng.integers(-60, 61, n), 0, 250).astype(np.uint32)
        s, b = bits(sgn(), es, man()), bits(sgn(), eb, man())
        if kind == "fast":
            s[2], b[3] = 0, 0  # a zero scale, a zero bias
        return s, b
    sf, bf = scale_bias_pairs("fast", n, rng)
    sl, bl = scale_bias_pairs("slow", n, rng)
    pick = rng.integers(0, 8, n) == 0
    return np.where(pick, sl, sf), np.where(pick, bl, bf)


@pytest.mark.parametrize("kind", ["fast", "slow", "mixed"])
@pytest.mark.parametrize("m", [64, 32, 4])
def test_qmm_one_hot_is_exact_dequant(kind, m):
    """y = x @ dequant(w).T with one-hot rows of x reads single dequantized weights, so the
    dequantization inside the matmul kernels must equal the oracle's bit for bit (zeros of
    either sign compare equal: the fp32 sum turns -0 into +0)."""
    n, k = 4096, 256
    rng = np.random.default_rng({"fast": 1, "slow": 2, "mixed": 3}[kind] * 100 + m)
    s, b = scale_bias_pairs(kind, n * (k // 64), rng)
    s, b = s.reshape(n, k // 64), b.reshape(n, k // 64)
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    deq = O.dequantize(w, s, b)
    dv = O.bf16_bits_to_f32(deq)
    assert np.isfinite(dv).all()
    # Subnormal bf16 weights would test the MFMA's handling of subnormals, not the dequant.
    sub = (deq & 0x7F80) == 0
    wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
    for k0 in range(0, k, m):
        x = np.zeros((m, k), dtype=np.uint16)
        x[np.arange(m), k0 + np.arange(m)] = 0x3F80  # 1.0
        y = host_bits(quantized_matmul(bf16_dev(x), wd, sd, bd))
        ref = deq[:, k0:k0 + m].T
        yv, rv = O.bf16_bits_to_f32(y), O.bf16_bits_to_f32(ref)
        keep = ~sub[:, k0:k0 + m].T
        bad = keep & (yv != rv)
        assert not bad.any(), f"{int(bad.sum())} mismatches at k0={k0}, first {np.argwhere(bad)[:3].tolist()}"


# ----------------------------------------------------------------------------- small / golden
@pytest.mark.parametrize("case", [c for c in golden_io.qmm_cases() if c["k"] % 128 == 0 and c["n"] % 16 == 0],
                         ids=lambda c: f"{c['m']}x{c['k']}x{c['n']}")
def test_qmm_bruteforce_cases(case):
    y = gpu_qmm(case["x"], case["w"], case["s"], case["b"])
    check_qmm(y, case["exact"], "golden", (case["x"], case["w"], case["s"], case["b"]))


ROWS = [1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 24, 31, 32, 33, 40, 47, 48, 63, 64]


@pytest.mark.parametrize("m", ROWS)
def test_qmm_skinny_rows(m):
    x, w, s, b = O.make_inputs(m, 512, 272, seed=m)  # N % 32 == 16: a half column tile
    check_qmm(gpu_qmm(x, w, s, b), O.quantized_matmul_exact(x, w, s, b), f"M={m}", (x, w, s, b))


@pytest.mark.parametrize("m", [1, 4, 16, 32, 64])
@pytest.mark.parametrize("k,n", [(128, 16), (5120, 1024), (17408, 256), (1024, 4112)])
def test_qmm_skinny_shapes(m, k, n):
    x, w, s, b = O.make_inputs(m, k, n, seed=k + n + m)
    check_qmm(gpu_qmm(x, w, s, b), O.quantized_matmul_exact(x, w, s, b), f"{m}x{k}x{n}", (x, w, s, b))


@pytest.mark.parametrize("m", [64, 100, 2048])
@pytest.mark.parametrize("k,n", [(512, 128), (1024, 192)])
def test_reference_prefill_kernel_shapes(m, k, n):
    """The shapes of the reference's only kernel test (tests/test_units.py:90-110): x is
    (1, m, k) with sigma 0.5."""
    x, w, s, b = O.make_inputs(m, k, n, sigma=0.5, seed=0)
    y = quantized_matmul(bf16_dev(x).reshape(1, m, k), u32_dev(w), bf16_dev(s), bf16_dev(b))
    assert tuple(y.shape) == (1, m, n)
    check_qmm(host_bits(y).reshape(m, n), O.quantized_matmul_exact(x, w, s, b), f"{m}x{k}x{n}", (x, w, s, b))


# 1800 x 5120 -> 4368: 144 whole 256 x 256 tiles with 8-group scale blocks (the role-split kernel),
# a partial last row of tiles (8 rows) and a partial last column (16 columns); 1536 x 512 -> 8192:
# the same kernel over the shortest K it takes (one 8-step scale block).
@pytest.mark.parametrize("m,k,n", [(65, 1152, 1024), (255, 128, 528), (256, 256, 256), (257, 1024, 784),
                                   (1024, 5120, 1040), (4096, 1024, 512), (1800, 5120, 4368), (1536, 512, 8192)])
def test_qmm_gemm_shapes(m, k, n):
    x, w, s, b = O.make_inputs(m, k, n, seed=m + k)
    check_qmm(gpu_qmm(x, w, s, b), O.quantized_matmul_exact(x, w, s, b), f"{m}x{k}x{n}", (x, w, s, b))


# ----------------------------------------------------------------------------- workloads
def workload_ref(x, w, s, b):
    return cpu.qmm_f32(x, w, s, b).astype(np.float64)


# Mid-size M with few output tiles takes the GEMM's stream-K form: 128 x 128 tiles x K units
# spread over every resident workgroup, tiles split between workgroups added by a fix-up kernel in
# K order. 65 rows over K = 17536 (40 tiles; K % 512 != 0 keeps 65 rows off the row-phase kernel,
# units of two K steps), the up projection at 128 rows, K = 1152 and K = 640, N = 784 and M = 200
# (partial column and row tiles).
# Also where whole 256 x 256 tiles would fill under half the CUs: 256 and 320 rows of the up
# projection (272 and 408 tiles of 128), on 128 x 256 tiles, as are 120 x 17408 -> 5120 (K >= 8192)
# and 136 x 5120 -> 10256 (partial row and column tiles), and 72 / 96 rows over the 65984-column
# head, where whole tiles would pad the rows to 256, and 320 / 384 rows at K >= 8192 (a last row of
# 256-row tiles at most half full: 384 x 12288 -> 5120, 384 x 17408 -> 5120, 320 x 12288 -> 5120)
# (route_cases.GEMM_STREAM_K_CASES labels the tile size of each). Long K with fewer whole 256 x 256
# tiles than CUs takes stream-K over those: 512 and 1024 rows of the down projection (40 and 80
# tiles), 1000 x 8192 -> 4112 (partial row and column tiles). Whole
# tiles whose last round has fewer quarters than CUs run it as stream-K over the quarters: 1024 x
# 5120 -> 17408 (272 tiles: 256 whole, 16 in quarters), 4096 x 1024 -> 1040 (80 tiles, a partial
# column of tiles).
@pytest.mark.parametrize("m,k,n", [(65, 17536, 5120), (128, 5120, 17408), (100, 1152, 4096), (200, 5120, 784),
                                   (96, 640, 1024), (256, 5120, 17408), (320, 5120, 17408),
                                   (1024, 17408, 5120), (512, 17408, 5120), (384, 12288, 5120), (384, 17408, 5120),
                                   (320, 12288, 5120),
                                   (1000, 8192, 4112), (1024, 5120, 17408), (4096, 1024, 1040),
                                   (120, 17408, 5120), (136, 5120, 10256), (72, 2048, 65984), (96, 5120, 65984)])
def test_gemm_stream_k_shapes(m, k, n):
    note(f"stream-K {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, sigma=0.5, seed=m * 19 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"stream-K {m}x{k}x{n}", (x, w, s, b))
    for _ in range(2):  # the same split points and fix-up order every call
        assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


def test_gemm_stream_k_unaligned_scales():
    """Scale and bias rows that are not 16-byte aligned: per-step scale loads and 2-step units."""
    m, k, n = 130, 1024, 512
    x, w, s, b = O.make_inputs(m, k, n, seed=77)
    pad = lambda a: bf16_dev(np.concatenate([np.zeros(2, np.uint16), a.reshape(-1)]))[2:].view(n, k // 64)
    sd, bd = pad(s), pad(b)
    assert sd.data_ptr() % 16 == 4
    from mlx_tree_spec_amd import _lib
    y = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    xd, wd = bf16_dev(x), u32_dev(w)
    rc = _lib.load().qmm4_affine_bf16(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), y.data_ptr(),
                                      m, n, k, 64, 4, 1, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.last_error()
    check_qmm(host_bits(y), O.quantized_matmul_exact(x, w, s, b), "stream-K unaligned scales", (x, w, s, b))


# One-hot rows through each form of the GEMM with 8-group scale blocks (K % 512 == 0): stream-K with
# tiles split between workgroups (128 rows), 128 x 128 quarter tiles (1024 rows), whole 256 x 256
# tiles (2048 rows, where x is the identity), stream-K over 256 x 256 tiles (512 rows, K = 8192),
# stream-K over 128 x 256 tiles (256 x 4096 -> 8192),
# stream-K over the quarters of a last round with fewer quarters than CUs (512 x 4096: 32 tiles,
# all in that round; 2048 x 8448: 264 tiles, 256 whole and 8 cut into quarters). Each output is one dequantized weight, so every K
# step's scale and bias group, in the fast and the general form, is checked bit for bit.
@pytest.mark.parametrize("m,n,k", [(128, 4096, 2048), (1024, 8192, 2048), (2048, 8192, 2048), (512, 8192, 8192),
                                   (512, 4096, 2048), (2048, 8448, 2048), (256, 8192, 4096)])
@pytest.mark.parametrize("kind", ["fast", "mixed", "slow"])
def test_gemm_one_hot_is_exact_dequant(kind, m, n, k):
    note(f"GEMM one-hot {kind} {m}x{k}x{n}")
    rng = np.random.default_rng({"fast": 31, "mixed": 32, "slow": 33}[kind] + m)
    s, b = scale_bias_pairs(kind, n * (k // 64), rng)
    s, b = s.reshape(n, k // 64), b.reshape(n, k // 64)
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    deq = O.dequantize(w, s, b)
    wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
    for k0 in range(0, k, m):
        x = np.zeros((m, k), dtype=np.uint16)
        x[np.arange(m), k0 + np.arange(m)] = 0x3F80  # 1.0
        y = host_bits(quantized_matmul(bf16_dev(x), wd, sd, bd))
        ref = np.ascontiguousarray(deq[:, k0:k0 + m].T)
        keep = (ref & 0x7F80) != 0  # subnormal bf16 weights test the MFMA, not the dequant
        bad = keep & (O.bf16_bits_to_f32(y) != O.bf16_bits_to_f32(ref))
        assert not bad.any(), f"{int(bad.sum())} mismatches at k0={k0}, first {np.argwhere(bad)[:3].tolist()}"


@pytest.mark.parametrize("index,m", [(0, 16), (1, 1), (1, 2), (1, 4), (2, 64), (3, 32)])
def test_workload_full(index, m):
    note(f"workload {index} M={m}")
    x, w, s, b = O.config_inputs(index, m=m)
    y = gpu_qmm(x, w, s, b)
    check_qmm(y, workload_ref(x, w, s, b), f"c{index} M={m}", (x, w, s, b))


# One GPU's share of an 8-way column split (the path shards by output columns): the decode gate+up
# at 34816 / 8 = 4352 columns and the vocab head at 151936 / 8 = 18992 columns, which is not a
# multiple of 32 (a 16-column tail). The first and the last shard of the configs' own weights.
@pytest.mark.parametrize("index,m,shard", [(1, 1, 0), (1, 4, 7), (3, 32, 0), (3, 32, 7)])
def test_workload_one_gpu_share(index, m, shard):
    note(f"workload {index} M={m} shard {shard} of 8")
    x, w, s, b = O.config_inputs(index, m=m)
    ns = w.shape[0] // 8
    rows = slice(shard * ns, (shard + 1) * ns)
    w, s, b = w[rows], s[rows], b[rows]
    check_qmm(gpu_qmm(x, w, s, b), workload_ref(x, w, s, b), f"c{index} M={m} shard {shard}", (x, w, s, b))


# Shapes of the format that the packed kernels do not take (K % 128 != 0, N % 16 != 0): the
# reference leaves them to MLX's own op (packed_linear.py:84-86); here the HIP dequantization and a
# bf16 GEMM with fp32 accumulation, held to the same tolerance against the oracle.
# Every eligible linear of the target model (experiments/qmm_prefill.py:24-26: MLP gate/up and
# down, GDN in_proj_qkv / in_proj_z / out_proj, attention q / k,v / o), its lm_head
# (5120 -> 248320, tree_spec.py:645-677) and the drafter's head (N = 65984), at the row counts
# the forward passes use: decode (1-4), tree verify (16-64 nodes), prompt tails (128, 512).
# Inputs are drawn once per shape and sliced.
MODEL_LINEARS = [(5120, 17408), (17408, 5120), (5120, 10240), (5120, 6144), (6144, 5120), (5120, 12288),
                 (5120, 1024)]


@pytest.mark.parametrize("k,n,rows", [(k, n, (1, 4, 16, 48, 64, 96, 128, 512)) for k, n in MODEL_LINEARS]
                         + [(5120, 248320, (1, 4, 16, 32)), (5120, 65984, (1, 4, 6, 16, 32, 64))],
                         ids=lambda v: str(v) if not isinstance(v, tuple) else "rows")
def test_model_linear_shapes(k, n, rows):
    x, w, s, b = O.make_inputs(max(rows), k, n, seed=k + n)
    wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
    for m in rows:
        note(f"model linear {m}x{k}x{n}")
        xm = np.ascontiguousarray(x[:m])
        y = host_bits(quantized_matmul(bf16_dev(xm), wd, sd, bd))
        check_qmm(y, workload_ref(xm, w, s, b), f"model linear {m}x{k}x{n}", (xm, w, s, b))


# Shapes drawn at random (seeded; kept here as a list so the set does not depend on the generator's
# version): rows from each band the dispatcher distinguishes (decode 1-4, small verify 5-16, verify
# 17-64, mid 65-300), K any multiple of 128 up to 8192 (so K % 512 is often not 0: other unit
# sizes, the verify and skinny kernels, the GEMM's 2-byte scale loads), N any multiple of 16 up to
# 41600 (partial ranges, tiles and blocks everywhere), at most 1.2e9 multiply-adds each. Every route
# and plan the planners give these shapes must match the oracle and repeat its bits.
RANDOM_SHAPES = [(4, 1536, 1104), (3, 3072, 19440), (1, 3072, 26768), (2, 6912, 32896), (3, 7424, 30016),
                 (1, 7040, 27168), (1, 2560, 6896), (4, 6016, 38272), (2, 5248, 25136), (4, 1024, 21440),
                 (3, 6784, 27296), (2, 3840, 14096), (6, 2304, 6080), (7, 7040, 21888), (5, 3584, 11280),
                 (12, 6912, 544), (8, 1408, 8144), (9, 4992, 13600), (9, 5504, 12480), (16, 1792, 38912),
                 (11, 4992, 8608), (9, 3456, 37472), (5, 2688, 16992), (12, 3456, 13056), (17, 2176, 4400),
                 (17, 3072, 14928), (63, 3968, 1424), (17, 384, 33040), (31, 768, 7280), (31, 512, 10672),
                 (20, 896, 39408), (24, 256, 1568), (20, 5504, 2496), (33, 768, 3872), (31, 128, 35392),
                 (48, 640, 27440), (100, 640, 11840), (100, 256, 27296), (65, 3584, 3504), (100, 640, 4912),
                 (72, 128, 14688), (80, 384, 4736), (129, 1280, 5312), (112, 1152, 7648), (65, 384, 22736),
                 (160, 5376, 944), (65, 896, 11728), (256, 5376, 640)]


@pytest.mark.parametrize("m,k,n", RANDOM_SHAPES)
def test_random_shapes(m, k, n):
    note(f"random shape {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, sigma=0.5 if k > 6144 else 1.0, seed=m * 7919 + k * 31 + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"random {m}x{k}x{n}", (x, w, s, b))
    assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


@pytest.mark.parametrize("m,k,n", [(3, 192, 64), (70, 320, 48), (5, 128, 24), (1, 5120, 1000), (200, 64, 40)])
def test_qmm_general_shapes(m, k, n):
    note(f"general shape {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m + k + n)
    check_qmm(gpu_qmm(x, w, s, b), O.quantized_matmul_exact(x, w, s, b), f"general {m}x{k}x{n}", (x, w, s, b))


def test_quantized_linear_ineligible_module_falls_back():
    """A module the packed path does not take (K % 128 != 0, or a linear bias) still computes
    x @ dequant(w).T (+ bias), as the reference's _call does through MLX (packed_linear.py:84-86)."""
    from mlx_tree_spec_amd import STATS, QuantizedLinear, eligible
    x, w, s, b = O.make_inputs(6, 192, 96, seed=5)
    mod = QuantizedLinear.from_quantized(u32_dev(w), bf16_dev(s), bf16_dev(b))
    assert not eligible(mod)
    before = STATS["fallback"]
    y = host_bits(mod(bf16_dev(x)))
    assert STATS["fallback"] == before + 1
    check_qmm(y, O.quantized_matmul_exact(x, w, s, b), "ineligible module", (x, w, s, b))
    x2, w2, s2, b2 = O.make_inputs(4, 256, 64, seed=6)
    bias = torch.linspace(-1, 1, 64, device=DEV).to(torch.bfloat16)
    mb = QuantizedLinear.from_quantized(u32_dev(w2), bf16_dev(s2), bf16_dev(b2), bias=bias)
    assert not eligible(mb)
    got = O.bf16_bits_to_f32(host_bits(mb(bf16_dev(x2)))).astype(np.float64)
    ref = O.bf16_bits_to_f32(O.quantized_matmul(x2, w2, s2, b2)).astype(np.float64) + bias.float().cpu().numpy()
    assert O.max_rel(got, ref) <= O.MAX_REL_TOL


def general_inputs(m, k, n, bits, group_size, seed):
    """Inputs in one of the general path's formats: codes uniform over 0 .. 2^bits - 1, scales
    |N(0, 1)| * 0.004 + 1e-4 and biases centring the codes, as make_inputs draws the 4-bit ones."""
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    w = rng.integers(0, 2**32, size=(n, k * bits // 32), dtype=np.uint32)
    s = O.f32_to_bf16_bits((np.abs(rng.standard_normal((n, k // group_size))) * 0.004 + 1e-4).astype(np.float32))
    b = O.f32_to_bf16_bits((-(2.0 ** (bits - 1)) * O.bf16_bits_to_f32(s)
                            + rng.standard_normal((n, k // group_size)) * 1e-3).astype(np.float32))
    return x, w, s, b


GENERAL_FORMATS = [(2, 32), (2, 64), (2, 128), (4, 32), (4, 128), (8, 32), (8, 64), (8, 128)]


@pytest.mark.parametrize("bits,group_size", GENERAL_FORMATS)
def test_dequant_general_formats(bits, group_size):
    """2-, 4- and 8-bit codes in groups of 32, 64 or 128 (mx.dequantize's parameters; the general
    path of modules the packed kernels do not take, packed_linear.py:84-86): bit-exact against the
    oracle, whose decode and dequant are pinned against row bit strings and exact rationals."""
    note(f"dequant {bits}-bit group {group_size}")
    for n, k in ((96, 1024), (33, 4096)):
        _, w, s, b = general_inputs(1, k, n, bits, group_size, seed=bits * 1000 + group_size + k)
        got = host_bits(dequantize(u32_dev(w), bf16_dev(s), bf16_dev(b), group_size=group_size, bits=bits))
        assert np.array_equal(got, O.dequantize(w, s, b, group_size, bits)), (bits, group_size, n, k)


@pytest.mark.parametrize("bits,group_size", GENERAL_FORMATS)
def test_qmm_general_formats(bits, group_size):
    """quantized_matmul in the general formats (exact HIP dequantize, then a bf16 GEMM with fp32
    accumulation) against the fp32-accumulated oracle, at decode, verify and prefill rows."""
    for m, k, n in ((1, 1024, 256), (16, 2048, 320), (80, 512, 1024), (300, 1024, 512)):
        note(f"qmm {bits}-bit group {group_size} {m}x{k}x{n}")
        x, w, s, b = general_inputs(m, k, n, bits, group_size, seed=m + k + n + bits)
        y = host_bits(quantized_matmul(bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b),
                                       group_size=group_size, bits=bits))
        check_qmm(y, O.quantized_matmul_exact(x, w, s, b, group_size, bits), f"{bits}-bit g{group_size} {m}x{k}x{n}")


def test_quantized_linear_other_formats_fall_back():
    """An 8-bit (or 2-bit, or group-128) module is not eligible for the packed kernels and runs the
    general path, as the reference's _call sends it to MLX's op (packed_linear.py:84-86)."""
    from mlx_tree_spec_amd import STATS, QuantizedLinear, eligible
    for bits, group_size in ((8, 64), (2, 32), (4, 128)):
        x, w, s, b = general_inputs(5, 512, 192, bits, group_size, seed=bits + group_size)
        mod = QuantizedLinear.from_quantized(u32_dev(w), bf16_dev(s), bf16_dev(b), group_size=group_size, bits=bits)
        assert not eligible(mod) and mod.input_dims == 512
        before = STATS["fallback"]
        y = host_bits(mod(bf16_dev(x)))
        assert STATS["fallback"] == before + 1
        check_qmm(y, O.quantized_matmul_exact(x, w, s, b, group_size, bits), f"{bits}-bit g{group_size} module")


def test_workload_prefill_sampled_rows():
    """The 4096 x 5120 -> 17408 prefill GEMM on the GPU; 256 sampled rows against the oracle."""
    x, w, s, b = O.config_inputs(4)
    y = gpu_qmm(x, w, s, b)
    rows = np.random.default_rng(4).choice(x.shape[0], 256, replace=False)
    rows.sort()
    check_qmm(y[rows], workload_ref(x[rows], w, s, b), "c4 sampled rows", (x[rows], w, s, b))


@pytest.mark.parametrize("index,m", [(0, 16), (1, 4), (2, 64), (3, 32), (4, 4096)])
def test_workload_deterministic_and_pow2_linear(index, m):
    x, w, s, b = O.config_inputs(index, m=m)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y1 = host_bits(quantized_matmul(xd, wd, sd, bd))
    y2 = host_bits(quantized_matmul(xd, wd, sd, bd))
    assert np.array_equal(y1, y2)
    y2x = host_bits(quantized_matmul(xd * 2, wd, sd, bd))
    assert np.array_equal(O.bf16_bits_to_f32(y2x), 2 * O.bf16_bits_to_f32(y1))


# ----------------------------------------------------------------------------- row-split path
# Up to 4 rows with enough output columns to give every CU its own rows take the row-split
# kernel (one workgroup per CU owning whole weight rows). N = 34816 + 32 leaves the last
# workgroup a partial range and a half row block; K = 4096 gives units of 4 super-steps, 5120 of 5.
@pytest.mark.parametrize("m,k,n", [(1, 5120, 34848), (3, 4096, 34816), (4, 5120, 34816), (2, 4096, 34848)])
def test_rowsplit_shapes(m, k, n):
    note(f"row-split {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 7 + k + n)
    check_qmm(gpu_qmm(x, w, s, b), workload_ref(x, w, s, b), f"row-split {m}x{k}x{n}", (x, w, s, b))


# Up to 4 rows over an N too small for every CU to own 4 row blocks over all of K: K in 2 or 4
# slices per column range, the last workgroup of a range adding the slices' fp32 sums in slice
# order. 5120 x 17408 is the decode down projection; N = 5168 leaves a partial last range; K =
# 34816 with N = 4096 gives slices of 17408.
@pytest.mark.parametrize("m,k,n", [(1, 17408, 5120), (4, 17408, 5120), (2, 17408, 5168), (3, 34816, 4096)])
def test_rowsplit_k_slices(m, k, n):
    note(f"row-split K slices {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, sigma=0.5, seed=m * 13 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"row-split K slices {m}x{k}x{n}", (x, w, s, b))
    # deterministic whichever slice arrives last; the arrival counters are back at zero
    for _ in range(3):
        assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


# Up to 4 rows where no K split leaves every workgroup 3 units per wave and the columns give a CU
# fewer than 4 row blocks (12288 -> 5120: 2 blocks, 24 steps): whole K all the same.
@pytest.mark.parametrize("m", [1, 4])
def test_rowsplit_whole_k_fallback(m):
    k, n = 12288, 5120
    note(f"row-split whole-K fallback {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 31 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"row-split whole-K fallback {m}x{k}x{n}", (x, w, s, b))
    assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


def test_rowsplit_k_slices_one_hot_is_exact_dequant():
    """One-hot rows in the first and the second K slice: each output is one dequantized weight."""
    n, k, m = 5120, 17408, 4
    rng = np.random.default_rng(21)
    s, b = scale_bias_pairs("mixed", n * (k // 64), rng)
    s, b = s.reshape(n, k // 64), b.reshape(n, k // 64)
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
    for k0 in (0, 8700, 8704, k - m):
        ks = k0 + np.arange(m)
        x = np.zeros((m, k), dtype=np.uint16)
        x[np.arange(m), ks] = 0x3F80  # 1.0
        y = host_bits(quantized_matmul(bf16_dev(x), wd, sd, bd))
        ref = np.empty((m, n), dtype=np.uint16)
        for i, kk in enumerate(ks):
            g = kk // 64
            ref[i] = O.dequantize(w[:, 8 * g:8 * g + 8], s[:, g:g + 1], b[:, g:g + 1])[:, kk - 64 * g]
        keep = (ref & 0x7F80) != 0
        bad = keep & (O.bf16_bits_to_f32(y) != O.bf16_bits_to_f32(ref))
        assert not bad.any(), f"{int(bad.sum())} mismatches at k0={k0}"


@pytest.mark.parametrize("kind", ["fast", "mixed", "slow"])
def test_rowsplit_one_hot_is_exact_dequant(kind):
    """One-hot rows of x on the row-split path: each output is one dequantized weight and must
    equal the oracle's bit for bit, for units dequantized in the fast form, in the general form
    ('slow'), and for a mix of the two."""
    n, k, m = 34848, 5120, 4
    rng = np.random.default_rng({"fast": 11, "mixed": 12, "slow": 13}[kind])
    s, b = scale_bias_pairs(kind, n * (k // 64), rng)
    s, b = s.reshape(n, k // 64), b.reshape(n, k // 64)
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
    for k0 in (0, 1276, 5116):
        ks = k0 + np.arange(m)
        x = np.zeros((m, k), dtype=np.uint16)
        x[np.arange(m), ks] = 0x3F80  # 1.0
        y = host_bits(quantized_matmul(bf16_dev(x), wd, sd, bd))
        ref = np.empty((m, n), dtype=np.uint16)
        for i, kk in enumerate(ks):
            g = kk // 64
            ref[i] = O.dequantize(w[:, 8 * g:8 * g + 8], s[:, g:g + 1], b[:, g:g + 1])[:, kk - 64 * g]
        keep = (ref & 0x7F80) != 0  # subnormal bf16 weights test the MFMA, not the dequant
        bad = keep & (O.bf16_bits_to_f32(y) != O.bf16_bits_to_f32(ref))
        assert not bad.any(), f"{int(bad.sum())} mismatches at k0={k0}, first {np.argwhere(bad)[:3].tolist()}"


# Small problems: 6-8 rows over at most one row block per CU (every unit in a wave's ring from the
# start, all of x in LDS) take the row-split kernel's SMALL form: N = 1024 (4 live rows per 16-row
# block), 4096, 2048 at K = 8192 (x of 8 rows is 128 KB of LDS). 1-5 rows over small N take whole
# K in the regular form (N = 1024; 5120 with 2 row blocks per CU; 4112, a partial last range).
@pytest.mark.parametrize("m,k,n", [(6, 5120, 1024), (8, 5120, 1024), (7, 2048, 4096), (8, 8192, 2048),
                                   (1, 5120, 1024), (4, 5120, 5120), (5, 5120, 5120), (3, 2048, 4112)])
def test_rowsplit_small_shapes(m, k, n):
    note(f"row-split small {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 11 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"row-split small {m}x{k}x{n}", (x, w, s, b))
    assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


# 5 to 8 rows: x rows in two lane groups of the MFMA, whole K (N = 34848 leaves a partial last
# range), the small form with x filling all 160 KB of LDS (6 x 10240 over N = 4096), and K in two
# slices (8 x 10240 over N = 5168: 30 units per workgroup over a whole-K x that does not fit).
@pytest.mark.parametrize("m,k,n", [(5, 5120, 34848), (8, 4096, 34816), (6, 10240, 4096), (8, 10240, 5168)])
def test_rowsplit_eight_row_shapes(m, k, n):
    note(f"row-split 8-row {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 17 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"row-split 8-row {m}x{k}x{n}", (x, w, s, b))
    for _ in range(2):
        assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


# 9 to 16 rows beyond the x-in-registers form's reach: the row-split kernel with 16-row fragments,
# x in LDS in up to 4 K slices (the MLP up projection at 9 and 16 rows: 2 slices; 12 rows over
# 34816 columns: 2 slices of 5-step units; K = 2048 over 16384 columns: the small form; K = 6144).
@pytest.mark.parametrize("m,k,n", [(9, 5120, 17408), (16, 5120, 17408), (12, 5120, 34816), (16, 5120, 10240),
                                   (16, 2048, 16384), (13, 6144, 5120)])
def test_rowsplit_sixteen_row_shapes(m, k, n):
    note(f"row-split 16-row {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 23 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"row-split 16-row {m}x{k}x{n}", (x, w, s, b))
    for _ in range(2):
        assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


# Whole K with units taken in groups (consecutive steps of a block summed into one LDS slot) where
# one slot per step does not fit: pairs for 1-4 rows over the 248320-column vocabulary head (61
# blocks x 10 steps per CU; N = 248336 leaves a partial last range), 6 rows over the 65984-column
# head (8-row fragments), 2 rows at K = 4096 (8 steps per block); groups of 5 for 5-8 rows over
# the 248320- and 151936-column heads (x of 8 rows leaves room for 2 slots per block).
@pytest.mark.parametrize("m,k,n", [(3, 5120, 248336), (6, 5120, 65984), (2, 4096, 262144), (5, 5120, 248320),
                                   (8, 5120, 151936)])
def test_rowsplit_paired_units(m, k, n):
    note(f"row-split paired units {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 29 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"row-split paired units {m}x{k}x{n}", (x, w, s, b))
    for _ in range(2):
        assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


# Whole K where no grouping of slots fits but all of x does, with at least two blocks per wave:
# each wave owns whole blocks and keeps their sums in registers. 9-16 rows over the 248320-column
# vocabulary head (61 blocks per CU; 16 rows fill all 160 KB of LDS with x), N = 248336 (a partial
# last range), 12 rows over the 151936-column head, 131072 columns (32 blocks per CU), K = 4096.
@pytest.mark.parametrize("m,k,n", [(16, 5120, 248336), (12, 5120, 151936), (16, 5120, 131072), (9, 4096, 262144)])
def test_rowsplit_own_blocks(m, k, n):
    note(f"row-split own blocks {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 37 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"row-split own blocks {m}x{k}x{n}", (x, w, s, b))
    for _ in range(2):
        assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


@pytest.mark.parametrize("kind", ["fast", "mixed", "slow"])
@pytest.mark.parametrize("m,n", [(8, 5120), (3, 1024), (6, 1024), (8, 34848), (16, 17408), (12, 34816),
                                 (2, 248320), (6, 65984), (16, 248320), (7, 151936)])
def test_rowsplit_small_and_eight_row_one_hot_is_exact_dequant(kind, m, n):
    """One-hot rows of x through the small form, the 8- and 16-row fragments, paired units and
    waves owning whole blocks: each output is one dequantized weight, equal to the oracle's bit for
    bit (fast form, general form, both)."""
    k = 5120
    rng = np.random.default_rng({"fast": 31, "mixed": 32, "slow": 33}[kind] + n + m)
    s, b = scale_bias_pairs(kind, n * (k // 64), rng)
    s, b = s.reshape(n, k // 64), b.reshape(n, k // 64)
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
    for k0 in (0, 2555, 5120 - m):
        ks = k0 + np.arange(m)
        x = np.zeros((m, k), dtype=np.uint16)
        x[np.arange(m), ks] = 0x3F80  # 1.0
        y = host_bits(quantized_matmul(bf16_dev(x), wd, sd, bd))
        ref = np.empty((m, n), dtype=np.uint16)
        for i, kk in enumerate(ks):
            g = kk // 64
            ref[i] = O.dequantize(w[:, 8 * g:8 * g + 8], s[:, g:g + 1], b[:, g:g + 1])[:, kk - 64 * g]
        keep = (ref & 0x7F80) != 0  # subnormal bf16 weights test the MFMA, not the dequant
        bad = keep & (O.bf16_bits_to_f32(y) != O.bf16_bits_to_f32(ref))
        assert not bad.any(), f"{int(bad.sum())} mismatches at k0={k0}, first {np.argwhere(bad)[:3].tolist()}"


# 9 to 16 rows over at most 32 weight rows per CU with K <= 6144: the row-split form with x loaded
# straight into registers, one wave per 512-k chunk. 16 x 5120 over 5120 columns (c0: 20 rows per
# workgroup, a half-live second block), 12 rows over 2048 (8 rows per workgroup), N = 8208 (a partial
# last range), 9 rows (fragment rows 9-15 repeat row 8).
@pytest.mark.parametrize("m,k,n", [(16, 5120, 5120), (12, 4096, 2048), (16, 2048, 8208), (9, 5120, 1024)])
def test_rowsplit_xreg_shapes(m, k, n):
    note(f"row-split x-in-registers {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 23 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"row-split xreg {m}x{k}x{n}", (x, w, s, b))
    assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


@pytest.mark.parametrize("kind", ["fast", "mixed", "slow"])
def test_rowsplit_xreg_one_hot_is_exact_dequant(kind):
    """One-hot rows of x through the x-in-registers form: single dequantized weights, bit for bit."""
    m, k, n = 16, 5120, 5120
    rng = np.random.default_rng({"fast": 41, "mixed": 42, "slow": 43}[kind])
    s, b = scale_bias_pairs(kind, n * (k // 64), rng)
    s, b = s.reshape(n, k // 64), b.reshape(n, k // 64)
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
    for k0 in (0, 2550, 5120 - m):
        ks = k0 + np.arange(m)
        x = np.zeros((m, k), dtype=np.uint16)
        x[np.arange(m), ks] = 0x3F80  # 1.0
        y = host_bits(quantized_matmul(bf16_dev(x), wd, sd, bd))
        ref = np.empty((m, n), dtype=np.uint16)
        for i, kk in enumerate(ks):
            g = kk // 64
            ref[i] = O.dequantize(w[:, 8 * g:8 * g + 8], s[:, g:g + 1], b[:, g:g + 1])[:, kk - 64 * g]
        keep = (ref & 0x7F80) != 0  # subnormal bf16 weights test the MFMA, not the dequant
        bad = keep & (O.bf16_bits_to_f32(y) != O.bf16_bits_to_f32(ref))
        assert not bad.any(), f"{int(bad.sum())} mismatches at k0={k0}, first {np.argwhere(bad)[:3].tolist()}"


# ----------------------------------------------------------------------------- row-phase path
# More than 16 rows (or up to 16 when N gives every wave its own blocks) take the row-phase kernel
# (K a multiple of 512). Wide shapes give each workgroup whole rows over all of K (N = 16 * 2049
# leaves the last range a partial one); narrow ones split K over the workgroups of a block range.
# K = 3072 ends in a partial scale window. 65984 columns (the drafter's head) give a workgroup 17
# blocks (the 3-blocks-per-wave variants), 99984 and 131072 columns 25 and 32 blocks (4 per wave).
# 24 rows over 5120 -> 17408: K split over ranges of 3 blocks per wave (46 ranges x 5 slices).
# Ranges of one block per wave where two would leave a workgroup at most 3 phases: 12 x 17408 ->
# 5120 (40 ranges x 6 slices of 6 phases), 48 x 6144 -> 5120 (4 phases), 32 x 2048 -> 8192.
@pytest.mark.parametrize("m,k,n", ROWPHASE_SHAPES)
def test_rowphase_shapes(m, k, n):
    note(f"row-phase {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 11 + k + n)
    check_qmm(gpu_qmm(x, w, s, b), workload_ref(x, w, s, b), f"row-phase {m}x{k}x{n}", (x, w, s, b))


# Wide row-phase plans whose blocks leave most waves a block short take variants that skip the
# last slot's arithmetic in those waves (route_cases.ROWPHASE_WIDE_CASES; the variant of each case
# is checked against the planner in tests/test_plans.py).
@pytest.mark.parametrize("m,n,k,form", ROWPHASE_WIDE_CASES)
def test_rowphase_wide_shapes(m, n, k, form):
    note(f"row-phase wide ({form}) {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, seed=m * 17 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"row-phase wide {m}x{k}x{n}", (x, w, s, b))
    assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


@pytest.mark.parametrize("n,m,k", ROWPHASE_ONE_HOT)
@pytest.mark.parametrize("kind", ["fast", "mixed", "slow"])
def test_rowphase_one_hot_is_exact_dequant(kind, n, m, k):
    """One-hot rows of x on the row-phase path (wide and K-split): each output is one dequantized
    weight and must equal the oracle's bit for bit, for scale windows dequantized in the fast
    form, in the general form, and for a mix of the two. 32800 / 33024 columns at 32 / 48 rows,
    65984 at 16, 32 and 64 rows and 34816 at 72 and 96 rows take the wide variants whose short
    waves skip the last block slot."""
    rng = np.random.default_rng({"fast": 21, "mixed": 22, "slow": 23}[kind] + n)
    s, b = scale_bias_pairs(kind, n * (k // 64), rng)
    s, b = s.reshape(n, k // 64), b.reshape(n, k // 64)
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
    for k0 in (0, 1000, k - m):
        ks = k0 + np.arange(m)
        x = np.zeros((m, k), dtype=np.uint16)
        x[np.arange(m), ks] = 0x3F80  # 1.0
        y = host_bits(quantized_matmul(bf16_dev(x), wd, sd, bd))
        ref = np.empty((m, n), dtype=np.uint16)
        for i, kk in enumerate(ks):
            g = kk // 64
            ref[i] = O.dequantize(w[:, 8 * g:8 * g + 8], s[:, g:g + 1], b[:, g:g + 1])[:, kk - 64 * g]
        keep = (ref & 0x7F80) != 0  # subnormal bf16 weights test the MFMA, not the dequant
        bad = keep & (O.bf16_bits_to_f32(y) != O.bf16_bits_to_f32(ref))
        assert not bad.any(), f"{int(bad.sum())} mismatches at k0={k0}, first {np.argwhere(bad)[:3].tolist()}"


# 65-128 rows (a verify batch past 64 tree nodes, a short prompt tail): the row-phase kernel with
# 80-128-row x blocks where its plan is narrow, else the GEMM (route_cases.MID_ROW_CASES; the routes
# are checked against the planner in tests/test_plans.py).
@pytest.mark.parametrize("m,n,k,route", MID_ROW_CASES)
def test_mid_rows(m, n, k, route):
    note(f"{route} {m}x{k}x{n}")
    x, w, s, b = O.make_inputs(m, k, n, sigma=0.5 if k > 6144 else 1.0, seed=m * 13 + k + n)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = host_bits(quantized_matmul(xd, wd, sd, bd))
    check_qmm(y, workload_ref(x, w, s, b), f"{route} {m}x{k}x{n}", (x, w, s, b))
    assert np.array_equal(host_bits(quantized_matmul(xd, wd, sd, bd)), y)


# Scale windows of the row-phase kernel are 32 groups (2048 values of k) of every row. Odd windows
# here hold scales that need the general form, even windows only fast-form scales, so a workgroup
# whose phases cross windows switches form at each window: wide ranges of 20 and 12 phases over 3
# and 2 windows (12 rows over 65552 columns on the one-row-block twin that skips short waves' last
# slot; 48 rows over 33024 with windows loaded a phase ahead), the K-split batched-verify shape
# (ranges of 5-6 phases, some across a window edge), a wide 32-row shape whose variant stages each
# window at its first phase (5 blocks per wave leave no registers for a window ahead), and 96 rows
# (two x stages).
@pytest.mark.parametrize("m,k,n", ROWPHASE_WINDOW_CASES)
def test_rowphase_window_form_switches(m, k, n):
    note(f"row-phase window switches {m}x{k}x{n}")
    rng = np.random.default_rng(m * 7 + k)
    groups = k // 64
    s, b = scale_bias_pairs("fast", n * groups, rng)
    sl, bl = scale_bias_pairs("slow", n * groups, rng)
    s, b, sl, bl = (a.reshape(n, groups) for a in (s, b, sl, bl))
    odd = ((np.arange(groups) // 32) % 2 == 1)[None, :]
    s, b = np.where(odd, sl, s), np.where(odd, bl, b)
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    wd, sd, bd = u32_dev(w), bf16_dev(s), bf16_dev(b)
    for win in range((k + 2047) // 2048):
        k0 = min(2048 * win + 1000, k - m)
        ks = k0 + np.arange(m)
        x = np.zeros((m, k), dtype=np.uint16)
        x[np.arange(m), ks] = 0x3F80  # 1.0
        y = host_bits(quantized_matmul(bf16_dev(x), wd, sd, bd))
        ref = np.empty((m, n), dtype=np.uint16)
        for i, kk in enumerate(ks):
            g = kk // 64
            ref[i] = O.dequantize(w[:, 8 * g:8 * g + 8], s[:, g:g + 1], b[:, g:g + 1])[:, kk - 64 * g]
        keep = (ref & 0x7F80) != 0  # subnormal bf16 weights test the MFMA, not the dequant
        bad = keep & (O.bf16_bits_to_f32(y) != O.bf16_bits_to_f32(ref))
        assert not bad.any(), f"{int(bad.sum())} mismatches in window {win}, first {np.argwhere(bad)[:3].tolist()}"


# ----------------------------------------------------------------------------- host integration
def test_side_stream_and_workspace_growth():
    cases = [O.make_inputs(16, 5120, 512, seed=1), O.make_inputs(64, 17408, 1024, seed=2), O.make_inputs(3, 256, 64, seed=3)]
    side = torch.cuda.Stream()
    for x, w, s, b in cases + cases[::-1]:
        ref = O.quantized_matmul_exact(x, w, s, b)
        check_qmm(gpu_qmm(x, w, s, b), ref, "default stream", (x, w, s, b))
        with torch.cuda.stream(side):
            y = quantized_matmul(bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b))
        side.synchronize()
        check_qmm(host_bits(y), ref, "side stream", (x, w, s, b))


def test_noncontiguous_and_empty():
    x, w, s, b = O.make_inputs(8, 256, 64, seed=9)
    xbig = bf16_dev(np.concatenate([x, x], axis=1))
    xv = xbig[:, 256:]  # non-contiguous view
    y = quantized_matmul(xv, u32_dev(w), bf16_dev(s), bf16_dev(b))
    check_qmm(host_bits(y), O.quantized_matmul_exact(x, w, s, b), "strided x", (x, w, s, b))
    y0 = quantized_matmul(bf16_dev(x[:0]), u32_dev(w), bf16_dev(s), bf16_dev(b))
    assert tuple(y0.shape) == (0, 64)


def test_quantized_linear_install():
    """The prebound launcher of install() against the oracle (not only against the library's own
    unbound call), at decode, verify and prefill row counts."""
    k, n = 1024, 256
    mods, wts = [], []
    for seed in range(3):
        _, w, s, b = O.make_inputs(1, k, n, seed=seed)
        mods.append(QuantizedLinear.from_quantized(u32_dev(w), bf16_dev(s), bf16_dev(b)))
        wts.append((w, s, b))
    model = torch.nn.Sequential(*mods)
    summary = install(model, verbose=False)
    assert summary["packed"] == 3
    assert all("_fast" in m.__dict__ for m in mods)
    for m in (1, 16, 100):
        x, *_ = O.make_inputs(m, k, n, seed=m)
        xd = bf16_dev(x).reshape(1, m, k)
        for i in (0, 2):
            before = dict(STATS)
            y = mods[i](xd)
            key = "skinny" if m <= 64 else "gemm"
            assert STATS[key] == before.get(key, 0) + 1
            assert STATS["rebound"] == before.get("rebound", 0)
            assert tuple(y.shape) == (1, m, n)
            check_qmm(host_bits(y).reshape(m, n), O.quantized_matmul_exact(x, *wts[i]), f"install M={m} mod={i}",
                      (x, *wts[i]))
            ref = quantized_matmul(xd, mods[i].weight, mods[i].scales, mods[i].biases)
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


def test_install_rebinds_replaced_buffers():
    """A launcher whose module's buffers were replaced after install() rebinds to the new ones (no
    read of the freed tensors), and a dtype the kernels cannot take raises."""
    k, n = 512, 128
    _, w, s, b = O.make_inputs(1, k, n, seed=21)
    mod = QuantizedLinear.from_quantized(u32_dev(w), bf16_dev(s), bf16_dev(b))
    install(mod, verbose=False)
    x, *_ = O.make_inputs(4, k, n, seed=22)
    check_qmm(host_bits(mod(bf16_dev(x))), O.quantized_matmul_exact(x, w, s, b), "bound", (x, w, s, b))
    _, w2, s2, b2 = O.make_inputs(1, k, n, seed=23)
    mod.weight, mod.scales, mod.biases = u32_dev(w2), bf16_dev(s2), bf16_dev(b2)
    torch.cuda.synchronize()
    before = STATS["rebound"]
    check_qmm(host_bits(mod(bf16_dev(x))), O.quantized_matmul_exact(x, w2, s2, b2), "rebound", (x, w2, s2, b2))
    assert STATS["rebound"] == before + 1 and "_fast" in mod.__dict__
    mod.to(torch.float32)  # scales and biases become fp32 tensors
    with pytest.raises(ValueError):
        mod(bf16_dev(x))


def test_misaligned_contiguous_inputs():
    """Contiguous views that start 2 bytes past a 16-byte boundary (accepted by MLX) are copied to
    aligned storage by the Python layer instead of being rejected by the C ABI."""
    m, k, n = 5, 1024, 256
    x, w, s, b = O.make_inputs(m, k, n, seed=31)
    xs = bf16_dev(np.concatenate([np.zeros(1, np.uint16), x.reshape(-1)]))[1:].view(m, k)
    ss = bf16_dev(np.concatenate([np.zeros(1, np.uint16), s.reshape(-1)]))[1:].view(n, k // 64)
    bs = bf16_dev(np.concatenate([np.zeros(1, np.uint16), b.reshape(-1)]))[1:].view(n, k // 64)
    assert xs.is_contiguous() and xs.data_ptr() % 16 == 2 and ss.data_ptr() % 16 == 2
    y = quantized_matmul(xs, u32_dev(w), ss, bs)
    check_qmm(host_bits(y), O.quantized_matmul_exact(x, w, s, b), "misaligned", (x, w, s, b))
    from mlx_tree_spec_amd import add_rms_norm_
    wn = bf16_dev(np.full(k, 0x3F80, np.uint16))
    h, nn = add_rms_norm_(xs, xs, wn, 1e-6)
    ho, no = O.add_rms_norm(x, x, np.full(k, 0x3F80, np.uint16), 1e-6)
    assert np.array_equal(host_bits(h), ho)


def test_capture_needs_existing_workspace():
    """Under graph capture a call that would have to allocate its split-K workspace returns
    QMM4_ERR_CAPTURE; after one eager call on the stream the same call captures and replays."""
    from mlx_tree_spec_amd import _lib
    m, n, k = 32, 1024, 5120  # the row-phase kernel with K split 20 ways: partial tiles in the workspace
    x, w, s, b = O.make_inputs(m, k, n, seed=41)
    xd, wd, sd, bd = bf16_dev(x), u32_dev(w), bf16_dev(s), bf16_dev(b)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    lib = _lib.load()
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    rc = None
    try:
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")  # the refused call leaves the captured graph empty
            with torch.cuda.graph(g, stream=st):
                rc = lib.qmm4_affine_bf16(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
                                          y.data_ptr(), m, n, k, 64, 4, 1, st.cuda_stream)
    except RuntimeError:
        pass  # an empty or invalidated capture may fail to instantiate
    assert rc == _lib.QMM4_ERR_CAPTURE, rc
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        assert lib.qmm4_affine_bf16(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), y.data_ptr(),
                                    m, n, k, 64, 4, 1, st.cuda_stream) == 0
    st.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        assert lib.qmm4_affine_bf16(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), y.data_ptr(),
                                    m, n, k, 64, 4, 1, st.cuda_stream) == 0
    ref = O.quantized_matmul_exact(x, w, s, b)
    for rep in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        check_qmm(host_bits(y), ref, f"captured replay {rep}", (x, w, s, b))
