"""CPU oracle for the packed 4-bit affine quantized matmul (MLX format) — TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only as the reference results are checked against: the product path (mlx-tree-spec_amd/) never calls it and fails loudly when
its HIP library is missing.

Restates, in numpy, the reference's arithmetic for the path:
  * codes:    q[n, 8c+i] = (w[n, c] >> 4i) & 0xF                 src/mlx_tree_spec/qmm_packed.py:115, 200-201
              (2- and 8-bit codes, the general path's other whole-word formats, in the same order)
  * groups:   g = k // 64, scales/biases bf16 [N, K/64]          qmm_packed.py:454, 630
  * dequant:  bf16_rne(fp32(s) * q + fp32(b))                    qmm_packed.py:200-201, 348-349, 635-636
  * matmul:   y = fp32(x) @ fp32(dequant(w)).T, bf16 out         tests/test_units.py:108 ("exact")
  * metrics:  max|y-ref| / max|ref|                              experiments/qmm_prefill.py:98
  * layouts:  pack_nax / its inverse                            qmm_packed.py:223-232, packed_linear.py:72-80
  * synthetic inputs of the five benchmark workloads (seeded PCG64; draw order fixed here).

bf16 values are carried as raw uint16 bit patterns throughout, so nothing here depends on a
bfloat16 dtype. How each function is pinned (golden vectors from an independent exact-arithmetic
brute force, closed forms, torch's own bf16 conversion, invariants) is listed in tests/test_oracle.py.
"""

from __future__ import annotations

import numpy as np

GROUP_SIZE = 64
BITS = 4


# ----------------------------------------------------------------------------- bf16 bit helpers
def f32_to_bf16_bits(a) -> np.ndarray:
    """Round fp32 values to bf16 (round to nearest, ties to even); NaN -> 0x7FC0 with its sign."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = np.isnan(a)
    if nan.any():
        r = np.where(nan, ((u >> 16).astype(np.uint32) & 0x8000) | 0x7FC0, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(u) -> np.ndarray:
    """bf16 bit patterns -> exact fp32 values."""
    u = np.asarray(u, dtype=np.uint16)
    return (u.astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- format
def unpack_codes(w, bits: int = BITS) -> np.ndarray:
    """uint32 [N, K * bits / 32] -> uint8 codes [N, K]; code k = (32 / bits) c + i sits in bits
    [bits i, bits i + bits) of word c (4 bits: qmm_packed.py:115, 200-201; 2 and 8 bits, the formats
    MLX packs into whole words, the same little-endian order)."""
    assert bits in (2, 4, 8)
    per = 32 // bits
    w = np.asarray(w, dtype=np.uint32)
    n, kw = w.shape
    shifts = (bits * np.arange(per, dtype=np.uint32))[None, None, :]
    q = (w[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return q.reshape(n, kw * per).astype(np.uint8)


def pack_codes(q, bits: int = BITS) -> np.ndarray:
    """uint8 codes [N, K] (values below 2^bits) -> uint32 [N, K * bits / 32]; inverse of unpack_codes."""
    assert bits in (2, 4, 8)
    per = 32 // bits
    q = np.asarray(q, dtype=np.uint32)
    n, k = q.shape
    assert k % per == 0
    q = q.reshape(n, k // per, per)
    w = np.zeros((n, k // per), dtype=np.uint32)
    for i in range(per):
        w |= (q[:, :, i] & np.uint32((1 << bits) - 1)) << np.uint32(bits * i)
    return w


def dequantize(w, scales, biases, group_size: int = GROUP_SIZE, bits: int = BITS) -> np.ndarray:
    """bf16 bits [N, K] of bf16_rne(fp32_rne(s * q + b)), s * q + b taken exactly (FMA semantics).

    s * q has at most 16 significant bits (8-bit codes), so it is exact in float64 (and float64
    has the exponent range to hold it even where it would overflow fp32 while s * q + b does not).
    The float64 sum is then rounded to fp32: rounding a sum of two values with <= 24-bit
    significands first to float64 and then to fp32 equals rounding it once to fp32 (53 >= 2*24 + 2).
    bits 2, 4 or 8; group_size 32, 64 or 128.
    """
    assert bits in (2, 4, 8) and group_size in (32, 64, 128)
    q = unpack_codes(w, bits).astype(np.float64)
    n, k = q.shape
    s = np.repeat(bf16_bits_to_f32(scales).astype(np.float64), group_size, axis=1)
    b = np.repeat(bf16_bits_to_f32(biases).astype(np.float64), group_size, axis=1)
    assert s.shape == (n, k) and b.shape == (n, k)
    with np.errstate(over="ignore", invalid="ignore"):
        v = (q * s + b).astype(np.float32)
    return f32_to_bf16_bits(v)


def quantized_matmul_exact(x, w, scales, biases, group_size: int = GROUP_SIZE, bits: int = BITS) -> np.ndarray:
    """The fp32-accumulated reference y = fp32(x) @ fp32(dequant(w)).T, computed in float64.

    x: bf16 bits [..., K]. Returns float64 [..., N] (not rounded to bf16).
    """
    x = np.asarray(x, dtype=np.uint16)
    k = x.shape[-1]
    wd = bf16_bits_to_f32(dequantize(w, scales, biases, group_size, bits)).astype(np.float64)
    assert wd.shape[1] == k
    xf = bf16_bits_to_f32(x.reshape(-1, k)).astype(np.float64)
    y = xf @ wd.T
    return y.reshape(*x.shape[:-1], wd.shape[0])


def quantized_matmul(x, w, scales, biases, transpose: bool = True, group_size: int = GROUP_SIZE,
                     bits: int = BITS) -> np.ndarray:
    """bf16 bits of y = x @ dequant(w).T with fp32-exact accumulation, rounded once to bf16."""
    assert transpose
    y = quantized_matmul_exact(x, w, scales, biases, group_size, bits)
    return f32_to_bf16_bits(y.astype(np.float32))


# ----------------------------------------------------------------------------- residual + RMS norm
def add_rms_norm(x, r, weight, eps: float):
    """bf16 bits (h, n), each [rows, D], of the residual add fused with the RMS norm after it
    (fused_ops.py:107-128): h = bf16(x + r); inv = 1 / sqrt(sum(h*h) / D + eps);
    n = bf16(w * bf16(h * inv)). The row sum is taken in float64 and rounded to fp32 (the
    reference's own fp32 summation order, a simdgroup reduction, is not reproducible: its last bit
    is parity unpinned); the mean, sqrt and reciprocal are correctly rounded fp32 operations."""
    x = np.asarray(x, dtype=np.uint16)
    d = x.shape[-1]
    h = f32_to_bf16_bits(bf16_bits_to_f32(x) + bf16_bits_to_f32(r))
    hf = bf16_bits_to_f32(h)
    ss = (hf.astype(np.float64) ** 2).sum(-1).astype(np.float32)
    inv = (np.float32(1.0) / np.sqrt(ss / np.float32(d) + np.float32(eps))).astype(np.float32)
    nh = f32_to_bf16_bits(hf * inv[..., None])
    n = f32_to_bf16_bits(bf16_bits_to_f32(weight) * bf16_bits_to_f32(nh))
    return h, n


# ----------------------------------------------------------------------------- MLP epilogue
def silu_mul(g, u) -> np.ndarray:
    """bf16 bits of silu(g) * u for bf16 bits g, u, one bf16 rounding per operation as the unfused
    MLP evaluates it on bf16 arrays (tree_verify.py:446: down_proj(silu(gate_proj(x)) *
    up_proj(x)); silu(x) = x * sigmoid(x)):  s = bf16(sigmoid(g)), t = bf16(g * s), bf16(t * u).
    sigmoid is evaluated in fp32 as 1 / (1 + exp(-g)). (MLX's own kernels for these elementwise
    ops are not in the reference: their last-ulp rounding of the sigmoid is parity unpinned; this
    restatement fixes one.)"""
    gf = bf16_bits_to_f32(g)
    with np.errstate(over="ignore"):
        sg = (np.float32(1.0) / (np.float32(1.0) + np.exp(-gf))).astype(np.float32)
    s = bf16_bits_to_f32(f32_to_bf16_bits(sg))
    t = bf16_bits_to_f32(f32_to_bf16_bits(gf * s))
    return f32_to_bf16_bits(t * bf16_bits_to_f32(u))


def gate_up_silu(x, w, scales, biases, group_size: int = GROUP_SIZE, bits: int = BITS) -> np.ndarray:
    """bf16 bits [M, N/2] of silu(x @ w_gate.T) * (x @ w_up.T), w = [w_gate; w_up]: each half rounded
    to bf16 as its own projection would store it, then silu_mul."""
    y = quantized_matmul(x, w, scales, biases, True, group_size, bits)
    h = y.shape[-1] // 2
    return silu_mul(y[..., :h], y[..., h:])


# ----------------------------------------------------------------------------- metrics
def max_rel(y, ref) -> float:
    """max|y - ref| / max|ref| (experiments/qmm_prefill.py:98)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / np.abs(ref).max())


def mean_rel(y, ref) -> float:
    """mean|y - ref| / mean|ref|."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).mean() / np.abs(ref).mean())


def rel_l2(y, ref) -> float:
    """||y - ref|| / ||ref|| (bench/ane/split_accuracy.py:50)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(y - ref) / np.linalg.norm(ref))


MAX_REL_TOL = 1e-2
MEAN_REL_TOL = 2e-3


# ----------------------------------------------------------------------------- layouts
def pack_nax(w, scales, biases):
    """The reference's relayout (qmm_packed.py:223-232): 32-row tiles, 16-wide K blocks.

    wq2[t][kb][r][j] = w[32t + r][2kb + j]; sp2[t][g][r] = s[32t + r][g] (same for biases).
    Returns flat arrays, like the reference.
    """
    w = np.asarray(w)
    n, kw = w.shape
    assert n % 32 == 0 and kw % 2 == 0
    wq2 = np.ascontiguousarray(w.reshape(n // 32, 32, kw // 2, 2).transpose(0, 2, 1, 3)).reshape(-1)
    g = np.asarray(scales).shape[1]
    sp2 = np.ascontiguousarray(np.asarray(scales).reshape(n // 32, 32, g).transpose(0, 2, 1)).reshape(-1)
    bp2 = np.ascontiguousarray(np.asarray(biases).reshape(n // 32, 32, g).transpose(0, 2, 1)).reshape(-1)
    return wq2, sp2, bp2


def unpack_nax(wq2, sp2, bp2, n: int):
    """Inverse of pack_nax (packed_linear._unpacked, packed_linear.py:72-80)."""
    kw = wq2.size // n
    g = sp2.size // n
    w = np.asarray(wq2).reshape(n // 32, kw // 2, 32, 2).transpose(0, 2, 1, 3).reshape(n, kw)
    s = np.asarray(sp2).reshape(n // 32, g, 32).transpose(0, 2, 1).reshape(n, g)
    b = np.asarray(bp2).reshape(n // 32, g, 32).transpose(0, 2, 1).reshape(n, g)
    return np.ascontiguousarray(w), np.ascontiguousarray(s), np.ascontiguousarray(b)


# ----------------------------------------------------------------------------- synthetic inputs
# The five benchmark workloads (decode/verify/vocab/prefill shapes of the 27B target model).
CONFIGS = {
    0: dict(name="tree-verify qmm 16x5120->5120", M=(16,), K=5120, N=5120, sigma=1.0),
    1: dict(name="decode gate+up 1,2,4x5120->34816", M=(1, 2, 4), K=5120, N=34816, sigma=1.0),
    2: dict(name="batched verify down 64x17408->5120", M=(64,), K=17408, N=5120, sigma=0.5),
    3: dict(name="vocab head 32x5120->151936", M=(32,), K=5120, N=151936, sigma=1.0),
    4: dict(name="chunked prefill 4096x5120->17408", M=(4096,), K=5120, N=17408, sigma=1.0),
}


def make_inputs(m: int, k: int, n: int, sigma: float = 1.0, seed: int = 0):
    """Seeded synthetic inputs: x ~ N(0, sigma^2) -> bf16; packed words uniform over uint32 (every
    code iid uniform 0..15); scales = bf16(|N(0,1)|*0.004 + 1e-4); biases = bf16(-8*s + N(0,1)*1e-3).
    Draw order: x, words, scale normals, bias normals (numpy PCG64)."""
    assert k % 64 == 0
    rng = np.random.Generator(np.random.PCG64(seed))
    x = f32_to_bf16_bits(rng.standard_normal((m, k), dtype=np.float32) * np.float32(sigma))
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    s32 = np.abs(rng.standard_normal((n, k // 64), dtype=np.float32)) * np.float32(0.004) + np.float32(1e-4)
    s = f32_to_bf16_bits(s32)
    b32 = np.float32(-8.0) * bf16_bits_to_f32(s) + rng.standard_normal((n, k // 64), dtype=np.float32) * np.float32(1e-3)
    b = f32_to_bf16_bits(b32.astype(np.float32))
    return x, w, s, b


def config_inputs(index: int, m: int | None = None):
    """Inputs of benchmark workload `index` (seed = index). Workload 1 draws x for M = 4 and
    slices rows for M = 1 and 2."""
    c = CONFIGS[index]
    mm = max(c["M"])
    x, w, s, b = make_inputs(mm, c["K"], c["N"], c["sigma"], seed=index)
    if m is not None:
        x = x[:m]
    return x, w, s, b


def bytes_per_call(m: int, k: int, n: int) -> int:
    """Algorithmic HBM bytes: 0.5625 B per weight (nibble + bf16 scale and bias per 64) plus x and y."""
    return n * k // 2 + 2 * 2 * n * (k // 64) + 2 * m * k + 2 * m * n


def flops_per_call(m: int, k: int, n: int) -> int:
    return 2 * m * n * k
