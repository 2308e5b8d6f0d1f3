"""Fused ops on the input side of the quantized matmuls, backed by libqmm4.so (gfx950 HIP).

Mirrors src/mlx_tree_spec/fused_ops.py:
  add_rms_norm(x, r, norm) -> (h, n)   == fused_ops.add_rms_norm (107-160): h = x + r and
                                          n = norm(h) in one dispatch, for an RMSNorm module `norm`
                                          (anything with .weight and .eps; torch.nn.RMSNorm works)
and folds that norm into the projection that consumes n (tree_verify.py:444-446):
  add_rms_norm_qmm_(x, r, weight, eps, w, scales, biases, silu_mul=False) -> (h, n, y)
  add_rms_norm_gate_up(x, r, norm, mlp) -> (h, n, t), t = silu(n w_gate^T) * (n w_up^T)
with the bits of add_rms_norm followed by quantized_matmul / gate_up_silu, in one launch for up to
4 rows.

Tensors are bfloat16 on a HIP device; there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib
from .qmm import _check_device, _check_format, _check_weights, aligned_contiguous


def add_rms_norm_(x: torch.Tensor, r: torch.Tensor, weight: torch.Tensor, eps: float):
    """(x + r, rmsnorm(x + r) * weight) as bf16, each shaped like x: h = bf16(x + r),
    n = bf16(weight * bf16(h / sqrt(mean(h^2) + eps))) over the last dimension."""
    for name, t in (("x", x), ("r", r), ("weight", weight)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"[add_rms_norm] {name} must be bfloat16, got {t.dtype}")
    if x.shape != r.shape:
        raise ValueError(f"[add_rms_norm] x {tuple(x.shape)} and r {tuple(r.shape)} differ")
    d = x.shape[-1]
    if tuple(weight.shape) != (d,):
        raise ValueError(f"[add_rms_norm] weight must have shape ({d},), got {tuple(weight.shape)}")
    dev = x.device
    if dev.type != "cuda" or r.device != dev or weight.device != dev:
        raise ValueError("[add_rms_norm] x, r and weight must be on one HIP device; there is no CPU path")
    x2 = aligned_contiguous(x.reshape(-1, d))
    r2 = aligned_contiguous(r.reshape(-1, d))
    w = aligned_contiguous(weight)
    h = torch.empty_like(x2)
    n = torch.empty_like(x2)
    lib = _lib.load()
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.qmm4_add_rms_norm_bf16(x2.data_ptr(), r2.data_ptr(), w.data_ptr(), h.data_ptr(), n.data_ptr(),
                                        x2.shape[0], d, float(eps), stream)
    _lib.check(rc, "add_rms_norm")
    return h.reshape(x.shape), n.reshape(x.shape)


def add_rms_norm(x: torch.Tensor, r: torch.Tensor, norm):
    """(x + r, norm(x + r)) for an RMSNorm module `norm`, in one dispatch (fused_ops.add_rms_norm)."""
    return add_rms_norm_(x, r, norm.weight, _norm_eps(norm))


def add_rms_norm_qmm_(x: torch.Tensor, r: torch.Tensor, weight: torch.Tensor, eps: float, w: torch.Tensor,
                      scales: torch.Tensor, biases: torch.Tensor, silu_mul: bool = False, group_size: int = 64,
                      bits: int = 4):
    """(h, n, y): h, n = add_rms_norm_(x, r, weight, eps) and y = quantized_matmul(n, w, scales,
    biases) (or gate_up_silu(n, w, scales, biases) when silu_mul), bit for bit, in one launch when
    the projection runs as the row-split kernel (up to 4 rows, K <= 8192)."""
    _check_format(group_size, bits)
    what = "add_rms_norm_qmm"
    for name, t in (("x", x), ("r", r), ("weight", weight)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"[{what}] {name} must be bfloat16, got {t.dtype}")
    if x.shape != r.shape:
        raise ValueError(f"[{what}] x {tuple(x.shape)} and r {tuple(r.shape)} differ")
    k = x.shape[-1]
    if tuple(weight.shape) != (k,):
        raise ValueError(f"[{what}] weight must have shape ({k},), got {tuple(weight.shape)}")
    n_rows, _ = _check_weights(w, scales, biases, k, group_size, bits, what)
    if silu_mul and n_rows % 32:
        raise ValueError(f"[{what}] w has {n_rows} rows; gate and up halves need a multiple of 32")
    dev = _check_device(what, x, r, weight, w, scales, biases)
    x2 = aligned_contiguous(x.reshape(-1, k))
    r2 = aligned_contiguous(r.reshape(-1, k))
    nw = aligned_contiguous(weight)
    w = aligned_contiguous(w)
    scales = aligned_contiguous(scales)
    biases = aligned_contiguous(biases)
    m = x2.shape[0]
    h = torch.empty_like(x2)
    n = torch.empty_like(x2)
    y = torch.empty((m, n_rows // 2 if silu_mul else n_rows), dtype=torch.bfloat16, device=dev)
    epilogue = _lib.QMM4_EPILOGUE_SILU_MUL if silu_mul else _lib.QMM4_EPILOGUE_NONE
    lib = _lib.load()
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.qmm4_add_rms_norm_qmm_bf16(x2.data_ptr(), r2.data_ptr(), nw.data_ptr(), float(eps), h.data_ptr(),
                                            n.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                                            y.data_ptr(), m, n_rows, k, group_size, bits, 1, epilogue, stream)
    _lib.check(rc, what)
    lead = x.shape[:-1]
    return h.reshape(x.shape), n.reshape(x.shape), y.reshape(*lead, y.shape[-1])


def _norm_eps(norm) -> float:
    eps = getattr(norm, "eps", None)
    if eps is None:  # torch.nn.RMSNorm(eps=None) uses the dtype's machine epsilon
        eps = torch.finfo(torch.bfloat16).eps
    return eps


def add_rms_norm_gate_up(x: torch.Tensor, r: torch.Tensor, norm, mlp):
    """(h, n, t) for an RMSNorm module `norm` and a QuantizedMLP `mlp`: h, n = add_rms_norm(x, r,
    norm) and t = silu(n w_gate^T) * (n w_up^T), the MLP's input to down_proj
    (tree_verify.py:444-446), the norm folded into the gate+up projection's x staging."""
    return add_rms_norm_qmm_(x, r, norm.weight, _norm_eps(norm), mlp.gate_up_weight, mlp.gate_up_scales,
                             mlp.gate_up_biases, silu_mul=True, group_size=mlp.group_size)
