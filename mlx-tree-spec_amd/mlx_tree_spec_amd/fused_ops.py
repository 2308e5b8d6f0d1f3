"""Fused ops on the input side of the quantized matmuls, backed by libqmm4.so (gfx950 HIP).

Mirrors src/mlx_tree_spec/fused_ops.py:
  add_rms_norm(x, r, norm) -> (h, n)   == fused_ops.add_rms_norm (107-160): h = x + r and
                                          n = norm(h) in one dispatch, for an RMSNorm module `norm`
                                          (anything with .weight and .eps; torch.nn.RMSNorm works)

Tensors are bfloat16 on a HIP device; there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib
from .qmm import aligned_contiguous


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
    eps = getattr(norm, "eps", None)
    if eps is None:  # torch.nn.RMSNorm(eps=None) uses the dtype's machine epsilon
        eps = torch.finfo(torch.bfloat16).eps
    return add_rms_norm_(x, r, norm.weight, eps)
