"""The quantized-linear operator on PyTorch-ROCm tensors, backed by libqmm4.so (gfx950 HIP).

Mirrors the reference's calls:
  quantized_matmul(x, w, scales, biases, transpose=True, group_size=64, bits=4)
      == mx.quantized_matmul as called at src/mlx_tree_spec/packed_linear.py:97
  dequantize(w, scales, biases, group_size=64, bits=4)
      == mx.dequantize as used by the exact reference at tests/test_units.py:108
  pack_nax / unpack_nax
      == the reference's install-time relayout and its inverse (qmm_packed.py:223-232,
         packed_linear.py:72-80), kept for interoperability: the gfx950 kernels read MLX's own
         [N, K/8] layout, so weights in the reference's packed layout are converted back once.

Tensors: x bfloat16 (..., K) on a HIP device; w int32 or uint32 [N, K * bits / 32] (the bits are
used as is); scales and biases bfloat16 [N, K / group_size]. Output bfloat16 (..., N), allocated here, written
asynchronously on the current stream of x's device.
"""

from __future__ import annotations

import torch

from . import _lib

_W_DTYPES = (torch.int32, torch.uint32)


# MLX affine formats whose codes fill whole uint32 words (code k = (32 / bits) c + i in bits
# [bits i, bits i + bits) of word c): dequantize takes them all, and so does quantized_matmul,
# whose packed kernels implement 4 bits in groups of 64 (other formats: dequantize, then a bf16
# GEMM, as the reference leaves them to MLX's own op, packed_linear.py:84-86). 3-, 5- and 6-bit
# codes, which MLX packs across word boundaries, are not supported.
GENERAL_BITS = (2, 4, 8)
GENERAL_GROUP_SIZES = (32, 64, 128)


def _check_format(group_size: int, bits: int, transpose: bool = True, mode: str = "affine",
                  general: bool = False) -> None:
    if mode != "affine":
        raise NotImplementedError(f"mode={mode!r}: only 'affine' quantization is supported")
    if general:
        if bits not in GENERAL_BITS:
            raise NotImplementedError(f"bits={bits}: only {', '.join(map(str, GENERAL_BITS))}-bit codes are supported")
        if group_size not in GENERAL_GROUP_SIZES:
            raise NotImplementedError(f"group_size={group_size}: only group sizes "
                                      f"{', '.join(map(str, GENERAL_GROUP_SIZES))} are supported")
    else:
        if bits != 4:
            raise NotImplementedError(f"bits={bits}: only 4-bit codes are supported")
        if group_size != 64:
            raise NotImplementedError(f"group_size={group_size}: only group_size=64 is supported")
    if not transpose:
        raise NotImplementedError("transpose=False: only y = x @ dequant(w).T is supported")


def _check_weights(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, k: int | None,
                   group_size: int, bits: int, what: str) -> tuple[int, int]:
    if w.dim() != 2 or w.dtype not in _W_DTYPES:
        raise ValueError(f"[{what}] w must be a 2-D int32/uint32 tensor, got {tuple(w.shape)} {w.dtype}")
    n, kw = w.shape
    kk = kw * 32 // bits
    if k is not None and kk != k:
        raise ValueError(f"[{what}] x.shape[-1]={k} does not match w.shape[-1]*32/bits={kk}")
    if scales is None or biases is None:
        raise ValueError(f"[{what}] affine quantization needs both scales and biases")
    for name, t in (("scales", scales), ("biases", biases)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"[{what}] {name} must be bfloat16, got {t.dtype}")
        if tuple(t.shape) != (n, kk // group_size):
            raise ValueError(f"[{what}] {name} shape {tuple(t.shape)} != {(n, kk // group_size)}")
    return n, kk


def _check_device(what: str, *ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    if dev.type != "cuda":
        raise ValueError(f"[{what}] tensors must be on a HIP device (got {dev}); there is no CPU path")
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"[{what}] all tensors must be on {dev}, got {t.device}")
    return dev


def aligned_contiguous(t: torch.Tensor, align: int = 16) -> torch.Tensor:
    """t itself when it is contiguous and its data starts on an `align`-byte boundary, else a copy
    in fresh storage (the caching allocator's blocks start on 512-byte boundaries). A contiguous
    view at an odd offset stays at that offset under .contiguous(), which the kernels reject."""
    if t.is_contiguous() and t.data_ptr() % align == 0:
        return t
    out = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    out.copy_(t)
    return out



def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                     transpose: bool = True, group_size: int = 64, bits: int = 4,
                     mode: str = "affine") -> torch.Tensor:
    """y = x @ dequant(w).T in bf16 with fp32 accumulation (HIP kernels; no CPU path).

    Shapes the packed kernels take (4-bit codes in groups of 64, K % 128 == 0, N % 16 == 0) run
    them. Other shapes (K % 64 == 0, any N) and formats (2-, 4- or 8-bit codes in groups of 32, 64
    or 128) are what the reference leaves to MLX's own op (packed_linear.py:56-57, 84-86): the
    weights are dequantized exactly by the HIP kernel and multiplied by a bf16 GEMM with fp32
    accumulation on the same stream.
    """
    _check_format(group_size, bits, transpose, mode, general=True)
    if x.dtype != torch.bfloat16:
        raise ValueError(f"[quantized_matmul] x must be bfloat16, got {x.dtype}")
    if x.dim() < 1:
        raise ValueError("[quantized_matmul] x must have at least one dimension")
    k = x.shape[-1]
    if k % group_size:
        raise ValueError(f"[quantized_matmul] x.shape[-1]={k} must be a multiple of group_size={group_size}")
    n, _ = _check_weights(w, scales, biases, k, group_size, bits, "quantized_matmul")
    dev = _check_device("quantized_matmul", x, w, scales, biases)
    x2 = aligned_contiguous(x.reshape(-1, k))
    m = x2.shape[0]
    if k % 128 or n % 16 or bits != 4 or group_size != 64:
        wd = dequantize(w, scales, biases, group_size, bits)
        return torch.nn.functional.linear(x2, wd).reshape(*x.shape[:-1], n)
    w = aligned_contiguous(w)
    scales = aligned_contiguous(scales)
    biases = aligned_contiguous(biases)
    y = torch.empty((*x.shape[:-1], n), dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.qmm4_affine_bf16(x2.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                                  y.data_ptr(), m, n, k, group_size, bits, 1, stream)
    _lib.check(rc, "quantized_matmul")
    return y


def gate_up_silu(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 group_size: int = 64, bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """silu(x @ dequant(w_gate).T) * (x @ dequant(w_up).T) for w = [w_gate; w_up] (N rows, gate
    first): the fused gate+up projection and SiLU·mul of an MLP, bf16 (..., N/2) (HIP kernels).

    Same value as splitting quantized_matmul(x, w, ...) into halves g, u and computing
    bf16(bf16(g * bf16(sigmoid(g))) * u) elementwise, the unfused composition of
    tree_verify.py:446's layer.mlp (down_proj(silu(gate_proj(x)) * up_proj(x))) up to down_proj.
    """
    _check_format(group_size, bits, True, mode)
    if x.dtype != torch.bfloat16:
        raise ValueError(f"[gate_up_silu] x must be bfloat16, got {x.dtype}")
    if x.dim() < 1:
        raise ValueError("[gate_up_silu] x must have at least one dimension")
    k = x.shape[-1]
    n, _ = _check_weights(w, scales, biases, k, group_size, bits, "gate_up_silu")
    if n % 32:
        raise ValueError(f"[gate_up_silu] w has {n} rows; gate and up halves need a multiple of 32")
    dev = _check_device("gate_up_silu", x, w, scales, biases)
    x2 = aligned_contiguous(x.reshape(-1, k))
    m = x2.shape[0]
    w = aligned_contiguous(w)
    scales = aligned_contiguous(scales)
    biases = aligned_contiguous(biases)
    y = torch.empty((*x.shape[:-1], n // 2), dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.qmm4_gate_up_silu_bf16(x2.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                                        y.data_ptr(), m, n, k, group_size, bits, 1, stream)
    _lib.check(rc, "gate_up_silu")
    return y


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int = 64,
               bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """bf16 [N, K] with w_deq = bf16_rne(fp32(s) * q + fp32(b)), bit-exact (HIP kernel); 2-, 4- or
    8-bit codes in groups of 32, 64 or 128 (mx.dequantize's parameters)."""
    _check_format(group_size, bits, True, mode, general=True)
    n, k = _check_weights(w, scales, biases, None, group_size, bits, "dequantize")
    dev = _check_device("dequantize", w, scales, biases)
    w = aligned_contiguous(w)
    scales = aligned_contiguous(scales)
    biases = aligned_contiguous(biases)
    out = torch.empty((n, k), dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.dequant4_affine_bf16(w.data_ptr(), scales.data_ptr(), biases.data_ptr(), out.data_ptr(),
                                      n, k, group_size, bits, stream)
    _lib.check(rc, "dequantize")
    return out


def pack_nax(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor):
    """MLX layout -> the reference's packed layout (qmm_packed.py:223-232), flat tensors:
    wq2[t][kb][r][j] = w[32t + r][2kb + j], sp2[t][g][r] = s[32t + r][g] (same for biases)."""
    n, kw = w.shape
    if n % 32 or kw % 2:
        raise ValueError(f"[pack_nax] need N % 32 == 0 and K % 16 == 0, got w {tuple(w.shape)}")
    g = scales.shape[1]
    wi = w.view(torch.int32) if w.dtype == torch.uint32 else w  # uint32 has few torch kernels
    wq2 = wi.reshape(n // 32, 32, kw // 2, 2).permute(0, 2, 1, 3).contiguous().reshape(-1).view(w.dtype)
    sp2 = scales.reshape(n // 32, 32, g).permute(0, 2, 1).contiguous().reshape(-1)
    bp2 = biases.reshape(n // 32, 32, g).permute(0, 2, 1).contiguous().reshape(-1)
    return wq2, sp2, bp2


def unpack_nax(wq2: torch.Tensor, sp2: torch.Tensor, bp2: torch.Tensor, n: int):
    """The reference's packed layout -> MLX layout (packed_linear._unpacked, packed_linear.py:72-80)."""
    kw = wq2.numel() // n
    g = sp2.numel() // n
    wi = wq2.view(torch.int32) if wq2.dtype == torch.uint32 else wq2
    w = wi.reshape(n // 32, kw // 2, 32, 2).permute(0, 2, 1, 3).contiguous().reshape(n, kw).view(wq2.dtype)
    s = sp2.reshape(n // 32, g, 32).permute(0, 2, 1).contiguous().reshape(n, g)
    b = bp2.reshape(n // 32, g, 32).permute(0, 2, 1).contiguous().reshape(n, g)
    return w, s, b
