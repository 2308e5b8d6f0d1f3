"""Quantized-linear drop-in: a torch module whose call is the gfx950 packed 4-bit kernel.

Mirrors src/mlx_tree_spec/packed_linear.py:
  eligible(mod)        -> packed_linear.eligible (49-58): 4-bit affine with biases, no linear
                          bias, N % 32 == 0, K % 128 == 0 (and group_size == 64, the one group
                          size these kernels implement)
  install(model)       -> packed_linear.install (136-179): prepares every eligible module and
                          prebinds its launcher; returns the same summary dict
  QuantizedLinear      -> mlx.nn.QuantizedLinear (weight uint32 [N, K/8], scales and biases
                          bf16 [N, K/64]) with __call__ = _call
  _call(mod, x)        -> packed_linear._call (83-104): rows = prod(x.shape[:-1]), dispatch by rows
  STATS                -> per-path call counters (packed_linear.py:46)

Differences by design (MI355X-first):
  * no relayout: the kernels read MLX's [N, K/8] layout directly, so install() keeps the weights
    as they are (no transient copy) instead of rewriting them with pack_nax;
  * no install-time timing race between kernels: the kernel is a fixed function of the row count
    (M <= SKINNY_MAX_ROWS: the HBM-bound skinny kernel; larger M: the MFMA GEMM), decided inside
    the library;
  * the prebound launcher skips the per-call argument checks (weights were validated once); it
    holds the bound tensors and rebinds when the module's buffers are replaced.
"""

from __future__ import annotations

import math
from collections import defaultdict

import torch

from . import _lib
from .qmm import aligned_contiguous, gate_up_silu, quantized_matmul

SKINNY_MAX_ROWS = 64  # rows <= this take the skinny kernel (the reference's PREFILL_M is 64)
STATS: dict[str, int] = defaultdict(int)


class QuantizedLinear(torch.nn.Module):
    """y = x @ dequant(weight).T (+ bias) for MLX-format affine weights: 4-bit codes in groups of
    64 on the packed kernels; 2-, 4- and 8-bit codes in groups of 32, 64 or 128 on the general path."""

    def __init__(self, input_dims: int, output_dims: int, bias: bool = False, group_size: int = 64,
                 bits: int = 4, mode: str = "affine", device=None):
        super().__init__()
        if input_dims % 32:
            raise ValueError(f"input_dims={input_dims} must be a multiple of 32 for {bits}-bit packing")
        self.group_size, self.bits, self.mode = group_size, bits, mode
        self.register_buffer("weight", torch.zeros(output_dims, input_dims * bits // 32, dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.zeros(output_dims, input_dims // group_size, dtype=torch.bfloat16, device=device))
        self.register_buffer("biases", torch.zeros(output_dims, input_dims // group_size, dtype=torch.bfloat16, device=device))
        self.bias = torch.nn.Parameter(torch.zeros(output_dims, dtype=torch.bfloat16, device=device)) if bias else None

    @classmethod
    def from_quantized(cls, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                       group_size: int = 64, bits: int = 4, bias: torch.Tensor | None = None) -> "QuantizedLinear":
        n, kw = weight.shape
        mod = cls(kw * 32 // bits, n, bias=bias is not None, group_size=group_size, bits=bits,
                  device=weight.device)
        mod.weight = weight.view(torch.int32) if weight.dtype == torch.uint32 else weight
        mod.scales, mod.biases = scales, biases
        if bias is not None:
            mod.bias = torch.nn.Parameter(bias)
        return mod

    @property
    def input_dims(self) -> int:
        return self.weight.shape[1] * 32 // self.bits

    @property
    def output_dims(self) -> int:
        return self.weight.shape[0]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _call(self, x)


class QuantizedMLP(torch.nn.Module):
    """down_proj(silu(gate_proj(x)) * up_proj(x)) over MLX-format 4-bit linears, with gate and up
    fused into one projection whose epilogue applies silu * up (tree_verify.py:446, layer.mlp).

    The gate and up weights (and their scales and biases) are stacked once, gate rows first, so a
    call is one gate_up_silu (one kernel for up to 4 rows) and one down_proj matmul.
    """

    def __init__(self, gate_proj: QuantizedLinear, up_proj: QuantizedLinear, down_proj: QuantizedLinear):
        super().__init__()
        for name, m in (("gate_proj", gate_proj), ("up_proj", up_proj), ("down_proj", down_proj)):
            if not eligible(m):
                raise ValueError(f"[QuantizedMLP] {name} is not an eligible 4-bit affine QuantizedLinear")
        if gate_proj.weight.shape != up_proj.weight.shape or gate_proj.group_size != up_proj.group_size:
            raise ValueError("[QuantizedMLP] gate_proj and up_proj must have the same shape and group size")
        if down_proj.input_dims != gate_proj.output_dims or down_proj.output_dims != gate_proj.input_dims:
            raise ValueError(f"[QuantizedMLP] down_proj {down_proj.input_dims}->{down_proj.output_dims} does not "
                             f"match gate/up {gate_proj.input_dims}->{gate_proj.output_dims}")
        self.group_size = gate_proj.group_size
        self.register_buffer("gate_up_weight", torch.cat([gate_proj.weight, up_proj.weight], 0).contiguous())
        self.register_buffer("gate_up_scales", torch.cat([gate_proj.scales, up_proj.scales], 0).contiguous())
        self.register_buffer("gate_up_biases", torch.cat([gate_proj.biases, up_proj.biases], 0).contiguous())
        self.down_proj = down_proj

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        STATS["gate_up_silu"] += 1
        h = gate_up_silu(x, self.gate_up_weight, self.gate_up_scales, self.gate_up_biases,
                         group_size=self.group_size)
        return self.down_proj(h)


def eligible(mod) -> bool:
    """packed_linear.eligible (packed_linear.py:49-58): the modules the packed kernels take.

    One condition more than the reference's: group_size == 64, the only group size the gfx950
    kernels implement (the reference's kernels take the group size as a parameter). A module
    with another group size is reported as not packed instead of failing at its first call.
    """
    return (
        isinstance(mod, QuantizedLinear)
        and mod.bits == 4
        and mod.group_size == 64
        and getattr(mod, "mode", "affine") == "affine"
        and mod.biases is not None
        and mod.bias is None
        and mod.weight.shape[0] % 32 == 0
        and (mod.weight.shape[1] * 8) % 128 == 0
    )


def _bindable(mod: QuantizedLinear) -> bool:
    """The module's buffers as a launcher binds them: on a HIP device, bf16 scales and biases,
    int32/uint32 codes."""
    return (mod.weight.device.type == "cuda" and mod.weight.dtype in (torch.int32, torch.uint32)
            and mod.scales.dtype == torch.bfloat16 and mod.biases.dtype == torch.bfloat16
            and mod.scales.device == mod.weight.device and mod.biases.device == mod.weight.device)


def _prepare(mod: QuantizedLinear) -> None:
    """Make the module's buffers contiguous and 16-byte aligned (copies only where needed)."""
    for name in ("weight", "scales", "biases"):
        t = getattr(mod, name)
        a = aligned_contiguous(t)
        if a is not t:
            setattr(mod, name, a)


def _launcher(mod: QuantizedLinear):
    """mod's matmul with weights, shape and library bound: per call only x is checked, plus a
    cheap test that the bound buffers are still the module's own (the same tensor objects, the
    same storage, bf16 scales and biases). The closure holds the tensors themselves, so their
    memory stays valid while it exists; when the module's buffers have been replaced (e.g.
    mod.to(dtype), a reassigned weight, .data swapped) the launcher returns None and the caller
    rebinds."""
    w, s, b = mod.weight, mod.scales, mod.biases
    n, k, gs = mod.output_dims, mod.input_dims, mod.group_size
    wp, sp, bp = w.data_ptr(), s.data_ptr(), b.data_ptr()
    dev = w.device
    fn = _lib.load().qmm4_affine_bf16

    def run(x: torch.Tensor) -> torch.Tensor | None:
        if (mod.weight is not w or mod.scales is not s or mod.biases is not b or w.data_ptr() != wp
                or s.data_ptr() != sp or b.data_ptr() != bp or s.dtype != torch.bfloat16
                or b.dtype != torch.bfloat16):
            return None
        if x.dtype != torch.bfloat16 or x.shape[-1] != k or x.device != dev:
            raise ValueError(f"[QuantizedLinear] expected bfloat16 (..., {k}) on {dev}, got "
                             f"{x.dtype} {tuple(x.shape)} on {x.device}")
        x2 = aligned_contiguous(x.reshape(-1, k))
        y = torch.empty((*x.shape[:-1], n), dtype=torch.bfloat16, device=dev)
        rc = fn(x2.data_ptr(), wp, sp, bp, y.data_ptr(), x2.shape[0], n, k, gs, 4, 1,
                torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(rc, "QuantizedLinear")
        return y

    return run


def _call(self: QuantizedLinear, x: torch.Tensor) -> torch.Tensor:
    sh = x.shape
    rows = math.prod(sh[:-1])
    if "_fast" not in self.__dict__ and not eligible(self):
        # packed_linear._call (84-86): a module the packed path does not take runs the general op
        # (here quantized_matmul's exact dequantize + bf16 GEMM form: 4-bit shapes the kernels
        # refuse, and 2-, 4- or 8-bit codes in groups of 32, 64 or 128; other widths raise
        # NotImplementedError).
        STATS["fallback"] += 1
        y = quantized_matmul(x, self.weight, self.scales, self.biases, transpose=True,
                             group_size=self.group_size, bits=self.bits, mode=self.mode)
        return y + self.bias if self.bias is not None else y
    STATS["skinny" if rows <= SKINNY_MAX_ROWS else "gemm"] += 1
    run = self.__dict__.get("_fast")
    y = run(x) if run is not None else None
    if y is None:
        if run is not None:
            # The bound buffers were replaced since install(): rebind to the current ones (or drop
            # the launcher when they no longer suit it; the checked call below then raises).
            STATS["rebound"] += 1
            self.__dict__.pop("_fast")
            if eligible(self) and _bindable(self):
                _prepare(self)
                object.__setattr__(self, "_fast", _launcher(self))
        y = quantized_matmul(x, self.weight, self.scales, self.biases, transpose=True,
                             group_size=self.group_size, bits=self.bits, mode=self.mode)
    if self.bias is not None:
        y = y + self.bias
    return y


def install(model: torch.nn.Module, verbose: bool = True) -> dict:
    """Prepare every eligible QuantizedLinear of `model` for the packed kernels.

    Weights must already be on the HIP device. Each module's buffers are made contiguous and
    16-byte aligned once (copied only where they are not) and a launcher with them bound is
    attached, so a forward's calls skip the generic argument checks; a launcher whose buffers
    were later replaced is rebound at the next call. Returns the reference's summary dict.
    """
    before = torch.cuda.memory_allocated() if torch.cuda.is_available() else 0
    groups: dict[tuple[int, int], int] = defaultdict(int)
    packed = 0
    for _, mod in model.named_modules():
        if not eligible(mod) or "_fast" in mod.__dict__:
            continue
        if mod.weight.device.type != "cuda":
            raise ValueError("install(): move the model to the HIP device first")
        if mod.scales.dtype != torch.bfloat16 or mod.biases.dtype != torch.bfloat16:
            raise ValueError("install(): scales and biases must be bfloat16")
        _prepare(mod)
        object.__setattr__(mod, "_fast", _launcher(mod))
        groups[(mod.input_dims, mod.output_dims)] += 1
        packed += 1
    if verbose:
        for (k, n), c in sorted(groups.items()):
            print(f"  packed {k:>6}->{n:<6} x{c}")
    after = torch.cuda.memory_allocated() if torch.cuda.is_available() else 0
    return dict(packed=packed, memory_before_gb=before / 1e9, memory_after_gb=after / 1e9)
