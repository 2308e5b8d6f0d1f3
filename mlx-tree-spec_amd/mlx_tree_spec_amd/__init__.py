"""MI355X (gfx950) packed 4-bit affine quantized matmul in MLX's format.

    from mlx_tree_spec_amd import quantized_matmul, dequantize, QuantizedLinear, install

All compute runs in libqmm4.so (hand-written HIP kernels, C ABI in include/qmm4.h); importing
this package does not load it, the first call does, and fails loudly if it is not built.
"""

from .fused_ops import add_rms_norm, add_rms_norm_, add_rms_norm_gate_up, add_rms_norm_qmm_
from .packed_linear import STATS, QuantizedLinear, QuantizedMLP, eligible, install
from .qmm import dequantize, gate_up_silu, pack_nax, quantized_matmul, unpack_nax
from .verify import GraphedTail, MLPLayer, layer_tail, stack_tail

__all__ = [
    "quantized_matmul", "gate_up_silu", "dequantize", "pack_nax", "unpack_nax", "add_rms_norm",
    "add_rms_norm_", "add_rms_norm_qmm_", "add_rms_norm_gate_up", "QuantizedLinear", "QuantizedMLP",
    "eligible", "install", "STATS", "MLPLayer", "layer_tail", "stack_tail", "GraphedTail",
]
__version__ = "0.1.0"
