"""The quantized layers inside a batched tree-verify forward, and their capture into a HIP graph.

Mirrors the MLP half of each layer of src/mlx_tree_spec/tree_verify.py batch_forward (414-447):
every request's tree nodes are concatenated into one batch of rows, the matmuls, norms and MLPs run
once over all rows, and each residual add is fused with the RMS norm that follows it:

    h, x = add_rms_norm(h, r, layer.post_attention_layernorm)     # tree_verify.py:444
    nxt  = next layer's input_layernorm, or the model's final norm # 445
    h, x = add_rms_norm(h, layer.mlp(x), nxt)                      # 446

`r` is the attention (or GatedDeltaNet) output of the layer, which this package does not compute.
When the MLP is a QuantizedMLP, the first norm is folded into its gate+up projection
(add_rms_norm_gate_up: the same bits, one launch fewer for up to 4 rows).
The row count M = the sum of the requests' tree nodes decides the kernel inside libqmm4 (row-split
for M <= 4, verify kernels up to 64, the GEMM above), as packed_linear._call's routing does.

The reference prebinds one launcher per module to keep the ~400 calls of a forward cheap on the
host (packed_linear.py:61-69, 136-171). Here the same end is reached with a HIP graph: the layers of
a forward are captured once for a fixed row count and replayed, so a replay costs one launch on
the host whatever the number of kernels. Every entry point used here is capturable: none allocates
or clears memory with a memset once its first call has set up its buffers.
"""

from __future__ import annotations

import torch

from .fused_ops import add_rms_norm, add_rms_norm_gate_up
from .packed_linear import STATS, QuantizedMLP


class MLPLayer(torch.nn.Module):
    """The parts of one decoder layer the MLP half uses: post_attention_layernorm and mlp."""

    def __init__(self, post_attention_layernorm: torch.nn.Module, mlp: torch.nn.Module):
        super().__init__()
        self.post_attention_layernorm = post_attention_layernorm
        self.mlp = mlp


def layer_tail(h: torch.Tensor, r: torch.Tensor, layer: MLPLayer, next_norm: torch.nn.Module):
    """(h, x) after one layer's residual adds, norms and MLP (tree_verify.py:444-446)."""
    mlp = layer.mlp
    if isinstance(mlp, QuantizedMLP):
        STATS["gate_up_silu"] += 1
        h, _, t = add_rms_norm_gate_up(h, r, layer.post_attention_layernorm, mlp)
        return add_rms_norm(h, mlp.down_proj(t), next_norm)
    h, x = add_rms_norm(h, r, layer.post_attention_layernorm)
    return add_rms_norm(h, mlp(x), next_norm)


def stack_tail(h: torch.Tensor, rs: list[torch.Tensor], layers: list[MLPLayer], final_norm: torch.nn.Module):
    """layer_tail over a stack of layers; rs[i] is layer i's attention output. Returns (h, x)."""
    if len(rs) != len(layers):
        raise ValueError(f"[stack_tail] {len(rs)} attention outputs for {len(layers)} layers")
    x = None
    for i, layer in enumerate(layers):
        nxt = layers[i + 1].post_attention_layernorm if i + 1 < len(layers) else final_norm
        h, x = layer_tail(h, rs[i], layer, nxt)
    return h, x


class GraphedTail:
    """stack_tail captured into a HIP graph for a fixed batch of rows.

    The inputs are copied into static buffers, the graph replays every kernel of the stack, and
    the outputs are views of static buffers that the next replay overwrites.
    """

    def __init__(self, layers: list[MLPLayer], final_norm: torch.nn.Module, rows: int, dim: int, device):
        self.layers, self.final_norm = layers, final_norm
        self.h_in = torch.zeros((rows, dim), dtype=torch.bfloat16, device=device)
        self.r_in = [torch.zeros((rows, dim), dtype=torch.bfloat16, device=device) for _ in layers]
        # The library keeps its split-K workspace and scratch per (device, stream): warm up on a
        # private stream (first calls allocate them), then capture on that same stream, so the
        # captured kernels use buffers that exist and that no later call on another stream regrows.
        self.stream = torch.cuda.Stream(device)
        self.stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(self.stream):
            stack_tail(self.h_in, self.r_in, layers, final_norm)
        torch.cuda.current_stream(device).wait_stream(self.stream)
        torch.cuda.synchronize(device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.h_out, self.x_out = stack_tail(self.h_in, self.r_in, layers, final_norm)

    def __call__(self, h: torch.Tensor, rs: list[torch.Tensor]):
        self.h_in.copy_(h)
        for dst, src in zip(self.r_in, rs):
            dst.copy_(src)
        self.graph.replay()
        return self.h_out, self.x_out
