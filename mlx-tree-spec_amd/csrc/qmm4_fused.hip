// Elementwise passes around the quantized matmul.
//
// silu_mul: y[m, j] = silu(t[m, j]) * t[m, n + j] for t = x @ [w_gate; w_up]^T as bf16 [M, 2n]: the
// epilogue of a fused gate+up projection when it does not run inside the row-split kernel. Same
// arithmetic as that kernel's epilogue (silu_mul_bf16), so both paths give the same bits. The MLP
// this feeds is down_proj(silu(gate_proj(x)) * up_proj(x)) (src/mlx_tree_spec/tree_verify.py:446,
// layer.mlp; bench/ane/exact_split.py:82 writes the same composition). HBM-bound: 16-byte loads of
// both halves and a 16-byte store per thread.
#include "qmm4_common.h"
#include "qmm4_kernels.h"

namespace qmm4 {

namespace {

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ t, uint16_t* __restrict__ y,
                                                        int M, int n) {
  const int per_row = n >> 3;  // 8 outputs per item
  const long long items = (long long)M * per_row;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < items;
       i += (long long)gridDim.x * blockDim.x) {
    const int m = (int)(i / per_row), c = (int)(i - (long long)m * per_row) * 8;
    const u32x4 g = *reinterpret_cast<const u32x4*>(t + (size_t)m * 2 * n + c);
    const u32x4 u = *reinterpret_cast<const u32x4*>(t + (size_t)m * 2 * n + n + c);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = silu_mul_bf16(g[e] & 0xFFFFu, u[e] & 0xFFFFu) | (silu_mul_bf16(g[e] >> 16, u[e] >> 16) << 16);
    *reinterpret_cast<u32x4*>(y + (size_t)m * n + c) = o;
  }
}

}  // namespace

hipError_t launch_silu_mul(const uint16_t* t, uint16_t* y, int M, int n, hipStream_t stream) {
  if (M <= 0 || n <= 0) return hipSuccess;
  const long long items = (long long)M * (n / 8);
  const long long want = (items + 255) / 256;
  const int blocks = (int)(want < 8192 ? want : 8192);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(256), 0, stream, t, y, M, n);
  return hipGetLastError();
}

}  // namespace qmm4
