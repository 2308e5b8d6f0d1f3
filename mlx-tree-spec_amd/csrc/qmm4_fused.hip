// Passes around the quantized matmul: the fused residual add + RMS norm in front of it, and the
// SiLU·mul epilogue of a gate+up projection behind it.
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

// add_rms_norm: h = x + r and n = rmsnorm(h) * w for each row of D values, in one pass over the row
// (src/mlx_tree_spec/fused_ops.py:107-128, the residual add fused with the RMS norm that follows it,
// tree_verify.py:444-446):
//   h  = bf16(x + r)                              (stored)
//   ss = sum over the row of h * h                (fp32)
//   inv = 1 / sqrt(ss / D + eps)                  (fp32, correctly rounded sqrt and division)
//   n  = bf16(w * bf16(h * inv))
// One workgroup of 256 threads per row; thread t holds the 16-byte chunks t, t + 256, ... of the row
// (h stays in registers between the sum and the normalization). The row sum adds each thread's
// chunks in order, then the 64 lanes of a wave by a butterfly, then the 4 waves in wave order.
constexpr int kNormThreads = 256;

template <int CPT>  // 16-byte chunks per thread
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(const uint16_t* __restrict__ x,
                                                                    const uint16_t* __restrict__ r,
                                                                    const uint16_t* __restrict__ w,
                                                                    uint16_t* __restrict__ h_out,
                                                                    uint16_t* __restrict__ n_out, int D,
                                                                    float eps) {
  __shared__ float red[kNormThreads / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  const int chunks = D >> 3;
  const size_t base = (size_t)row * D;
  u32x4 hv[CPT];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + i * kNormThreads;
    hv[i] = u32x4{0u, 0u, 0u, 0u};
    if (c < chunks) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(x + base + c * 8);
      const u32x4 b = *reinterpret_cast<const u32x4*>(r + base + c * 8);
      hv[i] = norm_add_chunk(a, b, ss);
      *reinterpret_cast<u32x4*>(h_out + base + c * 8) = hv[i];
    }
  }
  ss = norm_wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) total += red[i];
  const float inv = norm_inv(total, D, eps);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + i * kNormThreads;
    if (c < chunks) {
      const u32x4 wv = *reinterpret_cast<const u32x4*>(w + c * 8);
      *reinterpret_cast<u32x4*>(n_out + base + c * 8) = norm_scale_chunk(hv[i], wv, inv);
    }
  }
}

}  // namespace

int add_rms_norm_max_d() { return 8 * kNormThreads * 8; }

hipError_t launch_add_rms_norm(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* h,
                               uint16_t* n, int rows, int D, float eps, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int cpt = (D / 8 + kNormThreads - 1) / kNormThreads;
  if (cpt <= 1)
    hipLaunchKernelGGL(add_rms_norm_kernel<1>, dim3(rows), dim3(kNormThreads), 0, stream, x, r, w, h, n, D, eps);
  else if (cpt <= 2)
    hipLaunchKernelGGL(add_rms_norm_kernel<2>, dim3(rows), dim3(kNormThreads), 0, stream, x, r, w, h, n, D, eps);
  else if (cpt <= 4)
    hipLaunchKernelGGL(add_rms_norm_kernel<4>, dim3(rows), dim3(kNormThreads), 0, stream, x, r, w, h, n, D, eps);
  else
    hipLaunchKernelGGL(add_rms_norm_kernel<8>, dim3(rows), dim3(kNormThreads), 0, stream, x, r, w, h, n, D, eps);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const uint16_t* t, uint16_t* y, int M, int n, hipStream_t stream) {
  if (M <= 0 || n <= 0) return hipSuccess;
  const long long items = (long long)M * (n / 8);
  const long long want = (items + 255) / 256;
  const int blocks = (int)(want < 8192 ? want : 8192);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(256), 0, stream, t, y, M, n);
  return hipGetLastError();
}

}  // namespace qmm4
