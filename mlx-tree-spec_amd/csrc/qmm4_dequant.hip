// Bit-exact unpack + affine dequantization: out[n, k] = bf16_rne(fp32(s) * q + fp32(b)).
// The formula and nibble order are those of src/mlx_tree_spec/qmm_packed.py:200-201 and 635-636;
// the result is what mx.dequantize returns for 4-bit affine weights (tests/test_units.py:108).
//
// HBM-bound: each thread reads 4 packed words (16 B, 32 codes of one row, all in one group) plus
// the group's scale and bias, and writes 32 bf16 (64 B) with four 16-B stores.
#include "qmm4_common.h"
#include "qmm4_kernels.h"

namespace qmm4 {

__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ s,
                                                      const uint16_t* __restrict__ b,
                                                      uint16_t* __restrict__ out,
                                                      int64_t chunks, int64_t chunks_per_row,
                                                      int64_t K) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < chunks; i += stride) {
    const int64_t n = i / chunks_per_row;
    const int64_t c4 = i - n * chunks_per_row;  // 4-word chunk within the row
    const u32x4 v = *reinterpret_cast<const u32x4*>(w + n * (K >> 3) + c4 * 4);
    const int64_t g = (c4 * 32) >> 6;           // group of k = 32*c4
    const float sf = bf16_to_f32(s[n * (K >> 6) + g]);
    const float bf = bf16_to_f32(b[n * (K >> 6) + g]);
    const float s16 = sf * 0.0625f;
    u32x4* o = reinterpret_cast<u32x4*>(out + n * K + c4 * 32);
    o[0] = dequant_word(v.x, sf, s16, bf);
    o[1] = dequant_word(v.y, sf, s16, bf);
    o[2] = dequant_word(v.z, sf, s16, bf);
    o[3] = dequant_word(v.w, sf, s16, bf);
  }
}

hipError_t launch_dequant(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          uint16_t* out, int64_t N, int64_t K, hipStream_t stream) {
  const int64_t chunks_per_row = K / 32;
  const int64_t chunks = N * chunks_per_row;
  if (chunks == 0) return hipSuccess;
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;  // grid-stride beyond 64 waves per CU
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, w, s, b, out,
                     chunks, chunks_per_row, K);
  return hipGetLastError();
}

}  // namespace qmm4
