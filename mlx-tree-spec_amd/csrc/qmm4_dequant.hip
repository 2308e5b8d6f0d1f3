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

// The other affine formats MLX packs into whole uint32 words (bits 2 and 8; 4 with groups of 32
// or 128), for the general path (the reference hands modules its packed kernels do not take to
// MLX's own op, packed_linear.py:84-86): code k = (32 / BITS) c + i sits in bits
// [BITS i, BITS i + BITS) of word c, the same little-endian order as the 4-bit codes
// (qmm_packed.py:115), and the dequantization is the same single-rounded fma, then bf16:
// out[n, k] = bf16_rne(fp32(s) * q + fp32(b)) with s * q exact in fp32 (q < 256, 8-bit s).
// One word per thread (a word never straddles a group: groups of 32 or more codes start at
// multiples of 32, words at multiples of 32 / BITS).
template <int BITS>
__global__ __launch_bounds__(256) void dequant_general_kernel(const uint32_t* __restrict__ w,
                                                              const uint16_t* __restrict__ s,
                                                              const uint16_t* __restrict__ b,
                                                              uint16_t* __restrict__ out, int64_t words,
                                                              int64_t words_per_row, int64_t K, int gshift) {
  constexpr int kPer = 32 / BITS;  // codes per word
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride) {
    const int64_t n = i / words_per_row;
    const int64_t c = i - n * words_per_row;
    const uint32_t v = w[i];
    const int64_t k0 = c * kPer;
    const int64_t g = k0 >> gshift;
    const int64_t groups = K >> gshift;
    const float sf = bf16_to_f32(s[n * groups + g]);
    const float bf = bf16_to_f32(b[n * groups + g]);
    uint32_t o[kPer / 2];
#pragma unroll
    for (int j = 0; j < kPer / 2; ++j) {
      const float q0 = (float)((v >> (BITS * (2 * j))) & kMask);
      const float q1 = (float)((v >> (BITS * (2 * j + 1))) & kMask);
      o[j] = pack_bf16x2(__builtin_fmaf(q0, sf, bf), __builtin_fmaf(q1, sf, bf));
    }
    uint32_t* dst = reinterpret_cast<uint32_t*>(out + n * K + k0);
#pragma unroll
    for (int j = 0; j < kPer / 2; ++j) dst[j] = o[j];
  }
}

hipError_t launch_dequant(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint16_t* out, int64_t N,
                          int64_t K, int group_size, int bits, hipStream_t stream) {
  if (bits != 4 || group_size != 64) {
    const int gshift = group_size == 32 ? 5 : group_size == 64 ? 6 : group_size == 128 ? 7 : -1;
    if (gshift < 0 || (bits != 2 && bits != 4 && bits != 8) || K % group_size != 0) return hipErrorInvalidValue;
    const int64_t words_per_row = K * bits / 32;
    const int64_t words = N * words_per_row;
    if (words == 0) return hipSuccess;
    int64_t blocks = (words + 255) / 256;
    if (blocks > 256 * 64) blocks = 256 * 64;
    if (bits == 2)
      hipLaunchKernelGGL(dequant_general_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, stream, w, s, b, out, words,
                         words_per_row, K, gshift);
    else if (bits == 4)
      hipLaunchKernelGGL(dequant_general_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, stream, w, s, b, out, words,
                         words_per_row, K, gshift);
    else
      hipLaunchKernelGGL(dequant_general_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, stream, w, s, b, out, words,
                         words_per_row, K, gshift);
    return hipGetLastError();
  }
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
