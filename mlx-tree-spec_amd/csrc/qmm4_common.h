// Shared device helpers for the gfx950 packed 4-bit affine kernels.
//
// Format (MLX affine, 4 bits, group 64): w uint32 [N, K/8] holds q[n, 8c+i] in bits [4i, 4i+4) of
// w[n, c] (src/mlx_tree_spec/qmm_packed.py:115, 200-201); scales/biases bf16 [N, K/64]; the
// dequantized weight is bf16_rne(fp32(s) * q + fp32(b)) (qmm_packed.py:635-636).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmm4 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGroup = 64;  // quantization group along K

// Word 3 of a raw (stride 0) buffer resource on gfx9 CDNA: 32-bit data format, no swizzle.
constexpr int kBufferRsrcWord3 = 0x00020000;

// num_records of a buffer resource holding `bytes` bytes (the field is an unsigned 32-bit count;
// callers keep every buffer below 4 GiB).
__device__ __forceinline__ int rsrc_bytes(unsigned long long bytes) {
  return (int)(uint32_t)(bytes < 0xFFFFFFFFull ? bytes : 0xFFFFFFFFull);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Two fp32 values -> two bf16 (round to nearest even) in one dword, `a` in the low half.
// Compiles to a single v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  f32x2 v = {a, b};
  bf16x2 r = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t bf16_rne(float a) { return pack_bf16x2(a, 0.0f) & 0xFFFFu; }

// silu(g) * u on bf16 operands, one bf16 rounding per operation as the unfused MLP computes it
// (silu(x) = x * sigmoid(x), then the product with up; every intermediate a bf16 array):
//   s = bf16(sigmoid(g)), t = bf16(g * s), out = bf16(t * u),
// with sigmoid(g) = 1 / (1 + exp(-g)) in fp32 (exp(-g) overflowing to infinity gives 0; the
// complement form 1 - sigmoid(|g|) would cancel for g < -10).
__device__ __forceinline__ uint32_t silu_mul_bf16(uint32_t gbits, uint32_t ubits) {
  const float g = bf16_to_f32(gbits);
  const float sg = 1.0f / (1.0f + expf(-g));
  const float t = bf16_to_f32(bf16_rne(g * bf16_to_f32(bf16_rne(sg))));
  return bf16_rne(t * bf16_to_f32(ubits));
}

// The residual add + RMS norm of a row of D values (fused_ops.py:107-128), on 16-byte chunks of 8
// values. The norm kernel and the row-split kernel's normalising x staging both use these, with the
// same partition of a row over 256 threads, so they produce the same bits:
//   norm_add_chunk    h = bf16(x + r) per value, and ss += h * h per value in order (fused
//                     multiply-adds; a chunk of zeros leaves ss unchanged)
//   norm_wave_sum     the 64 lanes' sums added by an xor butterfly (every lane gets the total)
//   norm_inv          inv = 1 / sqrt(total / D + eps), correctly rounded division and square root
//   norm_scale_chunk  n = bf16(w * bf16(h * inv)) per value
__device__ __forceinline__ u32x4 norm_add_chunk(u32x4 a, u32x4 b, float& ss) {
  u32x4 h;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t lo = bf16_rne(bf16_to_f32(a[e] & 0xFFFFu) + bf16_to_f32(b[e] & 0xFFFFu));
    const uint32_t hi = bf16_rne(bf16_to_f32(a[e] >> 16) + bf16_to_f32(b[e] >> 16));
    h[e] = lo | (hi << 16);
    const float hl = bf16_to_f32(lo), hh = bf16_to_f32(hi);
    ss = __builtin_fmaf(hl, hl, ss);
    ss = __builtin_fmaf(hh, hh, ss);
  }
  return h;
}

__device__ __forceinline__ float norm_wave_sum(float ss) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  return ss;
}

__device__ __forceinline__ float norm_inv(float total, int D, float eps) {
  return __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(total, (float)D) + eps));
}

__device__ __forceinline__ u32x4 norm_scale_chunk(u32x4 h, u32x4 w, float inv) {
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float nl = bf16_to_f32(bf16_rne(bf16_to_f32(h[e] & 0xFFFFu) * inv));
    const float nh = bf16_to_f32(bf16_rne(bf16_to_f32(h[e] >> 16) * inv));
    o[e] = bf16_rne(bf16_to_f32(w[e] & 0xFFFFu) * nl) | (bf16_rne(bf16_to_f32(w[e] >> 16) * nh) << 16);
  }
  return o;
}

// Dequantize one packed word (codes for k = 8c .. 8c+7) with its group's scale and bias.
// Result dword j holds bf16 for k = 8c+2j (low half) and 8c+2j+1 (high half).
//
// Even nibbles are isolated with one AND (bytes = q0, q2, q4, q6) and odd nibbles with another
// AND left in place (bytes = 16*q1, ...); v_cvt_f32_ubyte{0..3} turns each byte into a float.
// The odd codes are then scaled by s16 = s / 16, which is exact for every bf16 s (fp32 keeps
// the bits through its subnormal range), so fma(16q, s/16, b) == fma(q, s, b): s*q is exact in
// fp32 (8-bit by 4-bit significands) and the single rounding is the one of fp32(s*q + b).
// 22 VALU instructions per word: 2 AND, 8 cvt, 8 FMA, 4 cvt_pk.
__device__ __forceinline__ u32x4 dequant_word(uint32_t w, float s, float s16, float b) {
  uint32_t lo = w & 0x0F0F0F0Fu;
  uint32_t hi = w & 0xF0F0F0F0u;
  // Keep the two masks opaque so the backend emits v_cvt_f32_ubyteN on them instead of
  // re-deriving each nibble with v_bfe_u32 + v_cvt_f32_ubyte0 (one extra op per code).
  asm volatile("" : "+v"(lo), "+v"(hi));
  const float q0 = (float)(lo & 0xFFu), q2 = (float)((lo >> 8) & 0xFFu);
  const float q4 = (float)((lo >> 16) & 0xFFu), q6 = (float)(lo >> 24);
  const float h1 = (float)(hi & 0xFFu), h3 = (float)((hi >> 8) & 0xFFu);
  const float h5 = (float)((hi >> 16) & 0xFFu), h7 = (float)(hi >> 24);
  u32x4 r;
  r.x = pack_bf16x2(__builtin_fmaf(q0, s, b), __builtin_fmaf(h1, s16, b));
  r.y = pack_bf16x2(__builtin_fmaf(q2, s, b), __builtin_fmaf(h3, s16, b));
  r.z = pack_bf16x2(__builtin_fmaf(q4, s, b), __builtin_fmaf(h5, s16, b));
  r.w = pack_bf16x2(__builtin_fmaf(q6, s, b), __builtin_fmaf(h7, s16, b));
  return r;
}

// Faster exact dequantization of one word: 17 VALU instead of 22 (1 shift, 4 AND, 8 v_fma_mix_f32,
// 4 cvt_pk).
//
// Each AND leaves two codes in the low mantissa bits of the two fp16 halves of a dword, where they
// read as fp16 subnormals: q * 2^-24 (code at bits 0-3 of a byte) or 16q * 2^-24 (bits 4-7).
// v_fma_mix_f32 widens an fp16 half to fp32 exactly (fp16 subnormals are preserved: the kernels
// run with denormal mode 3) and computes, with one rounding,
//     fma(q * 2^-24,   s * 2^24, b) = s*q + b
//     fma(16q * 2^-24, s * 2^20, b) = s*q + b
// so the result is fp32_rne(s*q + b), bit-identical to dequant_word, whenever s * 2^24 is finite
// (|s| < 2^104, see fast_scale_ok). s24 = s * 2^24 and s20 = s * 2^20 are exact multiplications.
__device__ __forceinline__ u32x4 dequant_word_fast(uint32_t w, float s24, float s20, float b) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const uint32_t w8 = w >> 8;
  const h2 d0 = __builtin_bit_cast(h2, w & 0x000F000Fu);   // k0, k4
  const h2 d1 = __builtin_bit_cast(h2, w & 0x00F000F0u);   // k1, k5 (x16)
  const h2 d2 = __builtin_bit_cast(h2, w8 & 0x000F000Fu);  // k2, k6
  const h2 d3 = __builtin_bit_cast(h2, w8 & 0x00F000F0u);  // k3, k7 (x16)
  u32x4 r;
  r.x = pack_bf16x2(__builtin_fmaf((float)d0.x, s24, b), __builtin_fmaf((float)d1.x, s20, b));
  r.y = pack_bf16x2(__builtin_fmaf((float)d2.x, s24, b), __builtin_fmaf((float)d3.x, s20, b));
  r.z = pack_bf16x2(__builtin_fmaf((float)d0.y, s24, b), __builtin_fmaf((float)d1.y, s20, b));
  r.w = pack_bf16x2(__builtin_fmaf((float)d2.y, s24, b), __builtin_fmaf((float)d3.y, s20, b));
  return r;
}

// dequant_word_fast is exact for a bf16 scale with exponent field <= 230 (|s| < 2^104, so s * 2^24
// is finite): every finite scale of practical size, zero and subnormal included. Larger and
// non-finite scales take dequant_word.
__device__ __forceinline__ bool fast_scale_ok(uint32_t sbits) { return (sbits & 0x7F80u) <= (230u << 7); }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// MFMA tiles used here (gfx950 bf16, fp32 accumulation).
//   16x16x32: A lane l holds row l%16, k-chunk l/16 (8 values); B lane l holds column l%16,
//             k-chunk l/16; D lane l, element r holds row 4*(l/16)+r, column l%16.
//   32x32x16: A lane l holds row l%32, k-chunk l/32; B lane l holds column l%32, k-chunk l/32;
//             D lane l, element r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
// Products pair A and B values held at the same (lane group, element) position, so any
// permutation of K applied identically to both operands gives the same sum; the kernels use
// that freedom to give each lane contiguous packed words.
template <int MT>
struct Mfma;

template <>
struct Mfma<16> {
  typedef f32x4 Acc;
  static constexpr int kAcc = 4;
  __device__ static __forceinline__ Acc mma(bf16x8 a, bf16x8 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ int row(int lane, int r) { return 4 * (lane >> 4) + r; }
};

template <>
struct Mfma<32> {
  typedef f32x16 Acc;
  static constexpr int kAcc = 16;
  __device__ static __forceinline__ Acc mma(bf16x8 a, bf16x8 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ int row(int lane, int r) {
    return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
  }
};

}  // namespace qmm4
