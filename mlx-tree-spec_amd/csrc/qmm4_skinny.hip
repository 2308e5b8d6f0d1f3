// Skinny quantized matmul for M = 1..64 rows (decode, tree verify): y = x @ dequant(w)^T.
//
// Replaces the reference's M <= 64 kernels (qmv_packed, the NAX verify tiles and the multi-row
// NAX kernel: src/mlx_tree_spec/qmm_packed.py:151-220, 296-394, 428-557) with one design that
// reads MLX's own [N, K/8] layout directly (no install-time relayout).
//
// The regime is HBM-bound: every packed weight is read once and used for all M rows.
//  * Work decomposition (stream-K): output columns are cut into tiles of CW columns; the tile's
//    K is cut into 128-wide super-steps (two quantization groups). The T*KS (tile, super-step)
//    units are split into G equal contiguous ranges, one per workgroup, so every workgroup
//    streams the same number of weight bytes whatever N and K are. A range that covers a whole
//    tile writes bf16 directly; a tile shared by several workgroups is summed from fp32 partials
//    by the last workgroup to finish it, in workgroup order (deterministic).
//  * Within a workgroup (4 waves), each wave owns CT column tiles of MT columns. Each lane loads
//    the packed words of one column with 16-B loads (prefetched PF super-steps ahead),
//    dequantizes them bit-exactly in registers and feeds them as the MFMA B operand; dequantized
//    weights never touch LDS. The activation slice x[:, k-range] is staged once per chunk of KC
//    super-steps in LDS, already in MFMA fragment order, and shared by all waves and column
//    tiles (rows >= M are zero).
//  * MFMA: 16x16x32 for M <= 16 (MT = 16), 32x32x16 for M <= 32 / 64 (MT = 32, MB = 1 / 2 row
//    blocks). K inside a super-step is permuted so that a lane's packed words are contiguous:
//    lane (column c, lane group g) takes words [g*ST, g*ST + ST) of the super-step's 16 words and
//    MFMA step t uses word g*ST + t; the activation fragment of lane (row r, g) at step t holds
//    x[r][128*ss + 2*MT*g + 8*t .. +8], the same k values.
#include "qmm4_common.h"
#include "qmm4_kernels.h"

namespace qmm4 {

struct SkinnyParams {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  float* part;    // [G][2][M][CW] fp32 partial tiles
  uint32_t* cnt;  // [T] arrival counters; zero before and after every launch
  int M, N, K;
  int KS;         // super-steps per tile = K / 128
  int G;          // workgroups
  long long U;    // units = T * KS
};

template <int MT_, int MB_, int CT_, int KC_, int PF_>
struct SkinnyCfg {
  static constexpr int MT = MT_, MB = MB_, CT = CT_, KC = KC_, PF = PF_;
  static constexpr int kWaves = 4;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int ST = MT / 4;              // MFMA steps (and words per lane) per super-step
  static constexpr int NV = ST / 4;              // 16-B word loads per lane per super-step
  static constexpr int CW = kWaves * CT * MT;    // columns per tile
  static constexpr int MPAD = MT * MB;
  static constexpr int SS_UNITS = ST * MB * 64;  // 16-B LDS units per staged super-step
};

// Workgroup owning unit u when U units are split into G ranges [p*U/G, (p+1)*U/G).
__device__ __forceinline__ int unit_owner(long long u, long long U, int G) {
  return (int)(((u + 1) * (long long)G + U - 1) / U) - 1;
}

__device__ __forceinline__ long long range_start(int p, long long U, int G) {
  return (long long)p * U / G;
}

// Stage x[0:MPAD, 128*ss0 : 128*ss1] into LDS in fragment order (rows >= M are zeros).
template <class C>
__device__ __forceinline__ void stage_x(u32x4* xs, const uint16_t* __restrict__ x, int M, int K,
                                        int ss0, int ss1) {
  const int nss = ss1 - ss0;
  const int per_row = nss * 16;  // 16-B chunks per row in the range
  const int total = C::MPAD * per_row;
  for (int idx = threadIdx.x; idx < total; idx += C::kThreads) {
    const int m = idx / per_row;
    const int rem = idx - m * per_row;
    const int dssl = rem >> 4;
    const int within = (rem & 15) * 8;  // k offset inside the super-step
    const int gg = within / (2 * C::MT);
    const int tt = (within % (2 * C::MT)) >> 3;
    const int rb = m / C::MT;
    const int lnn = (m % C::MT) + C::MT * gg;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (m < M)
      v = *reinterpret_cast<const u32x4*>(x + (size_t)m * K + (size_t)(ss0 + dssl) * 128 + within);
    xs[((dssl * C::ST + tt) * C::MB + rb) * 64 + lnn] = v;
  }
}

// At most 256 VGPRs per lane (two waves per SIMD): without the cap the scheduler hoists every
// dequantized fragment of a super-step and the 32-row variants fall to one wave per SIMD.
template <class C>
__global__ __launch_bounds__(C::kThreads) __attribute__((amdgpu_waves_per_eu(2))) void skinny_kernel(
    SkinnyParams P) {
  using F = Mfma<C::MT>;
  typedef typename F::Acc Acc;
  constexpr int MT = C::MT, MB = C::MB, CT = C::CT, ST = C::ST, NV = C::NV, PF = C::PF;
  constexpr int CW = C::CW;

  __shared__ u32x4 xs[C::KC * C::SS_UNITS];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane % MT;
  const int g = lane / MT;
  const int p = blockIdx.x;
  const long long u0 = range_start(p, P.U, P.G);
  const long long u1 = range_start(p + 1, P.U, P.G);
  const size_t KW = (size_t)(P.K >> 3);
  const size_t KG = (size_t)(P.K >> 6);

  int seg = 0;
  for (long long u = u0; u < u1; ++seg) {
    const int t = (int)(u / P.KS);
    const int a = (int)(u - (long long)t * P.KS);
    const long long left = u1 - u;
    const int e = (left < (long long)(P.KS - a)) ? a + (int)left : P.KS;
    u += e - a;

    // This lane's column in each of its column tiles (clamped to row 0 past N: loaded, never stored).
    const uint32_t* wp[CT];
    const uint16_t* sp[CT];
    const uint16_t* bp[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int n = t * CW + (wave * CT + ct) * MT + c;
      const size_t nn = (n < P.N) ? (size_t)n : 0;
      wp[ct] = P.w + nn * KW + g * ST;
      sp[ct] = P.s + nn * KG + (g * MT) / 32;
      bp[ct] = P.b + nn * KG + (g * MT) / 32;
    }

    Acc acc[MB][CT];
#pragma unroll
    for (int rb = 0; rb < MB; ++rb)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int r = 0; r < F::kAcc; ++r) acc[rb][ct][r] = 0.0f;

    u32x4 wv[PF][CT][NV];
    uint32_t sv[PF][CT], bv[PF][CT];
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int ss = a + j;
      if (ss < e) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
          for (int v = 0; v < NV; ++v)
            wv[j][ct][v] = *reinterpret_cast<const u32x4*>(wp[ct] + (size_t)ss * 16 + 4 * v);
          sv[j][ct] = sp[ct][2 * ss];
          bv[j][ct] = bp[ct][2 * ss];
        }
      }
    }

    for (int base = a; base < e; base += PF) {
#pragma unroll
      for (int j = 0; j < PF; ++j) {
        const int ss = base + j;
        if (ss < e) {
          const int rel = ss - a;
          if (rel % C::KC == 0) {
            __syncthreads();
            stage_x<C>(xs, P.x, P.M, P.K, ss, min(e, ss + C::KC));
            __syncthreads();
          }
          const u32x4* xa = xs + (rel % C::KC) * C::SS_UNITS + lane;
          float sf[CT], s16[CT], bf[CT];
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            sf[ct] = bf16_to_f32(sv[j][ct]);
            s16[ct] = sf[ct] * 0.0625f;
            bf[ct] = bf16_to_f32(bv[j][ct]);
          }
#pragma unroll
          for (int tt = 0; tt < ST; ++tt) {
            bf16x8 A[MB];
#pragma unroll
            for (int rb = 0; rb < MB; ++rb) A[rb] = as_bf16x8(xa[(tt * MB + rb) * 64]);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
              const uint32_t word = wv[j][ct][tt >> 2][tt & 3];
              const bf16x8 B = as_bf16x8(dequant_word(word, sf[ct], s16[ct], bf[ct]));
#pragma unroll
              for (int rb = 0; rb < MB; ++rb) acc[rb][ct] = F::mma(A[rb], B, acc[rb][ct]);
            }
          }
          const int nx = ss + PF;
          if (nx < e) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
              for (int v = 0; v < NV; ++v)
                wv[j][ct][v] = *reinterpret_cast<const u32x4*>(wp[ct] + (size_t)nx * 16 + 4 * v);
              sv[j][ct] = sp[ct][2 * nx];
              bv[j][ct] = bp[ct][2 * nx];
            }
          }
        }
      }
    }

    if (a == 0 && e == P.KS) {
      // Whole tile in this range: write bf16 directly.
#pragma unroll
      for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int n = t * CW + (wave * CT + ct) * MT + c;
#pragma unroll
          for (int r = 0; r < F::kAcc; ++r) {
            const int m = rb * MT + F::row(lane, r);
            if (m < P.M && n < P.N) P.y[(size_t)m * P.N + n] = (uint16_t)(pack_bf16x2(acc[rb][ct][r], 0.0f) & 0xFFFFu);
          }
        }
    } else {
      // Partial tile: publish fp32 partials, count arrivals, the last arrival reduces.
      const int slot = (seg == 0) ? 0 : 1;
      float* pp = P.part + ((size_t)p * 2 + slot) * (size_t)P.M * CW;
#pragma unroll
      for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int cl = (wave * CT + ct) * MT + c;
#pragma unroll
          for (int r = 0; r < F::kAcc; ++r) {
            const int m = rb * MT + F::row(lane, r);
            if (m < P.M) pp[(size_t)m * CW + cl] = acc[rb][ct][r];
          }
        }
      __threadfence();
      __syncthreads();
      const long long tile0 = (long long)t * P.KS;
      const int plo = unit_owner(tile0, P.U, P.G);
      const int phi = unit_owner(tile0 + P.KS - 1, P.U, P.G);
      if (tid == 0) {
        const uint32_t prev = atomicAdd(&P.cnt[t], 1u);
        s_last = (prev == (uint32_t)(phi - plo)) ? 1 : 0;
      }
      __syncthreads();
      if (s_last) {
        __threadfence();
        const int total = P.M * CW;
        for (int idx = tid; idx < total; idx += C::kThreads) {
          const int m = idx / CW;
          const int cl = idx - m * CW;
          float sum = 0.0f;
          for (int q = plo; q <= phi; ++q) {
            const int qs = (range_start(q, P.U, P.G) >= tile0) ? 0 : 1;
            sum += P.part[((size_t)q * 2 + qs) * (size_t)P.M * CW + idx];
          }
          const int n = t * CW + cl;
          if (n < P.N) P.y[(size_t)m * P.N + n] = (uint16_t)(pack_bf16x2(sum, 0.0f) & 0xFFFFu);
        }
        if (tid == 0) atomicExch(&P.cnt[t], 0u);
      }
    }
  }
}

// Kernel table: variant -> (MT, MB, CT, KC, PF).
typedef SkinnyCfg<16, 1, 2, 8, 4> CfgM16;   // M <= 16
typedef SkinnyCfg<32, 1, 2, 4, 4> CfgM32;   // M <= 32
typedef SkinnyCfg<32, 2, 1, 4, 4> CfgM64;   // M <= 64

int skinny_variant_for_rows(int M, int* tile_cols) {
  if (M <= 16) { *tile_cols = CfgM16::CW; return 0; }
  if (M <= 32) { *tile_cols = CfgM32::CW; return 1; }
  *tile_cols = CfgM64::CW;
  return 2;
}

static const void* skinny_func(int variant) {
  switch (variant) {
    case 0: return reinterpret_cast<const void*>(&skinny_kernel<CfgM16>);
    case 1: return reinterpret_cast<const void*>(&skinny_kernel<CfgM32>);
    default: return reinterpret_cast<const void*>(&skinny_kernel<CfgM64>);
  }
}

int skinny_occupancy(int variant) {
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, skinny_func(variant), 256, 0) != hipSuccess)
    return 1;
  return nb > 0 ? nb : 1;
}

hipError_t launch_skinny(const SkinnyPlan& plan, const uint16_t* x, const uint32_t* w,
                         const uint16_t* s, const uint16_t* b, uint16_t* y, float* part,
                         uint32_t* cnt, int M, int N, int K, hipStream_t stream) {
  SkinnyParams P;
  P.x = x; P.w = w; P.s = s; P.b = b; P.y = y; P.part = part; P.cnt = cnt;
  P.M = M; P.N = N; P.K = K; P.KS = K / 128; P.G = plan.blocks; P.U = plan.units;
  const dim3 grid((unsigned)plan.blocks), block(256);
  switch (plan.variant) {
    case 0: hipLaunchKernelGGL(skinny_kernel<CfgM16>, grid, block, 0, stream, P); break;
    case 1: hipLaunchKernelGGL(skinny_kernel<CfgM32>, grid, block, 0, stream, P); break;
    default: hipLaunchKernelGGL(skinny_kernel<CfgM64>, grid, block, 0, stream, P); break;
  }
  return hipGetLastError();
}

}  // namespace qmm4
