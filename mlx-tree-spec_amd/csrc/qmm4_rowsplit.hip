// Row-split decode kernel for up to 4 rows of x and many output columns: y = x @ dequant(w)^T.
//
// Same arithmetic and operand layout as the skinny kernel (qmm4_skinny.hip; replaces the
// reference's qmv_packed and 8/16-row NAX kernels for decode, src/mlx_tree_spec/qmm_packed.py:
// 151-220, 428-557), with a decomposition for the case where the output columns alone fill the
// GPU: workgroup p (one per CU, 12 waves) owns the R consecutive weight rows [p R, p R + R) over
// the whole of K, so workgroups share nothing and no partial sums leave a CU.
//
//  * Inside a workgroup, the RB = ceil(R / 16) row blocks x K/128 super-steps are one sequence
//    (block-major) cut into 12 equal contiguous wave ranges; a wave streams its range as one
//    pipeline of units of V super-steps (weights PF units ahead in a register ring), and
//    accumulates each block it touches with MFMA 16x16x32 (bf16, fp32 accumulation).
//  * Loads: lane (n = lane % 16, g = lane / 16) of a wave holds weight row 16 b + n of its block;
//    in a unit it loads V 16-byte pieces of that row, piece v at byte 64 v + 16 g of the unit's
//    V * 64-byte run, so each row is read as one contiguous run per unit. Rows past the workgroup's
//    range read as zero (an offset outside the buffer resource), as do prefetches past a wave's
//    range (a zero-length resource).
//  * x (M <= 4 rows, whole K) is staged once in LDS in A-fragment order, behind the first weight
//    prefetches; the stream has no barrier.
//  * Dequantization: dequant_word_fast, or dequant_word for a unit in which one of the wave's
//    rows has a scale outside the fast form's range (a wave-uniform branch per unit).
//  * At the end each wave leaves its per-block fp32 sums in LDS; after one barrier the workgroup
//    adds the contributions to each block in wave order (deterministic) and writes bf16 y.
#include <type_traits>

#include "qmm4_common.h"
#include "qmm4_kernels.h"

namespace qmm4 {

namespace {

constexpr int kRsWaves = 12;
constexpr int kRsThreads = 64 * kRsWaves;
constexpr int kRsMP = 4;  // x rows held per fragment (M <= 4)
constexpr int kRsPF = 2;
// A wave's range covers at most two row blocks (the launch keeps a range no longer than K).
constexpr int kRsSlots = 2;

struct RowSplitParams {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int M, N, K;
  int R;    // weight rows per workgroup (a multiple of 8)
  int RB;   // 16-row blocks per workgroup, ceil(R / 16)
  int IPW;  // super-steps (128 k) per wave range, a multiple of V, at most K / 128
};

template <int V>
struct Scales {
  uint32_t d[V];  // the 2V bf16 scales (or biases) of one row for one unit
};

template <int V>
__device__ __forceinline__ Scales<V> load_scales(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
  Scales<V> o;
  if constexpr (V == 5) {
    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    o.d[0] = t.x; o.d[1] = t.y; o.d[2] = t.z; o.d[3] = t.w;
    o.d[4] = __builtin_amdgcn_raw_buffer_load_b32(r, voff + 16u, soff, 0);
  } else {
    static_assert(V == 4, "units of 4 or 5 super-steps");
    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    o.d[0] = t.x; o.d[1] = t.y; o.d[2] = t.z; o.d[3] = t.w;
  }
  return o;
}

template <int V>
__global__ __launch_bounds__(kRsThreads) __attribute__((amdgpu_waves_per_eu(3)))
void rowsplit_kernel(RowSplitParams P) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int S = P.K >> 7;                       // super-steps per row
  const int SU = S / V;                         // units per row block
  u32x4* xs = reinterpret_cast<u32x4*>(lds);    // [S][16][kRsMP] x pieces (A-fragment order)
  f32x4* part = reinterpret_cast<f32x4*>(lds + (size_t)S * 16 * kRsMP * sizeof(u32x4));  // [waves][slots][64]

  const int tid = threadIdx.x;
  // The wave index is uniform across the wave; readfirstlane tells the compiler so (the wave's
  // range then lives in scalar registers and its buffer resources need no per-lane loop).
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int r0 = blockIdx.x * P.R;
  const int r1 = min(P.N, r0 + P.R);
  const int KG = P.K >> 6;

  // This wave's range, in units of the workgroup's block-major sequence.
  const int su0 = wave * P.IPW;
  const int su1 = min(su0 + P.IPW, P.RB * S);
  const int ub = su0 / V, ue = su1 > su0 ? su1 / V : ub;
  const int nunits = ue - ub;
  const int b_first = su0 / S;

  const int wrec = rsrc_bytes((unsigned long long)P.N * (P.K >> 1));
  const int srec = rsrc_bytes((unsigned long long)P.N * KG * 2);
  // Offset of a row outside the workgroup's range: past the end of every buffer (they are kept
  // below 1 GiB for this kernel), so its loads return zero.
  constexpr uint32_t kOut = 0x40000000u;

  u32x4 wv[kRsPF][V];
  Scales<V> sv[kRsPF], bv[kRsPF];
  int fi = 0;        // index of the next unit to fetch, relative to ub
  auto fetch = [&](int j) __attribute__((always_inline)) {
    const bool live = fi < nunits;
    const int u = ub + (live ? fi : 0);
    const int b = u / SU, st = u - b * SU;
    const int row = r0 + b * 16 + n;
    const uint32_t wo = row < r1 ? (uint32_t)row * (uint32_t)(P.K >> 1) + (uint32_t)g * 16u : kOut;
    const uint32_t so = row < r1 ? (uint32_t)row * (uint32_t)KG * 2u : kOut;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(P.w), 0, live ? wrec : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.s), 0, live ? srec : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.b), 0, live ? srec : 0, kBufferRsrcWord3);
#pragma unroll
    for (int v = 0; v < V; ++v) wv[j][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, wo + v * 64, st * V * 64, 0);
    sv[j] = load_scales<V>(rs, so, st * 4 * V);
    bv[j] = load_scales<V>(rb, so, st * 4 * V);
    ++fi;
  };
#pragma unroll
  for (int j = 0; j < kRsPF; ++j) fetch(j);

  // x, whole K, behind the first prefetches: piece (ss, q) of row m at ((ss * 16 + q) * MP + m).
  for (int i = tid; i < S * 16 * kRsMP; i += kRsThreads) {
    const int m = i & (kRsMP - 1), sq = i >> 2;
    if (m < P.M) xs[sq * kRsMP + m] = *reinterpret_cast<const u32x4*>(P.x + (size_t)m * P.K + (size_t)sq * 8);
  }
  __syncthreads();

  const int aoff = g * 4 * kRsMP + min(n, P.M - 1);
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  int b_cur = b_first;

  auto flush = [&](int b) __attribute__((always_inline)) {
    part[(wave * kRsSlots + (b - b_first)) * 64 + lane] = acc;
    acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  };

  auto compute = [&](int j, int st, auto fast) __attribute__((always_inline)) {
    constexpr bool FAST = decltype(fast)::value;
    const u32x4* xb = xs + (size_t)st * V * 16 * kRsMP;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e2 = 2 * v + (g >> 1);
      const uint32_t sbits = (sv[j].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu;
      const uint32_t bbits = (bv[j].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu;
      const float sf = bf16_to_f32(sbits), bf = bf16_to_f32(bbits);
      const float c1 = FAST ? sf * 16777216.0f : sf;
      const float c2 = FAST ? sf * 1048576.0f : sf * 0.0625f;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const u32x4 B = FAST ? dequant_word_fast(wv[j][v][tt], c1, c2, bf) : dequant_word(wv[j][v][tt], c1, c2, bf);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xb[(v * 16 + tt) * kRsMP + aoff]), as_bf16x8(B), acc,
                                                      0, 0, 0);
      }
    }
  };

  // One unit: consume ring slot J, refill it, close the block when it ends here.
  auto unit = [&](int i, auto jc) __attribute__((always_inline)) {
    constexpr int j = decltype(jc)::value;
    const int u = ub + i;
    const int b = u / SU, st = u - b * SU;
    if (b != b_cur) {
      flush(b_cur);
      b_cur = b;
    }
    bool bad = false;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e2 = 2 * v + (g >> 1);
      bad |= !fast_scale_ok((sv[j].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
    }
    if (__builtin_amdgcn_ballot_w64(bad) == 0)
      compute(j, st, std::true_type{});
    else
      compute(j, st, std::false_type{});
    fetch(j);
  };

  int i = 0;
  for (; i + kRsPF <= nunits; i += kRsPF) {
    unit(i, std::integral_constant<int, 0>{});
    unit(i + 1, std::integral_constant<int, 1>{});
  }
  if (i < nunits) unit(i, std::integral_constant<int, 0>{});
  if (nunits > 0) flush(b_cur);
  __syncthreads();

  // Sum each block's contributions in wave order; lane (n, g) element r is x row 4 g + r, weight
  // row 16 b + n of the block.
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      P.y, 0, rsrc_bytes((unsigned long long)P.M * P.N * 2), kBufferRsrcWord3);
  for (int idx = tid; idx < P.RB * 64; idx += kRsThreads) {
    const int b = idx >> 6, l = idx & 63;
    const int ln = l & 15, lg = l >> 4;
    const int row = r0 + b * 16 + ln;
    if (4 * lg >= P.M || row >= r1) continue;
    const int w0 = (b * S) / P.IPW, w1 = min(kRsWaves - 1, ((b + 1) * S - 1) / P.IPW);
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int wv2 = w0; wv2 <= w1; ++wv2) {
      const int slot = b - (wv2 * P.IPW) / S;
      const f32x4 c = part[(wv2 * kRsSlots + slot) * 64 + l];
      sum[0] += c[0]; sum[1] += c[1]; sum[2] += c[2]; sum[3] += c[3];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * lg + r;
      if (m < P.M)
        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(pack_bf16x2(sum[r], 0.0f) & 0xFFFFu), ry,
                                              (uint32_t)(m * P.N + row) * 2u, 0, 0);
    }
  }
}

template <int V>
size_t rowsplit_smem(int K) {
  return (size_t)(K >> 7) * 16 * kRsMP * sizeof(u32x4) + (size_t)kRsWaves * kRsSlots * 64 * sizeof(f32x4);
}

}  // namespace

bool rowsplit_plan(int M, int N, int K, int cus, RowSplitPlan* plan) {
  if (M < 1 || M > kRsMP || cus < 1) return false;
  const int S = K >> 7;
  const int V = S % 5 == 0 ? 5 : S % 4 == 0 ? 4 : 0;
  if (V == 0) return false;
  const int R = ((N + cus - 1) / cus + 7) / 8 * 8;
  const int RB = (R + 15) / 16;
  // Enough blocks for every wave (a range no longer than one row of K), and the same smem budget.
  int IPW = (RB * S + kRsWaves - 1) / kRsWaves;
  IPW = (IPW + V - 1) / V * V;
  if (RB < 4 || IPW > S) return false;
  const size_t smem = V == 5 ? rowsplit_smem<5>(K) : rowsplit_smem<4>(K);
  if (smem > 160 * 1024) return false;
  // Row offsets of this kernel stay below 1 GiB.
  if ((unsigned long long)(N + 256) * (unsigned long long)K / 2 >= (1ULL << 30)) return false;
  plan->V = V;
  plan->R = R;
  plan->RB = RB;
  plan->IPW = IPW;
  plan->blocks = (N + R - 1) / R;
  plan->smem = smem;
  return true;
}

hipError_t launch_rowsplit(const RowSplitPlan& plan, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                           const uint16_t* b, uint16_t* y, int M, int N, int K, hipStream_t stream) {
  RowSplitParams P;
  P.x = x; P.w = w; P.s = s; P.b = b; P.y = y;
  P.M = M; P.N = N; P.K = K;
  P.R = plan.R; P.RB = plan.RB; P.IPW = plan.IPW;
  const void* f = plan.V == 5 ? reinterpret_cast<const void*>(&rowsplit_kernel<5>)
                              : reinterpret_cast<const void*>(&rowsplit_kernel<4>);
  static bool attr_set[2] = {false, false};
  const int vi = plan.V == 5 ? 1 : 0;
  if (!attr_set[vi]) {
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set[vi] = true;
  }
  if (plan.V == 5)
    hipLaunchKernelGGL(rowsplit_kernel<5>, dim3(plan.blocks), dim3(kRsThreads), plan.smem, stream, P);
  else
    hipLaunchKernelGGL(rowsplit_kernel<4>, dim3(plan.blocks), dim3(kRsThreads), plan.smem, stream, P);
  return hipGetLastError();
}

}  // namespace qmm4
