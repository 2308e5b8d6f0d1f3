// Verify-shape quantized matmul for M = 1..64 rows: y = x @ dequant(w)^T.
//
// Serves the tree-verify, batched-verify and vocabulary-head shapes (the reference's NAX verify
// tiles and multi-row kernel, src/mlx_tree_spec/qmm_packed.py:151-220, 296-394), reading MLX's own
// [N, K/8] layout. Every packed weight is read once and used for all M rows (HBM-bound).
//
//  * Tiles: CW = 16 C output columns. A unit is (tile, step), a step being V super-steps of 128 k.
//    The T * NS units are split into G equal contiguous ranges, one per workgroup (stream-K).
//  * Inside a workgroup every wave works on the same tile, on different steps: the tile's steps in
//    the range go round-robin to the W waves, so each wave streams its own k-slices of the tile's
//    C * 16 weight rows and accumulates all M rows for all of them (MFMA 16x16x32, bf16 inputs,
//    fp32 sums). When the tile ends the waves' sums meet in LDS and are added in wave order
//    (deterministic), then stored as bf16 (a tile interior to the range) or as an fp32 partial (a
//    tile shared with the neighbouring workgroup; the last of its contributors adds the partials
//    in contributor order).
//  * Operands come straight from global memory into registers through a PF-unit ring: the lane's
//    pieces of the weight rows (lane (n = lane % 16, g = lane / 16) holds row n of each column
//    block, V 16-byte pieces at byte 64 v + 16 g of the step's run, so each row is read as one
//    contiguous V * 64-byte run per step), its scales and biases, and its x fragments (x is small
//    and stays in L2). Each x fragment feeds C MFMAs, one per column block, so x traffic per
//    weight byte is 4 MB / C (MB = 16-row blocks of x).
//  * Word t of piece v holds k = 128 (V st + v) + 32 g + 8 t: the B operand of MFMA (v, t) after
//    exact dequantization in registers; the A operand of that MFMA, lane (m, g), holds x[m] at the
//    same 8 k.
//  * Dequantization: dequant_word_fast (bit-identical to bf16_rne(fp32(s) * q + fp32(b)) for every
//    scale below 2^104), or dequant_word for a unit in which one of the wave's rows has a scale
//    outside that range (a wave-uniform branch per unit).
#include <algorithm>
#include <type_traits>

#include "qmm4_common.h"
#include "qmm4_kernels.h"

namespace qmm4 {

namespace {

struct VerifyParams {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  float* part;    // [G][2][MB*C*64] f32x4 partial tiles (MFMA accumulator order)
  uint32_t* cnt;  // [T] arrival counters; zero before and after every launch
  int M, N, K;
  int NS;         // steps per tile = K / (128 V)
  int G;          // workgroups
  long long U;    // units = T * NS
};

template <int MB_, int C_, int V_, int PF_, int W_>
struct VerifyCfg {
  static constexpr int MB = MB_;  // 16-row blocks of x (M <= 16 MB)
  static constexpr int MP = 16 * MB;
  static constexpr int C = C_;    // 16-column blocks per tile
  static constexpr int CW = 16 * C;
  static constexpr int V = V_;    // super-steps per step
  static constexpr int PF = PF_;  // units in flight per wave
  static constexpr int W = W_;    // waves per workgroup
  static constexpr int kThreads = 64 * W;
  static_assert(V == 1 || V == 2 || V == 4, "steps of 1, 2 or 4 super-steps");
  static_assert(PF >= 1 && PF <= 3, "ring of 1..3 units");
  // LDS slots for the tile-end reduction: one f32x4 per (wave, row block, column block, lane).
  static constexpr int kSlotF4 = MB * C * 64;
  static constexpr size_t kLds = (size_t)W * kSlotF4 * 16;
};

template <int V>
struct SB {
  uint32_t d[V];  // the 2V bf16 scales (or biases) of one row for one step
};

template <int V>
__device__ __forceinline__ SB<V> load_sb(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
  SB<V> o;
  if constexpr (V == 4) {
    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    o.d[0] = t.x; o.d[1] = t.y; o.d[2] = t.z; o.d[3] = t.w;
  } else if constexpr (V == 2) {
    const u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    o.d[0] = t.x; o.d[1] = t.y;
  } else {
    o.d[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  }
  return o;
}

__device__ __forceinline__ long long range_start(int p, long long U, int G) { return (long long)p * U / G; }

// Workgroup owning unit u when U units are split into G ranges [p*U/G, (p+1)*U/G).
__device__ __forceinline__ int unit_owner(long long u, long long U, int G) {
  return (int)(((u + 1) * (long long)G + U - 1) / U) - 1;
}

// Device-coherent fp32 stores and loads (cache policy sc1: coherent across the XCDs' L2s).
constexpr int kCoherent = 16;
__device__ __forceinline__ void store_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, kCoherent);
}
__device__ __forceinline__ f32x4 load_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCoherent));
}

__device__ __forceinline__ void store_y(__amdgpu_buffer_rsrc_t r, uint32_t elem, float v) {
  __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu), r, elem * 2u, 0, 0);
}

// One ring slot: everything a wave needs for one unit.
template <class C>
struct Slot {
  u32x4 w[C::C][C::V];             // weight pieces, per column block and super-step
  SB<C::V> s[C::C], b[C::C];       // scales and biases, per column block
  u32x4 a[C::MB][C::V][4];         // x fragments, per row block, super-step and word
};

template <class C>
__global__ __launch_bounds__(C::kThreads) void verify_kernel(VerifyParams P) {
  constexpr int MB = C::MB, NC = C::C, V = C::V, PF = C::PF, W = C::W, CW = C::CW;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  f32x4* slots = reinterpret_cast<f32x4*>(lds);
  __shared__ int s_last[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int p = blockIdx.x;
  const int NS = P.NS;
  const int KG = P.K >> 6;

  const long long u0 = range_start(p, P.U, P.G);
  const long long u1 = range_start(p + 1, P.U, P.G);
  const int t0 = (int)(u0 / NS), st0 = (int)(u0 - (long long)t0 * NS);
  const int t_last = (int)((u1 - 1) / NS);
  const int st_end = (int)(u1 - (long long)t_last * NS);        // end step (exclusive) in t_last
  const bool first_shared = st0 != 0;
  const bool last_shared = st_end != NS;

  const int wrec = rsrc_bytes((unsigned long long)P.N * (P.K >> 1));
  const int srec = rsrc_bytes((unsigned long long)P.N * KG * 2);
  const int xrec = rsrc_bytes((unsigned long long)P.M * P.K * 2);
  // Offset past the end of every buffer (they stay below 2 GiB for this kernel): loads read zero.
  constexpr uint32_t kOut = 0x80000000u;

  // Steps [sbeg(t), send(t)) of tile t lie in this workgroup's range; wave w takes sbeg + w,
  // sbeg + w + W, ...
  auto sbeg = [&](int t) { return t == t0 ? st0 : 0; };
  auto send = [&](int t) { return t == t_last ? st_end : NS; };

  // Fetch cursor: the next unit of this wave's sequence to load (ft > t_last: none left).
  int ft = t0, fst = sbeg(t0) + wave;
  auto advance = [&](int& t, int& st) {
    st += W;
    while (t <= t_last && st >= send(t)) {
      ++t;
      st = t <= t_last ? sbeg(t) + wave : 0;
    }
  };
  // Normalise the start (this wave may have no step in the first tiles).
  {
    while (ft <= t_last && fst >= send(ft)) {
      ++ft;
      fst = ft <= t_last ? sbeg(ft) + wave : 0;
    }
  }
  int ctile = ft, cst = fst;  // compute cursor: the unit in the oldest ring slot

  Slot<C> ring[PF];
  auto fetch = [&](Slot<C>& sl) __attribute__((always_inline)) {
    const bool live = ft <= t_last;
    const int t = live ? ft : t0, st = live ? fst : 0;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(P.w), 0, live ? wrec : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.s), 0, live ? srec : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.b), 0, live ? srec : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.x), 0, live ? xrec : 0, kBufferRsrcWord3);
#pragma unroll
    for (int ct = 0; ct < NC; ++ct) {
      const int col = t * CW + ct * 16 + n;
      const uint32_t wo = col < P.N ? (uint32_t)col * (uint32_t)(P.K >> 1) + (uint32_t)g * 16u : kOut;
      const uint32_t so = col < P.N ? (uint32_t)col * (uint32_t)KG * 2u : kOut;
#pragma unroll
      for (int v = 0; v < V; ++v) sl.w[ct][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, wo + v * 64, st * V * 64, 0);
      sl.s[ct] = load_sb<V>(rs, so, st * 4 * V);
      sl.b[ct] = load_sb<V>(rb, so, st * 4 * V);
    }
#pragma unroll
    for (int rb2 = 0; rb2 < MB; ++rb2) {
      const int m = min(rb2 * 16 + n, P.M - 1);
      const uint32_t xo = ((uint32_t)m * (uint32_t)P.K + (uint32_t)g * 32u) * 2u;
#pragma unroll
      for (int v = 0; v < V; ++v)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
          sl.a[rb2][v][tt] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + (uint32_t)(v * 256 + tt * 16),
                                                                   st * V * 256, 0);
    }
    if (live) advance(ft, fst);
  };

  f32x4 acc[MB][NC];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      P.y, 0, rsrc_bytes((unsigned long long)P.M * P.N * 2), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      P.part, 0, rsrc_bytes((unsigned long long)P.G * 2 * C::kSlotF4 * 16), kBufferRsrcWord3);

  // Item it = (row block i, column block j, lane l) of a tile holds rows 16 i + 4 (l / 16) + r,
  // r = 0..3, of column 16 j + l % 16 (the MFMA accumulator layout).
  auto store_item = [&](int t, int it, const f32x4& v) __attribute__((always_inline)) {
    const int blk = it >> 6, ln = it & 63;
    const int i = blk / NC, j = blk - i * NC;
    const int col = t * CW + j * 16 + (ln & 15);
    const int mrow = i * 16 + 4 * (ln >> 4);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (mrow + r < P.M && col < P.N) store_y(ry, (uint32_t)((mrow + r) * P.N + col), v[r]);
  };

  // Close tile t: every wave leaves its sums in its LDS slot; after a barrier the workgroup adds
  // the slots in wave order and stores bf16 y, or the fp32 partial of a shared tile (slot 0 for the
  // range's first tile, 1 for its last).
  auto close_tile = [&](int t) __attribute__((always_inline)) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        slots[(size_t)wave * C::kSlotF4 + (i * NC + j) * 64 + lane] = acc[i][j];
        acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    __syncthreads();
    const bool shared = (t == t0 && first_shared) || (t == t_last && last_shared);
    const int pslot = t == t0 ? 0 : 1;
    const uint32_t pbase = (uint32_t)(p * 2 + pslot) * (uint32_t)C::kSlotF4;
    for (int it = tid; it < C::kSlotF4; it += C::kThreads) {
      f32x4 sum = slots[it];
#pragma unroll
      for (int ww = 1; ww < W; ++ww) {
        const f32x4 c = slots[(size_t)ww * C::kSlotF4 + it];
        sum[0] += c[0]; sum[1] += c[1]; sum[2] += c[2]; sum[3] += c[3];
      }
      if (shared)
        store_coherent4(rp, (pbase + (uint32_t)it) * 16u, sum);
      else
        store_item(t, it, sum);
    }
  };

  auto compute = [&](const Slot<C>& sl, auto fast) __attribute__((always_inline)) {
    constexpr bool FAST = decltype(fast)::value;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e2 = 2 * v + (g >> 1);
#pragma unroll
      for (int ct = 0; ct < NC; ++ct) {
        const uint32_t sbits = (sl.s[ct].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu;
        const uint32_t bbits = (sl.b[ct].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu;
        const float sf = bf16_to_f32(sbits), bf = bf16_to_f32(bbits);
        const float c1 = FAST ? sf * 16777216.0f : sf;
        const float c2 = FAST ? sf * 1048576.0f : sf * 0.0625f;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const u32x4 B = FAST ? dequant_word_fast(sl.w[ct][v][tt], c1, c2, bf)
                               : dequant_word(sl.w[ct][v][tt], c1, c2, bf);
#pragma unroll
          for (int i = 0; i < MB; ++i)
            acc[i][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(sl.a[i][v][tt]), as_bf16x8(B), acc[i][ct],
                                                                 0, 0, 0);
        }
      }
    }
  };

  // Tiles before the one holding this wave's first unit close with nothing from this wave.
  int tclosed = t0;  // next tile to close
  while (tclosed < ctile && tclosed <= t_last) close_tile(tclosed++);

#pragma unroll
  for (int j = 0; j < PF; ++j) fetch(ring[j]);

  // One unit from ring slot J: compute, refill the slot, close every tile that ends before the
  // next unit of this wave.
  auto unit = [&](auto jc) __attribute__((always_inline)) {
    constexpr int j = decltype(jc)::value;
    bool bad = false;
#pragma unroll
    for (int ct = 0; ct < NC; ++ct)
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int e2 = 2 * v + (g >> 1);
        bad |= !fast_scale_ok((ring[j].s[ct].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
      }
    if (__builtin_amdgcn_ballot_w64(bad) == 0)
      compute(ring[j], std::true_type{});
    else
      compute(ring[j], std::false_type{});
    fetch(ring[j]);
    advance(ctile, cst);
    while (tclosed < ctile && tclosed <= t_last) close_tile(tclosed++);
  };

  // This wave's unit count, so that the loop runs whole groups of PF units with no exit inside
  // its body (an exit between ring slots would give the loop header a path on which the slots'
  // loads arrive in another order, and the compiler would then wait there for every load).
  int nunits = 0;
  for (int t = t0; t <= t_last; ++t) {
    const int c = send(t) - sbeg(t) - wave;
    if (c > 0) nunits += (c + W - 1) / W;
  }
  int base = 0;
  for (; base + PF <= nunits; base += PF) {
    unit(std::integral_constant<int, 0>{});
    if constexpr (PF > 1) unit(std::integral_constant<int, 1>{});
    if constexpr (PF > 2) unit(std::integral_constant<int, 2>{});
  }
  if constexpr (PF > 1)
    if (base < nunits) unit(std::integral_constant<int, 0>{});
  if constexpr (PF > 2)
    if (base + 1 < nunits) unit(std::integral_constant<int, 1>{});
  while (tclosed <= t_last) close_tile(tclosed++);

  if (!first_shared && !last_shared) return;
  // Count in on the shared tiles once the partials are at the device's coherence point.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const int tt0 = first_shared ? t0 : t_last;
  const int tt1 = (first_shared && last_shared && t_last != t0) ? t_last : -1;
  if (tid == 0 || (tid == 64 && tt1 >= 0)) {
    const int tt = (tid == 0) ? tt0 : tt1;
    const long long tile0 = (long long)tt * NS;
    const int plo = unit_owner(tile0, P.U, P.G);
    const int phi = unit_owner(tile0 + NS - 1, P.U, P.G);
    const uint32_t prev = __hip_atomic_fetch_add(&P.cnt[tt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last[tid >> 6] = (prev == (uint32_t)(phi - plo)) ? 1 : 0;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int tt = k == 0 ? tt0 : tt1;
    if (tt < 0 || !s_last[k]) continue;
    const long long tile0 = (long long)tt * NS;
    const int plo = unit_owner(tile0, P.U, P.G);
    const int phi = unit_owner(tile0 + NS - 1, P.U, P.G);
    // Contributor plo holds this tile in its slot 1 iff its range began in an earlier tile.
    const int lo_slot = (range_start(plo, P.U, P.G) < tile0) ? 1 : 0;
    const int nq = phi - plo + 1;
    // Loads go out in batches of kE items x kQ contributors per thread, all independent, so a
    // batch costs one memory round trip; sums run in contributor order.
    constexpr int kPer = C::kSlotF4 / C::kThreads;
    constexpr int kE = kPer < 1 ? 1 : kPer > 4 ? 4 : kPer, kQ = 4;
    static_assert(C::kSlotF4 < C::kThreads || C::kSlotF4 % (C::kThreads * kE) == 0, "whole batches of items");
    for (int base = tid; base < C::kSlotF4; base += C::kThreads * kE) {
      f32x4 sum[kE];
#pragma unroll
      for (int e = 0; e < kE; ++e) sum[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int q0 = 0; q0 < nq; q0 += kQ) {
        f32x4 v[kE][kQ];
#pragma unroll
        for (int e = 0; e < kE; ++e)
#pragma unroll
          for (int j = 0; j < kQ; ++j) {
            const int q = q0 + j;
            const uint32_t off = (q == 0) ? (uint32_t)(plo * 2 + lo_slot) * (uint32_t)C::kSlotF4
                                          : (uint32_t)((plo + q) * 2) * (uint32_t)C::kSlotF4;
            // Contributors past the last read zeros (an offset outside the resource).
            const uint32_t byte = q < nq ? (off + (uint32_t)(base + e * C::kThreads)) * 16u : 0x80000000u;
            v[e][j] = load_coherent4(rp, byte);
          }
#pragma unroll
        for (int e = 0; e < kE; ++e)
#pragma unroll
          for (int j = 0; j < kQ; ++j) {
            sum[e][0] += v[e][j][0]; sum[e][1] += v[e][j][1];
            sum[e][2] += v[e][j][2]; sum[e][3] += v[e][j][3];
          }
      }
#pragma unroll
      for (int e = 0; e < kE; ++e) store_item(tt, base + e * C::kThreads, sum[e]);
    }
    if (tid == 0) __hip_atomic_store(&P.cnt[tt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

// Kernel table: id -> (row blocks, column blocks, V, PF, waves).
#define QMM4_VERIFY_VARIANTS(X) \
  X(0, 1, 8, 1, 2, 4)           \
  X(1, 2, 8, 1, 2, 4)           \
  X(2, 4, 4, 1, 2, 4)           \
  X(3, 1, 8, 2, 2, 4)           \
  X(4, 2, 4, 2, 2, 4)           \
  X(5, 4, 2, 2, 2, 4)           \
  X(6, 1, 4, 2, 2, 8)           \
  X(7, 2, 4, 1, 2, 8)           \
  X(8, 4, 2, 1, 2, 8)           \
  X(9, 1, 4, 4, 2, 4)

#define QMM4_VCFG(id, mb, c, v, pf, w) typedef VerifyCfg<mb, c, v, pf, w> VCfg##id;
QMM4_VERIFY_VARIANTS(QMM4_VCFG)
#undef QMM4_VCFG

static const void* verify_func(int variant) {
  switch (variant) {
#define QMM4_VF(id, mb, c, v, pf, w) \
  case id: return reinterpret_cast<const void*>(&verify_kernel<VCfg##id>);
    QMM4_VERIFY_VARIANTS(QMM4_VF)
#undef QMM4_VF
    default: return nullptr;
  }
}

static void verify_geometry(int variant, int* cw, int* v, int* threads, size_t* lds, size_t* item_bytes = nullptr) {
  if (item_bytes) *item_bytes = 0;
  switch (variant) {
#define QMM4_VG(id, mb, c, vv, pf, w)                                                                       \
  case id:                                                                                                  \
    *cw = VCfg##id::CW; *v = VCfg##id::V; *threads = VCfg##id::kThreads; *lds = VCfg##id::kLds;             \
    if (item_bytes) *item_bytes = (size_t)VCfg##id::kSlotF4 * 16;                                           \
    return;
    QMM4_VERIFY_VARIANTS(QMM4_VG)
#undef QMM4_VG
    default: *cw = 0; *v = 0; *threads = 0; *lds = 0;
  }
}

int verify_variant(int M, int vmax) {
  const int mb = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  int id = mb == 1 ? 3 : mb == 2 ? 1 : 2;  // preferred variant per row blocks
  int cw, v, threads;
  size_t lds;
  verify_geometry(id, &cw, &v, &threads, &lds);
  if (v > vmax) id = mb == 1 ? 0 : mb == 2 ? 1 : 2;
  return id;
}

int verify_occupancy(int variant) {
  int cw, v, threads;
  size_t lds;
  verify_geometry(variant, &cw, &v, &threads, &lds);
  const void* f = verify_func(variant);
  if (!f) return 1;
  if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) return 1;
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, threads, lds) != hipSuccess) return 1;
  return nb > 0 ? nb : 1;
}

bool verify_plan(int M, int N, int K, int vmax, int cus, int occ, VerifyPlan* plan) {
  if (M < 1 || M > 64) return false;
  const int variant = verify_variant(M, vmax);
  int cw, v, threads;
  size_t lds, item_bytes;
  verify_geometry(variant, &cw, &v, &threads, &lds, &item_bytes);
  const int ks = K / 128;
  if (ks % v != 0) return false;
  // Row offsets of this kernel stay below 2 GiB (rows past the end are addressed at 2 GiB).
  if ((unsigned long long)(N + 256) * (unsigned long long)K / 2 >= (1ULL << 31)) return false;
  plan->variant = variant;
  plan->tile_cols = cw;
  plan->steps_v = v;
  plan->tiles = (N + cw - 1) / cw;
  plan->units = (long long)plan->tiles * (ks / v);
  long long slots = (long long)cus * std::max(1, occ);
  // At least one unit per wave of a workgroup.
  const long long cap = std::max(1LL, plan->units / 4);
  if (slots > cap) slots = cap;
  plan->blocks = (int)std::max(1LL, slots);
  plan->threads = threads;
  plan->lds = lds;
  plan->part_bytes = (size_t)plan->blocks * 2 * item_bytes;
  return true;
}

hipError_t launch_verify(const VerifyPlan& plan, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                         const uint16_t* b, uint16_t* y, float* part, uint32_t* cnt, int M, int N, int K,
                         hipStream_t stream) {
  VerifyParams P;
  P.x = x; P.w = w; P.s = s; P.b = b; P.y = y; P.part = part; P.cnt = cnt;
  P.M = M; P.N = N; P.K = K;
  P.NS = K / (128 * plan.steps_v);
  P.G = plan.blocks;
  P.U = plan.units;
  const dim3 grid((unsigned)plan.blocks), block((unsigned)plan.threads);
  switch (plan.variant) {
#define QMM4_VL(id, mb, c, v, pf, w) \
  case id: hipLaunchKernelGGL(verify_kernel<VCfg##id>, grid, block, plan.lds, stream, P); break;
    QMM4_VERIFY_VARIANTS(QMM4_VL)
#undef QMM4_VL
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace qmm4
