// Skinny quantized matmul for M = 1..64 rows (decode, tree verify): y = x @ dequant(w)^T.
//
// Replaces the reference's M <= 64 kernels (qmv_packed, the NAX verify tiles and the multi-row
// NAX kernel: src/mlx_tree_spec/qmm_packed.py:151-220, 296-394, 428-557) with one design that
// reads MLX's own [N, K/8] layout directly (no install-time relayout).
//
// The regime is HBM-bound: every packed weight is read once and used for all M rows.
//  * Loads: MFMA 16x16x32 (bf16, fp32 accumulation). A wave owns 16 output columns per column
//    block; lane (n = lane % 16, g = lane / 16) holds column n. A "step" is V super-steps of 128 k
//    (V*64 bytes of each weight row); in it the lane loads V 16-byte pieces of its row, piece v at
//    byte 64*v + 16*g, so the four lanes of a column read each 64-byte segment together and every
//    row is read as one contiguous V*64-byte run per step (row runs are what HBM streams fast:
//    16-byte pieces from 32 scattered rows per instruction stream at half the rate).
//    Word t of piece v holds k = 128*(V*step + v) + 32*g + 8*t; it is the B operand of MFMA (v, t)
//    after exact dequantization in registers. The A operand of that MFMA, lane (m, g), holds
//    x[m][the same 8 k].
//  * Dequantization: dequant_word_fast (v_fma_mix_f32 on fp16-subnormal codes, bit-identical to
//    bf16_rne(fp32(s)*q + fp32(b))) for every scale below 2^104; tiles holding a larger or
//    non-finite scale are listed and recomputed in the general form (dequant_word) at the end.
//  * Work decomposition (stream-K): output columns are cut into tiles of CW columns; the T*NS
//    (tile, step) units are split into G equal contiguous ranges, one per workgroup, so every
//    workgroup streams the same number of weight bytes. A workgroup streams its range as one
//    pipeline (weights PF steps ahead, x one step ahead) across tile boundaries. Tiles entirely
//    inside the range are written as bf16; the first and last tiles of a range may be shared with
//    neighbouring workgroups: their fp32 partials are stored with device-coherent stores, and
//    after the whole range has streamed the workgroup counts in on their counters; the last
//    contributor sums the partials in contributor order (deterministic).
//  * x: staged in LDS in A-fragment order with only the M real rows. Resident form (M <= 16 when
//    the range touches few enough steps): the slices of all the range's steps are staged once,
//    behind the first weight prefetches, and the stream has no barrier but the one closing each
//    tile. Staged form: each step's slice is staged as the step begins (double-buffered, one
//    barrier per step); the next step's slice is loaded into registers before that step's weight
//    prefetches are issued, so waiting for it never waits for weights still in flight (the vector
//    memory counter is in order).
#include <algorithm>
#include <type_traits>

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
  int NS;         // steps per tile = K / (128 * V)
  int G;          // workgroups
  long long U;    // units = T * NS
};

template <int MP_, int V_, int CT_, int PF_, int WPE_, int XS_, int WAVES_ = 4>
struct SkinnyCfg {
  static constexpr int MP = MP_;               // rows served (M <= MP), a power of two
  static constexpr int MB = (MP + 15) / 16;    // 16-row MFMA blocks
  static constexpr int V = V_;                 // super-steps per step (1, 2 or 4)
  static constexpr int CT = CT_, PF = PF_;
  static_assert(PF >= 1 && PF <= 4, "prefetch depth 1..4");
  static constexpr int kWavesPerSimd = WPE_;  // register budget: 512 / WPE VGPRs+AGPRs per lane
  static constexpr int kWaves = WAVES_;         // waves per workgroup (each owns CT column blocks)
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int CW = kWaves * CT * 16;  // columns per tile
  static constexpr int XU = MP * V * 16;       // 16-byte units of a step's x slice
  static constexpr int kXR = (XU + kThreads - 1) / kThreads;  // x-staging registers per thread
  static constexpr int LGV = V == 4 ? 2 : V == 2 ? 1 : 0;
  // Resident x: 0 = each step's x slice is staged in LDS as the step begins (double-buffered, one
  // barrier per step); XS > 0 = the x slices of every step the workgroup's range touches (at most
  // XS distinct steps) are staged once before the stream starts, and the stream has no barriers
  // but the one closing each tile.
  static constexpr int XS = XS_;
  static constexpr int kXSlots = XS > 0 ? XS : 2;
};

// LDS slot of step st when the range begins at step st0 (resident x).
__device__ __forceinline__ int x_slot(int st, int st0, int NS) {
  const int sl = st - st0;
  return sl < 0 ? sl + NS : sl;
}

// The 2V scales (or biases) of one row for one step: V dwords, loaded with one buffer load.
template <int V>
struct SB {
  uint32_t d[V];
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

__device__ __forceinline__ long long range_start(int p, long long U, int G) {
  return (long long)p * U / G;
}

// Workgroup owning unit u when U units are split into G ranges [p*U/G, (p+1)*U/G).
__device__ __forceinline__ int unit_owner(long long u, long long U, int G) {
  return (int)(((u + 1) * (long long)G + U - 1) / U) - 1;
}

// Device-coherent fp32 store/load through a buffer resource: cache policy sc1, the form gfx950
// uses for relaxed agent-scope atomic stores and loads (coherent across the XCDs' L2s).
// (The b32 buffer builtins move raw 32-bit words: floats cross them as bit patterns.)
constexpr int kCoherent = 16;  // cache-policy operand value for sc1
__device__ __forceinline__ void store_coherent(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, byte_off, 0, kCoherent);
}
__device__ __forceinline__ float load_coherent(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kCoherent));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t y_rsrc(const SkinnyParams& P) {
  return __builtin_amdgcn_make_buffer_rsrc(P.y, 0, rsrc_bytes((unsigned long long)P.M * P.N * 2),
                                           kBufferRsrcWord3);
}

__device__ __forceinline__ void store_y(__amdgpu_buffer_rsrc_t r, uint32_t elem, float v) {
  __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(pack_bf16x2(v, 0.0f) & 0xFFFFu), r, elem * 2u, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const SkinnyParams& P, int cw) {
  return __builtin_amdgcn_make_buffer_rsrc(P.part, 0,
                                           rsrc_bytes((unsigned long long)P.G * 2 * P.M * cw * sizeof(float)),
                                           kBufferRsrcWord3);
}

// x staging for one step. Items are the 16-byte pieces (row m, super-step v, piece q) with
// item = (m * V + v) * 16 + q; thread tid owns items tid + j * kThreads. LDS position of an item:
// (v * 16 + q) * MP + m, i.e. the A fragment of MFMA (v, q % 4) for lane group q / 4, row m.
// Rows M..MP-1 are never written (A-fragment rows >= M read row M-1: they only reach output
// rows that are never stored). Loads are unconditional (clamped to a valid piece): a conditional
// load would make the compiler copy its result at once, i.e. wait for it, and with it for every
// load issued before it.
template <class C>
__device__ __forceinline__ void load_x(u32x4 (&xr)[C::kXR], const uint16_t* __restrict__ x, int M, int K, int step) {
#pragma unroll
  for (int j = 0; j < C::kXR; ++j) {
    const int i = min((int)threadIdx.x + j * C::kThreads, C::XU - 1);
    const int m = min(i >> (C::LGV + 4), M - 1);
    const int v = (i >> 4) & (C::V - 1);
    const int q = i & 15;
    xr[j] = *reinterpret_cast<const u32x4*>(x + (size_t)m * K + (size_t)(step * C::V + v) * 128 + q * 8);
  }
}

template <class C>
__device__ __forceinline__ void store_x(u32x4* xs, const u32x4 (&xr)[C::kXR], int M) {
#pragma unroll
  for (int j = 0; j < C::kXR; ++j) {
    const int i = (int)threadIdx.x + j * C::kThreads;
    const int m = i >> (C::LGV + 4);
    const int v = (i >> 4) & (C::V - 1);
    const int q = i & 15;
    if (i < C::XU && m < M) xs[(v * 16 + q) * C::MP + m] = xr[j];
  }
}

// Last arrival of a shared tile: y[:, tile] = bf16(sum of the contributors' fp32 partials), summed
// in contributor order (deterministic). Loads go out in batches of kE elements x kQ contributors
// per thread, all independent, so a batch costs one memory round trip.
template <class C>
__device__ __forceinline__ void reduce_tile(const SkinnyParams& P, int t, int plo, int phi, int lo_slot) {
  constexpr int kE = 4, kQ = 4;
  const int total = P.M * C::CW;
  const int nq = phi - plo + 1;
  const __amdgpu_buffer_rsrc_t rp = part_rsrc(P, C::CW);
  const __amdgpu_buffer_rsrc_t ry = y_rsrc(P);
  for (int base = threadIdx.x; base < total; base += C::kThreads * kE) {
    float sum[kE];
#pragma unroll
    for (int i = 0; i < kE; ++i) sum[i] = 0.0f;
    for (int q0 = 0; q0 < nq; q0 += kQ) {
      float v[kE][kQ];
#pragma unroll
      for (int i = 0; i < kE; ++i)
#pragma unroll
        for (int j = 0; j < kQ; ++j) {
          const int idx = base + i * C::kThreads, q = q0 + j;
          const uint32_t off = (q == 0) ? (uint32_t)(plo * 2 + lo_slot) * (uint32_t)total
                                        : (uint32_t)((plo + q) * 2) * (uint32_t)total;
          v[i][j] = (idx < total && q < nq) ? load_coherent(rp, (off + (uint32_t)idx) * 4u) : 0.0f;
        }
#pragma unroll
      for (int i = 0; i < kE; ++i)
#pragma unroll
        for (int j = 0; j < kQ; ++j) sum[i] += v[i][j];
    }
#pragma unroll
    for (int i = 0; i < kE; ++i) {
      const int idx = base + i * C::kThreads;
      if (idx < total) {
        const int m = idx / C::CW;
        const int n = t * C::CW + (idx - m * C::CW);
        if (n < P.N) store_y(ry, (uint32_t)(m * P.N + n), sum[i]);
      }
    }
  }
}

// Per-lane state: buffer resources and this lane's place in the tile.
struct LaneCtx {
  __amdgpu_buffer_rsrc_t rw, rs, rb;
  int n, g, wave;
};

// Byte offsets of this lane's column of tile t in each of its column blocks (column 0 past N:
// loaded, never stored): its 16-byte piece of the first 64-byte segment, and the row's scales.
template <class C>
__device__ __forceinline__ void col_offsets(const SkinnyParams& P, const LaneCtx& L, int t,
                                            uint32_t (&wo)[C::CT], uint32_t (&so)[C::CT]) {
#pragma unroll
  for (int ct = 0; ct < C::CT; ++ct) {
    const int col = t * C::CW + (L.wave * C::CT + ct) * 16 + L.n;
    const uint32_t cc = (col < P.N) ? (uint32_t)col : 0u;
    wo[ct] = cc * (uint32_t)(P.K >> 1) + (uint32_t)L.g * 16u;
    so[ct] = cc * (uint32_t)(P.K >> 6) * 2u;
  }
}

// acc += x[:, k-range] @ dequant(w[tile t columns, k-range])^T over steps [a, e) of tile t, in
// the general dequantization form (dequant_word), with its own x staging and no prefetch: the rare
// path for tiles that hold a scale outside dequant_word_fast's range.
template <class C>
__device__ __forceinline__ void redo_segment(const SkinnyParams& P, const LaneCtx& L, int t, int a, int e,
                                             u32x4 (*xs)[C::XU], int st0, f32x4 (&acc)[C::MB][C::CT]) {
  constexpr int MB = C::MB, CT = C::CT, V = C::V;
  uint32_t wo[CT], so[CT];
  col_offsets<C>(P, L, t, wo, so);
  int aoff[MB];
#pragma unroll
  for (int rb = 0; rb < MB; ++rb) aoff[rb] = L.g * 4 * C::MP + min(rb * 16 + L.n, P.M - 1);
  u32x4 xr[C::kXR];
  for (int st = a; st < e; ++st) {
    u32x4* xb;
    if constexpr (C::XS > 0) {
      xb = xs[x_slot(st, st0, P.NS)];
    } else {
      __syncthreads();
      load_x<C>(xr, P.x, P.M, P.K, st);
      store_x<C>(xs[0], xr, P.M);
      __syncthreads();
      xb = xs[0];
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const SB<V> sv = load_sb<V>(L.rs, so[ct], st * 4 * V);
      const SB<V> bv = load_sb<V>(L.rb, so[ct], st * 4 * V);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const u32x4 wpc = __builtin_amdgcn_raw_buffer_load_b128(L.rw, wo[ct] + v * 64, st * V * 64, 0);
        const int e2 = 2 * v + (L.g >> 1);
        const float sf = bf16_to_f32((sv.d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
        const float bf = bf16_to_f32((bv.d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const u32x4 B = dequant_word(wpc[tt], sf, sf * 0.0625f, bf);
#pragma unroll
          for (int rb = 0; rb < MB; ++rb)
            acc[rb][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(xb[(v * 16 + tt) * C::MP + aoff[rb]]), as_bf16x8(B), acc[rb][ct], 0, 0, 0);
        }
      }
    }
  }
}

// Workgroup p owns units [u0, u1) (unit = (tile, step)) and streams them in order as one
// pipeline across tile boundaries.
template <class C>
__global__ __launch_bounds__(C::kThreads) __attribute__((amdgpu_waves_per_eu(C::kWavesPerSimd)))
void skinny_kernel(SkinnyParams P) {
  constexpr int MB = C::MB, CT = C::CT, CW = C::CW, PF = C::PF, V = C::V;
  constexpr int kMaxRedo = 32;
  __shared__ u32x4 xs[C::kXSlots][C::XU];
  __shared__ int s_last[2];
  __shared__ int s_nredo;
  __shared__ int s_redo[kMaxRedo][3];

  const int tid = threadIdx.x;
  const int p = blockIdx.x;
  const int NS = P.NS;
  const int KG = P.K >> 6;
  LaneCtx L;
  L.n = tid & 15;
  L.g = (tid >> 4) & 3;
  L.wave = tid >> 6;
  L.rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(P.w), 0,
                                           rsrc_bytes((unsigned long long)P.N * (P.K >> 1)), kBufferRsrcWord3);
  L.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.s), 0,
                                           rsrc_bytes((unsigned long long)P.N * KG * 2), kBufferRsrcWord3);
  L.rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.b), 0,
                                           rsrc_bytes((unsigned long long)P.N * KG * 2), kBufferRsrcWord3);
  if (tid == 0) s_nredo = 0;

  const long long u0 = range_start(p, P.U, P.G);
  const long long u1 = range_start(p + 1, P.U, P.G);
  const int nunits = (int)(u1 - u0);
  const int t0 = (int)(u0 / NS), st0 = (int)(u0 - (long long)t0 * NS);
  const int t_last = (int)((u1 - 1) / NS);
  const bool first_shared = st0 != 0;                              // tile t0 began earlier
  const bool last_shared = (u1 - (long long)t_last * NS) != NS;    // tile t_last goes on later
  const __amdgpu_buffer_rsrc_t ry = y_rsrc(P);
  const __amdgpu_buffer_rsrc_t rp = part_rsrc(P, CW);

  // Tile t's result: bf16 into y, or the fp32 partial of a shared tile (slot 0 for the range's
  // first tile, 1 for its last: a range that begins at a tile's start and ends inside it uses
  // slot 0, as the reducing workgroup expects of a contributor whose range begins in the tile).
  // Accumulator element r of lane (n, g) holds row 4*g + r of its 16-row block, column n.
  auto store_tile = [&](int t, const f32x4 (&acc)[MB][CT]) {
    const bool shared = (t == t0 && first_shared) || (t == t_last && last_shared);
    if (!shared) {
#pragma unroll
      for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int col = t * CW + (L.wave * CT + ct) * 16 + L.n;
          const uint32_t e0 = (uint32_t)((rb * 16 + 4 * L.g) * P.N + col);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = rb * 16 + 4 * L.g + r;
            if (m < P.M && col < P.N) store_y(ry, e0 + (uint32_t)(r * P.N), acc[rb][ct][r]);
          }
        }
    } else {
      const int slot = (t == t0) ? 0 : 1;
      const uint32_t pbase = (uint32_t)(p * 2 + slot) * (uint32_t)(P.M * CW);
#pragma unroll
      for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int cl = (L.wave * CT + ct) * 16 + L.n;
          const uint32_t lbase = (pbase + (uint32_t)((rb * 16 + 4 * L.g) * CW + cl)) * 4u;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = rb * 16 + 4 * L.g + r;
            if (m < P.M) store_coherent(rp, lbase + (uint32_t)(r * CW * 4), acc[rb][ct][r]);
          }
        }
    }
  };

  // This lane's A-fragment offset within a staged step (rows >= M read row M-1).
  int aoff[MB];
#pragma unroll
  for (int rb = 0; rb < MB; ++rb) aoff[rb] = L.g * 4 * C::MP + min(rb * 16 + L.n, P.M - 1);

  // x for the first step, into registers (staged x).
  u32x4 xr[C::kXR];
  if constexpr (C::XS == 0) load_x<C>(xr, P.x, P.M, P.K, st0);

  // Weight prefetch ring, PF steps ahead; (tp, sp) is the next unit to fetch, fi its index.
  // Fetches are unconditional so that the ring stays in fixed registers and the compiler waits
  // only for the slot being consumed. Past the range's end they go through zero-length buffer
  // resources: out-of-range buffer loads return zeros without a memory access (re-reading the
  // last unit instead would miss the L2 and cost up to PF units of HBM traffic per workgroup).
  const int wrec = rsrc_bytes((unsigned long long)P.N * (P.K >> 1));
  const int srec = rsrc_bytes((unsigned long long)P.N * KG * 2);
  u32x4 wv[PF][CT][V];
  SB<V> sv[PF][CT], bv[PF][CT];
  uint32_t wo[CT], so[CT];
  int tp = t0, sp = st0, fi = 0;
  col_offsets<C>(P, L, tp, wo, so);
  auto fetch = [&](int j) {
    const bool live = fi < nunits;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(P.w), 0, live ? wrec : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.s), 0, live ? srec : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.b), 0, live ? srec : 0, kBufferRsrcWord3);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
      for (int v = 0; v < V; ++v)
        wv[j][ct][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, wo[ct] + v * 64, sp * V * 64, 0);
      sv[j][ct] = load_sb<V>(rs, so[ct], sp * 4 * V);
      bv[j][ct] = load_sb<V>(rb, so[ct], sp * 4 * V);
    }
    if (++fi < nunits) {
      if (++sp == NS) {
        sp = 0;
        ++tp;
        col_offsets<C>(P, L, tp, wo, so);
      }
    }
  };
#pragma unroll
  for (int j = 0; j < PF; ++j) fetch(j);

  if constexpr (C::XS > 0) {
    // Resident x: stage the slices of the range's steps (st0, st0 + 1, ... wrapping at NS; at most
    // XS of them, as the launch guarantees) behind the first weight prefetches.
    const int nsl = nunits < NS ? nunits : NS;
    for (int i = tid; i < nsl * C::XU; i += C::kThreads) {
      const int sl = i / C::XU, it = i & (C::XU - 1);
      int stp = st0 + sl;
      if (stp >= NS) stp -= NS;
      const int m = it >> (C::LGV + 4), v = (it >> 4) & (C::V - 1), q = it & 15;
      if (m < P.M)
        xs[sl][(v * 16 + q) * C::MP + m] = *reinterpret_cast<const u32x4*>(
            P.x + (size_t)m * P.K + (size_t)(stp * V + v) * 128 + q * 8);
    }
    __syncthreads();
  }

  f32x4 acc[MB][CT];
#pragma unroll
  for (int rb = 0; rb < MB; ++rb)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[rb][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  bool bad = false;
  int t = t0, st = st0, tile_a = st0;  // current unit's tile and step; this tile's first step here

  // One unit of the stream: consume ring slot J (a compile-time index, so the ring stays in
  // registers), refill it PF units ahead, and close the tile when it ends here.
  auto unit = [&](int i, auto jc) {
    constexpr int j = decltype(jc)::value;
    // Publish this step's x (double-buffered: the barrier also tells that every wave is done
    // with step i-2, the previous user of this buffer), then fetch the next step's x.
    u32x4* xb;
    if constexpr (C::XS > 0) {
      xb = xs[x_slot(st, st0, NS)];
    } else {
      xb = xs[i & 1];
      store_x<C>(xb, xr, P.M);
      __syncthreads();
      load_x<C>(xr, P.x, P.M, P.K, (st + 1 < NS) ? st + 1 : 0);
    }

#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        // Group of piece v for this lane: 2*(step*V + v) + g/2 (element 2v + g/2 of the step's scales).
        const int e2 = 2 * v + (L.g >> 1);
        const uint32_t sbits = (sv[j][ct].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu;
        const uint32_t bbits = (bv[j][ct].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu;
        bad |= !fast_scale_ok(sbits);
        const float sf = bf16_to_f32(sbits);
        const float s24 = sf * 16777216.0f, s20 = sf * 1048576.0f, bf = bf16_to_f32(bbits);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const u32x4 B = dequant_word_fast(wv[j][ct][v][tt], s24, s20, bf);
#pragma unroll
          for (int rb = 0; rb < MB; ++rb)
            acc[rb][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(xb[(v * 16 + tt) * C::MP + aoff[rb]]), as_bf16x8(B), acc[rb][ct], 0, 0, 0);
        }
      }
    }
    fetch(j);

    if (st == NS - 1 || i == nunits - 1) {
      // Tile t ends here (for this workgroup): steps [tile_a, st] of it were streamed.
      if (__syncthreads_or(bad)) {
        if (tid == 0) {
          const int k = s_nredo++;
          if (k < kMaxRedo) { s_redo[k][0] = t; s_redo[k][1] = tile_a; s_redo[k][2] = st + 1; }
        }
        bad = false;
      } else {
        store_tile(t, acc);
      }
#pragma unroll
      for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[rb][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      ++t;
      st = 0;
      tile_a = 0;
    } else {
      ++st;
    }
  };
  // Whole groups of PF units in the loop, the rest after it: a conditional exit inside the loop
  // body would make the compiler assume a path on which later ring slots were never fetched and
  // wait for nearly every load.
  int base = 0;
  for (; base + PF <= nunits; base += PF) {
    unit(base, std::integral_constant<int, 0>{});
    if constexpr (PF > 1) unit(base + 1, std::integral_constant<int, 1 % PF>{});
    if constexpr (PF > 2) unit(base + 2, std::integral_constant<int, 2 % PF>{});
    if constexpr (PF > 3) unit(base + 3, std::integral_constant<int, 3 % PF>{});
  }
  if (base < nunits) unit(base, std::integral_constant<int, 0>{});
  if constexpr (PF > 2) if (base + 1 < nunits) unit(base + 1, std::integral_constant<int, 1 % PF>{});
  if constexpr (PF > 3) if (base + 2 < nunits) unit(base + 2, std::integral_constant<int, 2 % PF>{});

  // Tiles with scales outside the fast form: recompute in the general form. (More than kMaxRedo
  // such tiles in one range: recompute every tile of the range.)
  __syncthreads();
  const int nredo = s_nredo;
  if (nredo > 0) {
    const bool all = nredo > kMaxRedo;
    const int count = all ? (t_last - t0 + 1) : nredo;
    for (int k = 0; k < count; ++k) {
      int rt, ra, re;
      if (all) {
        rt = t0 + k;
        ra = (rt == t0) ? st0 : 0;
        re = (rt == t_last) ? (int)(u1 - (long long)t_last * NS) : NS;
      } else {
        rt = s_redo[k][0]; ra = s_redo[k][1]; re = s_redo[k][2];
      }
#pragma unroll
      for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[rb][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      redo_segment<C>(P, L, rt, ra, re, xs, st0, acc);
      store_tile(rt, acc);
    }
  }

  if (!first_shared && !last_shared) return;
  // Count in on the shared tiles. The partials must be complete at the device's coherence point
  // first: wait for every outstanding vector memory operation of this wave.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const int tt0 = first_shared ? t0 : t_last;                                   // shared tile 0
  const int tt1 = (first_shared && last_shared && t_last != t0) ? t_last : -1;  // shared tile 1
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
    // Contributor plo holds this tile in its slot 1 iff its range began in an earlier tile
    // (the tile is its last); every later contributor's range begins inside it (slot 0).
    const int lo_slot = (range_start(plo, P.U, P.G) < tile0) ? 1 : 0;
    reduce_tile<C>(P, tt, plo, phi, lo_slot);
    if (tid == 0) __hip_atomic_store(&P.cnt[tt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Kernel table: id -> (rows, V, CT, PF, waves per SIMD, resident x slots, waves per workgroup).
// The x slice of a step
// is at most 16 KB (rows * V <= 64), so larger row counts take shorter steps; V = 2 and 1 also
// serve K that four super-steps do not divide. Variants 12-14 are the resident-x twins of 0-2
// (48 KB of x slots each, three workgroups per CU).
// Prefetch depth 2 everywhere; 17-32 rows use 12-wave workgroups (192-column tiles, one x staging
// per 12 waves).
#define QMM4_SKINNY_VARIANTS(X) \
  X(0, 4, 4, 1, 2, 4, 0, 4)   \
  X(1, 8, 4, 1, 2, 4, 0, 4)   \
  X(2, 16, 4, 1, 2, 4, 0, 4)  \
  X(3, 32, 2, 1, 2, 4, 0, 12)                     \
  X(4, 64, 1, 1, 2, 4, 0, 4)                     \
  X(5, 4, 2, 1, 2, 4, 0, 4)                      \
  X(6, 8, 2, 1, 2, 4, 0, 4)                      \
  X(7, 16, 2, 1, 2, 4, 0, 4)                     \
  X(8, 4, 1, 1, 2, 4, 0, 4)                      \
  X(9, 8, 1, 1, 2, 4, 0, 4)                      \
  X(10, 16, 1, 1, 2, 4, 0, 4)                    \
  X(11, 32, 1, 1, 2, 4, 0, 4)                    \
  X(12, 4, 4, 1, 2, 4, 12, 4)    \
  X(13, 8, 4, 1, 2, 4, 6, 4)     \
  X(14, 16, 4, 1, 2, 4, 3, 4)

#define QMM4_CFG_TYPE(id, mp, v, ct, pf, wpe, xs, wv) typedef SkinnyCfg<mp, v, ct, pf, wpe, xs, wv> SkCfg##id;
QMM4_SKINNY_VARIANTS(QMM4_CFG_TYPE)
#undef QMM4_CFG_TYPE

// Columns per tile of a variant: the kernel's CW. The host sizes the split-K partials (and the
// tile count) from this, so it must be the kernel's own constant.
static int skinny_tile_cols(int variant) {
  switch (variant) {
#define QMM4_CW_OF(id, mp, v, ct, pf, wpe, xs, wv) \
  case id: return SkCfg##id::CW;
    QMM4_SKINNY_VARIANTS(QMM4_CW_OF)
#undef QMM4_CW_OF
    default: return 0;
  }
}

int skinny_variant(int M, int vmax, int* tile_cols, int* steps_v) {
  const int mp = M <= 4 ? 4 : M <= 8 ? 8 : M <= 16 ? 16 : M <= 32 ? 32 : 64;
  int v = mp == 64 ? 1 : mp == 32 ? 2 : 4;
  if (v > vmax) v = vmax;
  int id;
  if (mp == 64) id = 4;
  else if (v == 4) id = mp == 4 ? 0 : mp == 8 ? 1 : 2;
  else if (v == 2) id = mp == 4 ? 5 : mp == 8 ? 6 : mp == 16 ? 7 : 3;
  else id = mp == 4 ? 8 : mp == 8 ? 9 : mp == 16 ? 10 : 11;
  *tile_cols = skinny_tile_cols(id);
  *steps_v = v;
  return id;
}

__global__ __launch_bounds__(256) void zero_u32_kernel(uint32_t* __restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0u;
}

hipError_t launch_zero_u32(uint32_t* p, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p, n);
  return hipGetLastError();
}

int skinny_resident_twin(int variant, int* slots) {
  switch (variant) {
    case 0: *slots = SkCfg12::XS; return 12;
    case 1: *slots = SkCfg13::XS; return 13;
    case 2: *slots = SkCfg14::XS; return 14;
    default: *slots = 0; return -1;
  }
}

static int skinny_threads(int variant) {
  switch (variant) {
#define QMM4_THREADS(id, mp, v, ct, pf, wpe, xs, wv) \
  case id: return SkCfg##id::kThreads;
    QMM4_SKINNY_VARIANTS(QMM4_THREADS)
#undef QMM4_THREADS
    default: return 256;
  }
}

static const void* skinny_func(int variant) {
  switch (variant) {
#define QMM4_FUNC(id, mp, v, ct, pf, wpe, xs, wv) \
  case id: return reinterpret_cast<const void*>(&skinny_kernel<SkCfg##id>);
    QMM4_SKINNY_VARIANTS(QMM4_FUNC)
#undef QMM4_FUNC
    default: return nullptr;
  }
}

int skinny_occupancy(int variant) {
  int nb = 0;
  const void* f = skinny_func(variant);
  if (!f || hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, skinny_threads(variant), 0) != hipSuccess) return 1;
  return nb > 0 ? nb : 1;
}

hipError_t launch_skinny(const SkinnyPlan& plan, const uint16_t* x, const uint32_t* w,
                         const uint16_t* s, const uint16_t* b, uint16_t* y, float* part,
                         uint32_t* cnt, int M, int N, int K, hipStream_t stream) {
  SkinnyParams P;
  P.x = x; P.w = w; P.s = s; P.b = b; P.y = y; P.part = part; P.cnt = cnt;
  P.M = M; P.N = N; P.K = K; P.NS = K / (128 * plan.steps_v); P.G = plan.blocks; P.U = plan.units;
  const dim3 grid((unsigned)plan.blocks), block((unsigned)skinny_threads(plan.variant));
  switch (plan.variant) {
#define QMM4_LAUNCH(id, mp, v, ct, pf, wpe, xs, wv) \
  case id: hipLaunchKernelGGL(skinny_kernel<SkCfg##id>, grid, block, 0, stream, P); break;
    QMM4_SKINNY_VARIANTS(QMM4_LAUNCH)
#undef QMM4_LAUNCH
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace qmm4
