// Skinny quantized matmul for M = 1..64 rows (decode, tree verify): y = x @ dequant(w)^T.
//
// Replaces the reference's M <= 64 kernels (qmv_packed, the NAX verify tiles and the multi-row
// NAX kernel: src/mlx_tree_spec/qmm_packed.py:151-220, 296-394, 428-557) with one design that
// reads MLX's own [N, K/8] layout directly (no install-time relayout).
//
// The regime is HBM-bound: every packed weight is read once and used for all M rows, and the
// exact dequantization (VALU) is the work that has to keep pace with HBM.
//  * Work decomposition (stream-K): output columns are cut into tiles of CW columns; the tile's
//    K is cut into 128-wide super-steps (two quantization groups). The T*KS (tile, super-step)
//    units are split into G equal contiguous ranges, one per workgroup, so every workgroup
//    streams the same number of weight bytes whatever N and K are. A range that covers a whole
//    tile writes bf16 directly. A tile shared by several workgroups is summed from fp32 partials
//    by the last workgroup to finish it, in workgroup order (deterministic). The partials are
//    written and read with device-coherent accesses (relaxed agent-scope atomic stores/loads)
//    and the writer waits for its stores before it counts itself in, so no L2 writeback or
//    invalidate (a full device fence) is needed.
//  * Within a workgroup (4 waves), each wave owns CT column blocks of 32 columns. MFMA
//    32x32x16 (bf16, fp32 accumulation); lane (column c = lane % 32, half h = lane / 32) loads
//    the 8 packed words of k = 128*ss + 64h .. +64 of its column (two 16-B loads, prefetched PF
//    super-steps ahead) — exactly one quantization group — dequantizes them bit-exactly in
//    registers and feeds them as B operands of the 8 MFMA steps of the super-step. Dequantized
//    weights never touch LDS.
//  * The activation slice x[0:M, k-range] is staged in LDS per chunk of KC super-steps
//    (KC = 64/M rounded down to a power of two, so a chunk is at most 16 KB), in A-fragment
//    order with only the M real rows, and shared by all waves. A-fragment rows >= M read row M-1:
//    they only feed output rows >= M, which are never stored. The next chunk is loaded into
//    registers at the start of the current one, before that chunk's weight prefetches are
//    issued, so waiting for it never waits for weights that are still in flight (the vector
//    memory counter is in order).
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

template <int MP_, int CT_, int PF_, int XR_, int WPE_>
struct SkinnyCfg {
  static constexpr int MP = MP_;               // rows the variant serves (M <= MP), a power of two
  static constexpr int MB = (MP + 31) / 32;    // 32-row MFMA blocks
  static constexpr int CT = CT_, PF = PF_;
  static constexpr int kWavesPerSimd = WPE_;  // register budget: 512 / WPE VGPRs+AGPRs per lane
  static constexpr int kWaves = 4;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int CW = kWaves * CT * 32;  // columns per tile
  static constexpr int kXR = XR_;              // 16-B x-staging registers per thread
  static constexpr int kXUnits = kXR * kThreads;  // 16-B units of the LDS x chunk
  static constexpr int KC = kXUnits / (16 * MP);  // super-steps per x chunk
  static constexpr int LGKC = KC >= 64 ? 6 : KC >= 32 ? 5 : KC >= 16 ? 4 : KC >= 8 ? 3 : KC >= 4 ? 2 : KC >= 2 ? 1 : 0;
};

__device__ __forceinline__ long long range_start(int p, long long U, int G) {
  return (long long)p * U / G;
}

// Workgroup owning unit u when U units are split into G ranges [p*U/G, (p+1)*U/G).
__device__ __forceinline__ int unit_owner(long long u, long long U, int G) {
  return (int)(((u + 1) * (long long)G + U - 1) / U) - 1;
}

// Device-coherent fp32 store/load through a buffer resource: cache policy sc1, the form gfx950
// uses for relaxed agent-scope atomic stores and loads (coherent across the XCDs' L2s).
constexpr int kCoherent = 16;  // cache-policy operand value for sc1
// (The b32 buffer builtins move raw 32-bit words: floats cross them as bit patterns.)
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

// x chunk staging. Chunk items are the 16-B pieces (row m, super-step dss, piece q) with
// item = (m * KC + dss) * 16 + q; thread tid owns items tid + j * kThreads. LDS position of an
// item: ((dss * 8 + q % 8) * 2 + q / 8) * MP + m, i.e. the A fragment of MFMA step q % 8, lane
// half q / 8, row m of super-step dss. Rows M..MP-1 are never written.
template <class C>
__device__ __forceinline__ void load_x(u32x4 (&xr)[C::kXR], const uint16_t* __restrict__ x, int M, int K,
                                       int ss0, int nss) {
#pragma unroll
  for (int j = 0; j < C::kXR; ++j) {
    const int i = (int)threadIdx.x + j * C::kThreads;
    const int m = i >> (C::LGKC + 4);
    const int dss = (i >> 4) & (C::KC - 1);
    const int q = i & 15;
    // Unconditional (clamped to a valid piece): a conditional load would make the compiler copy
    // its result at once, i.e. wait for it, and with it for every load issued before it.
    const int mc = min(m, M - 1), dc = min(dss, nss - 1);
    xr[j] = *reinterpret_cast<const u32x4*>(x + (size_t)mc * K + (size_t)(ss0 + dc) * 128 + q * 8);
  }
}

template <class C>
__device__ __forceinline__ void store_x(u32x4* xs, const u32x4 (&xr)[C::kXR], int M, int nss) {
#pragma unroll
  for (int j = 0; j < C::kXR; ++j) {
    const int i = (int)threadIdx.x + j * C::kThreads;
    const int m = i >> (C::LGKC + 4);
    const int dss = (i >> 4) & (C::KC - 1);
    const int q = i & 15;
    if (m < M && dss < nss) xs[((dss * 8 + (q & 7)) * 2 + (q >> 3)) * C::MP + m] = xr[j];
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
  int c, h, wave;
};

// Byte offsets of this lane's column of tile t in each of its column blocks (column 0 past N:
// loaded, never stored): packed words k = 64h .. 64h+63 of super-step 0, and the scale/bias of
// group h.
template <class C>
__device__ __forceinline__ void col_offsets(const SkinnyParams& P, const LaneCtx& L, int t,
                                            uint32_t (&wo)[C::CT], uint32_t (&so)[C::CT]) {
#pragma unroll
  for (int ct = 0; ct < C::CT; ++ct) {
    const int n = t * C::CW + (L.wave * C::CT + ct) * 32 + L.c;
    const uint32_t nn = (n < P.N) ? (uint32_t)n : 0u;
    wo[ct] = nn * (uint32_t)(P.K >> 1) + (uint32_t)L.h * 32u;
    so[ct] = (nn * (uint32_t)(P.K >> 6) + (uint32_t)L.h) * 2u;
  }
}

// acc += x[:, k-range] @ dequant(w[tile t columns, k-range])^T over super-steps [a, e) of tile t,
// in the general dequantization form (dequant_word), with its own x staging and no prefetch:
// the rare path for tiles that hold a scale outside dequant_word_fast's range.
template <class C>
__device__ __forceinline__ void redo_segment(const SkinnyParams& P, const LaneCtx& L, int t, int a, int e,
                                             u32x4* xs, f32x16 (&acc)[C::MB][C::CT]) {
  constexpr int MB = C::MB, CT = C::CT, KC = C::KC;
  uint32_t wo[CT], so[CT];
  col_offsets<C>(P, L, t, wo, so);
  int aoff[MB];
#pragma unroll
  for (int rb2 = 0; rb2 < MB; ++rb2) aoff[rb2] = L.h * C::MP + min(rb2 * 32 + L.c, P.M - 1);
  u32x4 xr[C::kXR];
  for (int c0 = a; c0 < e; c0 += KC) {
    const int n = min(KC, e - c0);
    __syncthreads();
    load_x<C>(xr, P.x, P.M, P.K, c0, n);
    store_x<C>(xs, xr, P.M, n);
    __syncthreads();
    for (int rc = 0; rc < n; ++rc) {
      const int ss = c0 + rc;
      const u32x4* xa = xs + rc * 16 * C::MP;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const u32x4 w0 = __builtin_amdgcn_raw_buffer_load_b128(L.rw, wo[ct], ss * 64, 0);
        const u32x4 w1 = __builtin_amdgcn_raw_buffer_load_b128(L.rw, wo[ct] + 16u, ss * 64, 0);
        const float sf = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(L.rs, so[ct], ss * 4, 0));
        const float bf = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(L.rb, so[ct], ss * 4, 0));
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) {
          const u32x4 B = dequant_word((tt < 4 ? w0 : w1)[tt & 3], sf, sf * 0.0625f, bf);
#pragma unroll
          for (int rb2 = 0; rb2 < MB; ++rb2)
            acc[rb2][ct] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xa[tt * 2 * C::MP + aoff[rb2]]),
                                                                   as_bf16x8(B), acc[rb2][ct], 0, 0, 0);
        }
      }
    }
  }
}

// Workgroup p owns units [u0, u1) and streams them in order as one pipeline: the weight
// prefetch ring and the x chunks run across tile boundaries, so the memory pipe never waits on a
// tile's epilogue. A tile whose units all lie in the range is written as bf16 when it ends. The
// range's first and last tiles may be shared with neighbouring workgroups: their fp32 partials
// are stored when they end (without waiting), and only after the whole range has streamed does
// the workgroup count itself in on their counters; the last contributor of a tile sums it.
// Tiles holding a scale outside dequant_word_fast's range are listed and recomputed in the
// general form after the stream.
template <class C>
__global__ __launch_bounds__(C::kThreads) __attribute__((amdgpu_waves_per_eu(C::kWavesPerSimd)))
void skinny_kernel(SkinnyParams P) {
  constexpr int MB = C::MB, CT = C::CT, CW = C::CW, PF = C::PF, KC = C::KC;
  constexpr int kMaxRedo = 32;
  __shared__ u32x4 xs[C::kXUnits];
  __shared__ int s_last[2];
  __shared__ int s_nredo;
  __shared__ int s_redo[kMaxRedo][3];

  const int tid = threadIdx.x;
  const int p = blockIdx.x;
  const int KS = P.KS;
  const int KG = P.K >> 6;
  LaneCtx L;
  L.c = tid & 31;
  L.h = (tid >> 5) & 1;
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
  const int t0 = (int)(u0 / KS), ss0 = (int)(u0 - (long long)t0 * KS);
  const int t_last = (int)((u1 - 1) / KS);
  const bool first_shared = ss0 != 0;                              // tile t0 began earlier
  const bool last_shared = (u1 - (long long)t_last * KS) != KS;    // tile t_last goes on later
  const __amdgpu_buffer_rsrc_t ry = y_rsrc(P);
  const __amdgpu_buffer_rsrc_t rp = part_rsrc(P, CW);

  // Tile t's result: bf16 into y, or the fp32 partial of a shared tile (slot 0 for the range's
  // first tile, 1 for its last: a range that begins at a tile's start and ends inside it uses
  // slot 0, as the reducing workgroup expects of a contributor whose range begins in the tile). Accumulator element r of lane (c, h) holds row
  // 8*(r/4) + 4*h + r%4 of its 32-row block.
  auto store_tile = [&](int t, const f32x16 (&acc)[MB][CT]) {
    const bool shared = (t == t0 && first_shared) || (t == t_last && last_shared);
    if (!shared) {
#pragma unroll
      for (int rb2 = 0; rb2 < MB; ++rb2)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int n = t * CW + (L.wave * CT + ct) * 32 + L.c;
          const uint32_t e0 = (uint32_t)((rb2 * 32 + 4 * L.h) * P.N + n);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = rb2 * 32 + 8 * (r >> 2) + 4 * L.h + (r & 3);
            if (m < P.M && n < P.N) store_y(ry, e0 + (uint32_t)((8 * (r >> 2) + (r & 3)) * P.N), acc[rb2][ct][r]);
          }
        }
    } else {
      const int slot = (t == t0) ? 0 : 1;
      const uint32_t pbase = (uint32_t)(p * 2 + slot) * (uint32_t)(P.M * CW);
#pragma unroll
      for (int rb2 = 0; rb2 < MB; ++rb2)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int cl = (L.wave * CT + ct) * 32 + L.c;
          const uint32_t lbase = (pbase + (uint32_t)((rb2 * 32 + 4 * L.h) * CW + cl)) * 4u;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = rb2 * 32 + 8 * (r >> 2) + 4 * L.h + (r & 3);
            if (m < P.M) store_coherent(rp, lbase + (uint32_t)((8 * (r >> 2) + (r & 3)) * CW * 4), acc[rb2][ct][r]);
          }
        }
    }
  };

  int aoff[MB];
#pragma unroll
  for (int rb2 = 0; rb2 < MB; ++rb2) aoff[rb2] = L.h * C::MP + min(rb2 * 32 + L.c, P.M - 1);

  // x chunks: maximal runs of at most KC consecutive units inside one tile. The chunk starting at
  // unit i covers super-steps [ss(i), ss(i) + chunk_len(i)).
  auto unit_ss = [&](int i) { return (int)((u0 + i) % KS); };
  auto chunk_len = [&](int i) { const int sst = unit_ss(i); return min(KC, min(KS - sst, nunits - i)); };
  u32x4 xr[C::kXR];
  int cstart = 0, clen = chunk_len(0);  // the current chunk
  load_x<C>(xr, P.x, P.M, P.K, ss0, clen);
  store_x<C>(xs, xr, P.M, clen);
  __syncthreads();
  if (clen < nunits) load_x<C>(xr, P.x, P.M, P.K, unit_ss(clen), chunk_len(clen));

  // Weight prefetch ring, PF units ahead; (tp, sp) is the next unit to fetch, fi its index.
  // Fetches are unconditional (past the range's end they repeat its last unit) so that the ring
  // stays in fixed registers and the compiler waits only for the slot being consumed.
  u32x4 wv[PF][CT][2];
  uint32_t sv[PF][CT], bv[PF][CT];
  uint32_t wo[CT], so[CT];
  int tp = t0, sp = ss0, fi = 0;
  col_offsets<C>(P, L, tp, wo, so);
  auto fetch = [&](int j) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      wv[j][ct][0] = __builtin_amdgcn_raw_buffer_load_b128(L.rw, wo[ct], sp * 64, 0);
      wv[j][ct][1] = __builtin_amdgcn_raw_buffer_load_b128(L.rw, wo[ct] + 16u, sp * 64, 0);
      sv[j][ct] = __builtin_amdgcn_raw_buffer_load_b16(L.rs, so[ct], sp * 4, 0);
      bv[j][ct] = __builtin_amdgcn_raw_buffer_load_b16(L.rb, so[ct], sp * 4, 0);
    }
    if (++fi < nunits) {
      if (++sp == KS) {
        sp = 0;
        ++tp;
        col_offsets<C>(P, L, tp, wo, so);
      }
    }
  };
#pragma unroll
  for (int j = 0; j < PF; ++j) fetch(j);

  f32x16 acc[MB][CT];
#pragma unroll
  for (int rb2 = 0; rb2 < MB; ++rb2)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[rb2][ct][r] = 0.0f;
  bool bad = false;
  int t = t0, ss = ss0, tile_a = ss0;  // current unit's tile and super-step; this tile's first super-step here

  for (int base = 0; base < nunits; base += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = base + j;
      if (i >= nunits) break;
      if (i == cstart + clen) {
        // Next chunk: its x is in registers; publish it, then fetch the one after.
        cstart = i;
        clen = chunk_len(i);
        __syncthreads();
        store_x<C>(xs, xr, P.M, clen);
        __syncthreads();
        if (i + clen < nunits) load_x<C>(xr, P.x, P.M, P.K, unit_ss(i + clen), chunk_len(i + clen));
      }
      // Group constants of this unit, per column block.
      float g24[CT], g20[CT], gb[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        bad |= !fast_scale_ok(sv[j][ct]);
        const float sf = bf16_to_f32(sv[j][ct] & 0xFFFFu);
        g24[ct] = sf * 16777216.0f;
        g20[ct] = sf * 1048576.0f;
        gb[ct] = bf16_to_f32(bv[j][ct] & 0xFFFFu);
      }
      const u32x4* xa = xs + (i - cstart) * 16 * C::MP;
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        bf16x8 A[MB];
#pragma unroll
        for (int rb2 = 0; rb2 < MB; ++rb2) A[rb2] = as_bf16x8(xa[tt * 2 * C::MP + aoff[rb2]]);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const u32x4 B = dequant_word_fast(wv[j][ct][tt >> 2][tt & 3], g24[ct], g20[ct], gb[ct]);
#pragma unroll
          for (int rb2 = 0; rb2 < MB; ++rb2)
            acc[rb2][ct] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[rb2], as_bf16x8(B), acc[rb2][ct], 0, 0, 0);
        }
      }
      fetch(j);

      if (ss == KS - 1 || i == nunits - 1) {
        // Tile t ends here (for this workgroup): super-steps [tile_a, ss] of it were streamed.
        if (__syncthreads_or(bad)) {
          if (tid == 0) {
            const int k = s_nredo++;
            if (k < kMaxRedo) { s_redo[k][0] = t; s_redo[k][1] = tile_a; s_redo[k][2] = ss + 1; }
          }
          bad = false;
        } else {
          store_tile(t, acc);
        }
#pragma unroll
        for (int rb2 = 0; rb2 < MB; ++rb2)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[rb2][ct][r] = 0.0f;
        ++t;
        ss = 0;
        tile_a = 0;
      } else {
        ++ss;
      }
    }
  }

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
        ra = (rt == t0) ? ss0 : 0;
        re = (rt == t_last) ? (int)(u1 - (long long)t_last * KS) : KS;
      } else {
        rt = s_redo[k][0]; ra = s_redo[k][1]; re = s_redo[k][2];
      }
#pragma unroll
      for (int rb2 = 0; rb2 < MB; ++rb2)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[rb2][ct][r] = 0.0f;
      redo_segment<C>(P, L, rt, ra, re, xs, acc);
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
    const long long tile0 = (long long)tt * KS;
    const int plo = unit_owner(tile0, P.U, P.G);
    const int phi = unit_owner(tile0 + KS - 1, P.U, P.G);
    const uint32_t prev = __hip_atomic_fetch_add(&P.cnt[tt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last[tid >> 6] = (prev == (uint32_t)(phi - plo)) ? 1 : 0;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int tt = k == 0 ? tt0 : tt1;
    if (tt < 0 || !s_last[k]) continue;
    const long long tile0 = (long long)tt * KS;
    const int plo = unit_owner(tile0, P.U, P.G);
    const int phi = unit_owner(tile0 + KS - 1, P.U, P.G);
    // Contributor plo holds this tile in its slot 1 iff its range began in an earlier tile
    // (the tile is its last); every later contributor's range begins inside it (slot 0).
    const int lo_slot = (range_start(plo, P.U, P.G) < tile0) ? 1 : 0;
    reduce_tile<C>(P, tt, plo, phi, lo_slot);
    if (tid == 0) __hip_atomic_store(&P.cnt[tt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Kernel table: variant -> (rows, CT, PF, x registers, waves per SIMD). PF <= KC keeps the wait
// for the next x chunk clear of weights still in flight.
typedef SkinnyCfg<4, 1, 3, 4, 3> CfgR4;
typedef SkinnyCfg<8, 1, 3, 4, 3> CfgR8;
typedef SkinnyCfg<16, 1, 3, 4, 3> CfgR16;
typedef SkinnyCfg<32, 1, 2, 4, 4> CfgR32;
typedef SkinnyCfg<64, 1, 2, 8, 2> CfgR64;

int skinny_variant_for_rows(int M, int* tile_cols) {
  *tile_cols = CfgR4::CW;  // every variant tiles 128 columns
  if (M <= 4) return 0;
  if (M <= 8) return 1;
  if (M <= 16) return 2;
  if (M <= 32) return 3;
  return 4;
}

static const void* skinny_func(int variant) {
  switch (variant) {
    case 0: return reinterpret_cast<const void*>(&skinny_kernel<CfgR4>);
    case 1: return reinterpret_cast<const void*>(&skinny_kernel<CfgR8>);
    case 2: return reinterpret_cast<const void*>(&skinny_kernel<CfgR16>);
    case 3: return reinterpret_cast<const void*>(&skinny_kernel<CfgR32>);
    default: return reinterpret_cast<const void*>(&skinny_kernel<CfgR64>);
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
    case 0: hipLaunchKernelGGL(skinny_kernel<CfgR4>, grid, block, 0, stream, P); break;
    case 1: hipLaunchKernelGGL(skinny_kernel<CfgR8>, grid, block, 0, stream, P); break;
    case 2: hipLaunchKernelGGL(skinny_kernel<CfgR16>, grid, block, 0, stream, P); break;
    case 3: hipLaunchKernelGGL(skinny_kernel<CfgR32>, grid, block, 0, stream, P); break;
    default: hipLaunchKernelGGL(skinny_kernel<CfgR64>, grid, block, 0, stream, P); break;
  }
  return hipGetLastError();
}

}  // namespace qmm4
