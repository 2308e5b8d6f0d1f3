// Prefill quantized GEMM for M > 64 rows: y = x @ dequant(w)^T on bf16 MFMA, fp32 accumulation.
//
// Replaces the reference's prefill kernel (src/mlx_tree_spec/qmm_packed.py:561-725: MLX's
// affine_qmm_t_nax with a packed-layout loader). Same arithmetic: per K step, each weight of the
// BN x BK block is dequantized once to bf16 (qmm_packed.py:629-637) into LDS and multiplied with
// the BM x BK activation block; accumulation in fp32; bf16 out.
//
// Geometry: BM = BN = 256, BK = 64 (one quantization group per K step), 8 waves in a 2 x 4
// arrangement (two per SIMD, so one wave's loads, dequantization and LDS stores overlap the
// other's MFMAs), each wave a 128 x 64 block of 4 x 2 MFMA 32x32x16 tiles (64 x 32 in the 128 x 128
// tiles of stream-K and tail launches, 64 x 64 in the 128 x 256 tiles of stream-K launches). LDS holds two stages of [BM][64 + 8] bf16 for the
// activations and [BN][64 + 8] for the dequantized weights (147 KB at 256 x 256); the 144-byte
// row pitch keeps the 16-byte fragment reads free of bank conflicts.
//
// 256 x 256 tiles with 8-group scale blocks (K % 512 == 0, the prefill projections), whole or in
// stream-K segments, run gemm_ws_kernel instead: the same tiles, MFMA order and partial slots,
// with four extra waves doing all loads, dequantization and LDS stores while the eight MFMA waves
// only read fragments and multiply.
//
// Pipeline: the raw inputs of a K step (activation chunks, packed codes) are loaded into registers
// two steps ahead of their use (four in the stream-K launches), through buffer resources (rows past M and columns past N read as
// zero); scales and biases come 8 groups per 16-byte load when K % 512 == 0. While the MFMAs of
// step kt run from LDS stage kt % 2, the waves write step kt + 1 into the other stage: activations
// as loaded, weights dequantized exactly in registers (dequant_word_fast; a thread whose group has
// a scale outside its range rewrites its words with dequant_word). One barrier per step.
//
// Work decomposition, chosen by gemm_plan:
//  * More 128 x 128 tiles than CUs: whole 256 x 256 tiles, one per workgroup, in rounds of one per
//    CU; when the last round would leave most CUs idle, its tiles are cut into 128 x 128 quarters in
//    a second launch. Workgroup ids are remapped so that consecutive tiles land on one XCD, and
//    tiles are walked in groups of 4 row tiles, so a group shares weight and activation blocks in
//    L2.
//  * At most one 128 x 128 tile per CU (65-256 rows of the model's projections): stream-K over
//    128 x 128 tiles, or 128 x 256 past 128 rows or for K >= 8192 (with 8-group scale blocks). The
//    tiles x K units are split evenly over every resident workgroup (one per CU, with a 4-step
//    register ring when K % 512 == 0: 65-128 rows 2-6% faster than two per CU with a 2-step ring); a
//    workgroup's first and last segments may cover part of a tile and leave fp32 partial tiles,
//    which gemm_sk_reduce_kernel adds in K order (the same bits whichever workgroup ran a segment).
//  * Long K (>= 8192) with whole 256 x 256 tiles for at most 70% of the CUs and at least 256 rows
//    (512-2048 rows of the down projection): the same stream-K over 256 x 256 tiles, one workgroup per CU.
// The output tile is staged through LDS and stored as 16-byte row chunks.
#include <type_traits>

#include "qmm4_common.h"
#include "qmm4_kernels.h"

namespace qmm4 {

namespace {

constexpr int BK = 64, LDK = BK + 8;  // K step; LDS row pitch (bf16) of a K step
constexpr int kWaves = 8;  // a 2 x 4 wave grid, two waves per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kWavesN = kWaves / 2;
constexpr int kGroupM = 4;
constexpr int kTile = 256;            // the grid's tile; tail launches cut a tile into 128 x 128 quarters
constexpr int kSkRing = 4;            // K steps of raw inputs in registers, stream-K launches with SB8

struct GemmParams {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int M, N, K;
  int tiles_m, tiles_n;  // tiles of the grid (256 x 256, or BM x BN for a stream-K launch)
  int tile0;             // first tile (in walk order) of this launch
  int quarter;           // 1: each workgroup computes one 128 x 128 quarter of a 256 x 256 tile
  // Stream-K (sk = 1): the tiles x K units (ups K steps each) are split into G contiguous
  // ranges, one per workgroup; a workgroup runs its range tile segment by tile segment. A segment
  // covering a whole tile writes bf16 y; a workgroup's first and last segments may cover part of
  // a tile and then leave fp32 partial tiles in part[(workgroup * 2 + slot) * BM * BN] (slot 0:
  // first segment, 1: last), which the reduce kernel adds in K order.
  int sk;
  int sk_tiles;      // tiles in the split range (quarter = 1: 128 x 128 quarters of the 256 x 256
                     // tiles from tile0 on, quarter t of tile tile0 + t / 4)
  int upt;           // K units per tile
  int ups;           // K steps (BK) per unit
  long long U;       // tiles * upt
  float* part;
};

// Stream-K range of workgroup p: units [p U / G, (p + 1) U / G).
__host__ __device__ inline long long sk_start(int p, long long U, int G) { return (long long)p * U / G; }
// The workgroup whose range holds unit u.
__host__ __device__ inline int sk_owner(long long u, long long U, int G) {
  return (int)(((u + 1) * (long long)G + U - 1) / U) - 1;
}

template <int BM, int BN>
struct GemmCfg {
  static constexpr int WM = BM / 2, WN = BN / kWavesN;  // wave tile (2 x kWavesN waves)
  static constexpr int I = WM / 32, J = WN / 32;        // MFMA 32x32 blocks per wave
  static constexpr int RPP = kThreads / 8;              // activation rows per load pass
  static constexpr int AJ = BM / RPP;                   // activation chunks per thread per step
  static constexpr int WPT = BN * 8 / kThreads;         // code words per thread per step
  static constexpr int TPC = 8 / WPT;                   // threads per weight column
  static constexpr int WV = (WPT + 3) / 4;              // 16-byte word vectors per thread
  static constexpr int LDC = BN + 8;                    // LDS row pitch (bf16) of the output tile
  static constexpr size_t kSmem = (size_t)2 * (BM + BN) * LDK * sizeof(uint16_t);
  static constexpr int kPartF4 = BM * BN / 4;           // f32x4 items of a partial tile
  static_assert((size_t)BM * LDC * sizeof(uint16_t) <= kSmem, "output tile fits the K-step stages");
  static_assert(I >= 1 && J >= 1 && (WPT == 2 || WPT == 4 || WPT == 8) && AJ % 2 == 0, "tile shape");
};

// One K step's raw inputs held by a thread.
template <class C>
struct Raw {
  u32x4 a[C::AJ];     // activations: rows a_r0 + RPP j of the tile, 16-byte chunk a_kc of the step
  u32x4 w[C::WV];     // code words WPT * b_part .. + WPT - 1 of column n0 + b_col
  uint32_t s, b;      // that group's scale and bias (bf16 bits)
};

// Partial-tile item e (f32x4) of a wave's accumulators: item ((((wave * I + i) * J + j) * 4 + rq)
// * 64 + lane) holds acc[i][j][4 rq .. 4 rq + 3] of that lane.
template <class C>
__device__ __forceinline__ void part_item_coords(int e, int* m, int* n) {
  const int lane = e & 63;
  int rest = e >> 6;
  const int rq = rest & 3;
  rest >>= 2;
  const int j = rest % C::J;
  rest /= C::J;
  const int i = rest % C::I;
  const int wave = rest / C::I;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  *m = wm * C::WM + i * 32 + 8 * rq + 4 * (lane >> 5);  // rows m .. m + 3 of the item's four values
  *n = wn * C::WN + j * 32 + (lane & 31);
}

// SB8: scales and biases are loaded 8 groups (8 K steps) at a time with one 16-byte load per
// column (K % 512 == 0); otherwise one 2-byte load per K step.
// D: K steps of raw inputs held in registers (a ring; step kt + D is loaded as step kt is written
// out). The 128 x 128 configuration with D = 2 is held to 128 VGPRs so that two workgroups share a
// CU (the quarter tiles of full-tile launches); stream-K launches with SB8 use D = 4 at one
// workgroup per CU.
template <int BM, int BN, bool SB8, int D = 2>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(BM == 128 && D == 2 ? 4 : 2)))
void gemm_kernel(GemmParams P) {
  static_assert(D == 2 || (SB8 && D == 4), "raw ring depth: its index must be static in the loop unrolled by 8");
  using C = GemmCfg<BM, BN>;
  constexpr int I = C::I, J = C::J, AJ = C::AJ, WPT = C::WPT, LDC = C::LDC;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* As = smem;                    // [2][BM * LDK]
  uint16_t* Bs = smem + 2 * BM * LDK;     // [2][BN * LDK]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int nk = P.K / BK;  // even: K % 128 == 0

  // Workgroup order: an XCD-contiguous remap (consecutive walk positions on one XCD) for
  // full-tile and stream-K launches; a quarter launch gives each tile's four 128 x 128 quarters
  // to four consecutive workgroups.
  const int G = gridDim.x;
  int bid = blockIdx.x;
  int q = 0;
  if (P.quarter && !P.sk) {
    q = bid & 3;
    bid >>= 2;
  } else if ((G & 7) == 0) {
    bid = (bid & 7) * (G >> 3) + (bid >> 3);
  }
  // Tile id -> first row and column: a grouped row-major walk (kGroupM row tiles at a time, so a
  // group shares weight and activation blocks in L2).
  const int tile_rows = P.sk && !P.quarter ? BM : kTile, tile_cols = P.sk && !P.quarter ? BN : kTile;
  auto tile_origin = [&](int id, int* m0, int* n0) __attribute__((always_inline)) {
    const int per_group = kGroupM * P.tiles_n;
    const int group = id / per_group;
    const int first_m = group * kGroupM;
    const int gm = min(kGroupM, P.tiles_m - first_m);
    const int in_group = id - group * per_group;
    *m0 = (first_m + in_group % gm) * tile_rows + (q >> 1) * BM;
    *n0 = (in_group / gm) * tile_cols + (q & 1) * BN;
  };

  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.x), 0, rsrc_bytes((unsigned long long)P.M * P.K * 2), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(P.w), 0, rsrc_bytes((unsigned long long)P.N * (P.K >> 1)), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.s), 0, rsrc_bytes((unsigned long long)P.N * (P.K >> 6) * 2), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.b), 0, rsrc_bytes((unsigned long long)P.N * (P.K >> 6) * 2), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      P.y, 0, rsrc_bytes((unsigned long long)P.M * P.N * 2), kBufferRsrcWord3);

  // Loader roles. Activations: 16-byte chunk a_kc of rows a_r0 + 64 j (row j's offset goes in the
  // scalar offset). Weights: words WPT * b_part .. + WPT - 1 of column n0 + b_col.
  const int a_kc = tid & 7;
  const int a_r0 = tid >> 3;
  const int xrowp = C::RPP * P.K * 2;  // byte distance of consecutive load passes
  const int b_col = tid / C::TPC, b_part = tid % C::TPC;
  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 8;

  f32x16 acc[I][J];

  // One tile segment: K steps [kb, ke) of the tile at (m0, n0) into acc (kb and ke even; with
  // SB8 multiples of 8).
  auto run_segment = [&](int m0, int n0, int kb, int ke) __attribute__((always_inline)) {
    const uint32_t xoff = (uint32_t)(m0 + a_r0) * (uint32_t)P.K * 2u + (uint32_t)a_kc * 16u;
    const uint32_t col = (uint32_t)(n0 + b_col);
    const uint32_t woff = col * (uint32_t)(P.K >> 1) + (uint32_t)(b_part * WPT * 4);
    const uint32_t soff = col * (uint32_t)(P.K >> 6) * 2u;

    Raw<C> raw[D];
    // Steps past the segment's last are clamped to it (their data is written to an LDS stage
    // nobody reads).
    auto load = [&](int kt, Raw<C>& R) {
      const int k = kt < ke ? kt : ke - 1;
#pragma unroll
      for (int j = 0; j < AJ; ++j)
        R.a[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, xoff, k * BK * 2 + j * xrowp, 0);
      if constexpr (WPT >= 4) {
#pragma unroll
        for (int v = 0; v < C::WV; ++v) R.w[v] = __builtin_amdgcn_raw_buffer_load_b128(rw, woff + v * 16, k * 32, 0);
      } else {
        const u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(rw, woff, k * 32, 0);
        R.w[0] = u32x4{t.x, t.y, 0u, 0u};
      }
      if constexpr (!SB8) {
        R.s = __builtin_amdgcn_raw_buffer_load_b16(rs, soff, k * 2, 0);
        R.b = __builtin_amdgcn_raw_buffer_load_b16(rb, soff, k * 2, 0);
      }
    };
    // SB8: groups 8 q .. 8 q + 7 of this thread's column; scur holds the block of the step being
    // written to LDS, snext the following block (loaded 3 steps before it is first needed).
    u32x4 scur = {0u, 0u, 0u, 0u}, bcur = scur, snext = scur, bnext = scur;
    auto load_sb8 = [&](int kt, u32x4& s8, u32x4& b8) __attribute__((always_inline)) {
      const int k = kt < ke ? kt : kb;
      s8 = __builtin_amdgcn_raw_buffer_load_b128(rs, soff, k * 2, 0);
      b8 = __builtin_amdgcn_raw_buffer_load_b128(rb, soff, k * 2, 0);
    };
    // Group kt % 8 of a block: dword (kt % 8) / 2, half kt % 2 (wave-uniform selects).
    auto pick = [&](const u32x4& v, int kt) __attribute__((always_inline)) {
      const int d = (kt >> 1) & 3;
      const uint32_t w = d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w;
      return (kt & 1) ? (w >> 16) : (w & 0xFFFFu);
    };
    // Group G of a block held in registers, G known at compile time: a select on a run-time group
    // would read both blocks' registers, one of them possibly still being loaded, and make the
    // compiler wait for every load in flight at each step.
    auto pick_c = [&](const u32x4& v, auto gc) __attribute__((always_inline)) {
      constexpr int G = decltype(gc)::value;
      const uint32_t w = G / 2 == 0 ? v.x : G / 2 == 1 ? v.y : G / 2 == 2 ? v.z : v.w;
      return (G & 1) ? (w >> 16) : (w & 0xFFFFu);
    };
    // Scale and bias bits of step kt for the weight stores.
    auto sb_of =[&](const Raw<C>& R, int kt, uint32_t& sb, uint32_t& bb) __attribute__((always_inline)) {
      if constexpr (SB8) {
        sb = pick(scur, kt);
        bb = pick(bcur, kt);
      } else {
        sb = R.s & 0xFFFFu;
        bb = R.b & 0xFFFFu;
      }
    };
    auto store_a = [&](const Raw<C>& R, int st, int j0, int j1) {
      uint16_t* as = As + st * BM * LDK + a_r0 * LDK + a_kc * 8;
#pragma unroll
      for (int j = j0; j < j1; ++j) *reinterpret_cast<u32x4*>(as + C::RPP * j * LDK) = R.a[j];
    };
    auto store_b_fast = [&](const Raw<C>& R, int st, int j0, int j1, uint32_t sbits, uint32_t bbits) {
      uint16_t* bs = Bs + st * BN * LDK + b_col * LDK + b_part * WPT * 8;
      const float sf = bf16_to_f32(sbits), bf = bf16_to_f32(bbits);
      const float s24 = sf * 16777216.0f, s20 = sf * 1048576.0f;
#pragma unroll
      for (int j = j0; j < j1; ++j)
        *reinterpret_cast<u32x4*>(bs + j * 8) = dequant_word_fast(R.w[j >> 2][j & 3], s24, s20, bf);
    };
    auto store_b_exact = [&](const Raw<C>& R, int st, uint32_t sbits, uint32_t bbits) {
      uint16_t* bs = Bs + st * BN * LDK + b_col * LDK + b_part * WPT * 8;
      const float sf = bf16_to_f32(sbits), bf = bf16_to_f32(bbits);
#pragma unroll
      for (int j = 0; j < WPT; ++j)
        *reinterpret_cast<u32x4*>(bs + j * 8) = dequant_word(R.w[j >> 2][j & 3], sf, sf * 0.0625f, bf);
    };

#pragma unroll
    for (int i = 0; i < I; ++i)
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Step kt: MFMAs from LDS stage kt % 2 while step kt + 1 (raw[(kt + 1) % 2]) is written into
    // the other stage; then step kt + 3 is loaded into the registers just written out.
    auto step = [&](int kt, auto parity, auto ucst) {
      constexpr int ST = decltype(parity)::value;
      constexpr int U = decltype(ucst)::value;  // SB8: kt % 8 (the loop is unrolled by 8)
      Raw<C>& R = raw[D == 2 ? (ST ^ 1) : (U + 1) % D];
      uint32_t sbits, bbits;
      if constexpr (SB8) {
        // Step kt + 1's group: of the current block, or the first of the next one (step 7).
        constexpr int G1 = (U + 1) & 7;
        sbits = pick_c(U < 7 ? scur : snext, std::integral_constant<int, G1>{});
        bbits = pick_c(U < 7 ? bcur : bnext, std::integral_constant<int, G1>{});
      } else {
        sb_of(R, kt + 1, sbits, bbits);
      }
      const uint16_t* as = As + ST * BM * LDK + (wm * C::WM + lrow) * LDK + lk;
      const uint16_t* bs = Bs + ST * BN * LDK + (wn * C::WN + lrow) * LDK + lk;
      // Fragments are double-buffered across the four 16-k sub-steps: sub-step ks + 1's reads are
      // issued before sub-step ks's MFMAs, so LDS latency hides behind them.
      bf16x8 Af[2][I], Bf[2][J];
      auto frags = [&](int ks, int sl) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < I; ++i)
          Af[sl][i] = as_bf16x8(*reinterpret_cast<const u32x4*>(as + i * 32 * LDK + ks * 16));
#pragma unroll
        for (int j = 0; j < J; ++j)
          Bf[sl][j] = as_bf16x8(*reinterpret_cast<const u32x4*>(bs + j * 32 * LDK + ks * 16));
      };
      frags(0, 0);
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        if (ks + 1 < BK / 16) frags(ks + 1, (ks + 1) & 1);
#pragma unroll
        for (int i = 0; i < I; ++i)
#pragma unroll
          for (int j = 0; j < J; ++j) acc[i][j] = Mfma<32>::mma(Af[ks & 1][i], Bf[ks & 1][j], acc[i][j]);
        if (ks == 0) store_a(R, ST ^ 1, 0, AJ / 2);
        if (ks == 1) store_a(R, ST ^ 1, AJ / 2, AJ);
        if (ks == 2) store_b_fast(R, ST ^ 1, 0, WPT / 2, sbits, bbits);
        if (ks == 3) store_b_fast(R, ST ^ 1, WPT / 2, WPT, sbits, bbits);
      }
      if (!fast_scale_ok(sbits)) store_b_exact(R, ST ^ 1, sbits, bbits);
      __syncthreads();
      load(kt + 1 + D, R);
      if constexpr (SB8)
        if constexpr (U == (D == 2 ? 5 : 1)) load_sb8(kt + (D == 2 ? 3 : 7), snext, bnext);  // the next block, first used at step 7
      // Keep these loads right behind the barrier (the scheduler would sink them toward their use
      // two steps later, into the middle of the next step's MFMAs).
      __builtin_amdgcn_sched_barrier(0);
    };

    // Prologue: steps kb .. kb + D - 1 in registers, step kb in LDS, step kb + D in flight.
#pragma unroll
    for (int i = 0; i < D; ++i) load(kb + i, raw[i]);
    if constexpr (SB8) load_sb8(kb, scur, bcur);
    {
      uint32_t sbits, bbits;
      sb_of(raw[0], kb, sbits, bbits);
      store_a(raw[0], 0, 0, AJ);
      store_b_fast(raw[0], 0, 0, WPT, sbits, bbits);
      if (!fast_scale_ok(sbits)) store_b_exact(raw[0], 0, sbits, bbits);
    }
    load(kb + D, raw[0]);
    __syncthreads();

    auto two = [&](int kt, auto u0) __attribute__((always_inline)) {
      constexpr int U0 = decltype(u0)::value;
      step(kt, std::integral_constant<int, 0>{}, std::integral_constant<int, U0>{});
      step(kt + 1, std::integral_constant<int, 1>{}, std::integral_constant<int, U0 + 1>{});
    };
    if constexpr (SB8) {
      // Unrolled by 8 (kb and ke are multiples of 8), so every step knows its group statically and
      // the next block's registers become the current ones by a plain copy at the end.
      for (int kt = kb; kt < ke; kt += 8) {
        two(kt, std::integral_constant<int, 0>{});
        two(kt + 2, std::integral_constant<int, 2>{});
        two(kt + 4, std::integral_constant<int, 4>{});
        two(kt + 6, std::integral_constant<int, 6>{});
        scur = snext;
        bcur = bnext;
      }
    } else {
      for (int kt = kb; kt < ke; kt += 2) two(kt, std::integral_constant<int, 0>{});
    }
  };

  // The tile as bf16 through LDS (every wave is past the last step's reads), then 16-byte row
  // chunks; rows past M fall outside y's buffer resource, columns past N are skipped (N % 16 == 0,
  // so a chunk is entirely inside or outside).
  auto write_tile = [&](int m0, int n0) __attribute__((always_inline)) {
    uint16_t* Cs = smem;
#pragma unroll
    for (int i = 0; i < I; ++i)
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int n = wn * C::WN + j * 32 + lrow;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = wm * C::WM + i * 32 + Mfma<32>::row(lane, r);
          Cs[m * LDC + n] = (uint16_t)(pack_bf16x2(acc[i][j][r], 0.0f) & 0xFFFFu);
        }
      }
    __syncthreads();
    constexpr int kChunksPerRow = BN / 8;
#pragma unroll 4
    for (int c = tid; c < BM * kChunksPerRow; c += kThreads) {
      const int r = c / kChunksPerRow, ch = c % kChunksPerRow;
      const int gn = n0 + ch * 8;
      if (gn < P.N) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(Cs + r * LDC + ch * 8);
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, ((uint32_t)(m0 + r) * (uint32_t)P.N + (uint32_t)gn) * 2u, 0, 0);
      }
    }
  };

  if (!P.sk) {
    int m0, n0;
    tile_origin(P.tile0 + bid, &m0, &n0);
    run_segment(m0, n0, 0, nk);
    write_tile(m0, n0);
    return;
  }

  // Stream-K: this workgroup's units, tile segment by tile segment.
  const long long u0 = sk_start(bid, P.U, G), u1 = sk_start(bid + 1, P.U, G);
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      P.part, 0, rsrc_bytes((unsigned long long)G * 2 * C::kPartF4 * 16), kBufferRsrcWord3);
  for (long long u = u0; u < u1;) {
    const int t = (int)(u / P.upt);
    const long long tb = (long long)t * P.upt;
    const long long e = u1 < tb + P.upt ? u1 : tb + P.upt;
    const int kb = (int)(u - tb) * P.ups, ke = (int)(e - tb) * P.ups;
    int m0, n0;
    if (P.quarter) {
      q = t & 3;
      tile_origin(P.tile0 + (t >> 2), &m0, &n0);
    } else {
      tile_origin(t, &m0, &n0);
    }
    run_segment(m0, n0, kb, ke);
    if (kb == 0 && ke == nk) {
      write_tile(m0, n0);
    } else {
      // A part of the tile: its fp32 sums to this workgroup's slot (0: its first segment, 1: its
      // last), item-major per lane (16-byte stores).
      const uint32_t slot = (uint32_t)bid * 2u + (u == u0 ? 0u : 1u);
#pragma unroll
      for (int i = 0; i < I; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const uint32_t item = (uint32_t)((((wave * I + i) * J + j) * 4 + rq) * 64 + lane);
            const f32x4 v = {acc[i][j][4 * rq], acc[i][j][4 * rq + 1], acc[i][j][4 * rq + 2], acc[i][j][4 * rq + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp,
                                                   (slot * (uint32_t)C::kPartF4 + item) * 16u, 0, 0);
          }
    }
    u = e;
    __syncthreads();  // the next segment's prologue reuses the LDS stages (and the output tile)
  }
}

// Stream-K fix-up: the tiles split between workgroups, their partial sums added in K order (the
// owners of a tile's units in increasing order; a tile is the last segment of its first owner
// when that owner's range began in an earlier tile), one f32x4 item per thread, bf16 y.
constexpr int kSkRedThreads = 256;
template <int BM, int BN>
__global__ __launch_bounds__(kSkRedThreads) void gemm_sk_reduce_kernel(GemmParams P, int G) {
  using C = GemmCfg<BM, BN>;
  const long long it = (long long)blockIdx.x * kSkRedThreads + threadIdx.x;
  const int t = (int)(it / C::kPartF4);
  const int e = (int)(it - (long long)t * C::kPartF4);
  if (t >= P.sk_tiles) return;
  const long long tb = (long long)t * P.upt;
  const int lo = sk_owner(tb, P.U, G), hi = sk_owner(tb + P.upt - 1, P.U, G);
  if (lo == hi) return;  // one workgroup ran the whole tile and wrote it
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      P.part, 0, rsrc_bytes((unsigned long long)G * 2 * C::kPartF4 * 16), kBufferRsrcWord3);
  f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = lo; c <= hi; ++c) {
    const uint32_t slot = (uint32_t)c * 2u + ((c == lo && sk_start(lo, P.U, G) < tb) ? 1u : 0u);
    const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rp, (slot * (uint32_t)C::kPartF4 + (uint32_t)e) * 16u, 0, 0));
    sum[0] += v[0]; sum[1] += v[1]; sum[2] += v[2]; sum[3] += v[3];
  }
  // Tile origin (the same grouped walk as the main kernel; a quarter of a 256 x 256 tile when the
  // split range is the quarters of a full-tile launch's last tiles).
  const int id = P.quarter ? P.tile0 + (t >> 2) : t, qq = P.quarter ? t & 3 : 0;
  const int tr = P.quarter ? kTile : BM, tc = P.quarter ? kTile : BN;
  const int per_group = kGroupM * P.tiles_n;
  const int group = id / per_group;
  const int first_m = group * kGroupM;
  const int gm = min(kGroupM, P.tiles_m - first_m);
  const int in_group = id - group * per_group;
  const int m0 = (first_m + in_group % gm) * tr + (qq >> 1) * BM, n0 = (in_group / gm) * tc + (qq & 1) * BN;
  int mi, ni;
  part_item_coords<C>(e, &mi, &ni);
  const int n = n0 + ni;
  if (n >= P.N) return;
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      P.y, 0, rsrc_bytes((unsigned long long)P.M * P.N * 2), kBufferRsrcWord3);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = m0 + mi + r;
    if (m < P.M)
      __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(pack_bf16x2(sum[r], 0.0f) & 0xFFFFu), ry,
                                            ((uint32_t)m * (uint32_t)P.N + (uint32_t)n) * 2u, 0, 0);
  }
}

template <int BM, int BN, bool SB8, int D = 2>
hipError_t launch_tiles(const GemmParams& P, int blocks, hipStream_t stream) {
  constexpr size_t smem = GemmCfg<BM, BN>::kSmem;
  static bool attr_set = false;  // the attribute is per function; setting it twice is harmless
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<BM, BN, SB8, D>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((gemm_kernel<BM, BN, SB8, D>), dim3(blocks), dim3(kThreads), smem, stream, P);
  return hipGetLastError();
}

// 256 x 256 tiles with K % 512 == 0 (whole, or stream-K segments), waves split by role: waves 0-7
// (two per SIMD, the 2 x 4 wave grid and MFMA order of gemm_kernel, so the same bits) only read
// fragments and run MFMAs; waves 8-11 (one per SIMD) only load, dequantize and store the next K
// step into the other LDS stage. A SIMD overlaps one wave's MFMAs with another wave's VALU far
// better than MFMAs and VALU interleaved inside one wave: a dequantization wave beside an MFMA wave
// ran in the time of the dequantization alone, where waves mixing both ran in ~0.8 of the sum of
// the two. 12 waves share the SIMDs' 512 registers per lane: at most 168 per wave (154 used).
// Producer thread pt (0-255): activation chunk pt % 8 of rows pt / 8 + 32 j (j < 8) and the 8 code
// words (one group, 64 k) of column pt per K step, two steps ahead in registers; the column's scale
// and bias come 8 groups per 16-byte load.
constexpr int kWsProd = 4;                                  // producer waves
constexpr int kWsThreads = 64 * (kWaves + kWsProd);
constexpr int kWsD = 2;                                     // K steps of raw inputs in registers
__global__ __launch_bounds__(kWsThreads) __attribute__((amdgpu_waves_per_eu(3)))
void gemm_ws_kernel(GemmParams P) {
  using C = GemmCfg<256, 256>;
  constexpr int BM = 256, BN = 256, I = C::I, J = C::J, LDC = C::LDC;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* As = smem;
  uint16_t* Bs = smem + 2 * BM * LDK;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool mma = wave < kWaves;
  const int wm = wave / kWavesN, wn = wave % kWavesN;  // MFMA waves: the 2 x 4 grid of gemm_kernel
  const int nk = P.K / BK;                              // a multiple of 8
  const int G = gridDim.x;
  int bid = blockIdx.x;
  if ((G & 7) == 0) bid = (bid & 7) * (G >> 3) + (bid >> 3);  // gemm_kernel's XCD-contiguous remap
  auto tile_origin = [&](int id, int* m0, int* n0) __attribute__((always_inline)) {
    const int per_group = kGroupM * P.tiles_n;
    const int group = id / per_group;
    const int first_m = group * kGroupM;
    const int gm = min(kGroupM, P.tiles_m - first_m);
    const int in_group = id - group * per_group;
    *m0 = (first_m + in_group % gm) * kTile;
    *n0 = (in_group / gm) * kTile;
  };
  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 8;
  const int pt = tid - 64 * kWaves;  // producer thread
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.x), 0, rsrc_bytes((unsigned long long)P.M * P.K * 2), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(P.w), 0, rsrc_bytes((unsigned long long)P.N * (P.K >> 1)), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.s), 0, rsrc_bytes((unsigned long long)P.N * (P.K >> 6) * 2), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.b), 0, rsrc_bytes((unsigned long long)P.N * (P.K >> 6) * 2), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      P.y, 0, rsrc_bytes((unsigned long long)P.M * P.N * 2), kBufferRsrcWord3);
  // The output tile's 16-byte row chunks from LDS, by all 12 waves; rows past M fall outside y's
  // buffer resource, columns past N are skipped.
  auto store_chunks = [&](int m0, int n0) __attribute__((always_inline)) {
    const uint16_t* Cs = smem;
    constexpr int kChunksPerRow = BN / 8;
#pragma unroll 4
    for (int c = tid; c < BM * kChunksPerRow; c += kWsThreads) {
      const int r = c / kChunksPerRow, ch = c % kChunksPerRow;
      const int gn = n0 + ch * 8;
      if (gn < P.N) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(Cs + r * LDC + ch * 8);
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, ((uint32_t)(m0 + r) * (uint32_t)P.N + (uint32_t)gn) * 2u, 0, 0);
      }
    }
  };
  // The workgroup's tile segments: the whole K of tile P.tile0 + bid, or its stream-K range of units
  // (gemm_kernel's bookkeeping: the same ranges, segments and partial slots, so
  // gemm_sk_reduce_kernel adds the same bits). f(m0, n0, kb, ke, first) per segment.
  auto for_segments = [&](auto f) __attribute__((always_inline)) {
    if (!P.sk) {
      int m0, n0;
      tile_origin(P.tile0 + bid, &m0, &n0);
      f(m0, n0, 0, nk, true);
      return;
    }
    const long long u0 = sk_start(bid, P.U, G), u1 = sk_start(bid + 1, P.U, G);
    for (long long u = u0; u < u1;) {
      const int t = (int)(u / P.upt);
      const long long tb = (long long)t * P.upt;
      const long long e = u1 < tb + P.upt ? u1 : tb + P.upt;
      int m0, n0;
      tile_origin(t, &m0, &n0);
      f(m0, n0, (int)(u - tb) * P.ups, (int)(e - tb) * P.ups, u == u0);
      u = e;
    }
  };
  // Every segment passes the same barriers in both roles: one after the producers' prologue, one
  // per K step, one between the bf16 tile's LDS writes and its stores (whole tiles), one at the end
  // (the next segment's prologue reuses the LDS stages and the output tile).

  if (mma) {
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        P.part, 0, rsrc_bytes((unsigned long long)G * 2 * C::kPartF4 * 16), kBufferRsrcWord3);
    f32x16 acc[I][J];
    auto step = [&](int st) __attribute__((always_inline)) {
      const uint16_t* as = As + st * BM * LDK + (wm * C::WM + lrow) * LDK + lk;
      const uint16_t* bs = Bs + st * BN * LDK + (wn * C::WN + lrow) * LDK + lk;
      bf16x8 Af[2][I], Bf[2][J];
      auto frags = [&](int ks, int sl) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < I; ++i)
          Af[sl][i] = as_bf16x8(*reinterpret_cast<const u32x4*>(as + i * 32 * LDK + ks * 16));
#pragma unroll
        for (int j = 0; j < J; ++j)
          Bf[sl][j] = as_bf16x8(*reinterpret_cast<const u32x4*>(bs + j * 32 * LDK + ks * 16));
      };
      frags(0, 0);
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        if (ks + 1 < BK / 16) frags(ks + 1, (ks + 1) & 1);
#pragma unroll
        for (int i = 0; i < I; ++i)
#pragma unroll
          for (int j = 0; j < J; ++j) acc[i][j] = Mfma<32>::mma(Af[ks & 1][i], Bf[ks & 1][j], acc[i][j]);
      }
      __syncthreads();
    };
    for_segments([&](int m0, int n0, int kb, int ke, bool first) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < I; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
      __syncthreads();  // step kb is in stage 0
      for (int kt = kb; kt < ke; kt += 2) {
        step(0);
        step(1);
      }
      if (kb == 0 && ke == nk) {
        // The tile as bf16 into LDS (every wave is past the last step's reads).
        uint16_t* Cs = smem;
#pragma unroll
        for (int i = 0; i < I; ++i)
#pragma unroll
          for (int j = 0; j < J; ++j) {
            const int n = wn * C::WN + j * 32 + lrow;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int m = wm * C::WM + i * 32 + Mfma<32>::row(lane, r);
              Cs[m * LDC + n] = (uint16_t)(pack_bf16x2(acc[i][j][r], 0.0f) & 0xFFFFu);
            }
          }
        __syncthreads();
        store_chunks(m0, n0);
      } else {
        // A part of the tile: its fp32 sums to this workgroup's slot (0: its first segment, 1: its
        // last), item-major per lane, as gemm_kernel stores them.
        const uint32_t slot = (uint32_t)bid * 2u + (first ? 0u : 1u);
#pragma unroll
        for (int i = 0; i < I; ++i)
#pragma unroll
          for (int j = 0; j < J; ++j)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
              const uint32_t item = (uint32_t)((((wave * I + i) * J + j) * 4 + rq) * 64 + lane);
              const f32x4 v = {acc[i][j][4 * rq], acc[i][j][4 * rq + 1], acc[i][j][4 * rq + 2], acc[i][j][4 * rq + 3]};
              __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp,
                                                     (slot * (uint32_t)C::kPartF4 + item) * 16u, 0, 0);
            }
      }
      __syncthreads();
    });
    return;
  }

  // Producers.
  const int a_kc = pt & 7, a_r0 = pt >> 3;
  constexpr int kAJ = 8;  // activation chunks per thread and step (rows a_r0 + 32 j)
  const int xrowp = 32 * P.K * 2;
  struct RawW {
    u32x4 a[kAJ];
    u32x4 w[2];
  };
  auto pick_c = [&](const u32x4& v, auto gc) __attribute__((always_inline)) {
    constexpr int Gi = decltype(gc)::value;
    const uint32_t w = Gi / 2 == 0 ? v.x : Gi / 2 == 1 ? v.y : Gi / 2 == 2 ? v.z : v.w;
    return (Gi & 1) ? (w >> 16) : (w & 0xFFFFu);
  };
  for_segments([&](int m0, int n0, int kb, int ke, bool) __attribute__((always_inline)) {
    const uint32_t xoff = (uint32_t)(m0 + a_r0) * (uint32_t)P.K * 2u + (uint32_t)a_kc * 16u;
    const uint32_t col = (uint32_t)(n0 + pt);
    const uint32_t woff = col * (uint32_t)(P.K >> 1);
    const uint32_t soff = col * (uint32_t)(P.K >> 6) * 2u;
    RawW raw[kWsD];
    // Steps past the segment's last are clamped to it (loaded into registers that are not stored).
    auto load = [&](int kt, RawW& R) __attribute__((always_inline)) {
      const int k = kt < ke ? kt : ke - 1;
#pragma unroll
      for (int j = 0; j < kAJ; ++j) R.a[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, xoff, k * BK * 2 + j * xrowp, 0);
#pragma unroll
      for (int v = 0; v < 2; ++v) R.w[v] = __builtin_amdgcn_raw_buffer_load_b128(rw, woff + v * 16, k * 32, 0);
    };
    u32x4 scur, bcur, snext = {0u, 0u, 0u, 0u}, bnext = snext;
    auto load_sb8 = [&](int kt, u32x4& s8, u32x4& b8) __attribute__((always_inline)) {
      const int k = kt < ke ? kt : kb;
      s8 = __builtin_amdgcn_raw_buffer_load_b128(rs, soff, k * 2, 0);
      b8 = __builtin_amdgcn_raw_buffer_load_b128(rb, soff, k * 2, 0);
    };
    auto put = [&](const RawW& R, int st, uint32_t sbits, uint32_t bbits) __attribute__((always_inline)) {
      uint16_t* as = As + st * BM * LDK + a_r0 * LDK + a_kc * 8;
#pragma unroll
      for (int j = 0; j < kAJ; ++j) *reinterpret_cast<u32x4*>(as + 32 * j * LDK) = R.a[j];
      uint16_t* bs = Bs + st * BN * LDK + pt * LDK;
      const float sf = bf16_to_f32(sbits), bf = bf16_to_f32(bbits);
      if (fast_scale_ok(sbits)) {
        const float s24 = sf * 16777216.0f, s20 = sf * 1048576.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x4*>(bs + j * 8) = dequant_word_fast(R.w[j >> 2][j & 3], s24, s20, bf);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x4*>(bs + j * 8) = dequant_word(R.w[j >> 2][j & 3], sf, sf * 0.0625f, bf);
      }
    };
    // Prologue: steps kb .. kb + D - 1 in registers, step kb into stage 0, then step kb + D in flight.
#pragma unroll
    for (int i = 0; i < kWsD; ++i) load(kb + i, raw[i]);
    load_sb8(kb, scur, bcur);
    put(raw[0], 0, pick_c(scur, std::integral_constant<int, 0>{}), pick_c(bcur, std::integral_constant<int, 0>{}));
    load(kb + kWsD, raw[0]);
    __syncthreads();
    // Iteration kt (the MFMA waves on stage (kt - kb) % 2): step kt + 1 into the other stage, then
    // step kt + 1 + D loaded into its registers. Unrolled by 8, so each step's group is static.
    auto it = [&](int kt, auto uc) __attribute__((always_inline)) {
      constexpr int U = decltype(uc)::value;
      constexpr int G1 = (U + 1) & 7;
      RawW& R = raw[(U + 1) % kWsD];
      if (kt + 1 < ke) {
        const uint32_t sb = pick_c(U < 7 ? scur : snext, std::integral_constant<int, G1>{});
        const uint32_t bb = pick_c(U < 7 ? bcur : bnext, std::integral_constant<int, G1>{});
        put(R, (U + 1) & 1, sb, bb);
      }
      load(kt + 1 + kWsD, R);
      if constexpr (U == 1) load_sb8(kt + 7, snext, bnext);  // the next block, first used at step kt + 7
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int kt = kb; kt < ke; kt += 8) {
      it(kt, std::integral_constant<int, 0>{});
      it(kt + 1, std::integral_constant<int, 1>{});
      it(kt + 2, std::integral_constant<int, 2>{});
      it(kt + 3, std::integral_constant<int, 3>{});
      it(kt + 4, std::integral_constant<int, 4>{});
      it(kt + 5, std::integral_constant<int, 5>{});
      it(kt + 6, std::integral_constant<int, 6>{});
      it(kt + 7, std::integral_constant<int, 7>{});
      scur = snext;
      bcur = bnext;
    }
    if (kb == 0 && ke == nk) {
      __syncthreads();  // the MFMA waves' bf16 tile is in LDS
      store_chunks(m0, n0);
    }
    __syncthreads();
  });
}

hipError_t launch_ws(const GemmParams& P, int blocks, hipStream_t stream) {
  constexpr size_t smem = GemmCfg<256, 256>::kSmem;
  static bool attr_set = false;  // the attribute is per function; setting it twice is harmless
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_ws_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(gemm_ws_kernel, dim3(blocks), dim3(kWsThreads), smem, stream, P);
  return hipGetLastError();
}

template <int BM, int BN>
hipError_t launch_sk_reduce(const GemmParams& P, int G, hipStream_t stream) {
  const long long items = (long long)P.sk_tiles * GemmCfg<BM, BN>::kPartF4;
  hipLaunchKernelGGL((gemm_sk_reduce_kernel<BM, BN>), dim3((unsigned)((items + kSkRedThreads - 1) / kSkRedThreads)),
                     dim3(kSkRedThreads), 0, stream, P, G);
  return hipGetLastError();
}

// Resident workgroups per CU of a kernel with `smem` bytes of dynamic LDS (at most 2, at least 1).
int resident_per_cu(const void* f, size_t smem) {
  int nb = 0;
  if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, kThreads, smem) != hipSuccess || nb < 1)
    nb = 1;
  return nb < 2 ? nb : 2;
}

// Resident stream-K workgroups per CU (the 128 x 128 configuration: 74 KB of LDS each).
int sk_occupancy(bool sb8) {
  static int occ[2] = {0, 0};
  int& o = occ[sb8 ? 1 : 0];
  if (o == 0)
    o = resident_per_cu(sb8 ? reinterpret_cast<const void*>(&gemm_kernel<128, 128, true, kSkRing>)
                            : reinterpret_cast<const void*>(&gemm_kernel<128, 128, false>),
                        GemmCfg<128, 128>::kSmem);
  return o;
}

// Resident workgroups per CU of the stream-K launch over 128 x 256 tiles (one: 205 VGPRs).
int sk_wide_occupancy() {
  static int o = 0;
  if (o == 0)
    o = resident_per_cu(reinterpret_cast<const void*>(&gemm_kernel<128, 256, true, kSkRing>), GemmCfg<128, 256>::kSmem);
  return o;
}

bool scale_rows_16b(const uint16_t* s, const uint16_t* b, int K) {
  return K % 512 == 0 && (reinterpret_cast<uintptr_t>(s) % 16) == 0 && (reinterpret_cast<uintptr_t>(b) % 16) == 0;
}

// Whole-tile launches: the 256 x 256 tiles of a last round that would leave more than half the CUs
// idle, launched as 128 x 128 quarters after the others (0: none).
int gemm_tail(int M, int N, int cus) {
  const int c = cus > 0 ? cus : 1;
  const int total = ((M + kTile - 1) / kTile) * ((N + kTile - 1) / kTile);
  const int rem = total % c;
  return (rem > 0 && 4 * rem <= 2 * c) ? rem : 0;
}

}  // namespace

// More 128 x 128 tiles than CUs: whole rounds of 256 x 256 tiles (one per CU at a time) in one
// launch; when the last round would leave most CUs idle, its tiles are cut into 128 x 128 quarters
// and launched next. Fewer tiles (e.g. a short prompt tail or more than 64 tree nodes over a
// narrow output): stream-K over 128 x 128 tiles, the tiles x K units split evenly over every
// resident workgroup slot, then the fix-up of the split tiles; with long K and fewer whole
// 256 x 256 tiles than CUs, stream-K over those instead.
bool gemm_plan(int M, int N, int K, int cus, size_t ws_capacity, const uint16_t* s, const uint16_t* b, GemmPlan* plan) {
  const int c = cus > 0 ? cus : 1;
  plan->sk = false;
  plan->sk256 = false;
  plan->sk_wide = false;
  plan->tail_sk = false;
  plan->G = 0;
  plan->part_bytes = 0;
  const long long tiles256 = (long long)((M + 255) / 256) * ((N + 255) / 256);
  // Stream-K over 256 x 256 tiles (one workgroup per CU, 8-step units): at least 256 rows, K of
  // 8192 or more, whole tiles for at most 70% of the CUs and at least 3.5 units per workgroup. A 256-tile step
  // does 4x the MFMAs of a 128-tile step in ~2.1x the time, against 4x the partial-tile bytes
  // (~128 MB written and read back at 256 CUs, ~40 us), so it pays where K gives each workgroup
  // enough steps. Measured (A/B, interleaved rounds, against the rules below): 512 / 768 / 1024 /
  // 1536 x 17408 -> 5120 150.6 / 216.2 / 246.6 / 327.1 -> 120.5 / 151.7 / 195.0 / 271.9 us,
  // 512 x 12288 -> 5120 107.5 -> 91.0 us, 1024 x 8192 -> 5120 122.4 -> 108.5 us, 512 x 17408 ->
  // 10240 244.5 -> 196.3 us; slower with fewer units per workgroup (256 x 8192 -> 5120 44.0 -> 59.6
  // us, 256 x 12288 -> 6144 64.0 -> 68.7 us), at K = 5120 (the up projection at 256-4096 rows,
  // 2-13% slower) and with whole tiles for most CUs (2560 / 3072 x 17408 -> 5120, 200 / 240 tiles:
  // 413.9 / 446.0 -> 417.3 / 490.2 us; 2048 rows, 160 tiles: 358.9 -> 340.8 us). Between 256 and
  // 512 rows not when the last row of 256-row tiles is at most half full (a quarter to a third of
  // the MFMA work padding): stream-K over 128 x 256 tiles (below) is faster there, 320 / 384 x
  // 17408 -> 5120 105.4 / 107.7 -> 89.4 / 92.6 us, 320 / 384 x 12288 -> 5120 79.7 / 82.9 -> 70.3 /
  // 73.4 us, but not at 448 rows (111.5 / 85.3 -> 113.0 / 87.5 us) nor past 512 rows (640 / 896 /
  // 1152 / 1408 x 17408 -> 5120 139.2 / 178.9 / 226.2 / 257.9 us against 143.4 / 186.5 / 239.1 /
  // 285.3 on 128 x 256 tiles; A/B, interleaved rounds, within the parity tolerance).
  if (M >= 256 && (M > 512 || M % 256 == 0 || M % 256 > 128) && K >= 8192 && 10 * tiles256 <= 7LL * c &&
      scale_rows_16b(s, b, K) &&
      2 * tiles256 * (K / 512) >= 7LL * c) {
    const size_t slot256 = (size_t)GemmCfg<256, 256>::kPartF4 * 16 * 2;
    if ((size_t)c * slot256 <= ws_capacity) {
      plan->sk = true;
      plan->sk256 = true;
      plan->G = c;
      plan->part_bytes = (size_t)c * slot256;
      return true;
    }
  }
  // Stream-K over 128 x 128 tiles while there are no more such tiles than CUs; beyond that, whole
  // 256 x 256 tiles (a 128 x 128 tile reads its LDS fragments for half as many MFMAs) unless they
  // would fill less than half the CUs (and there are at most 1.25 128-tiles per CU), or less than
  // all of them with a half-empty last row of tiles (and at most 2 128-tiles per CU). Measured on
  // MI355X (A/B, interleaved rounds): 192 / 256 / 384 x 5120 -> 17408 85.7 / 89.6 / 118.4 -> 71.5
  // / 73.4 / 109.4 us (68 or 136 whole tiles), 1024 x 17408 -> 5120 278.3 -> 251.4 us (80 whole
  // tiles); 1536 x 17408 -> 5120 (120 full whole tiles, 480 quarters) 316 us, 419 on stream-K;
  // 512 and 1024 x 5120 -> 17408 (136 and 272 full tiles) stay on whole tiles. Stream-K (over
  // 128 x 256 tiles) wherever whole tiles fill less than one round was slower on the role-split
  // whole tiles: 640 / 768 x 5120 -> 17408 (204 tiles) 129.1 / 135.8 -> 146.9 / 168.2 us, 1536 /
  // 2048 x 5120 -> 5120 99.9 / 121.5 -> 109.8 / 133.7 us, 512 x 5120 -> 17408 118.9 -> 120.0 us;
  // 2-4% faster only at 96 tiles (512 x 5120 -> 12288, 1024 x 5120 -> 6144).
  const long long tiles = (long long)((M + 127) / 128) * ((N + 127) / 128);
  const bool sk_tiles = tiles <= c || (2 * tiles256 < c && 4 * tiles <= 5LL * c) ||
                        (M % 256 != 0 && tiles256 < c && tiles <= 2LL * c);
  // At most 128 rows over many columns: whole 256 x 256 tiles would pad the rows to 256, so
  // stream-K over 128 x 256 tiles instead when that gives every CU at least 3 units. A/B against
  // whole tiles (interleaved rounds, within the parity tolerance): 72 / 96 / 128 x 5120 -> 65984
  // 141.5 / 144.3 / 148.0 -> 116.2 / 119.7 / 124.6 us, 128 x 5120 -> 248320 523.0 -> 405.9 us.
  const bool sk_rows = !sk_tiles && M <= 128 && scale_rows_16b(s, b, K) &&
                       (long long)((N + 255) / 256) * (K / 512) >= 3LL * c;
  const bool sk = sk_tiles || sk_rows;
  if (!sk) {
    // A tail of fewer quarters than CUs: stream-K over the quarters (their K spread over every
    // CU) instead of one quarter per workgroup on a few CUs.
    const int tail = gemm_tail(M, N, c);
    if (tail > 0 && 4 * tail < c && scale_rows_16b(s, b, K)) {
      const long long Ut = 4LL * tail * (K / 512);
      long long Gt = (long long)c * sk_occupancy(true);
      if (Gt > Ut) Gt = Ut;
      const size_t slot = (size_t)GemmCfg<128, 128>::kPartF4 * 16 * 2;
      if ((size_t)Gt * slot <= ws_capacity && Gt >= 1) {
        plan->tail_sk = true;
        plan->G = (int)Gt;
        plan->part_bytes = (size_t)Gt * slot;
      }
    }
    return true;
  }
  const bool sb8 = scale_rows_16b(s, b, K);
  // 128 x 256 tiles (a step's fragment reads and barrier shared by twice the MFMAs, but partial
  // tiles twice as large) past 128 rows, for K >= 8192, or where stream-K replaces whole tiles at up
  // to 128 rows (sk_rows); 128 x 128 otherwise. A/B (interleaved rounds,
  // within the parity tolerance): 256 / 384 / 160 x 5120 -> 17408 75.2 / 107.8 / 71.3 -> 74.0 /
  // 94.4 / 69.5 us, 128 / 256 x 17408 -> 5120 51.1 / 82.2 -> 50.0 / 73.3 us, 200 x 5120 -> 10240
  // 52.5 -> 50.1 us; at 113 / 128 x 5120 -> 17408 48.9 / 50.0 -> 51.4 / 51.9 us. Those splits
  // give every workgroup at least 2.6 units; the wide tiles need at least 2 per CU.
  const int ups = sb8 ? 8 : 2;
  const long long tiles_w = (long long)((M + 127) / 128) * ((N + 255) / 256);
  const bool wide = sb8 && (M > 128 || K >= 8192 || sk_rows) && tiles_w * (K / BK / ups) >= 2LL * c;
  const long long tiles_sk = wide ? tiles_w : tiles;
  const long long U = tiles_sk * (K / BK / ups);
  long long G = (long long)c * (wide ? sk_wide_occupancy() : sk_occupancy(sb8));
  if (G > U) G = U;
  // two partial tiles per workgroup
  const size_t slot = (size_t)(wide ? GemmCfg<128, 256>::kPartF4 : GemmCfg<128, 128>::kPartF4) * 16 * 2;
  if ((size_t)G * slot > ws_capacity) G = (long long)(ws_capacity / slot);
  if (G < 1 || G < c / 2) return true;  // too little workspace to spread the tiles: whole tiles instead
  plan->sk = true;
  plan->sk_wide = wide;
  plan->G = (int)G;
  plan->part_bytes = (size_t)G * slot;
  return true;
}

hipError_t launch_gemm(const GemmPlan& plan, const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                       uint16_t* y, float* part, int M, int N, int K, int cus, hipStream_t stream) {
  GemmParams P;
  P.x = x; P.w = w; P.s = s; P.b = b; P.y = y;
  P.M = M; P.N = N; P.K = K;
  P.sk = 0; P.sk_tiles = 0; P.upt = 0; P.ups = 0; P.U = 0; P.part = part;
  // 16-byte loads of 8 groups need 16-byte aligned scale rows and pointers.
  const bool sb8 = scale_rows_16b(s, b, K);
  if (plan.sk256) {
    if (!sb8) return hipErrorInvalidValue;
    P.tiles_m = (M + 255) / 256;
    P.tiles_n = (N + 255) / 256;
    P.tile0 = 0;
    P.quarter = 0;
    P.sk = 1;
    P.ups = 8;
    P.upt = K / BK / P.ups;
    P.sk_tiles = P.tiles_m * P.tiles_n;
    P.U = (long long)P.sk_tiles * P.upt;
    hipError_t e = launch_ws(P, plan.G, stream);
    if (e != hipSuccess) return e;
    return launch_sk_reduce<256, 256>(P, plan.G, stream);
  }
  if (plan.sk) {
    if (plan.sk_wide && !sb8) return hipErrorInvalidValue;
    P.tiles_m = (M + 127) / 128;
    P.tiles_n = plan.sk_wide ? (N + 255) / 256 : (N + 127) / 128;
    P.tile0 = 0;
    P.quarter = 0;
    P.sk = 1;
    P.ups = sb8 ? 8 : 2;
    P.upt = K / BK / P.ups;
    P.sk_tiles = P.tiles_m * P.tiles_n;
    P.U = (long long)P.sk_tiles * P.upt;
    if (plan.sk_wide) {
      hipError_t e = launch_tiles<128, 256, true, kSkRing>(P, plan.G, stream);
      if (e != hipSuccess) return e;
      return launch_sk_reduce<128, 256>(P, plan.G, stream);
    }
    hipError_t e = sb8 ? launch_tiles<128, 128, true, kSkRing>(P, plan.G, stream)
                       : launch_tiles<128, 128, false>(P, plan.G, stream);
    if (e != hipSuccess) return e;
    return launch_sk_reduce<128, 128>(P, plan.G, stream);
  }
  P.tiles_m = (M + kTile - 1) / kTile;
  P.tiles_n = (N + kTile - 1) / kTile;
  const int main_tiles = P.tiles_m * P.tiles_n - gemm_tail(M, N, cus);
  const int tail = P.tiles_m * P.tiles_n - main_tiles;
  if (main_tiles > 0) {
    P.tile0 = 0;
    P.quarter = 0;
    hipError_t e = sb8 ? launch_ws(P, main_tiles, stream)
                       : launch_tiles<256, 256, false>(P, main_tiles, stream);
    if (e != hipSuccess) return e;
  }
  if (tail > 0 && plan.tail_sk) {
    if (!sb8) return hipErrorInvalidValue;
    P.tile0 = main_tiles;
    P.quarter = 1;
    P.sk = 1;
    P.ups = 8;
    P.upt = K / BK / P.ups;
    P.sk_tiles = 4 * tail;
    P.U = (long long)P.sk_tiles * P.upt;
    hipError_t e = launch_tiles<128, 128, true, kSkRing>(P, plan.G, stream);
    if (e != hipSuccess) return e;
    return launch_sk_reduce<128, 128>(P, plan.G, stream);
  }
  if (tail > 0) {
    P.tile0 = main_tiles;
    P.quarter = 1;
    hipError_t e = sb8 ? launch_tiles<128, 128, true>(P, 4 * tail, stream)
                       : launch_tiles<128, 128, false>(P, 4 * tail, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace qmm4
