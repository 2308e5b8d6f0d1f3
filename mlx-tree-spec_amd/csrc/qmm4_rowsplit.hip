// Row-split kernel for up to 16 rows of x and many output columns: y = x @ dequant(w)^T.
//
// Same arithmetic and operand layout as the skinny kernel (qmm4_skinny.hip; replaces the
// reference's qmv_packed and 8-row NAX kernels for decode and small verify batches,
// src/mlx_tree_spec/qmm_packed.py:151-220, 428-557), with a decomposition for the case where the
// output columns alone fill the GPU: workgroup p (one per CU, 8 waves) owns the R consecutive
// weight rows [p R, p R + R) over the whole of K, so workgroups share nothing and no partial sums
// leave a CU.
//
//  * Work units: the RB = ceil(R / 16) row blocks x SU = K / (128 V) steps of V super-steps (128 k)
//    each; unit u = b * SU + st. Waves take units from a counter in LDS as they free up, with
//    PF = 2 units in flight per wave (a register ring), so a wave the SIMD arbiter favours simply
//    does more units and every wave of a SIMD keeps working until the units run out. (A fixed split
//    leaves the youngest wave of each SIMD running alone for the last fifth of the stream.) A
//    wave's issue priority also falls with the units it has done, so that the oldest wave does
//    not take the units while the youngest sits on the two in its ring. V = 4 where K allows
//    (a unit then covers whole 128-byte lines of each row), else 5.
//  * Loads: lane (n = lane % 16, g = lane / 16) holds weight row 16 b + n of the unit's block; it
//    loads V 16-byte pieces of that row, piece v at byte 64 v + 16 g of the unit's V * 64-byte run,
//    so each row is read as one contiguous run per unit. Rows past the workgroup's range read as
//    zero (an offset outside the buffer resource), as do fetches past the last unit (a zero-length
//    resource).
//  * x (M <= MP rows, MP = 4, 8 or 16, whole K or the workgroup's K slice) is staged once in LDS in
//    A-fragment order. Every wave issues its x loads before any wave issues a weight fetch (a bare
//    barrier between the two), and the stores wait for the x loads alone (the vector memory
//    counter is in order).
//  * Dequantization: dequant_word_fast, or dequant_word for a unit in which one of the wave's
//    rows has a scale outside the fast form's range (a wave-uniform branch per unit).
//  * Each unit's fp32 sums (MFMA 16x16x32, bf16 inputs; output row 4 g + r in lane group g) go to
//    their own LDS slot, the MP / 4 lane groups g < MP / 4 of 16 lanes x 16 bytes. After one
//    barrier the workgroup adds the slots of each block in step order (deterministic whatever
//    wave ran which unit) and writes bf16 y.
//  * Small problems (every unit fits the waves' rings at once, all of x fits LDS): the SMALL form
//    fetches every unit at the start, loads x straight into LDS behind those fetches, and keeps
//    each wave's two unit sums in registers until x is dead; the slots then take the x area.
//  * Whole K over a large N whose slots do not fit (vocabulary heads): PAIR takes units in groups
//    of consecutive steps of one block, one slot per group (pairs at 1-4 rows, groups of 5 at 5-8);
//    OWN (9-16 rows, x alone filling up to all of LDS) gives wave w blocks w, w + 8, ... whole,
//    their sums kept in registers and stored to y as each block's last step is done.
//  * Fused gate+up (FUSED): w is [w_gate; w_up] (N rows, up rows from N / 2), y is [M, N / 2] =
//    silu(x @ w_gate^T) * (x @ w_up^T). Workgroup p owns output columns [p R, p R + R); its 2R
//    weight rows are listed gate rows first, then the up rows of the same columns (N / 2 further),
//    and cut into 16-row blocks (one block may hold both). Each column's gate and up sums are
//    formed exactly as above, rounded to bf16 (the values the unfused projection would store), and
//    combined by silu_mul_bf16.
#include <algorithm>
#include <type_traits>

#include "qmm4_common.h"
#include "qmm4_kernels.h"

namespace qmm4 {

namespace {

// Two waves per SIMD: with 16 (four per SIMD) every CU kept twice the units in flight, and the
// memory system served the decode shapes more slowly (A/B, interleaved rounds, identical bits:
// c1 at M = 1 / 2 / 4 26.40 / 26.62 / 27.10 -> 25.96 / 25.96 / 27.16 us, 5120 -> 17408 / 10240 /
// 12288 / 6144 / 1024 at 1-4 rows 5-9% faster, 9-16 rows over 17408 and 34816 2.5% faster; 16
// rows over the 248320-column head 1.5% slower).
constexpr int kRsWaves = 8;
constexpr int kRsThreads = 64 * kRsWaves;
// MP: x rows held per A fragment (4, 8 or 16; M <= MP). The MFMA's 16 rows are x rows
// min(row, M - 1); output rows 4 g + r lie in lane group g, so a unit's sums live in the MP / 4
// lane groups g < MP / 4.
constexpr int kRsPF = 2;  // units in flight per wave
constexpr int kRsXB = 4;  // x pieces per thread per staging batch
// SMALL plans: each wave holds at most kRsPF units for the whole launch, and all of x (at most
// kRsSmallXP 16-byte pieces per thread, 80 KB) is loaded global -> LDS directly; OWN plans hold
// at most as much x. (Allowing the whole LDS at 8 waves sent 9-16 rows over 65552-99984 columns
// to OWN instead of the row-phase kernel, 3.5-4% slower; 5-8 rows over a small N run the SMALL
// form 7% faster than with 16 waves either way.)
constexpr int kRsSmallXP = 10;
constexpr size_t kRsLds = 160 * 1024;
// NORM: each row of x is normalised by one group of 256 threads, 16-byte chunks t, t + 256, ... of
// the row per thread, at most kRsNormChunks each (K <= 8192); the workgroup's threads take the MP
// rows kRsNormRows at a time (the add_rms_norm kernel's thread layout and summation order).
constexpr int kRsNormThreads = 256;
constexpr int kRsNormChunks = 4;
constexpr int kRsNormRows = kRsThreads / kRsNormThreads;

struct RowSplitParams {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int M, N, K;
  int Nout;  // output columns: N, or N / 2 for the fused gate+up
  int R;     // output columns per workgroup (a multiple of 4)
  int RB;    // 16-row blocks per workgroup: ceil(R / 16), or ceil(2R / 16) for the fused gate+up
  int SU;    // units per block, Kp / (128 V)
  int KS;    // K slices per column range (1: each workgroup all of K)
  int Kp;    // K per slice
  int GU;    // PAIR: units per slot group (a divisor of SU, at least 2)
  float* part;    // KS > 1: fp32 row sums [workgroup][row] (f32x4 over the rows of x)
  uint32_t* cnt;  // KS > 1: arrivals per column range (0 between launches)
  // NORM: x is the residual stream's x, normalised while staged (see the kernel), with
  const uint16_t* r;   // the residual rows, bf16 [M, K]
  const uint16_t* nw;  // the norm weight, bf16 [K]
  uint16_t* h_out;     // h = bf16(x + r), bf16 [M, K] (written by workgroup 0)
  uint16_t* n_out;     // n = rmsnorm(h) * nw, bf16 [M, K] (written by workgroup 0)
  float eps;
};

constexpr int kCoherent = 16;  // buffer access flag: bypass non-coherent caches (cross-CU partials)

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

// Dynamic LDS: x pieces [S][16][MP] (A-fragment order), unit slots [U][MP / 4][16] f32x4, a spare
// 16-byte slot (the target of surplus x pieces, so that every x store is unconditional), the counter.
__host__ __device__ inline size_t rowsplit_xs_bytes(int K, int MP) { return (size_t)(K >> 7) * 16 * MP * 16; }
__host__ __device__ inline size_t rowsplit_part_bytes(int units, int MP) { return (size_t)units * (MP / 4) * 16 * 16; }

// LDS offset of the NORM row sums (4 floats per row group): past x and, unless SMALL, past the
// unit slots, the spare slot and the counter.
__host__ __device__ inline size_t rowsplit_red_offset(int Kp, int MP, int units, bool small) {
  return rowsplit_xs_bytes(Kp, MP) + (small ? 0 : rowsplit_part_bytes(units, MP) + 32);
}

// KSPLIT: K in P.KS slices (false: whole K, the slice arithmetic and the merge compiled out).
// SMALL: a problem whose units all fit the waves' rings at once (U <= 32): wave w computes units
// w and w + 16, both fetched at the start, then x goes straight into LDS; the sums stay in
// registers until every wave is past its last x read and then take the unit slots over the x
// area. Every load of such a launch is in flight from the start, which is what bounds small
// problems (decode and small verify batches over a small N, e.g. 1-8 x 5120 x 5120).
// NORM (up to 4 rows, K <= 8192): the residual add + RMS norm in front of the projection is folded
// into the x staging, so that x = rmsnorm(x + r) * nw never leaves the CU. Thread group m (256
// threads) of every workgroup forms row m of h = bf16(x + r) and its sum of squares over all of K
// exactly as the norm kernel does (norm_add_chunk over the same chunks per thread, the butterfly,
// then the 4 waves in order), so the staged rows are the bits that kernel would store for n, and y
// is the bits of the unfused pair. Each workgroup reads all of x and r (from L2 after the first),
// stages its K slice of n, and workgroup 0 writes h and n.
// PAIR: 0, or units taken in groups: 1 for pairs, 2 for groups of P.GU > 2.
template <int MP, int V, bool FUSED, bool KSPLIT, bool SMALL, bool NORM, int PAIR = 0, bool OWN = false>
__global__ __launch_bounds__(kRsThreads) __attribute__((amdgpu_waves_per_eu(kRsWaves / 4)))
void rowsplit_kernel(RowSplitParams P) {
  static_assert(MP == 4 || MP == 8 || MP == 16, "x rows per fragment");
  static_assert(!SMALL || (!FUSED && !KSPLIT && !NORM), "small plans are plain whole-K projections of 6+ rows");
  static_assert(!PAIR || (!FUSED && !KSPLIT && !SMALL && !NORM), "paired units are plain whole-K projections");
  static_assert(!OWN || (!FUSED && !KSPLIT && !SMALL && !NORM && !PAIR && V == 4), "own blocks: plain whole-K projections");
  static_assert(!NORM || (MP == 4 && MP % kRsNormRows == 0), "thread groups of 256 per normalised row");
  constexpr int G = MP / 4;  // lane groups holding output rows
  typedef f32x4 RowSums[G];  // the sums of one output column over x rows 4 g + r
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int S = P.Kp >> 7;  // super-steps per row in this workgroup's K slice
  const int SU = P.SU;
  const int U = P.RB * SU;
  // PAIR: a wave takes units in groups of GU consecutive steps of one block (GU divides SU) and
  // leaves each group's sum in one slot, so a block has SU / GU slots.
  const int SS = PAIR ? SU / P.GU : SU;
  u32x4* xs = reinterpret_cast<u32x4*>(lds);
  // SMALL: the slots take over the x area once x is dead.
  f32x4* part = reinterpret_cast<f32x4*>(lds + (SMALL ? 0 : rowsplit_xs_bytes(P.Kp, MP)));
  u32x4* spare = reinterpret_cast<u32x4*>(lds + rowsplit_xs_bytes(P.Kp, MP) + rowsplit_part_bytes(P.RB * SS, MP));
  int* next = reinterpret_cast<int*>(spare + 1);

  const int tid = threadIdx.x;
  // The wave index is uniform across the wave; readfirstlane tells the compiler so (unit indices
  // then live in scalar registers and buffer resources need no per-lane loop).
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  // Column range and K slice of this workgroup.
  const int range = KSPLIT ? blockIdx.x / P.KS : blockIdx.x;
  const int kq = KSPLIT ? (blockIdx.x - range * P.KS) * P.Kp : 0;
  const int r0 = range * P.R;
  const int r1 = min(P.Nout, r0 + P.R);
  const int KG = P.K >> 6;

  // x pieces: item i = sq * M + m is the 16-byte piece sq (k = 8 sq .. 8 sq + 7) of row m, stored
  // at LDS position sq * MP + m. All batches but the last are staged before any weight fetch;
  // the last batch is loaded before the first fetches and stored after them. Loads past the last
  // item go to an offset outside the buffer resource (zeros, no memory access); the stores are
  // unconditional (surplus pieces go to the spare slot): a store under a branch would let the
  // compiler move its load there, behind the fetches, and wait for all of them.
  const int xitems = S * 16 * P.M;
  const int nxb = (xitems + kRsThreads * kRsXB - 1) / (kRsThreads * kRsXB);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.x), 0, rsrc_bytes((unsigned long long)P.M * P.K * 2), kBufferRsrcWord3);
  u32x4 xr[kRsXB];
  auto load_x = [&](int batch) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kRsXB; ++j) {
      const int i = tid + (batch * kRsXB + j) * kRsThreads;
      const int sq = i / P.M, m = i - sq * P.M;
      const uint32_t off =
          i < xitems ? ((uint32_t)m * (uint32_t)P.K + (uint32_t)kq + (uint32_t)sq * 8u) * 2u : 0x80000000u;
      xr[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
    }
  };
  auto store_x = [&](int batch) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kRsXB; ++j) {
      const int i = tid + (batch * kRsXB + j) * kRsThreads;
      const int sq = i / P.M, m = i - sq * P.M;
      u32x4* dst = i < xitems ? xs + (sq * MP + m) : spare;
      *dst = xr[j];
    }
  };
  // SMALL: x straight into LDS (buffer loads with the LDS bit): LDS slot q = sq * MP + m holds
  // piece sq of row m, rows m >= M read as zero. A wave's instruction fills 64 consecutive slots
  // (the instruction's base + 16 lane); the slot count S * 16 * MP is a multiple of 64, so a wave
  // either fills whole slots or skips the instruction.
  typedef __attribute__((address_space(3))) void* lds_ptr;
  auto dma_x_all = [&]() __attribute__((always_inline)) {
    const int slots = S * 16 * MP;
#pragma unroll
    for (int j = 0; j < kRsSmallXP; ++j) {
      const int base = j * kRsThreads + 64 * wave;
      if (base < slots) {
        const int q = base + lane;
        const int sq = q / MP, m = q - sq * MP;
        const uint32_t off = m < P.M ? ((uint32_t)m * (uint32_t)P.K + (uint32_t)sq * 8u) * 2u : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(lds + (size_t)base * 16), 16, off, 0, 0, 0);
      }
    }
  };
  if constexpr (!SMALL && !NORM && !OWN) {
    for (int bt = 0; bt + 1 < nxb; ++bt) {
      load_x(bt);
      store_x(bt);
    }
    load_x(nxb - 1);
  }
  // NORM: in pass q, row q * kRsNormRows + tid / 256 of x and r, and the norm weight, for chunks
  // c = tn + 256 i (rows >= M and chunks past the row read as zero).
  constexpr int kNP = NORM ? MP / kRsNormRows : 1;  // row passes
  const int grp0 = tid / kRsNormThreads, tn = tid - grp0 * kRsNormThreads;
  u32x4 nx[kNP][kRsNormChunks], nr[kNP][kRsNormChunks], nwt[kRsNormChunks];
  if constexpr (NORM) {
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.r), 0, rsrc_bytes((unsigned long long)P.M * P.K * 2), kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.nw), 0, rsrc_bytes((unsigned long long)P.K * 2), kBufferRsrcWord3);
#pragma unroll
    for (int q = 0; q < kNP; ++q) {
      const int grp = q * kRsNormRows + grp0;
#pragma unroll
      for (int i = 0; i < kRsNormChunks; ++i) {
        const int c = tn + i * kRsNormThreads;
        const bool live = grp < P.M && c < (P.K >> 3);
        const uint32_t off = live ? ((uint32_t)grp * (uint32_t)P.K + (uint32_t)c * 8u) * 2u : 0x80000000u;
        nx[q][i] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
        nr[q][i] = __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < kRsNormChunks; ++i) {
      const int c = tn + i * kRsNormThreads;
      nwt[i] = __builtin_amdgcn_raw_buffer_load_b128(rn, c < (P.K >> 3) ? (uint32_t)c * 16u : 0x80000000u, 0, 0);
    }
  }
  // Every wave's x loads enter the CU's memory pipeline before any weight fetch: the pipeline
  // returns data in order, so an x load queued behind other waves' fetches would wait for them.
  // (A bare s_barrier: no fence, so no wait for the loads themselves.)
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  const int wrec = rsrc_bytes((unsigned long long)P.N * (P.K >> 1));
  const int srec = rsrc_bytes((unsigned long long)P.N * KG * 2);
  // Offset of a row outside the workgroup's range: past the end of every buffer (they are kept
  // below 1 GiB for this kernel), so its loads return zero.
  constexpr uint32_t kOut = 0x40000000u;

  u32x4 wv[kRsPF][V];
  Scales<V> sv[kRsPF], bv[kRsPF];
  auto fetch = [&](int j, int u) __attribute__((always_inline)) {
    const bool live = u < U;
    const int uu = live ? u : 0;
    const int b = uu / SU, st = uu - b * SU;
    // Output column of this lane's row, and the weight row (the up half sits N / 2 further).
    const int lrow = b * 16 + n;
    const bool up = FUSED && lrow >= P.R;
    const int col = r0 + (up ? lrow - P.R : lrow);
    const int row = col + (up ? P.Nout : 0);
    const uint32_t wo = col < r1 ? (uint32_t)row * (uint32_t)(P.K >> 1) + (uint32_t)g * 16u : kOut;
    const uint32_t so = col < r1 ? (uint32_t)row * (uint32_t)KG * 2u : kOut;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(P.w), 0, live ? wrec : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.s), 0, live ? srec : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(P.b), 0, live ? srec : 0, kBufferRsrcWord3);
    // The unit's byte offsets within the row: its K slice (kq / 2 code bytes, kq / 32 scale
    // bytes) plus its step.
#pragma unroll
    for (int v = 0; v < V; ++v)
      wv[j][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, wo + v * 64, (kq >> 1) + st * V * 64, 0);
    sv[j] = load_scales<V>(rs, so, (kq >> 5) + st * 4 * V);
    bv[j] = load_scales<V>(rb, so, (kq >> 5) + st * 4 * V);
  };
  // The ring holds units in the order they were taken, so the first unit past the end ends it.
  // Whole K: the ring's first fetches go out behind the x loads, before their stores. K slices
  // (few units per workgroup): the x stores first, then the fetches (measured: the decode down
  // projection M = 1 over 5120 x 17408 21.4 -> 20.1 us; with whole K, 27.4 -> 28.4 us the other way).
  // OWN: wave w takes the SU steps of blocks w, w + 16, ... in turn; q counts its units.
  const int own_nq = OWN && wave < P.RB ? (P.RB - wave + kRsWaves - 1) / kRsWaves * SU : 0;
  auto own_unit = [&](int q) { return q < own_nq ? (wave + kRsWaves * (q / SU)) * SU + q % SU : U; };
  int ua = PAIR ? P.GU * wave : wave, ub = PAIR ? P.GU * wave + 1 : wave + kRsWaves;
  if constexpr (OWN) {
    ua = own_unit(0);
    ub = own_unit(1);
  }
  // Units (groups) handed out by the LDS counter after the ring's first fill.
  constexpr int kFirst = PAIR ? kRsWaves : kRsPF * kRsWaves;
  if constexpr (!KSPLIT) {
    fetch(0, ua);
    fetch(1, ub);
    __builtin_amdgcn_sched_barrier(0);
  }

  if constexpr (NORM) {
    // h and the row's sum of squares, then the row sums of its group's 4 waves in wave order
    // (row grp's waves write red[4 grp .. 4 grp + 3]).
    float* red = reinterpret_cast<float*>(lds + rowsplit_red_offset(P.Kp, MP, U, SMALL));
#pragma unroll
    for (int q = 0; q < kNP; ++q) {
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < kRsNormChunks; ++i) nx[q][i] = norm_add_chunk(nx[q][i], nr[q][i], ss);
      ss = norm_wave_sum(ss);
      if (lane == 0) red[q * kRsWaves + wave] = ss;
    }
    __syncthreads();
    // n into the x stage (this workgroup's K slice: pieces kq / 8 .. kq / 8 + S * 16 - 1), and h, n
    // to memory from workgroup 0.
    const bool first = blockIdx.x == 0;
#pragma unroll
    for (int q = 0; q < kNP; ++q) {
      const int grp = q * kRsNormRows + grp0;
      float total = 0.0f;
#pragma unroll
      for (int i = 0; i < kRsNormThreads / 64; ++i) total += red[grp * (kRsNormThreads / 64) + i];
      const float inv = norm_inv(total, P.K, P.eps);
#pragma unroll
      for (int i = 0; i < kRsNormChunks; ++i) {
        const int c = tn + i * kRsNormThreads;
        if (grp < P.M && c < (P.K >> 3)) {
          const u32x4 nv = norm_scale_chunk(nx[q][i], nwt[i], inv);
          const int sq = c - (kq >> 3);
          if (sq >= 0 && sq < S * 16) xs[sq * MP + grp] = nv;
          if (first) {
            const size_t o = (size_t)grp * P.K + (size_t)c * 8;
            *reinterpret_cast<u32x4*>(P.h_out + o) = nx[q][i];
            *reinterpret_cast<u32x4*>(P.n_out + o) = nv;
          }
        }
      }
    }
    if constexpr (!SMALL) {
      if (tid == 0) *next = kFirst;
    }
  } else if constexpr (SMALL || OWN) {
    // The weights (from HBM, the longest latency) went out first; x follows from L2. Every wave
    // waits for all of its loads, then the barrier publishes x.
    dma_x_all();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    store_x(nxb - 1);
    if (tid == 0) *next = kFirst;
  }
  __syncthreads();
  if constexpr (KSPLIT) {
    fetch(0, ua);
    fetch(1, ub);
    __builtin_amdgcn_sched_barrier(0);
  }

  const int aoff = g * 4 * MP + min(n, P.M - 1);
  int ndone = 0;
  __builtin_amdgcn_s_setprio(3);

  auto compute = [&](int j, int st, auto fast, f32x4 acc) __attribute__((always_inline)) {
    constexpr bool FAST = decltype(fast)::value;
    const u32x4* xb = xs + (size_t)st * V * 16 * MP;
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
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xb[(v * 16 + tt) * MP + aoff]), as_bf16x8(B), acc,
                                                      0, 0, 0);
      }
    }
    return acc;
  };

  // One unit from ring slot J: take the next unit index (its LDS round trip overlaps the MFMAs),
  // compute, leave the sums in the unit's slot, refill the slot.
  auto unit = [&](int& u, auto jc) __attribute__((always_inline)) {
    constexpr int j = decltype(jc)::value;
    int taken = 0;
    if (lane == 0) taken = __hip_atomic_fetch_add(next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int nu = __builtin_amdgcn_readfirstlane(taken);
    const int b = u / SU, st = u - b * SU;
    bool bad = false;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e2 = 2 * v + (g >> 1);
      bad |= !fast_scale_ok((sv[j].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
    }
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc;
    if (__builtin_amdgcn_ballot_w64(bad) == 0)
      acc = compute(j, st, std::true_type{}, zero);
    else
      acc = compute(j, st, std::false_type{}, zero);
    if (g < G) part[(u * G + g) * 16 + n] = acc;
    ++ndone;
    // A wave's issue priority falls with the units it has done: the SIMD arbiter otherwise
    // favours the oldest wave, which then takes most units while the youngest holds its ring's
    // two units to the end and finishes them alone.
    if (ndone == 1) __builtin_amdgcn_s_setprio(2);
    else if (ndone == 2) __builtin_amdgcn_s_setprio(1);
    else if (ndone == 3) __builtin_amdgcn_s_setprio(0);
    u = nu;
    fetch(j, u);
  };

  if constexpr (SMALL) {
    // Units w and w + 16 (both in the ring since the start), sums kept until x is dead.
    auto unit_sums = [&](int u, auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      const int st = u - (u / SU) * SU;
      bool bad = false;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int e2 = 2 * v + (g >> 1);
        bad |= !fast_scale_ok((sv[j].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
      }
      const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
      if (__builtin_amdgcn_ballot_w64(bad) == 0) return compute(j, st, std::true_type{}, zero);
      return compute(j, st, std::false_type{}, zero);
    };
    f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
    if (ua < U) acc0 = unit_sums(ua, std::integral_constant<int, 0>{});
    if (ub < U) acc1 = unit_sums(ub, std::integral_constant<int, 1>{});
    __syncthreads();
    if (g < G) {
      if (ua < U) part[(ua * G + g) * 16 + n] = acc0;
      if (ub < U) part[(ub * G + g) * 16 + n] = acc1;
    }
  } else if constexpr (OWN) {
    // Unit q from slot q % 2 into the sums of its block, the slot refilled with unit q + 2; after
    // a block's last step its 16 columns go straight to y (lane (n, g) holds rows 4 g .. 4 g + 3 of
    // column n), so nothing but x uses LDS and no barrier follows the first.
    const __amdgpu_buffer_rsrc_t ryo = __builtin_amdgcn_make_buffer_rsrc(
        P.y, 0, rsrc_bytes((unsigned long long)P.M * P.Nout * 2), kBufferRsrcWord3);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    auto step = [&](int q, int& u, auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      const int b = u / SU, st = u - b * SU;
      bool bad = false;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int e2 = 2 * v + (g >> 1);
        bad |= !fast_scale_ok((sv[j].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
      }
      if (__builtin_amdgcn_ballot_w64(bad) == 0)
        acc = compute(j, st, std::true_type{}, acc);
      else
        acc = compute(j, st, std::false_type{}, acc);
      u = own_unit(q + 2);
      fetch(j, u);
      if (st == SU - 1) {
        const int col = r0 + b * 16 + n;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 4 * g + r;
          if (m < P.M && col < r1)
            __builtin_amdgcn_raw_buffer_store_b16((uint16_t)bf16_rne(acc[r]), ryo,
                                                  (uint32_t)(m * P.Nout + col) * 2u, 0, 0);
        }
        acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // Issue priority falls with the blocks done (as with units taken from the counter).
        ++ndone;
        if (ndone == 1) __builtin_amdgcn_s_setprio(2);
        else if (ndone == 2) __builtin_amdgcn_s_setprio(1);
        else if (ndone == 3) __builtin_amdgcn_s_setprio(0);
      }
    };
    int q = 0;
    for (; q + 1 < own_nq; q += 2) {
      step(q, ua, std::integral_constant<int, 0>{});
      step(q + 1, ub, std::integral_constant<int, 1>{});
    }
    if (q < own_nq) step(q, ua, std::integral_constant<int, 0>{});
    return;
  } else if constexpr (PAIR) {
    // The wave's units in sequence alternate between the ring's slots; the unit after a group's
    // last is the first of the next group taken from the counter. After computing a slot's unit
    // into the group's sums, the slot is refilled with the unit two ahead; a group's sums go to
    // its slot after its last unit.
    const int GU = P.GU;
    auto one = [&](int u, auto jc, f32x4 acc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      const int st = u - (u / SU) * SU;
      bool bad = false;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int e2 = 2 * v + (g >> 1);
        bad |= !fast_scale_ok((sv[j].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
      }
      if (__builtin_amdgcn_ballot_w64(bad) == 0) return compute(j, st, std::true_type{}, acc);
      return compute(j, st, std::false_type{}, acc);
    };
    // (A group taken one group ahead, to hide the atomic's round trip, made pairs 9% slower.)
    auto succ = [&](int u) __attribute__((always_inline)) {
      if ((u + 1) % GU != 0) return u + 1;
      int taken = 0;
      if (lane == 0) taken = __hip_atomic_fetch_add(next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      return __builtin_amdgcn_readfirstlane(taken) * GU;
    };
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // Slot J's unit u is computed, then u becomes the unit after `other` (the next in sequence).
    auto step = [&](int& u, int other, auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      acc = one(u, jc, acc);
      if ((u + 1) % GU == 0) {
        if (g < G) part[((u / GU) * G + g) * 16 + n] = acc;
        acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        ++ndone;
        if (ndone == 1) __builtin_amdgcn_s_setprio(2);
        else if (ndone == 2) __builtin_amdgcn_s_setprio(1);
        else if (ndone == 3) __builtin_amdgcn_s_setprio(0);
      }
      u = succ(other);
      fetch(j, u);
    };
    if constexpr (PAIR == 1) {
      // Pairs: the next pair is taken before this one's MFMAs, its half 0 fetched into slot 0 as
      // soon as this pair's half 0 is done (measured 3% faster than the general walk below).
      while (ua < U) {
        int taken = 0;
        if (lane == 0) taken = __hip_atomic_fetch_add(next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int np = __builtin_amdgcn_readfirstlane(taken);
        acc = one(ua, std::integral_constant<int, 0>{}, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        fetch(0, 2 * np);
        acc = one(ub, std::integral_constant<int, 1>{}, acc);
        if (g < G) part[((ua >> 1) * G + g) * 16 + n] = acc;
        ++ndone;
        if (ndone == 1) __builtin_amdgcn_s_setprio(2);
        else if (ndone == 2) __builtin_amdgcn_s_setprio(1);
        else if (ndone == 3) __builtin_amdgcn_s_setprio(0);
        fetch(1, 2 * np + 1);
        ua = 2 * np;
        ub = ua + 1;
      }
    } else {
      while (ua < U) {
        step(ua, ub, std::integral_constant<int, 0>{});
        if (ub >= U) break;
        step(ub, ua, std::integral_constant<int, 1>{});
      }
    }
  } else {
    for (;;) {
      if (ua >= U) break;
      unit(ua, std::integral_constant<int, 0>{});
      if (ub >= U) break;
      unit(ub, std::integral_constant<int, 1>{});
    }
  }
  __syncthreads();

  // y[m, col] = sum over the block's steps, in step order, of its unit slots; element r of a slot's
  // lane group g is x row 4 g + r. Fused: the same for the column's gate and up blocks, then
  // silu * up.
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      P.y, 0, rsrc_bytes((unsigned long long)P.M * P.Nout * 2), kBufferRsrcWord3);
  auto row_sum = [&](int lrow, RowSums& sum) __attribute__((always_inline)) {
    const int b = lrow >> 4, nn = lrow & 15;
#pragma unroll
    for (int gg = 0; gg < G; ++gg) sum[gg] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int st = 0; st < SS; ++st) {
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        const f32x4 c = part[((b * SS + st) * G + gg) * 16 + nn];
        sum[gg][0] += c[0]; sum[gg][1] += c[1]; sum[gg][2] += c[2]; sum[gg][3] += c[3];
      }
    }
  };
  auto write = [&](int col, const RowSums& sum, const RowSums& sup) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < MP; ++m)
      if (m < P.M) {
        const float v = sum[m >> 2][m & 3];
        const uint32_t o = FUSED ? silu_mul_bf16(bf16_rne(v), bf16_rne(sup[m >> 2][m & 3])) : bf16_rne(v);
        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)o, ry, (uint32_t)(m * P.Nout + col) * 2u, 0, 0);
      }
  };
  if constexpr (!KSPLIT) {
    for (int c = tid; c < P.R; c += kRsThreads) {
      const int col = r0 + c;
      if (col >= r1) continue;
      RowSums sum, sup;
      row_sum(c, sum);
      if (FUSED) row_sum(P.R + c, sup);
      write(col, sum, sup);
    }
    return;
  }

  // K slices: store this workgroup's fp32 row sums, count in, and let the last workgroup of the
  // column range add the slices in slice order (the same bits whichever arrives last).
  const int RR = FUSED ? 2 * P.R : P.R;
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      P.part, 0, rsrc_bytes((unsigned long long)gridDim.x * RR * G * 16), kBufferRsrcWord3);
  for (int lrow = tid; lrow < RR; lrow += kRsThreads) {
    RowSums sum;
    row_sum(lrow, sum);
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum[gg]), rp,
                                             (((uint32_t)blockIdx.x * RR + lrow) * G + gg) * 16u, 0, kCoherent);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&P.cnt[range], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *next = prev == (uint32_t)(P.KS - 1) ? 1 : 0;
  }
  __syncthreads();
  if (*next == 0) return;
  auto slice_sum = [&](int lrow, RowSums& sum) __attribute__((always_inline)) {
#pragma unroll
    for (int gg = 0; gg < G; ++gg) sum[gg] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int qq = 0; qq < P.KS; ++qq) {
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        const f32x4 c = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, (((uint32_t)(range * P.KS + qq) * RR + lrow) * G + gg) * 16u,
                                                         0, kCoherent));
        sum[gg][0] += c[0]; sum[gg][1] += c[1]; sum[gg][2] += c[2]; sum[gg][3] += c[3];
      }
    }
  };
  for (int c = tid; c < P.R; c += kRsThreads) {
    const int col = r0 + c;
    if (col >= r1) continue;
    RowSums sum, sup;
    slice_sum(c, sum);
    if (FUSED) slice_sum(P.R + c, sup);
    write(col, sum, sup);
  }
  if (tid == 0) __hip_atomic_store(&P.cnt[range], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Up to 16 rows of x over a small problem, whole K per workgroup, x never staged: workgroup p owns
// the R <= 32 rows [p R, p R + R) (RB <= 2 blocks of 16) and has one wave per K chunk of 512 k
// (at most 12: K <= 6144, three waves per SIMD, 170 registers each). Wave w computes chunk w for
// every block: it loads the chunk's A fragments of x (16 rows x 512 k,
// lane (m, g) holds x[min(m, M - 1)] at the MFMA's k) straight into registers, the chunk's weights,
// scales and biases of both blocks, and runs the chunk's MFMAs with each A fragment feeding both
// blocks. Every load of the workgroup is issued at the start and nothing waits for a barrier
// before the first MFMA; the chunk sums meet in LDS (one slot per chunk and block) and are added
// in chunk order (deterministic). One memory round trip plus the L2 reads of x bound such a
// launch (a verify tile of 16 x 5120 over 5120 columns: 160 KB of x per CU from L2, 57 KB of
// weights from HBM).
constexpr int kXrV = 4;        // super-steps per chunk (512 k)
constexpr int kXrMaxRB = 2;    // blocks per workgroup
constexpr int kXrMaxWaves = 12;
template <int NCH>
__global__ __launch_bounds__(64 * kXrMaxWaves) __attribute__((amdgpu_waves_per_eu(3)))
void rowsplit_xreg_kernel(RowSplitParams P) {
  constexpr int V = kXrV;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  f32x4* part = reinterpret_cast<f32x4*>(lds);  // [chunk][block][4 groups][16 lanes]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int SU = P.SU;  // chunks along K
  const int RB = P.RB;
  const int r0 = blockIdx.x * P.R;
  const int r1 = min(P.N, r0 + P.R);
  const int KG = P.K >> 6;
  constexpr uint32_t kOut = 0x40000000u;  // past the end of every buffer (each below 1 GiB)
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.x), 0, rsrc_bytes((unsigned long long)P.M * P.K * 2), kBufferRsrcWord3);
  const int wrec = rsrc_bytes((unsigned long long)P.N * (P.K >> 1));
  const int srec = rsrc_bytes((unsigned long long)P.N * KG * 2);
  const uint32_t xrow = (uint32_t)min(n, P.M - 1) * (uint32_t)P.K * 2u;

  u32x4 xa[NCH][V][4];
  u32x4 wv[NCH][kXrMaxRB][V];
  Scales<V> sv[NCH][kXrMaxRB], bv[NCH][kXrMaxRB];
  // Issue every load of this wave's chunks in two halves of its super-steps, each half's weights
  // (from HBM) before its x (from L2): the first half's MFMAs need only the first half's loads
  // (16 x 5120 -> 5120 14.5 -> 14.3 us, 9 rows 13.1 -> 12.9 us; quarters were no better).
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int st = wave + c * kXrMaxWaves;
      const bool live = st < SU;
      const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(P.w), 0,
                                                                          live ? wrec : 0, kBufferRsrcWord3);
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.s), 0,
                                                                          live ? srec : 0, kBufferRsrcWord3);
      const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.b), 0,
                                                                          live ? srec : 0, kBufferRsrcWord3);
#pragma unroll
      for (int b = 0; b < kXrMaxRB; ++b) {
        const int row = r0 + b * 16 + n;
        const bool ok = b < RB && row < r1;
        const uint32_t wo = ok ? (uint32_t)row * (uint32_t)(P.K >> 1) + (uint32_t)g * 16u : kOut;
        const uint32_t so = ok ? (uint32_t)row * (uint32_t)KG * 2u : kOut;
        if (h == 0) {
          sv[c][b] = load_scales<V>(rs, so, live ? st * 4 * V : 0);
          bv[c][b] = load_scales<V>(rb, so, live ? st * 4 * V : 0);
        }
#pragma unroll
        for (int v = h * V / 2; v < (h + 1) * V / 2; ++v)
          wv[c][b][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, wo + v * 64, live ? st * V * 64 : 0, 0);
      }
#pragma unroll
      for (int v = h * V / 2; v < (h + 1) * V / 2; ++v)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const uint32_t off = live ? xrow + (uint32_t)(st * V * 128 + v * 128 + g * 32 + tt * 8) * 2u : 0x80000000u;
          xa[c][v][tt] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int st = wave + c * kXrMaxWaves;
    if (st >= SU) break;
    f32x4 acc[kXrMaxRB];
#pragma unroll
    for (int b = 0; b < kXrMaxRB; ++b) acc[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bool bad = false;
#pragma unroll
    for (int b = 0; b < kXrMaxRB; ++b)
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int e2 = 2 * v + (g >> 1);
        bad |= !fast_scale_ok((sv[c][b].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
      }
    const bool fast = __builtin_amdgcn_ballot_w64(bad) == 0;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e2 = 2 * v + (g >> 1);
      float c1[kXrMaxRB], c2[kXrMaxRB], bf[kXrMaxRB];
#pragma unroll
      for (int b = 0; b < kXrMaxRB; ++b) {
        const float sf = bf16_to_f32((sv[c][b].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
        bf[b] = bf16_to_f32((bv[c][b].d[e2 >> 1] >> (16 * (e2 & 1))) & 0xFFFFu);
        c1[b] = fast ? sf * 16777216.0f : sf;
        c2[b] = fast ? sf * 1048576.0f : sf * 0.0625f;
      }
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int b = 0; b < kXrMaxRB; ++b) {
          if (b < RB) {
            const u32x4 B = fast ? dequant_word_fast(wv[c][b][v][tt], c1[b], c2[b], bf[b])
                                 : dequant_word(wv[c][b][v][tt], c1[b], c2[b], bf[b]);
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa[c][v][tt]), as_bf16x8(B), acc[b], 0, 0, 0);
          }
        }
    }
#pragma unroll
    for (int b = 0; b < kXrMaxRB; ++b)
      if (b < RB) part[((st * kXrMaxRB + b) * 4 + g) * 16 + n] = acc[b];
  }
  __syncthreads();

  // y[m, col]: the chunk sums of the column's block in chunk order; output row m = 4 g + r.
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      P.y, 0, rsrc_bytes((unsigned long long)P.M * P.N * 2), kBufferRsrcWord3);
  for (int it = tid; it < P.R * 4; it += (int)blockDim.x) {
    const int c = it >> 2, gg = it & 3;
    const int col = r0 + c;
    if (col >= r1 || 4 * gg >= P.M) continue;
    const int b = c >> 4, nn = c & 15;
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int st = 0; st < SU; ++st) {
      const f32x4 v = part[((st * kXrMaxRB + b) * 4 + gg) * 16 + nn];
      sum[0] += v[0]; sum[1] += v[1]; sum[2] += v[2]; sum[3] += v[3];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * gg + r;
      if (m < P.M)
        __builtin_amdgcn_raw_buffer_store_b16((uint16_t)bf16_rne(sum[r]), ry, (uint32_t)(m * P.N + col) * 2u, 0, 0);
    }
  }
}

}  // namespace

bool rowsplit_xreg_plan(int M, int N, int K, int cus, RowSplitPlan* plan) {
  if (M < 9 || M > 16 || cus < 1 || K % (128 * kXrV) != 0) return false;
  if ((unsigned long long)(N + 256) * (unsigned long long)K / 2 >= (1ULL << 30)) return false;
  const int R = ((N + cus - 1) / cus + 3) / 4 * 4;
  const int RB = (R + 15) / 16;
  const int SU = K / (128 * kXrV);
  if (RB > kXrMaxRB || SU > kXrMaxWaves) return false;
  plan->MP = 16;
  plan->small = true;
  plan->xreg = true;
  plan->pair = false;
  plan->GU = 0;
  plan->own = false;
  plan->V = kXrV;
  plan->fused = false;
  plan->Nout = N;
  plan->R = R;
  plan->RB = RB;
  plan->SU = SU;
  plan->KS = 1;
  plan->Kp = K;
  plan->ranges = (N + R - 1) / R;
  plan->blocks = plan->ranges;
  plan->part_bytes = 0;
  plan->smem = (size_t)SU * kXrMaxRB * 4 * 16 * 16;
  return true;
}

int rowsplit_mp(int M) { return M <= 4 ? 4 : M <= 8 ? 8 : 16; }

bool rowsplit_plan(int M, int N, int K, int cus, bool fused, RowSplitPlan* plan) {
  if (M < 1 || M > 16 || cus < 1) return false;
  if (fused && N % 32 != 0) return false;
  // Row offsets of this kernel stay below 1 GiB.
  if ((unsigned long long)(N + 256) * (unsigned long long)K / 2 >= (1ULL << 30)) return false;
  const int MP = rowsplit_mp(M);
  const int nout = fused ? N / 2 : N;
  // Up to 4 rows: whole K per workgroup when the columns alone give every CU at least 4 row
  // blocks, or when K <= 8192; otherwise K in 2 or 4 slices over as many workgroups per column
  // range, when each workgroup still has at least 3 units per wave. 5 to 16 rows (a verify batch
  // of up to 16 tree nodes): the fewest K slices whose x slice and unit slots fit in LDS (up to 8
  // slices for 8 rows, 4 for 16), starting from 2 for 6 rows or more when x is over a quarter of
  // a workgroup's weight bytes.
  // 6 to 8 rows over at most one row block per CU (N <= 16 x CUs), with all units in the waves'
  // rings at once and all of x in LDS: the SMALL form (every load in flight from the start, no K
  // slices). Against the other forms (A/B, interleaved rounds): 6 / 8 x 5120 -> 1024 10.6 / 10.9 ->
  // 10.1 / 10.7 us, while at 1-5 rows, or with 2-3 blocks per CU, whole K or 2 slices of the
  // regular form were 1-8% faster (e.g. 1 x 5120 -> 10240 15.1 -> 14.2 us, 12 x 5120 -> 10240
  // 18.5 -> 17.0 us).
  if (!fused && K % 512 == 0 && M >= 6 && (nout + cus - 1) / cus <= 16) {
    const int S = K >> 7;
    const int R = ((nout + cus - 1) / cus + 3) / 4 * 4;
    const int RB = (R + 15) / 16;
    const int SU = S / 4;
    const size_t xb = rowsplit_xs_bytes(K, MP);
    const size_t pb = rowsplit_part_bytes(RB * SU, MP);
    if (RB * SU <= kRsPF * kRsWaves && xb <= kRsLds && pb <= kRsLds &&
        (size_t)S * 16 * MP <= (size_t)kRsSmallXP * kRsThreads) {
      plan->MP = MP;
      plan->small = true;
      plan->xreg = false;
      plan->pair = false;
      plan->GU = 0;
      plan->own = false;
      plan->V = 4;
      plan->fused = false;
      plan->Nout = nout;
      plan->R = R;
      plan->RB = RB;
      plan->SU = SU;
      plan->KS = 1;
      plan->Kp = K;
      plan->ranges = (nout + R - 1) / R;
      plan->blocks = plan->ranges;
      plan->part_bytes = 0;
      plan->smem = std::max(xb, pb);
      return true;
    }
  }
  // 9 to 16 rows: at most 4 K slices (x slices of 16 rows are large; with 8 slices, e.g. the
  // 65984-column head, the cross-workgroup merge of the slices costs more than it saves).
  const int max_ks = MP == 8 ? 8 : 4;
  const long long xbytes = (long long)M * K * 2;
  const long long wbytes = (long long)((nout + cus - 1) / cus) * (fused ? 2 : 1) * (K / 2);
  const int ks0 = (M >= 6 && 4 * xbytes > wbytes && K % 256 == 0) ? 2 : 1;
  // A second pass takes whole K for up to 4 rows even with fewer than 4 row blocks per CU, when
  // no K split leaves each workgroup 3 units per wave (measured: 12288 -> 5120 at 1 row, 21.5 us
  // on the stream-K skinny kernel, 17.0 us so).
  for (int pass = 0; pass < 2; ++pass)
  for (int ks = pass == 0 ? ks0 : 1; ks <= (pass == 0 ? max_ks : 1); ks *= 2) {
    if (K % (128 * ks) != 0) continue;
    const int kp = K / ks;
    const int S = kp >> 7;
    // Units of 4 super-steps (256 bytes of a row: two whole 128-byte lines) where K allows: a unit
    // boundary inside a line splits it between two waves' fetches. Units of 5 where K does not
    // allow 4, or where the x slice and the 4-step units' slots do not fit: 9-16 rows over the
    // 34816 x 5120 gate+up then take 2 K slices of 5-step units instead of 4 slices (42.4 -> 35.5 us
    // at 16 rows, 16-19% at 9-16 rows, plain or fused).
    for (int V = 4; V <= 5; ++V) {
      if (S % V != 0) continue;
      const int target = std::max(1, cus / ks);
      const int R = ((nout + target - 1) / target + 3) / 4 * 4;
      const int RB = ((fused ? 2 * R : R) + 15) / 16;
      const int SU = S / V;
      if (MP == 4 && pass == 0 && (ks == 1 ? RB < 4 && K > 8192 : RB * SU < 3 * kRsWaves)) continue;
      size_t smem = rowsplit_xs_bytes(kp, MP) + rowsplit_part_bytes(RB * SU, MP) + 32;
      // Whole K whose unit slots do not fit: units in groups of the fewest steps that fit (one slot
      // per group) before K slices, e.g. pairs over the 248320-column vocabulary head at 1-4 rows
      // (61 blocks x 10 steps per CU) or the 65984-column head at 5-8 rows, groups of 5 over the
      // 248320- and 151936-column heads at 5-8 rows (163.7-172.3 -> 145.9-147.9 us and 108.1 ->
      // 97.8 us against waves owning whole blocks).
      bool pair = false;
      int gu = 0;
      for (int c = 2; c <= SU && smem > 160 * 1024 && ks == 1 && !fused && V == 4; ++c) {
        if (SU % c != 0) continue;
        const size_t ps = rowsplit_xs_bytes(kp, MP) + rowsplit_part_bytes(RB * SU / c, MP) + 32;
        if (ps <= 160 * 1024) {
          smem = ps;
          pair = true;
          gu = c;
        }
      }
      // Neither fits, but all of x does and a CU has at least two blocks per wave: each wave takes
      // whole blocks (all SU steps) and keeps their sums in registers (no slots), e.g. the
      // 248320-column vocabulary head at 5-16 rows (61 blocks per CU).
      bool own = false;
      if (smem > 160 * 1024 && ks == 1 && !fused && V == 4 && RB >= 2 * kRsWaves &&
          (size_t)S * 16 * MP <= (size_t)kRsSmallXP * kRsThreads && rowsplit_xs_bytes(kp, MP) <= kRsLds) {
        smem = rowsplit_xs_bytes(kp, MP);
        own = true;
      }
      if (smem > 160 * 1024) continue;
      const int ranges = (nout + R - 1) / R;
      plan->MP = MP;
      plan->small = false;
      plan->xreg = false;
      plan->pair = pair;
      plan->GU = gu;
      plan->own = own;
      plan->V = V;
      plan->fused = fused;
      plan->Nout = nout;
      plan->R = R;
      plan->RB = RB;
      plan->SU = SU;
      plan->KS = ks;
      plan->Kp = kp;
      plan->ranges = ranges;
      plan->blocks = ranges * ks;
      plan->part_bytes = ks > 1 ? (size_t)plan->blocks * (fused ? 2 * R : R) * (MP / 4) * 16 : 0;
      plan->smem = smem;
      return true;
    }
  }
  return false;
}

// Dynamic LDS of a launch: the plan's, plus the row sums of the normalising staging.
size_t rowsplit_smem(const RowSplitPlan& plan, bool norm) {
  if (!norm) return plan.smem;
  return std::max(plan.smem, rowsplit_red_offset(plan.Kp, plan.MP, plan.RB * plan.SU, plan.small) +
                                 sizeof(float) * plan.MP * (kRsNormThreads / 64));
}

template <int MP, int V, bool FUSED, bool KSPLIT, bool SMALL, bool NORM, int PAIR = 0, bool OWN = false>
hipError_t launch_rowsplit_t(const RowSplitPlan& plan, const RowSplitParams& P, hipStream_t stream) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&rowsplit_kernel<MP, V, FUSED, KSPLIT, SMALL, NORM, PAIR, OWN>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRsLds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((rowsplit_kernel<MP, V, FUSED, KSPLIT, SMALL, NORM, PAIR, OWN>), dim3(plan.blocks),
                     dim3(kRsThreads), rowsplit_smem(plan, NORM), stream, P);
  return hipGetLastError();
}

template <int MP, int V, bool FUSED, bool NORM>
hipError_t launch_rowsplit_k(const RowSplitPlan& plan, const RowSplitParams& P, hipStream_t stream) {
  return plan.KS > 1 ? launch_rowsplit_t<MP, V, FUSED, true, false, NORM>(plan, P, stream)
                     : launch_rowsplit_t<MP, V, FUSED, false, false, NORM>(plan, P, stream);
}

template <int MP, bool NORM>
hipError_t launch_rowsplit_m(const RowSplitPlan& plan, const RowSplitParams& P, hipStream_t stream) {
  if constexpr (NORM) {
    // The normalising staging runs with the regular forms only (rowsplit_norm_ok: 4-row
    // fragments, while the SMALL form starts at 6 rows).
    if (plan.small || plan.pair || plan.own) return hipErrorInvalidValue;
  } else {
    if (plan.small) return launch_rowsplit_t<MP, 4, false, false, true, false>(plan, P, stream);
    if (plan.pair)
      return plan.GU == 2 ? launch_rowsplit_t<MP, 4, false, false, false, false, 1>(plan, P, stream)
                          : launch_rowsplit_t<MP, 4, false, false, false, false, 2>(plan, P, stream);
    if (plan.own) return launch_rowsplit_t<MP, 4, false, false, false, false, 0, true>(plan, P, stream);
  }
  if (plan.fused)
    return plan.V == 5 ? launch_rowsplit_k<MP, 5, true, NORM>(plan, P, stream)
                       : launch_rowsplit_k<MP, 4, true, NORM>(plan, P, stream);
  return plan.V == 5 ? launch_rowsplit_k<MP, 5, false, NORM>(plan, P, stream)
                     : launch_rowsplit_k<MP, 4, false, NORM>(plan, P, stream);
}

hipError_t launch_rowsplit_xreg(const RowSplitPlan& plan, const RowSplitParams& P, hipStream_t stream) {
  hipLaunchKernelGGL((rowsplit_xreg_kernel<1>), dim3(plan.blocks), dim3(64 * plan.SU), plan.smem, stream, P);
  return hipGetLastError();
}

bool rowsplit_norm_ok(const RowSplitPlan& plan, int M, int K) {
  return !plan.xreg && !plan.small && !plan.pair && !plan.own && plan.MP == 4 && M >= 1 && M <= 4 && K % 8 == 0 &&
         K <= kRsNormThreads * kRsNormChunks * 8 && rowsplit_smem(plan, true) <= kRsLds;
}

hipError_t launch_rowsplit(const RowSplitPlan& plan, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                           const uint16_t* b, uint16_t* y, float* part, uint32_t* cnt, int M, int N, int K,
                           hipStream_t stream, const RowSplitNorm* norm) {
  if (M > plan.MP) return hipErrorInvalidValue;
  if (norm && !rowsplit_norm_ok(plan, M, K)) return hipErrorInvalidValue;
  RowSplitParams P;
  P.x = x; P.w = w; P.s = s; P.b = b; P.y = y;
  P.M = M; P.N = N; P.K = K;
  P.Nout = plan.Nout; P.R = plan.R; P.RB = plan.RB; P.SU = plan.SU;
  P.KS = plan.KS; P.Kp = plan.Kp; P.part = part; P.cnt = cnt;
  P.GU = plan.pair ? plan.GU : 1;
  P.r = norm ? norm->r : nullptr;
  P.nw = norm ? norm->weight : nullptr;
  P.h_out = norm ? norm->h : nullptr;
  P.n_out = norm ? norm->n : nullptr;
  P.eps = norm ? norm->eps : 0.0f;
  if (plan.xreg) return launch_rowsplit_xreg(plan, P, stream);
  if (norm) return launch_rowsplit_m<4, true>(plan, P, stream);
  switch (plan.MP) {
    case 4: return launch_rowsplit_m<4, false>(plan, P, stream);
    case 8: return launch_rowsplit_m<8, false>(plan, P, stream);
    case 16: return launch_rowsplit_m<16, false>(plan, P, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qmm4
