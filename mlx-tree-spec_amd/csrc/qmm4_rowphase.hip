// Row-phase quantized matmul for M = 1..64 rows: y = x @ dequant(w)^T.
//
// Serves the verify shapes (the reference's NAX verify tiles and multi-row kernel,
// src/mlx_tree_spec/qmm_packed.py:151-220, 296-394) from MLX's own [N, K/8] layout. The design
// follows from what bounds these shapes on gfx950: the vector memory address unit takes about one
// lane per clock, so every load instruction costs the same whether it carries 1 KB or 64 useful
// bytes. Every global load here moves 16 distinct bytes per lane, and x and the scales are read
// from global memory once per workgroup and phase, not once per wave and step:
//
//  * Workgroup p (8 waves, two per SIMD) owns a range of 16-row weight blocks and a range of
//    phases (PH = 128 V values of k each); the phase ranges of one block range partition K. When
//    N alone fills the GPU every workgroup takes all of K; otherwise K is split, each workgroup
//    stores its fp32 partial tile, and a second kernel adds each range's tiles in workgroup order
//    (deterministic), one item per thread over the whole GPU.
//  * Wave w owns blocks w, w + 8, w + 16, ... of the range (at most BPW) and holds one whole phase
//    of their weights in registers while the next phase's weights are in flight (double buffer).
//    Slots past a wave's blocks compute on zero weights (a straight-line loop), except that the
//    wide plans' variants skip the last slot in the waves that hold no block there.
//    Lane (n = lane % 16, g = lane / 16) loads V 16-byte pieces of row n of each block, piece v at
//    byte 64 v + 16 g of the row's PH / 2-byte run, so each row is read as one contiguous run.
//  * Word t of piece v holds k = PH p + 128 v + 32 g + 8 t: the B operand of MFMA 16x16x32 (v, t)
//    after exact dequantization in registers (dequant_word_fast, bit-identical to
//    bf16_rne(fp32(s) * q + fp32(b)); a phase holding a scale outside its range takes
//    dequant_word). The A operand, lane (m, g), is x[m] at the same 8 k; it is read from LDS once
//    per (v, t) and feeds the MFMAs of all of the wave's blocks.
//  * The next phase's x slice (A-fragment order) and the scales and biases of the range's rows are
//    staged in LDS (double-buffered) by the whole workgroup, behind the weight prefetch; one
//    barrier per phase publishes them.
//  * Nothing waits for a load before it is needed: the phase barrier is a bare s_barrier behind
//    an explicit count (a __syncthreads() fence would wait for the DMA of the phases ahead), the
//    weight refills are issued outside any branch (a load issued in both arms of a branch leaves
//    register copies at the join, and each copy waits for every older load), and the next scale
//    window is loaded into registers one phase before its first use where registers allow.
//  * The result leaves through LDS as 16-byte row chunks of y (or as fp32 partial tiles).
#include <type_traits>

#include "qmm4_common.h"
#include "qmm4_kernels.h"

namespace qmm4 {

namespace {


struct RowPhaseParams {
  const uint16_t* x;
  const uint16_t* s;
  const uint16_t* b;
  const uint32_t* w;
  uint16_t* y;
  float* part;    // [G][items] f32x4 partial tiles (K split only)
  int M, N, K;
  int NB;         // 16-row blocks of w (N / 16)
  int BW;         // blocks per range
  int S;          // workgroups per range (K split)
  int NP;         // phases along K
  int ranges;     // block ranges
  int fused;      // gate+up with the SiLU·mul epilogue (wide plans): w stacks [gate; up], y is [M, N / 2]
};

template <int MB_, int V_, int BPW_, int W_, int STG_ = 3, bool OPT_ = false>
struct RpCfg {
  static constexpr int kRpWaves = W_;  // waves per workgroup
  static constexpr int kRpThreads = 64 * W_;
  static constexpr int MB = MB_;      // 16-row blocks of x (M <= 16 MB)
  static constexpr int MP = 16 * MB;
  static constexpr int V = V_;        // super-steps (128 k) per phase
  static constexpr int PH = 128 * V;  // k per phase
  static constexpr int BPW = BPW_;    // blocks per wave (at most)
  static constexpr int RW = 16 * kRpWaves * BPW;  // rows per range (at most)
  // The last block slot's arithmetic runs only in the waves that hold a BPW-th block (wide plans
  // whose blocks leave some waves one short); otherwise every wave computes every slot.
  static constexpr bool kOptLast = OPT_ && BPW > 1;
  static constexpr bool kFusable = MB_ <= 6;  // the fused gate+up epilogue is built (up to 96 rows)
  static constexpr int kXPieces = V * 16 * MP;    // 16-byte x pieces per phase
  static constexpr int kSB = 4 * V;               // bytes of scales (or biases) per row and phase
  static constexpr int WP = 64 / kSB;             // phases per scale window (64 bytes of each row)
  static constexpr int kWB = WP * kSB;            // window bytes per row and array
  // LDS row stride of a window: 16 bytes of padding put the 16 rows one read touches (one per
  // lane n) in distinct banks (a 64-byte stride would give four rows per bank).
  static constexpr int kWS = kWB + 16;
  static constexpr size_t kXBytes = (size_t)kXPieces * 16;
  static constexpr size_t kWinBytes = (size_t)RW * kWS;  // one array's window
  // x stages: 3 = phase p in use, p + 1 staged, p + 2 being staged; 2 (80-row x, whose three
  // stages would not fit beside the windows) = phase p in use, p + 1 being staged.
  static constexpr int kStages = STG_;
  static constexpr size_t kYBytes = (size_t)MP * RW * 2;   // epilogue: bf16 tile of y
  static constexpr size_t kMain = kStages * kXBytes + 2 * kWinBytes;
  static constexpr size_t kLds = (kMain > kYBytes ? kMain : kYBytes);
  static constexpr int kItems = kRpWaves * BPW * MB * 64;  // f32x4 items of a partial tile
  static constexpr int kXL = (kXPieces + kRpThreads - 1) / kRpThreads;         // x loads per thread and phase
  static constexpr int kWL = (RW * (kWB / 16) + kRpThreads - 1) / kRpThreads;  // window loads per thread and array
  static_assert(V == 2 || V == 4, "phases of 2 or 4 super-steps");
  static_assert(STG_ == 2 || STG_ == 3, "two or three x stages");
};

// Device-coherent 16-byte stores and loads (cache policy sc1: coherent across the XCDs' L2s).
constexpr int kCoherent = 16;

template <class C>
__global__ __launch_bounds__(C::kRpThreads) __attribute__((amdgpu_waves_per_eu(C::kRpWaves / 4)))
void rowphase_kernel(RowPhaseParams P) {
  constexpr int MB = C::MB, MP = C::MP, V = C::V, BPW = C::BPW, RW = C::RW;
  constexpr int kRpWaves = C::kRpWaves, kRpThreads = C::kRpThreads;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ int s_bad[2];  // per window parity: a scale outside the fast range

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  // K split: workgroups that share a K slice of x sit on one XCD where the grid allows (workgroup
  // b runs on XCD b % 8; the XCD-major order q = (b % 8) * (G / 8) + b / 8 walks splits
  // outermost), so the slice is read from HBM into that XCD's L2 once instead of once per range.
  const int G = gridDim.x;
  const int q = (P.S > 1 && (G & 7) == 0) ? (int)((blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3)) : (int)blockIdx.x;
  const int split = P.S > 1 ? q / P.ranges : 0;
  const int range = P.S > 1 ? q - split * P.ranges : q;
  const int p = range * P.S + split;  // the partial tile's slot (range-major: the reduce kernel's order)
  // Fused gate+up: the range holds BW / 2 output blocks, gate blocks hb0 .. hb0 + hb - 1 (local
  // blocks 0 .. hb - 1) and the same blocks of the up half (local hb .. 2 hb - 1).
  // (Built for up to 96 rows: the fused planner takes no more.)
  const bool fused = C::kFusable && P.fused;
  const int NBh = P.NB >> 1;
  const int hb0 = range * (P.BW >> 1);
  const int hb = fused ? min(P.BW >> 1, NBh - hb0) : 0;
  const int b0 = range * P.BW;
  const int nbr = fused ? 2 * hb : min(P.BW, P.NB - b0);  // blocks in this range
  // Weight row of local row lr of the range.
  auto grow = [&](int lr) __attribute__((always_inline)) {
    const int lb = lr >> 4;
    const int gb = !fused ? b0 + lb : lb < hb ? hb0 + lb : NBh + hb0 + (lb - hb);
    return 16 * gb + (lr & 15);
  };
  const int pa = (int)((long long)split * P.NP / P.S);
  const int pb = (int)((long long)(split + 1) * P.NP / P.S);
  const int np = pb - pa;
  const int r0 = b0 * 16;                // first weight row of the range
  const int nrows = nbr * 16;
  // This wave's blocks: wave + W j for j < nbw.
  const int nbw = nbr > wave ? (nbr - wave + kRpWaves - 1) / kRpWaves : 0;
  const int KG = P.K >> 6;

  const int wrec = rsrc_bytes((unsigned long long)P.N * (P.K >> 1));
  const int srec = rsrc_bytes((unsigned long long)P.N * KG * 2);
  const int xrec = rsrc_bytes((unsigned long long)P.M * P.K * 2);
  // Offset past the end of every buffer (they stay below 2 GiB for this kernel): loads read zero.
  constexpr uint32_t kOut = 0x80000000u;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.x), 0, xrec,
                                                                      kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.s), 0, srec,
                                                                      kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.b), 0, srec,
                                                                      kBufferRsrcWord3);

  auto xs = [&](int j) { return reinterpret_cast<u32x4*>(lds + (size_t)j * C::kXBytes); };
  uint8_t* const ws_s = lds + C::kStages * C::kXBytes;  // scale window [RW][kWB]
  uint8_t* const ws_b = ws_s + C::kWinBytes;            // bias window

  // ---- staging of one phase's x pieces, global -> LDS directly (no registers) ----
  // x piece i = (v * 16 + g4 * 4 + t) * MP + m holds x[m][PH ph + 128 v + 32 g4 + 8 t .. + 8):
  // the A fragment of MFMA (v, t) for lane (m, g4). Rows m >= M read as zero. Wave w's j-th load
  // fills pieces j * kRpThreads + 64 w .. + 63, one contiguous kilobyte of the stage (the LDS
  // destination of a lane is the instruction's base + 16 lane). Completion is waited for with an
  // explicit vector memory count one phase later, before the barrier that publishes the stage.
  static_assert(C::kXPieces % kRpThreads == 0, "whole x loads per thread");
  typedef __attribute__((address_space(3))) void* lds_ptr;
  auto stage_x = [&](int st, int ph, bool live) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < C::kXL; ++j) {
      const int i = tid + j * kRpThreads;
      const int m = i % MP, q = i / MP;  // q = v * 16 + g4 * 4 + t
      const int v = q >> 4, g4 = (q >> 2) & 3, t = q & 3;
      const uint32_t off = (live && m < P.M)
                               ? ((uint32_t)m * (uint32_t)P.K + (uint32_t)(ph * C::PH + 128 * v + 32 * g4 + 8 * t)) * 2u
                               : kOut;
      const lds_ptr dst = (lds_ptr)(reinterpret_cast<uint8_t*>(xs(st)) + (size_t)(j * kRpThreads + 64 * wave) * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, dst, 16, off, 0, 0, 0);
    }
  };

  // ---- scale window: groups of phases [ph0, ph0 + WP) of the range's rows, 16-byte pieces of
  // each row's contiguous run (every scale line is read once per window, not once per phase).
  // Loaded into registers (scales, then biases), then stored to LDS once no wave still reads the
  // previous window. ----
  constexpr int kPR = C::kWB / 16;  // window pieces per row
  auto load_window = [&](int ph0, u32x4 (&r)[2][C::kWL]) __attribute__((always_inline)) {
    const int g0 = ph0 * (2 * V);  // first group of the window
#pragma unroll
    for (int arr = 0; arr < 2; ++arr)
#pragma unroll
      for (int j = 0; j < C::kWL; ++j) {
        const int i = tid + j * kRpThreads;
        const int row = i / kPR, pc = i - row * kPR;
        const bool ok = row < nrows && g0 + pc * 8 < KG;
        const uint32_t off = ok ? (uint32_t)grow(row) * (uint32_t)KG * 2u + (uint32_t)(g0 + pc * 8) * 2u : kOut;
        r[arr][j] = __builtin_amdgcn_raw_buffer_load_b128(arr == 0 ? rs : rb, off, 0, 0);
      }
  };
  // Returns whether this thread saw a scale outside the fast dequantization's range.
  auto store_window = [&](const u32x4 (&r)[2][C::kWL]) __attribute__((always_inline)) {
    bool bad = false;
#pragma unroll
    for (int arr = 0; arr < 2; ++arr) {
      u32x4* d = reinterpret_cast<u32x4*>(arr == 0 ? ws_s : ws_b);
#pragma unroll
      for (int j = 0; j < C::kWL; ++j) {
        const int i = tid + j * kRpThreads;
        // (Every variant's window is a whole number of pieces per thread: no store is skipped, so
        // no load is left pending on one path of a branch.)
        if ((RW * kPR) % kRpThreads == 0 || i < RW * kPR) {
          const int row = i / kPR, pc = i - row * kPR;
          d[row * (C::kWS / 16) + pc] = r[arr][j];
          if (arr == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) bad |= !fast_scale_ok(r[arr][j][e] & 0xFFFFu) || !fast_scale_ok(r[arr][j][e] >> 16);
          }
        }
      }
    }
    return bad;
  };

  // ---- weights: one phase of the wave's blocks, double-buffered in registers ----
  u32x4 wv[2][BPW][V];
  uint32_t wo[BPW];
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    wo[j] = (j < nbw) ? (uint32_t)grow(16 * (wave + kRpWaves * j) + n) * (uint32_t)(P.K >> 1) + (uint32_t)g * 16u : kOut;
  }
  // Piece v of every block of phase ph into register buffer J (a zero-length resource when the
  // phase does not exist: the loads then read zero without touching memory).
  auto fetch_v = [&](int J, int v, int ph, bool live) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(P.w), 0,
                                                                        live ? wrec : 0, kBufferRsrcWord3);
#pragma unroll
    for (int j = 0; j < BPW; ++j)
      wv[J][j][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, wo[j] + (uint32_t)(v * 64), ph * (C::PH / 2), 0);
  };

  f32x4 acc[BPW][MB];
#pragma unroll
  for (int j = 0; j < BPW; ++j)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[j][i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // ---- super-step v of one phase: LDS stage `st`, register buffer J ----
  auto compute_v = [&](int st, int pw, int v, auto jc, auto fast) __attribute__((always_inline)) {
    constexpr int J = decltype(jc)::value;
    constexpr bool FAST = decltype(fast)::value;
    const u32x4* xb = xs(st);
    // Phase pw of the window: dwords pw * V .. pw * V + V - 1 of each row's window run.
    // This lane's words of super-step v lie in group 2 v + g / 2 of the phase: bf16 2 v + g / 2 of
    // row (wave + W j) * 16 + n's window run, read alone (a 16-bit LDS read) so that no half needs
    // selecting in registers.
    const uint16_t* sb16 = reinterpret_cast<const uint16_t*>(ws_s) + pw * V * 2 + (g >> 1);
    const uint16_t* bb16 = reinterpret_cast<const uint16_t*>(ws_b) + pw * V * 2 + (g >> 1);
    constexpr int NJ = C::kOptLast ? BPW - 1 : BPW;  // slots every wave computes
    const bool full = !C::kOptLast || nbw == BPW;     // wave-uniform
    float c1[BPW], c2[BPW], bfv[BPW];
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      const int lrow = 16 * (wave + kRpWaves * j) + n;
      const uint32_t sbits = sb16[lrow * (C::kWS / 2) + 2 * v];
      const uint32_t bbits = bb16[lrow * (C::kWS / 2) + 2 * v];
      const float sf = bf16_to_f32(sbits);
      bfv[j] = bf16_to_f32(bbits);
      c1[j] = FAST ? sf * 16777216.0f : sf;
      c2[j] = FAST ? sf * 1048576.0f : sf * 0.0625f;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      u32x4 a[MB];
#pragma unroll
      for (int i = 0; i < MB; ++i) a[i] = xb[(v * 16 + g * 4 + t) * MP + i * 16 + n];
      // Blocks past this wave's count hold zero weights (their loads lie outside the buffer)
      // and sums that are never stored: computing them keeps the loop free of branches, except
      // for the last slot of an OPT variant, which only the waves holding a BPW-th block run.
#pragma unroll
      for (int j = 0; j < BPW; ++j) {
        if (j >= NJ && !full) continue;
        const u32x4 B = FAST ? dequant_word_fast(wv[J][j][v][t], c1[j], c2[j], bfv[j])
                             : dequant_word(wv[J][j][v][t], c1[j], c2[j], bfv[j]);
#pragma unroll
        for (int i = 0; i < MB; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[i]), as_bf16x8(B), acc[j][i], 0, 0, 0);
      }
    }
  };
  // ---- one phase; piece v of every block is refilled with phase `nph` (two phases ahead) as
  // soon as super-step v has been used. The refills stay outside the branch on the
  // dequantization form: loads issued in both arms of a branch leave register copies at the
  // join, and a copy of a register still being loaded waits for every load issued before it. ----
  auto compute = [&](int st, int pw, auto jc, bool fast, int nph, bool nlive) __attribute__((always_inline)) {
    constexpr int J = decltype(jc)::value;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      if (fast)
        compute_v(st, pw, v, jc, std::true_type{});
      else
        compute_v(st, pw, v, jc, std::false_type{});
      fetch_v(J, v, nph, nlive);
    }
  };

  // ---- prologue: x of phase pa (and pa + 1 with three stages), the weights of phases pa and
  // pa + 1, the scale window of phase pa ----
  constexpr int kSt = C::kStages;
  stage_x(0, pa, np > 0);
  if constexpr (kSt == 3) stage_x(1, pa + 1, np > 1);
#pragma unroll
  for (int v = 0; v < V; ++v) fetch_v(0, v, pa, np > 0);
#pragma unroll
  for (int v = 0; v < V; ++v) fetch_v(1, v, pa + 1, np > 1);
  // The window's loads return after the x loads above (the vector memory count is in order), so
  // its stores also find both x stages written.
  // Later windows are loaded into registers one phase ahead where the registers allow
  // (accumulators, two weight buffers and the window within 150 of the 256 VGPRs); otherwise a
  // window is loaded and stored at its first phase.
  constexpr bool kWinAhead = 4 * BPW * MB + 8 * BPW * V + 8 * C::kWL <= 150;
  u32x4 wr[2][C::kWL];
  // Windows start at the workgroup's first phase, rounded down so the window's first group is a
  // multiple of 8 (every 16-byte piece then 16-byte aligned): a K slice reads the scale bytes of
  // its own phases, not those of every WP-phase block of K it straddles (c2's 12 slices of 68
  // phases used to read two windows each where one covers them).
  const int wbase = pa - pa % (4 / V);
  load_window(wbase, wr);
  if (tid == 0) {
    s_bad[0] = 0;
    s_bad[1] = 0;
  }
  bool winbad = __syncthreads_or(store_window(wr)) != 0;

  // Loads issued after the x of phase ph + 1 by the end of phase ph: with three stages the rest of
  // phase ph - 1's weight refills, the x of phase ph + 2 and phase ph's refills; with two (x of
  // phase ph + 1 issued at the start of phase ph) phase ph's refills.
  constexpr int kAfter = kSt == 3 ? 2 * BPW * V + C::kXL : BPW * V;
  static_assert(kAfter < 64, "vector memory count range");

  // ---- phase ph from register buffer J and x stage (ph - pa) % kSt. Meanwhile the x of phase
  // ph + kSt - 1 goes into stage (ph - pa + kSt - 1) % kSt (last read in phase ph - 1), and the
  // weights of phase ph + 2 into buffer J as phase ph's pieces are used. A phase that starts a
  // scale window restages the window first (after the previous phase's barrier). ----
  auto phase = [&](int ph, auto jc) __attribute__((always_inline)) {
    const int k = ph - pa;
    const int st = k % kSt, st2 = (k + kSt - 1) % kSt, pw = (ph - wbase) % C::WP;
    if (pw == 0 && k > 0) {
      if constexpr (kWinAhead) {
        // The window's registers were loaded during the previous phase, and every wave is past
        // its last read of the old window (the previous phase's barrier).
        const int wpar = ((ph - wbase) / C::WP) & 1;
        if (store_window(wr)) s_bad[wpar] = 1;
        if (tid == 0) s_bad[wpar ^ 1] = 0;  // last read one window ago
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        winbad = s_bad[wpar] != 0;
      } else {
        load_window(ph, wr);
        winbad = __syncthreads_or(store_window(wr)) != 0;
      }
    }
    const bool live2 = ph + 2 < pb;
    if (kWinAhead && pw == C::WP - 1 && ph + 1 < pb) load_window(ph + 1, wr);
    stage_x(st2, ph + kSt - 1, ph + kSt - 1 < pb);
    compute(st, pw, jc, !winbad, ph + 2, live2);
    // The x of phase ph + 1 (issued at the start of phase ph + 2 - kSt) is in LDS; publish it. A bare
    // barrier: __syncthreads() would also wait for the x and weight loads of the phases ahead
    // (its fence covers the LDS writes of the DMA still in flight).
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kAfter) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  int i = 0;
  for (; i + 2 <= np; i += 2) {
    phase(pa + i, std::integral_constant<int, 0>{});
    phase(pa + i + 1, std::integral_constant<int, 1>{});
  }
  if (i < np) phase(pa + i, std::integral_constant<int, 0>{});

  // ---- epilogue ----
  const int ny = fused ? P.N >> 1 : P.N;  // columns of y
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      P.y, 0, rsrc_bytes((unsigned long long)P.M * ny * 2), kBufferRsrcWord3);
  // bf16 tile of y through LDS: tile[m][local column], then 16-byte row chunks.
  uint16_t* yt = reinterpret_cast<uint16_t*>(lds);
  auto write_y = [&]() __attribute__((always_inline)) {
    // Chunk c = m * (RW / 8) + q holds columns 8 q .. 8 q + 7 of row m.
    const int cpr = nrows / 8;  // chunks per row
    for (int c = tid; c < P.M * cpr; c += kRpThreads) {
      const int m = c / cpr, q = c - m * cpr;
      const u32x4 v = *reinterpret_cast<const u32x4*>(yt + m * RW + q * 8);
      __builtin_amdgcn_raw_buffer_store_b128(v, ry, ((uint32_t)m * (uint32_t)P.N + (uint32_t)(r0 + q * 8)) * 2u, 0, 0);
    }
  };
  // Fused: output columns 16 hb0 .. 16 (hb0 + hb) - 1 of y = silu(gate) * up, from the tile's gate
  // (local columns below 16 hb) and up halves, bf16 values as the unfused projection writes them.
  auto write_y_fused = [&]() __attribute__((always_inline)) {
    const int cpr = hb * 2;  // 8-column chunks per row
    for (int c = tid; c < P.M * cpr; c += kRpThreads) {
      const int m = c / cpr, q = c - m * cpr;
      const u32x4 gv = *reinterpret_cast<const u32x4*>(yt + m * RW + q * 8);
      const u32x4 uv = *reinterpret_cast<const u32x4*>(yt + m * RW + hb * 16 + q * 8);
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = silu_mul_bf16(gv[e] & 0xFFFFu, uv[e] & 0xFFFFu) | (silu_mul_bf16(gv[e] >> 16, uv[e] >> 16) << 16);
      __builtin_amdgcn_raw_buffer_store_b128(o, ry, ((uint32_t)m * (uint32_t)ny + (uint32_t)(16 * hb0 + q * 8)) * 2u, 0, 0);
    }
  };
  auto tile_to_lds = [&](const f32x4 (&a)[BPW][MB]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      if (j < nbw) {
        const int col = 16 * (wave + kRpWaves * j) + n;
#pragma unroll
        for (int ii = 0; ii < MB; ++ii)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = ii * 16 + 4 * g + r;
            yt[m * RW + col] = (uint16_t)(pack_bf16x2(a[j][ii][r], 0.0f) & 0xFFFFu);
          }
      }
    }
  };

  if (P.S == 1) {
    // The y tile reuses the x stages. The last phases still issued x DMA (zeros from outside the
    // buffer) that the phase barrier's count lets run on, so every wave first waits for all of its
    // loads, and a barrier makes sure no DMA of any wave can still land on the tile.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    tile_to_lds(acc);
    __syncthreads();
    if (fused)
      write_y_fused();
    else
      write_y();
    return;
  }

  // K split: store this workgroup's fp32 partial tile (item (wave, j, i) lane-major); the reduce
  // kernel that follows on the stream adds a range's partials in workgroup order.
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      P.part, 0, rsrc_bytes((unsigned long long)gridDim.x * C::kItems * 16), kBufferRsrcWord3);
#pragma unroll
  for (int j = 0; j < BPW; ++j)
#pragma unroll
    for (int ii = 0; ii < MB; ++ii) {
      const uint32_t item = (uint32_t)(((wave * BPW + j) * MB + ii) * 64 + lane);
      if (j < nbw)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[j][ii]), rp,
                                               ((uint32_t)p * C::kItems + item) * 16u, 0, kCoherent);
    }
}

// K split, second pass: y from the S partial tiles of each block range, added in workgroup order
// from +0 (the order a single workgroup adding them would use), one f32x4 item per thread. The
// sum of a range used to be formed by the range's last workgroup alone: 12 tiles of 64 KB read by
// one CU took 6.5-7.6 us at the end of the batched-verify down projection; spread over the GPU
// the same bytes take a few microseconds.
constexpr int kRedThreads = 256;
template <class C>
__global__ __launch_bounds__(kRedThreads) void rowphase_reduce_kernel(RowPhaseParams P) {
  constexpr int MB = C::MB, BPW = C::BPW, kRpWaves = C::kRpWaves;
  const int ranges = P.ranges;
  const int it = blockIdx.x * kRedThreads + threadIdx.x;
  const int range = it / C::kItems;
  if (range >= ranges) return;
  // Item = ((wave * BPW + j) * MB + ii) * 64 + lane of the first pass.
  const int item = it - range * C::kItems;
  const int lane = item & 63, rest = item >> 6;
  const int ii = rest % MB, wj = rest / MB;
  const int j = wj % BPW, wave = wj / BPW;
  const int blk = wave + kRpWaves * j;  // block within the range
  const int n = lane & 15, g = lane >> 4;
  // Fused gate+up: the range's gate blocks are its local blocks 0 .. hb - 1 and their up blocks
  // hb .. 2 hb - 1; a gate item's thread also adds its up item and writes silu(gate) * up.
  const bool fused = C::kFusable && P.fused;
  const int hb0 = range * (P.BW >> 1);
  const int hb = fused ? min(P.BW >> 1, (P.NB >> 1) - hb0) : 0;
  const int b0 = range * P.BW;
  if (fused ? blk >= hb : blk >= min(P.BW, P.NB - b0)) return;  // no such block (or an up block)
  const int col = fused ? (hb0 + blk) * 16 + n : (b0 + blk) * 16 + n;
  const int ublk = blk + hb;
  const int uitem = ((((ublk % kRpWaves) * BPW + ublk / kRpWaves) * MB + ii) << 6) + lane;
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      P.part, 0, rsrc_bytes((unsigned long long)ranges * P.S * C::kItems * 16), kBufferRsrcWord3);
  const uint32_t base = (uint32_t)range * (uint32_t)P.S;
  // The S partial tiles' item `itm` added in workgroup order. kRedBatch contributors' loads in
  // flight at a time (one memory round trip for the usual S of 10-12); past the last they read
  // zero (an offset outside the buffer), and adding +0 leaves a sum that is not -0 unchanged (a
  // sum from +0 never is -0).
  constexpr int kRedBatch = 16;
  auto add_slices = [&](int itm) __attribute__((always_inline)) {
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int q = 0; q < P.S; q += kRedBatch) {
      f32x4 v[kRedBatch];
#pragma unroll
      for (int u = 0; u < kRedBatch; ++u) {
        const uint32_t off =
            q + u < P.S ? ((base + (uint32_t)(q + u)) * C::kItems + (uint32_t)itm) * 16u : 0x80000000u;
        v[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, kCoherent));
      }
#pragma unroll
      for (int u = 0; u < kRedBatch; ++u) {
        sum[0] += v[u][0]; sum[1] += v[u][1]; sum[2] += v[u][2]; sum[3] += v[u][3];
      }
    }
    return sum;
  };
  const f32x4 sum = add_slices(item);
  const int ny = fused ? P.N >> 1 : P.N;  // columns of y
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      P.y, 0, rsrc_bytes((unsigned long long)P.M * ny * 2), kBufferRsrcWord3);
  if (fused) {
    const f32x4 up = add_slices(uitem);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = ii * 16 + 4 * g + r;
      if (m < P.M)
        __builtin_amdgcn_raw_buffer_store_b16(
            (uint16_t)silu_mul_bf16(pack_bf16x2(sum[r], 0.0f) & 0xFFFFu, pack_bf16x2(up[r], 0.0f) & 0xFFFFu), ry,
            ((uint32_t)m * (uint32_t)ny + (uint32_t)col) * 2u, 0, 0);
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = ii * 16 + 4 * g + r;
    if (m < P.M)
      __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(pack_bf16x2(sum[r], 0.0f) & 0xFFFFu), ry,
                                            ((uint32_t)m * (uint32_t)ny + (uint32_t)col) * 2u, 0, 0);
  }
}

}  // namespace

// Kernel table: id -> (row blocks of x, super-steps per phase, blocks per wave, waves, x stages,
// last slot computed only by the waves that hold a block there). Ids 20-27 are the wide plans'
// twins of ids 4, 5, 10, 2, 13, 15, 9 and 3: over 34816 and 65984 columns (9 and 17 blocks per
// workgroup) the waves short of a last block skip it, so the busiest SIMD runs 3 of 4 (5 of 6)
// block slots per phase: 9-64 rows over 5120 -> 34816 / 65984 9-17% faster, identical bits; 65-96
// rows over 34816 (ids 24, 25) then beat the GEMM.
#define QMM4_ROWPHASE_VARIANTS(X) \
  X(0, 1, 2, 5, 8, 3, 0)          \
  X(1, 2, 2, 5, 8, 3, 0)          \
  X(2, 4, 2, 3, 8, 3, 0)          \
  X(3, 1, 4, 2, 8, 3, 0)          \
  X(4, 2, 4, 2, 8, 3, 0)          \
  X(5, 4, 2, 2, 8, 3, 0)          \
  X(6, 1, 4, 1, 8, 3, 0)          \
  X(7, 2, 4, 1, 8, 3, 0)          \
  X(8, 4, 2, 1, 8, 3, 0)          \
  X(9, 1, 2, 3, 8, 3, 0)          \
  X(10, 2, 2, 3, 8, 3, 0)         \
  X(11, 1, 2, 4, 8, 3, 0)         \
  X(12, 2, 2, 4, 8, 3, 0)         \
  X(13, 5, 2, 2, 8, 2, 0)         \
  X(14, 5, 2, 1, 8, 2, 0)         \
  X(15, 6, 2, 2, 8, 2, 0)         \
  X(16, 6, 2, 1, 8, 2, 0)         \
  X(17, 7, 2, 2, 8, 2, 0)         \
  X(18, 7, 2, 1, 8, 2, 0)         \
  X(19, 8, 2, 1, 8, 2, 0)         \
  X(20, 2, 4, 2, 8, 3, 1)         \
  X(21, 4, 2, 2, 8, 3, 1)         \
  X(22, 2, 2, 3, 8, 3, 1)         \
  X(23, 4, 2, 3, 8, 3, 1)         \
  X(24, 5, 2, 2, 8, 2, 1)         \
  X(25, 6, 2, 2, 8, 2, 1)         \
  X(26, 1, 2, 3, 8, 3, 1)         \
  X(27, 1, 4, 2, 8, 3, 1)
constexpr int kRpVariants = 28;

#define QMM4_RPCFG(id, mb, v, bpw, w, stg, opt) typedef RpCfg<mb, v, bpw, w, stg, opt> RpCfg##id;
QMM4_ROWPHASE_VARIANTS(QMM4_RPCFG)
#undef QMM4_RPCFG

static bool rowphase_geometry(int id, int* mb, int* v, int* bpw, size_t* lds, int* items, int* waves = nullptr,
                              bool* opt = nullptr) {
  switch (id) {
#define QMM4_RPG(i, m, vv, b, w, stg, op)                                                                \
  case i:                                                                                           \
    *mb = m; *v = vv; *bpw = b; *lds = RpCfg##i::kLds; *items = RpCfg##i::kItems;                    \
    if (waves) *waves = w;                                                                          \
    if (opt) *opt = op;                                                                             \
    return true;
    QMM4_ROWPHASE_VARIANTS(QMM4_RPG)
#undef QMM4_RPG
    default: return false;
  }
}

static const void* rowphase_func(int id) {
  switch (id) {
#define QMM4_RPF(i, m, vv, b, w, stg, opt) \
  case i: return reinterpret_cast<const void*>(&rowphase_kernel<RpCfg##i>);
    QMM4_ROWPHASE_VARIANTS(QMM4_RPF)
#undef QMM4_RPF
    default: return nullptr;
  }
}

constexpr int kRpNarrowBpw = 2;  // blocks per wave when K is split

bool rowphase_plan(int M, int N, int K, int cus, RowPhasePlan* plan, bool fused) {
  if (M < 1 || M > 128 || N % (fused ? 32 : 16) != 0 || cus < 1) return false;
  // Row blocks of x: 16, 32 or 64 rows, then 80 to 128 (variants with two x stages).
  const int mb = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : (M + 15) / 16;
  const int NB = N / 16;
  const int ks = K / 128;
  // Row offsets of this kernel stay below 2 GiB (rows past the end are addressed at 2 GiB).
  if ((unsigned long long)(N + 256) * (unsigned long long)K / 2 >= (1ULL << 31)) return false;
  // Wide: every CU its own rows over all of K (at least one block per wave). Narrow: ranges of
  // kRpNarrowBpw blocks per wave, K split over the CUs.
  constexpr int kW = 8;  // waves per workgroup of every variant
  const bool wide = NB >= kW * cus;
  // Fused gate+up (N = 2 n stacked rows): each range the same BW / 2 blocks of both halves, so that
  // the SiLU·mul epilogue finds gate and up columns in one tile (the first pass's, or with K split
  // the reduce kernel's). Narrow plans keep the projection's: ceil(NB / BW) = ceil(NB / 2 / (BW / 2))
  // ranges either way, so the same K slices and the same bits.
  if (fused && M > 96) return false;
  const int NBh = NB / 2;
  // The variant for mb rows with the fewest blocks per wave that still holds `want` (or the most).
  auto pick = [&](int want) {
    int id = -1, best_b = 0;
    for (int c = 0; c < kRpVariants; ++c) {
      int cm, cv, cb, items, cw;
      size_t l;
      bool co;
      rowphase_geometry(c, &cm, &cv, &cb, &l, &items, &cw, &co);
      if (cm != mb || ks % cv != 0 || co) continue;
      const bool fits = cb >= want;
      const bool best_fits = best_b >= want;
      if (id < 0 || (fits && (!best_fits || cb < best_b)) || (!fits && !best_fits && cb > best_b)) {
        id = c;
        best_b = cb;
      }
    }
    return id;
  };
  // Wide: a CU's share of the blocks in ranges of one size, as many per CU as the largest variant
  // needs; the grid then holds about `passes` ranges per CU, which the hardware starts on each CU as
  // the previous one ends. Ranges of the largest variant's size would leave a partial last round:
  // lm_head 248320 x 5120 at 16 / 32 rows takes 388 ranges of 40 blocks in 226 / 250 us, 501 of 31
  // in 206 / 229 us. Up to 32 rows only: every range reads all of x, and at 64 rows (655 KB of x
  // per range at K = 5120) the extra ranges cost more than the balance gains (+4-7%).
  int passes = 1, bw = (NB + cus - 1) / cus;
  if (wide && mb <= 2) {
    const int maxb = [&] {
      int m = 0;
      for (int c = 0; c < kRpVariants; ++c) {
        int cm, cv, cb, items, cw;
        size_t l;
        bool co;
        rowphase_geometry(c, &cm, &cv, &cb, &l, &items, &cw, &co);
        if (cm == mb && ks % cv == 0 && !co && cb > m) m = cb;
      }
      return m;
    }();
    if (maxb == 0) return false;
    const int share = (NB + cus - 1) / cus;
    passes = (share + kW * maxb - 1) / (kW * maxb);
    bw = (NB + cus * passes - 1) / (cus * passes);
  }
  if (fused) bw = 2 * ((NBh + cus * passes - 1) / (cus * passes));
  // Narrow: ranges of kRpNarrowBpw or one more block per wave, whichever gives a workgroup the
  // shorter walk (blocks x phases of its K slice x super-steps per phase) with the grid filling
  // the CUs; a tie keeps the smaller ranges (fewer partial tiles to add). 17-32 rows over
  // 5120 -> 17408: 68 ranges x 3 slices (204 workgroups) took 31.0-32.0 us, 46 x 5 (230)
  // 28.1-28.7 us; 17408 -> 5120 ties and keeps 20 x 12 (14 x 18 of 3 blocks per wave: 16 / 48 /
  // 64 rows 22.6 / 30.9 / 32.3 -> 24.2 / 34.3 / 35.6 us). Ranges of one block per wave (twice the
  // ranges, half the K slices, the same walk) when those ranges would leave a workgroup at most
  // 3 phases, too few to pipeline: 32 / 64 x 5120 -> 5120 17.0 / 20.6 -> 16.0 / 19.4 us,
  // 16 / 32 x 17408 -> 5120 24.8 / 27.9 -> 22.6 / 26.5 us; with 6 phases (64 x 17408 -> 5120)
  // the doubled x reads cost more (33.5 -> 37.2 us). They also replace them when their walk is
  // strictly shorter: 48 / 64 x 5120 -> 10240 (80 ranges x 3 slices, 7 phases, against 40 x 6 of
  // 4) 27.0 / 27.4 -> 24.3 / 26.2 us.
  auto narrow = [&](int c, int* phases) {
    int cm, cv, cb, items;
    size_t l;
    rowphase_geometry(c, &cm, &cv, &cb, &l, &items);
    const int np = ks / cv;
    const int ranges = (NB + kW * cb - 1) / (kW * cb);
    int sp = cus / ranges;
    if (sp < 1) sp = 1;
    if (sp > np) sp = np;
    *phases = (np + sp - 1) / sp;
    return (long long)kW * cb * *phases * cv;
  };
  int id = pick(wide ? (bw + kW - 1) / kW : kRpNarrowBpw);
  if (!wide && id >= 0) {
    int ph = 0, ph2 = 0, ph1 = 0;
    long long walk = narrow(id, &ph);
    const int id2 = pick(kRpNarrowBpw + 1);
    if (id2 >= 0 && id2 != id) {
      const long long walk2 = narrow(id2, &ph2);
      if (walk2 < walk) {
        id = id2;
        walk = walk2;
        ph = ph2;
      }
    }
    const int id1 = pick(1);
    if (id1 >= 0 && id1 != id) {
      const long long walk1 = narrow(id1, &ph1);
      if (walk1 < walk || (walk1 == walk && ph <= 3)) id = id1;
    }
  }
  if (id < 0) return false;
  if (wide) {
    // A wide plan whose blocks leave some waves a slot short takes the variant that skips that
    // slot's arithmetic in those waves, where one is built.
    int cm0, cv0, cb0, items0, cw0;
    size_t l0;
    rowphase_geometry(id, &cm0, &cv0, &cb0, &l0, &items0, &cw0);
    const int bwp = bw < kW * cb0 ? bw : kW * cb0;
    if (bwp < kW * cb0)
      for (int c = 0; c < kRpVariants; ++c) {
        int cm, cv, cb, items, cw;
        size_t l;
        bool co;
        rowphase_geometry(c, &cm, &cv, &cb, &l, &items, &cw, &co);
        if (co && cm == cm0 && cv == cv0 && cb == cb0 && cw == cw0) id = c;
      }
  }
  int cm, v, bpw, items;
  size_t lds;
  rowphase_geometry(id, &cm, &v, &bpw, &lds, &items);
  const int NP = ks / v;
  int BW, S;
  if (wide) {
    BW = bw < kW * bpw ? bw : kW * bpw;  // even when fused: bw is, and so is kW * bpw
    S = 1;
  } else {
    BW = kW * bpw;
    const int ranges = (NB + BW - 1) / BW;
    S = cus / ranges;
    if (S < 1) S = 1;
    if (S > NP) S = NP;
  }
  plan->variant = id;
  plan->BW = BW;
  plan->S = S;
  plan->NP = NP;
  plan->ranges = fused ? (NBh + BW / 2 - 1) / (BW / 2) : (NB + BW - 1) / BW;
  plan->blocks = plan->ranges * S;
  plan->lds = lds;
  plan->part_bytes = S > 1 ? (size_t)plan->blocks * items * 16 : 0;
  plan->wide = wide;
  plan->fused = fused;
  return true;
}

hipError_t launch_rowphase(const RowPhasePlan& plan, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                           const uint16_t* b, uint16_t* y, float* part, int M, int N, int K, hipStream_t stream) {
  RowPhaseParams P;
  P.x = x; P.s = s; P.b = b; P.w = w; P.y = y; P.part = part;
  P.M = M; P.N = N; P.K = K;
  P.NB = N / 16; P.BW = plan.BW; P.S = plan.S; P.NP = plan.NP; P.ranges = plan.ranges;
  P.fused = plan.fused ? 1 : 0;
  if (plan.fused) {
    int cm, cv, cb, items;
    size_t l;
    if (!rowphase_geometry(plan.variant, &cm, &cv, &cb, &l, &items) || cm > 6 || plan.BW % 2 != 0 || N % 32 != 0)
      return hipErrorInvalidValue;
  }
  const void* f = rowphase_func(plan.variant);
  if (!f) return hipErrorInvalidValue;
  hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)plan.lds);
  if (e != hipSuccess) return e;
  // K split: the reduce kernel's grid has one thread per f32x4 item of every range's tile.
  switch (plan.variant) {
#define QMM4_RPL(i, m, vv, bb, w, stg, opt)                                                                   \
  case i:                                                                                                   \
    hipLaunchKernelGGL(rowphase_kernel<RpCfg##i>, dim3(plan.blocks), dim3(RpCfg##i::kRpThreads), plan.lds,   \
                       stream, P);                                                                          \
    if (plan.S > 1) {                                                                                       \
      e = hipGetLastError();                                                                                \
      if (e != hipSuccess) return e;                                                                        \
      const long long items = (long long)plan.ranges * RpCfg##i::kItems;                                    \
      hipLaunchKernelGGL(rowphase_reduce_kernel<RpCfg##i>, dim3((unsigned)((items + kRedThreads - 1) / kRedThreads)), \
                         dim3(kRedThreads), 0, stream, P);                                                  \
    }                                                                                                       \
    break;
    QMM4_ROWPHASE_VARIANTS(QMM4_RPL)
#undef QMM4_RPL
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace qmm4
