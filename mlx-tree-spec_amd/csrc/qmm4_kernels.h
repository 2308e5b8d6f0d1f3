// Kernel launch interface between the C ABI layer (qmm4_api.cpp) and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qmm4 {

// Skinny (M <= 64) stream-K kernel geometry, chosen by M, K and the scale/bias alignment.
struct SkinnyPlan {
  int variant;      // index into the kernel table (see qmm4_skinny.hip)
  int tile_cols;    // output columns per tile (CW)
  int steps_v;      // super-steps (128 k) per unit (V)
  int blocks;       // workgroups launched (G)
  int tiles;        // tiles along N (T)
  long long units;  // T * K / (128 * V)
};

constexpr int kSkinnyVariants = 15;
// Variant for M rows when a unit may span up to `vmax` super-steps (1, 2 or 4).
int skinny_variant(int M, int vmax, int* tile_cols, int* steps_v);
// The resident-x twin of a variant (same geometry; x staged once per workgroup) and its number of
// x slots: a launch may use it only if no workgroup's range touches more distinct steps than
// that. -1 when the variant has none.
int skinny_resident_twin(int variant, int* slots);
// Resident workgroups per CU for a variant (from the HIP occupancy API; cached by the caller).
int skinny_occupancy(int variant);
// Enqueue the skinny kernel. `part` holds blocks*2*M*tile_cols floats, `cnt` tiles zeroed uint32s.
hipError_t launch_skinny(const SkinnyPlan& plan, const uint16_t* x, const uint32_t* w,
                         const uint16_t* s, const uint16_t* b, uint16_t* y, float* part,
                         uint32_t* cnt, int M, int N, int K, hipStream_t stream);

// Verify-shape kernel (M <= 64): tiles of output columns shared by the waves of a workgroup, which
// split each tile's k-steps round-robin; stream-K ranges over (tile, step) units.
struct VerifyPlan {
  int variant;      // index into the kernel table (see qmm4_verify.hip)
  int tile_cols;    // output columns per tile (CW)
  int steps_v;      // super-steps (128 k) per unit (V)
  int blocks;       // workgroups launched (G)
  int tiles;        // tiles along N (T)
  long long units;  // T * K / (128 * V)
  int threads;      // threads per workgroup
  size_t lds;       // dynamic LDS bytes
  size_t part_bytes;  // split-K partial workspace bytes
};
constexpr int kVerifyVariants = 10;
// Variant for M rows when a unit may span up to `vmax` super-steps.
int verify_variant(int M, int vmax);
// Resident workgroups per CU for a variant (HIP occupancy API).
int verify_occupancy(int variant);
// Fills `plan` for M rows on `cus` CUs with `occ` resident workgroups per CU; false if unsupported.
bool verify_plan(int M, int N, int K, int vmax, int cus, int occ, VerifyPlan* plan);
// `part` holds plan.part_bytes, `cnt` tiles zeroed uint32s.
hipError_t launch_verify(const VerifyPlan& plan, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                         const uint16_t* b, uint16_t* y, float* part, uint32_t* cnt, int M, int N, int K,
                         hipStream_t stream);

// Row-phase kernel (M <= 64): each workgroup owns a range of 16-row weight blocks and a range of
// K phases; x and the scales are staged per phase in LDS; K is split when N is small.
struct RowPhasePlan {
  int variant;        // index into the kernel table (see qmm4_rowphase.hip)
  int BW;             // blocks per range
  int S;              // workgroups per range (K split)
  int NP;             // phases along K
  int ranges;         // block ranges
  int blocks;         // workgroups = ranges * S
  size_t lds;         // dynamic LDS bytes
  size_t part_bytes;  // partial-tile workspace (S > 1)
  bool wide;          // every workgroup takes all of K (N fills the GPU)
  bool fused;         // gate+up: w stacks [gate; up] (N = 2 n rows), y = silu(gate) * up is [M, n]
};
bool rowphase_plan(int M, int N, int K, int cus, RowPhasePlan* plan, bool fused = false);
// `part` holds plan.part_bytes (used when plan.S > 1: the partial tiles, added by a second kernel
// launched behind the first on the same stream). A fused plan writes y as [M, N / 2].
hipError_t launch_rowphase(const RowPhasePlan& plan, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                           const uint16_t* b, uint16_t* y, float* part, int M, int N, int K, hipStream_t stream);

// Row-split kernel (up to 16 rows, output columns split evenly over one workgroup per CU, K whole
// or in a few slices).
struct RowSplitPlan {
  int MP;       // x rows per A fragment (4 or 8)
  bool small;   // every unit in flight from the start, all of x in LDS, sums in registers
  bool xreg;    // 9-16 rows over a small problem: x loaded straight into registers per K chunk
  bool pair;    // whole K with units taken in groups (consecutive steps of a block, one slot per group)
  int GU;       // units per group when pair
  bool own;     // whole K, each wave owning whole blocks with their sums in registers (no slots)
  int V;        // super-steps (128 k) per unit
  bool fused;   // fused gate+up: y = silu(x w_gate^T) * (x w_up^T), w = [w_gate; w_up]
  int Nout;     // output columns (N, or N / 2 when fused)
  int R;        // output columns per workgroup
  int RB;       // 16-row blocks per workgroup: ceil(R / 16), or ceil(2R / 16) when fused
  int SU;       // units per block (Kp / (128 V))
  int KS;       // K slices per column range (1: whole K per workgroup)
  int Kp;       // K per slice
  int ranges;   // column ranges
  int blocks;   // workgroups (ranges x KS)
  size_t part_bytes;  // KS > 1: fp32 row sums in the workspace (counters: one per range)
  size_t smem;  // dynamic LDS bytes
};
// Fills `plan` and returns true when the shape suits the row-split kernel on `cus` CUs. N is the
// number of weight rows (for the fused gate+up, both halves).
bool rowsplit_plan(int M, int N, int K, int cus, bool fused, RowSplitPlan* plan);
// 9 to 16 rows over at most 32 weight rows per CU and K of at most 6144: one wave per 512-k chunk
// of both of its workgroup's blocks, x loaded straight into registers.
bool rowsplit_xreg_plan(int M, int N, int K, int cus, RowSplitPlan* plan);
// The residual add + RMS norm folded into the row-split kernel's x staging: the projection's
// input is n = rmsnorm(x + r) * weight over rows of K, and h = x + r and n are also stored.
struct RowSplitNorm {
  const uint16_t* r;       // bf16 [M, K]
  const uint16_t* weight;  // bf16 [K]
  uint16_t* h;             // bf16 [M, K]
  uint16_t* n;             // bf16 [M, K]
  float eps;
};
// Whether a launch of `plan` can normalise its x while staging it (up to 4 rows, K <= 8192, not
// the 9-16-row form).
bool rowsplit_norm_ok(const RowSplitPlan& plan, int M, int K);
// part / cnt: the workspace (plan.part_bytes, plan.ranges counters at zero) when plan.KS > 1.
// `norm` (optional, rowsplit_norm_ok): x is normalised as it is staged.
hipError_t launch_rowsplit(const RowSplitPlan& plan, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                           const uint16_t* b, uint16_t* y, float* part, uint32_t* cnt, int M, int N, int K,
                           hipStream_t stream, const RowSplitNorm* norm = nullptr);

// y[m, j] = silu_mul_bf16(t[m, j], t[m, n + j]) for t bf16 [M, 2n] (the unfused gate+up epilogue).
hipError_t launch_silu_mul(const uint16_t* t, uint16_t* y, int M, int n, hipStream_t stream);

// h = bf16(x + r), n = bf16(w * bf16(h / sqrt(mean(h^2) + eps))) per row of D (D % 8 == 0,
// D <= add_rms_norm_max_d(); all pointers 16-byte aligned).
int add_rms_norm_max_d();
hipError_t launch_add_rms_norm(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* h,
                               uint16_t* n, int rows, int D, float eps, hipStream_t stream);

// Zero n uint32 words (the skinny kernel's arrival counters when their workspace is allocated).
hipError_t launch_zero_u32(uint32_t* p, size_t n, hipStream_t stream);

// LDS-tiled MFMA GEMM for M > 64: whole 256 x 256 tiles when there are more 128 x 128 tiles than
// CUs, otherwise stream-K over 128 x 128 tiles, or over 256 x 256 tiles for long K and few tiles
// (fp32 partials of split tiles in the workspace, added by a fix-up kernel behind the first).
struct GemmPlan {
  bool sk;            // stream-K
  bool sk256;         // stream-K over 256 x 256 tiles (else 128 x 128, or 128 x 256 with sk_wide)
  bool sk_wide;       // stream-K over 128 x 256 tiles
  bool tail_sk;       // whole tiles whose quarter-tile tail runs as stream-K over the quarters
  int G;              // stream-K workgroups (of the whole launch, or of the tail)
  size_t part_bytes;  // stream-K partial tiles (two per workgroup)
};
// `ws_capacity`: the most partial-tile bytes the caller's workspace can hold (stream-K spreads
// over fewer workgroups when it is small).
bool gemm_plan(int M, int N, int K, int cus, size_t ws_capacity, const uint16_t* s, const uint16_t* b,
               GemmPlan* plan);
hipError_t launch_gemm(const GemmPlan& plan, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                       const uint16_t* b, uint16_t* y, float* part, int M, int N, int K, int cus,
                       hipStream_t stream);

// Bit-exact dequantization to bf16 [N, K]: 4-bit codes in groups of 64 (the packed kernels'
// format), or 2-, 4- or 8-bit codes in groups of 32, 64 or 128 (K % group_size == 0).
hipError_t launch_dequant(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint16_t* out, int64_t N,
                          int64_t K, int group_size, int bits, hipStream_t stream);

}  // namespace qmm4
