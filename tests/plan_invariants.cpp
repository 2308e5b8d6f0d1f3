// Host-only check of the kernel planners exported by libqmm4.so: over a grid of shapes and CU
// counts, every plan a planner accepts must satisfy what its kernel assumes (LDS within 160 KB,
// the output columns covered exactly once, K slices and units that tile K, the loop forms only in
// the configurations their launch paths instantiate). Prints one line per violation and a summary;
// the exit status is the number of violations (capped at 255). Built and run by
// tests/test_plans.py; no GPU is touched.
#include <cstdio>
#include <cstdint>
#include <string>

#include "qmm4_kernels.h"

namespace qmm4 {
// Defined in qmm4_rowsplit.hip (exported, not in the kernels header): the plan's dynamic LDS, with
// the norm's reduction slots when `norm`.
size_t rowsplit_smem(const RowSplitPlan& plan, bool norm);
}  // namespace qmm4

using namespace qmm4;

namespace {

constexpr size_t kLds = 160 * 1024;
long long g_fail = 0, g_checked = 0;

#define CHECK(cond, ...)                                  \
  do {                                                    \
    if (!(cond)) {                                        \
      if (g_fail < 50) {                                  \
        std::printf("FAIL %s: ", #cond);                  \
        std::printf(__VA_ARGS__);                         \
        std::printf("\n");                                \
      }                                                   \
      ++g_fail;                                           \
    }                                                     \
  } while (0)

size_t xs_bytes(int kp, int mp) { return (size_t)(kp >> 7) * 16 * mp * 16; }
size_t part_bytes(int units, int mp) { return (size_t)units * (mp / 4) * 16 * 16; }

// Waves of a row-split workgroup (kRsWaves in qmm4_rowsplit.hip) and units in flight per wave.
constexpr int kRowSplitWaves = 8;
constexpr int kRowSplitRing = 2;

void check_rowsplit(int M, int N, int K, int cus, bool fused) {
  RowSplitPlan p{};
  if (!rowsplit_plan(M, N, K, cus, fused, &p)) return;
  ++g_checked;
  const char* f = "rowsplit M=%d N=%d K=%d cus=%d fused=%d";
#define RS(cond) CHECK(cond, f, M, N, K, cus, (int)fused)
  RS(M >= 1 && M <= 16);
  RS(p.MP == 4 || p.MP == 8 || p.MP == 16);
  RS(p.MP >= M);
  RS(!p.xreg);
  RS(p.V == 4 || p.V == 5);
  RS(p.fused == fused);
  RS(p.Nout == (fused ? N / 2 : N));
  RS(p.KS >= 1 && (long long)p.KS * p.Kp == K);
  RS(p.Kp % (128 * p.V) == 0);
  RS(p.SU == p.Kp / (128 * p.V) && p.SU >= 1);
  RS(p.R >= 4 && p.R % 4 == 0);
  RS((long long)p.ranges * p.R >= p.Nout && (long long)(p.ranges - 1) * p.R < p.Nout);
  RS(p.RB == ((fused ? 2 * p.R : p.R) + 15) / 16);
  RS(p.blocks == p.ranges * p.KS);
  RS(p.smem <= kLds);
  RS(p.smem >= xs_bytes(p.Kp, p.MP));
  RS((p.KS > 1) == (p.part_bytes > 0));
  RS((unsigned long long)(N + 256) * (unsigned long long)K / 2 < (1ULL << 30));
  RS(rowsplit_smem(p, false) == p.smem);
  const int modes = (int)p.small + (int)p.pair + (int)p.own;
  RS(modes <= 1);
  if (p.small) {
    RS(p.KS == 1 && p.V == 4 && !fused);
    RS(p.RB * p.SU <= kRowSplitWaves * kRowSplitRing);  // every unit in the waves' rings at once
  }
  if (p.pair) {
    // Launched only as whole-K, unfused, 4-step units; the groups tile each block's steps.
    RS(p.KS == 1 && p.V == 4 && !fused);
    RS(p.GU >= 2 && p.SU % p.GU == 0);
    RS(p.smem == xs_bytes(p.Kp, p.MP) + part_bytes(p.RB * p.SU / p.GU, p.MP) + 32);
  }
  if (p.own) {
    // Launched only as whole-K, unfused, 4-step units; every wave owns at least two blocks.
    RS(p.KS == 1 && p.V == 4 && !fused);
    RS(p.RB >= 2 * kRowSplitWaves);
    RS(p.smem == xs_bytes(p.Kp, p.MP));
  }
  if (!p.small && !p.pair && !p.own)
    RS(p.smem == xs_bytes(p.Kp, p.MP) + part_bytes(p.RB * p.SU, p.MP) + 32);
  if (rowsplit_norm_ok(p, M, K)) RS(rowsplit_smem(p, true) <= kLds && M <= 4);
#undef RS
}

void check_xreg(int M, int N, int K, int cus) {
  RowSplitPlan p{};
  if (!rowsplit_xreg_plan(M, N, K, cus, &p)) return;
  ++g_checked;
  const char* f = "xreg M=%d N=%d K=%d cus=%d";
#define XR(cond) CHECK(cond, f, M, N, K, cus)
  XR(M >= 9 && M <= 16 && p.MP == 16 && p.xreg && p.small);
  XR(p.V == 4 && p.KS == 1 && p.Kp == K && p.SU * 512 == K);
  XR(p.SU >= 1 && p.SU <= 12);  // one wave per 512-k chunk, at most 12 waves
  XR(p.RB >= 1 && p.RB <= 2 && p.RB == (p.R + 15) / 16);
  XR((long long)p.ranges * p.R >= N && (long long)(p.ranges - 1) * p.R < N);
  XR(p.blocks == p.ranges);
  XR(p.smem == (size_t)p.SU * 2 * 4 * 16 * 16 && p.smem <= kLds);
  XR(p.part_bytes == 0);
#undef XR
}

void check_rowphase(int M, int N, int K, int cus) {
  RowPhasePlan p{};
  if (!rowphase_plan(M, N, K, cus, &p)) return;
  ++g_checked;
  const char* f = "rowphase M=%d N=%d K=%d cus=%d";
#define RP(cond) CHECK(cond, f, M, N, K, cus)
  RP(M >= 1 && M <= 128);
  RP(p.BW >= 1 && p.S >= 1 && p.NP >= 1 && p.ranges >= 1);
  RP((long long)p.ranges * p.BW * 16 >= N);
  RP(p.blocks == p.ranges * p.S);
  RP(p.lds <= kLds);
  RP((p.S > 1) == (p.part_bytes > 0));
  RP(!p.wide || p.S == 1);
  RP(!p.fused);
#undef RP
  // Fused gate+up: a wide plan whose ranges hold the same BW / 2 blocks of both halves.
  RowPhasePlan q{};
  if (N % 32 != 0 || !rowphase_plan(M, N, K, cus, &q, true)) return;
  ++g_checked;
  const char* ff = "rowphase fused M=%d N=%d K=%d cus=%d";
#define RF(cond) CHECK(cond, ff, M, N, K, cus)
  const int nbh = N / 32;
  RF(q.fused && M <= 96 && q.wide == p.wide);
  RF(q.BW >= 2 && q.BW % 2 == 0);
  RF((long long)q.ranges * (q.BW / 2) >= nbh && (long long)(q.ranges - 1) * (q.BW / 2) < nbh);
  RF(q.blocks == q.ranges * q.S && q.lds <= kLds && q.NP >= 1);
  if (q.wide) {
    RF(q.S == 1 && q.part_bytes == 0);
  } else {  // the projection's own plan (the same K slices: the same bits)
    RF(q.variant == p.variant && q.BW == p.BW && q.S == p.S && q.NP == p.NP && q.ranges == p.ranges &&
       q.part_bytes == p.part_bytes);
  }
#undef RF
}

void check_verify(int M, int N, int K, int cus) {
  for (int vmax : {1, 2, 4})
    for (int occ : {1, 2}) {
      VerifyPlan p{};
      if (!verify_plan(M, N, K, vmax, cus, occ, &p)) continue;
      ++g_checked;
      const char* f = "verify M=%d N=%d K=%d cus=%d vmax=%d occ=%d";
#define VP(cond) CHECK(cond, f, M, N, K, cus, vmax, occ)
      VP(p.variant >= 0 && p.variant < kVerifyVariants);
      VP(p.steps_v >= 1 && p.steps_v <= vmax && K % (128 * p.steps_v) == 0);
      VP(p.tile_cols >= 1 && (long long)p.tiles * p.tile_cols >= N &&
         (long long)(p.tiles - 1) * p.tile_cols < N);
      VP(p.units == (long long)p.tiles * (K / (128 * p.steps_v)));
      VP(p.blocks >= 1 && p.blocks <= p.units);
      VP(p.threads >= 64 && p.threads <= 1024 && p.threads % 64 == 0);
      VP(p.lds <= kLds);
#undef VP
    }
}

void check_gemm(int M, int N, int K, int cus) {
  const uint16_t* s = reinterpret_cast<const uint16_t*>(uintptr_t{0x100000});
  const uint16_t* b = reinterpret_cast<const uint16_t*>(uintptr_t{0x200000});
  for (size_t cap : {(size_t)1 << 34, (size_t)8 << 20, (size_t)0}) {
    GemmPlan p{};
    if (!gemm_plan(M, N, K, cus, cap, s, b, &p)) continue;
    ++g_checked;
    const char* f = "gemm M=%d N=%d K=%d cus=%d cap=%zu";
#define GP(cond) CHECK(cond, f, M, N, K, cus, cap)
    if (p.sk) {
      const int tm = p.sk256 ? 256 : 128, tn = p.sk256 || p.sk_wide ? 256 : 128;
      const long long tiles = (long long)((M + tm - 1) / tm) * ((N + tn - 1) / tn);
      const long long units = tiles * (K / 64 / (K % 512 == 0 ? 8 : 2));
      GP(p.G >= 1 && p.G <= units);
      GP(p.part_bytes == (size_t)p.G * tm * tn * 4 * 2);
      GP(p.part_bytes <= cap);
      GP(!(p.sk256 && p.sk_wide));
      if (p.sk256)  // 8-step units, one workgroup per CU; no half-empty last row of tiles below 512 rows
        GP(K % 512 == 0 && M >= 256 && (M > 512 || M % 256 == 0 || M % 256 > 128) && p.G == cus);
      if (p.sk_wide) GP(K % 512 == 0 && p.G <= cus);           // 8-step units, one workgroup per CU
    } else if (p.tail_sk) {
      // Whole tiles whose last round (fewer quarters than CUs) runs as stream-K over its quarters.
      const long long total = (long long)((M + 255) / 256) * ((N + 255) / 256);
      const long long rem = total % cus;
      GP(K % 512 == 0 && rem > 0 && 4 * rem < cus && !p.sk256);
      GP(p.G >= 1 && p.G <= 4 * rem * (K / 512));
      GP(p.part_bytes == (size_t)p.G * 128 * 128 * 4 * 2 && p.part_bytes <= cap);
    } else {
      GP(!p.sk256 && !p.sk_wide && p.part_bytes == 0);
    }
#undef GP
  }
}

}  // namespace

// Query mode (`plan_invariants query`): one shape per stdin line, "<planner> M N K cus", with
// planner rowsplit, rowsplit_fused, xreg, rowphase, rowphase_fused or gemm; prints one line per query with the
// plan's form ("none" when the planner declines), so tests can check which form a GPU test case
// reaches on a given CU count.
int query() {
  char kind[32];
  int M, N, K, cus;
  while (std::scanf("%31s %d %d %d %d", kind, &M, &N, &K, &cus) == 5) {
    const std::string k = kind;
    if (k == "rowsplit" || k == "rowsplit_fused") {
      RowSplitPlan p{};
      if (!rowsplit_plan(M, N, K, cus, k == "rowsplit_fused", &p)) {
        std::printf("none\n");
        continue;
      }
      std::printf("MP=%d KS=%d V=%d small=%d pair=%d own=%d norm_ok=%d blocks=%d\n", p.MP, p.KS, p.V, (int)p.small,
                  (int)p.pair, (int)p.own, (int)rowsplit_norm_ok(p, M, K), p.blocks);
    } else if (k == "xreg") {
      RowSplitPlan p{};
      std::printf(rowsplit_xreg_plan(M, N, K, cus, &p) ? "xreg blocks=%d\n" : "none\n", p.blocks);
    } else if (k == "rowphase" || k == "rowphase_fused") {
      RowPhasePlan p{};
      if (!rowphase_plan(M, N, K, cus, &p, k == "rowphase_fused")) {
        std::printf("none\n");
        continue;
      }
      std::printf("variant=%d S=%d wide=%d blocks=%d BW=%d\n", p.variant, p.S, (int)p.wide, p.blocks, p.BW);
    } else if (k == "gemm") {
      const uint16_t* s = reinterpret_cast<const uint16_t*>(uintptr_t{0x100000});
      const uint16_t* b = reinterpret_cast<const uint16_t*>(uintptr_t{0x200000});
      GemmPlan p{};
      if (!gemm_plan(M, N, K, cus, (size_t)1 << 34, s, b, &p)) {
        std::printf("none\n");
        continue;
      }
      std::printf("sk=%d sk256=%d sk_wide=%d tail_sk=%d G=%d\n", (int)p.sk, (int)p.sk256, (int)p.sk_wide,
                  (int)p.tail_sk, p.G);
    } else {
      std::printf("unknown\n");
    }
  }
  return 0;
}

// Every planner's checks on the shapes read from stdin ("M N K" each), at 256, 304 and 80 CUs.
void check_all(int M, int N, int K, int cus) {
  if (M <= 16) {
    check_rowsplit(M, N, K, cus, false);
    if (N % 32 == 0) check_rowsplit(M, N, K, cus, true);
    check_xreg(M, N, K, cus);
  }
  if (M <= 128) check_rowphase(M, N, K, cus);
  if (M <= 64) check_verify(M, N, K, cus);
  else check_gemm(M, N, K, cus);
}

int check_listed() {
  int M, N, K;
  while (std::scanf("%d %d %d", &M, &N, &K) == 3)
    for (int cus : {256, 304, 80}) check_all(M, N, K, cus);
  std::printf("plans checked: %lld, violations: %lld\n", g_checked, g_fail);
  return g_fail > 255 ? 255 : (int)g_fail;
}

int main(int argc, char** argv) {
  if (argc > 1 && std::string(argv[1]) == "query") return query();
  if (argc > 1 && std::string(argv[1]) == "check") return check_listed();
  const int Ms[] = {1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 15, 16, 17, 24, 32, 33, 48, 63, 64, 65, 80, 81, 96, 97, 112, 113,
                    128, 300, 1024, 4096};
  const int Ns[] = {16, 32, 48, 256, 1024, 1040, 2048, 3072, 4096, 4112, 5120, 6144, 10240, 12288,
                    17408, 34816, 65984, 131072, 151936, 248320, 248336, 262144};
  const int Ks[] = {128, 256, 384, 512, 640, 1024, 2048, 2560, 4096, 5120, 6144, 8192, 12288, 17408, 20480};
  const int CUs[] = {256, 304, 80, 7, 1};
  for (int cus : CUs)
    for (int M : Ms)
      for (int N : Ns)
        for (int K : Ks) check_all(M, N, K, cus);
  std::printf("plans checked: %lld, violations: %lld\n", g_checked, g_fail);
  return g_fail > 255 ? 255 : (int)g_fail;
}
