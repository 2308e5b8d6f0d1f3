// Prefill quantized GEMM for M > 64 rows: y = x @ dequant(w)^T on bf16 MFMA, fp32 accumulation.
//
// Replaces the reference's prefill kernel (src/mlx_tree_spec/qmm_packed.py:561-725: MLX's
// affine_qmm_t_nax with a packed-layout loader). Same arithmetic: per K step, each weight of the
// BN x BK block is dequantized once to bf16 (qmm_packed.py:629-637) into LDS and multiplied with
// the BM x BK activation block; accumulation in fp32; bf16 out.
//
// Geometry: BM = BN = 256, BK = 64 (one quantization group per K step), 4 waves in a 2 x 2
// arrangement, each wave a 128 x 128 block of 4 x 4 MFMA 32x32x16 tiles (256 fp32 accumulators
// per lane). LDS holds two stages of [256][64 + 8] bf16 for the activations and for the
// dequantized weights (147 KB); the next stage is prefetched into registers during the MFMAs of
// the current one. Workgroup ids are remapped so that consecutive tiles land on one XCD and tiles
// are walked in groups of 4 row tiles, so a group shares weight and activation blocks in L2.
#include "qmm4_common.h"
#include "qmm4_kernels.h"

namespace qmm4 {

namespace {

constexpr int BM = 256, BN = 256, BK = 64, LDK = BK + 8;  // LDS row pitch in bf16
constexpr int kThreads = 256;
constexpr int kGroupM = 4;

struct GemmParams {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int M, N, K;
  int tiles_m, tiles_n;
};

__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmParams P) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* As = smem;                    // [2][BM * LDK]
  uint16_t* Bs = smem + 2 * BM * LDK;     // [2][BN * LDK]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Tile id: XCD-contiguous remap, then grouped row-major walk.
  const int G = gridDim.x;
  int id = blockIdx.x;
  if ((G & 7) == 0) id = (id & 7) * (G >> 3) + (id >> 3);
  const int per_group = kGroupM * P.tiles_n;
  const int group = id / per_group;
  const int first_m = group * kGroupM;
  const int gm = min(kGroupM, P.tiles_m - first_m);
  const int in_group = id - group * per_group;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;
  const int m0 = tm * BM, n0 = tn * BN;

  const size_t KW = (size_t)(P.K >> 3), KG = (size_t)(P.K >> 6);
  const int nk = P.K / BK;

  // Loader roles. Activations: thread owns 16-B chunk (tid & 7) of rows (tid >> 3) + 32*j.
  const int a_kc = tid & 7;
  const int a_r0 = tid >> 3;
  // Weights: thread owns column n0 + tid, the 8 words (one group) of each K step.
  const int bn_col = n0 + tid;
  const bool b_ok = bn_col < P.N;
  const uint32_t* wrow = P.w + (b_ok ? (size_t)bn_col : 0) * KW;
  const uint16_t* srow = P.s + (b_ok ? (size_t)bn_col : 0) * KG;
  const uint16_t* brow = P.b + (b_ok ? (size_t)bn_col : 0) * KG;

  u32x4 ra[8];
  u32x4 rw[2];
  uint32_t rs = 0, rbias = 0;

  auto load_stage = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = m0 + a_r0 + 32 * j;
      if (r < P.M)
        ra[j] = *reinterpret_cast<const u32x4*>(P.x + (size_t)r * P.K + k0 + a_kc * 8);
      else
        ra[j] = u32x4{0u, 0u, 0u, 0u};
    }
    if (b_ok) {
      rw[0] = *reinterpret_cast<const u32x4*>(wrow + (size_t)kt * 8);
      rw[1] = *reinterpret_cast<const u32x4*>(wrow + (size_t)kt * 8 + 4);
      rs = srow[kt];
      rbias = brow[kt];
    } else {
      rw[0] = rw[1] = u32x4{0u, 0u, 0u, 0u};
      rs = rbias = 0;
    }
  };

  auto store_stage = [&](int st) {
    uint16_t* as = As + st * BM * LDK;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<u32x4*>(as + (a_r0 + 32 * j) * LDK + a_kc * 8) = ra[j];
    uint16_t* bs = Bs + st * BN * LDK + tid * LDK;
    const float sf = bf16_to_f32(rs), bf = bf16_to_f32(rbias), s16 = sf * 0.0625f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<u32x4*>(bs + j * 8) = dequant_word(rw[j >> 2][j & 3], sf, s16, bf);
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  load_stage(0);
  store_stage(0);
  __syncthreads();

  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt & 1;
    if (kt + 1 < nk) load_stage(kt + 1);
    const uint16_t* as = As + st * BM * LDK + (wm * 128 + lrow) * LDK + lk;
    const uint16_t* bs = Bs + st * BN * LDK + (wn * 128 + lrow) * LDK + lk;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8 Af[4], Bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        Af[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(as + i * 32 * LDK + ks * 16));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        Bf[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(bs + j * 32 * LDK + ks * 16));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Mfma<32>::mma(Af[i], Bf[j], acc[i][j]);
    }
    if (kt + 1 < nk) store_stage(st ^ 1);
    __syncthreads();
  }

  // Epilogue: fp32 -> bf16, row-guarded for the M tail and column-guarded for the N tail.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 128 + j * 32 + lrow;
      if (n >= P.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 128 + i * 32 + Mfma<32>::row(lane, r);
        if (m < P.M) P.y[(size_t)m * P.N + n] = (uint16_t)(pack_bf16x2(acc[i][j][r], 0.0f) & 0xFFFFu);
      }
    }
}

constexpr size_t kSmemBytes = (size_t)2 * (BM + BN) * LDK * sizeof(uint16_t);

}  // namespace

hipError_t launch_gemm(const uint16_t* x, const uint32_t* w, const uint16_t* s,
                       const uint16_t* b, uint16_t* y, int M, int N, int K, hipStream_t stream) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSmemBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  GemmParams P;
  P.x = x; P.w = w; P.s = s; P.b = b; P.y = y;
  P.M = M; P.N = N; P.K = K;
  P.tiles_m = (M + BM - 1) / BM;
  P.tiles_n = (N + BN - 1) / BN;
  const unsigned blocks = (unsigned)(P.tiles_m * P.tiles_n);
  hipLaunchKernelGGL(gemm_kernel, dim3(blocks), dim3(kThreads), kSmemBytes, stream, P);
  return hipGetLastError();
}

}  // namespace qmm4
