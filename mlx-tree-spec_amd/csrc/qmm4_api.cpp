// C ABI of the packed 4-bit affine quantized matmul (declared in include/qmm4.h).
//
// Mirrors the reference's drop-in boundary: the quantized-linear call
// mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size=64, bits=4)
// (src/mlx_tree_spec/packed_linear.py:97) and its dispatch by row count
// (packed_linear._call, packed_linear.py:83-104), with the argument checks the reference makes
// with asserts and eligibility tests (qmm_packed.py:227, 705; packed_linear.py:49-58) turned into
// error codes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "qmm4.h"
#include "qmm4_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(QMM4_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Per-device facts, queried once.
struct DeviceInfo {
  int cus = 0;
  int occ[qmm4::kSkinnyVariants] = {};  // resident skinny workgroups per CU, per variant
  int vocc[qmm4::kVerifyVariants] = {};  // resident verify workgroups per CU, per variant
};

// Split-K workspace for one (device, stream): [counters | partials]. Counters are zeroed when the
// buffer is (re)allocated and every launch leaves them at zero.
struct Workspace {
  void* base = nullptr;
  size_t counter_bytes = 0;
  size_t partial_bytes = 0;
};

std::mutex g_mu;
std::map<int, DeviceInfo> g_dev;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

int device_info(int dev, DeviceInfo** out) {
  auto it = g_dev.find(dev);
  if (it == g_dev.end()) {
    DeviceInfo d;
    hipError_t e = hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(MultiprocessorCount)");
    for (int v = 0; v < qmm4::kSkinnyVariants; ++v) d.occ[v] = qmm4::skinny_occupancy(v);
    for (int v = 0; v < qmm4::kVerifyVariants; ++v) d.vocc[v] = qmm4::verify_occupancy(v);
    it = g_dev.emplace(dev, d).first;
  }
  *out = &it->second;
  return QMM4_OK;
}

int get_workspace(int dev, hipStream_t stream, size_t counter_bytes, size_t partial_bytes,
                  uint32_t** cnt, float** part) {
  Workspace& ws = g_ws[std::make_pair(dev, stream)];
  if (ws.base == nullptr || ws.counter_bytes < counter_bytes || ws.partial_bytes < partial_bytes) {
    const size_t cb = std::max(ws.counter_bytes, (counter_bytes + 255) / 256 * 256);
    const size_t pb = std::max(ws.partial_bytes, (partial_bytes + 255) / 256 * 256);
    if (ws.base != nullptr) {
      hipError_t e = hipStreamSynchronize(stream);
      if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
      (void)hipFree(ws.base);
      ws = Workspace();
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, cb + pb);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return fail(QMM4_ERR_NOMEM, "workspace allocation of %zu bytes failed: %s", cb + pb,
                  hipGetErrorString(e));
    }
    // Counters start at zero (each launch leaves them at zero). Cleared by a kernel rather than
    // hipMemsetAsync, which misbehaves when recorded into a captured graph.
    e = qmm4::launch_zero_u32(static_cast<uint32_t*>(p), cb / sizeof(uint32_t), stream);
    if (e != hipSuccess) {
      (void)hipFree(p);
      return hip_fail(e, "workspace counter clear");
    }
    ws.base = p;
    ws.counter_bytes = cb;
    ws.partial_bytes = pb;
  }
  *cnt = static_cast<uint32_t*>(ws.base);
  *part = reinterpret_cast<float*>(static_cast<char*>(ws.base) + ws.counter_bytes);
  return QMM4_OK;
}

// Scratch for one (device, stream) that an entry point fills and reads back in the same call (the
// gate+up projection before its separate epilogue pass). Grown on demand; the old buffer is freed
// once the stream has finished with it.
struct Scratch {
  void* base = nullptr;
  size_t bytes = 0;
};
std::map<std::pair<int, hipStream_t>, Scratch> g_scratch;

int get_scratch(int dev, hipStream_t stream, size_t bytes, void** out) {
  Scratch& sc = g_scratch[std::make_pair(dev, stream)];
  if (sc.base == nullptr || sc.bytes < bytes) {
    const size_t nb = std::max(sc.bytes, (bytes + 255) / 256 * 256);
    if (sc.base != nullptr) {
      hipError_t e = hipStreamSynchronize(stream);
      if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
      (void)hipFree(sc.base);
      sc = Scratch();
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, nb);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return fail(QMM4_ERR_NOMEM, "scratch allocation of %zu bytes failed: %s", nb, hipGetErrorString(e));
    }
    sc.base = p;
    sc.bytes = nb;
  }
  *out = sc.base;
  return QMM4_OK;
}

int check_format(int group_size, int bits, int transpose) {
  if (bits != 4) return fail(QMM4_ERR_UNSUPPORTED, "bits=%d: only 4-bit codes are supported", bits);
  if (group_size != 64)
    return fail(QMM4_ERR_UNSUPPORTED, "group_size=%d: only group_size=64 is supported", group_size);
  if (transpose != 1)
    return fail(QMM4_ERR_UNSUPPORTED, "transpose=%d: only transpose=True (y = x @ w.T) is supported",
                transpose);
  return QMM4_OK;
}

int check_qmm_args(const void* x, const uint32_t* w, const void* scales, const void* biases, const void* y,
                   int64_t M, int64_t N, int64_t K, int group_size, int bits, int transpose);
int dispatch_qmm(int dev, DeviceInfo* di, const void* x, const uint32_t* w, const void* scales,
                 const void* biases, void* y, int64_t M, int64_t N, int64_t K, hipStream_t stream);

}  // namespace

extern "C" {

const char* qmm4_last_error(void) { return g_last_error.c_str(); }

int qmm4_abi_version(void) { return 1; }

int qmm4_affine_bf16(const void* x, const uint32_t* w, const void* scales, const void* biases,
                     void* y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                     int transpose, void* hip_stream) {
  g_last_error.clear();
  int rc = check_qmm_args(x, w, scales, biases, y, M, N, K, group_size, bits, transpose);
  if (rc || M == 0 || N == 0) return rc;
  hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceInfo* di = nullptr;
  rc = device_info(dev, &di);
  if (rc) return rc;
  return dispatch_qmm(dev, di, x, w, scales, biases, y, M, N, K, stream);
}

int qmm4_gate_up_silu_bf16(const void* x, const uint32_t* w, const void* scales, const void* biases,
                           void* y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                           int transpose, void* hip_stream) {
  g_last_error.clear();
  int rc = check_qmm_args(x, w, scales, biases, y, M, N, K, group_size, bits, transpose);
  if (rc) return rc;
  if (N % 32 != 0)
    return fail(QMM4_ERR_INVALID, "N=%lld must be a multiple of 32 (gate and up halves of whole 16-row blocks)",
                (long long)N);
  if (M == 0 || N == 0) return QMM4_OK;
  if (!aligned(y, 16)) return fail(QMM4_ERR_INVALID, "y must be 16-byte aligned");
  hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceInfo* di = nullptr;
  rc = device_info(dev, &di);
  if (rc) return rc;
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint16_t* sb = static_cast<const uint16_t*>(scales);
  const uint16_t* bb = static_cast<const uint16_t*>(biases);
  uint16_t* yb = static_cast<uint16_t*>(y);
#ifndef QMM4_NO_ROWSPLIT
  // Decode rows: the row-split kernel with the epilogue fused (one launch, no [M, N] round trip).
  qmm4::RowSplitPlan rplan;
  if (qmm4::rowsplit_plan((int)M, (int)N, (int)K, di->cus, true, &rplan)) {
    uint32_t* cnt = nullptr;
    float* part = nullptr;
    if (rplan.KS > 1) {
      rc = get_workspace(dev, stream, (size_t)rplan.ranges * sizeof(uint32_t), rplan.part_bytes, &cnt, &part);
      if (rc) return rc;
    }
    e = qmm4::launch_rowsplit(rplan, xb, w, sb, bb, yb, part, cnt, (int)M, (int)N, (int)K, stream);
    if (e != hipSuccess) return hip_fail(e, "fused gate+up row-split kernel launch");
    return QMM4_OK;
  }
#endif
  // Otherwise the projection into a library-held [M, N] buffer, then the epilogue as its own pass.
  void* t = nullptr;
  rc = get_scratch(dev, stream, (size_t)M * (size_t)N * sizeof(uint16_t), &t);
  if (rc) return rc;
  rc = dispatch_qmm(dev, di, x, w, scales, biases, t, M, N, K, stream);
  if (rc) return rc;
  e = qmm4::launch_silu_mul(static_cast<const uint16_t*>(t), yb, (int)M, (int)(N / 2), stream);
  if (e != hipSuccess) return hip_fail(e, "silu-mul kernel launch");
  return QMM4_OK;
}

}  // extern "C"

namespace {

int check_qmm_args(const void* x, const uint32_t* w, const void* scales, const void* biases, const void* y,
                   int64_t M, int64_t N, int64_t K, int group_size, int bits, int transpose) {
  int rc = check_format(group_size, bits, transpose);
  if (rc) return rc;
  if (M < 0 || N < 0 || K <= 0)
    return fail(QMM4_ERR_INVALID, "invalid shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                (long long)K);
  if (K % 128 != 0)
    return fail(QMM4_ERR_INVALID, "K=%lld must be a multiple of 128", (long long)K);
  if (N % 16 != 0)
    return fail(QMM4_ERR_INVALID, "N=%lld must be a multiple of 16", (long long)N);
  if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30))
    return fail(QMM4_ERR_INVALID, "shape M=%lld N=%lld K=%lld exceeds 2^30", (long long)M,
                (long long)N, (long long)K);
  if (M == 0 || N == 0) return QMM4_OK;
  if (!x || !w || !scales || !biases || !y) return fail(QMM4_ERR_INVALID, "null pointer argument");
  if (!aligned(x, 16) || !aligned(w, 16))
    return fail(QMM4_ERR_INVALID, "x and w must be 16-byte aligned");
  if (!aligned(scales, 4) || !aligned(biases, 4) || !aligned(y, 2))
    return fail(QMM4_ERR_INVALID, "scales and biases must be 4-byte aligned and y 2-byte aligned");
  // Kernels address w, x and y with 32-bit byte offsets (tiles may reach 256 rows or columns past
  // the end, which read as zero / are dropped), so each stays below 4 GiB with that margin.
  if ((unsigned long long)(N + 256) * (unsigned long long)K / 2 >= (1ULL << 32))
    return fail(QMM4_ERR_INVALID, "w of %lld x %lld codes exceeds 4 GiB", (long long)N, (long long)K);
  if ((unsigned long long)(M + 256) * (unsigned long long)K * 2 >= (1ULL << 32) ||
      (unsigned long long)(M + 256) * (unsigned long long)N * 2 >= (1ULL << 32))
    return fail(QMM4_ERR_INVALID, "x [%lld, %lld] or y [%lld, %lld] exceeds 4 GiB", (long long)M,
                (long long)K, (long long)M, (long long)N);
  return QMM4_OK;
}

// The kernel choice for y = x @ dequant(w)^T (arguments already checked, M and N > 0, g_mu held).
int dispatch_qmm(int dev, DeviceInfo* di, const void* x, const uint32_t* w, const void* scales,
                 const void* biases, void* y, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint16_t* sb = static_cast<const uint16_t*>(scales);
  const uint16_t* bb = static_cast<const uint16_t*>(biases);
  uint16_t* yb = static_cast<uint16_t*>(y);
  hipError_t e;
  int rc;

  if (M > 64) {
    e = qmm4::launch_gemm(xb, w, sb, bb, yb, (int)M, (int)N, (int)K, di->cus, stream);
    if (e != hipSuccess) return hip_fail(e, "gemm kernel launch");
    return QMM4_OK;
  }

#ifndef QMM4_NO_ROWSPLIT
  // Up to 4 rows and enough output columns to give every CU its own rows (whole K, or K in 2 or 4
  // slices when N is small): the row-split kernel.
  qmm4::RowSplitPlan rplan;
  if (qmm4::rowsplit_plan((int)M, (int)N, (int)K, di->cus, false, &rplan)) {
    uint32_t* rcnt = nullptr;
    float* rpart = nullptr;
    if (rplan.KS > 1) {
      rc = get_workspace(dev, stream, (size_t)rplan.ranges * sizeof(uint32_t), rplan.part_bytes, &rcnt, &rpart);
      if (rc) return rc;
    }
    e = qmm4::launch_rowsplit(rplan, xb, w, sb, bb, yb, rpart, rcnt, (int)M, (int)N, (int)K, stream);
    if (e != hipSuccess) return hip_fail(e, "row-split kernel launch");
    return QMM4_OK;
  }
#endif

  // A unit spans V super-steps; V must divide K / 128, and a unit's 2V scales (biases) of a row
  // are read with one 4V-byte load, so the scale and bias pointers must be 4V-byte aligned.
  int vmax = 4;
  const long long ks = K / 128;
  while (vmax > 1 && (ks % vmax != 0 || !aligned(scales, 4 * vmax) || !aligned(biases, 4 * vmax))) vmax >>= 1;
#ifndef QMM4_ROWPHASE_MIN_M
#define QMM4_ROWPHASE_MIN_M 5
#endif
#ifndef QMM4_NO_ROWPHASE
  // The row-phase kernel stages scale rows with 16-byte loads. It serves more than 16 rows, and
  // up to 16 rows when its plan fills at least half the CUs; fewer rows over a small N with K
  // split too few ways go to the verify kernel (its stream-K ranges balance better when there is
  // little work per CU).
#ifndef QMM4_ROWPHASE_NARROW_MIN_M
#define QMM4_ROWPHASE_NARROW_MIN_M 17
#endif
  if (M >= QMM4_ROWPHASE_MIN_M && aligned(scales, 16) && aligned(biases, 16) && K % 512 == 0) {
    qmm4::RowPhasePlan pplan;
    if (qmm4::rowphase_plan((int)M, (int)N, (int)K, di->cus, &pplan) &&
        (pplan.wide || M >= QMM4_ROWPHASE_NARROW_MIN_M || 2 * pplan.blocks >= di->cus)) {
      uint32_t* pcnt = nullptr;
      float* ppart = nullptr;
      if (pplan.S > 1) {
        rc = get_workspace(dev, stream, 0, pplan.part_bytes, &pcnt, &ppart);
        if (rc) return rc;
      }
      e = qmm4::launch_rowphase(pplan, xb, w, sb, bb, yb, ppart, (int)M, (int)N, (int)K, stream);
      if (e != hipSuccess) return hip_fail(e, "row-phase kernel launch");
      return QMM4_OK;
    }
  }
#endif
#ifndef QMM4_VERIFY_MIN_M
#define QMM4_VERIFY_MIN_M 5
#endif
#ifndef QMM4_NO_VERIFY
  if (M >= QMM4_VERIFY_MIN_M) {
    qmm4::VerifyPlan vplan;
    const int vv = qmm4::verify_variant((int)M, vmax);
    if (qmm4::verify_plan((int)M, (int)N, (int)K, vmax, di->cus, di->vocc[vv], &vplan)) {
      uint32_t* vcnt = nullptr;
      float* vpart = nullptr;
      rc = get_workspace(dev, stream, (size_t)vplan.tiles * sizeof(uint32_t),
                         vplan.part_bytes, &vcnt, &vpart);
      if (rc) return rc;
      e = qmm4::launch_verify(vplan, xb, w, sb, bb, yb, vpart, vcnt, (int)M, (int)N, (int)K, stream);
      if (e != hipSuccess) return hip_fail(e, "verify kernel launch");
      return QMM4_OK;
    }
  }
#endif
  qmm4::SkinnyPlan plan;
  plan.variant = qmm4::skinny_variant((int)M, vmax, &plan.tile_cols, &plan.steps_v);
  plan.tiles = (int)((N + plan.tile_cols - 1) / plan.tile_cols);
  plan.units = (long long)plan.tiles * (ks / plan.steps_v);
  // One resident workgroup per slot, but at least 2 units each: a tile split over fewer units
  // per workgroup costs more in fp32 partials than it gains in balance. Three workgroups per CU
  // (12 waves) measured faster than four on every skinny shape from M=1 to M=64.
#ifndef QMM4_SKINNY_MAX_WG_PER_CU
#define QMM4_SKINNY_MAX_WG_PER_CU 3
#endif
  auto blocks_for = [&](int variant) {
    long long slots = (long long)di->cus * std::min(di->occ[variant], QMM4_SKINNY_MAX_WG_PER_CU);
    const long long cap = std::max(1LL, plan.units / 2);
    if (slots > cap) slots = cap;
    if (slots < 1) slots = 1;
    return (int)(plan.units < slots ? plan.units : slots);
  };
  plan.blocks = blocks_for(plan.variant);
#ifndef QMM4_SKINNY_NO_RESIDENT_X
  // Resident x when every workgroup's range fits the twin's x slots: a range of u units touches
  // min(u, steps per tile) distinct steps, and no range holds more than ceil(units / blocks) units.
  int xslots = 0;
  const int twin = qmm4::skinny_resident_twin(plan.variant, &xslots);
  if (twin >= 0) {
    const int tb = blocks_for(twin);
    const long long per_wg = (plan.units + tb - 1) / tb;
    const long long ns = ks / plan.steps_v;
    if (std::min(per_wg, ns) <= xslots) {
      plan.variant = twin;
      plan.blocks = tb;
    }
  }
#endif

  uint32_t* cnt = nullptr;
  float* part = nullptr;
  rc = get_workspace(dev, stream, (size_t)plan.tiles * sizeof(uint32_t),
                     (size_t)plan.blocks * 2 * (size_t)M * plan.tile_cols * sizeof(float), &cnt, &part);
  if (rc) return rc;
  e = qmm4::launch_skinny(plan, xb, w, sb, bb, yb, part, cnt, (int)M, (int)N, (int)K, stream);
  if (e != hipSuccess) return hip_fail(e, "skinny kernel launch");
  return QMM4_OK;
}

}  // namespace

extern "C" {

int qmm4_add_rms_norm_bf16(const void* x, const void* r, const void* weight, void* h_out, void* n_out,
                           int64_t rows, int64_t D, float eps, void* hip_stream) {
  g_last_error.clear();
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > qmm4::add_rms_norm_max_d())
    return fail(QMM4_ERR_INVALID, "invalid shape rows=%lld D=%lld (D must be a positive multiple of 8, at most %d)",
                (long long)rows, (long long)D, qmm4::add_rms_norm_max_d());
  if (rows > (1LL << 30)) return fail(QMM4_ERR_INVALID, "rows=%lld exceeds 2^30", (long long)rows);
  if (!(eps >= 0.0f) || eps > 1e30f) return fail(QMM4_ERR_INVALID, "eps must be finite and >= 0");
  if (rows == 0) return QMM4_OK;
  if (!x || !r || !weight || !h_out || !n_out) return fail(QMM4_ERR_INVALID, "null pointer argument");
  if (!aligned(x, 16) || !aligned(r, 16) || !aligned(weight, 16) || !aligned(h_out, 16) || !aligned(n_out, 16))
    return fail(QMM4_ERR_INVALID, "x, r, weight, h_out and n_out must be 16-byte aligned");
  hipError_t e = qmm4::launch_add_rms_norm(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(r),
                                           static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(h_out),
                                           static_cast<uint16_t*>(n_out), (int)rows, (int)D, eps,
                                           static_cast<hipStream_t>(hip_stream));
  if (e != hipSuccess) return hip_fail(e, "add-rms-norm kernel launch");
  return QMM4_OK;
}

int dequant4_affine_bf16(const uint32_t* w, const void* scales, const void* biases, void* out,
                         int64_t N, int64_t K, int group_size, int bits, void* hip_stream) {
  g_last_error.clear();
  int rc = check_format(group_size, bits, 1);
  if (rc) return rc;
  if (N < 0 || K <= 0 || K % 64 != 0)
    return fail(QMM4_ERR_INVALID, "invalid shape N=%lld K=%lld (K must be a positive multiple of 64)",
                (long long)N, (long long)K);
  if (N == 0) return QMM4_OK;
  if (!w || !scales || !biases || !out) return fail(QMM4_ERR_INVALID, "null pointer argument");
  if (!aligned(w, 16) || !aligned(out, 16))
    return fail(QMM4_ERR_INVALID, "w and out must be 16-byte aligned");
  if (!aligned(scales, 2) || !aligned(biases, 2))
    return fail(QMM4_ERR_INVALID, "scales and biases must be 2-byte aligned");
  hipError_t e = qmm4::launch_dequant(w, static_cast<const uint16_t*>(scales),
                                      static_cast<const uint16_t*>(biases),
                                      static_cast<uint16_t*>(out), N, K,
                                      static_cast<hipStream_t>(hip_stream));
  if (e != hipSuccess) return hip_fail(e, "dequant kernel launch");
  return QMM4_OK;
}

}  // extern "C"
