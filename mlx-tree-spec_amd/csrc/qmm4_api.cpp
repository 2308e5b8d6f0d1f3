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
#include <cstdint>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "qmm4.h"
#include "qmm4_dispatch.h"
#include "qmm4_kernels.h"

namespace qmm4 {

namespace {
thread_local std::string g_last_error;
}  // namespace

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_error(hipError_t e, const char* what) {
  return set_error(QMM4_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

void clear_error() { g_last_error.clear(); }

std::mutex& api_mutex() {
  static std::mutex mu;
  return mu;
}

struct DeviceInfo {
  int cus = 0;
  int occ[kSkinnyVariants] = {};   // resident skinny workgroups per CU, per variant
  int vocc[kVerifyVariants] = {};  // resident verify workgroups per CU, per variant
};

int device_info(int dev, DeviceInfo** out) {
  static std::map<int, DeviceInfo> devs;
  auto it = devs.find(dev);
  if (it == devs.end()) {
    DeviceInfo d;
    hipError_t e = hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_error(e, "hipDeviceGetAttribute(MultiprocessorCount)");
    for (int v = 0; v < kSkinnyVariants; ++v) d.occ[v] = skinny_occupancy(v);
    for (int v = 0; v < kVerifyVariants; ++v) d.vocc[v] = verify_occupancy(v);
    it = devs.emplace(dev, d).first;
  }
  *out = &it->second;
  return QMM4_OK;
}

int device_cus(const DeviceInfo* di) { return di->cus; }

}  // namespace qmm4

namespace {

using qmm4::hip_error;
using qmm4::set_error;

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Whether the byte ranges [a, a + an) and [b, b + bn) share a byte (empty ranges share none).
bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return an > 0 && bn > 0 && pa < pb + bn && pb < pa + an;
}

// Whether work enqueued on `stream` now is being recorded into a graph (then nothing may be
// allocated, freed or synchronized, and any buffer it uses must outlive the graph).
int stream_capturing(hipStream_t stream, bool* capturing) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &st);
  if (e != hipSuccess) return hip_error(e, "hipStreamIsCapturing");
  *capturing = st != hipStreamCaptureStatusNone;
  return QMM4_OK;
}

// A device buffer that is grown on demand for one (device, stream). A buffer that a captured call
// used may be replayed by a graph at any later time, so it is never freed: when it must grow
// afterwards it is retired (kept until the process ends) and a new one is allocated. Growth while
// the stream is capturing is refused (no allocation can be recorded).
struct Buffer {
  void* base = nullptr;
  size_t bytes = 0;
  bool captured = false;
};

std::vector<void*>& retired_buffers() {
  static std::vector<void*> r;
  return r;
}

// Makes `buf` hold at least `bytes` (api_mutex held); `replace` forces a new buffer even when the
// old one is large enough. `zero_bytes` leading bytes of a new buffer are cleared with a kernel
// (not hipMemsetAsync, which misbehaves when replayed from a graph).
int grow(Buffer& buf, size_t bytes, bool replace, size_t zero_bytes, hipStream_t stream, const char* what) {
  bool capturing = false;
  int rc = stream_capturing(stream, &capturing);
  if (rc) return rc;
  if (buf.base == nullptr || buf.bytes < bytes || replace) {
    if (capturing)
      return set_error(QMM4_ERR_CAPTURE,
                       "%s of %zu bytes needed while the stream is being captured (it holds %zu): call once "
                       "with this shape on this stream before capturing",
                       what, bytes, buf.bytes);
    const size_t nb = std::max(buf.bytes, (bytes + 255) / 256 * 256);
    if (buf.base != nullptr) {
      if (buf.captured) {
        retired_buffers().push_back(buf.base);
      } else {
        hipError_t e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize");
        (void)hipFree(buf.base);
      }
      buf = Buffer();
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, nb);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return set_error(QMM4_ERR_NOMEM, "%s allocation of %zu bytes failed: %s", what, nb, hipGetErrorString(e));
    }
    if (zero_bytes > 0) {
      e = qmm4::launch_zero_u32(static_cast<uint32_t*>(p), zero_bytes / sizeof(uint32_t), stream);
      if (e != hipSuccess) {
        (void)hipFree(p);
        return hip_error(e, "workspace counter clear");
      }
    }
    buf.base = p;
    buf.bytes = nb;
  }
  if (capturing) buf.captured = true;
  return QMM4_OK;
}

// The library-held buffers of one (device, stream): the split-K workspace ([counters | partials])
// and the scratch of the two-pass gate+up epilogue.
struct StreamBuffers {
  Buffer ws;
  size_t counter_bytes = 0;  // the workspace's counter region; partials follow it
  Buffer scratch;
};

std::map<std::pair<int, hipStream_t>, StreamBuffers>& stream_buffers() {
  static std::map<std::pair<int, hipStream_t>, StreamBuffers> m;
  return m;
}

class StreamWorkspace final : public qmm4::WorkspaceSource {
 public:
  StreamWorkspace(int dev, hipStream_t stream) : stream_(stream), sb_(stream_buffers()[std::make_pair(dev, stream)]) {}

  int get(size_t counter_bytes, size_t partial_bytes, uint32_t** cnt, float** part) override {
    const size_t need_cb = (counter_bytes + 255) / 256 * 256;
    const size_t have_pb = sb_.ws.bytes > sb_.counter_bytes ? sb_.ws.bytes - sb_.counter_bytes : 0;
    const bool fits = sb_.ws.base != nullptr && need_cb <= sb_.counter_bytes && partial_bytes <= have_pb;
    // A new buffer keeps the larger of the old and the new needs, so that alternating shapes do
    // not reallocate on every call.
    const size_t cb = fits ? sb_.counter_bytes : std::max(need_cb, sb_.counter_bytes);
    const size_t pb = std::max(partial_bytes, have_pb);
    int rc = grow(sb_.ws, cb + pb, !fits, cb, stream_, "split-K workspace");
    if (rc) return rc;
    sb_.counter_bytes = cb;
    *cnt = static_cast<uint32_t*>(sb_.ws.base);
    *part = reinterpret_cast<float*>(static_cast<char*>(sb_.ws.base) + cb);
    return QMM4_OK;
  }

  size_t capacity() const override { return SIZE_MAX; }

  int get_scratch(size_t bytes, void** out) override {
    int rc = grow(sb_.scratch, bytes, false, 0, stream_, "gate+up scratch");
    if (rc) return rc;
    *out = sb_.scratch.base;
    return QMM4_OK;
  }

 private:
  hipStream_t stream_;
  StreamBuffers& sb_;
};

int check_format(int group_size, int bits, int transpose) {
  if (bits != 4) return set_error(QMM4_ERR_UNSUPPORTED, "bits=%d: only 4-bit codes are supported", bits);
  if (group_size != 64)
    return set_error(QMM4_ERR_UNSUPPORTED, "group_size=%d: only group_size=64 is supported", group_size);
  if (transpose != 1)
    return set_error(QMM4_ERR_UNSUPPORTED, "transpose=%d: only transpose=True (y = x @ w.T) is supported",
                     transpose);
  return QMM4_OK;
}

int current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return hip_error(e, "hipGetDevice");
  return QMM4_OK;
}

}  // namespace

extern "C" {

const char* qmm4_last_error(void) { return qmm4::g_last_error.c_str(); }

int qmm4_abi_version(void) { return 1; }

int qmm4_affine_bf16(const void* x, const uint32_t* w, const void* scales, const void* biases,
                     void* y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                     int transpose, void* hip_stream) {
  qmm4::clear_error();
  int rc = qmm4::check_qmm_args(x, w, scales, biases, y, M, N, K, group_size, bits, transpose);
  if (rc || M == 0 || N == 0) return rc;
  hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  int dev = 0;
  if ((rc = current_device(&dev))) return rc;
  std::lock_guard<std::mutex> lock(qmm4::api_mutex());
  qmm4::DeviceInfo* di = nullptr;
  if ((rc = qmm4::device_info(dev, &di))) return rc;
  StreamWorkspace ws(dev, stream);
  return qmm4::dispatch_qmm(di, x, w, scales, biases, y, M, N, K, stream, ws);
}

int qmm4_gate_up_silu_bf16(const void* x, const uint32_t* w, const void* scales, const void* biases,
                           void* y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                           int transpose, void* hip_stream) {
  qmm4::clear_error();
  int rc = qmm4::check_qmm_args(x, w, scales, biases, y, M, N, K, group_size, bits, transpose);
  if (rc) return rc;
  if (N % 32 != 0)
    return set_error(QMM4_ERR_INVALID, "N=%lld must be a multiple of 32 (gate and up halves of whole 16-row blocks)",
                     (long long)N);
  if (M == 0 || N == 0) return QMM4_OK;
  if (!aligned(y, 16)) return set_error(QMM4_ERR_INVALID, "y must be 16-byte aligned");
  hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  int dev = 0;
  if ((rc = current_device(&dev))) return rc;
  std::lock_guard<std::mutex> lock(qmm4::api_mutex());
  qmm4::DeviceInfo* di = nullptr;
  if ((rc = qmm4::device_info(dev, &di))) return rc;
  StreamWorkspace ws(dev, stream);
  return qmm4::dispatch_gate_up_silu(di, x, w, scales, biases, y, M, N, K, stream, ws);
}

}  // extern "C"

namespace qmm4 {

int check_qmm_args(const void* x, const uint32_t* w, const void* scales, const void* biases, const void* y,
                   int64_t M, int64_t N, int64_t K, int group_size, int bits, int transpose) {
  int rc = check_format(group_size, bits, transpose);
  if (rc) return rc;
  if (M < 0 || N < 0 || K <= 0)
    return set_error(QMM4_ERR_INVALID, "invalid shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                     (long long)K);
  if (K % 128 != 0)
    return set_error(QMM4_ERR_INVALID, "K=%lld must be a multiple of 128", (long long)K);
  if (N % 16 != 0)
    return set_error(QMM4_ERR_INVALID, "N=%lld must be a multiple of 16", (long long)N);
  if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30))
    return set_error(QMM4_ERR_INVALID, "shape M=%lld N=%lld K=%lld exceeds 2^30", (long long)M,
                     (long long)N, (long long)K);
  if (M == 0 || N == 0) return QMM4_OK;
  if (!x || !w || !scales || !biases || !y) return set_error(QMM4_ERR_INVALID, "null pointer argument");
  if (!aligned(x, 16) || !aligned(w, 16))
    return set_error(QMM4_ERR_INVALID, "x and w must be 16-byte aligned");
  if (!aligned(scales, 4) || !aligned(biases, 4) || !aligned(y, 2))
    return set_error(QMM4_ERR_INVALID, "scales and biases must be 4-byte aligned and y 2-byte aligned");
  // Kernels address w, x and y with 32-bit byte offsets (tiles may reach 256 rows or columns past
  // the end, which read as zero / are dropped), so each stays below 4 GiB with that margin.
  if ((unsigned long long)(N + 256) * (unsigned long long)K / 2 >= (1ULL << 32))
    return set_error(QMM4_ERR_INVALID, "w of %lld x %lld codes exceeds 4 GiB", (long long)N, (long long)K);
  if ((unsigned long long)(M + 256) * (unsigned long long)K * 2 >= (1ULL << 32) ||
      (unsigned long long)(M + 256) * (unsigned long long)N * 2 >= (1ULL << 32))
    return set_error(QMM4_ERR_INVALID, "x [%lld, %lld] or y [%lld, %lld] exceeds 4 GiB", (long long)M,
                     (long long)K, (long long)M, (long long)N);
  return QMM4_OK;
}

// Past 64 rows the row-phase kernel takes up to kRowPhaseMaxM rows over a small N (its weights are
// dequantized once for all rows), and up to kRowPhaseMaxMNarrow when N is at most
// kRowPhaseNarrowN (the GEMM then has too few 128 x 128 tiles). Measured against the GEMM (A/B,
// interleaved rounds, the model's up and down projections): 65 / 80 / 96 / 112 rows 38.5 / 40.2 /
// 44.2 / 47.4 us against 46.7 / 47.2 / 48.5 / 48.6 us (5120 -> 17408), 35.8 / 36.7 / 40.4 / 44.2
// against 45.5 / 46.5 / 47.8 / 48.8 (17408 -> 5120); at 120-128 rows (one block per wave) 53-74
// against 48-51 us, but 128 x 5120 -> 1024 17.3 against 47.6 us. A wide plan (every workgroup its
// own blocks over all of K) is taken up to kRowPhaseMaxMWide rows when it needs at most one range
// per CU: 65 / 80 / 96 x 5120 -> 34816 57.5 / 64.5 / 71.9 us against 71.8 / 73.3 / 73.5 us on the
// GEMM, 72 x 4096 -> 32768 43.6 against 50.1 us; at 112 rows 80.8 against 74.5 us.
constexpr int kRowPhaseMaxM = 112;
constexpr int kRowPhaseMaxMWide = 96;
constexpr int kRowPhaseMaxMNarrow = 128;
constexpr int kRowPhaseNarrowN = 2048;
// The fused gate+up row-phase plan's ranges hold whole blocks of both halves, so they may hold one
// block more than the projection's (N = 34816 on 256 CUs: 218 ranges of 10 against 242 of 9). From
// 17 rows and up to this M x K the saved epilogue pass outweighs that block (A/B, N = 34816):
// 24 x 16384 102.7 against 106.1 us, 48 x 10240 90.0 / 91.8, 96 x 5120 73.3 / 74.5; past it
// 80 x 8192 94.6 / 94.0, 64 x 16384 153.9 / 153.3; and 12 x 20480 113.5 / 108.1 (12 rows draw more
// of their time from HBM, where the 24 idle CUs count).
constexpr long long kFusedRowPhaseMaxMK = 1LL << 19;

int dispatch_gate_up_silu(DeviceInfo* di, const void* x, const uint32_t* w, const void* scales,
                          const void* biases, void* y, int64_t M, int64_t N, int64_t K, hipStream_t stream,
                          WorkspaceSource& ws) {
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint16_t* sb = static_cast<const uint16_t*>(scales);
  const uint16_t* bb = static_cast<const uint16_t*>(biases);
  uint16_t* yb = static_cast<uint16_t*>(y);
  hipError_t e;
  int rc;
  // Decode rows: the row-split kernel with the epilogue fused (one launch, no [M, N] round trip).
  RowSplitPlan rplan;
  if (rowsplit_plan((int)M, (int)N, (int)K, di->cus, true, &rplan)) {
    uint32_t* cnt = nullptr;
    float* part = nullptr;
    if (rplan.KS > 1) {
      rc = ws.get((size_t)rplan.ranges * sizeof(uint32_t), rplan.part_bytes, &cnt, &part);
      if (rc) return rc;
    }
    e = launch_rowsplit(rplan, xb, w, sb, bb, yb, part, cnt, (int)M, (int)N, (int)K, stream);
    if (e != hipSuccess) return hip_error(e, "fused gate+up row-split kernel launch");
    return QMM4_OK;
  }
  // Rows the projection would give the row-phase kernel (not the row-split kernel, up to 16 rows):
  // its plan with the epilogue fused, each range holding the same blocks of the gate and up
  // halves. Wide plans (every workgroup its own blocks over all of K) apply it in the kernel's
  // epilogue. Against the projection and the epilogue pass (A/B, 5120 -> 34816): 24 / 32 / 48 /
  // 64 / 80 / 96 rows 40.8 / 42.6 / 52.6 / 59.0 / 66.8 / 73.3 us against 42.6 / 44.0 / 54.2 /
  // 60.6 / 67.7 / 74.5 us, the same bits; 24 x 16384 -> 32768 (ranges of 8 blocks in both) 84.9
  // against 89.1 us. Narrow plans (K split over the CUs) are the projection's own, the epilogue in
  // their reduce kernel.
  if (M >= 5 && M <= kRowPhaseMaxMWide && aligned(scales, 16) && aligned(biases, 16) && K % 512 == 0 &&
      !(M <= 16 && (rowsplit_plan((int)M, (int)N, (int)K, di->cus, false, &rplan) ||
                    (M >= 9 && rowsplit_xreg_plan((int)M, (int)N, (int)K, di->cus, &rplan))))) {
    RowPhasePlan pplan, uplan;
    if (rowphase_plan((int)M, (int)N, (int)K, di->cus, &pplan, true) &&
        rowphase_plan((int)M, (int)N, (int)K, di->cus, &uplan)) {
      const bool take = pplan.wide ? (M <= 64 || pplan.ranges <= di->cus) &&
                                         (pplan.BW <= uplan.BW || (M >= 17 && M * K <= kFusedRowPhaseMaxMK))
                                   : M >= 17 || 2 * pplan.blocks >= di->cus;
      if (take) {
        uint32_t* pcnt = nullptr;
        float* ppart = nullptr;
        if (pplan.S > 1) {
          rc = ws.get(0, pplan.part_bytes, &pcnt, &ppart);
          if (rc) return rc;
        }
        e = launch_rowphase(pplan, xb, w, sb, bb, yb, ppart, (int)M, (int)N, (int)K, stream);
        if (e != hipSuccess) return hip_error(e, "fused gate+up row-phase kernel launch");
        return QMM4_OK;
      }
    }
  }
  // Otherwise the projection into a library-held [M, N] buffer, then the epilogue as its own pass.
  void* t = nullptr;
  rc = ws.get_scratch((size_t)M * (size_t)N * sizeof(uint16_t), &t);
  if (rc) return rc;
  rc = dispatch_qmm(di, x, w, scales, biases, t, M, N, K, stream, ws);
  if (rc) return rc;
  e = launch_silu_mul(static_cast<const uint16_t*>(t), yb, (int)M, (int)(N / 2), stream);
  if (e != hipSuccess) return hip_error(e, "silu-mul kernel launch");
  return QMM4_OK;
}


// The kernel choice for y = x @ dequant(w)^T (arguments already checked, M and N > 0, api_mutex held).
int dispatch_qmm(DeviceInfo* di, const void* x, const uint32_t* w, const void* scales, const void* biases,
                 void* y, int64_t M, int64_t N, int64_t K, hipStream_t stream, WorkspaceSource& ws) {
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint16_t* sb = static_cast<const uint16_t*>(scales);
  const uint16_t* bb = static_cast<const uint16_t*>(biases);
  uint16_t* yb = static_cast<uint16_t*>(y);
  hipError_t e;
  int rc;

  // The row-phase kernel on a plan (K split over the CUs when N is small, with its reduce kernel).
  auto run_rowphase = [&](const RowPhasePlan& pplan) -> int {
    uint32_t* pcnt = nullptr;
    float* ppart = nullptr;
    if (pplan.S > 1) {
      int rc2 = ws.get(0, pplan.part_bytes, &pcnt, &ppart);
      if (rc2) return rc2;
    }
    hipError_t e2 = launch_rowphase(pplan, xb, w, sb, bb, yb, ppart, (int)M, (int)N, (int)K, stream);
    if (e2 != hipSuccess) return hip_error(e2, "row-phase kernel launch");
    return QMM4_OK;
  };

  if (M > 64) {
    // 65-112 rows over a small N (a verify batch past 64 tree nodes, a short prompt tail): the
    // row-phase kernel with 80-112-row x blocks, K split over the CUs; up to 96 rows also a wide
    // plan of at most one range per CU (the MLP's 34816-column gate+up). Its weights are
    // dequantized once for all rows, where the GEMM's 128-row tiles pad these rows to 128.
    if ((M <= kRowPhaseMaxM || (M <= kRowPhaseMaxMNarrow && N <= kRowPhaseNarrowN)) && aligned(scales, 16) &&
        aligned(biases, 16) && K % 512 == 0) {
      RowPhasePlan pplan;
      if (rowphase_plan((int)M, (int)N, (int)K, di->cus, &pplan) &&
          (!pplan.wide || (M <= kRowPhaseMaxMWide && pplan.ranges <= di->cus)))
        return run_rowphase(pplan);
    }
    GemmPlan gplan;
    gemm_plan((int)M, (int)N, (int)K, di->cus, ws.capacity(), sb, bb, &gplan);
    uint32_t* gcnt = nullptr;
    float* gpart = nullptr;
    if (gplan.part_bytes > 0) {
      rc = ws.get(0, gplan.part_bytes, &gcnt, &gpart);
      if (rc) return rc;
    }
    e = launch_gemm(gplan, xb, w, sb, bb, yb, gpart, (int)M, (int)N, (int)K, di->cus, stream);
    if (e != hipSuccess) return hip_error(e, "gemm kernel launch");
    return QMM4_OK;
  }

  // 9 to 16 rows over a small problem (at most 32 weight rows per CU, K <= 6144): the row-split
  // kernel's form with x straight into registers, every load in flight from the start.
  RowSplitPlan rplan;
  if (M >= 9 && rowsplit_xreg_plan((int)M, (int)N, (int)K, di->cus, &rplan)) {
    e = launch_rowsplit(rplan, xb, w, sb, bb, yb, nullptr, nullptr, (int)M, (int)N, (int)K, stream);
    if (e != hipSuccess) return hip_error(e, "row-split kernel launch");
    return QMM4_OK;
  }
  // Up to 16 rows and enough output columns to give every CU its own rows (whole K, or K in a few
  // slices when N is small or x is large): the row-split kernel.
  if (rowsplit_plan((int)M, (int)N, (int)K, di->cus, false, &rplan)) {
    uint32_t* rcnt = nullptr;
    float* rpart = nullptr;
    if (rplan.KS > 1) {
      rc = ws.get((size_t)rplan.ranges * sizeof(uint32_t), rplan.part_bytes, &rcnt, &rpart);
      if (rc) return rc;
    }
    e = launch_rowsplit(rplan, xb, w, sb, bb, yb, rpart, rcnt, (int)M, (int)N, (int)K, stream);
    if (e != hipSuccess) return hip_error(e, "row-split kernel launch");
    return QMM4_OK;
  }

  // A unit spans V super-steps; V must divide K / 128, and a unit's 2V scales (biases) of a row
  // are read with one 4V-byte load, so the scale and bias pointers must be 4V-byte aligned.
  int vmax = 4;
  const long long ks = K / 128;
  while (vmax > 1 && (ks % vmax != 0 || !aligned(scales, 4 * vmax) || !aligned(biases, 4 * vmax))) vmax >>= 1;
  // The row-phase kernel stages scale rows with 16-byte loads. It serves more than 16 rows, and
  // from 5 rows when its plan fills at least half the CUs; fewer rows over a small N with K
  // split too few ways go to the verify kernel (its stream-K ranges balance better when there is
  // little work per CU).
  if (M >= 5 && aligned(scales, 16) && aligned(biases, 16) && K % 512 == 0) {
    RowPhasePlan pplan;
    if (rowphase_plan((int)M, (int)N, (int)K, di->cus, &pplan) &&
        (pplan.wide || M >= 17 || 2 * pplan.blocks >= di->cus))
      return run_rowphase(pplan);
  }
  if (M >= 5) {
    VerifyPlan vplan;
    const int vv = verify_variant((int)M, vmax);
    if (verify_plan((int)M, (int)N, (int)K, vmax, di->cus, di->vocc[vv], &vplan)) {
      uint32_t* vcnt = nullptr;
      float* vpart = nullptr;
      rc = ws.get((size_t)vplan.tiles * sizeof(uint32_t), vplan.part_bytes, &vcnt, &vpart);
      if (rc) return rc;
      e = launch_verify(vplan, xb, w, sb, bb, yb, vpart, vcnt, (int)M, (int)N, (int)K, stream);
      if (e != hipSuccess) return hip_error(e, "verify kernel launch");
      return QMM4_OK;
    }
  }
  SkinnyPlan plan;
  plan.variant = skinny_variant((int)M, vmax, &plan.tile_cols, &plan.steps_v);
  plan.tiles = (int)((N + plan.tile_cols - 1) / plan.tile_cols);
  plan.units = (long long)plan.tiles * (ks / plan.steps_v);
  // One resident workgroup per slot, but at least 2 units each: a tile split over fewer units
  // per workgroup costs more in fp32 partials than it gains in balance. Three workgroups per CU
  // (12 waves) measured faster than four on every skinny shape from M=1 to M=64.
  constexpr int kSkinnyMaxWgPerCu = 3;
  auto blocks_for = [&](int variant) {
    long long slots = (long long)di->cus * std::min(di->occ[variant], kSkinnyMaxWgPerCu);
    const long long cap = std::max(1LL, plan.units / 2);
    if (slots > cap) slots = cap;
    if (slots < 1) slots = 1;
    return (int)(plan.units < slots ? plan.units : slots);
  };
  plan.blocks = blocks_for(plan.variant);
  // Resident x when every workgroup's range fits the twin's x slots: a range of u units touches
  // min(u, steps per tile) distinct steps, and no range holds more than ceil(units / blocks) units.
  int xslots = 0;
  const int twin = skinny_resident_twin(plan.variant, &xslots);
  if (twin >= 0) {
    const int tb = blocks_for(twin);
    const long long per_wg = (plan.units + tb - 1) / tb;
    const long long ns = ks / plan.steps_v;
    if (std::min(per_wg, ns) <= xslots) {
      plan.variant = twin;
      plan.blocks = tb;
    }
  }

  uint32_t* cnt = nullptr;
  float* part = nullptr;
  rc = ws.get((size_t)plan.tiles * sizeof(uint32_t),
              (size_t)plan.blocks * 2 * (size_t)M * plan.tile_cols * sizeof(float), &cnt, &part);
  if (rc) return rc;
  e = launch_skinny(plan, xb, w, sb, bb, yb, part, cnt, (int)M, (int)N, (int)K, stream);
  if (e != hipSuccess) return hip_error(e, "skinny kernel launch");
  return QMM4_OK;
}

int dispatch_norm_qmm(DeviceInfo* di, const void* x, const void* r, const void* weight, float eps, void* h_out,
                      void* n_out, const uint32_t* w, const void* scales, const void* biases, void* y, int64_t M,
                      int64_t N, int64_t K, bool silu_mul, hipStream_t stream, WorkspaceSource& ws) {
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  uint16_t* nb = static_cast<uint16_t*>(n_out);
  hipError_t e;
  int rc;
  // The plan dispatch_qmm / dispatch_gate_up_silu would take for n (the row-split kernel comes first
  // in both for up to 8 rows), launched with the normalising x staging.
  RowSplitPlan rplan;
  if (N > 0 && M <= 4 && rowsplit_plan((int)M, (int)N, (int)K, di->cus, silu_mul, &rplan) &&
      rowsplit_norm_ok(rplan, (int)M, (int)K)) {
    uint32_t* cnt = nullptr;
    float* part = nullptr;
    if (rplan.KS > 1) {
      rc = ws.get((size_t)rplan.ranges * sizeof(uint32_t), rplan.part_bytes, &cnt, &part);
      if (rc) return rc;
    }
    const RowSplitNorm nm{static_cast<const uint16_t*>(r), static_cast<const uint16_t*>(weight),
                          static_cast<uint16_t*>(h_out), nb, eps};
    e = launch_rowsplit(rplan, xb, w, static_cast<const uint16_t*>(scales), static_cast<const uint16_t*>(biases),
                        static_cast<uint16_t*>(y), part, cnt, (int)M, (int)N, (int)K, stream, &nm);
    if (e != hipSuccess) return hip_error(e, "normalising row-split kernel launch");
    return QMM4_OK;
  }
  e = launch_add_rms_norm(xb, static_cast<const uint16_t*>(r), static_cast<const uint16_t*>(weight),
                          static_cast<uint16_t*>(h_out), nb, (int)M, (int)K, eps, stream);
  if (e != hipSuccess) return hip_error(e, "add-rms-norm kernel launch");
  if (N == 0) return QMM4_OK;
  return silu_mul ? dispatch_gate_up_silu(di, n_out, w, scales, biases, y, M, N, K, stream, ws)
                  : dispatch_qmm(di, n_out, w, scales, biases, y, M, N, K, stream, ws);
}

}  // namespace qmm4

extern "C" {

int qmm4_add_rms_norm_qmm_bf16(const void* x, const void* r, const void* weight, float eps, void* h_out,
                               void* n_out, const uint32_t* w, const void* scales, const void* biases, void* y,
                               int64_t M, int64_t N, int64_t K, int group_size, int bits, int transpose,
                               int epilogue, void* hip_stream) {
  qmm4::clear_error();
  int rc = qmm4::check_qmm_args(x, w, scales, biases, y, M, N, K, group_size, bits, transpose);
  if (rc) return rc;
  if (epilogue != QMM4_EPILOGUE_NONE && epilogue != QMM4_EPILOGUE_SILU_MUL)
    return set_error(QMM4_ERR_INVALID, "epilogue=%d: must be QMM4_EPILOGUE_NONE (0) or QMM4_EPILOGUE_SILU_MUL (1)",
                     epilogue);
  const bool silu_mul = epilogue == QMM4_EPILOGUE_SILU_MUL;
  if (silu_mul && N % 32 != 0)
    return set_error(QMM4_ERR_INVALID, "N=%lld must be a multiple of 32 (gate and up halves of whole 16-row blocks)",
                     (long long)N);
  if (K > qmm4::add_rms_norm_max_d())
    return set_error(QMM4_ERR_INVALID, "K=%lld exceeds the norm's largest row of %d", (long long)K,
                     qmm4::add_rms_norm_max_d());
  if (!(eps >= 0.0f) || eps > 1e30f) return set_error(QMM4_ERR_INVALID, "eps must be finite and >= 0");
  if (M == 0) return QMM4_OK;
  if (!x || !r || !weight || !h_out || !n_out || (N > 0 && (!w || !scales || !biases || !y)))
    return set_error(QMM4_ERR_INVALID, "null pointer argument");
  if (!aligned(x, 16) || !aligned(r, 16) || !aligned(weight, 16) || !aligned(h_out, 16) || !aligned(n_out, 16))
    return set_error(QMM4_ERR_INVALID, "x, r, weight, h_out and n_out must be 16-byte aligned");
  if (silu_mul && N > 0 && !aligned(y, 16)) return set_error(QMM4_ERR_INVALID, "y must be 16-byte aligned");
  // Every workgroup of the folded kernel reads all of x and r while the first writes h and n, and
  // every workgroup writes y: the outputs may not overlap the inputs or each other.
  const size_t rows_bytes = (size_t)M * (size_t)K * 2;
  const size_t y_bytes = N > 0 ? (size_t)M * (size_t)(silu_mul ? N / 2 : N) * 2 : 0;
  const size_t w_bytes = (size_t)N * (size_t)K / 2, sb_bytes = (size_t)N * (size_t)(K / 64) * 2;
  const struct {
    const void* p;
    size_t n;
  } in[] = {{x, rows_bytes}, {r, rows_bytes}, {weight, (size_t)K * 2}, {w, w_bytes}, {scales, sb_bytes},
            {biases, sb_bytes}},
    out[] = {{h_out, rows_bytes}, {n_out, rows_bytes}, {y, y_bytes}};
  for (const auto& o : out) {
    for (const auto& i : in)
      if (overlaps(o.p, o.n, i.p, i.n))
        return set_error(QMM4_ERR_INVALID, "h_out, n_out and y may not overlap x, r, weight, w, scales or biases");
    for (const auto& o2 : out)
      if (&o2 != &o && overlaps(o.p, o.n, o2.p, o2.n))
        return set_error(QMM4_ERR_INVALID, "h_out, n_out and y may not overlap each other");
  }
  hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  int dev = 0;
  if ((rc = current_device(&dev))) return rc;
  std::lock_guard<std::mutex> lock(qmm4::api_mutex());
  qmm4::DeviceInfo* di = nullptr;
  if ((rc = qmm4::device_info(dev, &di))) return rc;
  StreamWorkspace ws(dev, stream);
  return qmm4::dispatch_norm_qmm(di, x, r, weight, eps, h_out, n_out, w, scales, biases, y, M, N, K, silu_mul, stream,
                                 ws);
}

int qmm4_add_rms_norm_bf16(const void* x, const void* r, const void* weight, void* h_out, void* n_out,
                           int64_t rows, int64_t D, float eps, void* hip_stream) {
  qmm4::clear_error();
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > qmm4::add_rms_norm_max_d())
    return set_error(QMM4_ERR_INVALID, "invalid shape rows=%lld D=%lld (D must be a positive multiple of 8, at most %d)",
                (long long)rows, (long long)D, qmm4::add_rms_norm_max_d());
  if (rows > (1LL << 30)) return set_error(QMM4_ERR_INVALID, "rows=%lld exceeds 2^30", (long long)rows);
  if (!(eps >= 0.0f) || eps > 1e30f) return set_error(QMM4_ERR_INVALID, "eps must be finite and >= 0");
  if (rows == 0) return QMM4_OK;
  if (!x || !r || !weight || !h_out || !n_out) return set_error(QMM4_ERR_INVALID, "null pointer argument");
  if (!aligned(x, 16) || !aligned(r, 16) || !aligned(weight, 16) || !aligned(h_out, 16) || !aligned(n_out, 16))
    return set_error(QMM4_ERR_INVALID, "x, r, weight, h_out and n_out must be 16-byte aligned");
  hipError_t e = qmm4::launch_add_rms_norm(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(r),
                                           static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(h_out),
                                           static_cast<uint16_t*>(n_out), (int)rows, (int)D, eps,
                                           static_cast<hipStream_t>(hip_stream));
  if (e != hipSuccess) return hip_error(e, "add-rms-norm kernel launch");
  return QMM4_OK;
}

int dequant4_affine_bf16(const uint32_t* w, const void* scales, const void* biases, void* out,
                         int64_t N, int64_t K, int group_size, int bits, void* hip_stream) {
  qmm4::clear_error();
  // MLX's affine formats whose codes fill whole uint32 words: 2, 4 or 8 bits in groups of 32, 64
  // or 128 (mx.dequantize's parameters).
  if (bits != 2 && bits != 4 && bits != 8)
    return set_error(QMM4_ERR_UNSUPPORTED, "bits=%d: dequantize supports 2-, 4- and 8-bit codes", bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return set_error(QMM4_ERR_UNSUPPORTED, "group_size=%d: dequantize supports groups of 32, 64 and 128", group_size);
  if (N < 0 || K <= 0 || K % group_size != 0)
    return set_error(QMM4_ERR_INVALID, "invalid shape N=%lld K=%lld (K must be a positive multiple of group_size=%d)",
                     (long long)N, (long long)K, group_size);
  if (N > (1LL << 30) || K > (1LL << 30))
    return set_error(QMM4_ERR_INVALID, "shape N=%lld K=%lld exceeds 2^30", (long long)N, (long long)K);
  if (N == 0) return QMM4_OK;
  if (!w || !scales || !biases || !out) return set_error(QMM4_ERR_INVALID, "null pointer argument");
  if (!aligned(w, 16) || !aligned(out, 16))
    return set_error(QMM4_ERR_INVALID, "w and out must be 16-byte aligned");
  if (!aligned(scales, 2) || !aligned(biases, 2))
    return set_error(QMM4_ERR_INVALID, "scales and biases must be 2-byte aligned");
  hipError_t e = qmm4::launch_dequant(w, static_cast<const uint16_t*>(scales), static_cast<const uint16_t*>(biases),
                                      static_cast<uint16_t*>(out), N, K, group_size, bits,
                                      static_cast<hipStream_t>(hip_stream));
  if (e != hipSuccess) return hip_error(e, "dequant kernel launch");
  return QMM4_OK;
}

}  // extern "C"
