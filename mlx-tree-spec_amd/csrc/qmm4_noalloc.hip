// The quantized matmul for callers that cannot allocate (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc): the same kernels and the same results as
// qmm4_affine_bf16, with the split-K workspace taken from a static device array instead of a
// library allocation.
//
// The array holds kNoallocCounterBytes of arrival counters followed by the fp32 partial sums.
// Every GPU the library runs on holds its own copy until the process ends. Host code never uses
// the array's name as an address (on the host it names a stand-in, not device memory): the
// device address is looked up once per device with hipGetSymbolAddress, with that device current,
// and only that pointer is passed to kernels and fills. The counters are cleared by a fill kernel
// at that first call and every launch leaves them at zero again; the partials are always written
// before they are read. All calls on one GPU share the array, so calls that overlap on one GPU
// (on different streams, or from different threads without ordering) race.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "qmm4.h"
#include "qmm4_dispatch.h"
#include "qmm4_kernels.h"

namespace qmm4 {

namespace {

constexpr size_t kNoallocBytes = QMM4_NOALLOC_SCRATCH_BYTES;
constexpr size_t kNoallocCounterBytes = 64u << 10;
static_assert(kNoallocBytes > kNoallocCounterBytes && kNoallocCounterBytes % 256 == 0, "scratch layout");

__device__ __align__(256) uint8_t scratch[kNoallocBytes];

// Device address of `scratch` per device (api_mutex held).
std::map<int, uint8_t*>& scratch_ptrs() {
  static std::map<int, uint8_t*> m;
  return m;
}

int device_scratch(int dev, hipStream_t stream, uint8_t** out) {
  auto& ptrs = scratch_ptrs();
  auto it = ptrs.find(dev);
  if (it != ptrs.end()) {
    *out = it->second;
    return QMM4_OK;
  }
  // First call on this device (the caller made it current): look the array up and clear its
  // counters. A fill recorded into a graph would only run at replay, so this call must not be
  // captured.
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &st);
  if (e != hipSuccess) return hip_error(e, "hipStreamIsCapturing");
  if (st != hipStreamCaptureStatusNone)
    return set_error(QMM4_ERR_CAPTURE,
                     "qmm4_affine_bf16_noalloc: the first call on a device sets up its static scratch and "
                     "cannot be captured; call once outside capture first");
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
  e = launch_zero_u32(static_cast<uint32_t*>(p), kNoallocCounterBytes / sizeof(uint32_t), stream);
  if (e != hipSuccess) return hip_error(e, "static scratch counter clear");
  // The pointer is published only once the clear has finished, so a later call on another
  // stream cannot read counters that are not yet zero (this call is not captured: see above).
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_error(e, "static scratch counter clear (synchronize)");
  ptrs.emplace(dev, static_cast<uint8_t*>(p));
  *out = static_cast<uint8_t*>(p);
  return QMM4_OK;
}

class StaticWorkspace final : public WorkspaceSource {
 public:
  explicit StaticWorkspace(uint8_t* base) : base_(base) {}

  int get(size_t counter_bytes, size_t partial_bytes, uint32_t** cnt, float** part) override {
    if (counter_bytes > kNoallocCounterBytes || partial_bytes > kNoallocBytes - kNoallocCounterBytes)
      return set_error(QMM4_ERR_INVALID,
                       "qmm4_affine_bf16_noalloc: this shape needs %zu bytes of split-K counters and %zu bytes of "
                       "partial sums; the static scratch holds at most %zu and %zu (use qmm4_affine_bf16)",
                       counter_bytes, partial_bytes, kNoallocCounterBytes, kNoallocBytes - kNoallocCounterBytes);
    *cnt = reinterpret_cast<uint32_t*>(base_);
    *part = reinterpret_cast<float*>(base_ + kNoallocCounterBytes);
    return QMM4_OK;
  }

  size_t capacity() const override { return kNoallocBytes - kNoallocCounterBytes; }

  int get_scratch(size_t bytes, void**) override {
    return set_error(QMM4_ERR_INVALID, "qmm4_affine_bf16_noalloc: no scratch for %zu bytes", bytes);
  }

 private:
  uint8_t* base_;
};

}  // namespace

}  // namespace qmm4

extern "C" int qmm4_affine_bf16_noalloc(const void* x, const uint32_t* w, const void* scales, const void* biases,
                                        void* y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                        int transpose, void* hip_stream) {
  qmm4::clear_error();
  int rc = qmm4::check_qmm_args(x, w, scales, biases, y, M, N, K, group_size, bits, transpose);
  if (rc || M == 0 || N == 0) return rc;
  hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return qmm4::hip_error(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(qmm4::api_mutex());
  qmm4::DeviceInfo* di = nullptr;
  if ((rc = qmm4::device_info(dev, &di))) return rc;
  uint8_t* base = nullptr;
  if ((rc = qmm4::device_scratch(dev, stream, &base))) return rc;
  qmm4::StaticWorkspace ws(base);
  return qmm4::dispatch_qmm(di, x, w, scales, biases, y, M, N, K, stream, ws);
}
