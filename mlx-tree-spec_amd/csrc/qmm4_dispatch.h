// Shared host-side pieces of the C ABI: error reporting, argument checks and the kernel choice,
// used by every entry point of include/qmm4.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <mutex>

namespace qmm4 {

// Sets the calling host thread's message (returned by qmm4_last_error) and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_error(hipError_t e, const char* what);
void clear_error();

// Serializes the library's host-side state (device facts, workspaces) across host threads.
std::mutex& api_mutex();

// Per-device facts, queried once (api_mutex held).
struct DeviceInfo;
int device_info(int dev, DeviceInfo** out);
int device_cus(const DeviceInfo* di);

// Where a call's split-K buffer comes from: counters (zero between calls; every launch leaves them
// at zero) followed by fp32 partials. get() returns 0 or a negative QMM4_ERR_* code.
class WorkspaceSource {
 public:
  virtual int get(size_t counter_bytes, size_t partial_bytes, uint32_t** cnt, float** part) = 0;
  // The most partial bytes get() can provide.
  virtual size_t capacity() const = 0;
  // Scratch for the [M, N] projection of the two-pass gate+up epilogue.
  virtual int get_scratch(size_t bytes, void** out) = 0;

 protected:
  ~WorkspaceSource() = default;
};

// Format, shape and alignment checks shared by the quantized-matmul entry points.
int check_qmm_args(const void* x, const uint32_t* w, const void* scales, const void* biases, const void* y,
                   int64_t M, int64_t N, int64_t K, int group_size, int bits, int transpose);

// The kernel choice and launches of y = x @ dequant(w)^T (arguments checked, M and N > 0,
// api_mutex held).
int dispatch_qmm(DeviceInfo* di, const void* x, const uint32_t* w, const void* scales, const void* biases,
                 void* y, int64_t M, int64_t N, int64_t K, hipStream_t stream, WorkspaceSource& ws);

// The fused gate+up projection with its SiLU·mul epilogue (same preconditions, N % 32 == 0).
int dispatch_gate_up_silu(DeviceInfo* di, const void* x, const uint32_t* w, const void* scales,
                          const void* biases, void* y, int64_t M, int64_t N, int64_t K, hipStream_t stream,
                          WorkspaceSource& ws);

// (h, n, y) = (x + r, rmsnorm(x + r) * weight, n @ dequant(w)^T), or the gate+up SiLU·mul of it
// when `silu_mul`: the norm folded into the row-split kernel's x staging when its plan allows, else
// the norm kernel followed by dispatch_qmm / dispatch_gate_up_silu on n (the same bits either way).
// Arguments checked, M > 0, api_mutex held.
int dispatch_norm_qmm(DeviceInfo* di, const void* x, const void* r, const void* weight, float eps, void* h_out,
                      void* n_out, const uint32_t* w, const void* scales, const void* biases, void* y, int64_t M,
                      int64_t N, int64_t K, bool silu_mul, hipStream_t stream, WorkspaceSource& ws);

}  // namespace qmm4
