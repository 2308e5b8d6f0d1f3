// Measurement floors for the benchmark (libqmm4_floor.so, loaded by bench.py only; not part of the
// quantized-matmul ABI): what one launch costs with nothing to do, and how fast a plain kernel
// streams HBM. The benchmark reports each workload against these beside the spec peaks.
//
//   qmm4_floor_empty  a kernel that returns at once, launched with a given grid, block and
//                     dynamic LDS (the fixed cost of dispatching that grid and draining it);
//   qmm4_floor_read   reads `bytes` (a multiple of 16) with 16-byte loads, four in flight per
//                     thread, and stores one word per wave so the loads are not removed: the read
//                     bandwidth a streaming kernel reaches, the pattern of the weight streams.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ void floor_empty_kernel() {}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kReadThreads = 256;
constexpr int kReadUnroll = 4;

__global__ __launch_bounds__(kReadThreads) void floor_read_kernel(const u32x4* __restrict__ src, uint64_t n16,
                                                                 uint32_t* __restrict__ sink) {
  const uint64_t stride = (uint64_t)gridDim.x * kReadThreads * kReadUnroll;
  uint32_t acc = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * kReadThreads * kReadUnroll + threadIdx.x; i < n16; i += stride) {
    u32x4 v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const uint64_t j = i + (uint64_t)u * kReadThreads;
      v[u] = j < n16 ? __builtin_nontemporal_load(src + j) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  // One word per wave (any value: the store only keeps the loads alive).
  if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (kReadThreads / 64) + (threadIdx.x >> 6)] = acc;
}

}  // namespace

extern "C" {

// Returns 0 or a hipError_t code.
int qmm4_floor_empty(int blocks, int threads, int lds_bytes, void* stream) {
  hipLaunchKernelGGL(floor_empty_kernel, dim3(blocks), dim3(threads), (size_t)lds_bytes,
                     static_cast<hipStream_t>(stream));
  return (int)hipGetLastError();
}

// `sink` holds blocks * 4 uint32 words.
int qmm4_floor_read(const void* src, uint64_t bytes, uint32_t* sink, int blocks, void* stream) {
  hipLaunchKernelGGL(floor_read_kernel, dim3(blocks), dim3(kReadThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), bytes / 16, sink);
  return (int)hipGetLastError();
}

}  // extern "C"
