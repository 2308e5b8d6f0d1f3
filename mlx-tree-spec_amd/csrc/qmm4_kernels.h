// Kernel launch interface between the C ABI layer (qmm4_api.cpp) and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qmm4 {

// Skinny (M <= 64) stream-K kernel geometry, chosen by M.
struct SkinnyPlan {
  int variant;   // index into the kernel table (see qmm4_skinny.hip)
  int tile_cols; // output columns per tile (CW)
  int blocks;    // workgroups launched (G)
  int tiles;     // tiles along N (T)
  long long units;  // T * (K / 128)
};

// Returns the variant for M rows (1..64) and its columns per tile.
int skinny_variant_for_rows(int M, int* tile_cols);
// Resident workgroups per CU for a variant (from the HIP occupancy API; cached by the caller).
int skinny_occupancy(int variant);
// Enqueue the skinny kernel. `part` holds blocks*2*M*tile_cols floats, `cnt` tiles zeroed uint32s.
hipError_t launch_skinny(const SkinnyPlan& plan, const uint16_t* x, const uint32_t* w,
                         const uint16_t* s, const uint16_t* b, uint16_t* y, float* part,
                         uint32_t* cnt, int M, int N, int K, hipStream_t stream);

// LDS-tiled MFMA GEMM for M > 64.
hipError_t launch_gemm(const uint16_t* x, const uint32_t* w, const uint16_t* s,
                       const uint16_t* b, uint16_t* y, int M, int N, int K, hipStream_t stream);

// Bit-exact dequantization to bf16 [N, K].
hipError_t launch_dequant(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          uint16_t* out, int64_t N, int64_t K, hipStream_t stream);

}  // namespace qmm4
