/*
 * qmm4.h — C ABI of the MI355X (gfx950) packed 4-bit affine quantized matmul.
 *
 * Format (MLX affine, 4 bits, group 64; the layout of mlx.nn.QuantizedLinear as used by
 * src/mlx_tree_spec/packed_linear.py:49-58 and read by src/mlx_tree_spec/qmm_packed.py):
 *   w       uint32 [N, K/8]   code q[n, 8c+i] = (w[n, c] >> 4i) & 0xF        (qmm_packed.py:115, 200-201)
 *   scales  bf16   [N, K/64]  s[n, g],  g = k / 64                           (qmm_packed.py:454, 630)
 *   biases  bf16   [N, K/64]  b[n, g]
 *   dequant w_deq[n, k] = bf16_rne(fp32(s) * q + fp32(b))                   (qmm_packed.py:635-636)
 *   y[m, n] = bf16_rne(sum_k fp32(x[m, k]) * fp32(w_deq[n, k]))  (fp32 accumulation, any order)
 *
 * Conventions for every entry point:
 *   - all array pointers are caller-owned HIP device pointers on the current device, row-major and
 *     contiguous; bf16 arrays are passed as raw 16-bit words (void*), so no host type is implied;
 *   - work is enqueued asynchronously on `hip_stream` (a hipStream_t; NULL = the default stream);
 *   - return 0 on success or a negative QMM4_ERR_* code; qmm4_last_error() then returns a
 *     message for the calling host thread;
 *   - the library keeps one internal workspace per (device, stream) for split-K partial sums;
 *     calls on the same stream are ordered, calls on different streams use different workspaces.
 *     A workspace that a call used while its stream was being captured into a graph is never
 *     freed (the graph may replay on it later); a call that would need it to grow during capture
 *     returns QMM4_ERR_CAPTURE instead of allocating.
 */
#ifndef MI355X_QMM4_H
#define MI355X_QMM4_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QMM4_OK 0
#define QMM4_ERR_INVALID (-22)     /* bad shape, null pointer, misaligned pointer       */
#define QMM4_ERR_UNSUPPORTED (-95) /* bits != 4, group_size != 64, transpose == 0       */
#define QMM4_ERR_NOMEM (-12)       /* workspace allocation failed                       */
#define QMM4_ERR_HIP (-5)          /* a HIP runtime call failed (message has the name)  */
#define QMM4_ERR_CAPTURE (-16)     /* a library buffer must grow while the stream is    */
                                   /* being captured into a graph: call once with that  */
                                   /* shape on that stream before capturing             */

/*
 * y = x @ dequant(w)^T  — the quantized-matmul call of the verify, decode and prefill passes.
 * Replaces mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size=64, bits=4) as
 * called at src/mlx_tree_spec/packed_linear.py:97, and the packed kernels behind
 * packed_linear._call (packed_linear.py:83-104; qmm_packed.py:270-293, 372-394, 529-551, 701-725).
 *   x: bf16 [M, K]; w: uint32 [N, K/8]; scales, biases: bf16 [N, K/group_size]; y: bf16 [M, N].
 *   Requires M >= 0, N % 16 == 0, K % 128 == 0 (the reference's packed path requires K % 128 == 0,
 *   packed_linear.py:57), group_size == 64, bits == 4, transpose == 1, each of M, N, K <= 2^30,
 *   w, x and y each below 4 GiB (with 256 rows of margin: (N + 256) * K / 2, (M + 256) * K * 2 and
 *   (M + 256) * N * 2 bytes below 2^32), x and w 16-byte aligned, scales and biases
 *   4-byte aligned, y 2-byte aligned. M == 0 or N == 0 is a no-op. Rows M <= 64 run one of the
 *   HBM-bound verify/decode kernels (row-split's x-in-registers form for 9-16 rows over small
 *   problems; row-split for M <= 16 when its plan fits: whole K (units taken in groups of
 *   consecutive steps, or waves owning whole blocks, when N is as large as a vocabulary head) or a few K slices per workgroup,
 *   every unit in flight at once for small problems; row-phase for more than 16 rows, a large N,
 *   or fewer rows when its K split fills half the CUs; K-split verify or stream-K skinny
 *   otherwise); 65-112 rows (128 over at most 2048 columns) the row-phase kernel with 80-128-row
 *   x blocks when its plan is narrow; larger M the MFMA GEMM (whole 256 x 256 tiles, or stream-K
 *   over 128 x 128 tiles when whole tiles would leave many CUs idle, over 256 x 256 tiles when K
 *   is long too); the choice is a fixed function of the shape and the scale/bias alignment.
 *   Results are deterministic (bit-identical across calls and streams). Other formats (2- or
 *   8-bit codes, groups of 32 or 128) return QMM4_ERR_UNSUPPORTED: dequant4_affine_bf16 takes
 *   them, and the package's quantized_matmul multiplies its output with a bf16 GEMM.
 */
int qmm4_affine_bf16(const void* x, const uint32_t* w, const void* scales, const void* biases,
                     void* y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                     int transpose, void* hip_stream);

/*
 * y = x @ dequant(w)^T without any allocation: the same checks, kernels and results (bit for bit)
 * as qmm4_affine_bf16, with the split-K workspace in a static device array of
 * QMM4_NOALLOC_SCRATCH_BYTES per GPU (64 KiB of counters, the rest fp32 partial sums) instead of a
 * library allocation. The array holds the largest workspace any plan takes on a 256-CU MI355X (the
 * GEMM's stream-K over 256 x 256 tiles: 256 workgroups x two 256 KiB partial tiles), so every
 * shape whose arrival counters fit in 64 KiB gets the plan qmm4_affine_bf16 takes; on a GPU with
 * more CUs a plan that would not fit falls back to one that does (results then within the parity
 * tolerance, not bit for bit). It has no counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 *   - Calls no hipMalloc / hipFree / allocating routine. The first call on a device looks the array
 *     up, clears its counters on `hip_stream` and waits for that clear (that call must not be
 *     captured: QMM4_ERR_CAPTURE); later calls on that device may be captured. The array takes
 *     device memory from that first call on (HIP loads the code object holding it then), not
 *     when the library is loaded.
 *   - A shape whose split-K buffers exceed the array returns QMM4_ERR_INVALID with the sizes.
 *   - Every call on one GPU shares that GPU's array: calls that overlap on one GPU (different
 *     streams, or threads without ordering between them) race. Order them on one stream.
 */
#define QMM4_NOALLOC_SCRATCH_BYTES (136u * 1024u * 1024u)
int qmm4_affine_bf16_noalloc(const void* x, const uint32_t* w, const void* scales, const void* biases,
                             void* y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                             int transpose, void* hip_stream);

/*
 * y = silu(x @ dequant(w_gate)^T) * (x @ dequant(w_up)^T) — a fused gate+up projection with the
 * SiLU·mul epilogue, the input of down_proj in the MLP of the verify forward
 * (src/mlx_tree_spec/tree_verify.py:446: layer.mlp(x) = down_proj(silu(gate_proj(x)) * up_proj(x));
 * config "decode GEMV, fused gate+up projection"). Replaces the two quantized-matmul calls plus the
 * elementwise silu and multiply.
 *   w = [w_gate; w_up]: uint32 [N, K/8], gate rows 0 .. N/2 - 1, up rows N/2 .. N - 1; scales and
 *   biases bf16 [N, K/group_size] in the same row order; y: bf16 [M, N/2].
 *   The gate and up sums are rounded to bf16 (the values the two projections would store), then
 *   out = bf16(bf16(g * bf16(sigmoid(g))) * u), one rounding per operation of the unfused
 *   composition. Same requirements as qmm4_affine_bf16, plus N % 32 == 0 and y 16-byte aligned.
 *   Up to 16 rows whose row-split plan fits run as one kernel; otherwise the projection goes to a
 *   library-held [M, N] buffer (per device and stream, grown on demand) and the epilogue is a
 *   second pass. Deterministic.
 */
int qmm4_gate_up_silu_bf16(const void* x, const uint32_t* w, const void* scales, const void* biases,
                           void* y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                           int transpose, void* hip_stream);

/*
 * out = dequant(w) as bf16 [N, K] — the bit-exact unpack + affine dequant,
 * out[n, k] = bf16_rne(fp32(s) * q + fp32(b)).
 * Replaces mx.dequantize(w, scales, biases, group_size, bits) as used by the reference's
 * exact-reference definition (tests/test_units.py:108) and qmm_packed.py:200-201 / 635-636, and
 * by the general path the reference gives modules its packed kernels do not take
 * (packed_linear.py:84-86).
 *   bits 2, 4 or 8 (code k = (32 / bits) c + i in bits [bits i, bits i + bits) of word c of its
 *   row, w uint32 [N, K * bits / 32]); group_size 32, 64 or 128 (scales and biases
 *   [N, K / group_size]). Other bit widths return QMM4_ERR_UNSUPPORTED.
 *   Requires N >= 0, K % group_size == 0, 16-byte aligned w and out.
 */
int dequant4_affine_bf16(const uint32_t* w, const void* scales, const void* biases, void* out,
                         int64_t N, int64_t K, int group_size, int bits, void* hip_stream);

/*
 * (h, n) = (x + r, rmsnorm(x + r) * weight) — the residual add fused with the RMS norm that follows
 * it, the op in front of each quantized matmul of the verify forward. Replaces
 * fused_ops.add_rms_norm(x, r, norm) (src/mlx_tree_spec/fused_ops.py:107-160; called at
 * tree_verify.py:444-446).
 *   x, r, h_out, n_out: bf16 [rows, D]; weight: bf16 [D]; per row
 *     h = bf16(x + r), n = bf16(weight * bf16(h * inv)), inv = 1 / sqrt(sum(h * h) / D + eps),
 *   the sum in fp32 (its order, like the reference's simdgroup reduction, is the kernel's own).
 *   Requires rows >= 0, D % 8 == 0, D <= 16384, eps finite and >= 0, every pointer 16-byte
 *   aligned. rows == 0 is a no-op.
 */
int qmm4_add_rms_norm_bf16(const void* x, const void* r, const void* weight, void* h_out, void* n_out,
                           int64_t rows, int64_t D, float eps, void* hip_stream);

/*
 * (h, n, y) = (x + r, rmsnorm(x + r) * weight, projection of n) — the residual add + RMS norm and
 * the quantized projection that consumes its output, as one call. Replaces the pair
 * fused_ops.add_rms_norm (src/mlx_tree_spec/fused_ops.py:107-160) + the next layer's projection
 * at tree_verify.py:444-446 (h, x = add_rms_norm(h, r, post_attention_layernorm); layer.mlp(x)).
 *   epilogue QMM4_EPILOGUE_NONE:     y = n @ dequant(w)^T, bf16 [M, N]      (qmm4_affine_bf16)
 *   epilogue QMM4_EPILOGUE_SILU_MUL: y = silu(n w_gate^T) * (n w_up^T), bf16 [M, N/2]
 *                                                                          (qmm4_gate_up_silu_bf16)
 *   x, r, h_out, n_out: bf16 [M, K]; weight: bf16 [K]; w, scales, biases as for qmm4_affine_bf16.
 *   h_out, n_out and y hold exactly the bits of qmm4_add_rms_norm_bf16(x, r, weight, h_out, n_out,
 *   M, K, eps) followed by qmm4_affine_bf16 / qmm4_gate_up_silu_bf16 on n_out. Up to 4 rows whose
 *   projection runs as the row-split kernel (K <= 8192) take ONE launch: every workgroup forms h
 *   and n for its own K slice in its x staging (the norm's launch and the n round trip through
 *   memory disappear); other shapes run the two calls.
 *   Requires the projection's conditions (and N % 32 == 0, y 16-byte aligned for SILU_MUL), the
 *   norm's (K <= 16384, eps finite and >= 0, x, r, weight, h_out, n_out 16-byte aligned), and
 *   h_out, n_out, y overlapping neither each other nor x, r, weight, w, scales, biases. M == 0 is a
 *   no-op; N == 0 runs the norm alone.
 */
#define QMM4_EPILOGUE_NONE 0
#define QMM4_EPILOGUE_SILU_MUL 1
int qmm4_add_rms_norm_qmm_bf16(const void* x, const void* r, const void* weight, float eps, void* h_out,
                               void* n_out, const uint32_t* w, const void* scales, const void* biases, void* y,
                               int64_t M, int64_t N, int64_t K, int group_size, int bits, int transpose,
                               int epilogue, void* hip_stream);

/* Message for the last non-zero return on this host thread ("" if none). */
const char* qmm4_last_error(void);

/* Library ABI version (bumped when a signature above changes). */
int qmm4_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_QMM4_H */
