/*
 * gfxinfer_amd: MI355X (gfx950) speculative-verify hot path behind a C ABI.
 *
 * Each entry point replaces one reference launcher or runtime call; the comment
 * above it cites the reference declaration (include/gfxinfer/... or src/...).
 *
 * Conventions (reference include/gfxinfer/lowbit_gemv.h, qwen_ops.h):
 *  - every pointer is caller-owned device memory unless stated otherwise;
 *  - fp16 and bf16 tensors are passed as uint16_t bit patterns;
 *  - `stream` is a hipStream_t (NULL = the legacy default stream);
 *  - launchers validate their arguments first and return GFXI_INVALID_ARGUMENT
 *    or GFXI_UNSUPPORTED without launching; after a launch they report
 *    hipGetLastError as GFXI_HIP_ERROR;
 *  - launchers never allocate, copy or synchronize, so they are safe to record
 *    into a hipGraph with stream capture;
 *  - gfxinfer_last_error() returns the calling thread's last error text.
 */
#ifndef GFXINFER_AMD_H
#define GFXINFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: include/gfxinfer/status.h:11-20 (ErrorCode). */
#define GFXI_OK 0
#define GFXI_INVALID_ARGUMENT 1
#define GFXI_IO_ERROR 2
#define GFXI_CORRUPT_ARTIFACT 3
#define GFXI_UNSUPPORTED 4
#define GFXI_HIP_ERROR 5
#define GFXI_OUT_OF_MEMORY 6
#define GFXI_INTERNAL 7

/* Weight formats: include/gfxinfer/artifact.h:26-33 (Quantization). */
#define GFXI_W2G128 1
#define GFXI_W3G128 2
#define GFXI_W4G128 3

/* Thread-local text of the last failing call (status.h:22-36 message()). */
const char* gfxinfer_last_error(void);

/* Fail-closed device gate: gfx950 with 64-wide waves
 * (replaces require_gfx1200_device, src/device.cpp:65-90). */
int32_t gfxinfer_require_gfx950_device(int32_t device);

/* ---- packed weight layout (host-side, no device access) ------------------ */

/* src/quantization.cpp:154-161 packed_row_bytes. */
size_t gfxinfer_packed_row_bytes(int32_t format, size_t columns);

/* Converts reference-packed group-128 codes (quantization.cpp:94-124 storage,
 * [rows, packed_row_bytes]) and float scales [rows, K/128] into the gfx950 tile
 * layout, rounding scales to fp16 as the converter does.  Host memory.
 * Replaces tile_group128_for_gfx12 (quantization.cpp:253-318) together with the
 * fp16 scale write of converter.cpp:379-387.  W3G128 and W4G128. */
int32_t gfxinfer_tile_group128_for_gfx950(int32_t format, const uint8_t* packed_codes,
                                          const float* scales, size_t rows, size_t columns,
                                          uint8_t* tiled_codes, uint16_t* tiled_scales_f16);

/* Inverse view of the tile layout: signed integer weights [rows, columns] and
 * fp16 scales [rows, K/128] (host memory).  Counterpart of dequantized_weight
 * (quantization.cpp:222-235) for the gfx950 layout. */
int32_t gfxinfer_untile_group128_for_gfx950(int32_t format, const uint8_t* tiled_codes,
                                            const uint16_t* tiled_scales_f16, size_t rows,
                                            size_t columns, int8_t* weights,
                                            uint16_t* scales_f16);

/* ---- device launchers: src/kernels/lowbit_gemv.hip ------------------------ */

/* Group-128 weight quantizer on the device: fp32 weights [rows, columns] ->
 * gfx950 tiled codes + fp16 scales.  Same least-squares scale fit and codes as
 * quantize_group128 (quantization.cpp:163-220), scales rounded to fp16 as in
 * converter.cpp:379-387.  If non_finite_flag is not NULL it is set to 1 when the
 * input holds a non-finite value (the reference's invalid_argument case). */
int32_t gfxinfer_launch_quantize_group128_gfx950(int32_t format, const float* weights,
                                                 size_t rows, size_t columns,
                                                 uint8_t* tiled_codes, uint16_t* tiled_scales_f16,
                                                 int32_t* non_finite_flag, void* stream);

/* lowbit_gemv.h:79-87: fp16 [batch, columns] -> A4G128 codes [batch, columns/2]
 * (even column in the low nibble) + fp16 scales [batch, columns/128].  batch 1..32. */
int32_t gfxinfer_launch_quantize_activation_i4(const uint16_t* input, uint8_t* packed_output,
                                               uint16_t* scales, size_t columns, uint32_t batch,
                                               void* stream);

/* lowbit_gemv.h:89-95: A8G128 codes int8 [batch, columns] + fp16 scales. */
int32_t gfxinfer_launch_quantize_activation_i8(const uint16_t* input, int8_t* quantized_output,
                                               uint16_t* scales, size_t columns, uint32_t batch,
                                               void* stream);

/* lowbit_gemv.h:97-111 (launch_gfx12_i4_gemm): W{3,4}G128 x A4G128 -> fp32
 * output [batch, rows].  Weights/scales in the gfx950 tile layout; activations as
 * produced by gfxinfer_launch_quantize_activation_i4.  batch 1..32.
 * `sequential_w3` selected between the reference's two gfx12 W3 sub-layouts; the
 * gfx950 layout has one W3 form and the flag is accepted and ignored. */
int32_t gfxinfer_launch_gfx950_i4_gemm(int32_t format, const uint8_t* tiled_weights,
                                       const uint16_t* tiled_weight_scales,
                                       const uint8_t* packed_activations,
                                       const uint16_t* activation_scales, float* output,
                                       size_t rows, size_t columns, uint32_t batch,
                                       int32_t sequential_w3, void* stream);

/* lowbit_gemv.h:113-126 (launch_gfx12_i4_gemm_half): fp16 output [batch, rows]. */
int32_t gfxinfer_launch_gfx950_i4_gemm_half(int32_t format, const uint8_t* tiled_weights,
                                            const uint16_t* tiled_weight_scales,
                                            const uint8_t* packed_activations,
                                            const uint16_t* activation_scales, uint16_t* output,
                                            size_t rows, size_t columns, uint32_t batch,
                                            int32_t sequential_w3, void* stream);

/* lowbit_gemv.h:128-133 (Gfx12I4FusedMatrix). */
typedef struct gfxinfer_fused_matrix {
  const uint8_t* tiled_weights;
  const uint16_t* tiled_weight_scales;
  float* output;
  size_t rows;
} gfxinfer_fused_matrix;

/* lowbit_gemv.h:135-145 (launch_gfx12_i4_gemm_fused): 2..4 same-K, same-format
 * matrices in one grid sharing one quantized activation.  `matrices` is host
 * memory read at call time. */
int32_t gfxinfer_launch_gfx950_i4_gemm_fused(int32_t format,
                                             const gfxinfer_fused_matrix* matrices,
                                             size_t matrix_count,
                                             const uint8_t* packed_activations,
                                             const uint16_t* activation_scales, size_t columns,
                                             uint32_t batch, int32_t sequential_w3,
                                             void* stream);

/* lowbit_gemv.h:147-157 (launch_gfx12_i8_gemm): W{3,4}G128 x A8G128 -> fp32.
 * The reference accepts W2/W4 only; W3 x A8 is added here. */
int32_t gfxinfer_launch_gfx950_i8_gemm(int32_t format, const uint8_t* tiled_weights,
                                       const uint16_t* tiled_weight_scales,
                                       const int8_t* quantized_activations,
                                       const uint16_t* activation_scales, float* output,
                                       size_t rows, size_t columns, uint32_t batch,
                                       void* stream);

/* Debug view of the same kernels: the exact per-group int32 partial sums
 * P[b, n, g] = sum_{k in group g} w(n,k) * a(b,k), written to
 * partials [batch, rows, columns/128].  activation_bits is 4 or 8.  No reference
 * counterpart (the gfx12 WMMA accumulators are never materialized); it exists so
 * tests can check the integer accumulation bit for bit. */
int32_t gfxinfer_debug_gemm_partials(int32_t format, const uint8_t* tiled_weights,
                                     int32_t activation_bits, const void* activations,
                                     size_t rows, size_t columns, uint32_t batch,
                                     int32_t* partials, void* stream);

/* lowbit_gemv.h:46-54 (launch_lowbit_row_gather_tiled): fp16 row
 * out[c] = fp16(w(row, c) * ws(row, c/128)).  W3G128 and W4G128. */
int32_t gfxinfer_launch_lowbit_row_gather_tiled(int32_t format, const uint8_t* tiled_weights,
                                                const uint16_t* tiled_scales, uint16_t* output,
                                                size_t row, size_t rows, size_t columns,
                                                void* stream);

/* lowbit_gemv.h:56-64: same with the row index read from device memory; an
 * out-of-range row yields zeros (lowbit_gemv.hip:202-205). */
int32_t gfxinfer_launch_lowbit_row_gather_tiled_indirect(int32_t format,
                                                         const uint8_t* tiled_weights,
                                                         const uint16_t* tiled_scales,
                                                         uint16_t* output, const uint32_t* row,
                                                         size_t rows, size_t columns,
                                                         void* stream);

#ifdef __cplusplus
}
#endif
#endif
