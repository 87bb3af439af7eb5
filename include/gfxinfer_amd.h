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

/* No reference counterpart (split-K form of gfxinfer_launch_gfx950_i4_gemm for
 * matrices with few 16-row tiles, e.g. the [hidden, K] down/output projections):
 * writes `splits` fp32 planes [splits][batch][rows]; plane s holds the part of the
 * product over the s-th of `splits` equal ranges of K's groups, and the product is
 * the sum of the planes in plane order (the residual RMSNorm entry
 * gfxinfer_launch_residual_add_rms_norm_quantize_i4_planes consumes them).
 * splits in [1, 8] and at most K/128. */
int32_t gfxinfer_launch_gfx950_i4_gemm_split(int32_t format, const uint8_t* tiled_weights,
                                             const uint16_t* tiled_weight_scales,
                                             const uint8_t* packed_activations,
                                             const uint16_t* activation_scales,
                                             float* output_planes, size_t rows, size_t columns,
                                             uint32_t batch, uint32_t splits, void* stream);

/* The split count gfxinfer_launch_gfx950_i4_gemm_split is fastest with for a shape
 * (1 when the plain grid already fills the GPU). */
uint32_t gfxinfer_gemm_split_count(size_t rows, size_t columns, uint32_t batch);

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

/* Bytes of workspace gfxinfer_launch_gfx950_i4_gemm_argmax needs: one 8-byte key per
 * (token, 16-row tile). */
size_t gfxinfer_gemm_argmax_workspace_bytes(size_t rows, uint32_t batch);

/* W{3,4}G128 x A4G128 projection fused with greedy argmax: tokens[b] = the row of the
 * largest logit among rows [0, argmax_rows) (ties to the lowest row, NaN never wins,
 * index 0 when nothing wins), remapped through token_ids when it is not NULL.  Replaces
 * the LM-head projection + launch_argmax_batch pair of the verifier tail
 * (qwen_runtime.cpp:635-639) and the draft head + launch_argmax_mapped pair of the MTP
 * step (qwen_runtime.cpp:859-866) with two launches and no logits round trip; logits
 * [batch, rows] are written too when `logits` is not NULL.  With tokens NULL only the GEMM
 * runs and the workspace holds the per-(token, tile) keys for a later reduction
 * (gfxinfer_launch_mtp_input_quantize_i4_from_keys). */
int32_t gfxinfer_launch_gfx950_i4_gemm_argmax(int32_t format, const uint8_t* tiled_weights,
                                              const uint16_t* tiled_weight_scales,
                                              const uint8_t* packed_activations,
                                              const uint16_t* activation_scales, float* logits,
                                              size_t rows, size_t columns, uint32_t batch,
                                              size_t argmax_rows, const uint32_t* token_ids,
                                              void* workspace, size_t workspace_bytes,
                                              uint32_t* tokens, void* stream);

/* No reference counterpart: gfxinfer_launch_gfx950_i4_gemm_argmax with no workspace
 * argument, for callers that cannot allocate (code under hipGraph capture, serving loops
 * or harnesses that forbid hipMalloc).  The argmax keys live in a library-owned 4 MiB
 * device array per GPU, so batch * ceil(rows / 16) must not exceed 524288 (larger shapes
 * return GFXI_INVALID_ARGUMENT); the entry allocates nothing.  Every call on a GPU shares
 * that array: calls that overlap on one GPU (concurrent streams) race. */
int32_t gfxinfer_launch_gfx950_i4_gemm_argmax_no_alloc(
    int32_t format, const uint8_t* tiled_weights, const uint16_t* tiled_weight_scales,
    const uint8_t* packed_activations, const uint16_t* activation_scales, float* logits,
    size_t rows, size_t columns, uint32_t batch, size_t argmax_rows, const uint32_t* token_ids,
    uint32_t* tokens, void* stream);

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

/* Test and bench hook, no reference counterpart: one A4 GEMM launch through a named
 * kernel family, 1 = the MFMA kernels (16x16x64 int8, used for every shape by the
 * launchers above) or 2 = the v_dot8_i32_i4 kernel (W3/W4, 1-8 tokens, activation
 * scales 4-byte aligned, K/128 even; otherwise GFXI_UNSUPPORTED).  Both families
 * give bit-identical results.  The outputs are those of the launchers above:
 * `output` fp32 (or fp16 when half_output != 0) [splits][batch][rows]; with
 * `partials` non-null the int32 partials of gfxinfer_debug_gemm_partials instead
 * (scales unused); with `argmax_keys` non-null the fused head's per-tile keys
 * ([batch][rows/16], rows >= argmax_rows never win; `output` may then be NULL). */
int32_t gfxinfer_debug_gemm_family(int32_t family, int32_t format, const uint8_t* tiled_weights,
                                   const uint16_t* tiled_weight_scales,
                                   const uint8_t* packed_activations,
                                   const uint16_t* activation_scales, void* output,
                                   int32_t half_output, int32_t* partials,
                                   unsigned long long* argmax_keys, uint32_t argmax_rows,
                                   size_t rows, size_t columns, uint32_t batch, uint32_t splits,
                                   void* stream);

/* Calibration: a plain streaming read of `bytes` from `data` (16-byte aligned,
 * a nonzero multiple of 16) by `workgroups` x 256 lanes, so that a weight-streaming
 * kernel's time can be set beside what one launch reading the same bytes takes on the
 * same device.  `sink` must hold workgroups x 256 uint32; it is written only in the
 * unlikely case a lane's XOR of its data equals 0x9E3779B9.  No reference counterpart. */
int32_t gfxinfer_debug_stream_read(const void* data, size_t bytes, uint32_t* sink,
                                   uint32_t workgroups, void* stream);

/* Calibration: the same read with every load of a lane in flight at once (no loop):
 * ceil(bytes / (4096 * loads_per_lane)) workgroups of 256 lanes, each lane issuing
 * loads_per_lane (1, 2, 4 or 8) non-temporal 16-byte loads, as the GEMMs load their
 * weights.  `sink` must hold bytes / 16 uint32 and is written only in the unlikely
 * case a lane's XOR of its data equals 0x9E3779B9.  No reference counterpart. */
int32_t gfxinfer_debug_stream_read_oneshot(const void* data, size_t bytes, uint32_t* sink,
                                           uint32_t loads_per_lane, void* stream);

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

/* Rows 0..count-1 (count <= 32) of the two launchers above in one launch, row j written
 * at output + j * columns: row 0 is *first_row when first_row is set, else
 * host_rows[0]; row j >= 1 is rest_rows[j - 1] when rest_rows is set, else host_rows[j]
 * (host_rows travel as kernel arguments).  Out-of-range rows yield zeros.  No reference
 * counterpart: the reference gathers one row per launch (qwen_runtime.cpp:553-615). */
int32_t gfxinfer_launch_lowbit_row_gather_tiled_batch(int32_t format, const uint8_t* tiled_weights,
                                                      const uint16_t* tiled_scales, uint16_t* output,
                                                      const uint32_t* host_rows, const uint32_t* first_row,
                                                      const uint32_t* rest_rows, uint32_t count,
                                                      size_t rows, size_t columns, void* stream);


/* ---- decoder operators: src/kernels/qwen_ops.hip -------------------------- */

/* qwen_ops.h:14-21 launch_rms_norm: fp16 row -> fp16(x * rsqrt(mean(x^2) + eps) * (w [+1])). */
int32_t gfxinfer_launch_rms_norm(const uint16_t* input, const uint16_t* bf16_weight,
                                 uint16_t* output, size_t elements, float epsilon,
                                 int32_t add_unit_offset, void* stream);

/* qwen_ops.h:23-31 launch_rms_norm_batch: one row per token. */
int32_t gfxinfer_launch_rms_norm_batch(const uint16_t* input, const uint16_t* bf16_weight,
                                       uint16_t* output, size_t elements, uint32_t batch,
                                       float epsilon, int32_t add_unit_offset, void* stream);

/* qwen_ops.h:70-81 launch_residual_add_rms_norm_batch: r = fp16(res + upd) is written to
 * residual_output and RMS-normalized into normalized_output. */
int32_t gfxinfer_launch_residual_add_rms_norm_batch(const uint16_t* residual, const float* update,
                                                    uint16_t* residual_output,
                                                    const uint16_t* bf16_weight,
                                                    uint16_t* normalized_output, size_t elements,
                                                    uint32_t batch, float epsilon,
                                                    int32_t add_unit_offset, void* stream);

/* RMSNorm fused with the A4G128 quantizer of its fp16 output (codes [batch, elements/2],
 * scales [batch, elements/128]); normalized_output may be NULL.  No reference
 * counterpart: the reference runs launch_rms_norm_batch then
 * launch_quantize_activation_i4 (qwen_runtime.cpp:116-127); the codes are identical. */
int32_t gfxinfer_launch_rms_norm_quantize_i4(const uint16_t* input, const uint16_t* bf16_weight,
                                             uint16_t* normalized_output, uint8_t* packed_output,
                                             uint16_t* scales, size_t elements, uint32_t batch,
                                             float epsilon, int32_t add_unit_offset, void* stream);

/* Residual add + RMSNorm + A4G128 quantizer in one kernel; same codes as
 * launch_residual_add_rms_norm_batch followed by launch_quantize_activation_i4. */
int32_t gfxinfer_launch_residual_add_rms_norm_quantize_i4(
    const uint16_t* residual, const float* update, uint16_t* residual_output,
    const uint16_t* bf16_weight, uint16_t* normalized_output, uint8_t* packed_output,
    uint16_t* scales, size_t elements, uint32_t batch, float epsilon, int32_t add_unit_offset,
    void* stream);

/* No reference counterpart: gfxinfer_launch_residual_add_rms_norm_quantize_i4 with the
 * update given as `planes` (1..8) fp32 planes [planes][batch][elements], summed in
 * plane order (the output of gfxinfer_launch_gfx950_i4_gemm_split). */
int32_t gfxinfer_launch_residual_add_rms_norm_quantize_i4_planes(
    const uint16_t* residual, const float* update_planes, uint32_t planes,
    uint16_t* residual_output, const uint16_t* bf16_weight, uint16_t* normalized_output,
    uint8_t* packed_output, uint16_t* scales, size_t elements, uint32_t batch, float epsilon,
    int32_t add_unit_offset, void* stream);

/* qwen_ops.h:33-42 launch_dual_rms_norm_concat: [norm(left) | norm(right)]. */
int32_t gfxinfer_launch_dual_rms_norm_concat(const uint16_t* left, const uint16_t* left_bf16_weight,
                                             const uint16_t* right,
                                             const uint16_t* right_bf16_weight,
                                             uint16_t* concatenated_output, size_t elements,
                                             float epsilon, int32_t add_unit_offset, void* stream);

/* No reference counterpart: launch_dual_rms_norm_concat over `batch` rows ([batch][elements]
 * inputs, [batch][2 * elements] output), for the batched MTP cache update of a chunked
 * prefill; each row is computed exactly as the single-row launcher computes it. */
int32_t gfxinfer_launch_dual_rms_norm_concat_batch(const uint16_t* left,
                                                   const uint16_t* left_bf16_weight,
                                                   const uint16_t* right,
                                                   const uint16_t* right_bf16_weight,
                                                   uint16_t* concatenated_output, size_t elements,
                                                   uint32_t batch, float epsilon,
                                                   int32_t add_unit_offset, void* stream);

/* The MTP input in one launch: the token's embedding row dequantized from its tiled
 * matrix (as gfxinfer_launch_lowbit_row_gather_tiled writes it; zeros for a token
 * >= embedding_rows; indirect_token, if set, holds the token id), the dual RMSNorm/concat
 * with the conditioning row (gfxinfer_launch_dual_rms_norm_concat), and the A4G128
 * quantizer of the concatenated row (gfxinfer_launch_quantize_activation_i4): codes
 * [2 * elements / 2], scales [2 * elements / 128] bit for bit; concatenated_output
 * (fp16 [2 * elements]) may be null.  elements % 128 == 0, <= 6144.  No reference
 * counterpart (the reference launches the three: qwen_runtime.cpp:728-758 and the
 * quantizer of the fc projection's matrix() call, :779). */
int32_t gfxinfer_launch_mtp_input_quantize_i4(
    int32_t embedding_format, const uint8_t* embedding_codes, const uint16_t* embedding_scales,
    size_t embedding_rows, uint32_t token, const uint32_t* indirect_token,
    const uint16_t* embedding_bf16_norm, const uint16_t* conditioning,
    const uint16_t* conditioning_bf16_norm, uint16_t* concatenated_output, uint8_t* packed_output,
    uint16_t* scales, size_t elements, float epsilon, int32_t add_unit_offset, void* stream);

/* gfxinfer_launch_mtp_input_quantize_i4 whose token is the previous proposal's greedy
 * pick: the argmax of the `key_count` per-tile keys a gfxinfer_launch_gfx950_i4_gemm_argmax
 * call with tokens NULL left for one token (key_count = rows / 16 of that head), remapped
 * through token_ids when it is not NULL.  The token is written to *token_out (what that
 * call's own reduction would have written) and its embedding row feeds the dual
 * RMSNorm/concat and the A4 quantizer as above.  One launch where the MTP chain had the
 * draft head's argmax reduction and the next proposal's input (qwen_runtime.cpp:862-866,
 * then :728-758).  No reference counterpart. */
int32_t gfxinfer_launch_mtp_input_quantize_i4_from_keys(
    int32_t embedding_format, const uint8_t* embedding_codes, const uint16_t* embedding_scales,
    size_t embedding_rows, const uint64_t* argmax_keys, size_t key_count, const uint32_t* token_ids,
    uint32_t* token_out, const uint16_t* embedding_bf16_norm, const uint16_t* conditioning,
    const uint16_t* conditioning_bf16_norm, uint16_t* concatenated_output, uint8_t* packed_output,
    uint16_t* scales, size_t elements, float epsilon, int32_t add_unit_offset, void* stream);

/* qwen_ops.h:44-49 launch_silu_multiply: fp16(silu(g) * u); elements % 128 == 0. */
int32_t gfxinfer_launch_silu_multiply(const float* gate, const float* up, uint16_t* output,
                                      size_t elements, void* stream);

/* qwen_ops.h:51-61 launch_silu_multiply_quantize_i4. */
int32_t gfxinfer_launch_silu_multiply_quantize_i4(const float* gate, const float* up,
                                                  uint8_t* packed_output, uint16_t* scales,
                                                  size_t elements_per_row, uint32_t batch,
                                                  void* stream);

/* qwen_ops.h launch_float_to_half (qwen_ops.hip:809-815). */
int32_t gfxinfer_launch_float_to_half(const float* input, uint16_t* output, size_t elements,
                                      void* stream);

/* qwen_ops.h launch_gdn_conv_update_block (qwen_ops.hip:1020-1047): 4-tap causal conv + SiLU
 * over `batch` tokens; fp16 states [channels, 4]; appended_log [batch, channels] may be NULL. */
int32_t gfxinfer_launch_gdn_conv_update_block(const float* projected_qkv,
                                              const uint16_t* bf16_conv_weight,
                                              const uint16_t* initial_conv_state,
                                              uint16_t* final_conv_state, uint16_t* convolved_qkv,
                                              uint16_t* appended_log, size_t channels,
                                              uint32_t batch, void* stream);

/* qwen_ops.h launch_gdn_recurrent_decode_block (qwen_ops.hip:1076-1107): gated delta rule over a
 * window of batch <= 32 tokens.  Head counts are parameters (the reference hard-codes 48/16);
 * head_size must be 128.  States fp32 [value_heads, 128, 128] (row k, column v).  Logs:
 * key [batch, key_heads*128], delta [batch, value_heads*128], decay [batch, value_heads], any
 * may be NULL.  mixed_workspace: fp32 [batch, value_heads*128] scratch for the pre-norm output
 * (the reference has no such argument: its one-block-per-head kernel normalizes in place). */
int32_t gfxinfer_launch_gdn_recurrent_decode_block(
    const uint16_t* convolved_qkv, const float* projected_z, const float* projected_a,
    const float* projected_b, const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias,
    const uint16_t* bf16_norm_weight, const float* initial_recurrent_state,
    float* final_recurrent_state, uint16_t* output, float* key_log, float* delta_log,
    float* decay_log, uint32_t batch, uint32_t key_heads, uint32_t value_heads,
    uint32_t head_size, float* mixed_workspace, void* stream);

/* The two halves of gfxinfer_launch_gdn_recurrent_decode_block for callers that fuse the
 * out-projection's A4 quantization: the window recurrence writing the pre-norm output, and the
 * head RMSNorm * weight * SiLU(z) -> fp16 -> A4G128 step (a 128-wide head is one group). */
int32_t gfxinfer_launch_gdn_recurrent_window(
    const uint16_t* convolved_qkv, const float* projected_a, const float* projected_b,
    const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias, const float* initial_recurrent_state,
    float* final_recurrent_state, float* mixed, float* key_log, float* delta_log, float* decay_log,
    uint32_t batch, uint32_t key_heads, uint32_t value_heads, uint32_t head_size, void* stream);
int32_t gfxinfer_launch_gdn_output_quantize_i4(const float* mixed, const float* projected_z,
                                               const uint16_t* bf16_norm_weight, uint16_t* output,
                                               uint8_t* packed_output, uint16_t* scales,
                                               uint32_t batch, uint32_t value_heads,
                                               uint32_t head_size, void* stream);

/* gfxinfer_launch_gdn_conv_update_block followed by gfxinfer_launch_gdn_recurrent_window in one
 * launch, with the same arithmetic and outputs (the convolved channels are not written out).
 * No reference counterpart: the reference runs the two launches (qwen_runtime.cpp:502-518).
 * The conv state cannot be updated in place (final_conv_state != initial_conv_state). */
int32_t gfxinfer_launch_gdn_conv_window(
    const float* projected_qkv, const uint16_t* bf16_conv_weight, const uint16_t* initial_conv_state,
    uint16_t* final_conv_state, uint16_t* appended_log, const float* projected_a,
    const float* projected_b, const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias,
    const float* initial_recurrent_state, float* final_recurrent_state, float* mixed, float* key_log,
    float* delta_log, float* decay_log, uint32_t batch, uint32_t key_heads, uint32_t value_heads,
    uint32_t head_size, void* stream);

/* qwen_ops.h launch_gdn_restore_prefix_all (qwen_ops.hip:1141-1179): replay the first
 * accepted_tokens (1..maximum_logged_tokens) logged tokens of every layer onto the pre-window
 * conv and recurrent states, bit-identical to running only those tokens.  Logs are
 * [layer][maximum_logged_tokens][...]. */
int32_t gfxinfer_launch_gdn_restore_prefix_all(
    uint16_t* conv_states, float* recurrent_states, const uint16_t* appended_logs,
    const float* key_logs, const float* delta_logs, const float* decay_logs, size_t channels,
    uint32_t layer_count, uint32_t maximum_logged_tokens, uint32_t accepted_tokens,
    uint32_t key_heads, uint32_t value_heads, uint32_t head_size, void* stream);

/* qwen_ops.h:179-195 launch_qk_rms_norm_rope_block: per-head RMSNorm(1+w) and partial
 * rotate-half RoPE of the first rotary_size dims at positions base+t.  head_size 128,
 * rotary_size even and <= 64. */
int32_t gfxinfer_launch_qk_rms_norm_rope_block(
    const float* query_input, const uint16_t* query_bf16_weight, uint16_t* query_output,
    size_t query_head_count, size_t query_input_stride, const float* key_input,
    const uint16_t* key_bf16_weight, uint16_t* key_output, size_t key_head_count,
    size_t key_input_stride, size_t head_size, size_t rotary_size, uint64_t base_position,
    uint32_t batch, float rope_theta, void* stream);

/* qwen_ops.h:197-215: base position read from device memory (graph-capture variant). */
int32_t gfxinfer_launch_qk_rms_norm_rope_block_indirect_position(
    const float* query_input, const uint16_t* query_bf16_weight, uint16_t* query_output,
    size_t query_head_count, size_t query_input_stride, const float* key_input,
    const uint16_t* key_bf16_weight, uint16_t* key_output, size_t key_head_count,
    size_t key_input_stride, size_t head_size, size_t rotary_size,
    const uint64_t* base_position, uint32_t batch, float rope_theta, void* stream);

/* Q/K RMSNorm + RoPE followed by the K/V cache append of the same block in one launch:
 * the outputs of gfxinfer_launch_qk_rms_norm_rope_block, and the caches
 * ([capacity][key_head_count * head_size]) as gfxinfer_launch_kv_append_block leaves them
 * for key = key_output and value = value_input ([batch][key_head_count * head_size] fp32),
 * bit for bit.  No reference counterpart (the reference launches the pair,
 * qwen_runtime.cpp:439-468). */
int32_t gfxinfer_launch_qk_rms_norm_rope_kv_append_block(
    const float* query_input, const uint16_t* query_bf16_weight, uint16_t* query_output,
    size_t query_head_count, size_t query_input_stride, const float* key_input,
    const uint16_t* key_bf16_weight, uint16_t* key_output, size_t key_head_count,
    size_t key_input_stride, size_t head_size, size_t rotary_size, const float* value_input,
    uint16_t* key_cache, uint16_t* value_cache, size_t capacity, uint64_t base_position,
    uint32_t batch, float rope_theta, void* stream);
/* The same with the base position read from device memory (graph-capture variant). */
int32_t gfxinfer_launch_qk_rms_norm_rope_kv_append_block_indirect_position(
    const float* query_input, const uint16_t* query_bf16_weight, uint16_t* query_output,
    size_t query_head_count, size_t query_input_stride, const float* key_input,
    const uint16_t* key_bf16_weight, uint16_t* key_output, size_t key_head_count,
    size_t key_input_stride, size_t head_size, size_t rotary_size, const float* value_input,
    uint16_t* key_cache, uint16_t* value_cache, size_t capacity, const uint64_t* base_position,
    uint32_t batch, float rope_theta, void* stream);

/* qwen_ops.h launch_kv_append_block: K (fp16) and V (fp32 -> fp16) rows of `batch` tokens into
 * caches [capacity][kv_elements] at position..position+batch-1. */
int32_t gfxinfer_launch_kv_append_block(const uint16_t* key, const float* value,
                                        uint16_t* key_cache, uint16_t* value_cache,
                                        size_t position, size_t capacity, uint32_t batch,
                                        size_t kv_elements, void* stream);
int32_t gfxinfer_launch_kv_append_block_indirect_position(
    const uint16_t* key, const float* value, uint16_t* key_cache, uint16_t* value_cache,
    const uint64_t* position, size_t capacity, uint32_t batch, size_t kv_elements, void* stream);

/* qwen_ops.h launch_argmax_batch (qwen_ops.hip:1496-1514): per-row argmax over the first
 * vocabulary_size logits of stride row_stride; ties go to the lowest index. */
int32_t gfxinfer_launch_argmax_batch(const float* logits, uint32_t* tokens, size_t vocabulary_size,
                                     size_t row_stride, uint32_t batch, void* stream);

/* qwen_ops.h launch_argmax_mapped: token = token_ids[argmax] (MTP shortlist). */
int32_t gfxinfer_launch_argmax_mapped(const float* logits, const uint32_t* token_ids,
                                      uint32_t* token, size_t vocabulary_size, void* stream);


/* ---- verify attention: src/kernels/qwen_ops.hip:698-766 --------------------- */

/* Bytes of fp32 workspace gfxinfer_launch_gated_attention_decode_block needs for up to
 * `batch` tokens of q_heads heads of head_size (128 or 256; 0 for any other) over a cache
 * of `capacity` positions. */
size_t gfxinfer_attention_workspace_bytes(uint32_t batch, uint32_t q_heads, uint32_t head_size,
                                          size_t capacity);

/* qwen_ops.h:256-265 launch_gated_attention_decode_block: causal GQA decode attention of a
 * block of batch <= 32 tokens; token t sees the first base_token_count + t cached positions.
 * query fp16 [batch, q_heads, hd]; gate fp32 [batch, q_heads, 2 hd] (second half of each head
 * row); caches fp16 [capacity, kv_heads, hd]; output fp16 [batch, q_heads, hd]; head size hd
 * 128 or 256.  Head counts and size are parameters (the reference hard-codes 24/4 x 256).
 * workspace: split-local partial results, gfxinfer_attention_workspace_bytes() bytes (no
 * reference counterpart: the reference walks the context serially inside one block). */
int32_t gfxinfer_launch_gated_attention_decode_block(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, size_t base_token_count, size_t capacity, uint32_t batch, uint32_t q_heads,
    uint32_t kv_heads, uint32_t head_size, float* workspace, size_t workspace_bytes, void* stream);

/* qwen_ops.h:267-276: base_token_count = *base_position + 1 read from device memory. */
int32_t gfxinfer_launch_gated_attention_decode_block_indirect_position(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, const uint64_t* base_position, size_t capacity, uint32_t batch,
    uint32_t q_heads, uint32_t kv_heads, uint32_t head_size, float* workspace,
    size_t workspace_bytes, void* stream);

/* Attention followed by the A4G128 quantizer of its output in the same launch: output as
 * gfxinfer_launch_gated_attention_decode_block writes it, and codes [batch, q_heads * hd / 2] /
 * fp16 scales [batch, q_heads * hd / 128] as gfxinfer_launch_quantize_activation_i4 makes them
 * from that output (a head is hd / 128 groups), bit for bit.  No reference counterpart
 * (the reference quantizes the attention output in a launch of its own inside the o
 * projection's matrix() call, qwen_runtime.cpp:471-481 and :116-120). */
int32_t gfxinfer_launch_gated_attention_decode_block_quantize_i4(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, uint8_t* codes, uint16_t* scales, size_t base_token_count, size_t capacity,
    uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t head_size, float* workspace,
    size_t workspace_bytes, void* stream);
/* The same with base_token_count = *base_position + 1 read from device memory. */
int32_t gfxinfer_launch_gated_attention_decode_block_quantize_i4_indirect_position(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, uint8_t* codes, uint16_t* scales, const uint64_t* base_position, size_t capacity,
    uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t head_size, float* workspace,
    size_t workspace_bytes, void* stream);

/* No reference counterpart: gfxinfer_launch_qk_rms_norm_rope_kv_append_block followed by
 * gfxinfer_launch_gated_attention_decode_block_quantize_i4 (qwen_runtime.cpp:439-474, the
 * reference's launch_qk_rms_norm_rope_block, launch_kv_append_block and
 * launch_gated_attention_decode_block) in two launches instead of three, bit for bit: the
 * attention's split workgroups normalize and rotate their KV head's query rows themselves,
 * and the workgroup whose split holds a new position writes that position's K / V rows
 * (token t at position + t) to the caches.  The query/key outputs of the RoPE launcher are
 * not written.  rope_table, if not NULL, holds gfxinfer_launch_rope_table's (cos, sin)
 * values for every position of the cache (read instead of evaluated: same results).
 * Shapes gfxinfer_fused_rope_attention_supported() refuses return GFXI_UNSUPPORTED. */
int32_t gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4(
    const float* query_input, const uint16_t* query_bf16_weight, size_t query_input_stride,
    const float* key_input, const uint16_t* key_bf16_weight, size_t key_input_stride,
    const float* value_input, size_t rotary_size, float rope_theta, const float* rope_table,
    const float* gate,
    uint16_t* key_cache, uint16_t* value_cache, uint16_t* output, uint8_t* codes, uint16_t* scales,
    size_t position, size_t capacity, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
    uint32_t head_size, float* workspace, size_t workspace_bytes, void* stream);
/* The same with position = *base_position read from device memory. */
int32_t gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4_indirect_position(
    const float* query_input, const uint16_t* query_bf16_weight, size_t query_input_stride,
    const float* key_input, const uint16_t* key_bf16_weight, size_t key_input_stride,
    const float* value_input, size_t rotary_size, float rope_theta, const float* rope_table,
    const float* gate,
    uint16_t* key_cache, uint16_t* value_cache, uint16_t* output, uint8_t* codes, uint16_t* scales,
    const uint64_t* base_position, size_t capacity, uint32_t batch, uint32_t q_heads,
    uint32_t kv_heads, uint32_t head_size, float* workspace, size_t workspace_bytes, void* stream);
/* 1 if the fused entries take the shape: head size 128 or 256, at most 8 tokens, at most 8
 * query heads per KV head and at most 32 (head size 128) or 30 (256) query rows per KV
 * head (q_heads / kv_heads x batch); 0 otherwise. */
int32_t gfxinfer_fused_rope_attention_supported(uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                                                uint32_t head_size);

/* No reference counterpart: (cos, sin) of the RoPE angle position * theta^(-2 f / rotary)
 * for positions 0..positions-1 and frequencies f < rotary / 2, as float2
 * [positions][rotary / 2] (evaluated as the RoPE launchers evaluate it, bit for bit), for
 * the rope_table argument above.  rotary even, 2..64. */
size_t gfxinfer_rope_table_bytes(size_t positions, size_t rotary_size);
int32_t gfxinfer_launch_rope_table(float* table, size_t positions, size_t rotary_size, float rope_theta,
                                   void* stream);

/* ---- single-token launchers: the one-token calls of greedy_step and the MTP proposal ---
 * Each is its block launcher at batch 1 (same kernels, bit-identical results). */

/* qwen_ops.h:83-88 launch_gdn_conv_update (called at qwen_runtime.cpp:389): conv state
 * [channels][4] fp16 advanced in place by one token; convolved_qkv fp16 [channels].  The
 * reference fixes channels at its model's 10240. */
int32_t gfxinfer_launch_gdn_conv_update(const float* projected_qkv, const uint16_t* bf16_conv_weight,
                                        uint16_t* conv_state, uint16_t* convolved_qkv, size_t channels,
                                        void* stream);

/* qwen_ops.h:101-111 launch_gdn_recurrent_decode (called at qwen_runtime.cpp:394): one token
 * of the gated delta rule, recurrent state fp32 [value_heads][128][128] updated in place, no
 * logs.  mixed_workspace: fp32 [value_heads * 128] (as for the block form). */
int32_t gfxinfer_launch_gdn_recurrent_decode(
    const uint16_t* convolved_qkv, const float* projected_z, const float* projected_a,
    const float* projected_b, const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias,
    const uint16_t* bf16_norm_weight, float* recurrent_state, uint16_t* output, uint32_t key_heads,
    uint32_t value_heads, uint32_t head_size, float* mixed_workspace, void* stream);

/* qwen_ops.h:130-139 launch_gdn_restore_prefix: one layer's conv and recurrent states replayed
 * over the first accepted_tokens (>= 1) tokens of that layer's logs ([tokens][...]). */
int32_t gfxinfer_launch_gdn_restore_prefix(uint16_t* conv_state, float* recurrent_state,
                                           const uint16_t* appended_log, const float* key_log,
                                           const float* delta_log, const float* decay_log,
                                           size_t channels, uint32_t accepted_tokens, uint32_t key_heads,
                                           uint32_t value_heads, uint32_t head_size, void* stream);

/* qwen_ops.h:217-224 launch_kv_append (called at qwen_runtime.cpp:372 and :818): one token's
 * K (fp16) and V (fp32 -> fp16) rows of kv_elements at position < capacity. */
int32_t gfxinfer_launch_kv_append(const uint16_t* key, const float* value, uint16_t* key_cache,
                                  uint16_t* value_cache, size_t position, size_t capacity,
                                  size_t kv_elements, void* stream);

/* qwen_ops.h:246-254 launch_gated_attention_decode (called at qwen_runtime.cpp:375 and :831):
 * one token attending to the first token_count (1..capacity) cached positions; layouts and
 * workspace as gfxinfer_launch_gated_attention_decode_block with batch 1. */
int32_t gfxinfer_launch_gated_attention_decode(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, size_t token_count, size_t capacity, uint32_t q_heads, uint32_t kv_heads,
    uint32_t head_size, float* workspace, size_t workspace_bytes, void* stream);

/* qwen_ops.h:278-282 launch_argmax (called at qwen_runtime.cpp:866 and :1305): the index of
 * the largest of vocabulary_size logits; ties go to the lowest index. */
int32_t gfxinfer_launch_argmax(const float* logits, uint32_t* token, size_t vocabulary_size,
                               void* stream);

/* ---- the reference's scratch-free signatures at its own model's shapes ----------------
 * launch_gdn_recurrent_decode[_block] (qwen_ops.h:101-127) and
 * launch_gated_attention_decode[_block][_indirect_position] (qwen_ops.h:246-276) take no
 * workspace and hard-code the reference model (attention 24 Q / 4 KV heads x 256, GDN 16
 * key / 48 value heads x 128; qwen38_spec.h:22-29).  The entries below take exactly the
 * reference's arguments (no head counts, no workspace).  Their scratch is a device buffer
 * of gfxinfer_qwen38_scratch_bytes(max_batch, capacity) bytes that the caller allocates
 * and binds to the launch stream once, before any graph capture; a launch then only looks
 * it up on the host and allocates nothing, so it can be captured.  Launches on one stream
 * share its scratch and run in stream order; launches on two streams bound to one buffer
 * race.  A launch on a stream with no scratch bound, or with a batch or capacity above
 * the binding's, returns GFXI_INVALID_ARGUMENT without launching.  No reference
 * counterpart for the three scratch calls. */

/* Bytes of scratch for up to max_batch (1..32) tokens over caches of `capacity` positions;
 * 0 for invalid arguments. */
size_t gfxinfer_qwen38_scratch_bytes(uint32_t max_batch, size_t capacity);
/* Binds (or rebinds) a 256-byte aligned device buffer of at least
 * gfxinfer_qwen38_scratch_bytes(max_batch, capacity) bytes to `stream` (may be null: the
 * null stream).  The buffer stays the caller's; it must outlive the launches. */
int32_t gfxinfer_qwen38_bind_scratch(void* stream, void* scratch, size_t bytes, uint32_t max_batch,
                                     size_t capacity);
/* Forgets the stream's binding (GFXI_INVALID_ARGUMENT if it has none).  Bindings are
 * keyed by the stream handle: unbind before destroying the stream, since a stream
 * created later may reuse the handle and would otherwise find the old buffer. */
int32_t gfxinfer_qwen38_unbind_scratch(void* stream);

/* qwen_ops.h:246-254: one token attending to the first token_count cached positions. */
int32_t gfxinfer_qwen38_launch_gated_attention_decode(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, size_t token_count, size_t capacity, void* stream);
/* qwen_ops.h:256-265: gfxinfer_launch_gated_attention_decode_block at 24/4 x 256. */
int32_t gfxinfer_qwen38_launch_gated_attention_decode_block(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, size_t base_token_count, size_t capacity, uint32_t batch, void* stream);
/* qwen_ops.h:267-276: the same with base_token_count = *device_base_position + 1. */
int32_t gfxinfer_qwen38_launch_gated_attention_decode_block_indirect_position(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, const uint64_t* device_base_position, size_t capacity, uint32_t batch, void* stream);
/* qwen_ops.h:113-127: gfxinfer_launch_gdn_recurrent_decode_block at 16 key / 48 value heads
 * x 128 (10240 conv channels). */
int32_t gfxinfer_qwen38_launch_gdn_recurrent_decode_block(
    const uint16_t* convolved_qkv, const float* projected_z, const float* projected_a, const float* projected_b,
    const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias, const uint16_t* bf16_norm_weight,
    const float* initial_recurrent_state, float* final_recurrent_state, uint16_t* output, float* key_log,
    float* delta_log, float* decay_log, uint32_t batch, void* stream);
/* qwen_ops.h:101-111: one token, recurrent state updated in place, no logs. */
int32_t gfxinfer_qwen38_launch_gdn_recurrent_decode(
    const uint16_t* convolved_qkv, const float* projected_z, const float* projected_a, const float* projected_b,
    const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias, const uint16_t* bf16_norm_weight,
    float* recurrent_state, uint16_t* output, void* stream);

#ifdef __cplusplus
}
#endif
#endif
