/*
 * CPU oracle: a plain-C restatement of the reference gfxinfer semantics for the
 * speculative-verify hot path.  TEST INFRASTRUCTURE ONLY: it is the checker that
 * the tests, the smoke entry and the bench's cpu_baseline leg compare against.
 * No product code may link or call it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root).  Pinning of each function (golden vectors from
 * the compiled reference quantizer, closed forms, brute force) lives in tests/.
 */
#ifndef GFXINFER_ORACLE_H
#define GFXINFER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quantization tags: include/gfxinfer/artifact.h:26-33. */
enum { ORC_W2 = 1, ORC_W3 = 2, ORC_W4 = 3 };
/* ErrorCode values: include/gfxinfer/status.h:11-20. */
enum { ORC_OK = 0, ORC_INVALID_ARGUMENT = 1, ORC_UNSUPPORTED = 4 };

/* ---- fp16 / bf16 -------------------------------------------------------- */
uint16_t orc_f32_to_f16(float value);          /* IEEE binary16, round-to-nearest-even */
float orc_f16_to_f32(uint16_t bits);
void orc_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n);
float orc_bf16_to_f32(uint16_t bits);          /* qwen_ops.hip:27-29 */

/* ---- weight quantizer (src/quantization.cpp) ---------------------------- */
size_t orc_packed_row_bytes(int format, size_t columns);           /* :154-161 */
int orc_quantize_group128(const float* weights, size_t rows, size_t columns, int format,
                          uint8_t* codes, float* scales);          /* :163-220 */
uint8_t orc_load_code(const uint8_t* row_codes, size_t column, int format); /* :126-150 */
int orc_decode_value(uint8_t code, int format);                    /* :48-56 */
float orc_dequantized_weight(const uint8_t* codes, const float* scales, size_t rows,
                             size_t columns, int format, size_t row, size_t column); /* :222-235 */
/* Signed integer weight w(n,k) for every element, [rows, columns] int8. */
void orc_unpack_weights(const uint8_t* codes, size_t rows, size_t columns, int format,
                        int8_t* out);

/* ---- activation quantizers (src/kernels/lowbit_gemv.hip) ----------------- */
int orc_quantize_activation_i4(const uint16_t* input_f16, uint8_t* packed, uint16_t* scales_f16,
                               size_t columns, unsigned batch);    /* :373-407, :1067-1087 */
int orc_quantize_activation_i8(const uint16_t* input_f16, int8_t* codes, uint16_t* scales_f16,
                               size_t columns, unsigned batch);    /* :409-436, :1089-1109 */
/* Signed A4 codes -> int8 [batch, columns] (low nibble = even column). */
void orc_unpack_a4(const uint8_t* packed, size_t columns, unsigned batch, int8_t* out);

/* ---- integer GEMM + fp32 epilogue (lowbit_gemv.hip:461-553, 682-755) ---- */
/* w: int8 [N, K] signed weights; a: int8 [B, K] signed activations.
 * partials: int32 [B, N, G]  P[b,n,g] = sum_{k in g} w(n,k) a(b,k). */
void orc_gemm_partials(const int8_t* w, const int8_t* a, size_t rows, size_t columns,
                       unsigned batch, int32_t* partials);
/* y[b,n] = fmaf(float(P[b,n,g]), ws16(n,g) * as16(b,g), y) over g in order. */
void orc_gemm_epilogue(const int32_t* partials, const uint16_t* ws16, const uint16_t* as16,
                       size_t rows, size_t columns, unsigned batch, float* out);
/* The same epilogue with K cut into splits and ranges (the library's GEMM order):
 * plane s = ranges of split s, each a sequential epilogue, added in range order.
 * out: fp32 [splits, B, N]; splits = 1, one range = orc_gemm_epilogue. */
void orc_gemm_epilogue_ranges(const int32_t* partials, const uint16_t* ws16, const uint16_t* as16,
                              size_t rows, size_t columns, unsigned batch, unsigned splits, float* out);
/* Dequant-dot GEMV of the reference harness check (src/cli/main.cpp:1468-1495):
 * y[b,n] = fma chain over k of (w(n,k)*ws(n,g)) * (a(b,k)*as(b,g)).  OpenMP over rows. */
void orc_dequant_dot_gemv(const int8_t* w, const float* ws, const int8_t* a, const uint16_t* as16,
                          size_t rows, size_t columns, unsigned batch, float* out);
/* Same but reading W codes in the reference packed layout (no int8 expansion). */
void orc_dequant_dot_gemv_packed(const uint8_t* codes, int format, const float* ws,
                                 const int8_t* a, const uint16_t* as16, size_t rows,
                                 size_t columns, unsigned batch, float* out);
int orc_max_threads(void);

/* ---- decoder ops (src/kernels/qwen_ops.hip) ----------------------------- */
void orc_rms_norm(const uint16_t* in_f16, const uint16_t* w_bf16, uint16_t* out_f16,
                  size_t elements, unsigned batch, float epsilon, int unit_offset); /* :31-63 */
void orc_residual_add_rms_norm(const uint16_t* residual_f16, const float* update,
                               uint16_t* residual_out_f16, const uint16_t* w_bf16,
                               uint16_t* normalized_f16, size_t elements, unsigned batch,
                               float epsilon, int unit_offset);             /* :176-217 */
void orc_dual_rms_norm_concat(const uint16_t* left, const uint16_t* left_w,
                              const uint16_t* right, const uint16_t* right_w, uint16_t* out,
                              size_t elements, float epsilon, int unit_offset); /* :65-106 */
int orc_silu_multiply_quantize_i4(const float* gate, const float* up, uint8_t* packed,
                                  uint16_t* scales_f16, size_t columns, unsigned batch); /* :120-163 */
void orc_silu_multiply(const float* gate, const float* up, uint16_t* out_f16, size_t n); /* :108-118 */

/* GDN causal conv (qwen_ops.hip:219-261).  state/log fp16, proj fp32 [T, C]. */
void orc_gdn_conv_update(const float* projected, const uint16_t* w_bf16,
                         const uint16_t* initial_state, uint16_t* final_state,
                         uint16_t* out_f16, uint16_t* appended_log, size_t channels,
                         unsigned tokens);
/* Gated delta rule over a window (qwen_ops.hip:263-411), parameterized by head counts.
 * qkv fp16 [T, 2*Hk*d + Hv*d]; z fp32 [T, Hv*d]; a,b fp32 [T, Hv]; states fp32 [Hv, d, d]
 * (row k, column v).  Logs may be NULL. */
void orc_gdn_recurrent(const uint16_t* qkv, const float* z, const float* a, const float* b,
                       const uint16_t* a_log_bf16, const uint16_t* dt_bias_bf16,
                       const uint16_t* norm_w_bf16, const float* initial_states,
                       float* final_states, uint16_t* out_f16, float* key_log, float* delta_log,
                       float* decay_log, unsigned tokens, unsigned key_heads,
                       unsigned value_heads, unsigned head_size);
/* Replay of accepted tokens onto pre-window state (qwen_ops.hip:413-539). */
void orc_gdn_restore_conv(uint16_t* state, const uint16_t* appended_log, size_t channels,
                          unsigned accepted);
void orc_gdn_restore_recurrent(float* states, const float* key_log, const float* delta_log,
                               const float* decay_log, unsigned accepted, unsigned key_heads,
                               unsigned value_heads, unsigned head_size);

/* Per-head RMSNorm(1+w) + partial rotate-half RoPE (qwen_ops.hip:599-676). */
void orc_head_norm_rope(const float* input, size_t input_stride, const uint16_t* w_bf16,
                        uint16_t* out_f16, size_t head_count, size_t head_size,
                        size_t rotary, uint64_t base_position, unsigned tokens, float theta);
/* K/V append into contiguous cache [pos][Hkv][hd] (qwen_ops.hip:678-696). */
void orc_kv_append(const uint16_t* key_f16, const float* value, uint16_t* key_cache,
                   uint16_t* value_cache, size_t position, size_t kv_elements, unsigned tokens);
/* Causal gated GQA decode attention (qwen_ops.hip:698-766), parameterized. */
void orc_gated_attention(const uint16_t* query_f16, const float* gate_src, const uint16_t* key_cache,
                         const uint16_t* value_cache, uint16_t* out_f16, size_t base_token_count,
                         unsigned tokens, unsigned q_heads, unsigned kv_heads, unsigned head_size,
                         float score_scale);
/* Row argmax, ties -> lowest index (qwen_ops.hip:768-807). */
void orc_argmax(const float* logits, size_t vocabulary, size_t stride, unsigned rows,
                const uint32_t* token_ids, uint32_t* out);
/* Acceptance (qwen_runtime.cpp:1497-1501): first i < D with drafts[i] != targets[i]. */
size_t orc_accept(const uint32_t* drafts, const uint32_t* targets, size_t draft_count);
/* Synthetic checkpoint values, elements first .. first+count-1 (not a reference algorithm:
 * the generator of gfxinfer_model_create_synthetic; oracle.py's synthetic_values is the
 * same function in numpy). */
void orc_synthetic_values(uint64_t seed_xor_name_hash, size_t first, size_t count, float sigma,
                          float mean, float* out);

#ifdef __cplusplus
}
#endif
#endif
