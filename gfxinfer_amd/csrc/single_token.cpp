// Single-token launchers of the reference's decode path (qwen_ops.h:83,101,130,217,246,278):
// the one-token calls its greedy_step and MTP proposal make.  Each is the block launcher
// of the same operation at batch 1 (same kernels, so the outputs are bit-identical to
// the block form's first token), with the reference's argument meaning: states updated
// in place, the attention's token_count = cached positions the token attends to, one
// layer's logs for the restore.  Head counts are parameters here, where the reference
// hard-codes its model's (10240 conv channels, 48 value heads, 24/4 attention heads).
#include "common.hpp"

using namespace gfx950;

// qwen_ops.hip:999-1018: conv state [channels][4] advanced in place by one token.
extern "C" int32_t gfxinfer_launch_gdn_conv_update(const float* projected_qkv,
                                                   const uint16_t* bf16_conv_weight,
                                                   uint16_t* conv_state, uint16_t* convolved_qkv,
                                                   size_t channels, void* stream) {
  if (conv_state == nullptr) return fail(GFXI_INVALID_ARGUMENT, "invalid GDN convolution arguments");
  return gfxinfer_launch_gdn_conv_update_block(projected_qkv, bf16_conv_weight, conv_state, conv_state,
                                               convolved_qkv, nullptr, channels, 1, stream);
}

// qwen_ops.hip:1049-1074: recurrent state [value_heads][128][128] advanced in place by one
// token, no logs.  Each workgroup reads its own state columns before it writes them, so the
// window kernel updates in place.
extern "C" int32_t gfxinfer_launch_gdn_recurrent_decode(
    const uint16_t* convolved_qkv, const float* projected_z, const float* projected_a,
    const float* projected_b, const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias,
    const uint16_t* bf16_norm_weight, float* recurrent_state, uint16_t* output, uint32_t key_heads,
    uint32_t value_heads, uint32_t head_size, float* mixed_workspace, void* stream) {
  return gfxinfer_launch_gdn_recurrent_decode_block(
      convolved_qkv, projected_z, projected_a, projected_b, bf16_a_log, bf16_dt_bias, bf16_norm_weight,
      recurrent_state, recurrent_state, output, nullptr, nullptr, nullptr, 1, key_heads, value_heads,
      head_size, mixed_workspace, stream);
}

// qwen_ops.hip:1109-1139: one layer's states rolled forward over its first accepted_tokens
// logged tokens (logs [logged tokens][...] of that layer).
extern "C" int32_t gfxinfer_launch_gdn_restore_prefix(
    uint16_t* conv_state, float* recurrent_state, const uint16_t* appended_log, const float* key_log,
    const float* delta_log, const float* decay_log, size_t channels, uint32_t accepted_tokens,
    uint32_t key_heads, uint32_t value_heads, uint32_t head_size, void* stream) {
  if (accepted_tokens == 0) return fail(GFXI_INVALID_ARGUMENT, "invalid GDN prefix restore arguments");
  return gfxinfer_launch_gdn_restore_prefix_all(conv_state, recurrent_state, appended_log, key_log,
                                                delta_log, decay_log, channels, 1, accepted_tokens,
                                                accepted_tokens, key_heads, value_heads, head_size,
                                                stream);
}

// qwen_ops.hip:1328-1346: K (fp16) and V (fp32 -> fp16) of one token at `position`.
extern "C" int32_t gfxinfer_launch_kv_append(const uint16_t* key, const float* value,
                                             uint16_t* key_cache, uint16_t* value_cache,
                                             size_t position, size_t capacity, size_t kv_elements,
                                             void* stream) {
  if (position >= capacity) return fail(GFXI_INVALID_ARGUMENT, "invalid KV append arguments");
  return gfxinfer_launch_kv_append_block(key, value, key_cache, value_cache, position, capacity, 1,
                                         kv_elements, stream);
}

// qwen_ops.hip:1404-1424: one token attending to the first token_count cached positions.
extern "C" int32_t gfxinfer_launch_gated_attention_decode(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, size_t token_count, size_t capacity, uint32_t q_heads, uint32_t kv_heads,
    uint32_t head_size, float* workspace, size_t workspace_bytes, void* stream) {
  if (token_count == 0 || token_count > capacity) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid gated attention decode arguments");
  }
  return gfxinfer_launch_gated_attention_decode_block(query, gate, key_cache, value_cache, output,
                                                      token_count, capacity, 1, q_heads, kv_heads,
                                                      head_size, workspace, workspace_bytes, stream);
}

// qwen_ops.hip:1479-1494: argmax of one logits row (ties: lowest index).
extern "C" int32_t gfxinfer_launch_argmax(const float* logits, uint32_t* token, size_t vocabulary_size,
                                          void* stream) {
  return gfxinfer_launch_argmax_batch(logits, token, vocabulary_size, vocabulary_size, 1, stream);
}
