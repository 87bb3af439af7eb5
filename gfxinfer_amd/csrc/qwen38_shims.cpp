// The reference's scratch-free launch signatures at its own model's fixed shapes
// (qwen_ops.h:101-127 launch_gdn_recurrent_decode[_block], :246-276
// launch_gated_attention_decode[_block][_indirect_position]; shapes from
// qwen38_spec.h:22-29: attention 24 Q / 4 KV heads x 256, GDN 16 key / 48 value heads
// x 128).  The reference keeps the GDN mixed output inside its kernel and walks the
// attention context serially in one block, so its signatures carry no workspace; the
// kernels here need one (the GDN window's fp32 mixed rows, the attention's split-local
// partials).  It comes from a device buffer the caller binds to the launch stream once,
// before any graph capture (the reference issues everything on one stream per Engine,
// engine.cpp:170), so every launch below only looks the buffer up on the host and
// allocates nothing: the calls stay capture-safe (qwen_runtime.cpp:653-654).
#include <mutex>
#include <unordered_map>

#include "common.hpp"

using namespace gfx950;

namespace {

constexpr uint32_t kQueryHeads = 24, kKvHeads = 4, kAttentionHead = 256;
constexpr uint32_t kGdnKeyHeads = 16, kGdnValueHeads = 48, kGdnHead = 128;
constexpr uint32_t kMaxBatch = 32;

struct Scratch {
  char* base{nullptr};
  std::size_t bytes{0};
  uint32_t max_batch{0};
  std::size_t capacity{0};
};

std::mutex& registry_mutex() {
  static std::mutex m;
  return m;
}
std::unordered_map<hipStream_t, Scratch>& registry() {
  static std::unordered_map<hipStream_t, Scratch> r;
  return r;
}

std::size_t align256(std::size_t x) { return (x + 255u) & ~static_cast<std::size_t>(255u); }

std::size_t attention_part(uint32_t max_batch, std::size_t capacity) {
  return align256(gfxinfer_attention_workspace_bytes(max_batch, kQueryHeads, kAttentionHead, capacity));
}

std::size_t gdn_part(uint32_t max_batch) {
  return align256(static_cast<std::size_t>(max_batch) * kGdnValueHeads * kGdnHead * sizeof(float));
}

int32_t lookup(hipStream_t stream, uint32_t batch, Scratch& out) {
  std::lock_guard<std::mutex> lock(registry_mutex());
  const auto it = registry().find(stream);
  if (it == registry().end()) {
    return fail(GFXI_INVALID_ARGUMENT, "no scratch is bound to this stream (gfxinfer_qwen38_bind_scratch)");
  }
  if (batch == 0 || batch > it->second.max_batch) {
    return fail(GFXI_INVALID_ARGUMENT, "batch exceeds the batch the stream's scratch was bound for");
  }
  out = it->second;
  return ok();
}

int32_t attention(const uint16_t* query, const float* gate, const uint16_t* key_cache,
                  const uint16_t* value_cache, uint16_t* output, size_t base_token_count,
                  const uint64_t* device_base_position, size_t capacity, uint32_t batch, void* stream) {
  Scratch s;
  if (const int32_t status = lookup(static_cast<hipStream_t>(stream), batch, s); status != GFXI_OK) return status;
  if (capacity > s.capacity) {
    return fail(GFXI_INVALID_ARGUMENT, "capacity exceeds the capacity the stream's scratch was bound for");
  }
  float* workspace = reinterpret_cast<float*>(s.base);
  const std::size_t bytes = attention_part(s.max_batch, s.capacity);
  if (device_base_position != nullptr) {
    return gfxinfer_launch_gated_attention_decode_block_indirect_position(
        query, gate, key_cache, value_cache, output, device_base_position, capacity, batch, kQueryHeads, kKvHeads,
        kAttentionHead, workspace, bytes, stream);
  }
  return gfxinfer_launch_gated_attention_decode_block(query, gate, key_cache, value_cache, output,
                                                      base_token_count, capacity, batch, kQueryHeads, kKvHeads,
                                                      kAttentionHead, workspace, bytes, stream);
}

}  // namespace

extern "C" size_t gfxinfer_qwen38_scratch_bytes(uint32_t max_batch, size_t capacity) {
  if (max_batch == 0 || max_batch > kMaxBatch || capacity == 0) return 0;
  return attention_part(max_batch, capacity) + gdn_part(max_batch);
}

extern "C" int32_t gfxinfer_qwen38_bind_scratch(void* stream, void* scratch, size_t bytes, uint32_t max_batch,
                                                size_t capacity) {
  return guarded([&]() -> int32_t {
    const std::size_t need = gfxinfer_qwen38_scratch_bytes(max_batch, capacity);
    if (scratch == nullptr || need == 0 || capacity > (1u << 24) ||
        reinterpret_cast<uintptr_t>(scratch) % 256 != 0) {
      return fail(GFXI_INVALID_ARGUMENT, "invalid scratch binding (256-byte aligned buffer, batch 1..32)");
    }
    if (bytes < need) return fail(GFXI_INVALID_ARGUMENT, "scratch is smaller than gfxinfer_qwen38_scratch_bytes()");
    std::lock_guard<std::mutex> lock(registry_mutex());
    registry()[static_cast<hipStream_t>(stream)] = Scratch{static_cast<char*>(scratch), bytes, max_batch, capacity};
    return ok();
  });
}

extern "C" int32_t gfxinfer_qwen38_unbind_scratch(void* stream) {
  return guarded([&]() -> int32_t {
    std::lock_guard<std::mutex> lock(registry_mutex());
    if (registry().erase(static_cast<hipStream_t>(stream)) == 0) {
      return fail(GFXI_INVALID_ARGUMENT, "no scratch is bound to this stream");
    }
    return ok();
  });
}

// qwen_ops.h:246-254 / qwen_ops.hip:1404-1424: one token over token_count positions.
extern "C" int32_t gfxinfer_qwen38_launch_gated_attention_decode(const uint16_t* query, const float* gate,
                                                                 const uint16_t* key_cache,
                                                                 const uint16_t* value_cache, uint16_t* output,
                                                                 size_t token_count, size_t capacity,
                                                                 void* stream) {
  if (token_count == 0 || token_count > capacity) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid gated attention decode arguments");
  }
  return attention(query, gate, key_cache, value_cache, output, token_count, nullptr, capacity, 1, stream);
}

// qwen_ops.h:256-265 / qwen_ops.hip:1426-1450.
extern "C" int32_t gfxinfer_qwen38_launch_gated_attention_decode_block(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, size_t base_token_count, size_t capacity, uint32_t batch, void* stream) {
  return attention(query, gate, key_cache, value_cache, output, base_token_count, nullptr, capacity, batch,
                   stream);
}

// qwen_ops.h:267-276 / qwen_ops.hip:1452-1477.
extern "C" int32_t gfxinfer_qwen38_launch_gated_attention_decode_block_indirect_position(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, const uint64_t* device_base_position, size_t capacity, uint32_t batch, void* stream) {
  if (device_base_position == nullptr) return fail(GFXI_INVALID_ARGUMENT, "indirect position is null");
  return attention(query, gate, key_cache, value_cache, output, 0, device_base_position, capacity, batch,
                   stream);
}

// qwen_ops.h:113-127 / qwen_ops.hip:1076-1107: the block form with logs (any may be null).
extern "C" int32_t gfxinfer_qwen38_launch_gdn_recurrent_decode_block(
    const uint16_t* convolved_qkv, const float* projected_z, const float* projected_a, const float* projected_b,
    const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias, const uint16_t* bf16_norm_weight,
    const float* initial_recurrent_state, float* final_recurrent_state, uint16_t* output, float* key_log,
    float* delta_log, float* decay_log, uint32_t batch, void* stream) {
  Scratch s;
  if (const int32_t status = lookup(static_cast<hipStream_t>(stream), batch, s); status != GFXI_OK) return status;
  float* mixed = reinterpret_cast<float*>(s.base + attention_part(s.max_batch, s.capacity));
  return gfxinfer_launch_gdn_recurrent_decode_block(
      convolved_qkv, projected_z, projected_a, projected_b, bf16_a_log, bf16_dt_bias, bf16_norm_weight,
      initial_recurrent_state, final_recurrent_state, output, key_log, delta_log, decay_log, batch, kGdnKeyHeads,
      kGdnValueHeads, kGdnHead, mixed, stream);
}

// qwen_ops.h:101-111 / qwen_ops.hip:1049-1074: one token, state updated in place, no logs.
extern "C" int32_t gfxinfer_qwen38_launch_gdn_recurrent_decode(
    const uint16_t* convolved_qkv, const float* projected_z, const float* projected_a, const float* projected_b,
    const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias, const uint16_t* bf16_norm_weight,
    float* recurrent_state, uint16_t* output, void* stream) {
  if (recurrent_state == nullptr) return fail(GFXI_INVALID_ARGUMENT, "recurrent state is null");
  return gfxinfer_qwen38_launch_gdn_recurrent_decode_block(convolved_qkv, projected_z, projected_a, projected_b,
                                                           bf16_a_log, bf16_dt_bias, bf16_norm_weight,
                                                           recurrent_state, recurrent_state, output, nullptr,
                                                           nullptr, nullptr, 1, stream);
}
