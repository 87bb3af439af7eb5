// Decode session of the MTP speculative-verify path: one device arena of
// activations, states, logs and caches; the 64-layer causal verifier over a
// block of <= 32 tokens; the MTP proposal chain; acceptance on the device; GDN
// rollback by replay of the logged prefix or by a state-buffer swap; the chain +
// verifier captured as two hipGraphs (one per state-buffer parity).
//
// Reference: src/qwen_runtime.cpp (QwenDecodeSession), cited per function.
// Differences of design, not of semantics: every projection consumes A4 codes
// written by the producing kernel (fused norm -> A4, SwiGLU -> A4, GDN output norm
// -> A4); the acceptance rule runs on the device, so a round downloads one small
// result record instead of the drafts and target tokens.
#include <algorithm>
#include <array>
#include <chrono>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"
#include "runtime.hpp"

#define GFXI_TRY(expr)                      \
  do {                                      \
    const int32_t status_ = (expr);         \
    if (status_ != GFXI_OK) return status_; \
  } while (0)

namespace gfx950 {
namespace {

constexpr unsigned kMaxBlock = 32;  // qwen_runtime.cpp:40 kMaximumBlock
constexpr std::size_t kMaxPlanes = 8;  // split-K planes of a projection (GEMM entry limit)

struct Matrix {
  int32_t format{0};
  const uint8_t* weights{nullptr};
  const uint16_t* scales{nullptr};
  std::size_t rows{0};
  std::size_t columns{0};
};

// qwen_runtime.cpp:49-71 LayerBindings.
struct Layer {
  bool attention{false};
  std::size_t state_index{0};
  const uint16_t* input_norm{nullptr};
  const uint16_t* post_norm{nullptr};
  Matrix gate, up, down;
  Matrix q, k, v, o;
  const uint16_t* q_norm{nullptr};
  const uint16_t* k_norm{nullptr};
  Matrix qkv, z, a, b, out;
  const uint16_t* conv{nullptr};
  const uint16_t* a_log{nullptr};
  const uint16_t* dt_bias{nullptr};
  const uint16_t* gdn_norm{nullptr};
};

struct Graph {
  hipGraph_t graph{nullptr};
  hipGraphExec_t exec{nullptr};
};

// Per-round device scalars of the captured graphs (qwen_runtime.cpp:888-925 uploads
// them with three host copies; one tiny kernel writes them from its arguments here).
struct RoundScalars {
  uint32_t seed;
  int32_t forced;  // < 0: no acceptance override
  uint64_t base_position;
  uint64_t mtp_position;
};

// Result record written by accept_kernel: [0] accepted drafts, [1] token count,
// [2..] tokens (accepted drafts, then the target token at index accepted).
constexpr unsigned kResultWords = 2 + kMaxBlock;

__global__ void round_scalars_kernel(RoundScalars values, uint32_t* seed, int32_t* forced,
                                     uint64_t* base_position, uint64_t* mtp_positions,
                                     uint32_t draft_count) {
  const unsigned i = threadIdx.x;
  if (i == 0) {
    *seed = values.seed;
    *forced = values.forced;
    *base_position = values.base_position;
  }
  if (i < draft_count) mtp_positions[i] = values.mtp_position + i;
}

struct PlantedDrafts {
  uint32_t token[kMaxBlock];
};

__global__ void planted_drafts_kernel(PlantedDrafts values, uint32_t* drafts, uint32_t count) {
  if (threadIdx.x < count) drafts[threadIdx.x] = values.token[threadIdx.x];
}

// qwen_runtime.cpp:1497-1501 + 1537-1543: accepted = first i < D with
// drafts[i] != targets[i] (else D); tokens = drafts[:accepted] + [targets[accepted]].
__global__ void accept_kernel(const uint32_t* __restrict__ drafts,
                              const uint32_t* __restrict__ targets, const int32_t* forced,
                              uint32_t draft_count, uint32_t* __restrict__ result) {
  const unsigned lane = threadIdx.x;  // one wave of 64 >= 32 lanes
  const bool mismatch = lane < draft_count && drafts[lane] != targets[lane];
  const unsigned long long ballot = __ballot(mismatch);
  uint32_t accepted = ballot == 0 ? draft_count : static_cast<uint32_t>(__ffsll(ballot) - 1);
  const int32_t override_value = *forced;
  if (override_value >= 0) accepted = min(static_cast<uint32_t>(override_value), draft_count);
  if (lane == 0) {
    result[0] = accepted;
    result[1] = accepted + 1;
  }
  if (lane < accepted) result[2 + lane] = drafts[lane];
  if (lane == accepted) result[2 + lane] = targets[lane];
}

std::size_t align256(std::size_t x) { return (x + 255u) & ~static_cast<std::size_t>(255u); }

}  // namespace
}  // namespace gfx950

using namespace gfx950;

struct gfxinfer_session {
  gfxinfer_model* model{nullptr};
  gfxinfer_model_spec spec{};
  gfxinfer_session_config config{};
  gfxinfer_session_summary summary{};
  hipStream_t stream{nullptr};

  // Shape shorthands.
  std::size_t H{0}, I{0}, q_rows{0}, kv_rows{0}, attn_width{0};
  std::size_t gdn_key{0}, gdn_value{0}, channels{0}, V{0};
  std::size_t gdn_layers{0}, attn_layers{0};

  std::size_t current_position{0};
  std::size_t mtp_position{0};
  bool mtp_chain_active{false};
  bool record_rollback{false};
  bool parity{false};
  // Test hook: when set, eager verifier passes copy each layer's stage boundaries into
  // this device buffer (layout: trace_layout()).
  uint8_t* layer_trace{nullptr};
  const uint16_t* last_hidden{nullptr};

  std::vector<Layer> layers;
  Layer mtp;
  Matrix embedding, lm_head, draft_head, mtp_fc;
  const uint32_t* draft_token_ids{nullptr};  // draft-head row -> token id (null: identity)
  const uint16_t* final_norm{nullptr};
  const uint16_t* mtp_pre_embedding_norm{nullptr};
  const uint16_t* mtp_pre_hidden_norm{nullptr};
  const uint16_t* mtp_final_norm{nullptr};

  uint8_t* arena{nullptr};
  std::size_t arena_bytes{0};
  struct Buffer {
    const char* name;
    void** slot;
    std::size_t bytes;
  };
  std::vector<Buffer> buffers;

  uint16_t *hidden_a{}, *hidden_b{}, *post_attention{}, *mtp_hidden{}, *target_hidden_snapshot{};
  uint16_t *mtp_concat{}, *mtp_input{}, *convolved{}, *query{}, *key{}, *attention_output{};
  uint16_t* mtp_conditioning{};  // [32][H] target hidden states of a batched MTP update
  uint8_t* act_codes{};
  uint16_t* act_scales{};
  float *projected_main{}, *projected_z{}, *projected_a{}, *projected_b{}, *projected_k{};
  float *projected_v{}, *gdn_mixed{}, *mixer_update{}, *gate_output{}, *up_output{};
  float *mlp_update{}, *logits{}, *attention_workspace{};
  float* rope_table{};  // (cos, sin) per (position, rotary frequency), filled at creation
  // Split-K plane counts of the last projections into mixer_update / mlp_update.
  uint32_t mixer_planes = 1, mlp_planes = 1;
  void* argmax_keys{};
  std::size_t argmax_keys_bytes{0};
  std::size_t attention_workspace_bytes{0};
  uint32_t *selected{}, *draft_tokens{}, *verify_drafts{}, *result{}, *graph_seed{};
  // A4 input of the down projection (SwiGLU output), apart from act_codes
  uint8_t* mlp_codes{};
  uint16_t* mlp_scales{};
  int32_t* graph_forced{};
  uint64_t *graph_base_position{}, *graph_mtp_positions{};
  uint16_t *conv_states{}, *conv_snapshot{}, *conv_log{};
  float *gdn_states{}, *gdn_snapshot{}, *key_log{}, *delta_log{}, *decay_log{};
  uint16_t *key_caches{}, *value_caches{}, *mtp_key_cache{}, *mtp_value_cache{};
  uint32_t* host_result{nullptr};  // pinned

  std::array<Graph, 2> graphs{};

  ~gfxinfer_session() {
    if (model != nullptr) (void)hipSetDevice(model->device);
    if (stream != nullptr) (void)hipStreamSynchronize(stream);
    for (auto& g : graphs) {
      if (g.exec != nullptr) (void)hipGraphExecDestroy(g.exec);
      if (g.graph != nullptr) (void)hipGraphDestroy(g.graph);
    }
    if (host_result != nullptr) (void)hipHostFree(host_result);
    if (arena != nullptr) (void)hipFree(arena);
    if (model != nullptr) release_model_reference(model);
  }

  // ---- sizes of the per-layer state -----------------------------------------
  std::size_t conv_state_elements() const { return channels * 4; }
  std::size_t gdn_state_elements() const {
    return static_cast<std::size_t>(spec.gdn_value_head_count) * spec.gdn_head_size *
           spec.gdn_head_size;
  }

  // ---- projections (qwen_runtime.cpp:78-148, 263-347) -------------------------
  // Every projection reads the A4 codes/scales left in act_codes/act_scales by the
  // kernel that produced its input.
  int32_t gemm(const Matrix& m, float* out, unsigned batch) {
    return gfxinfer_launch_gfx950_i4_gemm(m.format, m.weights, m.scales, act_codes, act_scales,
                                          out, m.rows, m.columns, batch, 0, stream);
  }
  // [hidden, K] projections that feed a residual RMSNorm: split-K planes when the
  // plain grid would leave the GPU underfilled; the norm sums them.
  int32_t gemm_planes(const Matrix& m, float* out, unsigned batch, uint32_t& planes,
                      const uint8_t* codes = nullptr, const uint16_t* scales = nullptr) {
    planes = gfxinfer_gemm_split_count(m.rows, m.columns, batch);
    return gfxinfer_launch_gfx950_i4_gemm_split(m.format, m.weights, m.scales,
                                                codes != nullptr ? codes : act_codes,
                                                scales != nullptr ? scales : act_scales, out, m.rows,
                                                m.columns, batch, planes, stream);
  }
  int32_t gemm_fused(std::initializer_list<std::pair<const Matrix*, float*>> list,
                     unsigned batch) {
    std::array<gfxinfer_fused_matrix, 4> bind{};
    std::size_t n = 0;
    const Matrix* first = list.begin()->first;
    bool same = true;
    for (const auto& [m, out] : list) {
      same = same && m->format == first->format && m->columns == first->columns;
      bind[n++] = {m->weights, m->scales, out, m->rows};
    }
    if (!same) {
      for (const auto& [m, out] : list) GFXI_TRY(gemm(*m, out, batch));
      return ok();
    }
    return gfxinfer_launch_gfx950_i4_gemm_fused(first->format, bind.data(), n, act_codes,
                                                act_scales, first->columns, batch, 0, stream);
  }

  // Head projection fused with greedy argmax (qwen_runtime.cpp:635-639, 859-866); the
  // fp32 logits are kept only when the session was configured to keep them.
  int32_t gemm_argmax(const Matrix& m, unsigned batch, std::size_t argmax_rows, uint32_t* tokens,
                      const uint32_t* token_ids = nullptr) {
    return gfxinfer_launch_gfx950_i4_gemm_argmax(
        m.format, m.weights, m.scales, act_codes, act_scales,
        config.keep_logits != 0 ? logits : nullptr, m.rows, m.columns, batch, argmax_rows, token_ids,
        argmax_keys, argmax_keys_bytes, tokens, stream);
  }

  // Embedding rows of `count` tokens in one launch (row j at destination + j * H): token
  // 0 from *first (device) or host[0], tokens j >= 1 from rest[j - 1] (device) or host[j].
  int32_t gather_rows(uint16_t* destination, const uint32_t* host, const uint32_t* first,
                      const uint32_t* rest, unsigned count) {
    return gfxinfer_launch_lowbit_row_gather_tiled_batch(embedding.format, embedding.weights,
                                                         embedding.scales, destination, host, first, rest,
                                                         count, embedding.rows, embedding.columns, stream);
  }

  // Attention mixer of a block (qwen_runtime.cpp:432-474); input A4 codes ready.
  int32_t attention_mixer(const Layer& L, uint16_t* key_cache, uint16_t* value_cache,
                          unsigned batch, std::size_t position, const uint64_t* device_position,
                          bool stop_after_append) {
    GFXI_TRY(gemm_fused({{&L.q, projected_main}, {&L.k, projected_k}, {&L.v, projected_v}}, batch));
    const std::size_t hd = spec.attention_head_size;
    if (!stop_after_append && gfxinfer_fused_rope_attention_supported(batch, spec.attention_head_count,
                                                                      spec.kv_head_count,
                                                                      static_cast<uint32_t>(hd)) != 0) {
      // Blocks of up to eight tokens (the MTP proposal, short verifier blocks): Q/K norm +
      // RoPE, the K/V append and the attention in two launches, the split workgroups doing
      // the RoPE step with the session's cos / sin table; the same values as the three
      // launches below.
      if (device_position == nullptr) {
        GFXI_TRY(gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4(
            projected_main, L.q_norm, 2 * hd, projected_k, L.k_norm, hd, projected_v, spec.rotary_size,
            spec.rope_theta, rope_table, projected_main, key_cache, value_cache, attention_output, act_codes,
            act_scales, position, config.maximum_context_tokens, batch, spec.attention_head_count,
            spec.kv_head_count, spec.attention_head_size, attention_workspace, attention_workspace_bytes,
            stream));
      } else {
        GFXI_TRY(gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4_indirect_position(
            projected_main, L.q_norm, 2 * hd, projected_k, L.k_norm, hd, projected_v, spec.rotary_size,
            spec.rope_theta, rope_table, projected_main, key_cache, value_cache, attention_output, act_codes,
            act_scales, device_position, config.maximum_context_tokens, batch, spec.attention_head_count,
            spec.kv_head_count, spec.attention_head_size, attention_workspace, attention_workspace_bytes,
            stream));
      }
      GFXI_TRY(trace_codes(L, true, attn_width, batch));
      return gemm_planes(L.o, mixer_update, batch, mixer_planes);
    }
    // Q/K norm + RoPE and the K/V cache append of the block in one launch (the
    // reference's launch pair, bit for bit).
    if (device_position == nullptr) {
      GFXI_TRY(gfxinfer_launch_qk_rms_norm_rope_kv_append_block(
          projected_main, L.q_norm, query, spec.attention_head_count, 2 * hd, projected_k,
          L.k_norm, key, spec.kv_head_count, hd, hd, spec.rotary_size, projected_v, key_cache,
          value_cache, config.maximum_context_tokens, position, batch, spec.rope_theta, stream));
    } else {
      GFXI_TRY(gfxinfer_launch_qk_rms_norm_rope_kv_append_block_indirect_position(
          projected_main, L.q_norm, query, spec.attention_head_count, 2 * hd, projected_k,
          L.k_norm, key, spec.kv_head_count, hd, hd, spec.rotary_size, projected_v, key_cache,
          value_cache, config.maximum_context_tokens, device_position, batch, spec.rope_theta,
          stream));
    }
    if (stop_after_append) return ok();
    // Attention with the o projection's A4 quantizer in its combine launch.
    if (device_position == nullptr) {
      GFXI_TRY(gfxinfer_launch_gated_attention_decode_block_quantize_i4(
          query, projected_main, key_cache, value_cache, attention_output, act_codes, act_scales,
          position + 1, config.maximum_context_tokens, batch, spec.attention_head_count,
          spec.kv_head_count, spec.attention_head_size, attention_workspace,
          attention_workspace_bytes, stream));
    } else {
      GFXI_TRY(gfxinfer_launch_gated_attention_decode_block_quantize_i4_indirect_position(
          query, projected_main, key_cache, value_cache, attention_output, act_codes, act_scales,
          device_position, config.maximum_context_tokens, batch, spec.attention_head_count,
          spec.kv_head_count, spec.attention_head_size, attention_workspace,
          attention_workspace_bytes, stream));
    }
    GFXI_TRY(trace_codes(L, true, attn_width, batch));
    return gemm_planes(L.o, mixer_update, batch, mixer_planes);
  }

  // MLP half of a layer (qwen_runtime.cpp:512-543): residual + post norm -> A4,
  // gate/up, SwiGLU -> A4, down, residual + next norm -> A4 (+ optional fp16 norm).
  int32_t mlp_tail(const Layer& L, const uint16_t* input, uint16_t* output,
                   const uint16_t* next_norm, unsigned batch) {
    GFXI_TRY(gfxinfer_launch_residual_add_rms_norm_quantize_i4_planes(
        input, mixer_update, mixer_planes, post_attention, L.post_norm, nullptr, act_codes,
        act_scales, H, batch, spec.rms_norm_epsilon, 1, stream));
    GFXI_TRY(trace_post(L, batch));
    // The gate/up grid and SwiGLU -> A4 stay two launches: a one-launch form (the
    // workgroup completing each 128-row group writing its codes) measured slower on
    // MI355X, its cross-workgroup completion costing more than the second launch.
    GFXI_TRY(gemm_fused({{&L.gate, gate_output}, {&L.up, up_output}}, batch));
    GFXI_TRY(gfxinfer_launch_silu_multiply_quantize_i4(gate_output, up_output, mlp_codes,
                                                       mlp_scales, I, batch, stream));
    GFXI_TRY(trace_codes(L, false, I, batch, mlp_codes, mlp_scales));
    GFXI_TRY(gemm_planes(L.down, mlp_update, batch, mlp_planes, mlp_codes, mlp_scales));
    return gfxinfer_launch_residual_add_rms_norm_quantize_i4_planes(
        post_attention, mlp_update, mlp_planes, output, next_norm, nullptr, act_codes, act_scales,
        H, batch, spec.rms_norm_epsilon, 1, stream);
  }

  // qwen_runtime.cpp:421-544 launch_layer_block.
  int32_t layer_block(const Layer& L, const uint16_t* input, uint16_t* output, unsigned batch,
                      const uint16_t* next_norm, const uint64_t* device_position) {
    if (L.attention) {
      const std::size_t offset = L.state_index * config.maximum_context_tokens * kv_rows;
      GFXI_TRY(attention_mixer(L, key_caches + offset, value_caches + offset, batch,
                               current_position, device_position, false));
    } else {
      GFXI_TRY(gemm_fused({{&L.qkv, projected_main},
                           {&L.z, projected_z},
                           {&L.a, projected_a},
                           {&L.b, projected_b}},
                          batch));
      // The window always writes its final states into the snapshot buffers (the fused
      // conv cannot update in place); the caller keeps them by swapping buffers, or,
      // after a partial acceptance, replays the logged prefix onto the originals
      // (qwen_runtime.cpp:484-511 selects the same buffers when recording).
      const uint16_t* conv_state = conv_states + L.state_index * conv_state_elements();
      const float* state = gdn_states + L.state_index * gdn_state_elements();
      uint16_t* conv_final = conv_snapshot + L.state_index * conv_state_elements();
      float* state_final = gdn_snapshot + L.state_index * gdn_state_elements();
      const std::size_t log_token = L.state_index * kMaxBlock;
      GFXI_TRY(gfxinfer_launch_gdn_conv_window(
          projected_main, L.conv, conv_state, conv_final,
          record_rollback ? conv_log + log_token * channels : nullptr, projected_a, projected_b,
          L.a_log, L.dt_bias, state, state_final, gdn_mixed,
          record_rollback ? key_log + log_token * gdn_key : nullptr,
          record_rollback ? delta_log + log_token * gdn_value : nullptr,
          record_rollback ? decay_log + log_token * spec.gdn_value_head_count : nullptr, batch,
          spec.gdn_key_head_count, spec.gdn_value_head_count, spec.gdn_head_size, stream));
      GFXI_TRY(gfxinfer_launch_gdn_output_quantize_i4(gdn_mixed, projected_z, L.gdn_norm, nullptr,
                                                      act_codes, act_scales, batch,
                                                      spec.gdn_value_head_count,
                                                      spec.gdn_head_size, stream));
      GFXI_TRY(trace_codes(L, true, gdn_value, batch));
      GFXI_TRY(gemm_planes(L.out, mixer_update, batch, mixer_planes));
    }
    return mlp_tail(L, input, output, next_norm, batch);
  }

  // Layers + final norm + LM head + argmax over hidden_a[0..batch) (the body shared
  // by block_step and the verifier, qwen_runtime.cpp:615-640 / 1341-1376).
  // Layer trace sections (byte offsets), each sized for kMaxBlock tokens:
  //   residual [layers + 1][32][H] fp16: rows entering layer 0, then leaving each layer;
  //   post [layers][32][H] fp16: rows after the mixer's residual add;
  //   mixer codes [layers][32 * W / 2] + scales [layers][32 * W / 128] fp16: the A4 input
  //     of the o / out projection (W = the wider of the attention and GDN widths);
  //   mlp codes [layers][32 * I / 2] + scales [layers][32 * I / 128] fp16: the SwiGLU
  //     output's A4 codes, the down projection's input.
  // A layer's codes and scales are stored packed as [batch][width / 2] / [batch][width / 128].
  struct TraceLayout {
    std::size_t residual, post, mixer_codes, mixer_scales, mlp_codes, mlp_scales, total;
  };
  TraceLayout trace_layout() const {
    const std::size_t L = layers.size(), W = std::max(attn_width, gdn_value), B = kMaxBlock;
    TraceLayout t{};
    t.residual = 0;
    t.post = t.residual + (L + 1) * B * H * 2;
    t.mixer_codes = t.post + L * B * H * 2;
    t.mixer_scales = t.mixer_codes + L * B * W / 2;
    t.mlp_codes = t.mixer_scales + L * B * (W / 128) * 2;
    t.mlp_scales = t.mlp_codes + L * B * I / 2;
    t.total = t.mlp_scales + L * B * (I / 128) * 2;
    return t;
  }
  int32_t trace_copy(std::size_t offset, const void* source, std::size_t bytes) {
    if (auto e = hipMemcpyAsync(layer_trace + offset, source, bytes, hipMemcpyDeviceToDevice, stream);
        e != hipSuccess) {
      return hip_fail(e, "layer trace copy failed");
    }
    return ok();
  }
  int32_t trace_rows(std::size_t slot, const uint16_t* rows, unsigned batch) {
    if (layer_trace == nullptr) return ok();
    return trace_copy(trace_layout().residual + slot * kMaxBlock * H * 2, rows, batch * H * 2);
  }
  // Index of a decoder layer, or -1 for the MTP block (never traced).
  long layer_index(const Layer& L) const {
    return (&L >= layers.data() && &L < layers.data() + layers.size()) ? &L - layers.data() : -1;
  }
  // The A4 codes and scales in act_codes / act_scales of `width` columns.
  int32_t trace_codes(const Layer& L, bool mixer, std::size_t width, unsigned batch,
                      const uint8_t* codes_from = nullptr, const uint16_t* scales_from = nullptr) {
    const long i = layer_index(L);
    if (layer_trace == nullptr || i < 0) return ok();
    const TraceLayout t = trace_layout();
    const std::size_t W = mixer ? std::max(attn_width, gdn_value) : I;
    const std::size_t codes = (mixer ? t.mixer_codes : t.mlp_codes) + i * kMaxBlock * W / 2;
    const std::size_t scales = (mixer ? t.mixer_scales : t.mlp_scales) + i * kMaxBlock * (W / 128) * 2;
    GFXI_TRY(trace_copy(codes, codes_from != nullptr ? codes_from : act_codes, batch * width / 2));
    return trace_copy(scales, scales_from != nullptr ? scales_from : act_scales, batch * (width / 128) * 2);
  }
  int32_t trace_post(const Layer& L, unsigned batch) {
    const long i = layer_index(L);
    if (layer_trace == nullptr || i < 0) return ok();
    return trace_copy(trace_layout().post + i * kMaxBlock * H * 2, post_attention, batch * H * 2);
  }

  int32_t decoder_stack(unsigned batch, const uint64_t* device_position) {
    GFXI_TRY(gfxinfer_launch_rms_norm_quantize_i4(hidden_a, layers.front().input_norm, nullptr,
                                                  act_codes, act_scales, H, batch,
                                                  spec.rms_norm_epsilon, 1, stream));
    uint16_t* current = hidden_a;
    uint16_t* next = hidden_b;
    GFXI_TRY(trace_rows(0, current, batch));
    for (std::size_t i = 0; i < layers.size(); ++i) {
      const uint16_t* next_norm = i + 1 < layers.size() ? layers[i + 1].input_norm : final_norm;
      GFXI_TRY(layer_block(layers[i], current, next, batch, next_norm, device_position));
      GFXI_TRY(trace_rows(i + 1, next, batch));
      std::swap(current, next);
    }
    return gemm_argmax(lm_head, batch, spec.tokenizer_vocabulary_size, selected);
  }

  // qwen_runtime.cpp:546-640 enqueue_verifier_body: seed + D drafts (device ids).
  int32_t verifier(uint32_t seed, const uint32_t* device_seed, const uint32_t* drafts,
                   unsigned draft_count, const uint64_t* device_position) {
    uint32_t host[kMaxBlock] = {seed};
    GFXI_TRY(gather_rows(hidden_a, host, device_seed, drafts, draft_count + 1));
    return decoder_stack(draft_count + 1, device_position);
  }

  // qwen_runtime.cpp:715-867 launch_mtp_proposal.  output_token == nullptr only
  // advances the MTP K/V cache (826-829).  In a chain, keys_token (not null) takes the
  // token from the previous proposal's draft-head keys left in argmax_keys and writes it
  // there, and reduce == false leaves this proposal's own keys for the next one (its
  // token then reaches *output_token from that proposal's input launch).
  int32_t mtp_proposal(uint32_t token, const uint32_t* device_token, const uint16_t* conditioning,
                       std::size_t position, uint32_t* output_token,
                       const uint64_t* device_position, uint32_t* keys_token = nullptr,
                       bool reduce = true) {
    // embedding gather + dual norm/concat + A4 quantizer in one launch (+ the previous
    // proposal's argmax reduction)
    if (keys_token != nullptr) {
      GFXI_TRY(gfxinfer_launch_mtp_input_quantize_i4_from_keys(
          embedding.format, embedding.weights, embedding.scales, embedding.rows,
          static_cast<const uint64_t*>(argmax_keys), draft_head.rows / 16, draft_token_ids, keys_token,
          mtp_pre_embedding_norm, conditioning, mtp_pre_hidden_norm, nullptr, act_codes, act_scales, H,
          spec.rms_norm_epsilon, 1, stream));
    } else {
      GFXI_TRY(gfxinfer_launch_mtp_input_quantize_i4(
          embedding.format, embedding.weights, embedding.scales, embedding.rows, token, device_token,
          mtp_pre_embedding_norm, conditioning, mtp_pre_hidden_norm, nullptr, act_codes, act_scales, H,
          spec.rms_norm_epsilon, 1, stream));
    }
    GFXI_TRY(gfxinfer_launch_gfx950_i4_gemm_half(mtp_fc.format, mtp_fc.weights, mtp_fc.scales,
                                                 act_codes, act_scales, mtp_input, mtp_fc.rows,
                                                 mtp_fc.columns, 1, 0, stream));
    GFXI_TRY(gfxinfer_launch_rms_norm_quantize_i4(mtp_input, mtp.input_norm, nullptr, act_codes,
                                                  act_scales, H, 1, spec.rms_norm_epsilon, 1,
                                                  stream));
    GFXI_TRY(attention_mixer(mtp, mtp_key_cache, mtp_value_cache, 1, position, device_position,
                             output_token == nullptr));
    if (output_token == nullptr) return ok();
    GFXI_TRY(mlp_tail(mtp, mtp_input, mtp_hidden, mtp_final_norm, 1));
    return gemm_argmax(draft_head, 1, spec.mtp_draft_vocabulary, reduce ? output_token : nullptr,
                       draft_token_ids);
  }

  // The MTP K/V update of mtp_proposal(token, ..., nullptr) for `count` consecutive
  // cache entries at once: entry position + i from tokens[i] and conditioning row i
  // (mtp_conditioning).  Every kernel computes each row as the one-token path does.
  int32_t mtp_sync(const uint32_t* tokens, unsigned count, std::size_t position) {
    GFXI_TRY(gather_rows(hidden_b, tokens, nullptr, nullptr, count));
    GFXI_TRY(gfxinfer_launch_dual_rms_norm_concat_batch(hidden_b, mtp_pre_embedding_norm, mtp_conditioning,
                                                        mtp_pre_hidden_norm, mtp_concat, H, count,
                                                        spec.rms_norm_epsilon, 1, stream));
    GFXI_TRY(gfxinfer_launch_quantize_activation_i4(mtp_concat, act_codes, act_scales, 2 * H, count,
                                                    stream));
    GFXI_TRY(gfxinfer_launch_gfx950_i4_gemm_half(mtp_fc.format, mtp_fc.weights, mtp_fc.scales,
                                                 act_codes, act_scales, mtp_input, mtp_fc.rows,
                                                 mtp_fc.columns, count, 0, stream));
    GFXI_TRY(gfxinfer_launch_rms_norm_quantize_i4(mtp_input, mtp.input_norm, nullptr, act_codes,
                                                  act_scales, H, count, spec.rms_norm_epsilon, 1,
                                                  stream));
    return attention_mixer(mtp, mtp_key_cache, mtp_value_cache, count, position, nullptr, true);
  }

  // Chunked prefill: the target over the prompt in blocks of up to kMaxBlock tokens
  // and, with sync_mtp, the MTP cache over the same positions (entry j from token j + 1
  // and the target hidden state of position j), the state the serial loop of
  // cli/main.cpp:1055-1069 (greedy_step(p0); then mtp_draft(p_i) and greedy_step(p_i))
  // leaves.
  int32_t prefill(const uint32_t* tokens, std::size_t count, bool sync_mtp, uint32_t* next) {
    if (tokens == nullptr || next == nullptr || count == 0 ||
        count > config.maximum_context_tokens - current_position ||
        (sync_mtp && current_position != 0 && mtp_position + 1 != current_position) ||
        (sync_mtp && current_position == 0 && mtp_position != 0)) {
      return fail(GFXI_INVALID_ARGUMENT,
                  "prefill needs 1..context tokens and a fresh or MTP-aligned session");
    }
    uint32_t outputs[kMaxBlock];
    for (std::size_t a = 0; a < count; a += kMaxBlock) {
      const auto T = static_cast<unsigned>(std::min<std::size_t>(kMaxBlock, count - a));
      const bool previous = current_position != 0;  // a hidden state for position a - 1
      if (sync_mtp && previous) {
        if (auto e = hipMemcpyAsync(mtp_conditioning, last_hidden, H * 2, hipMemcpyDeviceToDevice, stream);
            e != hipSuccess) {
          return hip_fail(e, "prefill conditioning copy failed");
        }
      }
      GFXI_TRY(block(tokens + a, T, outputs));
      *next = outputs[T - 1];
      if (!sync_mtp) continue;
      const unsigned entries = previous ? T : T - 1;
      if (entries == 0) continue;
      if (T > 1) {
        if (auto e = hipMemcpyAsync(mtp_conditioning + (previous ? H : 0), hidden_a, (T - 1) * H * 2,
                                    hipMemcpyDeviceToDevice, stream);
            e != hipSuccess) {
          return hip_fail(e, "prefill conditioning copy failed");
        }
      }
      GFXI_TRY(mtp_sync(tokens + a + (previous ? 0 : 1), entries, mtp_position));
      GFXI_TRY(sync("prefill MTP cache update failed"));
      mtp_position += entries;
    }
    return ok();
  }

  // cli/main.cpp:1023-1120 generate, without the tokenizer.
  int32_t generate(const uint32_t* prompt, std::size_t count, const gfxinfer_generate_config& cfg,
                   uint32_t* output, std::size_t* output_count, gfxinfer_generate_stats* stats) {
    if (prompt == nullptr || output == nullptr || output_count == nullptr || count == 0 ||
        cfg.maximum_tokens == 0 || cfg.draft_count >= kMaxBlock ||
        (cfg.stop_count != 0 && cfg.stop_tokens == nullptr) ||
        count + cfg.maximum_tokens > config.maximum_context_tokens - current_position) {
      return fail(GFXI_INVALID_ARGUMENT,
                  "generate needs a prompt, 1+ output tokens, 0..31 drafts and prompt + output "
                  "within the session context");
    }
    using clock = std::chrono::steady_clock;
    const auto elapsed_ms = [](clock::time_point a, clock::time_point b) {
      return std::chrono::duration<double, std::milli>(b - a).count();
    };
    const auto stop = [&](uint32_t token) {
      for (uint32_t i = 0; i < cfg.stop_count; ++i) {
        if (cfg.stop_tokens[i] == token) return true;
      }
      return false;
    };
    gfxinfer_generate_stats st{};
    st.prompt_tokens = count;
    const auto start = clock::now();
    uint32_t next = 0;
    GFXI_TRY(prefill(prompt, count, cfg.draft_count != 0, &next));
    const auto first = clock::now();
    std::size_t produced = 0;
    output[produced++] = next;
    std::unique_ptr<gfxinfer_depth_policy> policy;
    if (cfg.adaptive_depth != 0 && cfg.draft_count != 0) {
      policy = std::make_unique<gfxinfer_depth_policy>(cfg.draft_count);
    }
    while (produced < cfg.maximum_tokens && !stop(next)) {
      if (cfg.draft_count == 0 || cfg.maximum_tokens - produced == 1) {
        GFXI_TRY(block(&next, 1, &next));  // greedy_step
        output[produced++] = next;
        continue;
      }
      const auto room = static_cast<uint32_t>(
          std::min<std::size_t>(cfg.draft_count, cfg.maximum_tokens - produced - 1));
      const uint32_t depth = policy ? policy->choose(room) : room;
      gfxinfer_speculative_result r{};
      const auto round_start = clock::now();
      GFXI_TRY(speculative(next, depth, -1, nullptr, &r));
      if (policy) policy->record(depth, r.token_count, elapsed_ms(round_start, clock::now()));
      st.proposed_drafts += r.proposed_drafts;
      st.accepted_drafts += r.accepted_drafts;
      ++st.speculative_rounds;
      bool terminal = false;
      for (uint32_t i = 0; i < r.token_count && produced < cfg.maximum_tokens; ++i) {
        output[produced++] = r.tokens[i];
        ++st.speculative_emitted;
        next = r.tokens[i];
        if (stop(next)) {
          terminal = true;
          break;
        }
      }
      if (terminal) break;
    }
    st.output_tokens = produced;
    st.prefill_ms = elapsed_ms(start, first);
    st.decode_ms = elapsed_ms(first, clock::now());
    *output_count = produced;
    if (stats != nullptr) *stats = st;
    return ok();
  }

  // The D proposals then the verifier with rollback logging (qwen_runtime.cpp:1448-1467,
  // 660-673).  verify_drafts is the buffer the verifier reads.
  int32_t chain_and_verify(uint32_t seed, bool indirect, unsigned draft_count,
                           std::size_t base_mtp, const PlantedDrafts* planted) {
    // Proposal i > 0 takes its token from proposal i - 1's draft-head keys and writes it
    // to draft_tokens[i - 1]; the last proposal reduces its own keys.
    for (unsigned i = 0; i < draft_count; ++i) {
      const uint32_t* device_token = i == 0 && indirect ? graph_seed : nullptr;
      const uint16_t* conditioning = i == 0 ? target_hidden_snapshot : mtp_hidden;
      GFXI_TRY(mtp_proposal(seed, device_token, conditioning, base_mtp + i, draft_tokens + i,
                            indirect ? graph_mtp_positions + i : nullptr,
                            i == 0 ? nullptr : draft_tokens + i - 1, i + 1 == draft_count));
    }
    const uint32_t* drafts = draft_tokens;
    if (planted != nullptr) {
      hipLaunchKernelGGL(planted_drafts_kernel, dim3(1), dim3(64), 0, stream, *planted,
                         verify_drafts, draft_count);
      GFXI_TRY(launch_status("planted draft upload failed"));
      drafts = verify_drafts;
    }
    record_rollback = true;
    const int32_t s = verifier(seed, indirect ? graph_seed : nullptr, drafts, draft_count,
                               indirect ? graph_base_position : nullptr);
    record_rollback = false;
    GFXI_TRY(s);
    hipLaunchKernelGGL(accept_kernel, dim3(1), dim3(64), 0, stream, drafts, selected, graph_forced,
                       draft_count, result);
    return launch_status("acceptance kernel launch failed");
  }

  int32_t write_round_scalars(uint32_t seed, int32_t forced, std::size_t base,
                              std::size_t base_mtp, unsigned draft_count) {
    RoundScalars v{seed, forced, base, base_mtp};
    hipLaunchKernelGGL(round_scalars_kernel, dim3(1), dim3(64), 0, stream, v, graph_seed,
                       graph_forced, graph_base_position, graph_mtp_positions,
                       std::max(draft_count, 1u));
    return launch_status("round scalar upload failed");
  }

  // qwen_runtime.cpp:642-713 prepare_speculative_graphs.
  int32_t prepare_graphs() {
    const unsigned batch = config.graph_verifier_batch;
    if (batch == 0) return ok();
    const unsigned draft_count = batch - 1;
    for (unsigned p = 0; p < 2; ++p) {
      if (p != 0) {
        std::swap(conv_states, conv_snapshot);
        std::swap(gdn_states, gdn_snapshot);
      }
      int32_t status = ok();
      if (auto e = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal); e != hipSuccess) {
        status = hip_fail(e, "speculative graph capture start failed");
      } else {
        status = chain_and_verify(0, true, draft_count, 0, nullptr);
        hipGraph_t graph = nullptr;
        const hipError_t end = hipStreamEndCapture(stream, &graph);
        if (status == GFXI_OK && end != hipSuccess) {
          status = hip_fail(end, "speculative graph capture end failed");
        }
        if (status == GFXI_OK) {
          hipGraphExec_t exec = nullptr;
          if (auto e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0); e != hipSuccess) {
            status = hip_fail(e, "speculative graph instantiation failed");
          } else {
            graphs[p] = {graph, exec};
            graph = nullptr;
          }
        }
        if (graph != nullptr) (void)hipGraphDestroy(graph);
      }
      if (p != 0) {
        std::swap(conv_states, conv_snapshot);
        std::swap(gdn_states, gdn_snapshot);
      }
      GFXI_TRY(status);
    }
    return ok();
  }

  int32_t sync(const char* what) {
    if (auto e = hipStreamSynchronize(stream); e != hipSuccess) return hip_fail(e, what);
    return ok();
  }

  // qwen_runtime.cpp:1421-1544 speculative_step (forced >= 0: acceptance override;
  // planted != nullptr: the verifier checks these drafts).
  int32_t speculative(uint32_t seed, std::size_t draft_count, int32_t forced,
                      const PlantedDrafts* planted, gfxinfer_speculative_result* out) {
    if (out == nullptr || last_hidden == nullptr || draft_count == 0 ||
        draft_count >= kMaxBlock || seed >= spec.tokenizer_vocabulary_size ||
        mtp_position + 1 != current_position ||
        draft_count + 1 > config.maximum_context_tokens - current_position ||
        (forced >= 0 && static_cast<std::size_t>(forced) > draft_count)) {
      return fail(GFXI_INVALID_ARGUMENT,
                  "speculative step requires 1..31 drafts and aligned target/MTP state");
    }
    const std::size_t base = current_position;
    const std::size_t base_mtp = mtp_position;
    const auto D = static_cast<unsigned>(draft_count);
    // snapshot_target_state (qwen_runtime.cpp:213-225).
    if (auto e = hipMemcpyAsync(target_hidden_snapshot, last_hidden, H * 2,
                                hipMemcpyDeviceToDevice, stream);
        e != hipSuccess) {
      return hip_fail(e, "target hidden-state snapshot failed");
    }
    int32_t status = write_round_scalars(seed, forced, base, base_mtp, D);
    const bool use_graph = planted == nullptr && D + 1 == config.graph_verifier_batch;
    if (status == GFXI_OK) {
      if (use_graph) {
        const Graph& g = graphs[parity ? 1 : 0];
        if (g.exec == nullptr) {
          status = fail(GFXI_INTERNAL, "prepared speculative graph is unavailable");
        } else if (auto e = hipGraphLaunch(g.exec, stream); e != hipSuccess) {
          status = hip_fail(e, "speculative graph launch failed");
        }
      } else {
        status = chain_and_verify(seed, false, D, base_mtp, planted);
      }
    }
    if (status == GFXI_OK) {
      if (auto e = hipMemcpyAsync(host_result, result, kResultWords * 4, hipMemcpyDeviceToHost,
                                  stream);
          e != hipSuccess) {
        status = hip_fail(e, "speculative result download failed");
      }
    }
    if (status == GFXI_OK) status = sync("speculative proposal/verifier chain failed");
    if (status != GFXI_OK) {
      // qwen_runtime.cpp:1469-1481: the pre-window state is untouched.
      record_rollback = false;
      mtp_chain_active = false;
      mtp_position = base_mtp;
      current_position = base;
      last_hidden = target_hidden_snapshot;
      (void)hipStreamSynchronize(stream);
      return status;
    }
    const uint32_t accepted = host_result[0];
    std::memset(out, 0, sizeof(*out));
    out->proposed_drafts = D;
    out->accepted_drafts = accepted;
    out->token_count = accepted + 1;
    std::memcpy(out->tokens, host_result + 2, (accepted + 1) * sizeof(uint32_t));
    if (accepted != D) {
      // qwen_runtime.cpp:1503-1520: replay the seed + accepted drafts onto the
      // untouched pre-window states.
      GFXI_TRY(gfxinfer_launch_gdn_restore_prefix_all(
          conv_states, gdn_states, conv_log, key_log, delta_log, decay_log, channels,
          static_cast<uint32_t>(gdn_layers), kMaxBlock, accepted + 1, spec.gdn_key_head_count,
          spec.gdn_value_head_count, spec.gdn_head_size, stream));
      current_position = base + accepted + 1;
      mtp_position = base_mtp + accepted + 1;
      mtp_chain_active = false;
      last_hidden = hidden_a + static_cast<std::size_t>(accepted) * H;
    } else {
      // qwen_runtime.cpp:1520-1535: keep the window's final states by a buffer swap,
      // then advance the MTP cache through the last draft.
      std::swap(conv_states, conv_snapshot);
      std::swap(gdn_states, gdn_snapshot);
      parity = !parity;
      current_position = base + D + 1;
      last_hidden = hidden_a + static_cast<std::size_t>(D) * H;
      mtp_position = base_mtp + D;
      GFXI_TRY(mtp_proposal(out->tokens[D - 1], nullptr, last_hidden - H, mtp_position, nullptr,
                            nullptr));
      mtp_chain_active = false;
      ++mtp_position;
    }
    return ok();
  }

  int32_t block(const uint32_t* tokens, std::size_t count, uint32_t* outputs) {
    if (tokens == nullptr || outputs == nullptr || count == 0 || count > kMaxBlock ||
        count > config.maximum_context_tokens - current_position) {
      return fail(GFXI_INVALID_ARGUMENT,
                  "decode block must contain a supported number of valid tokens within the "
                  "context limit");
    }
    for (std::size_t i = 0; i < count; ++i) {
      if (tokens[i] >= spec.vocabulary_size) {
        return fail(GFXI_INVALID_ARGUMENT, "decode token is outside the vocabulary");
      }
    }
    const auto batch = static_cast<unsigned>(count);
    GFXI_TRY(gather_rows(hidden_a, tokens, nullptr, nullptr, batch));
    GFXI_TRY(decoder_stack(batch, nullptr));
    // The windows wrote the advanced states into the snapshot buffers: keep them.
    std::swap(conv_states, conv_snapshot);
    std::swap(gdn_states, gdn_snapshot);
    parity = !parity;
    if (auto e = hipMemcpyAsync(host_result, selected, count * 4, hipMemcpyDeviceToHost, stream);
        e != hipSuccess) {
      return hip_fail(e, "decode block token download failed");
    }
    GFXI_TRY(sync("decode block failed"));
    std::memcpy(outputs, host_result, count * 4);
    last_hidden = hidden_a + (count - 1) * H;
    current_position += count;
    return ok();
  }
};

namespace {

Matrix bind_matrix(const gfxinfer_model& m, const std::string& name, bool& missing) {
  const Tensor* t = m.find(name);
  if (t == nullptr || t->format == kBf16) {
    missing = true;
    return {};
  }
  return {t->format, static_cast<const uint8_t*>(m.data(t)),
          static_cast<const uint16_t*>(m.auxiliary(t)), t->rows, t->columns};
}

const uint16_t* bind_vector(const gfxinfer_model& m, const std::string& name, bool& missing) {
  const Tensor* t = m.find(name);
  if (t == nullptr || t->format != kBf16) {
    missing = true;
    return nullptr;
  }
  return static_cast<const uint16_t*>(m.data(t));
}

void bind_attention(const gfxinfer_model& m, const std::string& p, Layer& L, bool& missing) {
  L.q = bind_matrix(m, p + "self_attn.q_proj.weight", missing);
  L.k = bind_matrix(m, p + "self_attn.k_proj.weight", missing);
  L.v = bind_matrix(m, p + "self_attn.v_proj.weight", missing);
  L.o = bind_matrix(m, p + "self_attn.o_proj.weight", missing);
  L.q_norm = bind_vector(m, p + "self_attn.q_norm.weight", missing);
  L.k_norm = bind_vector(m, p + "self_attn.k_norm.weight", missing);
}

void bind_mlp(const gfxinfer_model& m, const std::string& p, Layer& L, bool& missing) {
  L.input_norm = bind_vector(m, p + "input_layernorm.weight", missing);
  L.post_norm = bind_vector(m, p + "post_attention_layernorm.weight", missing);
  L.gate = bind_matrix(m, p + "mlp.gate_proj.weight", missing);
  L.up = bind_matrix(m, p + "mlp.up_proj.weight", missing);
  L.down = bind_matrix(m, p + "mlp.down_proj.weight", missing);
}

}  // namespace

extern "C" int32_t gfxinfer_session_create(gfxinfer_model* model,
                                           const gfxinfer_session_config* config,
                                           gfxinfer_session** out) {
  return guarded([&]() -> int32_t {
    if (model == nullptr || config == nullptr || out == nullptr ||
        config->maximum_context_tokens == 0 ||
        (config->graph_verifier_batch != 0 &&
         (config->graph_verifier_batch < 2 || config->graph_verifier_batch > kMaxBlock))) {
      return fail(GFXI_INVALID_ARGUMENT, "invalid decode session configuration");
    }
    *out = nullptr;
    if (auto e = hipSetDevice(model->device); e != hipSuccess) return hip_fail(e, "hipSetDevice failed");
    auto s = new gfxinfer_session();
    retain_model(model);
    s->model = model;
    s->spec = model->spec;
    s->config = *config;
    s->stream = model->stream;
    const auto& sp = s->spec;
    s->H = sp.hidden_size;
    s->I = sp.intermediate_size;
    s->attn_width = static_cast<std::size_t>(sp.attention_head_count) * sp.attention_head_size;
    s->q_rows = 2 * s->attn_width;
    s->kv_rows = static_cast<std::size_t>(sp.kv_head_count) * sp.attention_head_size;
    s->gdn_key = static_cast<std::size_t>(sp.gdn_key_head_count) * sp.gdn_head_size;
    s->gdn_value = static_cast<std::size_t>(sp.gdn_value_head_count) * sp.gdn_head_size;
    s->channels = 2 * s->gdn_key + s->gdn_value;
    s->V = sp.vocabulary_size;

    // Bindings (qwen_runtime.cpp:1011-1095).
    bool missing = false;
    s->embedding = bind_matrix(*model, "model.language_model.embed_tokens.weight", missing);
    s->lm_head = bind_matrix(*model, "lm_head.weight", missing);
    s->final_norm = bind_vector(*model, "model.language_model.norm.weight", missing);
    s->layers.resize(sp.layer_count);
    for (uint32_t i = 0; i < sp.layer_count; ++i) {
      Layer& L = s->layers[i];
      const std::string p = "model.language_model.layers." + std::to_string(i) + ".";
      L.attention = is_attention_layer(sp, i);
      L.state_index = L.attention ? s->attn_layers++ : s->gdn_layers++;
      bind_mlp(*model, p, L, missing);
      if (L.attention) {
        bind_attention(*model, p, L, missing);
      } else {
        L.qkv = bind_matrix(*model, p + "linear_attn.in_proj_qkv.weight", missing);
        L.z = bind_matrix(*model, p + "linear_attn.in_proj_z.weight", missing);
        L.a = bind_matrix(*model, p + "linear_attn.in_proj_a.weight", missing);
        L.b = bind_matrix(*model, p + "linear_attn.in_proj_b.weight", missing);
        L.out = bind_matrix(*model, p + "linear_attn.out_proj.weight", missing);
        L.conv = bind_vector(*model, p + "linear_attn.conv1d.weight", missing);
        L.a_log = bind_vector(*model, p + "linear_attn.A_log", missing);
        L.dt_bias = bind_vector(*model, p + "linear_attn.dt_bias", missing);
        L.gdn_norm = bind_vector(*model, p + "linear_attn.norm.weight", missing);
      }
    }
    s->mtp_fc = bind_matrix(*model, "mtp.fc.weight", missing);
    s->mtp_pre_embedding_norm = bind_vector(*model, "mtp.pre_fc_norm_embedding.weight", missing);
    s->mtp_pre_hidden_norm = bind_vector(*model, "mtp.pre_fc_norm_hidden.weight", missing);
    s->mtp_final_norm = bind_vector(*model, "mtp.norm.weight", missing);
    s->mtp.attention = true;
    bind_mlp(*model, "mtp.layers.0.", s->mtp, missing);
    bind_attention(*model, "mtp.layers.0.", s->mtp, missing);
    if (missing) {
      delete s;
      return fail(GFXI_CORRUPT_ARTIFACT, "model lacks a tensor the decode session needs");
    }
    // The MTP draft head (qwen_runtime.cpp:994-1008): the converter's ranked rows
    // "mtp.draft_head.weight" with their token ids when the model has them, else the LM
    // head's first rows (in the tile layout a row prefix is a byte prefix of codes and
    // scales) with the identity map.
    if (const Tensor* ids = model->find("mtp.draft_head_token_ids"); ids != nullptr) {
      bool absent = false;
      s->draft_head = bind_matrix(*model, "mtp.draft_head.weight", absent);
      if (absent || ids->format != kI32 || ids->columns != s->draft_head.rows ||
          s->draft_head.rows != sp.mtp_draft_vocabulary) {
        delete s;
        return fail(GFXI_CORRUPT_ARTIFACT, "MTP draft head and token ids do not match the spec");
      }
      s->draft_token_ids = static_cast<const uint32_t*>(model->data(ids));
    } else {
      s->draft_head = s->lm_head;
      s->draft_head.rows = sp.mtp_draft_vocabulary;
    }

    // Arena (qwen_runtime.cpp:1117-1184).
    const std::size_t B = kMaxBlock, ctx = config->maximum_context_tokens;
    const std::size_t max_k = std::max({s->I, 2 * s->H, s->attn_width, s->gdn_value});
    s->attention_workspace_bytes =
        gfxinfer_attention_workspace_bytes(kMaxBlock, sp.attention_head_count, sp.attention_head_size, ctx);
    s->argmax_keys_bytes = gfxinfer_gemm_argmax_workspace_bytes(s->V, kMaxBlock);
    const std::size_t conv_bytes = s->gdn_layers * s->conv_state_elements() * 2;
    const std::size_t gdn_bytes = s->gdn_layers * s->gdn_state_elements() * 4;
    const std::size_t kv_bytes = s->attn_layers * ctx * s->kv_rows * 2;
    const std::size_t mtp_kv_bytes = ctx * s->kv_rows * 2;
    s->buffers = {
        {"hidden", reinterpret_cast<void**>(&s->hidden_a), B * s->H * 2},
        {"hidden_b", reinterpret_cast<void**>(&s->hidden_b), B * s->H * 2},
        {"post_attention", reinterpret_cast<void**>(&s->post_attention), B * s->H * 2},
        {"mtp_hidden", reinterpret_cast<void**>(&s->mtp_hidden), s->H * 2},
        {"target_hidden_snapshot", reinterpret_cast<void**>(&s->target_hidden_snapshot), s->H * 2},
        {"mtp_concat", reinterpret_cast<void**>(&s->mtp_concat), B * 2 * s->H * 2},
        {"mtp_input", reinterpret_cast<void**>(&s->mtp_input), B * s->H * 2},
        {"mtp_conditioning", reinterpret_cast<void**>(&s->mtp_conditioning), B * s->H * 2},
        {"convolved", reinterpret_cast<void**>(&s->convolved), B * s->channels * 2},
        {"query", reinterpret_cast<void**>(&s->query), B * s->attn_width * 2},
        {"key", reinterpret_cast<void**>(&s->key), B * s->kv_rows * 2},
        {"attention_output", reinterpret_cast<void**>(&s->attention_output), B * s->attn_width * 2},
        {"act_codes", reinterpret_cast<void**>(&s->act_codes), B * max_k / 2},
        {"act_scales", reinterpret_cast<void**>(&s->act_scales), B * (max_k / 128) * 2},
        {"projected_main", reinterpret_cast<void**>(&s->projected_main),
         B * std::max(s->q_rows, s->channels) * 4},
        {"projected_z", reinterpret_cast<void**>(&s->projected_z), B * s->gdn_value * 4},
        {"projected_a", reinterpret_cast<void**>(&s->projected_a), B * sp.gdn_value_head_count * 4},
        {"projected_b", reinterpret_cast<void**>(&s->projected_b), B * sp.gdn_value_head_count * 4},
        {"projected_k", reinterpret_cast<void**>(&s->projected_k), B * s->kv_rows * 4},
        {"projected_v", reinterpret_cast<void**>(&s->projected_v), B * s->kv_rows * 4},
        {"gdn_mixed", reinterpret_cast<void**>(&s->gdn_mixed), B * s->gdn_value * 4},
        {"mixer_update", reinterpret_cast<void**>(&s->mixer_update), kMaxPlanes * B * s->H * 4},
        {"gate_output", reinterpret_cast<void**>(&s->gate_output), B * s->I * 4},
        {"up_output", reinterpret_cast<void**>(&s->up_output), B * s->I * 4},
        {"mlp_codes", reinterpret_cast<void**>(&s->mlp_codes), B * s->I / 2},
        {"mlp_scales", reinterpret_cast<void**>(&s->mlp_scales), B * (s->I / 128) * 2},
        {"mlp_update", reinterpret_cast<void**>(&s->mlp_update), kMaxPlanes * B * s->H * 4},
        {"logits", reinterpret_cast<void**>(&s->logits), B * s->V * 4},
        {"argmax_keys", &s->argmax_keys, s->argmax_keys_bytes},
        {"attention_workspace", reinterpret_cast<void**>(&s->attention_workspace),
         s->attention_workspace_bytes},
        {"rope_table", reinterpret_cast<void**>(&s->rope_table), gfxinfer_rope_table_bytes(ctx, sp.rotary_size)},
        {"selected", reinterpret_cast<void**>(&s->selected), B * 4},
        {"drafts", reinterpret_cast<void**>(&s->draft_tokens), B * 4},
        {"verify_drafts", reinterpret_cast<void**>(&s->verify_drafts), B * 4},
        {"result", reinterpret_cast<void**>(&s->result), kResultWords * 4},
        {"graph_seed", reinterpret_cast<void**>(&s->graph_seed), 4},
        {"graph_forced", reinterpret_cast<void**>(&s->graph_forced), 4},
        {"graph_base_position", reinterpret_cast<void**>(&s->graph_base_position), 8},
        {"graph_mtp_positions", reinterpret_cast<void**>(&s->graph_mtp_positions), B * 8},
        {"conv_states", reinterpret_cast<void**>(&s->conv_states), conv_bytes},
        {"conv_snapshot", reinterpret_cast<void**>(&s->conv_snapshot), conv_bytes},
        {"gdn_states", reinterpret_cast<void**>(&s->gdn_states), gdn_bytes},
        {"gdn_snapshot", reinterpret_cast<void**>(&s->gdn_snapshot), gdn_bytes},
        {"conv_log", reinterpret_cast<void**>(&s->conv_log), s->gdn_layers * B * s->channels * 2},
        {"key_log", reinterpret_cast<void**>(&s->key_log), s->gdn_layers * B * s->gdn_key * 4},
        {"delta_log", reinterpret_cast<void**>(&s->delta_log), s->gdn_layers * B * s->gdn_value * 4},
        {"decay_log", reinterpret_cast<void**>(&s->decay_log),
         s->gdn_layers * B * sp.gdn_value_head_count * 4},
        {"key_caches", reinterpret_cast<void**>(&s->key_caches), kv_bytes},
        {"value_caches", reinterpret_cast<void**>(&s->value_caches), kv_bytes},
        {"mtp_key_cache", reinterpret_cast<void**>(&s->mtp_key_cache), mtp_kv_bytes},
        {"mtp_value_cache", reinterpret_cast<void**>(&s->mtp_value_cache), mtp_kv_bytes},
    };
    std::size_t cursor = 0;
    std::vector<std::size_t> offsets;
    for (const auto& b : s->buffers) {
      cursor = align256(cursor);
      offsets.push_back(cursor);
      cursor += b.bytes;
    }
    s->arena_bytes = align256(cursor);
    std::size_t free_bytes = 0, total_bytes = 0;
    int32_t status = ok();
    if (auto e = hipMemGetInfo(&free_bytes, &total_bytes); e != hipSuccess) {
      status = hip_fail(e, "hipMemGetInfo before session allocation failed");
    } else if (s->arena_bytes > free_bytes) {
      status = fail(GFXI_OUT_OF_MEMORY, "decode session arena exceeds currently free GPU memory");
    } else if (auto e2 = hipMalloc(reinterpret_cast<void**>(&s->arena), s->arena_bytes);
               e2 != hipSuccess) {
      s->arena = nullptr;
      status = hip_fail(e2, "decode session arena allocation failed");
    } else if (auto e3 = hipHostMalloc(reinterpret_cast<void**>(&s->host_result), 256,
                                       hipHostMallocDefault);
               e3 != hipSuccess) {
      s->host_result = nullptr;
      status = hip_fail(e3, "pinned result buffer allocation failed");
    }
    if (status == GFXI_OK) {
      for (std::size_t i = 0; i < s->buffers.size(); ++i) {
        *s->buffers[i].slot = s->arena + offsets[i];
      }
      // qwen_runtime.cpp:1246-1256: zero recurrent state; also the scalars.
      for (auto* p : {static_cast<void*>(s->conv_states), static_cast<void*>(s->gdn_states)}) {
        const std::size_t bytes = p == s->conv_states ? conv_bytes : gdn_bytes;
        if (auto e = hipMemsetAsync(p, 0, bytes, s->stream); e != hipSuccess) {
          status = hip_fail(e, "recurrent state initialization failed");
        }
      }
      if (status == GFXI_OK) {
        status = gfxinfer_launch_rope_table(s->rope_table, ctx, sp.rotary_size, sp.rope_theta, s->stream);
      }
      if (status == GFXI_OK) status = s->write_round_scalars(0, -1, 0, 0, 1);
      if (status == GFXI_OK) status = s->sync("decode session initialization failed");
      if (status == GFXI_OK) status = s->prepare_graphs();
      if (status == GFXI_OK) status = s->sync("speculative graph preparation failed");
    }
    if (status != GFXI_OK) {
      delete s;
      return status;
    }
    s->summary = {s->arena_bytes, ctx, conv_bytes + gdn_bytes, kv_bytes * 2, mtp_kv_bytes * 2};
    *out = s;
    return ok();
  });
}

extern "C" void gfxinfer_session_destroy(gfxinfer_session* session) { delete session; }

namespace {
int32_t enter(const gfxinfer_session* s) {
  if (s == nullptr) return fail(GFXI_INVALID_ARGUMENT, "session handle is null");
  if (auto e = hipSetDevice(s->model->device); e != hipSuccess) return hip_fail(e, "hipSetDevice failed");
  return ok();
}
}  // namespace

extern "C" int32_t gfxinfer_session_block_step(gfxinfer_session* session,
                                               const uint32_t* input_tokens, size_t count,
                                               uint32_t* output_tokens) {
  GFXI_TRY(enter(session));
  return session->block(input_tokens, count, output_tokens);
}

extern "C" int32_t gfxinfer_session_prefill(gfxinfer_session* session, const uint32_t* tokens,
                                            size_t count, int32_t sync_mtp, uint32_t* next_token) {
  return guarded([&]() -> int32_t {
    GFXI_TRY(enter(session));
    return session->prefill(tokens, count, sync_mtp != 0, next_token);
  });
}

extern "C" int32_t gfxinfer_session_generate(gfxinfer_session* session, const uint32_t* prompt,
                                             size_t prompt_count, const gfxinfer_generate_config* config,
                                             uint32_t* output, size_t* output_count,
                                             gfxinfer_generate_stats* stats) {
  return guarded([&]() -> int32_t {
    GFXI_TRY(enter(session));
    if (config == nullptr) return fail(GFXI_INVALID_ARGUMENT, "generate needs a configuration");
    return session->generate(prompt, prompt_count, *config, output, output_count, stats);
  });
}

extern "C" int32_t gfxinfer_session_greedy_step(gfxinfer_session* session, uint32_t input_token,
                                                uint32_t* output_token) {
  GFXI_TRY(enter(session));
  if (session->current_position >= session->config.maximum_context_tokens) {
    return fail(GFXI_INVALID_ARGUMENT, "decode token or session position is invalid");
  }
  return session->block(&input_token, 1, output_token);
}

extern "C" int32_t gfxinfer_session_mtp_draft(gfxinfer_session* session, uint32_t next_token,
                                              uint32_t* output_token) {
  GFXI_TRY(enter(session));
  auto* s = session;
  if (output_token == nullptr || s->last_hidden == nullptr ||
      (!s->mtp_chain_active && s->mtp_position + 1 != s->current_position) ||
      next_token >= s->spec.tokenizer_vocabulary_size ||
      s->mtp_position >= s->config.maximum_context_tokens) {
    return fail(GFXI_INVALID_ARGUMENT, "MTP drafting is not aligned with the target state");
  }
  const uint16_t* conditioning = s->mtp_chain_active ? s->mtp_hidden : s->last_hidden;
  GFXI_TRY(s->mtp_proposal(next_token, nullptr, conditioning, s->mtp_position, s->selected,
                           nullptr));
  if (auto e = hipMemcpyAsync(s->host_result, s->selected, 4, hipMemcpyDeviceToHost, s->stream);
      e != hipSuccess) {
    return hip_fail(e, "MTP selected token download failed");
  }
  GFXI_TRY(s->sync("MTP draft step failed"));
  *output_token = s->host_result[0];
  ++s->mtp_position;
  return ok();
}

extern "C" int32_t gfxinfer_session_speculative_step(gfxinfer_session* session,
                                                     uint32_t seed_token, size_t draft_count,
                                                     gfxinfer_speculative_result* result) {
  GFXI_TRY(enter(session));
  return session->speculative(seed_token, draft_count, -1, nullptr, result);
}

extern "C" int32_t gfxinfer_session_speculative_step_forced(gfxinfer_session* session,
                                                            uint32_t seed_token,
                                                            size_t draft_count,
                                                            uint32_t forced_accepted,
                                                            gfxinfer_speculative_result* result) {
  GFXI_TRY(enter(session));
  if (forced_accepted > draft_count) {
    return fail(GFXI_INVALID_ARGUMENT, "forced acceptance exceeds the draft count");
  }
  return session->speculative(seed_token, draft_count, static_cast<int32_t>(forced_accepted),
                              nullptr, result);
}

extern "C" int32_t gfxinfer_session_speculative_step_planted(gfxinfer_session* session,
                                                             uint32_t seed_token,
                                                             size_t draft_count,
                                                             const uint32_t* planted_drafts,
                                                             gfxinfer_speculative_result* result) {
  GFXI_TRY(enter(session));
  if (planted_drafts == nullptr || draft_count == 0 || draft_count >= kMaxBlock) {
    return fail(GFXI_INVALID_ARGUMENT, "planted drafts need 1..31 host tokens");
  }
  PlantedDrafts planted{};
  for (std::size_t i = 0; i < draft_count; ++i) {
    if (planted_drafts[i] >= session->spec.vocabulary_size) {
      return fail(GFXI_INVALID_ARGUMENT, "planted draft is outside the vocabulary");
    }
    planted.token[i] = planted_drafts[i];
  }
  return session->speculative(seed_token, draft_count, -1, &planted, result);
}

extern "C" size_t gfxinfer_session_position(const gfxinfer_session* session) {
  return session == nullptr ? 0 : session->current_position;
}

extern "C" size_t gfxinfer_session_mtp_position(const gfxinfer_session* session) {
  return session == nullptr ? 0 : session->mtp_position;
}

extern "C" int32_t gfxinfer_session_get_summary(const gfxinfer_session* session,
                                            gfxinfer_session_summary* out) {
  if (session == nullptr || out == nullptr) {
    return fail(GFXI_INVALID_ARGUMENT, "summary needs a session and an output");
  }
  *out = session->summary;
  return ok();
}

namespace {
const gfxinfer_session::Buffer* find_buffer(const gfxinfer_session* s, const char* name) {
  if (s == nullptr || name == nullptr) return nullptr;
  for (const auto& b : s->buffers) {
    if (std::strcmp(b.name, name) == 0) return &b;
  }
  return nullptr;
}
}  // namespace

extern "C" size_t gfxinfer_session_layer_trace_bytes(const gfxinfer_session* session) {
  return session == nullptr ? 0 : session->trace_layout().total;
}

extern "C" int32_t gfxinfer_session_set_layer_trace(gfxinfer_session* session, void* device_trace,
                                                    size_t bytes) {
  GFXI_TRY(enter(session));
  if (device_trace != nullptr && bytes < session->trace_layout().total) {
    return fail(GFXI_INVALID_ARGUMENT, "layer trace buffer is smaller than gfxinfer_session_layer_trace_bytes");
  }
  session->layer_trace = static_cast<uint8_t*>(device_trace);
  return ok();
}

extern "C" size_t gfxinfer_session_buffer_bytes(const gfxinfer_session* session, const char* name) {
  const auto* b = find_buffer(session, name);
  return b == nullptr ? 0 : b->bytes;
}

extern "C" int32_t gfxinfer_session_copy_buffer(const gfxinfer_session* session, const char* name,
                                                size_t offset, void* host, size_t bytes) {
  GFXI_TRY(enter(session));
  const auto* b = find_buffer(session, name);
  if (b == nullptr || host == nullptr || offset > b->bytes || bytes > b->bytes - offset) {
    return fail(GFXI_INVALID_ARGUMENT, "unknown session buffer or range");
  }
  const auto* source = static_cast<const uint8_t*>(*b->slot) + offset;
  if (auto e = hipMemcpyAsync(host, source, bytes, hipMemcpyDeviceToHost, session->stream);
      e != hipSuccess) {
    return hip_fail(e, "session buffer download failed");
  }
  return const_cast<gfxinfer_session*>(session)->sync("session buffer download failed");
}
