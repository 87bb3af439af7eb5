// Internal definitions shared by the synthetic model ("engine") and the decode
// session: the tensor table and the model handle behind gfxinfer_model.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "gfxinfer_runtime.h"

namespace gfx950 {

constexpr int32_t kBf16 = 0;   // tensor format tag of bf16 vectors / small matrices
constexpr int32_t kI32 = -1;   // tensor format tag of int32 vectors (draft-head token ids)

// One named tensor of the weight arena (engine.h:47-60 DeviceTensorView).
struct Tensor {
  std::string name;
  int32_t format{kBf16};
  uint64_t rows{0};
  uint64_t columns{0};
  std::size_t data_offset{0};
  std::size_t data_bytes{0};
  std::size_t auxiliary_offset{0};
  std::size_t auxiliary_bytes{0};
  // Synthetic value law: mean + sigma * N(0, 1).
  float mean{0.0F};
  float sigma{0.0F};
};

// Layer i is full attention iff (i + 1) % interval == 0 (qwen38_spec.h:45-47).
inline bool is_attention_layer(const gfxinfer_model_spec& spec, uint32_t layer) {
  return (layer + 1u) % spec.full_attention_interval == 0;
}

// Tensor table of a spec, in converter naming (converter.cpp:78-119,
// qwen_runtime.cpp:1025-1080), with formats and value laws; offsets unset.
std::vector<Tensor> model_tensors(const gfxinfer_model_spec& spec);
// Checks the shape constraints the kernels rely on; returns GFXI_OK or the error.
int32_t validate_spec(const gfxinfer_model_spec& spec);
// Lays the tensors out in one 256-byte-aligned device arena (engine.cpp:166-205) and
// creates the compute stream; the arena is left unfilled.
int32_t allocate_model(const gfxinfer_model_spec& spec, int32_t device, std::vector<Tensor> tensors,
                       gfxinfer_model** out);

// Session references to a model.  A session borrows its model's compute stream and
// arena, so gfxinfer_model_destroy with sessions still open only marks the model
// released, and the last session to end frees it (a session ending after its model
// would otherwise synchronize a destroyed stream).
void retain_model(gfxinfer_model* model);
void release_model_reference(gfxinfer_model* model);

// FNV-1a of a tensor name: the per-tensor key of the synthetic generator.
inline uint64_t name_hash(const std::string& name) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : name) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

}  // namespace gfx950

struct gfxinfer_model {
  gfxinfer_model_spec spec{};
  int device{0};
  hipStream_t stream{nullptr};
  uint8_t* arena{nullptr};
  std::size_t arena_bytes{0};
  std::vector<gfx950::Tensor> tensors;
  std::unordered_map<std::string, std::size_t> index;
  // Lifetime: open sessions and whether gfxinfer_model_destroy has been called.
  std::mutex lifetime;
  uint32_t sessions{0};
  bool released{false};

  const gfx950::Tensor* find(const std::string& name) const {
    const auto it = index.find(name);
    return it == index.end() ? nullptr : &tensors[it->second];
  }
  void* data(const gfx950::Tensor* t) const { return arena + t->data_offset; }
  void* auxiliary(const gfx950::Tensor* t) const {
    return t->auxiliary_bytes == 0 ? nullptr : arena + t->auxiliary_offset;
  }
};

// Online MTP depth selection by emitted tokens per millisecond (the policy behind
// gfxinfer_depth_policy_*; gfxinfer_session_generate uses it with adaptive_depth).
struct gfxinfer_depth_policy {
  struct Candidate {
    uint32_t depth;
    uint32_t rounds;
    double tokens;  // exponential average of tokens emitted per round
    double ms;      // exponential average of milliseconds per round
  };
  std::vector<Candidate> candidates;
  uint64_t round{0};
  uint32_t probe{0};  // next candidate to re-measure

  explicit gfxinfer_depth_policy(uint32_t maximum_depth);
  uint32_t choose(uint32_t limit);
  bool record(uint32_t depth, uint32_t emitted, double milliseconds);
};
