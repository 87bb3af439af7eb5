// Synthetic checkpoint for the speculative-verify path: the tensor table of a
// Qwen3.8-shaped model in the converter's naming and formats, generated on the
// device from a counter-based hash and quantized as it is generated into the
// gfx950 tile layout (one wave per row group, no fp32 staging).
//
// Reference: Engine::create + the converter's tensor rules
// (src/engine.cpp:166-205 single weight arena; src/converter.cpp:78-119 format
// choice, :379-387 fp16 scales; include/gfxinfer/qwen38_spec.h names).
#include <algorithm>
#include <cstring>
#include <limits>
#include <string>

#include "common.hpp"
#include "runtime.hpp"

namespace gfx950 {
namespace {

// splitmix64 finalizer (Steele, Lea, Flood 2014).
__host__ __device__ inline uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Irwin-Hall(12) numerator: sum of twelve 16-bit uniforms (v + 1/2) / 65536 minus
// 6, times 65536, as an exact integer in [-393210, 393216].
__device__ inline int normal_numerator(uint64_t key, uint64_t index) {
  int sum = 0;
#pragma unroll
  for (uint64_t j = 0; j < 3; ++j) {
    const uint64_t h = splitmix64(key + 3u * index + j);
    sum += static_cast<int>(h & 0xffffu) + static_cast<int>((h >> 16) & 0xffffu) +
           static_cast<int>((h >> 32) & 0xffffu) + static_cast<int>(h >> 48);
  }
  return sum + 6 - 6 * 65536;
}

// value = mean + float(numerator) * (sigma / 65536), two IEEE fp32 operations.
__device__ inline float synthetic_value(uint64_t key, uint64_t index, float scale, float mean) {
  float v = static_cast<float>(normal_numerator(key, index)) * scale;
  asm volatile("" : "+v"(v));  // keep the product rounded before the add
  return mean + v;
}

__device__ inline double wave_sum_f64(double x) {
#pragma unroll
  for (int offset = 32; offset != 0; offset >>= 1) x += __shfl_xor(x, offset);
  return x;
}

__device__ inline float wave_max_f32(float x) {
#pragma unroll
  for (int offset = 32; offset != 0; offset >>= 1) x = fmaxf(x, __shfl_xor(x, offset));
  return x;
}

// Generates one (row, group-128) of a synthetic matrix and quantizes it exactly as
// quantize_group128 (quantization.cpp:163-220) does, writing gfx950 tiled codes and
// the fp16 scale (converter.cpp:379-387).  One wave per group, two values per lane.
// The double sums of the scale refit are exact (every nonzero term v*q has
// |v| >= s/2, so all terms fit one 53-bit window), so the wave-order reduction
// gives the reference's sequential sums bit for bit.
template <int Format>
__global__ __launch_bounds__(256) void synthetic_quantize_kernel(
    uint64_t key, float scale_law, float mean, std::size_t rows, std::size_t columns,
    uint8_t* __restrict__ codes, __half* __restrict__ scales, int32_t* __restrict__ non_finite) {
  __shared__ int8_t levels[4][kGroup];
  const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const std::size_t groups = columns / kGroup;
  const std::size_t id = static_cast<std::size_t>(blockIdx.x) * 4 + wave;
  if (id >= rows * groups) return;  // wave-uniform
  const std::size_t row = id / groups, group = id - row * groups;
  const uint64_t first = row * columns + group * kGroup + 2u * lane;
  const float v0 = synthetic_value(key, first, scale_law, mean);
  const float v1 = synthetic_value(key, first + 1, scale_law, mean);
  if (!isfinite(v0) || !isfinite(v1)) *non_finite = 1;
  const float maximum = wave_max_f32(fmaxf(fabsf(v0), fabsf(v1)));
  float scale = 1.0F;
  if (maximum != 0.0F) {  // choose_scale, quantization.cpp:67-92
    scale = maximum / (Format == GFXI_W3G128 ? 4.0F : 8.0F);
    for (int iteration = 0; iteration < 4; ++iteration) {
      const int q0 = encode_level<Format>(v0, scale), q1 = encode_level<Format>(v1, scale);
      const double numerator =
          wave_sum_f64(static_cast<double>(v0) * q0 + static_cast<double>(v1) * q1);
      const double denominator = wave_sum_f64(static_cast<double>(q0 * q0 + q1 * q1));
      if (denominator == 0.0) break;
      scale = static_cast<float>(numerator / denominator);
    }
    scale = fmaxf(scale, std::numeric_limits<float>::min());
  }
  levels[wave][2 * lane] = static_cast<int8_t>(encode_level<Format>(v0, scale));
  levels[wave][2 * lane + 1] = static_cast<int8_t>(encode_level<Format>(v1, scale));
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane == 0) scales[scale_offset(row, group, groups)] = to_half(scale);
  if (lane < 4) {
    uint8_t packed[16];
    pack_lane_chunk(Format, levels[wave] + lane * 32, packed);
    uint8_t* destination = codes + chunk_offset(Format, row, group * kGroup + lane * 32, groups);
    for (unsigned i = 0; i < lane_bytes(Format); ++i) destination[i] = packed[i];
  }
}

__device__ inline uint16_t f32_to_bf16_rne(float x) {
  const uint32_t u = __float_as_uint(x);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);  // finite inputs only
}

__global__ __launch_bounds__(256) void synthetic_bf16_kernel(uint16_t* __restrict__ out,
                                                             std::size_t count, uint64_t key,
                                                             float scale, float mean) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= count) return;
  out[i] = f32_to_bf16_rne(synthetic_value(key, i, scale, mean));
}

std::size_t align256(std::size_t x) { return (x + 255u) & ~static_cast<std::size_t>(255u); }

}  // namespace

int32_t validate_spec(const gfxinfer_model_spec& s) {
  const bool valid =
      s.hidden_size != 0 && s.hidden_size % 128 == 0 && s.intermediate_size != 0 &&
      s.intermediate_size % 128 == 0 && s.layer_count != 0 && s.layer_count % 2 == 0 &&
      s.full_attention_interval != 0 && s.attention_head_count != 0 && s.kv_head_count != 0 &&
      s.attention_head_count % s.kv_head_count == 0 &&
      (s.attention_head_size == 128 || s.attention_head_size == 256) &&
      s.rotary_size != 0 && s.rotary_size % 2 == 0 && s.rotary_size <= 64 &&
      s.gdn_key_head_count != 0 && s.gdn_value_head_count != 0 &&
      s.gdn_value_head_count % s.gdn_key_head_count == 0 && s.gdn_value_head_count % 16 == 0 &&
      s.gdn_head_size == 128 && s.vocabulary_size != 0 && s.vocabulary_size % 16 == 0 &&
      s.tokenizer_vocabulary_size != 0 && s.tokenizer_vocabulary_size <= s.vocabulary_size &&
      s.mtp_draft_vocabulary != 0 && s.mtp_draft_vocabulary % 16 == 0 &&
      s.mtp_draft_vocabulary <= s.vocabulary_size && s.w3_mlp_layers <= s.layer_count &&
      s.rms_norm_epsilon > 0.0F && s.rope_theta > 0.0F;
  if (!valid) {
    return fail(GFXI_INVALID_ARGUMENT,
                "model spec needs hidden/intermediate % 128 == 0, an even layer count, attention "
                "head size 128 or 256, kv heads dividing attention heads, GDN head size 128, GDN "
                "value heads a multiple of 16 and of the key heads, rotary <= 64, and vocabulary "
                "sizes % 16 == 0 in range");
  }
  return ok();
}

std::vector<Tensor> model_tensors(const gfxinfer_model_spec& s) {
  std::vector<Tensor> t;
  const uint64_t H = s.hidden_size, I = s.intermediate_size, hd = s.attention_head_size;
  const uint64_t q_rows = 2ull * s.attention_head_count * hd;  // query + gate per head
  const uint64_t kv_rows = static_cast<uint64_t>(s.kv_head_count) * hd;
  const uint64_t gk = static_cast<uint64_t>(s.gdn_key_head_count) * s.gdn_head_size;
  const uint64_t gv = static_cast<uint64_t>(s.gdn_value_head_count) * s.gdn_head_size;
  const uint64_t channels = 2 * gk + gv;
  constexpr float kMatrix = 0.02F;
  auto matrix = [&](std::string name, int32_t format, uint64_t rows, uint64_t columns) {
    Tensor x;
    x.name = std::move(name);
    x.format = format;
    x.rows = rows;
    x.columns = columns;
    x.sigma = kMatrix;
    t.push_back(std::move(x));
  };
  auto vector = [&](std::string name, uint64_t rows, uint64_t columns, float mean, float sigma) {
    Tensor x;
    x.name = std::move(name);
    x.format = kBf16;
    x.rows = rows;
    x.columns = columns;
    x.mean = mean;
    x.sigma = sigma;
    t.push_back(std::move(x));
  };
  auto norm = [&](const std::string& name, uint64_t n) { vector(name, 1, n, 0.0F, kMatrix); };
  auto attention = [&](const std::string& p) {
    matrix(p + "self_attn.q_proj.weight", GFXI_W4G128, q_rows, H);
    matrix(p + "self_attn.k_proj.weight", GFXI_W4G128, kv_rows, H);
    matrix(p + "self_attn.v_proj.weight", GFXI_W4G128, kv_rows, H);
    norm(p + "self_attn.q_norm.weight", hd);
    norm(p + "self_attn.k_norm.weight", hd);
    matrix(p + "self_attn.o_proj.weight", GFXI_W4G128, H, s.attention_head_count * hd);
  };
  auto mlp = [&](const std::string& p, int32_t format) {
    norm(p + "input_layernorm.weight", H);
    norm(p + "post_attention_layernorm.weight", H);
    matrix(p + "mlp.gate_proj.weight", format, I, H);
    matrix(p + "mlp.up_proj.weight", format, I, H);
    matrix(p + "mlp.down_proj.weight", format, H, I);
  };

  matrix("model.language_model.embed_tokens.weight", GFXI_W4G128, s.vocabulary_size, H);
  norm("model.language_model.norm.weight", H);
  matrix("lm_head.weight", GFXI_W4G128, s.vocabulary_size, H);
  for (uint32_t layer = 0; layer < s.layer_count; ++layer) {
    const std::string p = "model.language_model.layers." + std::to_string(layer) + ".";
    mlp(p, layer < s.w3_mlp_layers ? GFXI_W3G128 : GFXI_W4G128);
    if (is_attention_layer(s, layer)) {
      attention(p);
    } else {
      matrix(p + "linear_attn.in_proj_qkv.weight", GFXI_W4G128, channels, H);
      matrix(p + "linear_attn.in_proj_z.weight", GFXI_W4G128, gv, H);
      matrix(p + "linear_attn.in_proj_a.weight", GFXI_W4G128, s.gdn_value_head_count, H);
      matrix(p + "linear_attn.in_proj_b.weight", GFXI_W4G128, s.gdn_value_head_count, H);
      vector(p + "linear_attn.conv1d.weight", channels, 4, 0.0F, 0.5F);
      vector(p + "linear_attn.A_log", 1, s.gdn_value_head_count, 0.0F, 0.5F);
      vector(p + "linear_attn.dt_bias", 1, s.gdn_value_head_count, 0.0F, 0.5F);
      vector(p + "linear_attn.norm.weight", 1, s.gdn_head_size, 1.0F, kMatrix);
      matrix(p + "linear_attn.out_proj.weight", GFXI_W4G128, H, gv);
    }
  }
  matrix("mtp.fc.weight", GFXI_W4G128, H, 2 * H);
  norm("mtp.pre_fc_norm_embedding.weight", H);
  norm("mtp.pre_fc_norm_hidden.weight", H);
  norm("mtp.norm.weight", H);
  mlp("mtp.layers.0.", GFXI_W4G128);
  attention("mtp.layers.0.");
  return t;
}

}  // namespace gfx950

using namespace gfx950;

extern "C" void gfxinfer_model_spec_qwen38_27b(gfxinfer_model_spec* spec) {
  if (spec == nullptr) return;
  *spec = {};
  spec->hidden_size = 5120;
  spec->intermediate_size = 17408;
  spec->layer_count = 64;
  spec->full_attention_interval = 4;
  spec->attention_head_count = 40;
  spec->kv_head_count = 8;
  spec->attention_head_size = 128;
  spec->rotary_size = 64;
  spec->gdn_key_head_count = 16;
  spec->gdn_value_head_count = 32;
  spec->gdn_head_size = 128;
  spec->vocabulary_size = 151936;
  spec->tokenizer_vocabulary_size = 151936;
  spec->mtp_draft_vocabulary = 98304;
  spec->w3_mlp_layers = 56;
  spec->rms_norm_epsilon = 1.0e-6F;
  spec->rope_theta = 10000000.0F;
}

extern "C" void gfxinfer_model_spec_qwen38_reference(gfxinfer_model_spec* spec) {
  if (spec == nullptr) return;
  gfxinfer_model_spec_qwen38_27b(spec);
  spec->attention_head_count = 24;
  spec->kv_head_count = 4;
  spec->attention_head_size = 256;
  spec->gdn_value_head_count = 48;
  spec->vocabulary_size = 248320;
  spec->tokenizer_vocabulary_size = 248077;
}

namespace {

int32_t generate(gfxinfer_model& m, uint64_t seed) {
  int32_t* flag = nullptr;
  if (auto e = hipMalloc(reinterpret_cast<void**>(&flag), sizeof(int32_t)); e != hipSuccess) {
    return hip_fail(e, "synthetic weight flag allocation failed");
  }
  int32_t status = ok();
  if (auto e = hipMemsetAsync(flag, 0, sizeof(int32_t), m.stream); e != hipSuccess) {
    status = hip_fail(e, "synthetic weight flag clear failed");
  }
  for (const auto& t : m.tensors) {
    if (status != GFXI_OK) break;
    const uint64_t key = splitmix64(seed ^ name_hash(t.name));
    const float scale = t.sigma * 0x1p-16F;
    if (t.format == kBf16) {
      const std::size_t count = t.rows * t.columns;
      hipLaunchKernelGGL(synthetic_bf16_kernel, dim3(static_cast<unsigned>((count + 255) / 256)),
                         dim3(256), 0, m.stream, reinterpret_cast<uint16_t*>(m.data(&t)), count,
                         key, scale, t.mean);
      status = launch_status("synthetic bf16 generation failed");
      continue;
    }
    const std::size_t group_count = t.rows * (t.columns / kGroup);
    const dim3 grid(static_cast<unsigned>((group_count + 3) / 4));
    auto* codes = static_cast<uint8_t*>(m.data(&t));
    auto* scales = static_cast<__half*>(m.auxiliary(&t));
    if (t.format == GFXI_W3G128) {
      hipLaunchKernelGGL(synthetic_quantize_kernel<GFXI_W3G128>, grid, dim3(256), 0, m.stream, key,
                         scale, t.mean, t.rows, t.columns, codes, scales, flag);
    } else {
      hipLaunchKernelGGL(synthetic_quantize_kernel<GFXI_W4G128>, grid, dim3(256), 0, m.stream, key,
                         scale, t.mean, t.rows, t.columns, codes, scales, flag);
    }
    status = launch_status("synthetic weight generation failed");
  }
  int32_t non_finite = 0;
  if (status == GFXI_OK) {
    if (auto e = hipMemcpyAsync(&non_finite, flag, sizeof(int32_t), hipMemcpyDeviceToHost,
                                m.stream);
        e != hipSuccess) {
      status = hip_fail(e, "synthetic weight flag download failed");
    }
  }
  if (auto e = hipStreamSynchronize(m.stream); e != hipSuccess && status == GFXI_OK) {
    status = hip_fail(e, "synthetic weight generation failed");
  }
  (void)hipFree(flag);
  if (status == GFXI_OK && non_finite != 0) {
    status = fail(GFXI_INTERNAL, "synthetic weights produced a non-finite value");
  }
  return status;
}

}  // namespace

namespace gfx950 {

int32_t allocate_model(const gfxinfer_model_spec& spec, int32_t device, std::vector<Tensor> tensors,
                       gfxinfer_model** out) {
  *out = nullptr;
  if (int32_t s = validate_spec(spec); s != GFXI_OK) return s;
  if (int32_t s = gfxinfer_require_gfx950_device(device); s != GFXI_OK) return s;
  if (auto e = hipSetDevice(device); e != hipSuccess) return hip_fail(e, "hipSetDevice failed");
  auto m = new gfxinfer_model();
  m->spec = spec;
  m->device = device;
  m->tensors = std::move(tensors);
  std::size_t cursor = 0;
  for (std::size_t i = 0; i < m->tensors.size(); ++i) {
    auto& t = m->tensors[i];
    m->index.emplace(t.name, i);
    if (t.format == kBf16) {
      t.data_bytes = t.rows * t.columns * 2;
    } else if (t.format == kI32) {
      t.data_bytes = t.rows * t.columns * 4;
    } else {
      t.data_bytes = t.rows * t.columns * (t.format == GFXI_W3G128 ? 3 : 4) / 8;
      t.auxiliary_bytes = t.rows * (t.columns / kGroup) * 2;
    }
    cursor = align256(cursor);
    t.data_offset = cursor;
    cursor += t.data_bytes;
    if (t.auxiliary_bytes != 0) {
      cursor = align256(cursor);
      t.auxiliary_offset = cursor;
      cursor += t.auxiliary_bytes;
    }
  }
  m->arena_bytes = align256(cursor);
  int32_t status = ok();
  if (auto e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking); e != hipSuccess) {
    status = hip_fail(e, "compute stream creation failed");
  } else if (auto e2 = hipMalloc(reinterpret_cast<void**>(&m->arena), m->arena_bytes);
             e2 != hipSuccess) {
    m->arena = nullptr;
    status = hip_fail(e2, "weight arena allocation failed");
  }
  if (status != GFXI_OK) {
    gfxinfer_model_destroy(m);
    return status;
  }
  *out = m;
  return ok();
}

}  // namespace gfx950

extern "C" int32_t gfxinfer_model_create_synthetic(const gfxinfer_model_spec* spec, uint64_t seed,
                                                   int32_t device, gfxinfer_model** out) {
  return guarded([&]() -> int32_t {
    if (spec == nullptr || out == nullptr) {
      return fail(GFXI_INVALID_ARGUMENT, "model creation needs a spec and an output handle");
    }
    *out = nullptr;
    gfxinfer_model* m = nullptr;
    if (const int32_t status = allocate_model(*spec, device, model_tensors(*spec), &m);
        status != GFXI_OK) {
      return status;
    }
    if (const int32_t status = generate(*m, seed); status != GFXI_OK) {
      gfxinfer_model_destroy(m);
      return status;
    }
    *out = m;
    return ok();
  });
}

namespace gfx950 {
namespace {
void free_model(gfxinfer_model* model) {
  (void)hipSetDevice(model->device);
  if (model->stream != nullptr) (void)hipStreamSynchronize(model->stream);
  if (model->arena != nullptr) (void)hipFree(model->arena);
  if (model->stream != nullptr) (void)hipStreamDestroy(model->stream);
  delete model;
}
}  // namespace

void retain_model(gfxinfer_model* model) {
  const std::lock_guard<std::mutex> hold(model->lifetime);
  ++model->sessions;
}

void release_model_reference(gfxinfer_model* model) {
  bool last = false;
  {
    const std::lock_guard<std::mutex> hold(model->lifetime);
    --model->sessions;
    last = model->released && model->sessions == 0;
  }
  if (last) free_model(model);
}
}  // namespace gfx950

extern "C" void gfxinfer_model_destroy(gfxinfer_model* model) {
  if (model == nullptr) return;
  bool unused = false;
  {
    const std::lock_guard<std::mutex> hold(model->lifetime);
    model->released = true;
    unused = model->sessions == 0;
  }
  if (unused) gfx950::free_model(model);
}

extern "C" size_t gfxinfer_model_spec_tensor_count(const gfxinfer_model_spec* spec) {
  if (spec == nullptr || validate_spec(*spec) != GFXI_OK) return 0;
  return model_tensors(*spec).size();
}

extern "C" int32_t gfxinfer_model_spec_tensor(const gfxinfer_model_spec* spec, size_t index,
                                              gfxinfer_spec_tensor* out) {
  return guarded([&]() -> int32_t {
    if (spec == nullptr || out == nullptr) {
      return fail(GFXI_INVALID_ARGUMENT, "tensor enumeration needs a spec and an output");
    }
    if (const int32_t status = validate_spec(*spec); status != GFXI_OK) return status;
    const std::vector<Tensor> tensors = model_tensors(*spec);
    if (index >= tensors.size()) return fail(GFXI_INVALID_ARGUMENT, "tensor index past the table");
    const Tensor& t = tensors[index];
    if (t.name.size() >= sizeof out->name) return fail(GFXI_INTERNAL, "tensor name too long");
    *out = {};
    std::memcpy(out->name, t.name.c_str(), t.name.size() + 1);
    out->format = t.format;
    out->rows = t.rows;
    out->columns = t.columns;
    out->mean = t.mean;
    out->sigma = t.sigma;
    return ok();
  });
}

extern "C" void* gfxinfer_model_stream(const gfxinfer_model* model) {
  return model == nullptr ? nullptr : model->stream;
}

extern "C" size_t gfxinfer_model_weight_bytes(const gfxinfer_model* model) {
  return model == nullptr ? 0 : model->arena_bytes;
}

extern "C" int32_t gfxinfer_model_find_tensor(const gfxinfer_model* model, const char* name,
                                              gfxinfer_tensor_view* out) {
  if (model == nullptr || name == nullptr || out == nullptr) {
    return fail(GFXI_INVALID_ARGUMENT, "tensor lookup needs a model, a name and an output");
  }
  const Tensor* t = model->find(name);
  if (t == nullptr) return fail(GFXI_INVALID_ARGUMENT, std::string("no tensor named ") + name);
  out->format = t->format;
  out->rows = t->rows;
  out->columns = t->columns;
  out->data = model->data(t);
  out->auxiliary = model->auxiliary(t);
  out->data_bytes = t->data_bytes;
  out->auxiliary_bytes = t->auxiliary_bytes;
  return ok();
}

extern "C" int32_t gfxinfer_model_copy_tensor(const gfxinfer_model* model, const char* name,
                                              int32_t auxiliary, void* host, size_t bytes) {
  gfxinfer_tensor_view view;
  if (int32_t s = gfxinfer_model_find_tensor(model, name, &view); s != GFXI_OK) return s;
  const void* source = auxiliary != 0 ? view.auxiliary : view.data;
  const std::size_t size = auxiliary != 0 ? view.auxiliary_bytes : view.data_bytes;
  if (host == nullptr || source == nullptr || bytes != size) {
    return fail(GFXI_INVALID_ARGUMENT, "tensor copy needs a host buffer of the tensor's size");
  }
  if (auto e = hipMemcpyAsync(host, source, bytes, hipMemcpyDeviceToHost, model->stream);
      e != hipSuccess) {
    return hip_fail(e, "tensor download failed");
  }
  if (auto e = hipStreamSynchronize(model->stream); e != hipSuccess) {
    return hip_fail(e, "tensor download failed");
  }
  return ok();
}
