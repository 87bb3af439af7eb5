// Decoder-block operators of the speculative verify step for gfx950: RMSNorms
// (plus fused RMSNorm -> A4 quantization), SwiGLU -> A4, the GDN (gated delta
// network) causal conv, window recurrence with per-token logs and prefix
// rollback, per-head Q/K RMSNorm + partial RoPE, KV append, greedy argmax.
//
// Reference semantics: src/kernels/qwen_ops.hip.  Shapes the reference bakes in
// (48 value heads, 16 key heads, 24/4 attention heads x 256) are parameters here.
#include <algorithm>
#include <cmath>
#include <limits>
#include <string>
#include <utility>

#include "common.hpp"

namespace gfx950 {
namespace {

using u32x4 = unsigned __attribute__((ext_vector_type(4)));
using f32x4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float silu(float x) { return x / (1.0F + expf(-x)); }


// Sum of squares of an fp16 row staged in LDS, in the order of the reference's rms_norm
// (qwen_ops.hip:31-63: 256 threads of wave32): partial t (t < 256) is the fmaf chain over
// elements t, t + 256, ... in index order; each 32 partials are reduced by the shfl_down
// tree (lane l adds lane l + d, d = 16, 8, 4, 2, 1), here on the two 32-lane halves of
// each wave64; the eight group sums by the same tree (lanes 8..31 hold zeros, which add
// exactly).  Summing in the reference's order makes the normalized fp16 rows, and so the
// A4 codes of the next projection, independent of this build's launch shape: a code that
// flips between two summation orders changes a projection by a whole quantization step.
// Needs blockDim.x >= 256; all threads return the total.  The caller synchronizes the
// workgroup between writing `row` and this call.  The tree runs on VALU lane moves, not
// LDS round trips: step 16 takes the upper row of each 32-lane half with
// v_permlane16_swap, steps 8..1 are DPP row_shl moves (lane l reads lane l + d of its
// row); the lanes that feed lane 0 of each half add exactly the values the shfl_down
// tree adds, in the same order.
// MaxElements bounds `elements` (one batch of LDS reads per chain when it is at most
// 256 x 24, no loop).
template <uint32_t MaxElements = 32768>
__device__ float reference_square_sum(const __half* row, uint32_t elements, float* scratch) {
  const unsigned t = threadIdx.x;
  float s = 0.0F;
  __builtin_assume(elements <= MaxElements);
  if (t < 256u) {
    // Every chain of rows up to 6144 elements in one batch of LDS reads; the fmaf
    // chain keeps index order.
    constexpr unsigned kBatch = 24;
    for (uint32_t i0 = t; i0 < elements; i0 += 256u * kBatch) {
      float f[kBatch];
#pragma unroll
      for (unsigned k = 0; k < kBatch; ++k) {
        const uint32_t i = i0 + 256u * k;
        f[k] = __half2float(row[i < elements ? i : 0u]);  // unconditional read, used if in range
      }
#pragma unroll
      for (unsigned k = 0; k < kBatch; ++k) {
        if (i0 + 256u * k < elements) s = fmaf(f[k], f[k], s);
      }
    }
  }
  {
    const unsigned u = __float_as_uint(s);
    const auto swapped = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    s += __uint_as_float(swapped[1]);  // rows 0 and 2 now read rows 1 and 3
  }
  s += dpp_move<0x108>(s);  // row_shl:8
  s += dpp_move<0x104>(s);  // row_shl:4
  s += dpp_move<0x102>(s);  // row_shl:2
  s += dpp_move<0x101>(s);  // row_shl:1
  if (t < 256u && (t & 31u) == 0u) scratch[t >> 5] = s;
  __syncthreads();
  const float a0 = scratch[0] + scratch[4], a1 = scratch[1] + scratch[5];
  const float a2 = scratch[2] + scratch[6], a3 = scratch[3] + scratch[7];
  return (a0 + a2) + (a1 + a3);
}

// Inverse RMS from the reference-ordered sum: the correctly rounded 1 / sqrt (the build
// rounds fp32 division and square root correctly), where the reference calls rsqrtf, the
// hardware approximation within 1 ulp; a CPU restatement reproduces this value exactly.
__device__ __forceinline__ float inverse_rms(float total, uint32_t elements, float epsilon) {
  return 1.0F / sqrtf(total / static_cast<float>(elements) + epsilon);
}

// ---------------------------------------------------------------------------
// RMSNorm family (qwen_ops.hip:31-106, 176-217).  One workgroup per row.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float norm_scale(const uint16_t* weight, std::size_t i, bool unit) {
  float s = bf16_to_float(weight[i]);
  return unit ? s + 1.0F : s;
}

// Mode 0: plain RMSNorm.  Mode 1: residual add (fp16 round) then RMSNorm of the
// rounded sum.  Quantize: also (or only) emit A4 codes + scales of the output.
template <bool Residual, bool Quantize>
__global__ __launch_bounds__(256) void rms_norm_kernel(
    const __half* __restrict__ input, const float* __restrict__ update,
    __half* __restrict__ residual_out, const uint16_t* __restrict__ weight,
    __half* __restrict__ output, uint8_t* __restrict__ codes, __half* __restrict__ scales,
    uint32_t elements, float epsilon, bool unit_offset, uint32_t planes, uint64_t plane_stride) {
  extern __shared__ __align__(16) uint8_t smem[];
  __half* row = reinterpret_cast<__half*>(smem);           // [elements] staged values
  float* scratch = reinterpret_cast<float*>(smem + ((elements * 2 + 15) & ~15u));
  const std::size_t base = static_cast<std::size_t>(blockIdx.x) * elements;
  for (uint32_t i = threadIdx.x; i < elements; i += blockDim.x) {
    __half v = input[base + i];
    if constexpr (Residual) {
      float u = update[base + i];
      for (uint32_t p = 1; p < planes; ++p) u += update[p * plane_stride + base + i];
      v = to_half(__half2float(v) + u);
      residual_out[base + i] = v;
    }
    row[i] = v;
  }
  __syncthreads();
  const float inverse = inverse_rms(reference_square_sum(row, elements, scratch), elements, epsilon);
  for (uint32_t i = threadIdx.x; i < elements; i += blockDim.x) {
    const __half n = to_half(__half2float(row[i]) * inverse * norm_scale(weight, i, unit_offset));
    row[i] = n;
    if (output != nullptr) output[base + i] = n;
  }
  if constexpr (Quantize) {
    __syncthreads();
    const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const uint32_t groups = elements / 128u;
    for (uint32_t g = wave; g < groups; g += waves) {
      quantize_group_a4(row[g * 128u + 2u * lane], row[g * 128u + 2u * lane + 1u],
                        codes + static_cast<std::size_t>(blockIdx.x) * (elements / 2) + g * 64u,
                        scales + static_cast<std::size_t>(blockIdx.x) * groups + g, lane);
    }
  }
}

// Register-resident variant for rows of up to Slots * 16 * 128 elements (even
// count): up to 16 waves per workgroup, wave w owns 128-element slots w, w + waves, ...;
// each lane keeps its two values per slot in registers, so the row is read once and
// reduced once.  Every global load (row, all update planes) is issued before the first
// use.  The update is the sum of `planes` fp32 planes `plane_stride` apart, added in
// plane order (the split-K GEMM's output).  Same arithmetic per element as
// rms_norm_kernel.
//
// A row may be shared by `parts` workgroups: each one loads and reduces the whole row
// (the sum of squares needs every element), then normalizes, quantizes and stores only
// its own share of the row's 128-element slots.  The per-element work after the sum
// (normalization, the A4 quantizer's maximum and exact divisions) is most of a row's
// VALU time; split over `parts` compute units it no longer serializes on one.  Workgroup
// b runs row (b / 8 / parts) * 8 + b % 8, part (b / 8) % parts, so that with the
// round-robin dispatch over the eight XCDs the parts of a row share one L2.  Outputs
// must not overlap the inputs when parts > 1 (the host falls back to one part).
constexpr unsigned kNormSlots = 10;
constexpr unsigned kNormPlaneSlots = 3;  // split-update variant: rows up to 6144
constexpr unsigned kNormMaxPlanes = 8;
constexpr uint32_t kNormFastMax = kNormSlots * 16u * 128u;
// Rows longer than this do not fit the LDS row the reference-ordered sum reads (64 KB).
constexpr std::size_t kNormMaxElements = 32768;

template <bool Residual, bool Quantize, unsigned Slots, unsigned MaxPlanes, bool ExactPlanes = false>
__global__ __launch_bounds__(1024) void rms_norm_rows_kernel(
    const __half* __restrict__ input, const float* __restrict__ update,
    __half* __restrict__ residual_out, const uint16_t* __restrict__ weight,
    __half* __restrict__ output, uint8_t* __restrict__ codes, __half* __restrict__ scales,
    uint32_t elements, float epsilon, bool unit_offset, uint32_t planes, uint64_t plane_stride,
    uint32_t rows, uint32_t parts) {
  __shared__ float scratch[16];
  __shared__ __half staged[Slots * 16u * 128u];  // the row, for the reference-ordered sum
  const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const uint32_t k = blockIdx.x / 8u;
  const uint32_t row = (k / parts) * 8u + blockIdx.x % 8u;
  if (row >= rows) return;  // whole workgroup: padding of the XCD-major grid
  const uint32_t part = k % parts;
  const uint32_t slot_count = (elements + 127u) / 128u;
  const uint32_t own_begin = slot_count * part / parts, own_end = slot_count * (part + 1u) / parts;
  const std::size_t base = static_cast<std::size_t>(row) * elements;
  // 1) Loads.  Dead slots read element 0 (always valid) and are ignored.  The weights
  //    are loaded for the slots this workgroup normalizes: own_begin + wave + j * waves.
  uint32_t hin[Slots];
  uint32_t wpair[Slots];  // the two bf16 weights of each lane's pair
  float2 upd[Slots][MaxPlanes];
#pragma unroll
  for (unsigned j = 0; j < Slots; ++j) {
    const uint32_t i = (wave + j * waves) * 128u + 2u * lane;
    const uint32_t at = i < elements ? i : 0u;
    hin[j] = *reinterpret_cast<const uint32_t*>(input + base + at);
    const uint32_t wi = (own_begin + wave + j * waves) * 128u + 2u * lane;
    wpair[j] = *reinterpret_cast<const uint32_t*>(weight + (wi < elements ? wi : 0u));
    if constexpr (Residual) {
#pragma unroll
      for (unsigned p = 0; p < MaxPlanes; ++p) {
        if (ExactPlanes || p < planes) {
          upd[j][p] = *reinterpret_cast<const float2*>(update + p * plane_stride + base + at);
        }
      }
    }
  }
  // 2) Residual add (fp16 rounding of the sum), staged for the sum of squares.  The
  //    residual rows go to memory only at the end, so that no wave waits for those
  //    stores on the way through the reduction.
  __half2 sum_pair[Slots];
#pragma unroll
  for (unsigned j = 0; j < Slots; ++j) {
    const uint32_t i = (wave + j * waves) * 128u + 2u * lane;
    if (i < elements) {
      __half a = __ushort_as_half(static_cast<unsigned short>(hin[j] & 0xffffu));
      __half b = __ushort_as_half(static_cast<unsigned short>(hin[j] >> 16));
      if constexpr (Residual) {
        float2 u = upd[j][0];
#pragma unroll
        for (unsigned p = 1; p < MaxPlanes; ++p) {
          if (ExactPlanes || p < planes) {
            u.x += upd[j][p].x;
            u.y += upd[j][p].y;
          }
        }
        a = to_half(__half2float(a) + u.x);
        b = to_half(__half2float(b) + u.y);
      }
      sum_pair[j] = __halves2half2(a, b);
      *reinterpret_cast<__half2*>(staged + i) = sum_pair[j];
    }
  }
  __syncthreads();
  const float inverse =
      inverse_rms(reference_square_sum<Slots * 16u * 128u>(staged, elements, scratch), elements, epsilon);
  // 3) This workgroup's slots: normalized values from the staged row, A4 codes.
#pragma unroll
  for (unsigned j = 0; j < Slots; ++j) {
    const uint32_t g = own_begin + wave + j * waves;
    if (g >= own_end) break;  // wave-uniform
    const uint32_t i = g * 128u + 2u * lane;
    __half n0 = __float2half(0.0F), n1 = n0;
    if (i < elements) {
      const __half2 v = *reinterpret_cast<const __half2*>(staged + i);
      const float w0 = bf16_to_float(static_cast<uint16_t>(wpair[j] & 0xffffu));
      const float w1 = bf16_to_float(static_cast<uint16_t>(wpair[j] >> 16));
      n0 = to_half(__low2float(v) * inverse * (unit_offset ? w0 + 1.0F : w0));
      n1 = to_half(__high2float(v) * inverse * (unit_offset ? w1 + 1.0F : w1));
      if (output != nullptr) *reinterpret_cast<__half2*>(output + base + i) = __halves2half2(n0, n1);
    }
    if constexpr (Quantize) {
      const uint32_t groups = elements / 128u;
      quantize_group_a4(n0, n1, codes + static_cast<std::size_t>(row) * (elements / 2) + g * 64u,
                        scales + static_cast<std::size_t>(row) * groups + g, lane);
    }
  }
  if constexpr (Residual) {
#pragma unroll
    for (unsigned j = 0; j < Slots; ++j) {
      const uint32_t g = wave + j * waves;
      const uint32_t i = g * 128u + 2u * lane;
      if (g >= own_begin && g < own_end && i < elements) {
        *reinterpret_cast<__half2*>(residual_out + base + i) = sum_pair[j];
      }
    }
  }
}

// qwen_ops.hip:65-106: two RMSNorms written side by side.
__global__ __launch_bounds__(256) void dual_rms_norm_kernel(
    const __half* __restrict__ left, const uint16_t* __restrict__ left_weight,
    const __half* __restrict__ right, const uint16_t* __restrict__ right_weight,
    __half* __restrict__ output, uint32_t elements, float epsilon, bool unit_offset) {
  __shared__ float scratch[16];
  // Row blockIdx.y of [rows][elements] inputs -> row blockIdx.y of [rows][2 * elements].
  const std::size_t row = blockIdx.y;
  const bool second = blockIdx.x != 0;
  const __half* input = (second ? right : left) + row * elements;
  const uint16_t* weight = second ? right_weight : left_weight;
  output += row * 2u * elements + (second ? elements : 0);
  extern __shared__ __align__(16) uint8_t dual_smem[];
  __half* staged = reinterpret_cast<__half*>(dual_smem);  // [elements]
  for (uint32_t i = threadIdx.x; i < elements; i += blockDim.x) staged[i] = input[i];
  __syncthreads();
  const float inverse = inverse_rms(reference_square_sum(staged, elements, scratch), elements, epsilon);
  for (uint32_t i = threadIdx.x; i < elements; i += blockDim.x) {
    output[i] = to_half(__half2float(staged[i]) * inverse * norm_scale(weight, i, unit_offset));
  }
}

// Register-resident form of dual_rms_norm_kernel for even rows of up to Slots * 16 *
// 128 elements (the MTP conditioning norms): sixteen waves, lane pairs in 128-element
// slots as in rms_norm_rows_kernel, every load issued before the first use.  Same
// per-element arithmetic as dual_rms_norm_kernel; the sum of squares runs in the slot
// order of rms_norm_rows_kernel.  Two optional fusions for the MTP input: with
// EmbedFormat != 0 the left row is the embedding row of a token dequantized from its
// tiled matrix exactly as row_gather_kernel writes it (zeros for a token past the
// table), and with Quantize each 128-slot of the concatenated fp16 row is quantized to
// A4G128 by the wave that holds it, as quantize_activation_i4 does.
struct DualNormArgs {
  const __half* left;           // [rows][elements] fp16 (EmbedFormat == 0)
  const uint16_t* left_weight;  // bf16 [elements]
  const __half* right;          // [rows][elements] fp16
  const uint16_t* right_weight;
  __half* output;               // [rows][2 * elements] fp16, or null
  uint8_t* codes;               // A4 [rows][elements] bytes (Quantize)
  __half* scales;               // [rows][2 * elements / 128] (Quantize)
  const uint8_t* embed_codes;   // tiled [embed_rows][elements] (EmbedFormat != 0)
  const __half* embed_scales;
  uint32_t embed_rows, token;
  const uint32_t* indirect_token;  // if set, the token id is read here
  // If set, the token is the argmax of these per-tile keys of one token's fused head GEMM
  // (mapped through key_token_ids if set) and is also written to *key_token_out.
  const unsigned long long* keys;
  uint32_t key_count;
  const uint32_t* key_token_ids;
  uint32_t* key_token_out;
  uint32_t elements;
  float epsilon;
  bool unit_offset;
};

template <unsigned Slots, int EmbedFormat, bool Quantize>
__global__ __launch_bounds__(1024) void dual_rms_norm_rows_kernel(DualNormArgs a) {
  __shared__ float scratch[16];
  __shared__ __half staged[Slots * 16u * 128u];  // the half row, for the reference-ordered sum
  const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const uint32_t elements = a.elements;
  const std::size_t row = blockIdx.y;
  // gridDim.x = 2 * parts: each half row is shared by `parts` workgroups, which all load
  // and reduce the whole half and normalize / quantize their own share of its slots.
  const uint32_t parts = gridDim.x / 2u;
  const bool second = blockIdx.x >= parts;
  const uint32_t part = blockIdx.x % parts;
  const uint32_t slot_count = (elements + 127u) / 128u;
  const uint32_t own_begin = slot_count * part / parts, own_end = slot_count * (part + 1u) / parts;
  const uint16_t* weight = second ? a.right_weight : a.left_weight;
  const uint32_t half_offset = second ? elements : 0u;
  uint32_t hin[Slots], wpair[Slots];
#pragma unroll
  for (unsigned j = 0; j < Slots; ++j) {
    const uint32_t wi = (own_begin + wave + j * waves) * 128u + 2u * lane;
    wpair[j] = *reinterpret_cast<const uint32_t*>(weight + (wi < elements ? wi : 0u));
  }
  if (EmbedFormat != 0 && !second) {
    // the token's embedding row, dequantized per column pair; the token is the previous
    // proposal's greedy pick when its argmax keys are given (a workgroup-uniform branch)
    uint32_t token;
    if (a.keys != nullptr) {
      __shared__ unsigned long long key_partial[16];
      const uint32_t index = argmax_key_row(block_max_key(a.keys, a.key_count, key_partial));
      token = a.key_token_ids != nullptr ? a.key_token_ids[index] : index;
      if (threadIdx.x == 0 && part == 0) *a.key_token_out = token;
    } else {
      token = a.indirect_token != nullptr ? *a.indirect_token : a.token;
    }
    const std::size_t groups = elements / kGroup;
    if constexpr (EmbedFormat == GFXI_W4G128) {
      // W4: one byte holds the lane pair's two codes (even column in the low nibble).
      // Every slot's loads go out before the first use (row 0 / column 0 stand in for a
      // dead slot or a token past the table, whose values are zeros).
      const bool in_table = token < a.embed_rows;
      const uint32_t table_row = in_table ? token : 0u;
      uint32_t code[Slots];
      uint16_t scale_bits[Slots];
#pragma unroll
      for (unsigned j = 0; j < Slots; ++j) {
        const uint32_t i = (wave + j * waves) * 128u + 2u * lane;
        const uint32_t at = i < elements ? i : 0u;
        code[j] = a.embed_codes[chunk_offset(EmbedFormat, table_row, at, groups) + (at % 32u) / 2u];
        scale_bits[j] = __half_as_ushort(a.embed_scales[scale_offset(table_row, at / kGroup, groups)]);
      }
#pragma unroll
      for (unsigned j = 0; j < Slots; ++j) {
        const uint32_t i = (wave + j * waves) * 128u + 2u * lane;
        const int lo = static_cast<int>(code[j] & 0xfu), hi = static_cast<int>(code[j] >> 4);
        const int w0 = lo >= 8 ? lo - 16 : lo, w1 = hi >= 8 ? hi - 16 : hi;
        const float scale = __half2float(__ushort_as_half(scale_bits[j]));
        const uint32_t value =
            static_cast<uint32_t>(__half_as_ushort(to_half(static_cast<float>(w0) * scale))) |
            (static_cast<uint32_t>(__half_as_ushort(to_half(static_cast<float>(w1) * scale))) << 16);
        hin[j] = i < elements && in_table ? value : 0u;
      }
    } else {
#pragma unroll
    for (unsigned j = 0; j < Slots; ++j) {
      const uint32_t i = (wave + j * waves) * 128u + 2u * lane;
      hin[j] = 0u;
      if (i < elements && token < a.embed_rows) {
        const uint8_t* chunk = a.embed_codes + chunk_offset(EmbedFormat, token, i, groups);
        const int w0 = unpack_lane_code(EmbedFormat, chunk, i % 32u);
        const int w1 = unpack_lane_code(EmbedFormat, chunk, (i + 1u) % 32u);
        const float scale = __half2float(a.embed_scales[scale_offset(token, i / kGroup, groups)]);
        hin[j] = static_cast<uint32_t>(__half_as_ushort(to_half(static_cast<float>(w0) * scale))) |
                 (static_cast<uint32_t>(__half_as_ushort(to_half(static_cast<float>(w1) * scale))) << 16);
      }
    }
    }
  } else {
    const __half* input = (second ? a.right : a.left) + row * elements;
#pragma unroll
    for (unsigned j = 0; j < Slots; ++j) {
      const uint32_t i = (wave + j * waves) * 128u + 2u * lane;
      const uint32_t at = i < elements ? i : 0u;
      hin[j] = *reinterpret_cast<const uint32_t*>(input + at);
    }
  }
#pragma unroll
  for (unsigned j = 0; j < Slots; ++j) {
    const uint32_t i = (wave + j * waves) * 128u + 2u * lane;
    if (i < elements) *reinterpret_cast<uint32_t*>(staged + i) = hin[j];
  }
  __syncthreads();
  const float inverse =
      inverse_rms(reference_square_sum<Slots * 16u * 128u>(staged, elements, scratch), elements, a.epsilon);
#pragma unroll
  for (unsigned j = 0; j < Slots; ++j) {
    const uint32_t g = own_begin + wave + j * waves;
    const uint32_t i = g * 128u + 2u * lane;
    if (g >= own_end) break;  // wave-uniform
    __half n0 = __float2half(0.0F), n1 = n0;
    if (i < elements) {
      const __half2 v = *reinterpret_cast<const __half2*>(staged + i);
      const float w0 = bf16_to_float(static_cast<uint16_t>(wpair[j] & 0xffffu));
      const float w1 = bf16_to_float(static_cast<uint16_t>(wpair[j] >> 16));
      n0 = to_half(__low2float(v) * inverse * (a.unit_offset ? w0 + 1.0F : w0));
      n1 = to_half(__high2float(v) * inverse * (a.unit_offset ? w1 + 1.0F : w1));
      if (a.output != nullptr) {
        *reinterpret_cast<__half2*>(a.output + row * 2u * elements + half_offset + i) = __halves2half2(n0, n1);
      }
    }
    if constexpr (Quantize) {
      const std::size_t groups2 = 2u * elements / kGroup;
      quantize_group_a4(n0, n1, a.codes + row * elements + (half_offset + g * 128u) / 2u,
                        a.scales + row * groups2 + half_offset / kGroup + g, lane);
    }
  }
}

// qwen_ops.hip:108-163: fp16(silu(g) * u), then the A4 quantizer.  One wave per
// (token, group of 128).
template <bool Quantize>
__global__ __launch_bounds__(256) void silu_multiply_kernel(
    const float* __restrict__ gate, const float* __restrict__ up, __half* __restrict__ output,
    uint8_t* __restrict__ codes, __half* __restrict__ scales, uint32_t columns, uint32_t total_groups) {
  const uint32_t linear = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (linear >= total_groups) return;
  const unsigned lane = threadIdx.x & 63u;
  const uint32_t groups = columns / 128u;
  const uint32_t token = linear / groups, group = linear - token * groups;
  const std::size_t at = static_cast<std::size_t>(token) * columns + group * 128u + 2u * lane;
  const float2 g = *reinterpret_cast<const float2*>(gate + at);
  const float2 u = *reinterpret_cast<const float2*>(up + at);
  const __half p0 = to_half(silu(g.x) * u.x);
  const __half p1 = to_half(silu(g.y) * u.y);
  if (output != nullptr) {
    output[at] = p0;
    output[at + 1] = p1;
  }
  if constexpr (Quantize) {
    quantize_group_a4(p0, p1, codes + static_cast<std::size_t>(token) * (columns / 2) + group * 64u,
                      scales + linear, lane);
  }
}

__global__ void float_to_half_kernel(const float* __restrict__ in, __half* __restrict__ out,
                                     std::size_t n) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = to_half(in[i]);
}

// ---------------------------------------------------------------------------
// GDN causal depthwise conv (qwen_ops.hip:219-261).  Thread per channel.
// ---------------------------------------------------------------------------

template <unsigned MaxTokens>
__global__ __launch_bounds__(64) void gdn_conv_kernel(
    const float* __restrict__ projected, const uint16_t* __restrict__ weight,
    const __half* initial_state, __half* final_state,  // may alias (in-place update)
    __half* __restrict__ output, __half* __restrict__ appended_log, uint32_t channels,
    uint32_t tokens) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= channels) return;
  // Every token's input is loaded up front (independent loads, one latency); the
  // conv is a window over inputs, not a recurrence.
  __half x[MaxTokens];
#pragma unroll
  for (unsigned t = 0; t < MaxTokens; ++t) {
    if (t < tokens) x[t] = to_half(projected[static_cast<std::size_t>(t) * channels + c]);
  }
  __half state[4];
  float w[4];
#pragma unroll
  for (int tap = 0; tap < 4; ++tap) {
    state[tap] = initial_state[static_cast<std::size_t>(c) * 4 + tap];
    w[tap] = bf16_to_float(weight[static_cast<std::size_t>(c) * 4 + tap]);
  }
#pragma unroll
  for (unsigned t = 0; t < MaxTokens; ++t) {
    if (t < tokens) {
      state[0] = state[1];
      state[1] = state[2];
      state[2] = state[3];
      state[3] = x[t];
      if (appended_log != nullptr) appended_log[static_cast<std::size_t>(t) * channels + c] = state[3];
      float conv = 0.0F;
#pragma unroll
      for (int tap = 0; tap < 4; ++tap) conv = fmaf(__half2float(state[tap]), w[tap], conv);
      output[static_cast<std::size_t>(t) * channels + c] = to_half(silu(conv));
    }
  }
#pragma unroll
  for (int tap = 0; tap < 4; ++tap) final_state[static_cast<std::size_t>(c) * 4 + tap] = state[tap];
}

// ---------------------------------------------------------------------------
// GDN window recurrence (qwen_ops.hip:263-411), gfx950 layout.
//
// Workgroup = (value head h, block of 16 state columns); 256 threads = 4 waves x
// (4 columns x 16 k-slices).  Lane (ks, col) holds the 8 state rows ks*8..ks*8+7
// of its column in registers for the whole window, so each token costs two
// 16-lane xor reductions and no barrier.  A prologue puts the normalized q/k
// of every token, the per-token decay and beta, and the 16 value columns into
// LDS; the state tile is loaded and stored through LDS so global accesses are
// row-contiguous.  The unnormalized output o[t][h][v] goes to `mixed`; a second
// kernel applies the head RMSNorm, weight and SiLU(z) gate.
// ---------------------------------------------------------------------------

constexpr unsigned kGdnD = 128;      // head size (both key and value)
constexpr unsigned kGdnCols = 16;    // state columns per workgroup
constexpr unsigned kGdnMaxTokens = 32;

// The gated delta rule over a window for one lane (k-slice ks: state rows ks*8 ..
// ks*8+7 of column `col`, held in S): per token S = S * decay; memory = sum_i S_i k_i
// (an fmaf chain over the lane's rows, then the 16-lane xor tree); delta = (v - memory)
// * beta; S = fmaf(k, delta, S); o = the same chain and tree over S_i q_i.  Lane ks == 0
// writes o (and delta to the log).  Every LDS operand of token t + 1 (its key and query
// slices, value, decay and beta) is read while token t computes, and the loop body is
// unrolled by two so the hand-over costs no register moves.  The arithmetic per token
// does not depend on the window length, so a window equals the same tokens one by one.
template <unsigned VC>
__device__ __forceinline__ void gdn_scan(float (&S)[8], const float (*kn)[kGdnD], const float (*qn)[kGdnD],
                                         const float (*vv)[VC], const float* decay_s,
                                         const float* beta_s, unsigned T, unsigned ks, unsigned col,
                                         float* mixed, float* delta_log, std::size_t value_elements,
                                         std::size_t out_column) {
  struct Operands {
    float k[8], q[8], value, decay, beta;
  };
  auto fetch = [&](Operands& o, unsigned t) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      o.k[i] = kn[t][ks * 8 + i];
      o.q[i] = qn[t][ks * 8 + i];
    }
    o.value = vv[t][col];
    o.decay = decay_s[t];
    o.beta = beta_s[t];
  };
  auto step = [&](const Operands& o, unsigned t) __attribute__((always_inline)) {
    float memory = 0.0F;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      S[i] = S[i] * o.decay;
      memory = fmaf(S[i], o.k[i], memory);
    }
    memory = row16_sum(memory);
    const float delta = (o.value - memory) * o.beta;
    float out = 0.0F;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      S[i] = fmaf(o.k[i], delta, S[i]);
      out = fmaf(S[i], o.q[i], out);
    }
    out = row16_sum(out);
    if (ks == 0) {
      mixed[static_cast<std::size_t>(t) * value_elements + out_column] = out;
      if (delta_log != nullptr) delta_log[static_cast<std::size_t>(t) * value_elements + out_column] = delta;
    }
  };
  Operands a, b;
  fetch(a, 0);
  unsigned t = 0;
  for (; t + 1 < T; t += 2) {
    fetch(b, t + 1);
    step(a, t);
    fetch(a, t + 2 < T ? t + 2 : t + 1);
    step(b, t + 1);
  }
  if (t < T) step(a, t);
}

struct GdnArgs {
  const __half* qkv;        // conv output [T][2*Hk*D + Hv*D]
  const float* a;           // [T][Hv]
  const float* b;           // [T][Hv]
  const uint16_t* a_log;    // bf16 [Hv]
  const uint16_t* dt_bias;  // bf16 [Hv]
  const float* initial;     // [Hv][D][D]
  float* final_state;       // [Hv][D][D]
  float* mixed;             // [T][Hv*D] unnormalized output
  float* key_log;           // [T][Hk*D] or null
  float* delta_log;         // [T][Hv*D] or null
  float* decay_log;         // [T][Hv] or null
  uint32_t tokens;
  uint32_t key_heads;
  uint32_t value_heads;
};

__global__ __launch_bounds__(256) void gdn_recurrent_kernel(GdnArgs args) {
  constexpr unsigned D = kGdnD;
  __shared__ float qn[kGdnMaxTokens][D];
  __shared__ float kn[kGdnMaxTokens][D];
  __shared__ float vv[kGdnMaxTokens][kGdnCols];
  __shared__ float decay_s[kGdnMaxTokens];
  __shared__ float beta_s[kGdnMaxTokens];
  __shared__ float tile[D][kGdnCols + 1];

  const unsigned blocks_per_head = D / kGdnCols;
  const unsigned h = blockIdx.x / blocks_per_head;
  const unsigned cb = blockIdx.x - h * blocks_per_head;
  const unsigned ratio = args.value_heads / args.key_heads;
  const unsigned kh = h / ratio;
  const unsigned T = args.tokens;
  const std::size_t key_elements = static_cast<std::size_t>(args.key_heads) * D;
  const std::size_t value_elements = static_cast<std::size_t>(args.value_heads) * D;
  const std::size_t stride = 2 * key_elements + value_elements;
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const bool log_keys = args.key_log != nullptr && (h % ratio) == 0 && cb == 0;

  // Prologue (a): normalized q (with the 1/sqrt(D) query scale) and k per token.
  const float query_scale = 0.08838834764831845F;  // 1/sqrt(128), qwen_ops.hip:325
  for (unsigned t = wave; t < T; t += 4) {
    const __half* row = args.qkv + static_cast<std::size_t>(t) * stride;
    const float q0 = __half2float(row[kh * D + 2 * lane]);
    const float q1 = __half2float(row[kh * D + 2 * lane + 1]);
    const float k0 = __half2float(row[key_elements + kh * D + 2 * lane]);
    const float k1 = __half2float(row[key_elements + kh * D + 2 * lane + 1]);
    const float qs = wave_sum(q0 * q0 + q1 * q1);
    const float ks = wave_sum(k0 * k0 + k1 * k1);
    const float iq = rsqrtf(qs + 1.0e-6F) * query_scale;
    const float ik = rsqrtf(ks + 1.0e-6F);
    qn[t][2 * lane] = q0 * iq;
    qn[t][2 * lane + 1] = q1 * iq;
    kn[t][2 * lane] = k0 * ik;
    kn[t][2 * lane + 1] = k1 * ik;
    if (log_keys) {
      float* kl = args.key_log + static_cast<std::size_t>(t) * key_elements + kh * D;
      kl[2 * lane] = k0 * ik;
      kl[2 * lane + 1] = k1 * ik;
    }
  }
  // Prologue (b): decay and beta per token (qwen_ops.hip:342-349).
  if (tid < T) {
    const float a_value = args.a[static_cast<std::size_t>(tid) * args.value_heads + h] +
                          bf16_to_float(args.dt_bias[h]);
    const float softplus = a_value > 20.0F ? a_value : log1pf(expf(a_value));
    const float g = -expf(bf16_to_float(args.a_log[h])) * softplus;
    const float decay = expf(g);
    decay_s[tid] = decay;
    beta_s[tid] = 1.0F / (1.0F + expf(-args.b[static_cast<std::size_t>(tid) * args.value_heads + h]));
    if (args.decay_log != nullptr && cb == 0) {
      args.decay_log[static_cast<std::size_t>(tid) * args.value_heads + h] = decay;
    }
  }
  // Prologue (c): the 16 value columns of every token.
  for (unsigned i = tid; i < T * kGdnCols; i += blockDim.x) {
    const unsigned t = i / kGdnCols, c = i - t * kGdnCols;
    vv[t][c] = __half2float(args.qkv[static_cast<std::size_t>(t) * stride + 2 * key_elements +
                                     static_cast<std::size_t>(h) * D + cb * kGdnCols + c]);
  }
  // Prologue (d): state tile [D rows][16 columns], row-contiguous 64-byte reads.
  const float* initial = args.initial + static_cast<std::size_t>(h) * D * D + cb * kGdnCols;
  for (unsigned i = tid; i < D * (kGdnCols / 4); i += blockDim.x) {
    const unsigned r = i / (kGdnCols / 4), c4 = i - r * (kGdnCols / 4);
    const f32x4 v = *reinterpret_cast<const f32x4*>(initial + static_cast<std::size_t>(r) * D + c4 * 4);
    tile[r][c4 * 4 + 0] = v[0];
    tile[r][c4 * 4 + 1] = v[1];
    tile[r][c4 * 4 + 2] = v[2];
    tile[r][c4 * 4 + 3] = v[3];
  }
  __syncthreads();

  const unsigned ks = lane & 15u;              // k-slice: rows ks*8 .. ks*8+7
  const unsigned col = wave * 4u + (lane >> 4);  // column within the block
  float S[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) S[i] = tile[ks * 8 + i][col];
  const std::size_t out_column = static_cast<std::size_t>(h) * D + cb * kGdnCols + col;
  gdn_scan(S, kn, qn, vv, decay_s, beta_s, T, ks, col, args.mixed, args.delta_log, value_elements, out_column);

  // Epilogue: state back through the LDS tile, row-contiguous stores.
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) tile[ks * 8 + i][col] = S[i];
  __syncthreads();
  float* final_state = args.final_state + static_cast<std::size_t>(h) * D * D + cb * kGdnCols;
  for (unsigned i = tid; i < D * (kGdnCols / 4); i += blockDim.x) {
    const unsigned r = i / (kGdnCols / 4), c4 = i - r * (kGdnCols / 4);
    f32x4 v = {tile[r][c4 * 4 + 0], tile[r][c4 * 4 + 1], tile[r][c4 * 4 + 2], tile[r][c4 * 4 + 3]};
    *reinterpret_cast<f32x4*>(final_state + static_cast<std::size_t>(r) * D + c4 * 4) = v;
  }
}

// Causal conv + gated delta rule over a window in one launch (the pair
// gdn_conv_kernel -> gdn_recurrent_kernel with identical arithmetic).  Each
// workgroup (value head h, Cols = 16 or 32 state columns) needs the conv outputs of
// the 2 x 128 query/key channels of its key head and of its own Cols value channels:
// it stages fp16(projected) of those 2 x 128 + Cols channels for every token in LDS
// (independent loads), computes the 4-tap conv + SiLU per (token, channel) in
// parallel, then normalizes and runs the recurrence.  The query/key conv channels are
// shared by value_heads/key_heads x 128/Cols workgroups; the one with h % ratio == 0
// and column block 0 writes their final conv state and log, every workgroup writes
// those of its value channels.  Conv states must not be updated in place (other workgroups may
// still read the initial state).
struct GdnWindowArgs {
  const float* projected;       // [T][C] fp32 (C = 2*Hk*D + Hv*D)
  const uint16_t* conv_weight;  // bf16 [C][4]
  const __half* conv_initial;   // [C][4]
  __half* conv_final;           // [C][4]
  __half* conv_log;             // [T][C] or null
  GdnArgs gdn;                  // .qkv unused
};

// Sixteen waves share the loads, the conv and the norms; waves 0 .. Cols/4 - 1 (Cols
// columns x 16 row slices) run the recurrence, whose arithmetic per column is the same
// at any workgroup size.  Cols = 16 or 32 state columns per workgroup: the results do
// not depend on it (every column, conv channel and norm is computed the same way), only
// the grid does.  A 1024-thread workgroup holds a CU alone (two of them never share
// one, whatever their LDS), so a grid past one workgroup per CU runs in two rounds;
// launches whose 16-column grid would overfill the GPU take 32 columns per workgroup
// instead, half the grid, and each of those shares the query/key conv of its key head
// among half as many workgroups.
constexpr unsigned kWindowThreads = 1024;

template <unsigned Cols>
__global__ __launch_bounds__(kWindowThreads) void gdn_window_kernel(GdnWindowArgs w) {
  constexpr unsigned D = kGdnD;
  constexpr unsigned kWindowChannels = 2 * D + Cols;  // q and k of the key head, Cols v columns
  constexpr unsigned kWindowRecurrenceWaves = Cols / 4;
  static_assert(Cols % 16 == 0 && kWindowRecurrenceWaves <= kWindowThreads / 64, "column block");
  const GdnArgs& args = w.gdn;
  __shared__ float qn[kGdnMaxTokens][D];
  __shared__ float kn[kGdnMaxTokens][D];
  __shared__ float vv[kGdnMaxTokens][Cols];
  __shared__ __half xs[kGdnMaxTokens + 3][kWindowChannels];  // x[t-3..T-1] per channel
  __shared__ float cw[kWindowChannels][4];
  __shared__ float decay_s[kGdnMaxTokens];
  __shared__ float beta_s[kGdnMaxTokens];
  __shared__ float tile[D][Cols + 1];

  const unsigned blocks_per_head = D / Cols;
  const unsigned h = blockIdx.x / blocks_per_head;
  const unsigned cb = blockIdx.x - h * blocks_per_head;
  const unsigned ratio = args.value_heads / args.key_heads;
  const unsigned kh = h / ratio;
  const unsigned T = args.tokens;
  const std::size_t key_elements = static_cast<std::size_t>(args.key_heads) * D;
  const std::size_t value_elements = static_cast<std::size_t>(args.value_heads) * D;
  const std::size_t C = 2 * key_elements + value_elements;
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const bool owner = (h % ratio) == 0 && cb == 0;  // writes the shared q/k conv channels
  const bool log_keys = args.key_log != nullptr && owner;

  // Local channel j -> global channel: q of kh, k of kh, then 16 v columns of h.
  auto channel = [&](unsigned j) -> std::size_t {
    if (j < D) return static_cast<std::size_t>(kh) * D + j;
    if (j < 2 * D) return key_elements + static_cast<std::size_t>(kh) * D + (j - D);
    return 2 * key_elements + static_cast<std::size_t>(h) * D + cb * Cols + (j - 2 * D);
  };

  // Stage 1: every global load is issued before the first use (one memory latency):
  // the state tile, fp16(projected) of the 2 D + Cols channels per token as 4-channel
  // runs, a/b of the head, the conv weights and the initial conv state.
  constexpr unsigned NT = kWindowThreads;
  constexpr unsigned kQuads = kWindowChannels / 4;                          // 68 / 72
  constexpr unsigned kTileQuads = D * (Cols / 4);                           // 512 / 1024
  constexpr unsigned kTileLoads = (kTileQuads + NT - 1) / NT;               // 1
  constexpr unsigned kInputLoads = (kGdnMaxTokens * kQuads + NT - 1) / NT;  // 3
  constexpr unsigned kChannelLoads = (kWindowChannels + NT - 1) / NT;       // 1
  const unsigned quads = T * kQuads;
  const float* initial = args.initial + static_cast<std::size_t>(h) * D * D + cb * Cols;
  f32x4 tv[kTileLoads];
#pragma unroll
  for (unsigned u = 0; u < kTileLoads; ++u) {
    const unsigned i = tid + u * NT, r = i / (Cols / 4), c4 = i - r * (Cols / 4);
    if (i < kTileQuads) {
      tv[u] = *reinterpret_cast<const f32x4*>(initial + static_cast<std::size_t>(r) * D + c4 * 4);
    }
  }
  f32x4 xv[kInputLoads];
#pragma unroll
  for (unsigned u = 0; u < kInputLoads; ++u) {
    const unsigned i = tid + u * NT;
    if (i < quads) {
      const unsigned t = i / kQuads, q = i - t * kQuads;
      xv[u] = *reinterpret_cast<const f32x4*>(w.projected + static_cast<std::size_t>(t) * C +
                                              channel(q * 4));
    }
  }
  // Token `lane`'s a/b for the last wave, which computes decay and beta (token 0's for
  // lanes past the window: loaded, never used), and the head's dt_bias / A_log, all
  // unconditionally so that no load waits on a branch.
  const std::size_t ab = static_cast<std::size_t>(lane < T ? lane : 0u) * args.value_heads + h;
  const float a_in = args.a[ab], b_in = args.b[ab];
  const uint16_t dt_bias = args.dt_bias[h], a_log = args.a_log[h];
  uint16_t wv[kChannelLoads][4];
  __half iv[kChannelLoads][4];
#pragma unroll
  for (unsigned u = 0; u < kChannelLoads; ++u) {
    const unsigned j = tid + u * NT;
    if (j < kWindowChannels) {
      const std::size_t c = channel(j);
#pragma unroll
      for (int tap = 0; tap < 4; ++tap) {
        wv[u][tap] = w.conv_weight[c * 4 + tap];
        iv[u][tap] = w.conv_initial[c * 4 + tap];
      }
    }
  }

#pragma unroll
  for (unsigned u = 0; u < kTileLoads; ++u) {
    const unsigned i = tid + u * NT, r = i / (Cols / 4), c4 = i - r * (Cols / 4);
    if (i < kTileQuads) {
#pragma unroll
      for (int e = 0; e < 4; ++e) tile[r][c4 * 4 + e] = tv[u][e];
    }
  }
#pragma unroll
  for (unsigned u = 0; u < kInputLoads; ++u) {
    const unsigned i = tid + u * NT;
    if (i < quads) {
      const unsigned t = i / kQuads, q = i - t * kQuads;
      uint32_t bits[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const __half x = to_half(xv[u][e]);
        xs[t + 3][q * 4 + e] = x;
        bits[e] = __half_as_ushort(x);
      }
      if (w.conv_log != nullptr && (owner || q * 4 >= 2 * D)) {
        const uint2 packed = {bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
        *reinterpret_cast<uint2*>(w.conv_log + static_cast<std::size_t>(t) * C + channel(q * 4)) =
            packed;
      }
    }
  }
#pragma unroll
  for (unsigned u = 0; u < kChannelLoads; ++u) {
    const unsigned j = tid + u * NT;
    if (j < kWindowChannels) {
#pragma unroll
      for (int tap = 0; tap < 4; ++tap) cw[j][tap] = bf16_to_float(wv[u][tap]);
      xs[0][j] = iv[u][1];
      xs[1][j] = iv[u][2];
      xs[2][j] = iv[u][3];
    }
  }
  __syncthreads();

  // Final conv state = the last four inputs x[T-4..T-1] = xs[T-1..T+2] (xs[0..2]
  // hold the initial state's taps 1..3 when T < 4), written by the channel owners.
  for (unsigned j = tid; j < kWindowChannels; j += blockDim.x) {
    if (owner || j >= 2 * D) {
      const std::size_t c = channel(j);
      uint32_t bits[4];
#pragma unroll
      for (int tap = 0; tap < 4; ++tap) bits[tap] = __half_as_ushort(xs[T - 1 + tap][j]);
      *reinterpret_cast<uint2*>(w.conv_final + c * 4) = {bits[0] | (bits[1] << 16),
                                                         bits[2] | (bits[3] << 16)};
    }
  }

  // Stage 2: conv + SiLU per (token, channel) -> fp16 -> float (gdn_conv_kernel order).
  // Wave w convolves the query and key channels of tokens w, w + 16, ... (lane l: channels
  // 2l, 2l + 1 of each) and normalizes them in registers: the norms' sums then run over
  // the same lane layout as a separate pass over the staged values would.  The value
  // channels go to the threads from the last one down, so that waves without a token of
  // their own take them first; the last wave also computes decay and beta.
  constexpr unsigned NTHREADS = kWindowThreads;
  auto conv_silu = [&](unsigned t, unsigned j) {
    float conv = 0.0F;
#pragma unroll
    for (int tap = 0; tap < 4; ++tap) conv = fmaf(__half2float(xs[t + tap][j]), cw[j][tap], conv);
    return __half2float(to_half(silu(conv)));
  };
  const float query_scale = 0.08838834764831845F;  // 1/sqrt(128), qwen_ops.hip:325
  for (unsigned t = wave; t < T; t += NTHREADS / 64) {
    const float q0 = conv_silu(t, 2 * lane), q1 = conv_silu(t, 2 * lane + 1);
    const float k0 = conv_silu(t, D + 2 * lane), k1 = conv_silu(t, D + 2 * lane + 1);
    const float iq = rsqrtf(wave_sum(q0 * q0 + q1 * q1) + 1.0e-6F) * query_scale;
    const float ik = rsqrtf(wave_sum(k0 * k0 + k1 * k1) + 1.0e-6F);
    qn[t][2 * lane] = q0 * iq;
    qn[t][2 * lane + 1] = q1 * iq;
    kn[t][2 * lane] = k0 * ik;
    kn[t][2 * lane + 1] = k1 * ik;
    if (log_keys) {
      float* kl = args.key_log + static_cast<std::size_t>(t) * key_elements + kh * D;
      kl[2 * lane] = k0 * ik;
      kl[2 * lane + 1] = k1 * ik;
    }
  }
  for (unsigned i = NTHREADS - 1u - tid; i < T * Cols; i += NTHREADS) {
    const unsigned t = i / Cols, c = i - t * Cols;
    vv[t][c] = conv_silu(t, 2 * D + c);
  }
  // decay and beta per token (qwen_ops.hip:342-349), lane t of the last wave.
  if (wave == NTHREADS / 64 - 1u && lane < T) {
    const float a_value = a_in + bf16_to_float(dt_bias);
    const float softplus = a_value > 20.0F ? a_value : log1pf(expf(a_value));
    const float g = -expf(bf16_to_float(a_log)) * softplus;
    const float decay = expf(g);
    decay_s[lane] = decay;
    beta_s[lane] = 1.0F / (1.0F + expf(-b_in));
    if (args.decay_log != nullptr && cb == 0) {
      args.decay_log[static_cast<std::size_t>(lane) * args.value_heads + h] = decay;
    }
  }
  __syncthreads();

  // Stage 4: the recurrence (gdn_scan, as gdn_recurrent_kernel), on waves 0 .. Cols/4 - 1.
  const unsigned ks = lane & 15u;
  const unsigned col = wave * 4u + (lane >> 4);
  const bool recurrent = wave < kWindowRecurrenceWaves;
  float S[8];
  if (recurrent) {
#pragma unroll
    for (int i = 0; i < 8; ++i) S[i] = tile[ks * 8 + i][col];
    const std::size_t out_column = static_cast<std::size_t>(h) * D + cb * Cols + col;
    gdn_scan(S, kn, qn, vv, decay_s, beta_s, T, ks, col, args.mixed, args.delta_log, value_elements,
             out_column);
  }  // recurrent
  __syncthreads();
  if (recurrent) {
#pragma unroll
    for (int i = 0; i < 8; ++i) tile[ks * 8 + i][col] = S[i];
  }
  __syncthreads();
  float* final_state = args.final_state + static_cast<std::size_t>(h) * D * D + cb * Cols;
  for (unsigned i = tid; i < D * (Cols / 4); i += blockDim.x) {
    const unsigned r = i / (Cols / 4), c4 = i - r * (Cols / 4);
    f32x4 v = {tile[r][c4 * 4 + 0], tile[r][c4 * 4 + 1], tile[r][c4 * 4 + 2], tile[r][c4 * 4 + 3]};
    *reinterpret_cast<f32x4*>(final_state + static_cast<std::size_t>(r) * D + c4 * 4) = v;
  }
}

// Head RMSNorm * weight * SiLU(z) (qwen_ops.hip:386-409) of the mixed output,
// optionally followed by the A4 quantizer (a head is exactly one 128 group).
// One wave per (token, value head).
template <bool Quantize>
__global__ __launch_bounds__(256) void gdn_output_kernel(
    const float* __restrict__ mixed, const float* __restrict__ z, const uint16_t* __restrict__ weight,
    __half* __restrict__ output, uint8_t* __restrict__ codes, __half* __restrict__ scales,
    uint32_t value_heads, uint32_t total) {
  const uint32_t linear = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (linear >= total) return;
  const unsigned lane = threadIdx.x & 63u;
  const uint32_t t = linear / value_heads, h = linear - t * value_heads;
  const std::size_t row = static_cast<std::size_t>(t) * value_heads * kGdnD + h * kGdnD;
  // Every load before the first use: the mixed row, the gate row and the norm weights.
  const float2 o = *reinterpret_cast<const float2*>(mixed + row + 2 * lane);
  const float2 g = *reinterpret_cast<const float2*>(z + row + 2 * lane);
  const uint32_t w2 = *reinterpret_cast<const uint32_t*>(weight + 2 * lane);
  const float inverse = rsqrtf(wave_sum(o.x * o.x + o.y * o.y) / static_cast<float>(kGdnD) + 1.0e-6F);
  const __half r0 = to_half(o.x * inverse * bf16_to_float(static_cast<uint16_t>(w2 & 0xffffu)) * silu(g.x));
  const __half r1 = to_half(o.y * inverse * bf16_to_float(static_cast<uint16_t>(w2 >> 16)) * silu(g.y));
  if (output != nullptr) {
    output[row + 2 * lane] = r0;
    output[row + 2 * lane + 1] = r1;
  }
  if constexpr (Quantize) {
    quantize_group_a4(r0, r1, codes + row / 2, scales + linear, lane);
  }
}

// ---------------------------------------------------------------------------
// Prefix rollback over all GDN layers (qwen_ops.hip:467-539): replay the first
// `accepted` logged tokens onto the pre-window states with the forward pass's
// exact fp32 operations (S = S * decay, then S = fmaf(k, delta, S)).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void gdn_restore_conv_kernel(
    __half* __restrict__ states, const __half* __restrict__ logs, uint32_t channels,
    uint32_t layers, uint32_t max_logged, uint32_t accepted) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<std::size_t>(layers) * channels) return;
  const std::size_t layer = i / channels, c = i - layer * channels;
  __half* s = states + i * 4;
  const __half* log = logs + layer * max_logged * channels;
  // After `accepted` shifts the state is the last four of [state, log_0 .. log_{A-1}]:
  // word j is element A + j of that sequence (no chain of dependent loads).
  __half w[4];
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t n = accepted + j;
    w[j] = n < 4 ? s[n] : log[static_cast<std::size_t>(n - 4) * channels + c];
  }
  s[0] = w[0];
  s[1] = w[1];
  s[2] = w[2];
  s[3] = w[3];
}

// Thread per four consecutive state columns of one row.
// One workgroup per (layer, value head): the head's logged keys, deltas and decays of
// the accepted tokens are staged in LDS once, then each thread replays them onto 16
// four-column pieces of the 128 x 128 state (per element the same operations in token
// order as the recurrence), so the logs cross the memory hierarchy once per head
// instead of once per state piece.
constexpr unsigned kRestoreThreads = 256;

__global__ __launch_bounds__(kRestoreThreads) void gdn_restore_recurrent_kernel(
    float* __restrict__ states, const float* __restrict__ key_logs, const float* __restrict__ delta_logs,
    const float* __restrict__ decay_logs, uint32_t max_logged, uint32_t accepted, uint32_t key_heads,
    uint32_t value_heads) {
  constexpr unsigned D = kGdnD;
  constexpr unsigned kPieces = D * D / 4 / kRestoreThreads;  // 16 f32x4 per thread
  __shared__ float keys[kGdnMaxTokens][D];
  __shared__ float deltas[kGdnMaxTokens][D];
  __shared__ float decays[kGdnMaxTokens];
  const unsigned layer = blockIdx.x / value_heads, h = blockIdx.x - layer * value_heads;
  const unsigned kh = h / (value_heads / key_heads);
  const unsigned tid = threadIdx.x;
  const std::size_t key_elements = static_cast<std::size_t>(key_heads) * D;
  const std::size_t value_elements = static_cast<std::size_t>(value_heads) * D;
  f32x4* state = reinterpret_cast<f32x4*>(states + (static_cast<std::size_t>(layer) * value_heads + h) * D * D);
  f32x4 S[kPieces];
#pragma unroll
  for (unsigned j = 0; j < kPieces; ++j) S[j] = state[tid + j * kRestoreThreads];
  const float* key_log = key_logs + static_cast<std::size_t>(layer) * max_logged * key_elements + kh * D;
  const float* delta_log = delta_logs + static_cast<std::size_t>(layer) * max_logged * value_elements + h * D;
  for (unsigned e = tid; e < accepted * D; e += kRestoreThreads) {
    const unsigned t = e / D, c = e - t * D;
    keys[t][c] = key_log[static_cast<std::size_t>(t) * key_elements + c];
    deltas[t][c] = delta_log[static_cast<std::size_t>(t) * value_elements + c];
  }
  if (tid < accepted) {
    decays[tid] = decay_logs[(static_cast<std::size_t>(layer) * max_logged + tid) * value_heads + h];
  }
  __syncthreads();
#pragma unroll
  for (unsigned j = 0; j < kPieces; ++j) {
    const unsigned piece = tid + j * kRestoreThreads;
    const unsigned k = piece / (D / 4), v = (piece % (D / 4)) * 4;
    f32x4 x = S[j];
    for (uint32_t t = 0; t < accepted; ++t) {
      const float decay = decays[t], key = keys[t][k];
      const f32x4 delta = *reinterpret_cast<const f32x4*>(&deltas[t][v]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[q] = x[q] * decay;
        x[q] = fmaf(key, delta[q], x[q]);
      }
    }
    state[piece] = x;
  }
}

// ---------------------------------------------------------------------------
// Per-head RMSNorm(1 + w) + partial rotate-half RoPE for Q and K heads
// (qwen_ops.hip:599-676).  One wave per (token, head) of D = 128 or 256 dims; lane owns
// dims l + 64 j (j < D / 64), so the rotary dims (< 64) all sit in the lane's first value.
// ---------------------------------------------------------------------------

struct RopeArgs {
  const float* query_input;  // [T][Hq][query_stride]
  const uint16_t* query_weight;
  __half* query_output;      // [T][Hq][D]
  const float* key_input;    // [T][Hkv][key_stride]
  const uint16_t* key_weight;
  __half* key_output;        // [T][Hkv][D]
  uint32_t query_heads, query_stride, key_heads, key_stride, rotary, tokens;
  uint64_t base_position;
  const uint64_t* indirect_position;
  float theta;
  // Optional K/V cache append ([capacity][key_heads * D], rows base + t): the key
  // head waves also store their fp16 key row and the fp16 value row of their head.
  const float* value_input;  // [T][key_heads * D] or null (no append)
  __half* key_cache;
  __half* value_cache;
};

template <unsigned D>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(RopeArgs a) {
  constexpr unsigned J = D / 64;  // values per lane
  const uint32_t heads = a.query_heads + a.key_heads;
  const uint32_t linear = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (linear >= heads * a.tokens) return;
  const unsigned lane = threadIdx.x & 63u;
  const uint32_t t = linear / heads, local = linear - t * heads;
  const bool is_key = local >= a.query_heads;
  const uint32_t head = is_key ? local - a.query_heads : local;
  const uint32_t count = is_key ? a.key_heads : a.query_heads;
  const uint32_t stride = is_key ? a.key_stride : a.query_stride;
  const float* in = (is_key ? a.key_input : a.query_input) + (static_cast<std::size_t>(t) * count + head) * stride;
  const uint16_t* w = is_key ? a.key_weight : a.query_weight;
  __half* out = (is_key ? a.key_output : a.query_output) + (static_cast<std::size_t>(t) * count + head) * D;
  const uint64_t base = a.indirect_position != nullptr ? *a.indirect_position : a.base_position;
  const float position = static_cast<float>(base + t);
  // Every load before the first use: the head row, its norm weights and (for a key head
  // with the cache append) the value row.
  float x[J], value[J];
  uint16_t wb[J];
#pragma unroll
  for (unsigned j = 0; j < J; ++j) {
    x[j] = in[lane + 64 * j];
    wb[j] = w[lane + 64 * j];
    value[j] = 0.0F;
  }
  const bool append = is_key && a.value_input != nullptr;
  if (append) {
    const float* v = a.value_input + (static_cast<std::size_t>(t) * count + head) * D;
#pragma unroll
    for (unsigned j = 0; j < J; ++j) value[j] = v[lane + 64 * j];
  }
  float c = 1.0F, sn = 0.0F;
  if (lane < a.rotary) rope_cos_sin(position, a.rotary, a.theta, lane, c, sn);
  __half h[J];
  norm_rope_row<D>(x, wb, a.rotary, c, sn, lane, h);
#pragma unroll
  for (unsigned j = 0; j < J; ++j) out[lane + 64 * j] = h[j];
  if (append) {
    const std::size_t row = (static_cast<std::size_t>(base + t) * count + head) * D;
#pragma unroll
    for (unsigned j = 0; j < J; ++j) {
      a.key_cache[row + lane + 64 * j] = h[j];
      a.value_cache[row + lane + 64 * j] = to_half(value[j]);
    }
  }
}

// (cos, sin) per (position, rotary frequency): rope_cos_sin's values, for the fused RoPE
// attention's table.
__global__ __launch_bounds__(256) void rope_table_kernel(float2* table, uint32_t positions, uint32_t rotary,
                                                         float theta) {
  const uint32_t half = rotary / 2;
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<std::size_t>(positions) * half) return;
  const uint32_t p = static_cast<uint32_t>(i / half), f = static_cast<uint32_t>(i % half);
  float c, sn;
  rope_cos_sin(static_cast<float>(p), rotary, theta, f, c, sn);
  table[i] = float2{c, sn};
}

// K (fp16) and V (fp32 -> fp16) rows into the contiguous cache at the (device)
// position (qwen_ops.hip:678-696).
__global__ __launch_bounds__(256) void kv_append_kernel(
    const __half* __restrict__ key, const float* __restrict__ value, __half* __restrict__ key_cache,
    __half* __restrict__ value_cache, uint64_t position, const uint64_t* __restrict__ indirect,
    uint32_t elements, uint32_t tokens) {
  if (indirect != nullptr) position = *indirect;
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<std::size_t>(tokens) * elements) return;
  const std::size_t at = position * elements + i;
  key_cache[at] = key[i];
  value_cache[at] = to_half(value[i]);
}

// ---------------------------------------------------------------------------
// Greedy argmax per row, ties -> lowest index (qwen_ops.hip:768-807), optional
// id remap.  One 256-thread workgroup per row.
// ---------------------------------------------------------------------------

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(256) void argmax_kernel(
    const float* __restrict__ logits, const uint32_t* __restrict__ token_ids, uint32_t* __restrict__ out,
    uint32_t vocabulary, std::size_t stride) {
  __shared__ float best_value[4];
  __shared__ uint32_t best_index[4];
  const float* row = logits + static_cast<std::size_t>(blockIdx.x) * stride;
  float bv = -INFINITY;
  uint32_t bi = 0;
  for (uint32_t i = threadIdx.x; i < vocabulary; i += blockDim.x) {
    const float v = row[i];
    if (v > bv) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int offset = 32; offset != 0; offset >>= 1) {
    const float ov = __shfl_xor(bv, offset);
    const uint32_t oi = __shfl_xor(bi, offset);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  if (lane == 0) {
    best_value[wave] = bv;
    best_index[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (unsigned w = 1; w < blockDim.x / 64; ++w) {
      if (better(best_value[w], best_index[w], bv, bi)) {
        bv = best_value[w];
        bi = best_index[w];
      }
    }
    out[blockIdx.x] = token_ids != nullptr ? token_ids[bi] : bi;
  }
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------

bool valid_epsilon(float epsilon) { return std::isfinite(epsilon) && epsilon > 0.0F; }

// Workgroups per row of rms_norm_rows_kernel: enough that the rows' workgroups cover
// the GPU (at most 256, one per CU for a 1024-thread workgroup), at most kNormMaxParts
// and never more than the row's 128-element slots.
constexpr uint32_t kNormMaxParts = 10;
uint32_t norm_parts(uint32_t rows, uint32_t elements) {
  const uint32_t row_octets = (rows + 7u) / 8u;
  const uint32_t slots = (elements + 127u) / 128u;
  return std::max(1u, std::min({kNormMaxParts, slots, 32u / row_octets}));
}

template <bool Residual, bool Quantize>
void launch_norm(bool fast, unsigned per_wave_slots, uint32_t planes, dim3 block, std::size_t smem,
                 uint32_t batch, uint32_t parts, hipStream_t stream, const __half* in, const float* update,
                 __half* ro, const uint16_t* weight, __half* out, uint8_t* codes, __half* sc,
                 uint32_t e, float epsilon, bool unit, uint64_t plane_stride) {
  const dim3 grid(parts == 1 ? batch : 8u * parts * ((batch + 7u) / 8u));
  if (fast && per_wave_slots <= kNormPlaneSlots && (planes == 1 || Residual)) {
    if (planes == 1) {
      hipLaunchKernelGGL((rms_norm_rows_kernel<Residual, Quantize, kNormPlaneSlots, 1>), grid,
                         block, 0, stream, in, update, ro, weight, out, codes, sc, e, epsilon, unit,
                         planes, plane_stride, batch, parts);
    } else if (planes == 4) {  // the session's split-K plane count: loads without conditions
      hipLaunchKernelGGL((rms_norm_rows_kernel<Residual, Quantize, kNormPlaneSlots, Residual ? 4 : 1, true>),
                         grid, block, 0, stream, in, update, ro, weight, out, codes, sc, e,
                         epsilon, unit, planes, plane_stride, batch, parts);
    } else {
      hipLaunchKernelGGL((rms_norm_rows_kernel<Residual, Quantize, kNormPlaneSlots,
                                               Residual ? kNormMaxPlanes : 1>),
                         grid, block, 0, stream, in, update, ro, weight, out, codes, sc, e,
                         epsilon, unit, planes, plane_stride, batch, parts);
    }
  } else if (fast && planes == 1) {
    hipLaunchKernelGGL((rms_norm_rows_kernel<Residual, Quantize, kNormSlots, 1>), grid, block,
                       0, stream, in, update, ro, weight, out, codes, sc, e, epsilon, unit, planes,
                       plane_stride, batch, parts);
  } else {
    hipLaunchKernelGGL((rms_norm_kernel<Residual, Quantize>), dim3(batch), dim3(256), smem, stream,
                       in, update, ro, weight, out, codes, sc, e, epsilon, unit, planes,
                       plane_stride);
  }
}

// planes > 1 (residual only): the update is the sum of `planes` fp32 planes of
// [batch][elements], one after the other.
int32_t norm_entry(const char* name, bool residual, bool quantize, const uint16_t* input,
                   const float* update, uint16_t* residual_out, const uint16_t* weight,
                   uint16_t* output, uint8_t* codes, uint16_t* scales, std::size_t elements,
                   uint32_t batch, float epsilon, bool unit, hipStream_t stream,
                   uint32_t planes = 1) {
  if (input == nullptr || weight == nullptr || elements == 0 || batch == 0 ||
      !valid_epsilon(epsilon) || elements > kNormMaxElements ||
      (residual && (update == nullptr || residual_out == nullptr)) ||
      (!quantize && output == nullptr) ||
      (quantize && (codes == nullptr || scales == nullptr || elements % 128 != 0)) ||
      planes == 0 || planes > kNormMaxPlanes || (planes > 1 && !residual)) {
    return fail(GFXI_INVALID_ARGUMENT, std::string("invalid ") + name + " arguments");
  }
  const auto e = static_cast<uint32_t>(elements);
  const std::size_t smem = ((e * 2 + 15) & ~15u) + 64;
  auto* in = reinterpret_cast<const __half*>(input);
  auto* ro = reinterpret_cast<__half*>(residual_out);
  auto* out = reinterpret_cast<__half*>(output);
  auto* sc = reinterpret_cast<__half*>(scales);
  auto aligned = [](const void* p, std::uintptr_t a) {
    return p == nullptr || reinterpret_cast<std::uintptr_t>(p) % a == 0;
  };
  const bool fast = e % 2 == 0 && e <= kNormFastMax && aligned(input, 4) &&
                    aligned(residual_out, 4) && aligned(output, 4) && aligned(update, 8) &&
                    aligned(weight, 4);
  const unsigned slots = (e + 127u) / 128u;
  // slots <= 16 * kNormSlots on the fast path; at least four waves for the 256 partial
  // sums of the reference-ordered sum of squares
  const unsigned waves = std::max(4u, std::min(16u, slots));
  const unsigned per_wave = (slots + waves - 1) / waves;
  const dim3 block(64u * waves);
  const uint64_t stride = static_cast<uint64_t>(batch) * e;
  // Several workgroups per row only when no output overlaps an input: a part's stores
  // must not reach what another part of the same row still reads (in-place calls run
  // one workgroup per row, whose loads all precede its stores).
  auto range = [](const void* p, std::size_t bytes) {
    const auto b = reinterpret_cast<std::uintptr_t>(p);
    return std::pair<std::uintptr_t, std::uintptr_t>{b, p == nullptr ? b : b + bytes};
  };
  const std::size_t row_bytes = static_cast<std::size_t>(batch) * e * 2;
  const std::pair<std::uintptr_t, std::uintptr_t> reads[] = {
      range(input, row_bytes), range(residual ? update : nullptr, planes * stride * 4), range(weight, e * 2)};
  const std::pair<std::uintptr_t, std::uintptr_t> writes[] = {
      range(residual ? residual_out : nullptr, row_bytes), range(output, row_bytes),
      range(quantize ? codes : nullptr, row_bytes / 4), range(quantize ? scales : nullptr, row_bytes / 128)};
  bool disjoint = true;
  for (const auto& w : writes) {
    for (const auto& r : reads) disjoint = disjoint && (w.first == w.second || r.first == r.second ||
                                                        w.second <= r.first || r.second <= w.first);
  }
  const uint32_t parts = disjoint ? norm_parts(batch, e) : 1u;
  if (residual && quantize) {
    launch_norm<true, true>(fast, per_wave, planes, block, smem, batch, parts, stream, in, update, ro,
                            weight, out, codes, sc, e, epsilon, unit, stride);
  } else if (residual) {
    launch_norm<true, false>(fast, per_wave, planes, block, smem, batch, parts, stream, in, update, ro,
                             weight, out, codes, sc, e, epsilon, unit, stride);
  } else if (quantize) {
    launch_norm<false, true>(fast, per_wave, planes, block, smem, batch, parts, stream, in, update, ro,
                             weight, out, codes, sc, e, epsilon, unit, stride);
  } else {
    launch_norm<false, false>(fast, per_wave, planes, block, smem, batch, parts, stream, in, update, ro,
                              weight, out, codes, sc, e, epsilon, unit, stride);
  }
  return launch_status((std::string(name) + " launch failed").c_str());
}

}  // namespace
}  // namespace gfx950

using namespace gfx950;

// ---- norms ------------------------------------------------------------------

extern "C" int32_t gfxinfer_launch_rms_norm(const uint16_t* input, const uint16_t* bf16_weight,
                                            uint16_t* output, size_t elements, float epsilon,
                                            int32_t add_unit_offset, void* stream) {
  return norm_entry("RMSNorm", false, false, input, nullptr, nullptr, bf16_weight, output, nullptr,
                    nullptr, elements, 1, epsilon, add_unit_offset != 0, static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_rms_norm_batch(const uint16_t* input, const uint16_t* bf16_weight,
                                                  uint16_t* output, size_t elements, uint32_t batch,
                                                  float epsilon, int32_t add_unit_offset,
                                                  void* stream) {
  return norm_entry("batched RMSNorm", false, false, input, nullptr, nullptr, bf16_weight, output,
                    nullptr, nullptr, elements, batch, epsilon, add_unit_offset != 0,
                    static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_residual_add_rms_norm_batch(
    const uint16_t* residual, const float* update, uint16_t* residual_output,
    const uint16_t* bf16_weight, uint16_t* normalized_output, size_t elements, uint32_t batch,
    float epsilon, int32_t add_unit_offset, void* stream) {
  return norm_entry("fused residual/RMSNorm", true, false, residual, update, residual_output,
                    bf16_weight, normalized_output, nullptr, nullptr, elements, batch, epsilon,
                    add_unit_offset != 0, static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_rms_norm_quantize_i4(const uint16_t* input,
                                                        const uint16_t* bf16_weight,
                                                        uint16_t* normalized_output,
                                                        uint8_t* packed_output, uint16_t* scales,
                                                        size_t elements, uint32_t batch,
                                                        float epsilon, int32_t add_unit_offset,
                                                        void* stream) {
  return norm_entry("RMSNorm/A4", false, true, input, nullptr, nullptr, bf16_weight,
                    normalized_output, packed_output, scales, elements, batch, epsilon,
                    add_unit_offset != 0, static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_residual_add_rms_norm_quantize_i4(
    const uint16_t* residual, const float* update, uint16_t* residual_output,
    const uint16_t* bf16_weight, uint16_t* normalized_output, uint8_t* packed_output,
    uint16_t* scales, size_t elements, uint32_t batch, float epsilon, int32_t add_unit_offset,
    void* stream) {
  return norm_entry("fused residual/RMSNorm/A4", true, true, residual, update, residual_output,
                    bf16_weight, normalized_output, packed_output, scales, elements, batch,
                    epsilon, add_unit_offset != 0, static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_residual_add_rms_norm_quantize_i4_planes(
    const uint16_t* residual, const float* update_planes, uint32_t planes,
    uint16_t* residual_output, const uint16_t* bf16_weight, uint16_t* normalized_output,
    uint8_t* packed_output, uint16_t* scales, size_t elements, uint32_t batch, float epsilon,
    int32_t add_unit_offset, void* stream) {
  return norm_entry("fused residual(planes)/RMSNorm/A4", true, true, residual, update_planes,
                    residual_output, bf16_weight, normalized_output, packed_output, scales,
                    elements, batch, epsilon, add_unit_offset != 0, static_cast<hipStream_t>(stream),
                    planes);
}

namespace {
bool aligned4(const void* pointer) { return reinterpret_cast<std::uintptr_t>(pointer) % 4 == 0; }

// Rows of up to 3 * 16 * 128 even elements with 4-byte aligned rows take the
// register-resident kernel, others the strided one.
void launch_dual_norm(const uint16_t* left, const uint16_t* lw, const uint16_t* right, const uint16_t* rw,
                      uint16_t* out, std::size_t elements, uint32_t batch, float epsilon, bool unit,
                      hipStream_t stream) {
  const bool rows = elements % 2 == 0 && elements <= 3u * 16u * 128u && aligned4(left) && aligned4(right) &&
                    aligned4(lw) && aligned4(rw) && aligned4(out);
  if (rows) {
    DualNormArgs a{};
    a.left = reinterpret_cast<const __half*>(left);
    a.left_weight = lw;
    a.right = reinterpret_cast<const __half*>(right);
    a.right_weight = rw;
    a.output = reinterpret_cast<__half*>(out);
    a.elements = static_cast<uint32_t>(elements);
    a.epsilon = epsilon;
    a.unit_offset = unit;
    hipLaunchKernelGGL((dual_rms_norm_rows_kernel<3, 0, false>), dim3(2, batch), dim3(1024), 0, stream, a);
  } else {
    hipLaunchKernelGGL(dual_rms_norm_kernel, dim3(2, batch), dim3(256), (elements * 2 + 15) & ~std::size_t{15}, stream,
                       reinterpret_cast<const __half*>(left), lw, reinterpret_cast<const __half*>(right), rw,
                       reinterpret_cast<__half*>(out), static_cast<uint32_t>(elements), epsilon, unit);
  }
}
}  // namespace

extern "C" int32_t gfxinfer_launch_dual_rms_norm_concat(
    const uint16_t* left, const uint16_t* left_bf16_weight, const uint16_t* right,
    const uint16_t* right_bf16_weight, uint16_t* concatenated_output, size_t elements,
    float epsilon, int32_t add_unit_offset, void* stream) {
  if (left == nullptr || left_bf16_weight == nullptr || right == nullptr ||
      right_bf16_weight == nullptr || concatenated_output == nullptr || elements == 0 ||
      elements > kNormMaxElements || !valid_epsilon(epsilon)) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid dual RMSNorm/concat arguments");
  }
  launch_dual_norm(left, left_bf16_weight, right, right_bf16_weight, concatenated_output, elements, 1,
                   epsilon, add_unit_offset != 0, static_cast<hipStream_t>(stream));
  return launch_status("dual RMSNorm/concat launch failed");
}

extern "C" int32_t gfxinfer_launch_dual_rms_norm_concat_batch(
    const uint16_t* left, const uint16_t* left_bf16_weight, const uint16_t* right,
    const uint16_t* right_bf16_weight, uint16_t* concatenated_output, size_t elements, uint32_t batch,
    float epsilon, int32_t add_unit_offset, void* stream) {
  if (left == nullptr || left_bf16_weight == nullptr || right == nullptr ||
      right_bf16_weight == nullptr || concatenated_output == nullptr || elements == 0 ||
      elements > kNormMaxElements || batch == 0 || batch > 65535 || !valid_epsilon(epsilon)) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid batched dual RMSNorm/concat arguments");
  }
  launch_dual_norm(left, left_bf16_weight, right, right_bf16_weight, concatenated_output, elements, batch,
                   epsilon, add_unit_offset != 0, static_cast<hipStream_t>(stream));
  return launch_status("batched dual RMSNorm/concat launch failed");
}

namespace gfx950 {
namespace {
int32_t mtp_input_entry(int32_t embedding_format, const uint8_t* embedding_codes, const uint16_t* embedding_scales,
                        size_t embedding_rows, DualNormArgs a, const uint16_t* embedding_bf16_norm,
                        const uint16_t* conditioning, const uint16_t* conditioning_bf16_norm,
                        uint16_t* concatenated_output, uint8_t* packed_output, uint16_t* scales,
                        size_t elements, float epsilon, int32_t add_unit_offset, void* stream) {
  if (!valid_weight_format(embedding_format)) {
    return fail(GFXI_UNSUPPORTED, "MTP input: embedding format must be W2G128, W3G128 or W4G128");
  }
  if (embedding_codes == nullptr || embedding_scales == nullptr || embedding_rows == 0 ||
      embedding_rows % 16 != 0 || embedding_rows > (1u << 31) || embedding_bf16_norm == nullptr ||
      conditioning == nullptr || conditioning_bf16_norm == nullptr || packed_output == nullptr ||
      scales == nullptr || elements == 0 || elements % kGroup != 0 || elements > 3u * 16u * 128u ||
      !valid_epsilon(epsilon) || !aligned4(embedding_bf16_norm) || !aligned4(conditioning) ||
      !aligned4(conditioning_bf16_norm) || !aligned4(concatenated_output)) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid MTP input arguments (K divisible by 128 up to 6144, "
                                       "4-byte aligned rows)");
  }
  a.left_weight = embedding_bf16_norm;
  a.right = reinterpret_cast<const __half*>(conditioning);
  a.right_weight = conditioning_bf16_norm;
  a.output = reinterpret_cast<__half*>(concatenated_output);
  a.codes = packed_output;
  a.scales = reinterpret_cast<__half*>(scales);
  a.embed_codes = embedding_codes;
  a.embed_scales = reinterpret_cast<const __half*>(embedding_scales);
  a.embed_rows = static_cast<uint32_t>(embedding_rows);
  a.elements = static_cast<uint32_t>(elements);
  a.epsilon = epsilon;
  a.unit_offset = add_unit_offset != 0;
  const auto s = static_cast<hipStream_t>(stream);
  // Each half row is shared by up to kNormMaxParts workgroups (the A4 quantizer of a
  // whole half is VALU-bound on one compute unit) unless an output overlaps the
  // conditioning row or the argmax keys, which every part reads.
  auto disjoint = [](const void* w, std::size_t wn, const void* r, std::size_t rn) {
    const auto wb = reinterpret_cast<std::uintptr_t>(w), rb = reinterpret_cast<std::uintptr_t>(r);
    return w == nullptr || r == nullptr || wb + wn <= rb || rb + rn <= wb;
  };
  bool separate = true;
  for (const auto& [w, wn] : {std::pair<const void*, std::size_t>{concatenated_output, 4 * elements},
                              {packed_output, elements}, {scales, 4 * elements / kGroup}}) {
    separate = separate && disjoint(w, wn, conditioning, 2 * elements) &&
               disjoint(w, wn, a.keys, std::size_t{a.key_count} * 8u);
  }
  const dim3 grid(2u * (separate ? std::min<uint32_t>(kNormMaxParts, static_cast<uint32_t>(elements / kGroup)) : 1u));
  if (embedding_format == GFXI_W2G128) {
    hipLaunchKernelGGL((dual_rms_norm_rows_kernel<3, GFXI_W2G128, true>), grid, dim3(1024), 0, s, a);
  } else if (embedding_format == GFXI_W3G128) {
    hipLaunchKernelGGL((dual_rms_norm_rows_kernel<3, GFXI_W3G128, true>), grid, dim3(1024), 0, s, a);
  } else {
    hipLaunchKernelGGL((dual_rms_norm_rows_kernel<3, GFXI_W4G128, true>), grid, dim3(1024), 0, s, a);
  }
  return launch_status("MTP input (embedding + dual RMSNorm + A4) launch failed");
}
}  // namespace
}  // namespace gfx950

extern "C" int32_t gfxinfer_launch_mtp_input_quantize_i4(
    int32_t embedding_format, const uint8_t* embedding_codes, const uint16_t* embedding_scales,
    size_t embedding_rows, uint32_t token, const uint32_t* indirect_token,
    const uint16_t* embedding_bf16_norm, const uint16_t* conditioning,
    const uint16_t* conditioning_bf16_norm, uint16_t* concatenated_output, uint8_t* packed_output,
    uint16_t* scales, size_t elements, float epsilon, int32_t add_unit_offset, void* stream) {
  DualNormArgs a{};
  a.token = token;
  a.indirect_token = indirect_token;
  return mtp_input_entry(embedding_format, embedding_codes, embedding_scales, embedding_rows, a,
                         embedding_bf16_norm, conditioning, conditioning_bf16_norm, concatenated_output,
                         packed_output, scales, elements, epsilon, add_unit_offset, stream);
}

extern "C" int32_t gfxinfer_launch_mtp_input_quantize_i4_from_keys(
    int32_t embedding_format, const uint8_t* embedding_codes, const uint16_t* embedding_scales,
    size_t embedding_rows, const uint64_t* argmax_keys, size_t key_count, const uint32_t* token_ids,
    uint32_t* token_out, const uint16_t* embedding_bf16_norm, const uint16_t* conditioning,
    const uint16_t* conditioning_bf16_norm, uint16_t* concatenated_output, uint8_t* packed_output,
    uint16_t* scales, size_t elements, float epsilon, int32_t add_unit_offset, void* stream) {
  if (argmax_keys == nullptr || token_out == nullptr || key_count == 0 || key_count > (1u << 26)) {
    return fail(GFXI_INVALID_ARGUMENT, "MTP input from keys: keys and token output must be set, "
                                       "1..2^26 keys");
  }
  DualNormArgs a{};
  a.keys = reinterpret_cast<const unsigned long long*>(argmax_keys);
  a.key_count = static_cast<uint32_t>(key_count);
  a.key_token_ids = token_ids;
  a.key_token_out = token_out;
  return mtp_input_entry(embedding_format, embedding_codes, embedding_scales, embedding_rows, a,
                         embedding_bf16_norm, conditioning, conditioning_bf16_norm, concatenated_output,
                         packed_output, scales, elements, epsilon, add_unit_offset, stream);
}

// ---- SwiGLU -----------------------------------------------------------------

extern "C" int32_t gfxinfer_launch_silu_multiply_quantize_i4(const float* gate, const float* up,
                                                             uint8_t* packed_output,
                                                             uint16_t* scales,
                                                             size_t elements_per_row,
                                                             uint32_t batch, void* stream) {
  if (gate == nullptr || up == nullptr || packed_output == nullptr || scales == nullptr ||
      elements_per_row == 0 || elements_per_row % 128 != 0 || batch == 0 || batch > 32 ||
      elements_per_row > (1u << 30)) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid fused SiLU/A4 quantization arguments");
  }
  const auto columns = static_cast<uint32_t>(elements_per_row);
  const uint32_t total = columns / 128 * batch;
  hipLaunchKernelGGL(silu_multiply_kernel<true>, dim3((total + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream), gate, up, nullptr, packed_output,
                     reinterpret_cast<__half*>(scales), columns, total);
  return launch_status("fused SiLU/A4 quantization launch failed");
}

extern "C" int32_t gfxinfer_launch_silu_multiply(const float* gate, const float* up,
                                                 uint16_t* output, size_t elements,
                                                 void* stream) {
  if (gate == nullptr || up == nullptr || output == nullptr || elements == 0 ||
      elements % 128 != 0 || elements > (1u << 30)) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid SiLU multiply arguments (elements must be a "
                                       "nonzero multiple of 128)");
  }
  const auto columns = static_cast<uint32_t>(elements);
  const uint32_t total = columns / 128;
  hipLaunchKernelGGL(silu_multiply_kernel<false>, dim3((total + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream), gate, up, reinterpret_cast<__half*>(output),
                     nullptr, nullptr, columns, total);
  return launch_status("SiLU multiply launch failed");
}

extern "C" int32_t gfxinfer_launch_float_to_half(const float* input, uint16_t* output,
                                                 size_t elements, void* stream) {
  if (input == nullptr || output == nullptr || elements == 0) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid float-to-half arguments");
  }
  hipLaunchKernelGGL(float_to_half_kernel, dim3(static_cast<unsigned>((elements + 255) / 256)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), input,
                     reinterpret_cast<__half*>(output), elements);
  return launch_status("float-to-half launch failed");
}

// ---- GDN ----------------------------------------------------------------------

extern "C" int32_t gfxinfer_launch_gdn_conv_update_block(
    const float* projected_qkv, const uint16_t* bf16_conv_weight, const uint16_t* initial_conv_state,
    uint16_t* final_conv_state, uint16_t* convolved_qkv, uint16_t* appended_log, size_t channels,
    uint32_t batch, void* stream) {
  if (projected_qkv == nullptr || bf16_conv_weight == nullptr || initial_conv_state == nullptr ||
      final_conv_state == nullptr || convolved_qkv == nullptr || channels == 0 || batch == 0 ||
      channels > (1u << 30)) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid block GDN convolution arguments");
  }
  const auto c = static_cast<uint32_t>(channels);
  if (batch > kGdnMaxTokens) {
    return fail(GFXI_INVALID_ARGUMENT, "block GDN convolution supports at most 32 tokens");
  }
  hipLaunchKernelGGL(gdn_conv_kernel<kGdnMaxTokens>, dim3((c + 63) / 64), dim3(64), 0,
                     static_cast<hipStream_t>(stream), projected_qkv, bf16_conv_weight,
                     reinterpret_cast<const __half*>(initial_conv_state),
                     reinterpret_cast<__half*>(final_conv_state), reinterpret_cast<__half*>(convolved_qkv),
                     reinterpret_cast<__half*>(appended_log), c, batch);
  return launch_status("block GDN convolution update launch failed");
}

namespace {
int32_t gdn_check(const char* name, uint32_t batch, uint32_t key_heads, uint32_t value_heads,
                  uint32_t head_size) {
  if (batch == 0 || batch > kGdnMaxTokens || key_heads == 0 || value_heads == 0 ||
      value_heads % key_heads != 0 || head_size != kGdnD) {
    return fail(GFXI_INVALID_ARGUMENT,
                std::string(name) + " requires 1..32 tokens, value heads a multiple of key heads "
                                    "and head size 128");
  }
  return GFXI_OK;
}
}  // namespace

extern "C" int32_t gfxinfer_launch_gdn_recurrent_decode_block(
    const uint16_t* convolved_qkv, const float* projected_z, const float* projected_a,
    const float* projected_b, const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias,
    const uint16_t* bf16_norm_weight, const float* initial_recurrent_state,
    float* final_recurrent_state, uint16_t* output, float* key_log, float* delta_log,
    float* decay_log, uint32_t batch, uint32_t key_heads, uint32_t value_heads,
    uint32_t head_size, float* mixed_workspace, void* stream) {
  if (convolved_qkv == nullptr || projected_z == nullptr || projected_a == nullptr ||
      projected_b == nullptr || bf16_a_log == nullptr || bf16_dt_bias == nullptr ||
      bf16_norm_weight == nullptr || initial_recurrent_state == nullptr ||
      final_recurrent_state == nullptr || output == nullptr || mixed_workspace == nullptr) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid block GDN recurrent decode arguments");
  }
  if (const int32_t s = gdn_check("block GDN recurrent decode", batch, key_heads, value_heads, head_size);
      s != GFXI_OK) {
    return s;
  }
  auto st = static_cast<hipStream_t>(stream);
  GdnArgs args{reinterpret_cast<const __half*>(convolved_qkv), projected_a, projected_b, bf16_a_log,
               bf16_dt_bias, initial_recurrent_state, final_recurrent_state, mixed_workspace,
               key_log, delta_log, decay_log, batch, key_heads, value_heads};
  hipLaunchKernelGGL(gdn_recurrent_kernel, dim3(value_heads * (kGdnD / kGdnCols)), dim3(256), 0, st, args);
  if (const int32_t s = launch_status("block GDN recurrent decode launch failed"); s != GFXI_OK) return s;
  const uint32_t total = batch * value_heads;
  hipLaunchKernelGGL(gdn_output_kernel<false>, dim3((total + 3) / 4), dim3(256), 0, st,
                     mixed_workspace, projected_z, bf16_norm_weight, reinterpret_cast<__half*>(output),
                     nullptr, nullptr, value_heads, total);
  return launch_status("block GDN output norm launch failed");
}

extern "C" int32_t gfxinfer_launch_gdn_output_quantize_i4(
    const float* mixed, const float* projected_z, const uint16_t* bf16_norm_weight,
    uint16_t* output, uint8_t* packed_output, uint16_t* scales, uint32_t batch,
    uint32_t value_heads, uint32_t head_size, void* stream) {
  if (mixed == nullptr || projected_z == nullptr || bf16_norm_weight == nullptr ||
      packed_output == nullptr || scales == nullptr || batch == 0 || batch > kGdnMaxTokens ||
      value_heads == 0 || head_size != kGdnD) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid GDN output/A4 arguments");
  }
  const uint32_t total = batch * value_heads;
  hipLaunchKernelGGL(gdn_output_kernel<true>, dim3((total + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream), mixed, projected_z, bf16_norm_weight,
                     reinterpret_cast<__half*>(output), packed_output, reinterpret_cast<__half*>(scales),
                     value_heads, total);
  return launch_status("GDN output/A4 launch failed");
}

extern "C" int32_t gfxinfer_launch_gdn_recurrent_window(
    const uint16_t* convolved_qkv, const float* projected_a, const float* projected_b,
    const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias, const float* initial_recurrent_state,
    float* final_recurrent_state, float* mixed, float* key_log, float* delta_log, float* decay_log,
    uint32_t batch, uint32_t key_heads, uint32_t value_heads, uint32_t head_size, void* stream) {
  if (convolved_qkv == nullptr || projected_a == nullptr || projected_b == nullptr ||
      bf16_a_log == nullptr || bf16_dt_bias == nullptr || initial_recurrent_state == nullptr ||
      final_recurrent_state == nullptr || mixed == nullptr) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid GDN recurrent window arguments");
  }
  if (const int32_t s = gdn_check("GDN recurrent window", batch, key_heads, value_heads, head_size);
      s != GFXI_OK) {
    return s;
  }
  GdnArgs args{reinterpret_cast<const __half*>(convolved_qkv), projected_a, projected_b, bf16_a_log,
               bf16_dt_bias, initial_recurrent_state, final_recurrent_state, mixed, key_log,
               delta_log, decay_log, batch, key_heads, value_heads};
  hipLaunchKernelGGL(gdn_recurrent_kernel, dim3(value_heads * (kGdnD / kGdnCols)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), args);
  return launch_status("GDN recurrent window launch failed");
}

extern "C" int32_t gfxinfer_launch_gdn_conv_window(
    const float* projected_qkv, const uint16_t* bf16_conv_weight, const uint16_t* initial_conv_state,
    uint16_t* final_conv_state, uint16_t* appended_log, const float* projected_a,
    const float* projected_b, const uint16_t* bf16_a_log, const uint16_t* bf16_dt_bias,
    const float* initial_recurrent_state, float* final_recurrent_state, float* mixed, float* key_log,
    float* delta_log, float* decay_log, uint32_t batch, uint32_t key_heads, uint32_t value_heads,
    uint32_t head_size, void* stream) {
  if (projected_qkv == nullptr || bf16_conv_weight == nullptr || initial_conv_state == nullptr ||
      final_conv_state == nullptr || final_conv_state == initial_conv_state ||
      projected_a == nullptr || projected_b == nullptr || bf16_a_log == nullptr ||
      bf16_dt_bias == nullptr || initial_recurrent_state == nullptr ||
      final_recurrent_state == nullptr || mixed == nullptr) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid fused GDN conv/window arguments (the conv state "
                                       "cannot be updated in place)");
  }
  if (const int32_t s = gdn_check("fused GDN conv/window", batch, key_heads, value_heads, head_size);
      s != GFXI_OK) {
    return s;
  }
  // 4-channel vector accesses: 16-byte inputs and states, 8-byte conv states and log.
  const auto misaligned = [](const void* p, std::uintptr_t a) {
    return p != nullptr && reinterpret_cast<std::uintptr_t>(p) % a != 0;
  };
  if (misaligned(projected_qkv, 16) || misaligned(initial_recurrent_state, 16) ||
      misaligned(final_recurrent_state, 16) || misaligned(final_conv_state, 8) ||
      misaligned(appended_log, 8)) {
    return fail(GFXI_INVALID_ARGUMENT,
                "fused GDN conv/window needs 16-byte aligned fp32 inputs and states and 8-byte "
                "aligned conv state and log");
  }
  GdnWindowArgs w{projected_qkv, bf16_conv_weight, reinterpret_cast<const __half*>(initial_conv_state),
                  reinterpret_cast<__half*>(final_conv_state), reinterpret_cast<__half*>(appended_log),
                  GdnArgs{nullptr, projected_a, projected_b, bf16_a_log, bf16_dt_bias,
                          initial_recurrent_state, final_recurrent_state, mixed, key_log, delta_log,
                          decay_log, batch, key_heads, value_heads}};
  const auto st = static_cast<hipStream_t>(stream);
  if (value_heads * (kGdnD / 16) > kComputeUnits) {
    hipLaunchKernelGGL(gdn_window_kernel<32>, dim3(value_heads * (kGdnD / 32)), dim3(kWindowThreads), 0, st, w);
  } else {
    hipLaunchKernelGGL(gdn_window_kernel<16>, dim3(value_heads * (kGdnD / 16)), dim3(kWindowThreads), 0, st, w);
  }
  return launch_status("fused GDN conv/window launch failed");
}

extern "C" int32_t gfxinfer_launch_gdn_restore_prefix_all(
    uint16_t* conv_states, float* recurrent_states, const uint16_t* appended_logs,
    const float* key_logs, const float* delta_logs, const float* decay_logs, size_t channels,
    uint32_t layer_count, uint32_t maximum_logged_tokens, uint32_t accepted_tokens,
    uint32_t key_heads, uint32_t value_heads, uint32_t head_size, void* stream) {
  if (conv_states == nullptr || recurrent_states == nullptr || appended_logs == nullptr ||
      key_logs == nullptr || delta_logs == nullptr || decay_logs == nullptr || channels == 0 ||
      layer_count == 0 || maximum_logged_tokens == 0 || accepted_tokens == 0 ||
      accepted_tokens > maximum_logged_tokens || accepted_tokens > kGdnMaxTokens ||
      channels > (1u << 24) || key_heads == 0 || value_heads == 0 || value_heads % key_heads != 0 ||
      head_size != kGdnD || static_cast<uint64_t>(layer_count) * value_heads > (1u << 30)) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid all-layer GDN prefix restore arguments (at most 32 "
                                       "accepted tokens)");
  }
  auto st = static_cast<hipStream_t>(stream);
  const std::size_t conv_threads = static_cast<std::size_t>(layer_count) * channels;
  hipLaunchKernelGGL(gdn_restore_conv_kernel, dim3(static_cast<unsigned>((conv_threads + 255) / 256)),
                     dim3(256), 0, st, reinterpret_cast<__half*>(conv_states),
                     reinterpret_cast<const __half*>(appended_logs), static_cast<uint32_t>(channels),
                     layer_count, maximum_logged_tokens, accepted_tokens);
  if (const int32_t s = launch_status("all-layer GDN convolution prefix restore launch failed"); s != GFXI_OK) {
    return s;
  }
  hipLaunchKernelGGL(gdn_restore_recurrent_kernel, dim3(layer_count * value_heads), dim3(kRestoreThreads), 0,
                     st, recurrent_states, key_logs, delta_logs, decay_logs, maximum_logged_tokens,
                     accepted_tokens, key_heads, value_heads);
  return launch_status("all-layer GDN recurrent prefix restore launch failed");
}

// ---- attention helpers ----------------------------------------------------------

namespace {
int32_t rope_entry(const float* query_input, const uint16_t* query_weight, uint16_t* query_output,
                   size_t query_heads, size_t query_stride, const float* key_input,
                   const uint16_t* key_weight, uint16_t* key_output, size_t key_heads,
                   size_t key_stride, size_t head_size, size_t rotary, uint64_t base,
                   const uint64_t* indirect, uint32_t batch, float theta, hipStream_t stream,
                   const float* value_input = nullptr, uint16_t* key_cache = nullptr,
                   uint16_t* value_cache = nullptr, size_t capacity = 0) {
  if (value_input != nullptr &&
      (key_cache == nullptr || value_cache == nullptr ||
       (indirect == nullptr && (base > capacity || batch > capacity - base)))) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid fused K/V cache append arguments");
  }
  if (query_input == nullptr || query_weight == nullptr || query_output == nullptr ||
      key_input == nullptr || key_weight == nullptr || key_output == nullptr || query_heads == 0 ||
      key_heads == 0 || (head_size != 128 && head_size != 256) || rotary == 0 || rotary > 64 ||
      rotary % 2 != 0 ||
      query_stride < head_size || key_stride < head_size || batch == 0 || !std::isfinite(theta) ||
      theta <= 0.0F || query_heads > 4096 || key_heads > 4096) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid Q/K RMSNorm/RoPE arguments (head size 128 or 256, "
                                       "even rotary size <= 64)");
  }
  RopeArgs a{query_input, query_weight, reinterpret_cast<__half*>(query_output), key_input, key_weight,
             reinterpret_cast<__half*>(key_output), static_cast<uint32_t>(query_heads),
             static_cast<uint32_t>(query_stride), static_cast<uint32_t>(key_heads),
             static_cast<uint32_t>(key_stride), static_cast<uint32_t>(rotary), batch, base, indirect,
             theta, value_input, reinterpret_cast<__half*>(key_cache),
             reinterpret_cast<__half*>(value_cache)};
  const uint32_t waves = static_cast<uint32_t>(query_heads + key_heads) * batch;
  if (head_size == 128) {
    hipLaunchKernelGGL(qk_norm_rope_kernel<128>, dim3((waves + 3) / 4), dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL(qk_norm_rope_kernel<256>, dim3((waves + 3) / 4), dim3(256), 0, stream, a);
  }
  return launch_status("Q/K RMSNorm/RoPE launch failed");
}

int32_t kv_entry(const uint16_t* key, const float* value, uint16_t* key_cache, uint16_t* value_cache,
                 uint64_t position, const uint64_t* indirect, size_t capacity, uint32_t batch,
                 size_t kv_elements, hipStream_t stream) {
  if (key == nullptr || value == nullptr || key_cache == nullptr || value_cache == nullptr ||
      batch == 0 || kv_elements == 0 || kv_elements > (1u << 24) ||
      (indirect == nullptr && position + batch > capacity)) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid block KV append arguments");
  }
  const std::size_t n = static_cast<std::size_t>(batch) * kv_elements;
  hipLaunchKernelGGL(kv_append_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                     reinterpret_cast<const __half*>(key), value, reinterpret_cast<__half*>(key_cache),
                     reinterpret_cast<__half*>(value_cache), position, indirect,
                     static_cast<uint32_t>(kv_elements), batch);
  return launch_status("block KV append launch failed");
}
}  // namespace

extern "C" int32_t gfxinfer_launch_qk_rms_norm_rope_block(
    const float* query_input, const uint16_t* query_bf16_weight, uint16_t* query_output,
    size_t query_head_count, size_t query_input_stride, const float* key_input,
    const uint16_t* key_bf16_weight, uint16_t* key_output, size_t key_head_count,
    size_t key_input_stride, size_t head_size, size_t rotary_size, uint64_t base_position,
    uint32_t batch, float rope_theta, void* stream) {
  return rope_entry(query_input, query_bf16_weight, query_output, query_head_count, query_input_stride,
                    key_input, key_bf16_weight, key_output, key_head_count, key_input_stride, head_size,
                    rotary_size, base_position, nullptr, batch, rope_theta,
                    static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_qk_rms_norm_rope_block_indirect_position(
    const float* query_input, const uint16_t* query_bf16_weight, uint16_t* query_output,
    size_t query_head_count, size_t query_input_stride, const float* key_input,
    const uint16_t* key_bf16_weight, uint16_t* key_output, size_t key_head_count,
    size_t key_input_stride, size_t head_size, size_t rotary_size,
    const uint64_t* base_position, uint32_t batch, float rope_theta, void* stream) {
  if (base_position == nullptr) return fail(GFXI_INVALID_ARGUMENT, "indirect position is null");
  return rope_entry(query_input, query_bf16_weight, query_output, query_head_count, query_input_stride,
                    key_input, key_bf16_weight, key_output, key_head_count, key_input_stride, head_size,
                    rotary_size, 0, base_position, batch, rope_theta, static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_qk_rms_norm_rope_kv_append_block(
    const float* query_input, const uint16_t* query_bf16_weight, uint16_t* query_output,
    size_t query_head_count, size_t query_input_stride, const float* key_input,
    const uint16_t* key_bf16_weight, uint16_t* key_output, size_t key_head_count,
    size_t key_input_stride, size_t head_size, size_t rotary_size, const float* value_input,
    uint16_t* key_cache, uint16_t* value_cache, size_t capacity, uint64_t base_position,
    uint32_t batch, float rope_theta, void* stream) {
  if (value_input == nullptr) return fail(GFXI_INVALID_ARGUMENT, "fused K/V append needs the value rows");
  return rope_entry(query_input, query_bf16_weight, query_output, query_head_count, query_input_stride,
                    key_input, key_bf16_weight, key_output, key_head_count, key_input_stride, head_size,
                    rotary_size, base_position, nullptr, batch, rope_theta,
                    static_cast<hipStream_t>(stream), value_input, key_cache, value_cache, capacity);
}

extern "C" int32_t gfxinfer_launch_qk_rms_norm_rope_kv_append_block_indirect_position(
    const float* query_input, const uint16_t* query_bf16_weight, uint16_t* query_output,
    size_t query_head_count, size_t query_input_stride, const float* key_input,
    const uint16_t* key_bf16_weight, uint16_t* key_output, size_t key_head_count,
    size_t key_input_stride, size_t head_size, size_t rotary_size, const float* value_input,
    uint16_t* key_cache, uint16_t* value_cache, size_t capacity, const uint64_t* base_position,
    uint32_t batch, float rope_theta, void* stream) {
  if (value_input == nullptr || base_position == nullptr) {
    return fail(GFXI_INVALID_ARGUMENT, "fused K/V append needs the value rows and a position");
  }
  return rope_entry(query_input, query_bf16_weight, query_output, query_head_count, query_input_stride,
                    key_input, key_bf16_weight, key_output, key_head_count, key_input_stride, head_size,
                    rotary_size, 0, base_position, batch, rope_theta, static_cast<hipStream_t>(stream),
                    value_input, key_cache, value_cache, capacity);
}

extern "C" int32_t gfxinfer_launch_kv_append_block(const uint16_t* key, const float* value,
                                                   uint16_t* key_cache, uint16_t* value_cache,
                                                   size_t position, size_t capacity,
                                                   uint32_t batch, size_t kv_elements,
                                                   void* stream) {
  return kv_entry(key, value, key_cache, value_cache, position, nullptr, capacity, batch, kv_elements,
                  static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_kv_append_block_indirect_position(
    const uint16_t* key, const float* value, uint16_t* key_cache, uint16_t* value_cache,
    const uint64_t* position, size_t capacity, uint32_t batch, size_t kv_elements, void* stream) {
  if (position == nullptr) return fail(GFXI_INVALID_ARGUMENT, "indirect position is null");
  return kv_entry(key, value, key_cache, value_cache, 0, position, capacity, batch, kv_elements,
                  static_cast<hipStream_t>(stream));
}

// ---- argmax -------------------------------------------------------------------------

extern "C" int32_t gfxinfer_launch_argmax_batch(const float* logits, uint32_t* tokens,
                                                size_t vocabulary_size, size_t row_stride,
                                                uint32_t batch, void* stream) {
  if (logits == nullptr || tokens == nullptr || vocabulary_size == 0 || row_stride < vocabulary_size ||
      batch == 0 || vocabulary_size > 0xffffffffu) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid batched argmax arguments");
  }
  hipLaunchKernelGGL(argmax_kernel, dim3(batch), dim3(256), 0, static_cast<hipStream_t>(stream),
                     logits, nullptr, tokens, static_cast<uint32_t>(vocabulary_size), row_stride);
  return launch_status("batched argmax launch failed");
}

extern "C" int32_t gfxinfer_launch_argmax_mapped(const float* logits, const uint32_t* token_ids,
                                                 uint32_t* token, size_t vocabulary_size,
                                                 void* stream) {
  if (logits == nullptr || token_ids == nullptr || token == nullptr || vocabulary_size == 0 ||
      vocabulary_size > 0xffffffffu) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid mapped argmax arguments");
  }
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), logits,
                     token_ids, token, static_cast<uint32_t>(vocabulary_size), vocabulary_size);
  return launch_status("mapped argmax launch failed");
}

extern "C" size_t gfxinfer_rope_table_bytes(size_t positions, size_t rotary_size) {
  if (positions == 0 || positions > (1u << 24) || rotary_size < 2 || rotary_size > 64 || rotary_size % 2 != 0) {
    return 0;
  }
  return positions * (rotary_size / 2) * 2 * sizeof(float);
}

extern "C" int32_t gfxinfer_launch_rope_table(float* table, size_t positions, size_t rotary_size, float rope_theta,
                                              void* stream) {
  if (table == nullptr || gfxinfer_rope_table_bytes(positions, rotary_size) == 0 || !std::isfinite(rope_theta) ||
      rope_theta <= 0.0F) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid RoPE table arguments (1..2^24 positions, even rotary size 2..64)");
  }
  const std::size_t n = positions * (rotary_size / 2);
  hipLaunchKernelGGL(rope_table_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), reinterpret_cast<float2*>(table),
                     static_cast<uint32_t>(positions), static_cast<uint32_t>(rotary_size), rope_theta);
  return launch_status("RoPE table launch failed");
}
