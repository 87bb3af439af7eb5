// Shared definitions for the gfx950 speculative-verify library: status codes,
// error text, launch checks and the MI355X packed-weight tile layout.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <exception>
#include <new>
#include <string>

#include "gfxinfer_amd.h"

namespace gfx950 {

constexpr std::size_t kGroup = 128;  // quantization group along K
// MI355X: 256 CUs.  A workgroup of more than eight waves holds a CU alone (two of
// them never share one), so a grid of such workgroups larger than this runs in rounds.
constexpr unsigned kComputeUnits = 256;
constexpr unsigned kWave = 64;       // CDNA wavefront

// Records the message for gfxinfer_last_error() and returns the code.
int32_t fail(int32_t code, const std::string& message);

// Runs a C-ABI entry point's body so that a host allocation failure (or any other
// exception) becomes a status instead of crossing the C boundary.
template <typename Body>
int32_t guarded(Body&& body) noexcept {
  try {
    return body();
  } catch (const std::bad_alloc&) {
    return fail(GFXI_OUT_OF_MEMORY, "host allocation failed");
  } catch (const std::exception& error) {
    return fail(GFXI_INTERNAL, error.what());
  }
}
int32_t ok();
// Maps a HIP error to GFXI_HIP_ERROR with context (reference device.cpp:24-35).
int32_t hip_fail(hipError_t error, const char* context);
// hipGetLastError after a launch, as every reference launcher does.
int32_t launch_status(const char* context);

// fp32 -> fp16 (round to nearest even) of a value first rounded to fp32.  The
// empty asm pins the fp32 value in a register so the compiler cannot fold a
// preceding multiply or add into v_fma_mixlo_f16, which rounds the exact result
// to fp16 once instead of rounding to fp32 first as the source states.
__device__ __forceinline__ __half to_half(float x) {
  asm volatile("" : "+v"(x));
  return __float2half(x);
}

// Cross-lane reductions through DPP lane moves (VALU, no LDS round trip as
// __shfl_xor's ds_bpermute takes).  DPP controls: quad_perm [1,0,3,2] (lane ^ 1),
// quad_perm [2,3,0,1] (lane ^ 2), row_half_mirror (lane i <-> 7 - i within 8 lanes),
// row_mirror (lane i <-> 15 - i within 16 lanes).  After the two quad steps every
// lane of a quad holds the quad's value, so the mirrors pair equal partials exactly
// as xor 4 and xor 8 would: the 16-lane results are bit-identical to the xor tree.
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int Ctrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}

// Sum / maximum over the 16 lanes of each row, in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_move<kDppXor1>(v);
  v += dpp_move<kDppXor2>(v);
  v += dpp_move<kDppHalfMirror>(v);
  v += dpp_move<kDppMirror>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_move<kDppXor1>(v));
  v = fmaxf(v, dpp_move<kDppXor2>(v));
  v = fmaxf(v, dpp_move<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_move<kDppMirror>(v));
  return v;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Wave-wide sum / maximum (all 64 lanes active), wave-uniform result:
// (row0 + row1) + (row2 + row3) of the row sums.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Largest 64-bit key over the wave, in every lane: DPP moves of both words within each
// 16-lane row (the pairings of row16_max), then the four row maxima read out to
// scalars.  Keys compare as integers, so the pairing does not change the result.
template <int Ctrl>
__device__ __forceinline__ unsigned long long dpp_move_key(unsigned long long v) {
  const unsigned lo = static_cast<unsigned>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<unsigned>(v)), Ctrl, 0xF, 0xF, false));
  const unsigned hi = static_cast<unsigned>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<unsigned>(v >> 32)), Ctrl, 0xF, 0xF, false));
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}
__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long v) {
  unsigned long long o = dpp_move_key<kDppXor1>(v);
  v = o > v ? o : v;
  o = dpp_move_key<kDppXor2>(v);
  v = o > v ? o : v;
  o = dpp_move_key<kDppHalfMirror>(v);
  v = o > v ? o : v;
  o = dpp_move_key<kDppMirror>(v);
  v = o > v ? o : v;
  unsigned long long best = 0ull;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<unsigned>(v)), 16 * r));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<unsigned>(v >> 32)), 16 * r));
    const unsigned long long k = (static_cast<unsigned long long>(hi) << 32) | lo;
    best = k > best ? k : best;
  }
  return best;
}

// The row an argmax key names: the key's low word is 0xffffffff - row (so that equal
// values keep the lowest row); key 0 ("no candidate") names row 0.
__device__ __forceinline__ uint32_t argmax_key_row(unsigned long long key) {
  return key == 0ull ? 0u : 0xffffffffu - static_cast<uint32_t>(key);
}

// The largest of `count` argmax keys, reduced by the whole workgroup (blockDim.x a
// multiple of 64, at most 1024 threads), in every thread; `partial` holds one key per
// wave.  Keys are compared as integers, so the order of the reduction does not matter.
__device__ __forceinline__ unsigned long long block_max_key(const unsigned long long* keys, uint32_t count,
                                                            unsigned long long* partial) {
  constexpr unsigned kLoads = 8;
  unsigned long long best = 0ull;
  for (uint32_t base = 0; base < count; base += blockDim.x * kLoads) {
    unsigned long long k[kLoads];
#pragma unroll
    for (unsigned u = 0; u < kLoads; ++u) {
      const uint32_t i = base + u * blockDim.x + threadIdx.x;
      const unsigned long long key = keys[i < count ? i : 0u];  // unconditional: no load waits on a branch
      k[u] = i < count ? key : 0ull;
    }
#pragma unroll
    for (unsigned u = 0; u < kLoads; ++u) best = k[u] > best ? k[u] : best;
  }
  best = wave_max_key(best);
  if ((threadIdx.x & 63u) == 0) partial[threadIdx.x >> 6] = best;
  __syncthreads();
  best = partial[0];
  for (unsigned w = 1; w < blockDim.x / 64; ++w) best = partial[w] > best ? partial[w] : best;
  return best;
}

__device__ __forceinline__ float bf16_to_float(uint16_t value) {
  return __uint_as_float(static_cast<uint32_t>(value) << 16U);  // qwen_ops.hip:27-29
}

// RoPE rotation of lane `lane` < rotary at `position` (qwen_ops.hip:599-676): the angle
// position * theta^(-2 (lane % (rotary / 2)) / rotary); cos and sin of it.
__device__ __forceinline__ void rope_cos_sin(float position, unsigned rotary, float theta, unsigned lane,
                                             float& c, float& s) {
  const unsigned half = rotary / 2;
  const unsigned fi = lane % half;
  const float exponent = (2.0F * static_cast<float>(fi)) / static_cast<float>(rotary);
  const float inverse_frequency = powf(theta, -exponent);
  const float angle = position * inverse_frequency;
  c = cosf(angle);
  s = sinf(angle);
}

// Q/K RMSNorm (eps 1e-6, weights 1 + w) then RoPE of one head row of D values held by
// one wave (all 64 lanes active): lane l holds elements l + 64 j of the row and of its
// bf16 weights.  Dims < rotary rotate with their partner i +- rotary/2 (at rotary 64,
// the other half of the wave: one v_permlane32_swap); c / s are rope_cos_sin's values
// for the lane (unused past rotary).
template <unsigned D>
__device__ __forceinline__ void norm_rope_row(const float (&x)[D / 64], const uint16_t (&wb)[D / 64],
                                              unsigned rotary, float c, float s, unsigned lane,
                                              __half (&h)[D / 64]) {
  constexpr unsigned J = D / 64;
  float square = 0.0F;
#pragma unroll
  for (unsigned j = 0; j < J; ++j) square += x[j] * x[j];
  const float inverse = rsqrtf(wave_sum(square) / static_cast<float>(D) + 1.0e-6F);
  float n[J];
#pragma unroll
  for (unsigned j = 0; j < J; ++j) n[j] = x[j] * (inverse * (1.0F + bf16_to_float(wb[j])));
  float v0 = n[0];
  const unsigned half = rotary / 2;
  float partner;
  if (half == 32u) {
    const unsigned u = __float_as_uint(n[0]);
    const auto swapped = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    partner = __uint_as_float(lane < 32u ? swapped[1] : swapped[0]);
  } else {
    partner = __shfl(n[0], lane < half ? lane + half : lane - half);
  }
  if (lane < rotary) {
    const float rotated = lane < half ? -partner : partner;
    v0 = fmaf(n[0], c, rotated * s);
  }
  h[0] = to_half(v0);
#pragma unroll
  for (unsigned j = 1; j < J; ++j) h[j] = to_half(n[j]);
}

// One wave quantizes 128 fp16 values (two per lane) to A4G128 exactly as
// quantize_activation_i4 (lowbit_gemv.hip:373-407) does.
__device__ __forceinline__ void quantize_group_a4(__half x0h, __half x1h, uint8_t* codes,
                                                  __half* scale_out, unsigned lane) {
  const float x0 = __half2float(x0h), x1 = __half2float(x1h);
  const float maximum = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  const __half scale16 = to_half(maximum == 0.0F ? 1.0F : maximum / 7.0F);
  const float scale = __half2float(scale16);
  const int low = max(-7, min(7, __float2int_rn(x0 / scale)));
  const int high = max(-7, min(7, __float2int_rn(x1 / scale)));
  codes[lane] = static_cast<uint8_t>((low & 0x0f) | ((high & 0x0f) << 4));
  if (lane == 0) *scale_out = scale16;
}

// Signed quantization level of value at scale (quantization.cpp:29-56: encode_value
// then decode_value), clamped to the format's range.
template <int Format>
__device__ __forceinline__ int encode_level(float value, float scale) {
  const float normalized = scale == 0.0F ? 0.0F : value / scale;
  const float rounded = rintf(normalized);
  int q = static_cast<int>(fminf(fmaxf(rounded, -2147483648.0F), 2147483520.0F));
  if constexpr (Format == GFXI_W2G128) {
    // nearest_w2 (quantization.cpp:15-27): first of {-3, -1, 1, 3} with the smallest
    // error, so ties go to the lower level and NaN maps to -3.
    int best = -3;
    float best_error = INFINITY;
    for (int level = -3; level <= 3; level += 2) {
      const float error = fabsf(normalized - static_cast<float>(level));
      if (error < best_error) {
        best = level;
        best_error = error;
      }
    }
    return best;
  } else if constexpr (Format == GFXI_W3G128) {
    return max(-4, min(3, q));
  } else {
    return max(-8, min(7, q));
  }
}

inline bool valid_weight_format(int32_t format) {
  return format == GFXI_W2G128 || format == GFXI_W3G128 || format == GFXI_W4G128;
}

// ---------------------------------------------------------------------------
// gfx950 tile layout of a group-128 packed matrix [N, K] (N % 16 == 0).
//
// codes : [N/16 row tiles][K/128 groups][64 lanes][L bytes]  L = 8 (W2), 12 (W3), 16 (W4)
// scales: [N/16 row tiles][K/128 groups][16 rows] fp16
//
// Lane l of a (tile, group) chunk holds row m = l % 16 of the tile and the 32
// columns kb*32 .. kb*32+31 of the group, kb = l / 16.  Those 32 columns feed two
// v_mfma_i32_16x16x64_i8 K-steps (h = 0, 1; 16 columns each) as the A operand.
// Inside one K-step, operand byte j = 4*reg + byte maps to column
//     16*h + 8*(reg >> 1) + 2*byte + (reg & 1)
// which is the order in which packed 4-bit activations expand with two masks
// (even columns from the low nibbles, odd columns from the high nibbles).
//
// W4: the 16 lane bytes are the 32 columns packed two per byte, even column in
//     the low nibble -- the reference's own W4 byte format for 32 consecutive
//     columns.  A nibble masked into bits 4..7 of a byte reads as 16*w in int8.
// W3: the 12 lane bytes are three dwords S0, S1, S2 holding the eight operand
//     registers out[o] (o = 4*h + reg) as 3-bit two's complement fields that land
//     in bits 5..7 of each byte (int8 value 32*w) with one shift and one mask:
//       out0 = (S0<<5)&E  out1 = (S0<<2)&E  out2 = (S1<<5)&E  out3 = (S1<<2)&E
//       out4 = (S2<<5)&E  out5 = (S2<<2)&E                     (E = 0xE0E0E0E0)
//       out6 = (S0&0xC0C0C0C0) | ((S1>>1)&0x20202020)
//       out7 = (S2&0xC0C0C0C0) | ((S1>>2)&0x20202020)
// ---------------------------------------------------------------------------

// W2: the 8 lane bytes are one dword D_h per K-step h; the code c = (w + 3) / 2 of
//     operand slot (h, reg, byte) sits at bits 8*byte + 2*reg of D_h, so that
//       out_reg = ((D_h << (6 - 2*reg)) & 0xC0C0C0C0) ^ 0xA0A0A0A0
//     puts 64*c - 96 = 32*w (w = 2c - 3 in {-3, -1, 1, 3}) in every byte.
__host__ __device__ constexpr unsigned lane_bytes(int32_t format) {
  return format == GFXI_W2G128 ? 8u : (format == GFXI_W3G128 ? 12u : 16u);
}

// Column (0..31 within the lane's 32) of operand slot (h, reg, byte).
__host__ __device__ constexpr unsigned slot_column(unsigned h, unsigned reg, unsigned byte) {
  return 16u * h + 8u * (reg >> 1) + 2u * byte + (reg & 1u);
}

// Inverse: (h, reg, byte) of lane column c (0..31).
__host__ __device__ inline void column_slot(unsigned c, unsigned& h, unsigned& reg,
                                            unsigned& byte) {
  h = c / 16u;
  const unsigned j = c % 16u;
  reg = 2u * (j / 8u) + (j & 1u);
  byte = (j % 8u) / 2u;
}

// Packs 32 signed weights (column order) of one lane chunk.
__host__ __device__ inline void pack_lane_chunk(int32_t format, const int8_t* w32,
                                                uint8_t* out) {
  if (format == GFXI_W2G128) {
    uint32_t d[2] = {0, 0};
    for (unsigned c = 0; c < 32; ++c) {
      unsigned h, reg, byte;
      column_slot(c, h, reg, byte);
      const uint32_t code = static_cast<uint32_t>((w32[c] + 3) / 2) & 3u;
      d[h] |= code << (8u * byte + 2u * reg);
    }
    for (unsigned h = 0; h < 2; ++h) {
      for (unsigned i = 0; i < 4; ++i) out[4 * h + i] = static_cast<uint8_t>(d[h] >> (8 * i));
    }
    return;
  }
  if (format == GFXI_W4G128) {
    for (unsigned i = 0; i < 16; ++i) {
      out[i] = static_cast<uint8_t>((static_cast<unsigned>(w32[2 * i]) & 0xfu) |
                                    ((static_cast<unsigned>(w32[2 * i + 1]) & 0xfu) << 4));
    }
    return;
  }
  uint32_t s[3] = {0, 0, 0};
  for (unsigned c = 0; c < 32; ++c) {
    unsigned h, reg, byte;
    column_slot(c, h, reg, byte);
    const unsigned o = 4u * h + reg;
    const uint32_t f = static_cast<uint32_t>(w32[c]) & 7u;
    const unsigned base = 8u * byte;
    switch (o) {
      case 0: s[0] |= f << base; break;
      case 1: s[0] |= f << (base + 3); break;
      case 2: s[1] |= f << base; break;
      case 3: s[1] |= f << (base + 3); break;
      case 4: s[2] |= f << base; break;
      case 5: s[2] |= f << (base + 3); break;
      case 6:
        s[0] |= (f >> 1) << (base + 6);
        s[1] |= (f & 1u) << (base + 6);
        break;
      default:
        s[2] |= (f >> 1) << (base + 6);
        s[1] |= (f & 1u) << (base + 7);
        break;
    }
  }
  for (unsigned d = 0; d < 3; ++d) {
    for (unsigned i = 0; i < 4; ++i) out[4 * d + i] = static_cast<uint8_t>(s[d] >> (8 * i));
  }
}

// Signed weight at lane-chunk column c (0..31).
__host__ __device__ inline int unpack_lane_code(int32_t format, const uint8_t* chunk,
                                                unsigned c) {
  if (format == GFXI_W2G128) {
    unsigned h, reg, byte;
    column_slot(c, h, reg, byte);
    const unsigned code = (chunk[4 * h + byte] >> (2u * reg)) & 3u;
    return 2 * static_cast<int>(code) - 3;
  }
  if (format == GFXI_W4G128) {
    const unsigned v = (chunk[c / 2] >> ((c & 1u) * 4u)) & 0xfu;
    return v >= 8u ? static_cast<int>(v) - 16 : static_cast<int>(v);
  }
  uint32_t s[3];
  for (unsigned d = 0; d < 3; ++d) {
    s[d] = static_cast<uint32_t>(chunk[4 * d]) | (static_cast<uint32_t>(chunk[4 * d + 1]) << 8) |
           (static_cast<uint32_t>(chunk[4 * d + 2]) << 16) |
           (static_cast<uint32_t>(chunk[4 * d + 3]) << 24);
  }
  unsigned h, reg, byte;
  column_slot(c, h, reg, byte);
  const unsigned o = 4u * h + reg;
  const unsigned base = 8u * byte;
  uint32_t f;
  switch (o) {
    case 0: f = s[0] >> base; break;
    case 1: f = s[0] >> (base + 3); break;
    case 2: f = s[1] >> base; break;
    case 3: f = s[1] >> (base + 3); break;
    case 4: f = s[2] >> base; break;
    case 5: f = s[2] >> (base + 3); break;
    case 6: f = (((s[0] >> (base + 6)) & 3u) << 1) | ((s[1] >> (base + 6)) & 1u); break;
    default: f = (((s[2] >> (base + 6)) & 3u) << 1) | ((s[1] >> (base + 7)) & 1u); break;
  }
  f &= 7u;
  return f >= 4u ? static_cast<int>(f) - 8 : static_cast<int>(f);
}

// Byte offset of the lane chunk holding (row, column) in the tiled codes.
__host__ __device__ inline std::size_t chunk_offset(int32_t format, std::size_t row,
                                                    std::size_t column, std::size_t groups) {
  const std::size_t tile = row / 16, m = row % 16;
  const std::size_t group = column / kGroup, kb = (column % kGroup) / 32;
  return ((tile * groups + group) * 64 + (kb * 16 + m)) * lane_bytes(format);
}

__host__ __device__ inline std::size_t scale_offset(std::size_t row, std::size_t group,
                                                    std::size_t groups) {
  return ((row / 16) * groups + group) * 16 + row % 16;
}

}  // namespace gfx950
