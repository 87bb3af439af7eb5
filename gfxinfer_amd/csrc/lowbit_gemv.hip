// Packed low-bit GEMV / skinny GEMM for gfx950 (MI355X), plus the activation
// quantizers, the device weight quantizer and the tiled row gather.
//
// Reference semantics: src/kernels/lowbit_gemv.hip (launchers :838-1363) and
// src/quantization.cpp.  The gfx12 WMMA iu4 path has no CDNA4 counterpart, so
// both operands are widened to int8 and multiplied on v_mfma_i32_16x16x64_i8:
// a W3 code lands in bits 5..7 of a byte (value 32*w), a W4 or A4 nibble in bits
// 4..7 (16*w), an A8 code stays as is.  The MFMA sum is therefore F times the
// exact integer dot (F = 512, 256, 32 or 16), and the fp32 epilogue folds 1/F
// into the activation scale, which keeps fmaf(float(P), ws*as, acc) exact.
#include <cstdlib>
#include <cstring>
#include <limits>
#include <mutex>
#include <string>
#include <type_traits>

#include "common.hpp"

namespace gfx950 {
namespace {

using i32x4 = int __attribute__((ext_vector_type(4)));
using u32x4 = unsigned __attribute__((ext_vector_type(4)));
using u32x3 = unsigned __attribute__((ext_vector_type(3)));
using u32x2 = unsigned __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Activation quantizers (lowbit_gemv.hip:373-436): one wave per (token, group);
// lane i owns columns 2i and 2i+1.  The group maximum is exact under any
// reduction order, and x / float(scale16) is an IEEE division, so codes and
// scales are bit-identical to the reference.
// ---------------------------------------------------------------------------

template <int Bits>
__global__ __launch_bounds__(256) void quantize_activation_kernel(
    const __half2* __restrict__ input, uint8_t* __restrict__ output, __half* __restrict__ scales,
    uint32_t columns, uint32_t groups, uint32_t total_groups) {
  const uint32_t linear = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (linear >= total_groups) return;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t batch = linear / groups;
  const uint32_t group = linear - batch * groups;
  const __half2 pair = input[(static_cast<std::size_t>(batch) * columns + group * kGroup) / 2 + lane];
  const float x0 = __low2float(pair);
  const float x1 = __high2float(pair);
  const float maximum = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  constexpr float kLevels = Bits == 4 ? 7.0F : 127.0F;
  constexpr int kClamp = Bits == 4 ? 7 : 127;
  const __half scale16 = to_half(maximum == 0.0F ? 1.0F : maximum / kLevels);
  const float scale = __half2float(scale16);
  const int low = max(-kClamp, min(kClamp, __float2int_rn(x0 / scale)));
  const int high = max(-kClamp, min(kClamp, __float2int_rn(x1 / scale)));
  if constexpr (Bits == 4) {
    output[static_cast<std::size_t>(batch) * (columns / 2) + group * 64u + lane] =
        static_cast<uint8_t>((low & 0x0f) | ((high & 0x0f) << 4));
  } else {
    const uint16_t both = static_cast<uint16_t>((low & 0xff) | ((high & 0xff) << 8));
    reinterpret_cast<uint16_t*>(output)[(static_cast<std::size_t>(batch) * columns +
                                         group * kGroup) / 2 + lane] = both;
  }
  if (lane == 0) scales[linear] = scale16;
}

// ---------------------------------------------------------------------------
// Device weight quantizer: quantization.cpp:163-220 restated per (row, group)
// thread, writing the gfx950 tile layout and fp16 scales (converter.cpp:379-387).
// ---------------------------------------------------------------------------

template <int Format>
__global__ __launch_bounds__(256) void quantize_group128_kernel(
    const float* __restrict__ weights, std::size_t rows, std::size_t columns, std::size_t groups,
    uint8_t* __restrict__ codes, __half* __restrict__ scales, int32_t* __restrict__ non_finite) {
  const std::size_t id = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= rows * groups) return;
  const std::size_t row = id / groups;
  const std::size_t group = id - row * groups;
  const float* source = weights + row * columns + group * kGroup;
  float maximum = 0.0F;
  bool bad = false;
  for (unsigned i = 0; i < kGroup; ++i) {
    const float value = source[i];
    if (!isfinite(value)) {
      bad = true;
      continue;
    }
    maximum = fmaxf(maximum, fabsf(value));
  }
  if (bad && non_finite != nullptr) *non_finite = 1;
  // choose_scale, quantization.cpp:67-92
  float scale = 1.0F;
  if (maximum != 0.0F) {
    scale = maximum / (Format == GFXI_W2G128 ? 3.0F : (Format == GFXI_W3G128 ? 4.0F : 8.0F));
    for (int iteration = 0; iteration < 4; ++iteration) {
      double numerator = 0.0;
      double denominator = 0.0;
      for (unsigned i = 0; i < kGroup; ++i) {
        const float value = source[i];
        const int level = encode_level<Format>(value, scale);
        numerator += static_cast<double>(value) * level;
        denominator += static_cast<double>(level) * level;
      }
      if (denominator == 0.0) break;
      scale = static_cast<float>(numerator / denominator);
    }
    scale = fmaxf(scale, std::numeric_limits<float>::min());
  }
  scales[scale_offset(row, group, groups)] = to_half(scale);
  for (unsigned kb = 0; kb < 4; ++kb) {
    int8_t chunk[32];
    for (unsigned c = 0; c < 32; ++c) {
      chunk[c] = static_cast<int8_t>(encode_level<Format>(source[kb * 32 + c], scale));
    }
    uint8_t packed[16];
    pack_lane_chunk(Format, chunk, packed);
    uint8_t* destination = codes + chunk_offset(Format, row, group * kGroup + kb * 32, groups);
    for (unsigned i = 0; i < lane_bytes(Format); ++i) destination[i] = packed[i];
  }
}

// Buffer descriptors: one SGPR resource per stream, a lane-constant VGPR offset
// and a wave-uniform SGPR offset per access, so a load costs no address VGPRs.
// Reads past num_records return zeros (used for a missing last group).
constexpr int kBufferWord3 = 0x00020000;  // gfx9-family raw buffer, 32-bit data format
constexpr int kStreaming = 2;             // nt: weights are read exactly once

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           kBufferWord3);
}

// ---------------------------------------------------------------------------
// Operand expansion.  Every function returns int8 lanes for one 16x16x64 MFMA
// K-step in the slot order documented in common.hpp.
// ---------------------------------------------------------------------------

// Two packed-nibble dwords (16 columns) -> four operand registers (value 16*x).
__device__ __forceinline__ i32x4 expand_nibbles(unsigned x0, unsigned x1) {
  i32x4 r;
  r[0] = static_cast<int>((x0 << 4) & 0xF0F0F0F0u);
  r[1] = static_cast<int>(x0 & 0xF0F0F0F0u);
  r[2] = static_cast<int>((x1 << 4) & 0xF0F0F0F0u);
  r[3] = static_cast<int>(x1 & 0xF0F0F0F0u);
  return r;
}

// Three W3 dwords (32 columns) -> operand registers of both K-steps (value 32*w).
__device__ __forceinline__ void expand_w3(unsigned s0, unsigned s1, unsigned s2, i32x4& h0,
                                          i32x4& h1) {
  constexpr unsigned E = 0xE0E0E0E0u;
  h0[0] = static_cast<int>((s0 << 5) & E);
  h0[1] = static_cast<int>((s0 << 2) & E);
  h0[2] = static_cast<int>((s1 << 5) & E);
  h0[3] = static_cast<int>((s1 << 2) & E);
  h1[0] = static_cast<int>((s2 << 5) & E);
  h1[1] = static_cast<int>((s2 << 2) & E);
  h1[2] = static_cast<int>((s0 & 0xC0C0C0C0u) | ((s1 >> 1) & 0x20202020u));
  h1[3] = static_cast<int>((s2 & 0xC0C0C0C0u) | ((s1 >> 2) & 0x20202020u));
}

// One W2 dword (16 columns) -> four operand registers (value 32*w): the code of
// register reg sits at bits 2*reg of each byte; 64*c - 96 = ((c << 6) ^ 0xA0) per byte.
__device__ __forceinline__ i32x4 expand_w2(unsigned d) {
  constexpr unsigned M = 0xC0C0C0C0u, X = 0xA0A0A0A0u;
  i32x4 r;
  r[0] = static_cast<int>(((d << 6) & M) ^ X);
  r[1] = static_cast<int>(((d << 4) & M) ^ X);
  r[2] = static_cast<int>(((d << 2) & M) ^ X);
  r[3] = static_cast<int>((d & M) ^ X);
  return r;
}

// Sixteen int8 activations in column order -> operand registers in slot order.
__device__ __forceinline__ i32x4 permute_i8(unsigned d0, unsigned d1, unsigned d2, unsigned d3) {
  i32x4 r;
  r[0] = static_cast<int>(__builtin_amdgcn_perm(d1, d0, 0x06040200u));
  r[1] = static_cast<int>(__builtin_amdgcn_perm(d1, d0, 0x07050301u));
  r[2] = static_cast<int>(__builtin_amdgcn_perm(d3, d2, 0x06040200u));
  r[3] = static_cast<int>(__builtin_amdgcn_perm(d3, d2, 0x07050301u));
  return r;
}

// ---------------------------------------------------------------------------
// GEMM kernel.
//
// One workgroup per 16-row tile (tiles of up to four fused matrices are
// concatenated); its W waves split the K groups and combine in LDS.
// A operand = weights (MFMA rows = matrix rows), B operand = activations
// (MFMA columns = tokens).  Each group is one pair of 16x16x64 MFMAs whose A
// operand is the group's 768/1024 contiguous bytes read with lane l = layout
// lane l.  For batches of at most 4 or 8 tokens the 16 MFMA columns are split
// into GP = 4 or 2 token windows of 16/GP slots: group j of a pack feeds only
// window j (the other B lanes are zero), so one set of four accumulators per
// lane collects GP groups and the fp32 epilogue runs once per pack instead of
// once per group.
// ---------------------------------------------------------------------------

struct GemmMatrix {
  const uint8_t* weights;
  const __half* scales;
  void* output;
  uint32_t tiles;
};

struct GemmArgs {
  GemmMatrix matrix[4];
  uint32_t tile_begin[5];
  const uint8_t* activations;
  const __half* activation_scales;
  int32_t* partials;
  unsigned long long* argmax_keys;  // [batch][tiles] tile-local argmax keys, or null
  uint32_t argmax_rows;             // rows >= this never win the argmax
  uint32_t columns;
  uint32_t groups;
  uint32_t batch;
  // Split-K: workgroup b computes split b % splits of the packs of K for tile (block)
  // b / splits and writes fp32 plane `split` ([splits][batch][rows] per matrix); the
  // consumer sums the planes in plane order.  1 = one plane, the plain product.
  uint32_t splits;
};

// Canonical summation over K.  Every GEMM variant adds the int32 group partials the
// same way, so an output depends only on (row, token, K, splits): not on the batch,
// the kernel family or the launch shape, and a block of tokens gives each token
// exactly what a one-token step gives it (as the reference's sequential epilogue does).
//   * split s of S owns groups [G s / S, G (s + 1) / S) of the G groups;
//   * a split of n groups [b, b + n) is cut into R = range_count(n) ranges, range r
//     holding groups [b + n r / R, b + n (r + 1) / R);
//   * a range's value is v = fmaf(float(partial_g), ws_g * as_g, v) over its groups g
//     in increasing order, from v = 0 (partial_g: the group's exact int32 MFMA sum;
//     ws_g, as_g: the row's fp16 weight scale and the token's activation scale times
//     1/F, as fp32);
//   * a split's output is ((range_0 + range_1) + range_2) + ... in range order.
// A kernel may give a wave several consecutive ranges.  Load chunks start at the
// range's first group and hold CH packs of GP groups; the MFMA pair of a pack leaves
// group pg + w in the lanes of token window w, and add_pack folds the pack's groups
// into the value held by the window-0 lanes in group order.  Groups past the range's
// end are skipped.
struct GroupRange {
  unsigned begin, end;  // groups [begin, end)
};

__host__ __device__ inline GroupRange split_groups(unsigned groups, unsigned split, unsigned splits) {
  return {groups * split / splits, groups * (split + 1u) / splits};
}

__host__ __device__ inline unsigned range_count(unsigned groups_in_split) {
  const unsigned r = (groups_in_split + 9u) / 10u;  // about ten groups per range
  return r < 1u ? 1u : (r > 16u ? 16u : r);
}

__host__ __device__ inline GroupRange canonical_range(unsigned groups, unsigned split, unsigned splits,
                                                      unsigned range, unsigned ranges) {
  const GroupRange own = split_groups(groups, split, splits);
  const unsigned n = own.end - own.begin;
  return {own.begin + n * range / ranges, own.begin + n * (range + 1u) / ranges};
}

// v <- the pack's groups added to v in order: the lane's own group (window 0) and
// then windows 1 .. GP - 1 of the same token slot, moved in from lanes + w * TPAD of
// the 16-lane row (DPP row_shl; lanes of other windows compute values never used).
template <unsigned GP, unsigned TPAD>
__device__ __forceinline__ float add_pack(float v, float c, float p) {
  v = fmaf(c, p, v);
  if constexpr (GP >= 2) v = fmaf(dpp_move<0x100 + TPAD>(c), dpp_move<0x100 + TPAD>(p), v);
  if constexpr (GP == 4) {
    v = fmaf(dpp_move<0x100 + 2 * TPAD>(c), dpp_move<0x100 + 2 * TPAD>(p), v);
    v = fmaf(dpp_move<0x100 + 3 * TPAD>(c), dpp_move<0x100 + 3 * TPAD>(p), v);
  }
  return v;
}

// Fewest ranges of any split of a launch: a workgroup has at most that many waves.
inline unsigned min_range_count(unsigned groups, unsigned splits) {
  unsigned m = 16u;
  for (unsigned s = 0; s < splits; ++s) {
    const GroupRange g = split_groups(groups, s, splits);
    const unsigned r = range_count(g.end - g.begin);
    m = r < m ? r : m;
  }
  return m;
}

// Orderable argmax key of logit v at row: the high word orders values (a total
// order on floats with -0 folded into +0), the low word is ~row so that equal
// values keep the lowest row, as the strict > scan of argmax_logits does
// (qwen_ops.hip:768-807).  NaN and -inf never win and map to 0, the key of
// "no candidate" (the reference then returns index 0).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t row, uint32_t limit) {
  if (row >= limit || !(v > -INFINITY)) return 0ull;
  uint32_t bits = __float_as_uint(v == 0.0F ? 0.0F : v);
  bits = (bits & 0x80000000u) != 0 ? ~bits : (bits | 0x80000000u);
  return (static_cast<unsigned long long>(bits) << 32) | (0xffffffffu - row);
}

// Dynamic LDS: one private region per wave holding the activations of the
// wave's current chunk of groups for every live token ([batch][pitch]), a 16-byte
// zero line read by lanes outside a group's token window, and the chunk's
// activation scales as fp32 already multiplied by 1/F.  A4 activations arrive as
// packed nibbles straight from memory (buffer_load_dwordx4 ... lds, one 16-byte
// piece per lane at LDS base + 16 * lane; a zero piece pads each token row, which
// rotates the LDS banks of consecutive tokens) and are expanded to MFMA operand
// bytes when read; A8 activations are staged through registers already permuted
// to operand order ([group][lane block kb][K-step h][16 bytes]).  After the MFMA
// loop the range values wait in their own area for the ordered sum of the split.
struct GemmLds {
  uint32_t pitch;           // bytes per token row (chunk bytes + 16: rotates LDS banks)
  uint32_t zero_offset;     // zero line
  uint32_t scale_offset;    // fp32 scales [batch][chunk groups]
  uint32_t wscale_offset;   // fp16 weight scales of the chunk [chunk groups][16 rows]
  uint32_t region;          // bytes per wave
  uint32_t results_offset;  // after the wave regions: [ranges][NTB][4][64] fp32 range values
};

__host__ __device__ inline GemmLds gemm_lds_layout(uint32_t chunk_groups, uint32_t batch, int abits,
                                                    uint32_t ntb) {
  GemmLds l{};
  // A4: 64 packed bytes per token per group + a zero piece; A8: 128 operand bytes + 16
  l.pitch = abits == 4 ? chunk_groups * 64u + 16u : chunk_groups * 128u + 16u;
  l.zero_offset = batch * l.pitch;
  if (abits == 4) {
    // whole DMA instructions: 64 pieces of 16 bytes each
    const uint32_t pieces = batch * (l.pitch / 16u);
    l.zero_offset = (pieces + 63u) / 64u * 1024u;
  }
  l.scale_offset = l.zero_offset + 16u;
  l.wscale_offset = (l.scale_offset + batch * chunk_groups * 4u + 15u) & ~15u;
  uint32_t region = l.wscale_offset + chunk_groups * 32u;
  const uint32_t reduce = ntb * 4u * 64u * 4u;
  if (region < reduce) region = reduce;
  l.region = (region + 15u) & ~15u;
  return l;
}

// The LDS kernel's final step for one tile: the split's value from the range values in
// LDS (several ranges) or registers, the fused argmax keys and the output rows.
template <int GP, int NTB, bool HalfOut>
__device__ __forceinline__ void gemm_store_tile(const GemmArgs& args, const GemmMatrix& matrix,
                                                float (&total)[NTB][4], unsigned ranges, unsigned lane,
                                                uint32_t results_offset, unsigned tile, unsigned split,
                                                uint32_t rows) {
  extern __shared__ __align__(16) uint8_t lds_all[];
  constexpr unsigned TPAD = 16 / GP;
  const unsigned n = lane & 15u, kb = lane >> 4;
  const unsigned slot = n % TPAD, window = n / TPAD;
  const uint32_t batch = args.batch;
  if (ranges > 1) {
    const float* results = reinterpret_cast<const float*>(lds_all + results_offset);
#pragma unroll
    for (int t = 0; t < NTB; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) total[t][r] = results[(t * 4 + r) * 64 + lane];
    }
    for (unsigned rg = 1; rg < ranges; ++rg) {
#pragma unroll
      for (int t = 0; t < NTB; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) total[t][r] += results[(rg * NTB * 4u + t * 4 + r) * 64 + lane];
      }
    }
  }
  if (args.argmax_keys != nullptr) {
    // Fused greedy argmax: the best of the tile's 16 rows per token (rows 4kb+r of
    // lanes n, n+16, n+32, n+48), one key per (token, tile).
#pragma unroll
    for (int t = 0; t < NTB; ++t) {
      unsigned long long best = 0ull;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned long long key = argmax_key(total[t][r], tile * 16u + 4u * kb + r, args.argmax_rows);
        best = key > best ? key : best;
      }
      unsigned long long other = __shfl_xor(best, 16);
      best = other > best ? other : best;
      other = __shfl_xor(best, 32);
      best = other > best ? other : best;
      const unsigned token = t * 16u + slot;
      if (kb == 0 && window == 0 && token < batch) {
        args.argmax_keys[static_cast<std::size_t>(token) * matrix.tiles + tile] = best;
      }
    }
  }
  if (window != 0 || matrix.output == nullptr) return;
  const std::size_t plane = static_cast<std::size_t>(split) * batch * rows;
#pragma unroll
  for (int t = 0; t < NTB; ++t) {
    if (t * 16u + slot >= batch) continue;
    const std::size_t out =
        plane + static_cast<std::size_t>(t * 16u + slot) * rows + tile * 16u + 4u * kb;
    if constexpr (HalfOut) {
      __half* o = reinterpret_cast<__half*>(matrix.output) + out;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = to_half(total[t][r]);
    } else {
      float4 value = {total[t][0], total[t][1], total[t][2], total[t][3]};
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(matrix.output) + out) = value;
    }
  }
}

// Workgroups of up to 16 waves (large K) for the 16-token variants; the
// 32-token and A8 variants need more registers and stop at 8 waves.
template <int Format, int ABits, int GP, int NTB, int CH, bool HalfOut, bool Partials>
__global__ __launch_bounds__((NTB == 2 || ABits == 8) ? 512 : 1024) void lowbit_gemm_kernel(
    GemmArgs args, GemmLds layout) {
  constexpr unsigned LB = lane_bytes(Format);
  constexpr unsigned WD = LB / 4;        // weight dwords per lane per group
  constexpr unsigned TPAD = 16 / GP;     // token slots per window
  constexpr unsigned CHG = CH * GP;      // groups per chunk
  constexpr unsigned AGB = ABits == 4 ? 64u : 128u;  // activation bytes per token per group
  constexpr float kInvF =
      1.0F / static_cast<float>((Format == GFXI_W4G128 ? 16 : 32) * (ABits == 4 ? 16 : 1));
  constexpr int kShift = (Format == GFXI_W4G128 ? 4 : 5) + (ABits == 4 ? 4 : 0);
  constexpr bool kDma = ABits == 4;  // A4 pieces go straight from memory to LDS

  extern __shared__ __align__(16) uint8_t lds_all[];

  const unsigned lane = threadIdx.x & 63u;
  // Wave-uniform by construction; readfirstlane lets the compiler keep every
  // per-wave offset in SGPRs (buffer soffset) instead of waterfall loops.
  const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned waves = blockDim.x >> 6;
  uint8_t* lds = lds_all + wave * layout.region;

  // Matrix selection for fused launches.
  const unsigned split = blockIdx.x % args.splits;
  unsigned tile = blockIdx.x / args.splits;
  unsigned index = 0;
#pragma unroll
  for (unsigned i = 1; i < 4; ++i) {
    if (tile >= args.tile_begin[i]) index = i;
  }
  const GemmMatrix matrix = args.matrix[index];
  tile -= args.tile_begin[index];
  const uint32_t groups = args.groups;
  const uint32_t batch = args.batch;
  const uint32_t rows = matrix.tiles * 16u;
  const uint32_t row_bytes = ABits == 4 ? args.columns / 2 : args.columns;
  const auto weights = buffer(matrix.weights + static_cast<std::size_t>(tile) * groups * 64u * LB,
                              groups * 64u * LB);
  const auto weight_scales =
      buffer(matrix.scales + static_cast<std::size_t>(tile) * groups * 16u, groups * 32u);
  const auto activations = buffer(args.activations, batch * row_bytes);

  const unsigned n = lane & 15u;   // B/C column
  const unsigned kb = lane >> 4;   // K lane block (A, B) / row block (C)
  const unsigned slot = n % TPAD;  // token slot of column n
  const unsigned window = n / TPAD;
  const unsigned w_voffset = lane * LB;

  // This wave's ranges of the canonical K partition (waves <= ranges).
  const GroupRange own = split_groups(groups, split, args.splits);
  const unsigned ranges = range_count(own.end - own.begin);
  const unsigned range_begin = ranges * wave / waves;
  const unsigned range_end = ranges * (wave + 1u) / waves;

  // LDS byte offset of this lane's B operand for group j of a pack, token block t
  // (relative to the pack's first group); lanes outside the window read zeros.
  uint32_t b_offset[GP][NTB];
#pragma unroll
  for (unsigned j = 0; j < GP; ++j) {
#pragma unroll
    for (int t = 0; t < NTB; ++t) {
      const unsigned token = t * 16u + slot;
      b_offset[j][t] = (window == j && token < batch)
                           ? token * layout.pitch + j * (kDma ? 64u : 128u) + kb * (kDma ? 16u : 32u)
                           : 0xffffffffu;
    }
  }
  if (lane < 4) reinterpret_cast<uint32_t*>(lds + layout.zero_offset)[lane] = 0u;

  float acc[NTB * 4];    // value of the current range: [token block * 4 + row]
  float total[NTB][4];   // the range value (one range) or the split's sum

  constexpr unsigned kPieces = AGB / 16;  // 16-byte source pieces per token per group
  constexpr unsigned kRowPieces = CHG * kPieces;
  constexpr unsigned kMaxTokens = TPAD * NTB;  // batch capacity of this variant
  constexpr unsigned kDmaRow = kRowPieces + 1; // pieces per token row incl. the zero pad
  constexpr unsigned kMaxPieces = kDma ? 1u : (kMaxTokens * kRowPieces + 63u) / 64u;
  constexpr unsigned kMaxDma = (kMaxTokens * kDmaRow + 63u) / 64u;
  const auto act_scales = buffer(args.activation_scales, batch * groups * 2u);
  for (unsigned range = range_begin; range < range_end; ++range) {
  const GroupRange span = canonical_range(groups, split, args.splits, range, ranges);
#pragma unroll
  for (unsigned m = 0; m < NTB * 4; ++m) acc[m] = 0.0F;
  for (unsigned g0 = span.begin; g0 < span.end; g0 += CHG) {
    // 1) Activation pieces of this chunk (L2-resident), loaded first.  Piece i
    //    is token i / kRowPieces, bytes (i % kRowPieces) * 16 of the chunk.
    const unsigned total_pieces = batch * kRowPieces;
    u32x4 stage[kMaxPieces];
    constexpr unsigned kScaleIters = (kMaxTokens * CHG + 63u) / 64u;
    unsigned short stage_scale[kScaleIters];
    if constexpr (kDma) {
      // Piece i = (token i / kDmaRow, piece i % kDmaRow) lands at LDS byte 16 * i =
      // token * pitch + 16 * piece; the pad piece and absent tokens read zeros.
      const unsigned dma_pieces = batch * kDmaRow;
#pragma unroll
      for (unsigned p = 0; p < kMaxDma; ++p) {
        if (p * 64u >= dma_pieces) break;  // wave-uniform
        const unsigned i = p * 64u + lane;
        const unsigned token = i / kDmaRow;
        const unsigned rem = i - token * kDmaRow;
        const unsigned off = (i < dma_pieces && rem < kRowPieces) ? token * row_bytes + rem * 16u : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(activations, (lds_void*)(lds + p * 1024u),
                                                 16, off, g0 * AGB, 0, 0);
      }
      // Nothing moves above the DMA: the explicit wait below counts the loads after it.
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (unsigned p = 0; p < kMaxPieces; ++p) {
      if constexpr (kDma) break;
      // Pieces of absent tokens read past the descriptor (zeros, no memory request).
      const unsigned i = p * 64u + lane;
      const unsigned token = i / kRowPieces;
      const unsigned rem = i % kRowPieces;
      const unsigned off = i < total_pieces ? token * row_bytes + rem * 16u : 0x80000000u;
      stage[p] = __builtin_amdgcn_raw_buffer_load_b128(activations, off, g0 * AGB, 0);
    }
    // The chunk's weight scales ([CHG groups][16 rows] fp16, contiguous in the tile):
    // one coalesced 16-byte load per lane (lanes < 2 * CHG), staged through LDS, instead
    // of one small scattered load per pack that would stall each pack's epilogue.
    u32x4 wschunk = u32x4{0u, 0u, 0u, 0u};
    if constexpr (!Partials) {
      wschunk = __builtin_amdgcn_raw_buffer_load_b128(weight_scales, lane < 2u * CHG ? lane * 16u : 0x80000000u,
                                                      g0 * 32u, 0);
    }
    if constexpr (!Partials) {
      // entry e < batch * CHG: scale of (token e / CHG, group g0 + e % CHG)
#pragma unroll
      for (unsigned it = 0; it < kScaleIters; ++it) {
        const unsigned e = it * 64u + lane;
        const unsigned off = e < batch * CHG ? ((e / CHG) * groups + e % CHG) * 2u : 0x80000000u;
        stage_scale[it] = __builtin_amdgcn_raw_buffer_load_b16(act_scales, off, g0 * 2u, 0);
      }
    }
    // Keep these small loads ahead of the weight stream: loads complete in issue
    // order, so staging them then waits for them alone (a weight-scale load moved
    // behind the weights would make the staging, and so every MFMA, wait for the
    // whole chunk).
    __builtin_amdgcn_sched_barrier(0);
    // 2) Weights and weight scales of CH packs, all in flight together.
    unsigned wreg[CH][GP][WD];
#pragma unroll
    for (unsigned ci = 0; ci < CH; ++ci) {
#pragma unroll
      for (unsigned j = 0; j < GP; ++j) {
        // groups past the range's end load its last group again (never used)
        const unsigned g_offset = min(g0 + ci * GP + j, span.end - 1u) * 64u * LB;
        if constexpr (Format == GFXI_W2G128) {
          const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(weights, w_voffset, g_offset, kStreaming);
          wreg[ci][j][0] = w[0];
          wreg[ci][j][1] = w[1];
        } else if constexpr (Format == GFXI_W3G128) {
          const u32x3 w = __builtin_amdgcn_raw_buffer_load_b96(weights, w_voffset, g_offset, kStreaming);
          wreg[ci][j][0] = w[0];
          wreg[ci][j][1] = w[1];
          wreg[ci][j][2] = w[2];
        } else {
          const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(weights, w_voffset, g_offset, kStreaming);
          wreg[ci][j][0] = w[0];
          wreg[ci][j][1] = w[1];
          wreg[ci][j][2] = w[2];
          wreg[ci][j][3] = w[3];
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kDma) {
      // The compiler does not order LDS reads after buffer->LDS loads: wait here
      // until only the loads issued after the DMA (weight-scale chunk, activation
      // scales, weights) may still be in flight; loads complete in issue order.
      constexpr unsigned kAfter = (Partials ? 0u : 1u + kScaleIters) + CH * GP;
      static_assert(kAfter <= 63, "vmcnt holds at most 63");
      __builtin_amdgcn_s_waitcnt(static_cast<int>((kAfter & 15u) | ((kAfter >> 4) << 14) | (7u << 4) | (15u << 8)));
    }
    // 3) Expand the activations into operand bytes and stage them (and the
    //    scales) into this wave's LDS region.
#pragma unroll
    for (unsigned p = 0; p < kMaxPieces; ++p) {
      if constexpr (kDma) break;
      const unsigned i = p * 64u + lane;
      if (i < total_pieces) {
        const unsigned token = i / kRowPieces;
        const unsigned rem = i % kRowPieces;
        const u32x4 x = stage[p];
        if constexpr (ABits == 4) {
          // 32 columns (group rem / 4, lane block rem % 4) -> two K-steps
          *reinterpret_cast<i32x4*>(lds + token * layout.pitch + rem * 32u) = expand_nibbles(x[0], x[1]);
          *reinterpret_cast<i32x4*>(lds + token * layout.pitch + rem * 32u + 16u) = expand_nibbles(x[2], x[3]);
        } else {
          // 16 columns = one K-step of (group rem / 8, lane block (rem / 2) % 4)
          *reinterpret_cast<i32x4*>(lds + token * layout.pitch + rem * 16u) = permute_i8(x[0], x[1], x[2], x[3]);
        }
      }
    }
    if constexpr (!Partials) {
#pragma unroll
      for (unsigned it = 0; it < kScaleIters; ++it) {
        const unsigned e = it * 64u + lane;
        if (e < batch * CHG) {
          reinterpret_cast<float*>(lds + layout.scale_offset)[e] =
              __half2float(__ushort_as_half(stage_scale[it])) * kInvF;
        }
      }
      if (lane < 2u * CHG) *reinterpret_cast<u32x4*>(lds + layout.wscale_offset + lane * 16u) = wschunk;
    }
    __builtin_amdgcn_sched_barrier(0);
    // 4) Compute.
#pragma unroll
    for (unsigned ci = 0; ci < CH; ++ci) {
      const unsigned pg = g0 + ci * GP;  // the pack's first group
      if (pg >= span.end) break;
      i32x4 c[NTB];
#pragma unroll
      for (int t = 0; t < NTB; ++t) c[t] = i32x4{0, 0, 0, 0};
#pragma unroll
      for (unsigned j = 0; j < GP; ++j) {
        if (pg + j >= span.end) break;  // wave-uniform: partial last pack of the range
        i32x4 a0, a1;
        if constexpr (Format == GFXI_W2G128) {
          a0 = expand_w2(wreg[ci][j][0]);
          a1 = expand_w2(wreg[ci][j][1]);
        } else if constexpr (Format == GFXI_W3G128) {
          expand_w3(wreg[ci][j][0], wreg[ci][j][1], wreg[ci][j][2], a0, a1);
        } else {
          a0 = expand_nibbles(wreg[ci][j][0], wreg[ci][j][1]);
          a1 = expand_nibbles(wreg[ci][j][2], wreg[ci][j][3]);
        }
#pragma unroll
        for (int t = 0; t < NTB; ++t) {
          const bool on = b_offset[j][t] != 0xffffffffu;
          i32x4 b0, b1;
          if constexpr (kDma) {
            const uint32_t off = on ? b_offset[j][t] + ci * GP * 64u : layout.zero_offset;
            const u32x4 x = *reinterpret_cast<const u32x4*>(lds + off);
            b0 = expand_nibbles(x[0], x[1]);
            b1 = expand_nibbles(x[2], x[3]);
          } else {
            const uint32_t off = on ? b_offset[j][t] + ci * GP * 128u : layout.zero_offset;
            b0 = *reinterpret_cast<const i32x4*>(lds + off);
            b1 = *reinterpret_cast<const i32x4*>(lds + (on ? off + 16u : off));
          }
          c[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, c[t], 0, 0, 0);
          c[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, c[t], 0, 0, 0);
        }
      }
      // Epilogue: lane holds rows 4*kb + r of column n = (token slot, group g_c).
      const unsigned g_c = pg + window;
      if constexpr (Partials) {
#pragma unroll
        for (int t = 0; t < NTB; ++t) {
          const unsigned token = t * 16u + slot;
          if (g_c < span.end && token < batch) {
            const std::size_t row0 = static_cast<std::size_t>(token) * rows + tile * 16u + 4u * kb;
#pragma unroll
            for (int r = 0; r < 4; ++r) args.partials[(row0 + r) * groups + g_c] = c[t][r] >> kShift;
          }
        }
      } else {
        // Columns of dead tokens or of a group past the range hold exact zeros.
        const u32x2 pw = *reinterpret_cast<const u32x2*>(
            lds + layout.wscale_offset + (min(g_c, span.end - 1u) - g0) * 32u + 8u * kb);
        float ws[4];
        ws[0] = __half2float(__ushort_as_half(static_cast<unsigned short>(pw[0] & 0xffffu)));
        ws[1] = __half2float(__ushort_as_half(static_cast<unsigned short>(pw[0] >> 16)));
        ws[2] = __half2float(__ushort_as_half(static_cast<unsigned short>(pw[1] & 0xffffu)));
        ws[3] = __half2float(__ushort_as_half(static_cast<unsigned short>(pw[1] >> 16)));
        const float* scales = reinterpret_cast<const float*>(lds + layout.scale_offset);
        const unsigned gl = min(g_c, span.end - 1u) - g0;
#pragma unroll
        for (int t = 0; t < NTB; ++t) {
          const unsigned token = min(t * 16u + slot, batch - 1u);
          const float as = scales[token * CHG + gl];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc[t * 4 + r] = add_pack<GP, TPAD>(acc[t * 4 + r], static_cast<float>(c[t][r]), ws[r] * as);
          }
        }
      }
    }
  }
  if constexpr (!Partials) {
    // The range value, valid in the lanes of window 0 (the only ones stored).
#pragma unroll
    for (int t = 0; t < NTB; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) total[t][r] = acc[t * 4 + r];
    }
    if (ranges > 1) {
      float* slot_out = reinterpret_cast<float*>(lds_all + layout.results_offset) + range * NTB * 4u * 64u;
#pragma unroll
      for (int t = 0; t < NTB; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) slot_out[(t * 4 + r) * 64 + lane] = total[t][r];
      }
    }
  }
  }  // ranges
  if constexpr (Partials) return;

  if (ranges > 1) {
    // The split's value: range values added in range order, by wave 0.
    __syncthreads();
    if (wave != 0) return;
  }
  gemm_store_tile<GP, NTB, HalfOut>(args, matrix, total, ranges, lane, layout.results_offset, tile, split,
                                    rows);
}

// ---------------------------------------------------------------------------
// Direct-operand GEMM.
//
// Same arithmetic as lowbit_gemm_kernel (one 16x16x64 MFMA pair per group, GP
// token windows, per-pack fp32 epilogue), but the B operands never touch LDS:
// each lane loads the 16 (A4) or 32 (A8) activation bytes of its own (token,
// group, lane block) straight from the L2-resident activation codes and expands
// them in registers with the same masks as the W4 weights; the window mask of
// group j is folded into the expansion masks.  Out-of-range tokens and groups
// read zeros through the buffer descriptor.  A wave reuses its activation
// registers for R consecutive 16-row tiles, so the L2 traffic per weight byte
// falls by R; LDS only holds the final cross-wave reduction, so occupancy is set
// by registers alone.  Workgroup = R tiles x W waves splitting K.
// ---------------------------------------------------------------------------

// Two packed-nibble dwords -> four operand registers (value 16*x), AND-ed with m.
__device__ __forceinline__ i32x4 expand_nibbles_masked(unsigned x0, unsigned x1, unsigned m) {
  i32x4 r;
  r[0] = static_cast<int>((x0 << 4) & m);
  r[1] = static_cast<int>(x0 & m);
  r[2] = static_cast<int>((x1 << 4) & m);
  r[3] = static_cast<int>(x1 & m);
  return r;
}

// Lane `source` of each 16-lane row, broadcast over its row (DPP row_newbcast); source
// is a compile-time constant wherever the callers' loops are unrolled.
template <int Source>
__device__ __forceinline__ unsigned row_broadcast_lane(unsigned v) {
  return static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x150 + Source, 0xF, 0xF, false));
}
__device__ __forceinline__ unsigned row_broadcast(unsigned v, unsigned source) {
  switch (source) {
    case 0: return row_broadcast_lane<0>(v);
    case 1: return row_broadcast_lane<1>(v);
    case 2: return row_broadcast_lane<2>(v);
    case 3: return row_broadcast_lane<3>(v);
    case 4: return row_broadcast_lane<4>(v);
    case 5: return row_broadcast_lane<5>(v);
    case 6: return row_broadcast_lane<6>(v);
    case 7: return row_broadcast_lane<7>(v);
    case 8: return row_broadcast_lane<8>(v);
    case 9: return row_broadcast_lane<9>(v);
    case 10: return row_broadcast_lane<10>(v);
    case 11: return row_broadcast_lane<11>(v);
    case 12: return row_broadcast_lane<12>(v);
    case 13: return row_broadcast_lane<13>(v);
    case 14: return row_broadcast_lane<14>(v);
    default: return row_broadcast_lane<15>(v);
  }
}

// Waves per workgroup of the direct kernel: the stream sets of the canonical
// summation need up to ~190 VGPRs at 32 tokens, so a workgroup stops at eight waves.
constexpr unsigned kDirectMaxWaves = 8;

template <int GP, int NTB, int R, bool HalfOut>
__device__ __forceinline__ void direct_finish(const GemmArgs& args, const GemmMatrix& matrix,
                                              float (&total)[R][NTB][4], unsigned ranges, unsigned lane,
                                              unsigned tile0, unsigned valid, unsigned split);

template <int Format, int ABits, int GP, int NTB, int CH, int R, bool HalfOut, bool Partials>
__global__ __launch_bounds__(kDirectMaxWaves * 64) void lowbit_gemm_direct_kernel(GemmArgs args) {
  constexpr unsigned LB = lane_bytes(Format);
  constexpr unsigned WD = LB / 4;                     // weight dwords per lane per group
  constexpr unsigned TPAD = 16 / GP;                  // token slots per window
  constexpr unsigned CHG = CH * GP;                   // groups per chunk
  constexpr unsigned AGB = ABits == 4 ? 64u : 128u;   // activation bytes per token per group
  constexpr unsigned AD = ABits == 4 ? 4u : 8u;       // activation dwords per lane per group
  constexpr float kInvF =
      1.0F / static_cast<float>((Format == GFXI_W4G128 ? 16 : 32) * (ABits == 4 ? 16 : 1));
  constexpr int kShift = (Format == GFXI_W4G128 ? 4 : 5) + (ABits == 4 ? 4 : 0);
  constexpr unsigned kOut = 0x80000000u;              // voffset that reads zeros

  extern __shared__ __align__(16) uint8_t lds_all[];
  const unsigned lane = threadIdx.x & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned waves = blockDim.x >> 6;

  const unsigned split = blockIdx.x % args.splits;
  unsigned block = blockIdx.x / args.splits;
  unsigned index = 0;
#pragma unroll
  for (unsigned i = 1; i < 4; ++i) {
    if (block >= args.tile_begin[i]) index = i;
  }
  const GemmMatrix matrix = args.matrix[index];
  block -= args.tile_begin[index];
  const unsigned tile0 = block * R;
  const unsigned valid = min(static_cast<unsigned>(R), matrix.tiles - tile0);  // wave-uniform
  const uint32_t groups = args.groups;
  const uint32_t batch = args.batch;
  const uint32_t rows = matrix.tiles * 16u;
  const uint32_t row_bytes = ABits == 4 ? args.columns / 2 : args.columns;
  const uint32_t tile_bytes = groups * 64u * LB;
  const auto weights = buffer(matrix.weights + static_cast<std::size_t>(tile0) * tile_bytes,
                              valid * tile_bytes);
  const auto weight_scales =
      buffer(matrix.scales + static_cast<std::size_t>(tile0) * groups * 16u, valid * groups * 32u);
  const auto activations = buffer(args.activations, batch * row_bytes);
  // Scale rows are read as aligned dwords; the range is rounded up to the enclosing
  // dword (never past the page of the last scale) so that the last half is not
  // dropped by the descriptor's per-dword range check.
  const auto act_scales = buffer(args.activation_scales, (batch * groups * 2u + 3u) & ~3u);

  const unsigned n = lane & 15u;
  const unsigned kb = lane >> 4;
  const unsigned slot = n % TPAD;
  const unsigned window = n / TPAD;
  const unsigned w_lane = lane * LB;
  const unsigned ws_voffset = (window * 16u + 4u * kb) * 2u;
  // With one window (GP == 1) the activation loads run in quad-coalesced order
  // (lanes 4m..4m+3 read the 64 contiguous bytes of token m) and ds_bpermute routes
  // each dword to MFMA order (lane kb*16 + n holds token n, lane block kb): in MFMA
  // order each quad would touch four token rows, i.e. four cache lines.
  constexpr bool kCoalesced = GP == 1 && ABits == 4;
  const unsigned load_token = kCoalesced ? lane >> 2 : slot;
  const unsigned load_piece = kCoalesced ? lane & 3u : kb;
  const int permute_from = static_cast<int>((n * 4u + kb) * 4u);
  unsigned a_voffset[NTB], as_voffset[NTB];
#pragma unroll
  for (int t = 0; t < NTB; ++t) {
    const unsigned token = t * 16u + load_token;  // >= batch lands past the buffer: zeros
    a_voffset[t] = token * row_bytes + window * AGB + load_piece * (AGB / 4u);
    as_voffset[t] = ((t * 16u + slot) * groups + window) * 2u;
  }

  // This wave's ranges of the canonical K partition (waves <= ranges).
  const GroupRange own = split_groups(groups, split, args.splits);
  const unsigned ranges = range_count(own.end - own.begin);
  const unsigned range_begin = ranges * wave / waves;
  const unsigned range_end = ranges * (wave + 1u) / waves;

  float acc[R * NTB * 4];   // value of the current range: [(tile, token block) * 4 + row]
  float total[R][NTB][4];   // the range value (one range) or the split's sum
  for (unsigned range = range_begin; range < range_end; ++range) {
  const GroupRange span = canonical_range(groups, split, args.splits, range, ranges);
#pragma unroll
  for (unsigned m = 0; m < R * NTB * 4; ++m) acc[m] = 0.0F;

  for (unsigned g0 = span.begin; g0 < span.end; g0 += CHG) {
    // 1) Loads of CH packs: activations + their scales (L2), weights + scales (HBM).
    unsigned areg[CH][NTB][AD];
    unsigned short asreg[CH][NTB];
    unsigned wreg[R][CHG][WD];
    u32x2 wsreg[R][CH];
    // GP == 1: the weight scales of the chunk's CH groups in one load per tile: lane
    // 16 kb + n holds rows 4 kb .. 4 kb + 3 of group g0 + n, and group g0 + ci reaches
    // every lane of row kb by a DPP row broadcast of lane ci (no lane loads a scale that
    // another lane of its row also loads).
    u32x2 wsrow[R];
    if constexpr (GP == 1 && !Partials) {
      static_assert(CHG <= 16, "one scale per lane of a 16-lane row");
      const unsigned wsv = n < CHG && g0 + n < span.end ? n * 32u + kb * 8u : kOut;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        wsrow[r] = __builtin_amdgcn_raw_buffer_load_b64(weight_scales, static_cast<unsigned>(r) < valid ? wsv : kOut,
                                                        r * groups * 32u + g0 * 32u, 0);
      }
    }
    // GP == 1: the activation scales of the chunk's CH groups, one load per token block
    // (a token's scales are contiguous over groups but may start at an odd half, so
    // the aligned dwords around them are loaded and shifted into place; entries past
    // the chunk or the row are never used).
    constexpr unsigned kScaleDwords = (CH + 1) / 2 + 1;
    static_assert(kScaleDwords <= 4, "chunk too long for one scale load");
    unsigned asrow[NTB][4];
    unsigned as_odd[NTB];
    if constexpr (GP == 1 && !Partials) {
#pragma unroll
      for (int t = 0; t < NTB; ++t) {
        const unsigned first = (t * 16u + slot) * groups + g0;  // half index
        as_odd[t] = first & 1u;
        const unsigned off = t * 16u + slot < batch ? (first & ~1u) * 2u : kOut;
        if constexpr (kScaleDwords == 2) {
          const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(act_scales, off, 0, 0);
          asrow[t][0] = v[0];
          asrow[t][1] = v[1];
        } else if constexpr (kScaleDwords == 3) {
          const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(act_scales, off, 0, 0);
          asrow[t][0] = v[0];
          asrow[t][1] = v[1];
          asrow[t][2] = v[2];
        } else {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(act_scales, off, 0, 0);
          asrow[t][0] = v[0];
          asrow[t][1] = v[1];
          asrow[t][2] = v[2];
          asrow[t][3] = v[3];
        }
      }
    }
    // Activations (L2) of all CH packs first, then the weight stream (HBM): loads
    // complete in issue order, so routing the activations waits for them alone.
#pragma unroll
    for (unsigned ci = 0; ci < CH; ++ci) {
      // a pack past the range's end loads its last group again (never used)
      const unsigned pg = min(g0 + ci * GP, span.end - 1u);
      const bool live = pg + window < span.end;
#pragma unroll
      for (int t = 0; t < NTB; ++t) {
        const unsigned off = live ? a_voffset[t] : kOut;
        const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(activations, off, pg * AGB, 0);
        areg[ci][t][0] = x[0];
        areg[ci][t][1] = x[1];
        areg[ci][t][2] = x[2];
        areg[ci][t][3] = x[3];
        if constexpr (ABits == 8) {
          const u32x4 y =
              __builtin_amdgcn_raw_buffer_load_b128(activations, off + 16u, pg * AGB, 0);
          areg[ci][t][4] = y[0];
          areg[ci][t][5] = y[1];
          areg[ci][t][6] = y[2];
          areg[ci][t][7] = y[3];
        }
        if constexpr (!Partials && GP > 1) {
          asreg[ci][t] = __builtin_amdgcn_raw_buffer_load_b16(act_scales, live ? as_voffset[t] : kOut,
                                                              pg * 2u, 0);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (unsigned ci = 0; ci < CH; ++ci) {
      const unsigned pg = min(g0 + ci * GP, span.end - 1u);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        // a tile past the matrix (short last block) reads zeros and is never stored
        const unsigned w_voffset = static_cast<unsigned>(r) < valid ? w_lane : kOut;
#pragma unroll
        for (unsigned j = 0; j < GP; ++j) {
          const unsigned g_offset = r * tile_bytes + min(pg + j, span.end - 1u) * 64u * LB;
          if constexpr (Format == GFXI_W2G128) {
            const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(weights, w_voffset, g_offset, kStreaming);
            wreg[r][ci * GP + j][0] = w[0];
            wreg[r][ci * GP + j][1] = w[1];
          } else if constexpr (Format == GFXI_W3G128) {
            const u32x3 w = __builtin_amdgcn_raw_buffer_load_b96(weights, w_voffset, g_offset, kStreaming);
            wreg[r][ci * GP + j][0] = w[0];
            wreg[r][ci * GP + j][1] = w[1];
            wreg[r][ci * GP + j][2] = w[2];
          } else {
            const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(weights, w_voffset, g_offset, kStreaming);
            wreg[r][ci * GP + j][0] = w[0];
            wreg[r][ci * GP + j][1] = w[1];
            wreg[r][ci * GP + j][2] = w[2];
            wreg[r][ci * GP + j][3] = w[3];
          }
        }
        if constexpr (!Partials && GP > 1) {
          wsreg[r][ci] = __builtin_amdgcn_raw_buffer_load_b64(
              weight_scales, static_cast<unsigned>(r) < valid ? ws_voffset : kOut, r * groups * 32u + pg * 32u, 0);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kCoalesced) {
      // Quad-coalesced load order -> MFMA lane order.
#pragma unroll
      for (unsigned ci = 0; ci < CH; ++ci)
#pragma unroll
        for (int t = 0; t < NTB; ++t)
#pragma unroll
          for (unsigned d = 0; d < 4; ++d) {
            areg[ci][t][d] = static_cast<unsigned>(
                __builtin_amdgcn_ds_bpermute(permute_from, static_cast<int>(areg[ci][t][d])));
          }
    }
    if constexpr (GP == 1 && !Partials) {
#pragma unroll
      for (int t = 0; t < NTB; ++t) {
        unsigned row[kScaleDwords - 1];
#pragma unroll
        for (unsigned d = 0; d + 1 < kScaleDwords; ++d) {
          row[d] = __builtin_amdgcn_alignbit(asrow[t][d + 1], asrow[t][d], as_odd[t] * 16u);
        }
#pragma unroll
        for (unsigned ci = 0; ci < CH; ++ci) {
          // group g0 + ci sits at half ci of the shifted row (or is past the range)
          asreg[ci][t] = static_cast<unsigned short>(row[ci / 2] >> ((ci & 1u) * 16u));
        }
      }
    }
    // 2) Compute.
#pragma unroll
    for (unsigned ci = 0; ci < CH; ++ci) {
      const unsigned pg = g0 + ci * GP;  // the pack's first group
      if (pg >= span.end) break;
      // B operands of every group of the pack: this lane's activations where its
      // window is the group's, zeros elsewhere.
      i32x4 b[GP][NTB][2];
#pragma unroll
      for (unsigned j = 0; j < GP; ++j) {
        const unsigned on = (GP == 1 || window == j) ? 0xffffffffu : 0u;
#pragma unroll
        for (int t = 0; t < NTB; ++t) {
          if constexpr (ABits == 4) {
            b[j][t][0] = expand_nibbles_masked(areg[ci][t][0], areg[ci][t][1], 0xF0F0F0F0u & on);
            b[j][t][1] = expand_nibbles_masked(areg[ci][t][2], areg[ci][t][3], 0xF0F0F0F0u & on);
          } else {
            const i32x4 p0 = permute_i8(areg[ci][t][0], areg[ci][t][1], areg[ci][t][2], areg[ci][t][3]);
            const i32x4 p1 = permute_i8(areg[ci][t][4], areg[ci][t][5], areg[ci][t][6], areg[ci][t][7]);
            const int m = static_cast<int>(on);
            b[j][t][0] = i32x4{p0[0] & m, p0[1] & m, p0[2] & m, p0[3] & m};
            b[j][t][1] = i32x4{p1[0] & m, p1[1] & m, p1[2] & m, p1[3] & m};
          }
        }
      }
      float as[NTB];
      if constexpr (!Partials) {
#pragma unroll
        for (int t = 0; t < NTB; ++t) as[t] = __half2float(__ushort_as_half(asreg[ci][t])) * kInvF;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (static_cast<unsigned>(r) >= valid) break;  // wave-uniform: short last block
        i32x4 c[NTB];
#pragma unroll
        for (int t = 0; t < NTB; ++t) c[t] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (unsigned j = 0; j < GP; ++j) {
          if (pg + j >= span.end) break;  // wave-uniform: partial last pack of the range
          i32x4 a0, a1;
          const unsigned* w = wreg[r][ci * GP + j];
          if constexpr (Format == GFXI_W2G128) {
            a0 = expand_w2(w[0]);
            a1 = expand_w2(w[1]);
          } else if constexpr (Format == GFXI_W3G128) {
            expand_w3(w[0], w[1], w[2], a0, a1);
          } else {
            a0 = expand_nibbles(w[0], w[1]);
            a1 = expand_nibbles(w[2], w[3]);
          }
#pragma unroll
          for (int t = 0; t < NTB; ++t) {
            c[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b[j][t][0], c[t], 0, 0, 0);
            c[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b[j][t][1], c[t], 0, 0, 0);
          }
        }
        const unsigned g_c = pg + window;
        if constexpr (Partials) {
#pragma unroll
          for (int t = 0; t < NTB; ++t) {
            const unsigned token = t * 16u + slot;
            if (g_c < span.end && token < batch) {
              const std::size_t row0 =
                  static_cast<std::size_t>(token) * rows + (tile0 + r) * 16u + 4u * kb;
#pragma unroll
              for (int i = 0; i < 4; ++i) args.partials[(row0 + i) * groups + g_c] = c[t][i] >> kShift;
            }
          }
        } else {
          // Dead tokens and a missing last group hold exact zeros (and zero scales).
          u32x2 pw;
          if constexpr (GP == 1) {
            pw[0] = row_broadcast(wsrow[r][0], ci);
            pw[1] = row_broadcast(wsrow[r][1], ci);
          } else {
            pw = wsreg[r][ci];
          }
          float ws[4];
          ws[0] = __half2float(__ushort_as_half(static_cast<unsigned short>(pw[0] & 0xffffu)));
          ws[1] = __half2float(__ushort_as_half(static_cast<unsigned short>(pw[0] >> 16)));
          ws[2] = __half2float(__ushort_as_half(static_cast<unsigned short>(pw[1] & 0xffffu)));
          ws[3] = __half2float(__ushort_as_half(static_cast<unsigned short>(pw[1] >> 16)));
#pragma unroll
          for (int t = 0; t < NTB; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float& a = acc[(r * NTB + t) * 4 + i];
              a = add_pack<GP, TPAD>(a, static_cast<float>(c[t][i]), ws[i] * as[t]);
            }
          }
        }
      }
    }
  }
  if constexpr (!Partials) {
    // The range value, valid in the lanes of window 0 (the only ones stored).
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < NTB; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) total[r][t][i] = acc[(r * NTB + t) * 4 + i];
    if (ranges > 1) {
      float* out = reinterpret_cast<float*>(lds_all) + range * R * NTB * 4u * 64u;
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NTB; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) out[((r * NTB + t) * 4 + i) * 64 + lane] = total[r][t][i];
    }
  }
  }  // ranges
  if constexpr (Partials) return;
  if (ranges > 1) {
    // The split's value: range values added in range order, by wave 0.
    __syncthreads();
    if (wave != 0) return;
  }
  direct_finish<GP, NTB, R, HalfOut>(args, matrix, total, ranges, lane, tile0, valid, split);
}

// The direct kernels' final step for R tiles (in the wave that holds the split's value
// in `total`, or after the range values were written to LDS): the ordered sum of the
// range values, the fused argmax keys, the output rows and the SwiGLU arrival.
template <int GP, int NTB, int R, bool HalfOut>
__device__ __forceinline__ void direct_finish(const GemmArgs& args, const GemmMatrix& matrix,
                                              float (&total)[R][NTB][4], unsigned ranges, unsigned lane,
                                              unsigned tile0, unsigned valid, unsigned split) {
  extern __shared__ __align__(16) uint8_t lds_all[];
  constexpr unsigned TPAD = 16 / GP;
  const unsigned n = lane & 15u, kb = lane >> 4;
  const unsigned slot = n % TPAD, window = n / TPAD;
  const uint32_t batch = args.batch;
  const uint32_t rows = matrix.tiles * 16u;
  if (ranges > 1) {
    const float* results = reinterpret_cast<const float*>(lds_all);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < NTB; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) total[r][t][i] = results[((r * NTB + t) * 4 + i) * 64 + lane];
    for (unsigned rg = 1; rg < ranges; ++rg) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NTB; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            total[r][t][i] += results[(((rg * R + r) * NTB + t) * 4 + i) * 64 + lane];
          }
    }
  }
  const std::size_t plane = static_cast<std::size_t>(split) * batch * rows;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (static_cast<unsigned>(r) >= valid) break;
    const unsigned tile = tile0 + r;
    if (args.argmax_keys != nullptr) {
#pragma unroll
      for (int t = 0; t < NTB; ++t) {
        unsigned long long best = 0ull;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const unsigned long long key = argmax_key(total[r][t][i], tile * 16u + 4u * kb + i, args.argmax_rows);
          best = key > best ? key : best;
        }
        unsigned long long other = __shfl_xor(best, 16);
        best = other > best ? other : best;
        other = __shfl_xor(best, 32);
        best = other > best ? other : best;
        const unsigned token = t * 16u + slot;
        if (kb == 0 && window == 0 && token < batch) {
          args.argmax_keys[static_cast<std::size_t>(token) * matrix.tiles + tile] = best;
        }
      }
    }
    if (window != 0 || matrix.output == nullptr) continue;
#pragma unroll
    for (int t = 0; t < NTB; ++t) {
      if (t * 16u + slot >= batch) continue;
      const std::size_t out =
          plane + static_cast<std::size_t>(t * 16u + slot) * rows + tile * 16u + 4u * kb;
      if constexpr (HalfOut) {
        __half* o = reinterpret_cast<__half*>(matrix.output) + out;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = to_half(total[r][t][i]);
      } else {
        float4 value = {total[r][t][0], total[r][t][1], total[r][t][2], total[r][t][3]};
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(matrix.output) + out) = value;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Dot-product GEMV: W3/W4 weights x A4 activations, 1-8 tokens, on v_dot8_i32_i4
// (eight signed nibble products per lane per instruction) instead of MFMA.
//
// A wave serves a quad of four consecutive 16-row tiles and one range of the
// canonical K partition.  It loads each (tile, group) chunk exactly as the MFMA
// kernels do -- lane l gets piece (kb = l / 16, row m = l % 16), one coalesced
// 768/1024-byte load per chunk -- and then exchanges pieces between the four lane
// rows (v_permlane32_swap, v_permlane16_swap) so that lane (q, m) holds the whole
// 128-column group of row m of tile q.  Every lane then works on the same group, so
// a token's 64 bytes of A4 codes are wave-uniform: they come from scalar loads and
// feed v_dot8 from SGPRs, with no activation staging, no LDS and no operand
// expansion on the activation side.  W4 nibbles are used as stored; a W3 lane piece
// becomes four nibble dwords holding 2w per column with about four instructions each.
// Each lane owns one (row, token) value per token, so the fp32 epilogue is one
// fmaf per (row, token, group) and no cross-lane sum is needed.
// ---------------------------------------------------------------------------

constexpr unsigned kDotMaxWaves = 8;
constexpr unsigned kDotMaxGroups = 10;  // largest canonical range (range_count: at most ten groups)

// Per-wave LDS staging of a range: A4 codes [NT][kDotMaxGroups][64 B] filled by whole
// 1 KiB DMA instructions, then the activation scales (six dwords per token).
template <int NT>
constexpr unsigned kDotCodeDma = (NT * kDotMaxGroups * 4u + 63u) / 64u;
template <int NT>
constexpr unsigned kDotCodeRegion = kDotCodeDma<NT> * 1024u;
template <int NT>
constexpr unsigned kDotRegion = kDotCodeRegion<NT> + 256u;

// Three W3 dwords of one lane piece (32 columns) -> four nibble dwords in column
// order: nibble i of dword j holds 2w of column 8j + i (the 3-bit two's complement
// code in bits 1..3 of a nibble reads as 2w).  Per byte of s0/s1/s2 the codes of
// operand registers 0/2/4 sit in bits 0..2 and those of 1/3/5 in bits 3..5, so
// ((s & 0x3F) + (s & 0x38)) << 1 puts them in bits 1..3 and 5..7 (no carry: the
// sum is below 128); registers 6 and 7 are split over bits 6..7 of s0/s2 and s1.
__device__ __forceinline__ void w3_nibbles(unsigned s0, unsigned s1, unsigned s2, unsigned* n) {
  n[0] = ((s0 & 0x3F3F3F3Fu) + (s0 & 0x38383838u)) << 1;
  n[1] = ((s1 & 0x3F3F3F3Fu) + (s1 & 0x38383838u)) << 1;
  n[2] = ((s2 & 0x3F3F3F3Fu) + (s2 & 0x38383838u)) << 1;
  n[3] = ((s0 >> 4) & 0x0C0C0C0Cu) | ((s1 >> 5) & 0x02020202u) | (s2 & 0xC0C0C0C0u) |
         ((s1 >> 2) & 0x20202020u);
}

// 4 x 4 exchange between the lane rows (16 lanes each): on entry r[q] holds, in lane
// row k, a dword of piece k of tile q; on exit r[k] holds, in lane row q, the same
// dword of piece k of tile q.  v_permlane32_swap exchanges the upper half of its
// first operand with the lower half of its second, v_permlane16_swap the odd rows of
// its first operand with the even rows of its second.
__device__ __forceinline__ void exchange_rows(unsigned& r0, unsigned& r1, unsigned& r2, unsigned& r3) {
  const u32x2 a = __builtin_amdgcn_permlane32_swap(r0, r2, false, false);
  const u32x2 b = __builtin_amdgcn_permlane32_swap(r1, r3, false, false);
  const u32x2 c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const u32x2 d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  r0 = c[0];
  r1 = c[1];
  r2 = d[0];
  r3 = d[1];
}

// NT = the launch's token count.
template <int Format, int NT, bool HalfOut, bool Partials>
__global__ __launch_bounds__(kDotMaxWaves * 64) void lowbit_gemm_dot_kernel(GemmArgs args) {
  static_assert(Format == GFXI_W3G128 || Format == GFXI_W4G128, "nibble dot needs W3 or W4");
  constexpr unsigned LB = lane_bytes(Format);
  constexpr unsigned WD = LB / 4;
  // The dot of 2w (W3) or w (W4) with a: 1/F folded into the activation scale keeps
  // fmaf(float(P), ws * as, v) exact, as in the MFMA kernels.
  constexpr float kInvF = Format == GFXI_W3G128 ? 0.5F : 1.0F;
  constexpr int kShift = Format == GFXI_W3G128 ? 1 : 0;
  // Dynamic LDS: one staging region per wave (kDotRegion), then the range values
  // [ranges][NT][64] fp32 summed in range order at the end.
  extern __shared__ __align__(16) uint8_t dot_lds[];

  const unsigned lane = threadIdx.x & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned waves = blockDim.x >> 6;
  const unsigned q = lane >> 4, m = lane & 15u;

  const unsigned split = blockIdx.x % args.splits;
  unsigned quad = blockIdx.x / args.splits;
  unsigned index = 0;
#pragma unroll
  for (unsigned i = 1; i < 4; ++i) {
    if (quad >= args.tile_begin[i]) index = i;
  }
  const GemmMatrix matrix = args.matrix[index];
  quad -= args.tile_begin[index];
  const unsigned tile0 = quad * 4u;
  const unsigned valid = min(4u, matrix.tiles - tile0);  // tiles of this quad inside the matrix
  const uint32_t groups = args.groups;
  const uint32_t batch = args.batch;
  const uint32_t rows = matrix.tiles * 16u;
  const auto weights = buffer(matrix.weights + static_cast<std::size_t>(tile0) * groups * 64u * LB,
                              valid * groups * 64u * LB);
  const auto weight_scales =
      buffer(matrix.scales + static_cast<std::size_t>(tile0) * groups * 16u, valid * groups * 32u);
  const uint32_t row_bytes = args.columns / 2u;
  const auto activations = buffer(args.activations, batch * row_bytes);
  const auto activation_scales = buffer(args.activation_scales, Partials ? 0u : batch * groups * 2u);
  uint8_t* stage = dot_lds + wave * kDotRegion<NT>;
  float* dot_results = reinterpret_cast<float*>(dot_lds + waves * kDotRegion<NT>);
  const unsigned row = (tile0 + q) * 16u + m;
  const bool live = q < valid;

  const GroupRange own = split_groups(groups, split, args.splits);
  const unsigned ranges = range_count(own.end - own.begin);
  const unsigned range_begin = ranges * wave / waves;
  const unsigned range_end = ranges * (wave + 1u) / waves;
  const unsigned ws_voffset = live ? (q * groups * 16u + m) * 2u : 0x80000000u;

  float total[NT];
  for (unsigned range = range_begin; range < range_end; ++range) {
    const GroupRange span = canonical_range(groups, split, args.splits, range, ranges);
    const unsigned count = span.end - span.begin;  // 1..kDotMaxGroups
    // 1) The range's A4 codes ([token][group][64 B]) and activation scales go memory ->
    //    LDS first: anything requested after the weight stream arrives about one stream
    //    time later.  Scales: six dwords per token from the pair holding its first group.
#pragma unroll
    for (unsigned d = 0; d < kDotCodeDma<NT>; ++d) {
      const unsigned piece = d * 64u + lane;
      const unsigned t = piece / (kDotMaxGroups * 4u), rem = piece % (kDotMaxGroups * 4u);
      const unsigned i = rem / 4u, j = rem % 4u;
      const unsigned off = (t < NT && i < count) ? t * row_bytes + (span.begin + i) * 64u + j * 16u : 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(activations, (lds_void*)(stage + d * 1024u), 16, off, 0, 0, 0);
    }
    if constexpr (!Partials) {
      const unsigned t = lane / 6u, d = lane % 6u;
      const unsigned off = t < NT ? (((t * groups + span.begin) >> 1) + d) * 4u : 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(activation_scales, (lds_void*)(stage + kDotCodeRegion<NT>), 4, off, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2) The range's weight scales, then all of its weights, in flight together.  Every
    //    load is issued (past the range or the matrix through an out-of-range offset:
    //    zeros, no traffic) so that the count of loads after the DMA is a constant.
    unsigned short wsr[kDotMaxGroups];
#pragma unroll
    for (unsigned i = 0; i < kDotMaxGroups; ++i) {
      if constexpr (!Partials) {
        wsr[i] = __builtin_amdgcn_raw_buffer_load_b16(weight_scales, i < count ? ws_voffset + i * 32u : 0x80000000u,
                                                      span.begin * 32u, 0);
      }
    }
    constexpr unsigned kChunk = 64u * LB;  // bytes of one (tile, group) chunk
    constexpr unsigned kHalf = kDotMaxGroups / 2;
    // The range's first group in one SGPR, the group within the range as the immediate
    // offset (the second half of the range has an SGPR of its own: 9 x 1024 B would
    // overflow the 12-bit immediate), the tile in the lane offset.
    const unsigned first = __builtin_amdgcn_readfirstlane(span.begin * kChunk);
    const unsigned second = __builtin_amdgcn_readfirstlane((span.begin + kHalf) * kChunk);
    unsigned w[kDotMaxGroups][4][WD];
#pragma unroll
    for (unsigned i = 0; i < kDotMaxGroups; ++i) {
      const unsigned soffset = i < kHalf ? first : second;
      const unsigned imm = (i % kHalf) * kChunk;
#pragma unroll
      for (unsigned t = 0; t < 4; ++t) {
        const unsigned voffset = (t < valid && i < count) ? t * groups * kChunk + lane * LB + imm : 0x80000000u;
        if constexpr (Format == GFXI_W3G128) {
          const u32x3 x = __builtin_amdgcn_raw_buffer_load_b96(weights, voffset, soffset, kStreaming);
          w[i][t][0] = x[0];
          w[i][t][1] = x[1];
          w[i][t][2] = x[2];
        } else {
          const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(weights, voffset, soffset, kStreaming);
          w[i][t][0] = x[0];
          w[i][t][1] = x[1];
          w[i][t][2] = x[2];
          w[i][t][3] = x[3];
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // The compiler does not order LDS reads after buffer -> LDS loads: wait until only the
    // loads issued after the DMA may still be in flight (loads complete in issue order).
    constexpr unsigned kAfter = (Partials ? 0u : kDotMaxGroups) + kDotMaxGroups * 4u;
    static_assert(kAfter <= 63, "vmcnt holds at most 63");
    __builtin_amdgcn_s_waitcnt(static_cast<int>((kAfter & 15u) | ((kAfter >> 4) << 14) | (7u << 4) | (15u << 8)));
    __builtin_amdgcn_sched_barrier(0);
    const uint16_t* stage_scales = reinterpret_cast<const uint16_t*>(stage + kDotCodeRegion<NT>);
    float v[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) v[t] = 0.0F;
#pragma unroll
    for (unsigned i = 0; i < kDotMaxGroups; ++i) {
      if (i >= count) continue;  // wave-uniform
      const unsigned g = span.begin + i;
#pragma unroll
      for (unsigned d = 0; d < WD; ++d) exchange_rows(w[i][0][d], w[i][1][d], w[i][2][d], w[i][3][d]);
      // nib[4k + j]: columns 32k + 8j .. 32k + 8j + 7 of the group, in A4 nibble order
      unsigned nib[16];
#pragma unroll
      for (unsigned k = 0; k < 4; ++k) {
        if constexpr (Format == GFXI_W3G128) {
          w3_nibbles(w[i][k][0], w[i][k][1], w[i][k][2], nib + 4 * k);
        } else {
#pragma unroll
          for (unsigned j = 0; j < 4; ++j) nib[4 * k + j] = w[i][k][j];
        }
      }
      float ws = 0.0F;
      if constexpr (!Partials) ws = __half2float(__ushort_as_half(wsr[i]));
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        // the token's 128 codes of group g: the same LDS address in every lane (broadcast)
        const u32x4* a = reinterpret_cast<const u32x4*>(stage + (t * kDotMaxGroups + i) * 64u);
        int p0 = 0, p1 = 0;
#pragma unroll
        for (unsigned j = 0; j < 4; ++j) {
          const u32x4 x = a[j];
          p0 = __builtin_amdgcn_sdot8(static_cast<int>(x[0]), static_cast<int>(nib[4 * j]), p0, false);
          p1 = __builtin_amdgcn_sdot8(static_cast<int>(x[1]), static_cast<int>(nib[4 * j + 1]), p1, false);
          p0 = __builtin_amdgcn_sdot8(static_cast<int>(x[2]), static_cast<int>(nib[4 * j + 2]), p0, false);
          p1 = __builtin_amdgcn_sdot8(static_cast<int>(x[3]), static_cast<int>(nib[4 * j + 3]), p1, false);
        }
        const int p = p0 + p1;  // exact
        if constexpr (Partials) {
          if (live) args.partials[(static_cast<std::size_t>(t) * rows + row) * groups + g] = p >> kShift;
        } else {
          const unsigned short h = stage_scales[t * 12u + (span.begin & 1u) + i];
          const float as = __half2float(__ushort_as_half(h)) * kInvF;
          v[t] = fmaf(static_cast<float>(p), ws * as, v[t]);
        }
      }
    }
    if constexpr (!Partials) {
#pragma unroll
      for (int t = 0; t < NT; ++t) total[t] = v[t];
      if (ranges > 1) {
#pragma unroll
        for (int t = 0; t < NT; ++t) dot_results[(range * NT + t) * 64u + lane] = v[t];
      }
    }
  }
  if constexpr (Partials) return;

  if (ranges > 1) {
    // The split's value: range values added in range order, by wave 0.
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < NT; ++t) total[t] = dot_results[t * 64u + lane];
    for (unsigned rg = 1; rg < ranges; ++rg) {
#pragma unroll
      for (int t = 0; t < NT; ++t) total[t] += dot_results[(rg * NT + t) * 64u + lane];
    }
  }
  if (args.argmax_keys != nullptr) {
    // Fused greedy argmax: the best of each tile's 16 rows (one lane row) per token.
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      unsigned long long best = live ? argmax_key(total[t], row, args.argmax_rows) : 0ull;
#pragma unroll
      for (int step = 0; step < 4; ++step) {
        const unsigned long long other = __shfl_xor(best, 1 << step);
        best = other > best ? other : best;
      }
      if (live && m == 0) args.argmax_keys[static_cast<std::size_t>(t) * matrix.tiles + tile0 + q] = best;
    }
  }
  if (!live || matrix.output == nullptr) return;
  const std::size_t plane = static_cast<std::size_t>(split) * batch * rows;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const std::size_t out = plane + static_cast<std::size_t>(t) * rows + row;
    if constexpr (HalfOut) {
      reinterpret_cast<__half*>(matrix.output)[out] = to_half(total[t]);
    } else {
      reinterpret_cast<float*>(matrix.output)[out] = total[t];
    }
  }
}

// ---------------------------------------------------------------------------
// Tiled row gather (lowbit_gemv.hip:191-231): out[c] = fp16(w(row,c) * ws(row,g)).
// ---------------------------------------------------------------------------

// Rows of a gather: row j is first[0] (device) or host[0] for j == 0, then rest[j - 1]
// (device) or host[j]; up to kGatherRows rows per launch, one grid row each.
constexpr unsigned kGatherRows = 32;
struct GatherRows {
  uint32_t host[kGatherRows];
  const uint32_t* first;
  const uint32_t* rest;
};

template <int Format>
__global__ __launch_bounds__(256) void row_gather_kernel(
    const uint8_t* __restrict__ weights, const __half* __restrict__ scales,
    __half* __restrict__ output, GatherRows ids, std::size_t rows, std::size_t columns) {
  const std::size_t column = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (column >= columns) return;
  const unsigned j = blockIdx.y;
  std::size_t row = ids.host[j];
  if (j == 0 && ids.first != nullptr) row = *ids.first;
  if (j != 0 && ids.rest != nullptr) row = ids.rest[j - 1];
  output += static_cast<std::size_t>(j) * columns;
  if (row >= rows) {
    output[column] = __float2half(0.0F);
    return;
  }
  const std::size_t groups = columns / kGroup;
  const uint8_t* chunk = weights + chunk_offset(Format, row, column, groups);
  const int w = unpack_lane_code(Format, chunk, static_cast<unsigned>(column % 32));
  output[column] = to_half(static_cast<float>(w) *
                                __half2float(scales[scale_offset(row, column / kGroup, groups)]));
}

// Second half of the fused argmax: the best tile key of each token row.  One
// 1024-thread workgroup per row; every thread issues all its loads (up to
// kArgmaxLoads keys, coalesced across the workgroup) before the first comparison,
// so a row of up to 16384 tiles costs one memory round trip instead of a chain.
constexpr unsigned kArgmaxThreads = 1024;
constexpr unsigned kArgmaxLoads = 16;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_keys_kernel(
    const unsigned long long* __restrict__ keys, uint32_t count, const uint32_t* __restrict__ token_ids,
    uint32_t* __restrict__ out) {
  __shared__ unsigned long long partial[kArgmaxThreads / 64];
  const unsigned long long* row = keys + static_cast<std::size_t>(blockIdx.x) * count;
  unsigned long long best = 0ull;
  for (uint32_t base = 0; base < count; base += kArgmaxThreads * kArgmaxLoads) {
    unsigned long long k[kArgmaxLoads];
#pragma unroll
    for (unsigned u = 0; u < kArgmaxLoads; ++u) {
      const uint32_t i = base + u * kArgmaxThreads + threadIdx.x;
      const unsigned long long key = row[i < count ? i : 0u];  // unconditional: no load waits on a branch
      k[u] = i < count ? key : 0ull;
    }
#pragma unroll
    for (unsigned u = 0; u < kArgmaxLoads; ++u) best = k[u] > best ? k[u] : best;
  }
  best = wave_max_key(best);
  if ((threadIdx.x & 63u) == 0) partial[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (unsigned w = 1; w < kArgmaxThreads / 64; ++w) best = partial[w] > best ? partial[w] : best;
    const uint32_t index = argmax_key_row(best);
    out[blockIdx.x] = token_ids != nullptr ? token_ids[index] : index;
  }
}

// ---------------------------------------------------------------------------
// Host launch helpers
// ---------------------------------------------------------------------------

bool aligned(const void* pointer, std::size_t bytes) {
  return (reinterpret_cast<std::uintptr_t>(pointer) % bytes) == 0;
}

constexpr unsigned kLdsBytes = 160u * 1024u;  // gfx950 LDS per CU (and per workgroup)
constexpr uint32_t kMaxSplits = 8;            // split-K planes per GEMM

// Waves per workgroup: about ten groups of K (one load chunk) per wave.
unsigned choose_waves(uint32_t groups) {
  unsigned waves = (groups + 9) / 10;
  if (waves < 1) waves = 1;
  if (waves > 16) waves = 16;
  return waves;
}

template <int Format, int ABits, bool HalfOut, bool Partials>
void launch_direct_kernel(const GemmArgs& base_args, uint32_t total_tiles, hipStream_t stream) {
  const uint32_t batch = base_args.batch;
  auto go = [&](auto kernel, unsigned r, unsigned ntb) {
    GemmArgs args = base_args;
    uint32_t blocks = 0;
    for (unsigned i = 0; i < 4; ++i) {
      args.tile_begin[i] = blocks;
      // unused trailing slots repeat the last matrix with zero tiles
      const bool used = i == 0 || base_args.tile_begin[i] != base_args.tile_begin[4];
      if (used) blocks += (args.matrix[i].tiles + r - 1) / r;
    }
    args.tile_begin[4] = blocks;
    unsigned max_ranges = 1;
    for (unsigned sp = 0; sp < args.splits; ++sp) {
      const GroupRange g = split_groups(args.groups, sp, args.splits);
      max_ranges = std::max(max_ranges, range_count(g.end - g.begin));
    }
    // range values of the canonical K partition, summed in order at the end
    const std::size_t lds = max_ranges > 1 ? static_cast<std::size_t>(max_ranges) * r * ntb * 4u * 64u * 4u : 0;
    const unsigned waves =
        std::min({choose_waves(args.groups / args.splits), min_range_count(args.groups, args.splits),
                  kDirectMaxWaves});
    hipLaunchKernelGGL(kernel, dim3(blocks * args.splits), dim3(64 * waves), lds, stream, args);
  };
  // Row tiles per wave (R) and groups per load chunk (CH), by grid shape (measured on
  // MI355X over the verifier's projections at 16 and 32 tokens, weights rotated past the
  // Infinity Cache).  More tiles share each activation load and its expansion; shorter
  // chunks need fewer registers, so more waves stay resident.  A split of one canonical
  // range (the o and GDN out projections: 8-10 groups per split) runs one wave per
  // workgroup and keeps one tile; otherwise, by row tiles x splits:
  //   >= 2048 (gate/up): 3 tiles, 2-group chunks (32 tokens 25.3 -> 21.4 us);
  //   1024..2047 (down as four splits): 3 tiles, 3-group chunks (16.0 -> 14.3 us);
  //   < 1024 (q/k/v, GDN in-projection): 2 tiles, 2-group chunks at 17-32 tokens
  //   (15.3 -> 12.2 us), 2 tiles of 5-group chunks at 9-16 tokens.
  uint64_t tile_splits = 0;
  for (unsigned i = 0; i < 4; ++i) {
    const bool used = i == 0 || base_args.tile_begin[i] != base_args.tile_begin[4];
    if (used) tile_splits += static_cast<uint64_t>(base_args.matrix[i].tiles) * base_args.splits;
  }
  const bool one_range = min_range_count(base_args.groups, base_args.splits) <= 1;
  int shape;  // 1: 1 x 4, 2: 2 x 5, 3: 3 x 2, 4: 3 x 3, 5: 2 x 2
  if (one_range) {
    shape = 1;
  } else if (tile_splits >= 2048) {
    shape = 3;
  } else if (tile_splits >= 1024) {
    shape = 4;
  } else {
    shape = batch > 16 ? 5 : 2;
  }
  (void)total_tiles;
  if (batch <= 4) {
    go(lowbit_gemm_direct_kernel<Format, ABits, 4, 1, 3, 1, HalfOut, Partials>, 1, 1);
  } else if (batch <= 8) {
    go(lowbit_gemm_direct_kernel<Format, ABits, 2, 1, 6, 1, HalfOut, Partials>, 1, 1);
  } else if (batch <= 16) {
    switch (shape) {
      case 2: go(lowbit_gemm_direct_kernel<Format, ABits, 1, 1, 5, 2, HalfOut, Partials>, 2, 1); break;
      case 3: go(lowbit_gemm_direct_kernel<Format, ABits, 1, 1, 2, 3, HalfOut, Partials>, 3, 1); break;
      case 4: go(lowbit_gemm_direct_kernel<Format, ABits, 1, 1, 3, 3, HalfOut, Partials>, 3, 1); break;
      default: go(lowbit_gemm_direct_kernel<Format, ABits, 1, 1, 4, 1, HalfOut, Partials>, 1, 1); break;
    }
  } else if constexpr (ABits == 8) {
    go(lowbit_gemm_direct_kernel<Format, ABits, 1, 2, 4, 1, HalfOut, Partials>, 1, 2);
  } else {
    switch (shape) {
      case 2: go(lowbit_gemm_direct_kernel<Format, ABits, 1, 2, 5, 2, HalfOut, Partials>, 2, 2); break;
      case 3: go(lowbit_gemm_direct_kernel<Format, ABits, 1, 2, 2, 3, HalfOut, Partials>, 3, 2); break;
      case 4: go(lowbit_gemm_direct_kernel<Format, ABits, 1, 2, 3, 3, HalfOut, Partials>, 3, 2); break;
      case 5: go(lowbit_gemm_direct_kernel<Format, ABits, 1, 2, 2, 2, HalfOut, Partials>, 2, 2); break;
      default: go(lowbit_gemm_direct_kernel<Format, ABits, 1, 2, 4, 1, HalfOut, Partials>, 1, 2); break;
    }
  }
}

// Kernel family of a GEMM launch: chosen by shape, or forced by the test/bench entry.
enum GemmFamily : int32_t { kFamilyAuto = 0, kFamilyMfma = 1, kFamilyDot = 2 };

// Whether the dot kernel can run a launch: W3/W4 x A4 at 1-8 tokens, activation scales
// read as aligned dword pairs (4-byte aligned, even group count).
bool dot_supported(int32_t format, int abits, const GemmArgs& args, bool partials) {
  return abits == 4 && (format == GFXI_W3G128 || format == GFXI_W4G128) && args.batch <= 8 &&
         (partials || (args.groups % 2 == 0 && aligned(args.activation_scales, 4)));
}

template <int Format, bool HalfOut, bool Partials>
void launch_dot_kernel(const GemmArgs& base_args, hipStream_t stream) {
  if constexpr (Format == GFXI_W3G128 || Format == GFXI_W4G128) {
    GemmArgs args = base_args;
    uint32_t blocks = 0;
    for (unsigned i = 0; i < 4; ++i) {
      args.tile_begin[i] = blocks;
      // unused trailing slots repeat the last matrix with zero tiles
      const bool used = i == 0 || base_args.tile_begin[i] != base_args.tile_begin[4];
      if (used) blocks += (args.matrix[i].tiles + 3) / 4;
    }
    args.tile_begin[4] = blocks;
    unsigned max_ranges = 1;
    for (unsigned sp = 0; sp < args.splits; ++sp) {
      const GroupRange g = split_groups(args.groups, sp, args.splits);
      max_ranges = std::max(max_ranges, range_count(g.end - g.begin));
    }
    const unsigned waves = std::min(min_range_count(args.groups, args.splits), kDotMaxWaves);
    auto go = [&](auto kernel, auto nt) {
      constexpr int NT = decltype(nt)::value;
      const std::size_t lds = static_cast<std::size_t>(waves) * kDotRegion<NT> +
                              (max_ranges > 1 ? static_cast<std::size_t>(max_ranges) * NT * 64u * 4u : 0);
      hipLaunchKernelGGL(kernel, dim3(blocks * args.splits), dim3(64 * waves), lds, stream, args);
    };
    switch (args.batch) {
      case 1: go(lowbit_gemm_dot_kernel<Format, 1, HalfOut, Partials>, std::integral_constant<int, 1>{}); break;
      case 2: go(lowbit_gemm_dot_kernel<Format, 2, HalfOut, Partials>, std::integral_constant<int, 2>{}); break;
      case 3: go(lowbit_gemm_dot_kernel<Format, 3, HalfOut, Partials>, std::integral_constant<int, 3>{}); break;
      case 4: go(lowbit_gemm_dot_kernel<Format, 4, HalfOut, Partials>, std::integral_constant<int, 4>{}); break;
      case 5: go(lowbit_gemm_dot_kernel<Format, 5, HalfOut, Partials>, std::integral_constant<int, 5>{}); break;
      case 6: go(lowbit_gemm_dot_kernel<Format, 6, HalfOut, Partials>, std::integral_constant<int, 6>{}); break;
      case 7: go(lowbit_gemm_dot_kernel<Format, 7, HalfOut, Partials>, std::integral_constant<int, 7>{}); break;
      default: go(lowbit_gemm_dot_kernel<Format, 8, HalfOut, Partials>, std::integral_constant<int, 8>{}); break;
    }
  } else {
    (void)base_args;
    (void)stream;
  }
}

template <int Format, int ABits, bool HalfOut, bool Partials>
void launch_gemm_kernel(const GemmArgs& args, uint32_t total_tiles, hipStream_t stream, int32_t family) {
  if (family == kFamilyDot) {
    launch_dot_kernel<Format, HalfOut, Partials>(args, stream);
    return;
  }
  // Direct operands pay off from 9 tokens on (one token window, quad-coalesced
  // activation loads, two row tiles per workgroup); up to 8 tokens the LDS-staged
  // kernel with its packed token windows is as fast or faster.
  if (args.batch > 8) {
    launch_direct_kernel<Format, ABits, HalfOut, Partials>(args, total_tiles, stream);
    return;
  }
  const uint32_t batch = args.batch;
  auto go = [&](auto kernel, unsigned gp, unsigned ch, unsigned ntb) {
    // One wave per range of the canonical K partition (at most the fewest ranges of
    // any split), within the register and LDS limits.
    unsigned waves = std::min(choose_waves(args.groups / args.splits), min_range_count(args.groups, args.splits));
    if ((ntb == 2 || ABits == 8) && waves > 8) waves = 8;
    // More workgroups than CUs: keep them at eight waves or fewer, each wave taking
    // consecutive ranges, so that two share a CU and the grid runs in one round (the
    // range values and their sum are the same whichever wave computes a range).
    if (waves > 8 && static_cast<uint64_t>(total_tiles) * args.splits > kComputeUnits) {
      const unsigned per_wave = (waves + 7) / 8;
      waves = (waves + per_wave - 1) / per_wave;
    }
    GemmLds layout = gemm_lds_layout(gp * ch, batch, ABits, ntb);
    unsigned max_ranges = 1;
    for (unsigned sp = 0; sp < args.splits; ++sp) {
      const GroupRange g = split_groups(args.groups, sp, args.splits);
      max_ranges = std::max(max_ranges, range_count(g.end - g.begin));
    }
    const uint32_t results = max_ranges > 1 ? max_ranges * ntb * 4u * 64u * 4u : 0u;
    // A workgroup may hold at most the CU's 160 KiB of LDS (32 tokens x 136 groups
    // would otherwise ask for 8 x 21 KiB).
    const unsigned lds_waves = (kLdsBytes - results) / layout.region;
    if (waves > lds_waves) waves = lds_waves;
    layout.results_offset = layout.region * waves;
    hipLaunchKernelGGL(kernel, dim3(total_tiles * args.splits), dim3(64 * waves),
                       layout.results_offset + results, stream, args, layout);
  };
  // CH = packs per load chunk: about ten groups of weights in flight per wave, whole
  // quads of groups per chunk.
  if (batch <= 8) {
    go(lowbit_gemm_kernel<Format, ABits, 2, 1, 5, HalfOut, Partials>, 2, 5, 1);
  } else if (batch <= 16) {
    go(lowbit_gemm_kernel<Format, ABits, 1, 1, 8, HalfOut, Partials>, 1, 8, 1);
  } else {
    go(lowbit_gemm_kernel<Format, ABits, 1, 2, 4, HalfOut, Partials>, 1, 4, 2);
  }
}

template <int ABits, bool HalfOut, bool Partials>
void dispatch_gemm(int32_t format, const GemmArgs& args, uint32_t total_tiles, hipStream_t stream,
                   int32_t family) {
  if (format == GFXI_W2G128) {
    launch_gemm_kernel<GFXI_W2G128, ABits, HalfOut, Partials>(args, total_tiles, stream, family);
  } else if (format == GFXI_W3G128) {
    launch_gemm_kernel<GFXI_W3G128, ABits, HalfOut, Partials>(args, total_tiles, stream, family);
  } else {
    launch_gemm_kernel<GFXI_W4G128, ABits, HalfOut, Partials>(args, total_tiles, stream, family);
  }
}

struct MatrixBinding {
  const uint8_t* weights;
  const uint16_t* scales;
  void* output;
  std::size_t rows;
};

// Shared validation + launch for every GEMM entry point (argument rules of
// lowbit_gemv.hip:1123-1130, :1232-1255, :1303-1310).
int32_t gemm_entry(const char* name, int32_t format, const MatrixBinding* bindings,
                   std::size_t count, int32_t activation_bits, const void* activations,
                   const uint16_t* activation_scales, int32_t* partials, std::size_t columns,
                   uint32_t batch, bool half_out, hipStream_t stream,
                   unsigned long long* argmax_keys = nullptr, uint32_t argmax_rows = 0,
                   uint32_t splits = 1, int32_t family = kFamilyAuto) {
  if (!valid_weight_format(format)) {
    return fail(GFXI_UNSUPPORTED, std::string(name) + " supports W2G128, W3G128 and W4G128");
  }
  if (count == 0 || count > 4 || activations == nullptr ||
      (partials == nullptr && activation_scales == nullptr) || columns == 0 ||
      columns % kGroup != 0 || batch == 0 || batch > 32 ||
      columns > std::numeric_limits<uint32_t>::max() / 2) {
    return fail(GFXI_INVALID_ARGUMENT, std::string(name) +
                " requires non-null buffers, N divisible by 16, K divisible by 128, and batch "
                "in [1,32]");
  }
  if (!aligned(activations, 16)) {
    return fail(GFXI_INVALID_ARGUMENT, std::string(name) + " requires 16-byte aligned activations");
  }
  if (splits == 0 || splits > kMaxSplits || splits > columns / kGroup ||
      (splits > 1 && (half_out || partials != nullptr || argmax_keys != nullptr))) {
    return fail(GFXI_INVALID_ARGUMENT, std::string(name) + " split count must be in [1, " +
                                           std::to_string(kMaxSplits) +
                                           "], at most K/128, and 1 for fp16, partial or argmax "
                                           "outputs");
  }
  GemmArgs args{};
  uint64_t tiles = 0;
  for (std::size_t i = 0; i < count; ++i) {
    const MatrixBinding& b = bindings[i];
    if (b.weights == nullptr || b.scales == nullptr ||
        (partials == nullptr && argmax_keys == nullptr && b.output == nullptr) || b.rows == 0 ||
        b.rows % 16 != 0) {
      return fail(GFXI_INVALID_ARGUMENT, std::string(name) + " matrix binding is invalid");
    }
    if (!aligned(b.weights, 16) || !aligned(b.scales, 8) ||
        (b.output != nullptr && !half_out && !aligned(b.output, 16))) {
      return fail(GFXI_INVALID_ARGUMENT, std::string(name) + " requires 16-byte aligned weights "
                                                             "and outputs, 8-byte aligned scales");
    }
    args.matrix[i] = {b.weights, reinterpret_cast<const __half*>(b.scales), b.output,
                      static_cast<uint32_t>(b.rows / 16)};
    args.tile_begin[i] = static_cast<uint32_t>(tiles);
    tiles += b.rows / 16;
  }
  if (tiles > std::numeric_limits<uint32_t>::max() / 2) {
    return fail(GFXI_INVALID_ARGUMENT, std::string(name) + " grid is too large");
  }
  for (std::size_t i = count; i < 4; ++i) {
    args.matrix[i] = args.matrix[count - 1];
    args.tile_begin[i] = static_cast<uint32_t>(tiles);
  }
  args.tile_begin[4] = static_cast<uint32_t>(tiles);
  args.activations = static_cast<const uint8_t*>(activations);
  args.activation_scales = reinterpret_cast<const __half*>(activation_scales);
  args.partials = partials;
  args.argmax_keys = argmax_keys;
  args.argmax_rows = argmax_rows;
  args.columns = static_cast<uint32_t>(columns);
  args.groups = static_cast<uint32_t>(columns / kGroup);
  args.batch = batch;
  args.splits = splits;
  if (tiles * splits > std::numeric_limits<uint32_t>::max() / 2) {
    return fail(GFXI_INVALID_ARGUMENT, std::string(name) + " grid is too large");
  }
  const auto total = static_cast<uint32_t>(tiles);
  const bool dot_ok = dot_supported(format, activation_bits, args, partials != nullptr);
  if (family == kFamilyDot && !dot_ok) {
    return fail(GFXI_UNSUPPORTED, std::string(name) +
                                      ": the dot kernel runs W3/W4 x A4 at 1-8 tokens with 4-byte "
                                      "aligned activation scales and an even group count");
  }
  if (family == kFamilyAuto) family = kFamilyMfma;
  if (partials != nullptr) {
    if (activation_bits == 4) dispatch_gemm<4, false, true>(format, args, total, stream, family);
    else dispatch_gemm<8, false, true>(format, args, total, stream, family);
  } else if (activation_bits == 4) {
    if (half_out) dispatch_gemm<4, true, false>(format, args, total, stream, family);
    else dispatch_gemm<4, false, false>(format, args, total, stream, family);
  } else {
    dispatch_gemm<8, false, false>(format, args, total, stream, family);
  }
  return launch_status((std::string(name) + " launch failed").c_str());
}

int32_t quantize_activation_entry(int bits, const uint16_t* input, void* output, uint16_t* scales,
                                  std::size_t columns, uint32_t batch, hipStream_t stream) {
  if (input == nullptr || output == nullptr || scales == nullptr || columns == 0 ||
      columns % kGroup != 0 || batch == 0 || batch > 32 ||
      columns > std::numeric_limits<uint32_t>::max()) {
    return fail(GFXI_INVALID_ARGUMENT,
                std::string(bits == 4 ? "A4" : "A8") +
                    " quantization requires non-null buffers, batch in [1,32], and K divisible by 128");
  }
  if (!aligned(input, 4) || (bits == 8 && !aligned(output, 2))) {
    return fail(GFXI_INVALID_ARGUMENT, "activation quantization requires aligned buffers");
  }
  const auto groups = static_cast<uint32_t>(columns / kGroup);
  const uint32_t total = groups * batch;
  const dim3 grid((total + 3) / 4);
  if (bits == 4) {
    hipLaunchKernelGGL(quantize_activation_kernel<4>, grid, dim3(256), 0, stream,
                       reinterpret_cast<const __half2*>(input), static_cast<uint8_t*>(output),
                       reinterpret_cast<__half*>(scales), static_cast<uint32_t>(columns), groups,
                       total);
    return launch_status("A4 activation quantization launch failed");
  }
  hipLaunchKernelGGL(quantize_activation_kernel<8>, grid, dim3(256), 0, stream,
                     reinterpret_cast<const __half2*>(input), static_cast<uint8_t*>(output),
                     reinterpret_cast<__half*>(scales), static_cast<uint32_t>(columns), groups,
                     total);
  return launch_status("A8 activation quantization launch failed");
}

int32_t row_gather_entry(int32_t format, const uint8_t* weights, const uint16_t* scales,
                         uint16_t* output, const GatherRows& ids, unsigned count, std::size_t rows,
                         std::size_t columns, hipStream_t stream) {
  if (!valid_weight_format(format)) {
    return fail(GFXI_UNSUPPORTED, "tiled row gather supports W2G128, W3G128 and W4G128");
  }
  if (weights == nullptr || scales == nullptr || output == nullptr || rows == 0 ||
      rows % 16 != 0 || columns == 0 || columns % kGroup != 0 || count == 0 || count > kGatherRows) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid tiled low-bit row gather arguments");
  }
  constexpr unsigned threads = 256;
  const dim3 grid(static_cast<unsigned>((columns + threads - 1) / threads), count);
  const auto* ws = reinterpret_cast<const __half*>(scales);
  auto* out = reinterpret_cast<__half*>(output);
  if (format == GFXI_W2G128) {
    hipLaunchKernelGGL(row_gather_kernel<GFXI_W2G128>, grid, dim3(threads), 0, stream, weights, ws,
                       out, ids, rows, columns);
  } else if (format == GFXI_W3G128) {
    hipLaunchKernelGGL(row_gather_kernel<GFXI_W3G128>, grid, dim3(threads), 0, stream, weights, ws,
                       out, ids, rows, columns);
  } else {
    hipLaunchKernelGGL(row_gather_kernel<GFXI_W4G128>, grid, dim3(threads), 0, stream, weights, ws,
                       out, ids, rows, columns);
  }
  return launch_status("tiled low-bit row gather launch failed");
}

}  // namespace
}  // namespace gfx950

using namespace gfx950;

extern "C" int32_t gfxinfer_launch_quantize_group128_gfx950(int32_t format, const float* weights,
                                                            size_t rows, size_t columns,
                                                            uint8_t* tiled_codes,
                                                            uint16_t* tiled_scales_f16,
                                                            int32_t* non_finite_flag,
                                                            void* stream) {
  if (!valid_weight_format(format)) {
    return fail(GFXI_UNSUPPORTED, "device quantizer supports W2G128, W3G128 and W4G128");
  }
  if (weights == nullptr || tiled_codes == nullptr || tiled_scales_f16 == nullptr || rows == 0 ||
      rows % 16 != 0 || columns == 0 || columns % kGroup != 0) {
    return fail(GFXI_INVALID_ARGUMENT, "group-128 quantization requires nonzero dimensions, N "
                                       "divisible by 16, and K divisible by 128");
  }
  const std::size_t groups = columns / kGroup;
  const std::size_t total = rows * groups;
  if (total / 256 + 1 > std::numeric_limits<uint32_t>::max()) {
    return fail(GFXI_INVALID_ARGUMENT, "device quantizer grid is too large");
  }
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  auto s = static_cast<hipStream_t>(stream);
  auto* scales = reinterpret_cast<__half*>(tiled_scales_f16);
  if (format == GFXI_W2G128) {
    hipLaunchKernelGGL(quantize_group128_kernel<GFXI_W2G128>, grid, dim3(256), 0, s, weights, rows,
                       columns, groups, tiled_codes, scales, non_finite_flag);
  } else if (format == GFXI_W3G128) {
    hipLaunchKernelGGL(quantize_group128_kernel<GFXI_W3G128>, grid, dim3(256), 0, s, weights, rows,
                       columns, groups, tiled_codes, scales, non_finite_flag);
  } else {
    hipLaunchKernelGGL(quantize_group128_kernel<GFXI_W4G128>, grid, dim3(256), 0, s, weights, rows,
                       columns, groups, tiled_codes, scales, non_finite_flag);
  }
  return launch_status("device weight quantizer launch failed");
}

extern "C" int32_t gfxinfer_launch_quantize_activation_i4(const uint16_t* input,
                                                          uint8_t* packed_output, uint16_t* scales,
                                                          size_t columns, uint32_t batch,
                                                          void* stream) {
  return quantize_activation_entry(4, input, packed_output, scales, columns, batch,
                                   static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_quantize_activation_i8(const uint16_t* input,
                                                          int8_t* quantized_output,
                                                          uint16_t* scales, size_t columns,
                                                          uint32_t batch, void* stream) {
  return quantize_activation_entry(8, input, quantized_output, scales, columns, batch,
                                   static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_gfx950_i4_gemm(int32_t format, const uint8_t* tiled_weights,
                                                  const uint16_t* tiled_weight_scales,
                                                  const uint8_t* packed_activations,
                                                  const uint16_t* activation_scales, float* output,
                                                  size_t rows, size_t columns, uint32_t batch,
                                                  int32_t sequential_w3, void* stream) {
  (void)sequential_w3;
  const MatrixBinding binding{tiled_weights, tiled_weight_scales, output, rows};
  return gemm_entry("gfx950 INT4 GEMM", format, &binding, 1, 4, packed_activations,
                    activation_scales, nullptr, columns, batch, false,
                    static_cast<hipStream_t>(stream));
}

extern "C" uint32_t gfxinfer_gemm_split_count(size_t rows, size_t columns, uint32_t batch) {
  // Enough row-tile x split workgroups to fill the chip about four times over (a grid
  // below that leaves CUs idle or runs a partial second round), each split keeping at
  // least eight groups of K.  The count depends on the shape only, never on the batch:
  // the split is part of the summation order, so a block of tokens and one-token
  // steps must use the same one.  1024 workgroups: four planes for the 320-tile
  // projections, the best of 1-5 planes in 27B verify rounds.
  constexpr uint64_t target = 1024;
  (void)batch;
  if (rows == 0 || columns < kGroup) return 1;
  const uint64_t tiles = (rows + 15) / 16;
  uint64_t splits = (target + tiles - 1) / tiles;
  splits = std::min<uint64_t>(splits, kMaxSplits);
  splits = std::min<uint64_t>(splits, columns / kGroup / 8);
  return static_cast<uint32_t>(std::max<uint64_t>(splits, 1));
}

extern "C" int32_t gfxinfer_launch_gfx950_i4_gemm_split(int32_t format, const uint8_t* tiled_weights,
                                                        const uint16_t* tiled_weight_scales,
                                                        const uint8_t* packed_activations,
                                                        const uint16_t* activation_scales,
                                                        float* output_planes, size_t rows,
                                                        size_t columns, uint32_t batch,
                                                        uint32_t splits, void* stream) {
  const MatrixBinding binding{tiled_weights, tiled_weight_scales, output_planes, rows};
  return gemm_entry("gfx950 split-K INT4 GEMM", format, &binding, 1, 4, packed_activations,
                    activation_scales, nullptr, columns, batch, false,
                    static_cast<hipStream_t>(stream), nullptr, 0, splits);
}

extern "C" int32_t gfxinfer_launch_gfx950_i4_gemm_half(int32_t format, const uint8_t* tiled_weights,
                                                       const uint16_t* tiled_weight_scales,
                                                       const uint8_t* packed_activations,
                                                       const uint16_t* activation_scales,
                                                       uint16_t* output, size_t rows,
                                                       size_t columns, uint32_t batch,
                                                       int32_t sequential_w3, void* stream) {
  (void)sequential_w3;
  const MatrixBinding binding{tiled_weights, tiled_weight_scales, output, rows};
  return gemm_entry("gfx950 INT4 GEMM FP16 epilogue", format, &binding, 1, 4, packed_activations,
                    activation_scales, nullptr, columns, batch, true,
                    static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_gfx950_i4_gemm_fused(int32_t format,
                                                        const gfxinfer_fused_matrix* matrices,
                                                        size_t matrix_count,
                                                        const uint8_t* packed_activations,
                                                        const uint16_t* activation_scales,
                                                        size_t columns, uint32_t batch,
                                                        int32_t sequential_w3, void* stream) {
  (void)sequential_w3;
  if (matrices == nullptr || matrix_count < 2 || matrix_count > 4) {
    return fail(GFXI_INVALID_ARGUMENT,
                "gfx950 fused INT4 GEMM requires 2..4 matrices and batch in [1,32]");
  }
  MatrixBinding bindings[4];
  for (std::size_t i = 0; i < matrix_count; ++i) {
    bindings[i] = {matrices[i].tiled_weights, matrices[i].tiled_weight_scales, matrices[i].output,
                   matrices[i].rows};
  }
  return gemm_entry("gfx950 fused INT4 GEMM", format, bindings, matrix_count, 4,
                    packed_activations, activation_scales, nullptr, columns, batch, false,
                    static_cast<hipStream_t>(stream));
}

extern "C" size_t gfxinfer_gemm_argmax_workspace_bytes(size_t rows, uint32_t batch) {
  return ((rows + 15) / 16) * static_cast<std::size_t>(batch) * sizeof(unsigned long long);
}

extern "C" int32_t gfxinfer_launch_gfx950_i4_gemm_argmax(
    int32_t format, const uint8_t* tiled_weights, const uint16_t* tiled_weight_scales,
    const uint8_t* packed_activations, const uint16_t* activation_scales, float* logits,
    size_t rows, size_t columns, uint32_t batch, size_t argmax_rows, const uint32_t* token_ids,
    void* workspace, size_t workspace_bytes, uint32_t* tokens, void* stream) {
  if (workspace == nullptr || argmax_rows == 0 || argmax_rows > rows || rows > 0xffffffffu ||
      workspace_bytes < gfxinfer_gemm_argmax_workspace_bytes(rows, batch) || !aligned(workspace, 8)) {
    return fail(GFXI_INVALID_ARGUMENT, "fused GEMM argmax needs 1 <= argmax rows <= rows and an "
                                       "8-byte aligned workspace of gfxinfer_gemm_argmax_workspace_bytes() "
                                       "bytes");
  }
  const MatrixBinding binding{tiled_weights, tiled_weight_scales, logits, rows};
  auto* keys = static_cast<unsigned long long*>(workspace);
  auto s = static_cast<hipStream_t>(stream);
  const int32_t status = gemm_entry("fused GEMM argmax", format, &binding, 1, 4, packed_activations,
                                    activation_scales, nullptr, columns, batch, false, s, keys,
                                    static_cast<uint32_t>(argmax_rows));
  if (status != GFXI_OK || tokens == nullptr) return status;  // no tokens: the keys are the output
  hipLaunchKernelGGL(argmax_keys_kernel, dim3(batch), dim3(kArgmaxThreads), 0, s, keys,
                     static_cast<uint32_t>(rows / 16), token_ids, tokens);
  return launch_status("fused GEMM argmax reduction launch failed");
}

// ---------------------------------------------------------------------------
// Allocation-free fused head.  The per-(token, tile) argmax keys of
// gfxinfer_launch_gfx950_i4_gemm_argmax live in this file-scope device array instead of
// a caller workspace: 4 MiB, i.e. batch * ceil(rows / 16) <= 524288 keys (every LM head
// up to 262144 rows at 32 tokens).  Each GPU holds its own copy until the process ends;
// host code reaches it only through the address hipGetSymbolAddress returns on that
// device (the array's name is a host-side stand-in, not a device address).  Every key
// the reduction reads is written by the GEMM of the same call, so nothing needs to be
// cleared between calls; calls that overlap on one GPU (concurrent streams) race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned long long scratch[1u << 19];
namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_address[kScratchDevices] = {};

// The calling thread's current device's copy of `scratch`, looked up on the first call
// on that device (with it current) and kept.
int32_t scratch_address(void** out) {
  int device = 0;
  if (auto e = hipGetDevice(&device); e != hipSuccess) return hip_fail(e, "hipGetDevice failed");
  if (device < 0 || device >= kScratchDevices) {
    return fail(GFXI_UNSUPPORTED, "device index beyond the allocation-free entry's table");
  }
  const std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (g_scratch_address[device] == nullptr) {
    void* address = nullptr;
    if (auto e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)); e != hipSuccess) {
      return hip_fail(e, "address of the argmax key scratch array");
    }
    g_scratch_address[device] = address;
  }
  *out = g_scratch_address[device];
  return ok();
}

}  // namespace

extern "C" int32_t gfxinfer_launch_gfx950_i4_gemm_argmax_no_alloc(
    int32_t format, const uint8_t* tiled_weights, const uint16_t* tiled_weight_scales,
    const uint8_t* packed_activations, const uint16_t* activation_scales, float* logits,
    size_t rows, size_t columns, uint32_t batch, size_t argmax_rows, const uint32_t* token_ids,
    uint32_t* tokens, void* stream) {
  if (gfxinfer_gemm_argmax_workspace_bytes(rows, batch) > sizeof(scratch)) {
    return fail(GFXI_INVALID_ARGUMENT, "allocation-free fused GEMM argmax holds at most 524288 keys "
                                       "(batch * ceil(rows / 16)); use the workspace entry point");
  }
  void* keys = nullptr;
  if (const int32_t status = scratch_address(&keys); status != GFXI_OK) return status;
  return gfxinfer_launch_gfx950_i4_gemm_argmax(format, tiled_weights, tiled_weight_scales,
                                               packed_activations, activation_scales, logits, rows,
                                               columns, batch, argmax_rows, token_ids, keys,
                                               sizeof(scratch), tokens, stream);
}

extern "C" int32_t gfxinfer_launch_gfx950_i8_gemm(int32_t format, const uint8_t* tiled_weights,
                                                  const uint16_t* tiled_weight_scales,
                                                  const int8_t* quantized_activations,
                                                  const uint16_t* activation_scales, float* output,
                                                  size_t rows, size_t columns, uint32_t batch,
                                                  void* stream) {
  const MatrixBinding binding{tiled_weights, tiled_weight_scales, output, rows};
  return gemm_entry("gfx950 INT8 GEMM", format, &binding, 1, 8, quantized_activations,
                    activation_scales, nullptr, columns, batch, false,
                    static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_debug_gemm_partials(int32_t format, const uint8_t* tiled_weights,
                                                int32_t activation_bits, const void* activations,
                                                size_t rows, size_t columns, uint32_t batch,
                                                int32_t* partials, void* stream) {
  if (activation_bits != 4 && activation_bits != 8) {
    return fail(GFXI_INVALID_ARGUMENT, "activation_bits must be 4 or 8");
  }
  if (partials == nullptr) return fail(GFXI_INVALID_ARGUMENT, "partials buffer is null");
  // Scales are not read on this path; any non-null 8-byte aligned pointer will do.
  const MatrixBinding binding{tiled_weights, reinterpret_cast<const uint16_t*>(tiled_weights),
                              nullptr, rows};
  return gemm_entry("gfx950 GEMM partials", format, &binding, 1, activation_bits, activations,
                    nullptr, partials, columns, batch, false, static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_debug_gemm_family(int32_t family, int32_t format, const uint8_t* tiled_weights,
                                              const uint16_t* tiled_weight_scales,
                                              const uint8_t* packed_activations,
                                              const uint16_t* activation_scales, void* output,
                                              int32_t half_output, int32_t* partials,
                                              unsigned long long* argmax_keys, uint32_t argmax_rows,
                                              size_t rows, size_t columns, uint32_t batch,
                                              uint32_t splits, void* stream) {
  if (family != kFamilyMfma && family != kFamilyDot) {
    return fail(GFXI_INVALID_ARGUMENT, "kernel family must be 1 (MFMA) or 2 (dot)");
  }
  const uint16_t* scales =
      partials != nullptr ? reinterpret_cast<const uint16_t*>(tiled_weights) : tiled_weight_scales;
  const MatrixBinding binding{tiled_weights, scales, output, rows};
  return gemm_entry("gfx950 GEMM (kernel family)", format, &binding, 1, 4, packed_activations,
                    partials != nullptr ? nullptr : activation_scales, partials, columns, batch,
                    half_output != 0, static_cast<hipStream_t>(stream), argmax_keys, argmax_rows, splits,
                    family);
}

extern "C" int32_t gfxinfer_launch_lowbit_row_gather_tiled(int32_t format,
                                                           const uint8_t* tiled_weights,
                                                           const uint16_t* tiled_scales,
                                                           uint16_t* output, size_t row,
                                                           size_t rows, size_t columns,
                                                           void* stream) {
  if (row >= rows) return fail(GFXI_INVALID_ARGUMENT, "invalid tiled low-bit row gather arguments");
  GatherRows ids{};
  ids.host[0] = static_cast<uint32_t>(row);
  return row_gather_entry(format, tiled_weights, tiled_scales, output, ids, 1, rows, columns,
                          static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_lowbit_row_gather_tiled_indirect(
    int32_t format, const uint8_t* tiled_weights, const uint16_t* tiled_scales, uint16_t* output,
    const uint32_t* row, size_t rows, size_t columns, void* stream) {
  if (row == nullptr) return fail(GFXI_INVALID_ARGUMENT, "indirect row pointer is null");
  GatherRows ids{};
  ids.first = row;
  return row_gather_entry(format, tiled_weights, tiled_scales, output, ids, 1, rows, columns,
                          static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_lowbit_row_gather_tiled_batch(
    int32_t format, const uint8_t* tiled_weights, const uint16_t* tiled_scales, uint16_t* output,
    const uint32_t* host_rows, const uint32_t* first_row, const uint32_t* rest_rows, uint32_t count,
    size_t rows, size_t columns, void* stream) {
  if (count == 0 || count > kGatherRows) {
    return fail(GFXI_INVALID_ARGUMENT, "a batched row gather takes 1..32 rows");
  }
  if (host_rows == nullptr && (first_row == nullptr || (count > 1 && rest_rows == nullptr))) {
    return fail(GFXI_INVALID_ARGUMENT, "rows without a host or device source");
  }
  GatherRows ids{};
  if (host_rows != nullptr) {
    for (uint32_t j = 0; j < count; ++j) ids.host[j] = host_rows[j];
  }
  ids.first = first_row;
  ids.rest = rest_rows;
  return row_gather_entry(format, tiled_weights, tiled_scales, output, ids, count, rows, columns,
                          static_cast<hipStream_t>(stream));
}

// HBM read floor: a plain streaming read of `bytes` (16-byte loads, grid-stride, two
// loads in flight per lane), the yardstick for what one launch of a weight-streaming
// kernel can reach at a given size on this device.  Each lane folds what it read into
// an XOR; the one store is taken only when the fold equals a fixed odd constant, so
// the reads stay live and the sink is written (by whichever lanes hit it) at most once.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ data,
                                                          size_t count, uint32_t* sink) {
  const size_t lane = static_cast<size_t>(blockIdx.x) * 256u + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * 256u;
  uint32_t fold = 0;
  size_t i = lane;
  for (; i + stride < count; i += 2 * stride) {
    const uint4 a = data[i];
    const uint4 b = data[i + stride];
    fold ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
  }
  if (i < count) {
    const uint4 a = data[i];
    fold ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (fold == 0x9E3779B9u) sink[lane] = fold;
}

// The same read with no loop: lane l of workgroup b issues all of its U 16-byte loads
// at once (pieces b * 256 U + u * 256 + l, u < U, non-temporal as the GEMMs' weight
// loads), so every byte of the launch is requested in the first instructions of its
// waves.  Lanes past the end read the last piece again.
template <int U>
__global__ __launch_bounds__(256) void stream_read_oneshot_kernel(const uint4* __restrict__ data, size_t count,
                                                                  uint32_t* sink) {
  const size_t base = static_cast<size_t>(blockIdx.x) * 256u * U + threadIdx.x;
  u32x4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const size_t i = min(base + static_cast<size_t>(u) * 256u, count - 1u);
    v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(data) + i);
  }
  uint32_t fold = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) fold ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  if (fold == 0x9E3779B9u) sink[min(base, count - 1u)] = fold;
}

extern "C" int32_t gfxinfer_debug_stream_read_oneshot(const void* data, size_t bytes, uint32_t* sink,
                                                      uint32_t loads_per_lane, void* stream) {
  if (data == nullptr || sink == nullptr) return fail(GFXI_INVALID_ARGUMENT, "null buffer");
  if (bytes == 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(data) % 16 != 0) {
    return fail(GFXI_INVALID_ARGUMENT, "stream read needs a 16-byte aligned, nonzero multiple of 16 bytes");
  }
  const size_t count = bytes / 16;
  const size_t per_workgroup = static_cast<size_t>(256) * loads_per_lane;
  if (loads_per_lane == 0 || (count + per_workgroup - 1) / per_workgroup > (1u << 24)) {
    return fail(GFXI_INVALID_ARGUMENT, "loads_per_lane must be 1, 2, 4 or 8 and the grid at most 2^24 workgroups");
  }
  const dim3 grid(static_cast<unsigned>((count + per_workgroup - 1) / per_workgroup));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* d = static_cast<const uint4*>(data);
  switch (loads_per_lane) {
    case 1: hipLaunchKernelGGL(stream_read_oneshot_kernel<1>, grid, dim3(256), 0, s, d, count, sink); break;
    case 2: hipLaunchKernelGGL(stream_read_oneshot_kernel<2>, grid, dim3(256), 0, s, d, count, sink); break;
    case 4: hipLaunchKernelGGL(stream_read_oneshot_kernel<4>, grid, dim3(256), 0, s, d, count, sink); break;
    case 8: hipLaunchKernelGGL(stream_read_oneshot_kernel<8>, grid, dim3(256), 0, s, d, count, sink); break;
    default:
      return fail(GFXI_INVALID_ARGUMENT, "loads_per_lane must be 1, 2, 4 or 8 and the grid at most 2^24 workgroups");
  }
  return launch_status("one-shot stream read");
}

extern "C" int32_t gfxinfer_debug_stream_read(const void* data, size_t bytes, uint32_t* sink,
                                              uint32_t workgroups, void* stream) {
  if (data == nullptr || sink == nullptr) return fail(GFXI_INVALID_ARGUMENT, "null buffer");
  if (bytes == 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(data) % 16 != 0) {
    return fail(GFXI_INVALID_ARGUMENT, "stream read needs a 16-byte aligned, nonzero multiple of 16 bytes");
  }
  if (workgroups == 0 || workgroups > 65536) {
    return fail(GFXI_INVALID_ARGUMENT, "workgroups must be in [1, 65536]");
  }
  hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4*>(data), bytes / 16,
                     sink);
  return launch_status("stream read");
}
