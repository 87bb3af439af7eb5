// Causal gated GQA decode attention over a verify block (k+1 <= 32 query tokens)
// for gfx950: split-context flash decoding on v_mfma_f32_16x16x32_f16.
//
// Reference semantics: gated_attention_decode (src/kernels/qwen_ops.hip:698-766):
// token t of the block attends to the first base + t cached positions, scores
// are q.k / sqrt(head_size), softmax over positions, output = softmax(s).V *
// sigmoid(gate) rounded to fp16, the gate being the second half of each head's
// 2*head_size query-projection row.  The reference runs one 256-thread block per
// (head, token) that walks the whole context; here one workgroup per (KV head,
// split of positions) stages K and V^T in LDS once and serves all
// (q_heads/kv_heads) x tokens query rows of that KV head with MFMA, writing a
// split-local (max, sum, unnormalized output); a combine kernel merges splits.
// Head sizes 128 (64-position splits) and 256 (the reference model's 24/4 x 256,
// 32-position splits so that K, V^T and the P tiles stay within 64 KB of LDS).
#include <cmath>
#include <limits>
#include <string>

#include "common.hpp"

namespace gfx950 {
namespace {

using h8 = _Float16 __attribute__((ext_vector_type(8)));
using f4 = float __attribute__((ext_vector_type(4)));
using u32x4 = unsigned __attribute__((ext_vector_type(4)));

constexpr unsigned kPad = 8;  // LDS row padding (halves; rows stay 16-byte aligned)

// Positions per workgroup for a head size.
template <unsigned D>
constexpr unsigned split_positions() {
  static_assert(D == 128 || D == 256, "head size 128 or 256");
  return D == 128 ? 64 : 32;
}

std::size_t split_count(uint32_t head_size, std::size_t capacity) {
  const std::size_t split = head_size == 128 ? split_positions<128>() : split_positions<256>();
  return (capacity + split - 1) / split;
}

struct AttnArgs {
  const __half* query;        // [T][Hq][D]
  const __half* key_cache;    // [capacity][Hkv][D]
  const __half* value_cache;  // [capacity][Hkv][D]
  float* partial_o;           // [T*Hq][splits][D]
  float* partial_ml;          // [T*Hq][splits][2]  (max, sum)
  uint64_t base_count;        // positions visible to token 0
  const uint64_t* indirect_position;  // if set: base_count = *p + 1
  uint32_t tokens, q_heads, kv_heads, splits, capacity;
  float scale;
  // Fused Q/K RMSNorm + RoPE + K/V append (attention_split_kernel<D, W, true>): fp32
  // inputs as qk_norm_rope_kernel takes them (q_in [T][Hq][q_stride], k_in
  // [T][Hkv][k_stride], v_in [T][Hkv][D]); token t sits at position base_count - 1 + t.
  const float* q_in;
  const uint16_t* q_weight;
  const float* k_in;
  const uint16_t* k_weight;
  const float* v_in;
  __half* key_cache_out;    // == key_cache
  __half* value_cache_out;  // == value_cache
  uint32_t q_stride, k_stride, rotary;
  float theta;
  // Optional (cos, sin) of every position and rotary frequency ([capacity][rotary / 2]
  // float2, gfxinfer_launch_rope_table's values): read instead of evaluated.
  const float2* rope_table;
};

// Query rows (q_heads / kv_heads x tokens) a fused-RoPE attention workgroup normalizes,
// rotates and keeps in LDS (the LDS of the four-wave kernel stays within 64 KB).
constexpr unsigned fused_rope_rows(unsigned head_size) { return head_size == 128 ? 32u : 30u; }
// ... and at most two tokens per wave and eight query heads per KV head (the input rows
// are held in registers).  A wave's tokens cost their cos / sin (evaluated, or read from
// a table) and their query rows on the path to the first MFMA.
constexpr unsigned kRopeTokensPerWave = 2;
constexpr unsigned kRopeMaxGroup = 8;
bool fused_rope_supported(uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t head_size) {
  if ((head_size != 128 && head_size != 256) || kv_heads == 0 || q_heads % kv_heads != 0) return false;
  const uint32_t group = q_heads / kv_heads;
  return batch >= 1 && batch <= 4 * kRopeTokensPerWave && group <= kRopeMaxGroup &&
         group * batch <= fused_rope_rows(head_size);
}

__device__ __forceinline__ uint64_t base_count_of(const AttnArgs& a) {
  return a.indirect_position != nullptr ? *a.indirect_position + 1u : a.base_count;
}

// Waves = 4 or 8 per workgroup: each wave takes every Waves-th 16-row tile of the
// (token, q head) rows of its KV head; eight waves for blocks of more than four tiles.
//
// Rope = true (four waves, at most fused_rope_rows(kD) query rows): the workgroup also does
// what qk_norm_rope_kernel with the K/V append does for its KV head, with the same
// arithmetic: it normalizes and rotates its query rows into LDS (cos / sin once per
// token), and the workgroup whose split holds a new position writes that position's
// normalized, rotated K row and fp16 V row to the caches and to its own K / V^T tiles
// (the staging skips new positions, whose cache rows are not written yet).
template <unsigned kD, unsigned Waves, bool Rope = false>
__global__ __launch_bounds__(Waves * 64) void attention_split_kernel(AttnArgs a) {
  static_assert(!Rope || Waves == 4, "fused RoPE runs on the four-wave kernel");
  constexpr unsigned kSplit = split_positions<kD>();
  constexpr unsigned kTiles = kSplit / 16;  // score tiles of 16 positions
  constexpr unsigned kSteps = kSplit / 32;  // P.V K-steps of 32 positions
  constexpr unsigned kRow = kSplit + kPad;
  constexpr unsigned kQ = kD / 32;          // Q.K^T K-steps of 32 head dims
  __shared__ __align__(16) _Float16 ks[kSplit][kD + kPad];  // K rows of the split
  __shared__ __align__(16) _Float16 vt[kD][kRow];           // V transposed: [d][position]
  // Per-wave P tile as an fp16 pair p = hi + lo (hi = fp16(p), lo = fp16(p - hi)): two
  // f16 MFMAs then carry ~22 significant bits of p, close to the reference's fp32 P.V.
  __shared__ __align__(16) _Float16 ps[Waves][16][kRow];
  __shared__ __align__(16) _Float16 ps_lo[Waves][16][kRow];
  __shared__ __align__(16) _Float16 qs[Rope ? fused_rope_rows(kD) : 1][kD + kPad];  // rotated Q rows

  // Workgroups in split-major order (KV head fastest): the splits that hold visible
  // positions come first in dispatch order, ahead of the ones that exit at once.
  const unsigned split = blockIdx.x / a.kv_heads, hk = blockIdx.x - split * a.kv_heads;
  const uint64_t base = base_count_of(a);
  const uint64_t max_count = base + a.tokens - 1;  // visible positions of the last token
  const uint64_t p0 = static_cast<uint64_t>(split) * kSplit;
  if (p0 >= max_count) return;  // uniform: nothing visible in this split
  const unsigned tid = threadIdx.x, lane = tid & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const unsigned group = a.q_heads / a.kv_heads;
  const unsigned rows = group * a.tokens;

  const unsigned m = lane & 15u, kb = lane >> 4;
  const unsigned row_tiles = (rows + 15) / 16;
  // The Q operand of row tile rt (row = t * group + g -> head hk*group + g of token t),
  // zeros past the last row.
  auto load_q = [&](unsigned rt, h8 (&q)[kQ]) __attribute__((always_inline)) {
    const unsigned qrow = rt * 16 + m;
    if constexpr (Rope) {
#pragma unroll
      for (unsigned s = 0; s < kQ; ++s) {
        q[s] = rt < row_tiles && qrow < rows ? *reinterpret_cast<const h8*>(&qs[qrow][32 * s + 8 * kb]) : h8{};
      }
      return;
    }
    if (rt < row_tiles && qrow < rows) {
      const unsigned t = qrow / group, g = qrow - t * group;
      const __half* src = a.query + (static_cast<std::size_t>(t) * a.q_heads + hk * group + g) * kD + 8 * kb;
#pragma unroll
      for (unsigned s = 0; s < kQ; ++s) q[s] = *reinterpret_cast<const h8*>(src + 32 * s);
    } else {
#pragma unroll
      for (unsigned s = 0; s < kQ; ++s) q[s] = h8{};
    }
  };

  // Stage K [pos][d] and V^T [d][pos] for the split's positions (zeros past the
  // last visible position or the cache capacity).  Every K/V load of the split and the
  // wave's first Q tile are issued before the first LDS write (one memory latency).
  constexpr unsigned kThreads = Waves * 64;
  constexpr unsigned kStage = kSplit * (kD / 8) / kThreads;  // 16-byte K and V loads per thread
  const uint64_t limit = max_count < a.capacity ? max_count : a.capacity;
  // Positions past the limit load position p0 (always valid: p0 < limit) and are
  // zeroed when written, so no load waits on a branch.
  // K rows: thread i holds dims 8 (i % (D/8)) .. + 7 of position i / (D/8).  V: thread i
  // holds eight dims (chunk i / (split/2)) of positions 2 (i % (split/2)) and the one after,
  // so that it writes V^T as position pairs, one dword per dim (at head size 128 the 64
  // lanes of a wave land on 64 different LDS banks).
  constexpr unsigned kVItems = (kSplit / 2) * (kD / 8) / kThreads;
  static_assert(kStage >= 1 && kVItems >= 1 && kSplit * (kD / 8) % kThreads == 0 &&
                (kSplit / 2) * (kD / 8) % kThreads == 0, "staging covers the split exactly");
  u32x4 kr[kStage], va[kVItems], vb[kVItems];
#pragma unroll
  for (unsigned u = 0; u < kStage; ++u) {
    const unsigned i = tid + u * kThreads;
    const unsigned p = i / (kD / 8), d8 = (i % (kD / 8)) * 8;
    const uint64_t pos = p0 + p < limit ? p0 + p : p0;
    kr[u] = *reinterpret_cast<const u32x4*>(a.key_cache + (pos * a.kv_heads + hk) * kD + d8);
  }
#pragma unroll
  for (unsigned u = 0; u < kVItems; ++u) {
    const unsigned i = tid + u * kThreads;
    const unsigned pair = i % (kSplit / 2), d8 = (i / (kSplit / 2)) * 8;
    const uint64_t pa = p0 + 2 * pair < limit ? p0 + 2 * pair : p0;
    const uint64_t pb = p0 + 2 * pair + 1 < limit ? p0 + 2 * pair + 1 : p0;
    va[u] = *reinterpret_cast<const u32x4*>(a.value_cache + (pa * a.kv_heads + hk) * kD + d8);
    vb[u] = *reinterpret_cast<const u32x4*>(a.value_cache + (pb * a.kv_heads + hk) * kD + d8);
  }
  h8 q_next[kQ];
  if constexpr (!Rope) load_q(wave, q_next);
  // Positions from `fresh` on are the block's own tokens: with Rope their cache rows are
  // written by this launch, so the staging below leaves them to the RoPE step.
  const uint64_t fresh = Rope ? base - 1 : ~uint64_t{0};
  if constexpr (Rope) {
    // Wave w takes tokens w and w + 4 (at most eight tokens, at most eight query heads per
    // KV head): every input row is loaded up front (one memory latency, behind the K/V
    // tile loads), then cos / sin once per token, its query rows and, when the token's
    // position falls in this split, its K / V rows.
    constexpr unsigned J = kD / 64;
    float qx[kRopeTokensPerWave][kRopeMaxGroup][J], kx[kRopeTokensPerWave][J], vx[kRopeTokensPerWave][J];
    float2 cs[kRopeTokensPerWave];
    uint16_t qw[J], kw[J];
#pragma unroll
    for (unsigned j = 0; j < J; ++j) {
      qw[j] = a.q_weight[lane + 64 * j];
      kw[j] = a.k_weight[lane + 64 * j];
    }
#pragma unroll
    for (unsigned i = 0; i < kRopeTokensPerWave; ++i) {
      const unsigned t = wave + Waves * i;
      if (t >= a.tokens) break;  // wave-uniform
#pragma unroll
      for (unsigned g = 0; g < kRopeMaxGroup; ++g) {
        if (g >= group) break;  // workgroup-uniform
        const float* in = a.q_in + (static_cast<std::size_t>(t) * a.q_heads + hk * group + g) * a.q_stride;
#pragma unroll
        for (unsigned j = 0; j < J; ++j) qx[i][g][j] = in[lane + 64 * j];
      }
      const uint64_t position = fresh + t;
      cs[i] = float2{1.0F, 0.0F};
      if (a.rope_table != nullptr && lane < a.rotary) {
        cs[i] = a.rope_table[position * (a.rotary / 2) + lane % (a.rotary / 2)];
      }
      if (position >= p0 && position < p0 + kSplit) {  // wave-uniform
        const std::size_t src = static_cast<std::size_t>(t) * a.kv_heads + hk;
#pragma unroll
        for (unsigned j = 0; j < J; ++j) {
          kx[i][j] = a.k_in[src * a.k_stride + lane + 64 * j];
          vx[i][j] = a.v_in[src * kD + lane + 64 * j];
        }
      }
    }
#pragma unroll
    for (unsigned i = 0; i < kRopeTokensPerWave; ++i) {
      const unsigned t = wave + Waves * i;
      if (t >= a.tokens) break;
      const uint64_t position = fresh + t;
      float c = cs[i].x, sn = cs[i].y;
      if (a.rope_table == nullptr && lane < a.rotary) {
        rope_cos_sin(static_cast<float>(position), a.rotary, a.theta, lane, c, sn);
      }
#pragma unroll
      for (unsigned g = 0; g < kRopeMaxGroup; ++g) {
        if (g >= group) break;
        __half h[J];
        norm_rope_row<kD>(qx[i][g], qw, a.rotary, c, sn, lane, h);
#pragma unroll
        for (unsigned j = 0; j < J; ++j) {
          *reinterpret_cast<unsigned short*>(&qs[t * group + g][lane + 64 * j]) = __half_as_ushort(h[j]);
        }
      }
      if (position >= p0 && position < p0 + kSplit) {
        __half h[J];
        norm_rope_row<kD>(kx[i], kw, a.rotary, c, sn, lane, h);
        const std::size_t row = (position * a.kv_heads + hk) * kD;
        const unsigned local = static_cast<unsigned>(position - p0);
#pragma unroll
        for (unsigned j = 0; j < J; ++j) {
          const __half vh = to_half(vx[i][j]);
          a.key_cache_out[row + lane + 64 * j] = h[j];
          a.value_cache_out[row + lane + 64 * j] = vh;
          *reinterpret_cast<unsigned short*>(&ks[local][lane + 64 * j]) = __half_as_ushort(h[j]);
          *reinterpret_cast<unsigned short*>(&vt[lane + 64 * j][local]) = __half_as_ushort(vh);
        }
      }
    }
  }
#pragma unroll
  for (unsigned u = 0; u < kStage; ++u) {
    const unsigned i = tid + u * kThreads;
    const unsigned p = i / (kD / 8), d8 = (i % (kD / 8)) * 8;
    if (p0 + p >= limit) kr[u] = u32x4{0, 0, 0, 0};
    if (!Rope || p0 + p < fresh || p0 + p >= limit) *reinterpret_cast<u32x4*>(&ks[p][d8]) = kr[u];
  }
#pragma unroll
  for (unsigned u = 0; u < kVItems; ++u) {
    const unsigned i = tid + u * kThreads;
    const unsigned pair = i % (kSplit / 2), d8 = (i / (kSplit / 2)) * 8;
    const uint64_t pa = p0 + 2 * pair, pb = pa + 1;
    if (pa >= limit) va[u] = u32x4{0, 0, 0, 0};
    if (pb >= limit) vb[u] = u32x4{0, 0, 0, 0};
    // With Rope a pair may hold a new position (written by the RoPE step): then only the
    // older half (if any) is staged, as a 16-bit store.
    const bool a_staged = !Rope || pa < fresh || pa >= limit;
    const bool b_staged = !Rope || pb < fresh || pb >= limit;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const unsigned lo = (va[u][e / 2] >> (16 * (e % 2))) & 0xffffu;
      const unsigned hi = (vb[u][e / 2] >> (16 * (e % 2))) & 0xffffu;
      if (a_staged && b_staged) {
        *reinterpret_cast<unsigned*>(&vt[d8 + e][2 * pair]) = lo | (hi << 16);
      } else if (a_staged) {
        *reinterpret_cast<unsigned short*>(&vt[d8 + e][2 * pair]) = static_cast<unsigned short>(lo);
      } else if (b_staged) {
        *reinterpret_cast<unsigned short*>(&vt[d8 + e][2 * pair + 1]) = static_cast<unsigned short>(hi);
      }
    }
  }
  __syncthreads();
  if constexpr (Rope) load_q(wave, q_next);

  for (unsigned rt = wave; rt < row_tiles; rt += Waves) {
    // This tile's Q operand was loaded one tile ahead; the next tile's goes out now.
    h8 q[kQ];
#pragma unroll
    for (unsigned s = 0; s < kQ; ++s) q[s] = q_next[s];
    load_q(rt + Waves, q_next);
    // S = Q K^T for the split's positions (kTiles tiles of 16).
    f4 sc[kTiles];
#pragma unroll
    for (unsigned j = 0; j < kTiles; ++j) {
      f4 acc = {0, 0, 0, 0};
#pragma unroll
      for (unsigned s = 0; s < kQ; ++s) {
        const h8 kk = *reinterpret_cast<const h8*>(&ks[j * 16 + m][32 * s + 8 * kb]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(q[s], kk, acc, 0, 0, 0);
      }
      sc[j] = acc;
    }
    // Mask, scale, split-local softmax.  Lane holds rows 4*kb + r, position j*16 + m.
    float mx[4], sum[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const unsigned row = rt * 16 + 4 * kb + r;
      const uint64_t count = row < rows ? base + row / group : 0;  // visible positions
      float best = -INFINITY;
#pragma unroll
      for (unsigned j = 0; j < kTiles; ++j) {
        const uint64_t pos = p0 + j * 16 + m;
        const float s = pos < count ? sc[j][r] * a.scale : -INFINITY;
        sc[j][r] = s;
        best = fmaxf(best, s);
      }
      best = row16_max(best);
      float total = 0.0F;
#pragma unroll
      for (unsigned j = 0; j < kTiles; ++j) {
        const float p = best == -INFINITY ? 0.0F : expf(sc[j][r] - best);
        total += p;
        const _Float16 hi = static_cast<_Float16>(p);
        ps[wave][4 * kb + r][j * 16 + m] = hi;
        ps_lo[wave][4 * kb + r][j * 16 + m] = static_cast<_Float16>(p - static_cast<float>(hi));
      }
      total = row16_sum(total);
      mx[r] = best;
      sum[r] = total;
    }
    // O = P V: kD / 16 tiles of 16 head dims, kSteps K-steps of 32 positions.
    h8 pa[kSteps], pl[kSteps];
#pragma unroll
    for (unsigned s = 0; s < kSteps; ++s) {
      pa[s] = *reinterpret_cast<const h8*>(&ps[wave][m][32 * s + 8 * kb]);
      pl[s] = *reinterpret_cast<const h8*>(&ps_lo[wave][m][32 * s + 8 * kb]);
    }
#pragma unroll
    for (unsigned dj = 0; dj < kD / 16; ++dj) {
      f4 acc = {0, 0, 0, 0};
#pragma unroll
      for (unsigned s = 0; s < kSteps; ++s) {
        const h8 vv = *reinterpret_cast<const h8*>(&vt[dj * 16 + m][32 * s + 8 * kb]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[s], vv, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[s], vv, acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned row = rt * 16 + 4 * kb + r;
        if (row < rows) {
          const unsigned t = row / group, g = row - t * group;
          const std::size_t idx = static_cast<std::size_t>(t) * a.q_heads + hk * group + g;
          a.partial_o[(idx * a.splits + split) * kD + dj * 16 + m] = acc[r];
        }
      }
    }
    if (m == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned row = rt * 16 + 4 * kb + r;
        if (row < rows) {
          const unsigned t = row / group, g = row - t * group;
          const std::size_t idx = static_cast<std::size_t>(t) * a.q_heads + hk * group + g;
          a.partial_ml[(idx * a.splits + split) * 2] = mx[r];
          a.partial_ml[(idx * a.splits + split) * 2 + 1] = sum[r];
        }
      }
    }
  }
}

// Merge the splits of each (token, q head) and apply the sigmoid gate.  One wave per
// (token, head, 128-dim group j of the head); lane owns head dims 128 j + 2l and
// 128 j + 2l + 1.  The waves of a head's groups compute the same weights and sum.  With
// codes set, the wave also quantizes its group to A4G128 as quantize_activation_i4 does
// on the fp16 output row ([T][Hq * D] -> codes [T][Hq * D / 2], scales [T][Hq * D / 128]).
template <unsigned kD>
__global__ __launch_bounds__(256) void attention_combine_kernel(AttnArgs a, const float* __restrict__ gate,
                                                                __half* __restrict__ output,
                                                                uint8_t* __restrict__ codes,
                                                                __half* __restrict__ scales) {
  constexpr unsigned kSplit = split_positions<kD>();
  constexpr unsigned kGroups = kD / 128;  // 128-dim groups per head: one wave each
  constexpr unsigned kG = 1;              // groups per wave
  const uint32_t linear = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (linear >= a.tokens * a.q_heads * kGroups) return;
  const unsigned lane = threadIdx.x & 63u;
  const uint32_t th = linear / kGroups, group = linear - th * kGroups;  // (token, head), group
  const uint32_t t = th / a.q_heads, qh = th - t * a.q_heads;
  // The gate row first: it does not depend on the position.
  const float* g = gate + static_cast<std::size_t>(t) * a.q_heads * kD * 2 + static_cast<std::size_t>(qh) * kD * 2 + kD +
                   128 * group;
  float2 gv[kG];
#pragma unroll
  for (unsigned j = 0; j < kG; ++j) gv[j] = *reinterpret_cast<const float2*>(g + 128 * j + 2 * lane);
  const uint64_t count = base_count_of(a) + t;
  const unsigned used = static_cast<unsigned>((count + kSplit - 1) / kSplit);
  const float* ml = a.partial_ml + static_cast<std::size_t>(th) * a.splits * 2;
  const float* po = a.partial_o + static_cast<std::size_t>(th) * a.splits * kD + 128 * group + 2 * lane;
  float o0[kG], o1[kG], total = 0.0F;
#pragma unroll
  for (unsigned j = 0; j < kG; ++j) o0[j] = o1[j] = 0.0F;
  if (used <= 128u) {
    // Up to 128 splits (a 4096-position context at either head size): lane s holds the
    // (max, sum) of splits s and 64 + s, loaded at once; the maximum is a DPP wave
    // reduction and each split's weight exp(m - best) is computed once, in its lane,
    // and read out to a scalar where the output rows are accumulated.  The output rows
    // stream in batches of kBatch splits, each batch's loads issued while the previous
    // batch is accumulated; the accumulation keeps split order.
    const unsigned sa = lane, sb = 64u + lane;
    const float2 pa = *reinterpret_cast<const float2*>(ml + 2 * (sa < used ? sa : 0u));
    const float2 pb = *reinterpret_cast<const float2*>(ml + 2 * (sb < used ? sb : 0u));
    const float best = wave_max(fmaxf(sa < used ? pa.x : -INFINITY, sb < used ? pb.x : -INFINITY));
    const float wa = sa < used ? expf(pa.x - best) : 0.0F;
    const float wb = sb < used ? expf(pb.x - best) : 0.0F;
    total = wave_sum(fmaf(pb.y, wb, pa.y * wa));
    constexpr unsigned kBatch = 16;
    float2 cur[kBatch][kG], next[kBatch][kG];
    auto fetch = [&](float2 (&v)[kBatch][kG], unsigned s0) __attribute__((always_inline)) {
#pragma unroll
      for (unsigned k = 0; k < kBatch; ++k) {
        const unsigned s = s0 + k < used ? s0 + k : used - 1u;  // past the last split: loaded, not used
#pragma unroll
        for (unsigned j = 0; j < kG; ++j) {
          v[k][j] = *reinterpret_cast<const float2*>(po + static_cast<std::size_t>(s) * kD + 128 * j);
        }
      }
    };
    fetch(cur, 0);
    for (unsigned s0 = 0; s0 < used; s0 += kBatch) {
      if (s0 + kBatch < used) fetch(next, s0 + kBatch);
#pragma unroll
      for (unsigned k = 0; k < kBatch; ++k) {
        const unsigned s = s0 + k;
        if (s < used) {
          const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s < 64u ? wa : wb), s & 63u));
#pragma unroll
          for (unsigned j = 0; j < kG; ++j) {
            o0[j] = fmaf(cur[k][j].x, w, o0[j]);
            o1[j] = fmaf(cur[k][j].y, w, o1[j]);
          }
        }
      }
#pragma unroll
      for (unsigned k = 0; k < kBatch; ++k)
#pragma unroll
        for (unsigned j = 0; j < kG; ++j) cur[k][j] = next[k][j];
    }
  } else {
    // Longer contexts: splits in batches of kBatch with every load of a batch issued
    // before its first use; the sums run in split order.
    constexpr unsigned kBatch = 8;
    float best = -INFINITY;
    for (unsigned s0 = 0; s0 < used; s0 += kBatch) {
      float m[kBatch];
#pragma unroll
      for (unsigned k = 0; k < kBatch; ++k) m[k] = s0 + k < used ? ml[2 * (s0 + k)] : -INFINITY;
#pragma unroll
      for (unsigned k = 0; k < kBatch; ++k) best = fmaxf(best, m[k]);
    }
    for (unsigned s0 = 0; s0 < used; s0 += kBatch) {
      float2 mls[kBatch], v[kBatch][kG];
#pragma unroll
      for (unsigned k = 0; k < kBatch; ++k) {
        const unsigned s = s0 + k < used ? s0 + k : s0;
        mls[k] = *reinterpret_cast<const float2*>(ml + 2 * s);
#pragma unroll
        for (unsigned j = 0; j < kG; ++j) {
          v[k][j] = *reinterpret_cast<const float2*>(po + static_cast<std::size_t>(s) * kD + 128 * j);
        }
      }
#pragma unroll
      for (unsigned k = 0; k < kBatch; ++k) {
        if (s0 + k < used) {
          const float w = expf(mls[k].x - best);
          total = fmaf(mls[k].y, w, total);
#pragma unroll
          for (unsigned j = 0; j < kG; ++j) {
            o0[j] = fmaf(v[k][j].x, w, o0[j]);
            o1[j] = fmaf(v[k][j].y, w, o1[j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (unsigned j = 0; j < kG; ++j) {
    const float g0 = 1.0F / (1.0F + expf(-gv[j].x));
    const float g1 = 1.0F / (1.0F + expf(-gv[j].y));
    const unsigned jg = group + j;
    __half* out = output + static_cast<std::size_t>(th) * kD + 128 * jg + 2 * lane;
    const __half h0 = to_half(o0[j] / total * g0), h1 = to_half(o1[j] / total * g1);
    out[0] = h0;
    out[1] = h1;
    if (codes != nullptr) {
      quantize_group_a4(h0, h1, codes + static_cast<std::size_t>(th) * (kD / 2) + 64 * jg,
                        scales + static_cast<std::size_t>(th) * kGroups + jg, lane);
    }
  }
}

int32_t attention_entry(const uint16_t* query, const float* gate, const uint16_t* key_cache,
                        const uint16_t* value_cache, uint16_t* output, uint64_t base_count,
                        const uint64_t* indirect, size_t capacity, uint32_t batch, uint32_t q_heads,
                        uint32_t kv_heads, uint32_t head_size, float* workspace,
                        size_t workspace_bytes, hipStream_t stream, uint8_t* codes = nullptr,
                        uint16_t* scales = nullptr);

}  // namespace
}  // namespace gfx950

using namespace gfx950;

extern "C" size_t gfxinfer_attention_workspace_bytes(uint32_t batch, uint32_t q_heads,
                                                     uint32_t head_size, size_t capacity) {
  if (head_size != 128 && head_size != 256) return 0;
  return static_cast<std::size_t>(batch) * q_heads * split_count(head_size, capacity) * (head_size + 2) *
         sizeof(float);
}

namespace gfx950 {
namespace {
// The combine launch of a split launch: one wave per (token, head, 128-dim group).
int32_t launch_combine(const AttnArgs& args, const float* gate, uint16_t* output, uint8_t* codes,
                       uint16_t* scales, uint32_t head_size, hipStream_t stream) {
  const dim3 combine_grid((args.tokens * args.q_heads * (head_size / 128) + 3) / 4);
  __half* out16 = reinterpret_cast<__half*>(output);
  __half* scales16 = reinterpret_cast<__half*>(scales);
  if (head_size == 128) {
    hipLaunchKernelGGL(attention_combine_kernel<128>, combine_grid, dim3(256), 0, stream, args, gate, out16,
                       codes, scales16);
  } else {
    hipLaunchKernelGGL(attention_combine_kernel<256>, combine_grid, dim3(256), 0, stream, args, gate, out16,
                       codes, scales16);
  }
  return launch_status("gated attention combine launch failed");
}

int32_t attention_entry(const uint16_t* query, const float* gate, const uint16_t* key_cache,
                        const uint16_t* value_cache, uint16_t* output, uint64_t base_count,
                        const uint64_t* indirect, size_t capacity, uint32_t batch, uint32_t q_heads,
                        uint32_t kv_heads, uint32_t head_size, float* workspace,
                        size_t workspace_bytes, hipStream_t stream, uint8_t* codes,
                        uint16_t* scales) {
  if ((codes == nullptr) != (scales == nullptr)) {
    return fail(GFXI_INVALID_ARGUMENT, "A4 codes and scales of the attention output go together");
  }
  if (query == nullptr || gate == nullptr || key_cache == nullptr || value_cache == nullptr ||
      output == nullptr || workspace == nullptr || batch == 0 || batch > 32 || q_heads == 0 ||
      kv_heads == 0 || q_heads % kv_heads != 0 || (head_size != 128 && head_size != 256) ||
      capacity == 0 || capacity > (1u << 24) ||
      (indirect == nullptr && (base_count == 0 || base_count + batch - 1 > capacity))) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid gated attention decode arguments (head size 128 or "
                                       "256, 1..32 tokens, visible positions within capacity)");
  }
  if (workspace_bytes < gfxinfer_attention_workspace_bytes(batch, q_heads, head_size, capacity)) {
    return fail(GFXI_INVALID_ARGUMENT, "attention workspace is too small");
  }
  const auto splits = static_cast<uint32_t>(split_count(head_size, capacity));
  float* partial_o = workspace;
  float* partial_ml = workspace + static_cast<std::size_t>(batch) * q_heads * splits * head_size;
  AttnArgs args{};
  args.query = reinterpret_cast<const __half*>(query);
  args.key_cache = reinterpret_cast<const __half*>(key_cache);
  args.value_cache = reinterpret_cast<const __half*>(value_cache);
  args.partial_o = partial_o;
  args.partial_ml = partial_ml;
  args.base_count = base_count;
  args.indirect_position = indirect;
  args.tokens = batch;
  args.q_heads = q_heads;
  args.kv_heads = kv_heads;
  args.splits = splits;
  args.capacity = static_cast<uint32_t>(capacity);
  args.scale = 1.0F / std::sqrt(static_cast<float>(head_size));
  const unsigned rows = (q_heads / kv_heads) * batch;
  const bool wide = rows > 4 * 16;
  const dim3 grid(splits * kv_heads), block(wide ? 512 : 256);
  if (head_size == 128 && wide) {
    hipLaunchKernelGGL((attention_split_kernel<128, 8>), grid, block, 0, stream, args);
  } else if (head_size == 128) {
    hipLaunchKernelGGL((attention_split_kernel<128, 4>), grid, block, 0, stream, args);
  } else if (wide) {
    hipLaunchKernelGGL((attention_split_kernel<256, 8>), grid, block, 0, stream, args);
  } else {
    hipLaunchKernelGGL((attention_split_kernel<256, 4>), grid, block, 0, stream, args);
  }
  if (const int32_t s = launch_status("gated attention split launch failed"); s != GFXI_OK) return s;
  return launch_combine(args, gate, output, codes, scales, head_size, stream);
}

int32_t rope_attention_entry(const float* query_input, const uint16_t* query_weight, size_t query_stride,
                             const float* key_input, const uint16_t* key_weight, size_t key_stride,
                             const float* value_input, size_t rotary, float theta, const float* rope_table,
                             const float* gate,
                             uint16_t* key_cache, uint16_t* value_cache, uint16_t* output, uint8_t* codes,
                             uint16_t* scales, uint64_t position, const uint64_t* indirect, size_t capacity,
                             uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t head_size,
                             float* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (query_input == nullptr || query_weight == nullptr || key_input == nullptr || key_weight == nullptr ||
      value_input == nullptr || gate == nullptr || key_cache == nullptr || value_cache == nullptr ||
      output == nullptr || codes == nullptr || scales == nullptr || workspace == nullptr || batch == 0 ||
      q_heads == 0 || kv_heads == 0 || q_heads % kv_heads != 0 || (head_size != 128 && head_size != 256) ||
      rotary == 0 || rotary > 64 || rotary % 2 != 0 || query_stride < head_size || key_stride < head_size ||
      !std::isfinite(theta) || theta <= 0.0F || capacity == 0 || capacity > (1u << 24) ||
      (indirect == nullptr && (position >= capacity || batch > capacity - position))) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid fused Q/K RMSNorm/RoPE/K-V append/attention arguments");
  }
  if (!fused_rope_supported(batch, q_heads, kv_heads, head_size)) {
    return fail(GFXI_UNSUPPORTED, "fused RoPE attention takes at most 8 tokens, 8 query heads per KV head and " +
                                      std::to_string(fused_rope_rows(head_size)) +
                                      " query rows per KV head; use the RoPE launch then the attention launch");
  }
  if (workspace_bytes < gfxinfer_attention_workspace_bytes(batch, q_heads, head_size, capacity)) {
    return fail(GFXI_INVALID_ARGUMENT, "attention workspace is too small");
  }
  const auto splits = static_cast<uint32_t>(split_count(head_size, capacity));
  AttnArgs args{};
  args.query = nullptr;
  args.key_cache = reinterpret_cast<const __half*>(key_cache);
  args.value_cache = reinterpret_cast<const __half*>(value_cache);
  args.partial_o = workspace;
  args.partial_ml = workspace + static_cast<std::size_t>(batch) * q_heads * splits * head_size;
  args.base_count = position + 1;
  args.indirect_position = indirect;
  args.tokens = batch;
  args.q_heads = q_heads;
  args.kv_heads = kv_heads;
  args.splits = splits;
  args.capacity = static_cast<uint32_t>(capacity);
  args.scale = 1.0F / std::sqrt(static_cast<float>(head_size));
  args.q_in = query_input;
  args.q_weight = query_weight;
  args.k_in = key_input;
  args.k_weight = key_weight;
  args.v_in = value_input;
  args.key_cache_out = reinterpret_cast<__half*>(key_cache);
  args.value_cache_out = reinterpret_cast<__half*>(value_cache);
  args.q_stride = static_cast<uint32_t>(query_stride);
  args.k_stride = static_cast<uint32_t>(key_stride);
  args.rotary = static_cast<uint32_t>(rotary);
  args.theta = theta;
  args.rope_table = reinterpret_cast<const float2*>(rope_table);
  const dim3 grid(splits * kv_heads), block(256);
  if (head_size == 128) {
    hipLaunchKernelGGL((attention_split_kernel<128, 4, true>), grid, block, 0, stream, args);
  } else {
    hipLaunchKernelGGL((attention_split_kernel<256, 4, true>), grid, block, 0, stream, args);
  }
  if (const int32_t s = launch_status("fused RoPE attention split launch failed"); s != GFXI_OK) return s;
  return launch_combine(args, gate, output, codes, scales, head_size, stream);
}
}  // namespace
}  // namespace gfx950

extern "C" int32_t gfxinfer_launch_gated_attention_decode_block(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, size_t base_token_count, size_t capacity, uint32_t batch, uint32_t q_heads,
    uint32_t kv_heads, uint32_t head_size, float* workspace, size_t workspace_bytes, void* stream) {
  return attention_entry(query, gate, key_cache, value_cache, output, base_token_count, nullptr, capacity,
                         batch, q_heads, kv_heads, head_size, workspace, workspace_bytes,
                         static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_gated_attention_decode_block_indirect_position(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, const uint64_t* base_position, size_t capacity, uint32_t batch,
    uint32_t q_heads, uint32_t kv_heads, uint32_t head_size, float* workspace,
    size_t workspace_bytes, void* stream) {
  if (base_position == nullptr) return fail(GFXI_INVALID_ARGUMENT, "indirect position is null");
  return attention_entry(query, gate, key_cache, value_cache, output, 0, base_position, capacity, batch,
                         q_heads, kv_heads, head_size, workspace, workspace_bytes,
                         static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_gated_attention_decode_block_quantize_i4(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, uint8_t* codes, uint16_t* scales, size_t base_token_count, size_t capacity,
    uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t head_size, float* workspace,
    size_t workspace_bytes, void* stream) {
  if (codes == nullptr) return fail(GFXI_INVALID_ARGUMENT, "A4 codes of the attention output are null");
  return attention_entry(query, gate, key_cache, value_cache, output, base_token_count, nullptr, capacity,
                         batch, q_heads, kv_heads, head_size, workspace, workspace_bytes,
                         static_cast<hipStream_t>(stream), codes, scales);
}

extern "C" int32_t gfxinfer_launch_gated_attention_decode_block_quantize_i4_indirect_position(
    const uint16_t* query, const float* gate, const uint16_t* key_cache, const uint16_t* value_cache,
    uint16_t* output, uint8_t* codes, uint16_t* scales, const uint64_t* base_position, size_t capacity,
    uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t head_size, float* workspace,
    size_t workspace_bytes, void* stream) {
  if (base_position == nullptr || codes == nullptr) {
    return fail(GFXI_INVALID_ARGUMENT, "indirect position or A4 codes of the attention output are null");
  }
  return attention_entry(query, gate, key_cache, value_cache, output, 0, base_position, capacity, batch,
                         q_heads, kv_heads, head_size, workspace, workspace_bytes,
                         static_cast<hipStream_t>(stream), codes, scales);
}

extern "C" int32_t gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4(
    const float* query_input, const uint16_t* query_bf16_weight, size_t query_input_stride,
    const float* key_input, const uint16_t* key_bf16_weight, size_t key_input_stride, const float* value_input,
    size_t rotary_size, float rope_theta, const float* rope_table, const float* gate, uint16_t* key_cache,
    uint16_t* value_cache,
    uint16_t* output, uint8_t* codes, uint16_t* scales, size_t position, size_t capacity, uint32_t batch,
    uint32_t q_heads, uint32_t kv_heads, uint32_t head_size, float* workspace, size_t workspace_bytes,
    void* stream) {
  return rope_attention_entry(query_input, query_bf16_weight, query_input_stride, key_input, key_bf16_weight,
                              key_input_stride, value_input, rotary_size, rope_theta, rope_table, gate,
                              key_cache,
                              value_cache, output, codes, scales, position, nullptr, capacity, batch, q_heads,
                              kv_heads, head_size, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4_indirect_position(
    const float* query_input, const uint16_t* query_bf16_weight, size_t query_input_stride,
    const float* key_input, const uint16_t* key_bf16_weight, size_t key_input_stride, const float* value_input,
    size_t rotary_size, float rope_theta, const float* rope_table, const float* gate, uint16_t* key_cache,
    uint16_t* value_cache,
    uint16_t* output, uint8_t* codes, uint16_t* scales, const uint64_t* base_position, size_t capacity,
    uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t head_size, float* workspace,
    size_t workspace_bytes, void* stream) {
  if (base_position == nullptr) return fail(GFXI_INVALID_ARGUMENT, "indirect position is null");
  return rope_attention_entry(query_input, query_bf16_weight, query_input_stride, key_input, key_bf16_weight,
                              key_input_stride, value_input, rotary_size, rope_theta, rope_table, gate,
                              key_cache,
                              value_cache, output, codes, scales, 0, base_position, capacity, batch, q_heads,
                              kv_heads, head_size, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int32_t gfxinfer_fused_rope_attention_supported(uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                                                           uint32_t head_size) {
  return fused_rope_supported(batch, q_heads, kv_heads, head_size) ? 1 : 0;
}
