/*
 * CPU oracle for the speculative-verify hot path.  TEST INFRASTRUCTURE ONLY
 * (see oracle.h): only tests/, the smoke entry and bench.py's cpu_baseline leg
 * may load it, and only as the checker.
 *
 * Built with -ffp-contract=off so that every fused multiply-add below is an
 * explicit fmaf() exactly where the reference source has one.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define GROUP 128u

/* ------------------------------------------------------------------------ */
/* fp16 / bf16                                                                */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  return bits;
}

static float bits_f32(uint32_t bits) {
  float value;
  memcpy(&value, &bits, sizeof value);
  return value;
}

/* IEEE 754 binary32 -> binary16 with round-to-nearest-even.  This is what the
 * reference's __float2half (converter.cpp:383-386, lowbit_gemv.hip:388) does on
 * ROCm: a _Float16 conversion under the default rounding mode. */
uint16_t orc_f32_to_f16(float value) {
  const uint32_t x = f32_bits(value);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal */
    if (ax < 0x33000000u) return (uint16_t)sign;             /* below 2^-25 */
    const uint32_t exponent = ax >> 23;
    const uint32_t mantissa = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - exponent; /* 14..24 */
    uint32_t quotient = mantissa >> shift;
    const uint32_t remainder = mantissa & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (remainder > half || (remainder == half && (quotient & 1u))) ++quotient;
    return (uint16_t)(sign | quotient);
  }
  const uint32_t exponent = (ax >> 23) - 112u;
  const uint32_t mantissa = ax & 0x7fffffu;
  uint32_t result = (exponent << 10) | (mantissa >> 13);
  const uint32_t remainder = mantissa & 0x1fffu;
  if (remainder > 0x1000u || (remainder == 0x1000u && (result & 1u))) ++result;
  return (uint16_t)(sign | result);
}

float orc_f16_to_f32(uint16_t bits) {
  const uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
  const uint32_t exponent = ((uint32_t)bits >> 10) & 0x1fu;
  const uint32_t mantissa = (uint32_t)bits & 0x3ffu;
  if (exponent == 0) {
    /* zero or subnormal: exact in binary32 */
    const float magnitude = (float)mantissa * 5.9604644775390625e-08f; /* 2^-24 */
    return sign ? -magnitude : magnitude;
  }
  if (exponent == 31) return bits_f32(sign | 0x7f800000u | (mantissa << 13));
  return bits_f32(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

void orc_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}

void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

/* qwen_ops.hip:27-29 */
float orc_bf16_to_f32(uint16_t bits) { return bits_f32((uint32_t)bits << 16); }

static float h2f(uint16_t bits) { return orc_f16_to_f32(bits); }
static uint16_t f2h(float value) { return orc_f32_to_f16(value); }

/* GPU float->int conversion semantics of __float2int_rn (v_rndne + v_cvt_i32):
 * round half to even, NaN -> 0, saturate out of range. */
static int float2int_rn(float value) {
  if (value != value) return 0;
  const float rounded = nearbyintf(value);
  if (rounded >= 2147483648.0f) return 2147483647;
  if (rounded < -2147483648.0f) return (int)(-2147483647 - 1);
  return (int)rounded;
}

static int clampi(int value, int low, int high) {
  return value < low ? low : (value > high ? high : value);
}

/* ------------------------------------------------------------------------ */
/* Weight quantizer: src/quantization.cpp                                     */
/* ------------------------------------------------------------------------ */

/* quantization.cpp:15-27 -- first strictly-closer level wins. */
static int nearest_w2(float normalized) {
  static const int levels[4] = {-3, -1, 1, 3};
  int best = levels[0];
  float best_error = INFINITY;
  for (int i = 0; i < 4; ++i) {
    const float error = fabsf(normalized - (float)levels[i]);
    if (error < best_error) {
      best = levels[i];
      best_error = error;
    }
  }
  return best;
}

/* quantization.cpp:29-46 */
static uint8_t encode_value(float value, float scale, int format) {
  const float normalized = scale == 0.0f ? 0.0f : value / scale;
  switch (format) {
    case ORC_W2: return (uint8_t)((nearest_w2(normalized) + 3) / 2);
    case ORC_W3: return (uint8_t)(clampi((int)nearbyintf(normalized), -4, 3) + 4);
    case ORC_W4: return (uint8_t)(clampi((int)nearbyintf(normalized), -8, 7) & 0x0f);
    default: return 0;
  }
}

/* quantization.cpp:48-56 */
int orc_decode_value(uint8_t code, int format) {
  switch (format) {
    case ORC_W2: return (int)code * 2 - 3;
    case ORC_W3: return (int)code - 4;
    case ORC_W4: return (code & 0x08u) ? (int)code - 16 : (int)code;
    default: return 0;
  }
}

/* quantization.cpp:58-65 */
static float format_divisor(int format) {
  switch (format) {
    case ORC_W2: return 3.0f;
    case ORC_W3: return 4.0f;
    case ORC_W4: return 8.0f;
    default: return 1.0f;
  }
}

/* quantization.cpp:67-92 -- four least-squares refits in double, floor FLT_MIN. */
static float choose_scale(const float* values, float maximum, int format) {
  if (maximum == 0.0f) return 1.0f;
  float scale = maximum / format_divisor(format);
  for (int iteration = 0; iteration < 4; ++iteration) {
    double numerator = 0.0;
    double denominator = 0.0;
    for (unsigned i = 0; i < GROUP; ++i) {
      const int level = orc_decode_value(encode_value(values[i], scale, format), format);
      numerator += (double)values[i] * level;
      denominator += (double)level * level;
    }
    if (denominator == 0.0) break;
    scale = (float)(numerator / denominator);
  }
  return scale > FLT_MIN ? scale : FLT_MIN;
}

/* quantization.cpp:94-124 */
static void store_code(uint8_t* row, size_t column, uint8_t code, int format) {
  switch (format) {
    case ORC_W2: row[column / 4] |= (uint8_t)((code & 0x03u) << ((column & 3u) * 2u)); break;
    case ORC_W3: {
      const size_t group = column / GROUP, local = column % GROUP;
      for (unsigned plane = 0; plane < 3; ++plane) {
        row[group * 48 + plane * 16 + local / 8] |=
            (uint8_t)(((code >> plane) & 1u) << (local & 7u));
      }
      break;
    }
    case ORC_W4: row[column / 2] |= (uint8_t)((code & 0x0fu) << ((column & 1u) * 4u)); break;
    default: break;
  }
}

/* quantization.cpp:126-150 */
uint8_t orc_load_code(const uint8_t* row, size_t column, int format) {
  switch (format) {
    case ORC_W2: return (uint8_t)((row[column / 4] >> ((column & 3u) * 2u)) & 0x03u);
    case ORC_W3: {
      const size_t group = column / GROUP, local = column % GROUP;
      uint8_t code = 0;
      for (unsigned plane = 0; plane < 3; ++plane) {
        code |= (uint8_t)(((row[group * 48 + plane * 16 + local / 8] >> (local & 7u)) & 1u)
                          << plane);
      }
      return code;
    }
    case ORC_W4: return (uint8_t)((row[column / 2] >> ((column & 1u) * 4u)) & 0x0fu);
    default: return 0;
  }
}

/* quantization.cpp:154-161 */
size_t orc_packed_row_bytes(int format, size_t columns) {
  switch (format) {
    case ORC_W2: return (columns + 3) / 4;
    case ORC_W3: return (columns * 3 + 7) / 8;
    case ORC_W4: return (columns + 1) / 2;
    default: return 0;
  }
}

/* quantization.cpp:163-220 */
int orc_quantize_group128(const float* weights, size_t rows, size_t columns, int format,
                          uint8_t* codes, float* scales) {
  if (rows == 0 || columns == 0 || columns % GROUP != 0 || weights == NULL) {
    return ORC_INVALID_ARGUMENT;
  }
  if (format != ORC_W2 && format != ORC_W3 && format != ORC_W4) return ORC_UNSUPPORTED;
  const size_t row_bytes = orc_packed_row_bytes(format, columns);
  const size_t groups = columns / GROUP;
  memset(codes, 0, rows * row_bytes);
  int non_finite = 0;
#pragma omp parallel for schedule(static) reduction(| : non_finite)
  for (long long signed_row = 0; signed_row < (long long)rows; ++signed_row) {
    const size_t row = (size_t)signed_row;
    const float* source = weights + row * columns;
    uint8_t* destination = codes + row * row_bytes;
    for (size_t group = 0; group < groups; ++group) {
      float maximum = 0.0f;
      int group_non_finite = 0;
      for (size_t offset = 0; offset < GROUP; ++offset) {
        const float value = source[group * GROUP + offset];
        if (!isfinite(value)) {
          group_non_finite = 1;
          continue;
        }
        const float magnitude = fabsf(value);
        if (magnitude > maximum) maximum = magnitude;
      }
      if (group_non_finite) {
        /* The whole matrix is rejected below, so this group's codes and scale are never
           read; the reference still converts the NaN quotients to int, which is undefined
           behaviour in C, so the oracle leaves the group at zero codes and scale 1. */
        non_finite = 1;
        scales[row * groups + group] = 1.0f;
        continue;
      }
      const float scale = choose_scale(source + group * GROUP, maximum, format);
      scales[row * groups + group] = scale;
      for (size_t offset = 0; offset < GROUP; ++offset) {
        const size_t column = group * GROUP + offset;
        store_code(destination, column, encode_value(source[column], scale, format), format);
      }
    }
  }
  return non_finite ? ORC_INVALID_ARGUMENT : ORC_OK;
}

/* quantization.cpp:222-235 */
float orc_dequantized_weight(const uint8_t* codes, const float* scales, size_t rows,
                             size_t columns, int format, size_t row, size_t column) {
  if (row >= rows || column >= columns || columns % GROUP != 0) return NAN;
  const size_t row_bytes = orc_packed_row_bytes(format, columns);
  const uint8_t code = orc_load_code(codes + row * row_bytes, column, format);
  return (float)orc_decode_value(code, format) * scales[row * (columns / GROUP) + column / GROUP];
}

void orc_unpack_weights(const uint8_t* codes, size_t rows, size_t columns, int format,
                        int8_t* out) {
  const size_t row_bytes = orc_packed_row_bytes(format, columns);
#pragma omp parallel for schedule(static)
  for (long long r = 0; r < (long long)rows; ++r) {
    for (size_t c = 0; c < columns; ++c) {
      out[(size_t)r * columns + c] =
          (int8_t)orc_decode_value(orc_load_code(codes + (size_t)r * row_bytes, c, format), format);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Activation quantizers: src/kernels/lowbit_gemv.hip                         */
/* ------------------------------------------------------------------------ */

/* lowbit_gemv.hip:373-407.  Scale = fp16(max|x| / 7) (1 for an all-zero group),
 * codes = clamp(rint(x / float(scale16)), -7, 7), even column in the low nibble. */
int orc_quantize_activation_i4(const uint16_t* input, uint8_t* packed, uint16_t* scales,
                               size_t columns, unsigned batch) {
  if (columns == 0 || columns % GROUP != 0 || batch == 0 || batch > 32) {
    return ORC_INVALID_ARGUMENT;
  }
  const size_t groups = columns / GROUP;
  for (unsigned b = 0; b < batch; ++b) {
    for (size_t g = 0; g < groups; ++g) {
      const uint16_t* x = input + (size_t)b * columns + g * GROUP;
      float maximum = 0.0f;
      for (unsigned i = 0; i < GROUP; ++i) maximum = fmaxf(maximum, fabsf(h2f(x[i])));
      const uint16_t scale16 = f2h(maximum == 0.0f ? 1.0f : maximum / 7.0f);
      scales[(size_t)b * groups + g] = scale16;
      const float scale = h2f(scale16);
      for (unsigned i = 0; i < GROUP / 2; ++i) {
        const int low = clampi(float2int_rn(h2f(x[2 * i]) / scale), -7, 7);
        const int high = clampi(float2int_rn(h2f(x[2 * i + 1]) / scale), -7, 7);
        packed[(size_t)b * (columns / 2) + g * 64 + i] =
            (uint8_t)((low & 0x0f) | ((high & 0x0f) << 4));
      }
    }
  }
  return ORC_OK;
}

/* lowbit_gemv.hip:409-436 */
int orc_quantize_activation_i8(const uint16_t* input, int8_t* codes, uint16_t* scales,
                               size_t columns, unsigned batch) {
  if (columns == 0 || columns % GROUP != 0 || batch == 0 || batch > 32) {
    return ORC_INVALID_ARGUMENT;
  }
  const size_t groups = columns / GROUP;
  for (unsigned b = 0; b < batch; ++b) {
    for (size_t g = 0; g < groups; ++g) {
      const size_t base = (size_t)b * columns + g * GROUP;
      float maximum = 0.0f;
      for (unsigned i = 0; i < GROUP; ++i) maximum = fmaxf(maximum, fabsf(h2f(input[base + i])));
      const uint16_t scale16 = f2h(maximum == 0.0f ? 1.0f : maximum / 127.0f);
      scales[(size_t)b * groups + g] = scale16;
      const float scale = h2f(scale16);
      for (unsigned i = 0; i < GROUP; ++i) {
        codes[base + i] = (int8_t)clampi(float2int_rn(h2f(input[base + i]) / scale), -127, 127);
      }
    }
  }
  return ORC_OK;
}

void orc_unpack_a4(const uint8_t* packed, size_t columns, unsigned batch, int8_t* out) {
  for (unsigned b = 0; b < batch; ++b) {
    for (size_t c = 0; c < columns; ++c) {
      const unsigned code = (packed[(size_t)b * (columns / 2) + c / 2] >> ((c & 1u) * 4u)) & 0x0fu;
      out[(size_t)b * columns + c] = (int8_t)(code >= 8u ? (int)code - 16 : (int)code);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Integer GEMM + epilogue: lowbit_gemv.hip:461-553 (i4), 682-755 (i8)        */
/* ------------------------------------------------------------------------ */

void orc_gemm_partials(const int8_t* w, const int8_t* a, size_t rows, size_t columns,
                       unsigned batch, int32_t* partials) {
  const size_t groups = columns / GROUP;
#pragma omp parallel for schedule(static)
  for (long long n = 0; n < (long long)rows; ++n) {
    const int8_t* wr = w + (size_t)n * columns;
    for (unsigned b = 0; b < batch; ++b) {
      const int8_t* ar = a + (size_t)b * columns;
      for (size_t g = 0; g < groups; ++g) {
        int32_t dot = 0;
        for (unsigned i = 0; i < GROUP; ++i) dot += (int32_t)wr[g * GROUP + i] * ar[g * GROUP + i];
        partials[((size_t)b * rows + (size_t)n) * groups + g] = dot;
      }
    }
  }
}

/* acc = fmaf(float(dot), weight_scale * activation_scale, acc), groups in order
 * (lowbit_gemv.hip:540-551). */
void orc_gemm_epilogue(const int32_t* partials, const uint16_t* ws16, const uint16_t* as16,
                       size_t rows, size_t columns, unsigned batch, float* out) {
  const size_t groups = columns / GROUP;
#pragma omp parallel for schedule(static)
  for (long long n = 0; n < (long long)rows; ++n) {
    for (unsigned b = 0; b < batch; ++b) {
      float acc = 0.0f;
      for (size_t g = 0; g < groups; ++g) {
        const float scale = h2f(ws16[(size_t)n * groups + g]) * h2f(as16[(size_t)b * groups + g]);
        acc = fmaf((float)partials[((size_t)b * rows + (size_t)n) * groups + g], scale, acc);
      }
      out[(size_t)b * rows + (size_t)n] = acc;
    }
  }
}

/* The epilogue above with K cut into splits and ranges, the summation order of
 * gfxinfer_amd's GEMMs: split s of S owns groups [G s / S, G (s + 1) / S); a split
 * of n groups is cut into R = clamp(ceil(n / 10), 1, 16) ranges, range r holding
 * groups [b + n r / R, b + n (r + 1) / R); each range is the sequential epilogue
 * over its groups from 0, and plane s = ((range_0 + range_1) + range_2) + ...
 * With R = S = 1 this is orc_gemm_epilogue exactly.  out: fp32 [S, batch, rows]. */
static unsigned range_count(unsigned n) {
  unsigned r = (n + 9u) / 10u;
  return r < 1u ? 1u : (r > 16u ? 16u : r);
}

void orc_gemm_epilogue_ranges(const int32_t* partials, const uint16_t* ws16, const uint16_t* as16,
                              size_t rows, size_t columns, unsigned batch, unsigned splits, float* out) {
  const unsigned groups = (unsigned)(columns / GROUP);
#pragma omp parallel for schedule(static)
  for (long long n = 0; n < (long long)rows; ++n) {
    for (unsigned b = 0; b < batch; ++b) {
      const int32_t* p = partials + ((size_t)b * rows + (size_t)n) * groups;
      for (unsigned s = 0; s < splits; ++s) {
        const unsigned begin = groups * s / splits, count = groups * (s + 1u) / splits - begin;
        const unsigned ranges = range_count(count);
        float plane = 0.0f;
        for (unsigned r = 0; r < ranges; ++r) {
          float value = 0.0f;
          for (unsigned g = begin + count * r / ranges; g < begin + count * (r + 1u) / ranges; ++g) {
            const float scale = h2f(ws16[(size_t)n * groups + g]) * h2f(as16[(size_t)b * groups + g]);
            value = fmaf((float)p[g], scale, value);
          }
          plane = r == 0 ? value : plane + value;
        }
        out[((size_t)s * batch + b) * rows + (size_t)n] = plane;
      }
    }
  }
}

/* src/cli/main.cpp:1468-1495 over every row. */
void orc_dequant_dot_gemv(const int8_t* w, const float* ws, const int8_t* a, const uint16_t* as16,
                          size_t rows, size_t columns, unsigned batch, float* out) {
  const size_t groups = columns / GROUP;
#pragma omp parallel for schedule(static)
  for (long long n = 0; n < (long long)rows; ++n) {
    for (unsigned b = 0; b < batch; ++b) {
      float expected = 0.0f;
      for (size_t c = 0; c < columns; ++c) {
        const float weight = (float)w[(size_t)n * columns + c] * ws[(size_t)n * groups + c / GROUP];
        const float activation = (float)a[(size_t)b * columns + c] * h2f(as16[(size_t)b * groups + c / GROUP]);
        expected = fmaf(weight, activation, expected);
      }
      out[(size_t)b * rows + (size_t)n] = expected;
    }
  }
}

void orc_dequant_dot_gemv_packed(const uint8_t* codes, int format, const float* ws,
                                 const int8_t* a, const uint16_t* as16, size_t rows,
                                 size_t columns, unsigned batch, float* out) {
  const size_t groups = columns / GROUP;
  const size_t row_bytes = orc_packed_row_bytes(format, columns);
  float* as = (float*)malloc(sizeof(float) * batch * groups);
  for (size_t i = 0; i < (size_t)batch * groups; ++i) as[i] = h2f(as16[i]);
#pragma omp parallel for schedule(static)
  for (long long n = 0; n < (long long)rows; ++n) {
    const uint8_t* row = codes + (size_t)n * row_bytes;
    for (unsigned b = 0; b < batch; ++b) {
      float expected = 0.0f;
      for (size_t c = 0; c < columns; ++c) {
        const float weight = (float)orc_decode_value(orc_load_code(row, c, format), format) *
                             ws[(size_t)n * groups + c / GROUP];
        const float activation = (float)a[(size_t)b * columns + c] * as[(size_t)b * groups + c / GROUP];
        expected = fmaf(weight, activation, expected);
      }
      out[(size_t)b * rows + (size_t)n] = expected;
    }
  }
  free(as);
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Decoder ops: src/kernels/qwen_ops.hip                                      */
/* ------------------------------------------------------------------------ */

static float norm_scale(uint16_t w, int unit_offset) {
  float scale = orc_bf16_to_f32(w);
  if (unit_offset) scale += 1.0f;
  return scale;
}

/* qwen_ops.hip:31-63 */
/* Sum of squares of an fp16 row in the order of the reference's rms_norm kernel
 * (qwen_ops.hip:31-63, 256 threads of wave32): partial t = fmaf chain over elements
 * t, t + 256, ... in index order; each group of 32 partials reduced by the shfl_down
 * tree (lane l += lane l + d for d = 16, 8, 4, 2, 1); the eight group sums by the same
 * tree over lanes 0..7 (lanes 8..31 hold zeros).  The inverse RMS is then the correctly
 * rounded 1 / sqrtf; the reference's rsqrtf is the hardware approximation, within 1 ulp. */
static float reference_square_sum(const uint16_t* x, size_t n) {
  float partial[256];
  for (size_t t = 0; t < 256; ++t) {
    float s = 0.0f;
    for (size_t i = t; i < n; i += 256) s = fmaf(h2f(x[i]), h2f(x[i]), s);
    partial[t] = s;
  }
  float group[8];
  for (size_t g = 0; g < 8; ++g) {
    float* p = partial + 32 * g;
    for (size_t d = 16; d >= 1; d /= 2) {
      for (size_t l = 0; l < d; ++l) p[l] = p[l] + p[l + d];
    }
    group[g] = p[0];
  }
  return ((group[0] + group[4]) + (group[2] + group[6])) + ((group[1] + group[5]) + (group[3] + group[7]));
}

void orc_rms_norm(const uint16_t* in, const uint16_t* w, uint16_t* out, size_t n, unsigned batch,
                  float epsilon, int unit_offset) {
  for (unsigned b = 0; b < batch; ++b) {
    const uint16_t* x = in + (size_t)b * n;
    const float sum = reference_square_sum(x, n);
    const float inverse = 1.0f / sqrtf(sum / (float)n + epsilon);
    for (size_t i = 0; i < n; ++i) {
      out[(size_t)b * n + i] = f2h(h2f(x[i]) * inverse * norm_scale(w[i], unit_offset));
    }
  }
}

/* qwen_ops.hip:176-217 */
void orc_residual_add_rms_norm(const uint16_t* residual, const float* update, uint16_t* residual_out,
                               const uint16_t* w, uint16_t* normalized, size_t n, unsigned batch,
                               float epsilon, int unit_offset) {
  for (unsigned b = 0; b < batch; ++b) {
    const size_t base = (size_t)b * n;
    for (size_t i = 0; i < n; ++i) residual_out[base + i] = f2h(h2f(residual[base + i]) + update[base + i]);
    const float sum = reference_square_sum(residual_out + base, n);
    const float inverse = 1.0f / sqrtf(sum / (float)n + epsilon);
    for (size_t i = 0; i < n; ++i) {
      normalized[base + i] = f2h(h2f(residual_out[base + i]) * inverse * norm_scale(w[i], unit_offset));
    }
  }
}

/* qwen_ops.hip:65-106 */
void orc_dual_rms_norm_concat(const uint16_t* left, const uint16_t* left_w, const uint16_t* right,
                              const uint16_t* right_w, uint16_t* out, size_t n, float epsilon,
                              int unit_offset) {
  orc_rms_norm(left, left_w, out, n, 1, epsilon, unit_offset);
  orc_rms_norm(right, right_w, out + n, n, 1, epsilon, unit_offset);
}

static float silu(float x) { return x / (1.0f + expf(-x)); }

/* qwen_ops.hip:108-118 */
void orc_silu_multiply(const float* gate, const float* up, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = f2h(silu(gate[i]) * up[i]);
}

/* qwen_ops.hip:120-163: fp16(silu(g) * u), then the A4 quantizer of lowbit_gemv.hip:373-407. */
int orc_silu_multiply_quantize_i4(const float* gate, const float* up, uint8_t* packed,
                                  uint16_t* scales, size_t columns, unsigned batch) {
  if (columns == 0 || columns % GROUP != 0 || batch == 0 || batch > 32) {
    return ORC_INVALID_ARGUMENT;
  }
  uint16_t* product = (uint16_t*)malloc(sizeof(uint16_t) * columns * batch);
  orc_silu_multiply(gate, up, product, columns * batch);
  const int status = orc_quantize_activation_i4(product, packed, scales, columns, batch);
  free(product);
  return status;
}

/* qwen_ops.hip:219-261 */
void orc_gdn_conv_update(const float* projected, const uint16_t* w, const uint16_t* initial_state,
                         uint16_t* final_state, uint16_t* out, uint16_t* appended_log,
                         size_t channels, unsigned tokens) {
  for (size_t c = 0; c < channels; ++c) {
    uint16_t state[4];
    for (unsigned tap = 0; tap < 4; ++tap) state[tap] = initial_state[c * 4 + tap];
    for (unsigned t = 0; t < tokens; ++t) {
      state[0] = state[1];
      state[1] = state[2];
      state[2] = state[3];
      state[3] = f2h(projected[(size_t)t * channels + c]);
      if (appended_log) appended_log[(size_t)t * channels + c] = state[3];
      float convolution = 0.0f;
      for (unsigned tap = 0; tap < 4; ++tap) {
        convolution = fmaf(h2f(state[tap]), orc_bf16_to_f32(w[c * 4 + tap]), convolution);
      }
      out[(size_t)t * channels + c] = f2h(silu(convolution));
    }
    for (unsigned tap = 0; tap < 4; ++tap) final_state[c * 4 + tap] = state[tap];
  }
}

/* qwen_ops.hip:263-411 with the head counts as parameters.  The reference hard
 * codes 48 value heads, 16 key heads, d = 128 and the query scale 1/sqrt(128). */
void orc_gdn_recurrent(const uint16_t* qkv, const float* z, const float* a, const float* b,
                       const uint16_t* a_log, const uint16_t* dt_bias, const uint16_t* norm_w,
                       const float* initial_states, float* final_states, uint16_t* out,
                       float* key_log, float* delta_log, float* decay_log, unsigned tokens,
                       unsigned key_heads, unsigned value_heads, unsigned d) {
  const size_t key_elements = (size_t)key_heads * d;
  const size_t value_elements = (size_t)value_heads * d;
  const size_t qkv_stride = 2 * key_elements + value_elements;
  const unsigned ratio = value_heads / key_heads;
  const float query_scale = (float)(1.0 / sqrt((double)d));
  float* query = (float*)malloc(sizeof(float) * d);
  float* key = (float*)malloc(sizeof(float) * d);
  float* delta = (float*)malloc(sizeof(float) * d);
  float* mixed = (float*)malloc(sizeof(float) * d);
  for (unsigned h = 0; h < value_heads; ++h) {
    const unsigned kh = h / ratio;
    const float* initial = initial_states + (size_t)h * d * d;
    float* state = final_states + (size_t)h * d * d;
    for (unsigned t = 0; t < tokens; ++t) {
      const uint16_t* tq = qkv + (size_t)t * qkv_stride;
      float qs = 0.0f, ks = 0.0f;
      for (unsigned i = 0; i < d; ++i) {
        query[i] = h2f(tq[kh * d + i]);
        key[i] = h2f(tq[key_elements + kh * d + i]);
        qs += query[i] * query[i];
        ks += key[i] * key[i];
      }
      const float inverse_query = (1.0f / sqrtf(qs + 1.0e-6f)) * query_scale;
      const float inverse_key = 1.0f / sqrtf(ks + 1.0e-6f);
      const float a_value = a[(size_t)t * value_heads + h] + orc_bf16_to_f32(dt_bias[h]);
      const float softplus = a_value > 20.0f ? a_value : log1pf(expf(a_value));
      const float g = -expf(orc_bf16_to_f32(a_log[h])) * softplus;
      const float decay = expf(g);
      const float beta = 1.0f / (1.0f + expf(-b[(size_t)t * value_heads + h]));
      for (unsigned i = 0; i < d; ++i) {
        query[i] *= inverse_query;
        key[i] *= inverse_key;
      }
      if (decay_log) decay_log[(size_t)t * value_heads + h] = decay;
      if (key_log && h % ratio == 0) {
        for (unsigned i = 0; i < d; ++i) key_log[(size_t)t * key_elements + kh * d + i] = key[i];
      }
      for (size_t i = 0; i < (size_t)d * d; ++i) {
        const float previous = t == 0 ? initial[i] : state[i];
        state[i] = previous * decay;
      }
      for (unsigned v = 0; v < d; ++v) {
        float memory = 0.0f;
        for (unsigned k = 0; k < d; ++k) memory = fmaf(state[(size_t)k * d + v], key[k], memory);
        const float value = h2f(tq[2 * key_elements + (size_t)h * d + v]);
        delta[v] = (value - memory) * beta;
        if (delta_log) delta_log[(size_t)t * value_elements + (size_t)h * d + v] = delta[v];
      }
      for (unsigned k = 0; k < d; ++k) {
        for (unsigned v = 0; v < d; ++v) {
          state[(size_t)k * d + v] = fmaf(key[k], delta[v], state[(size_t)k * d + v]);
        }
      }
      float os = 0.0f;
      for (unsigned v = 0; v < d; ++v) {
        float value = 0.0f;
        for (unsigned k = 0; k < d; ++k) value = fmaf(state[(size_t)k * d + v], query[k], value);
        mixed[v] = value;
        os += value * value;
      }
      const float inverse_out = 1.0f / sqrtf(os / (float)d + 1.0e-6f);
      for (unsigned v = 0; v < d; ++v) {
        const size_t index = (size_t)h * d + v;
        const float gate = silu(z[(size_t)t * value_elements + index]);
        const float normalized = mixed[v] * inverse_out * orc_bf16_to_f32(norm_w[v]);
        out[(size_t)t * value_elements + index] = f2h(normalized * gate);
      }
    }
    if (tokens == 0) memcpy(state, initial, sizeof(float) * d * d);
  }
  free(query);
  free(key);
  free(delta);
  free(mixed);
}

/* qwen_ops.hip:413-429 */
void orc_gdn_restore_conv(uint16_t* state, const uint16_t* appended_log, size_t channels,
                          unsigned accepted) {
  for (size_t c = 0; c < channels; ++c) {
    for (unsigned t = 0; t < accepted; ++t) {
      state[c * 4 + 0] = state[c * 4 + 1];
      state[c * 4 + 1] = state[c * 4 + 2];
      state[c * 4 + 2] = state[c * 4 + 3];
      state[c * 4 + 3] = appended_log[(size_t)t * channels + c];
    }
  }
}

/* qwen_ops.hip:431-465 */
void orc_gdn_restore_recurrent(float* states, const float* key_log, const float* delta_log,
                               const float* decay_log, unsigned accepted, unsigned key_heads,
                               unsigned value_heads, unsigned d) {
  const size_t key_elements = (size_t)key_heads * d;
  const size_t value_elements = (size_t)value_heads * d;
  const unsigned ratio = value_heads / key_heads;
  for (unsigned h = 0; h < value_heads; ++h) {
    float* state = states + (size_t)h * d * d;
    const unsigned kh = h / ratio;
    for (unsigned t = 0; t < accepted; ++t) {
      const float decay = decay_log[(size_t)t * value_heads + h];
      for (size_t i = 0; i < (size_t)d * d; ++i) state[i] *= decay;
      for (unsigned k = 0; k < d; ++k) {
        const float key = key_log[(size_t)t * key_elements + (size_t)kh * d + k];
        for (unsigned v = 0; v < d; ++v) {
          state[(size_t)k * d + v] =
              fmaf(key, delta_log[(size_t)t * value_elements + (size_t)h * d + v],
                   state[(size_t)k * d + v]);
        }
      }
    }
  }
}

/* qwen_ops.hip:599-676 */
void orc_head_norm_rope(const float* input, size_t input_stride, const uint16_t* w,
                        uint16_t* out, size_t head_count, size_t head_size, size_t rotary,
                        uint64_t base_position, unsigned tokens, float theta) {
  float* normalized = (float*)malloc(sizeof(float) * head_size);
  for (unsigned t = 0; t < tokens; ++t) {
    const uint64_t position = base_position + t;
    for (size_t h = 0; h < head_count; ++h) {
      const float* x = input + (size_t)t * head_count * input_stride + h * input_stride;
      float sum = 0.0f;
      for (size_t i = 0; i < head_size; ++i) {
        normalized[i] = x[i];
        sum += x[i] * x[i];
      }
      const float inverse = 1.0f / sqrtf(sum / (float)head_size + 1.0e-6f);
      for (size_t i = 0; i < head_size; ++i) {
        normalized[i] *= inverse * (1.0f + orc_bf16_to_f32(w[i]));
      }
      for (size_t i = 0; i < head_size; ++i) {
        float value = normalized[i];
        if (i < rotary) {
          const size_t half = rotary / 2;
          const size_t fi = i % half;
          const float exponent = (2.0f * (float)fi) / (float)rotary;
          const float inverse_frequency = powf(theta, -exponent);
          const float angle = (float)position * inverse_frequency;
          const float partner = normalized[i < half ? i + half : i - half];
          const float rotated = i < half ? -partner : partner;
          value = fmaf(value, cosf(angle), rotated * sinf(angle));
        }
        out[(size_t)t * head_count * head_size + h * head_size + i] = f2h(value);
      }
    }
  }
  free(normalized);
}

/* qwen_ops.hip:678-696 */
void orc_kv_append(const uint16_t* key, const float* value, uint16_t* key_cache,
                   uint16_t* value_cache, size_t position, size_t kv_elements, unsigned tokens) {
  for (unsigned t = 0; t < tokens; ++t) {
    for (size_t i = 0; i < kv_elements; ++i) {
      key_cache[(position + t) * kv_elements + i] = key[(size_t)t * kv_elements + i];
      value_cache[(position + t) * kv_elements + i] = f2h(value[(size_t)t * kv_elements + i]);
    }
  }
}

/* qwen_ops.hip:698-766.  Token t attends to base_token_count + t cached positions;
 * the gate is the second half of each head's 2*hd query-projection row. */
void orc_gated_attention(const uint16_t* query, const float* gate_src, const uint16_t* key_cache,
                         const uint16_t* value_cache, uint16_t* out, size_t base_token_count,
                         unsigned tokens, unsigned q_heads, unsigned kv_heads, unsigned hd,
                         float score_scale) {
  const unsigned group = q_heads / kv_heads;
  float* accumulator = (float*)malloc(sizeof(float) * hd);
  for (unsigned t = 0; t < tokens; ++t) {
    const size_t count = base_token_count + t;
    for (unsigned qh = 0; qh < q_heads; ++qh) {
      const unsigned kvh = qh / group;
      const uint16_t* q = query + ((size_t)t * q_heads + qh) * hd;
      float maximum = -INFINITY, denominator = 0.0f;
      for (unsigned i = 0; i < hd; ++i) accumulator[i] = 0.0f;
      for (size_t p = 0; p < count; ++p) {
        const uint16_t* k = key_cache + (p * kv_heads + kvh) * hd;
        const uint16_t* v = value_cache + (p * kv_heads + kvh) * hd;
        float score = 0.0f;
        for (unsigned i = 0; i < hd; ++i) score += h2f(q[i]) * h2f(k[i]);
        score *= score_scale;
        const float next = fmaxf(maximum, score);
        const float alpha = expf(maximum - next);
        const float beta = expf(score - next);
        denominator = denominator * alpha + beta;
        maximum = next;
        for (unsigned i = 0; i < hd; ++i) accumulator[i] = accumulator[i] * alpha + h2f(v[i]) * beta;
      }
      for (unsigned i = 0; i < hd; ++i) {
        const float gate = gate_src[(size_t)t * q_heads * hd * 2 + (size_t)qh * hd * 2 + hd + i];
        const float gate_scale = 1.0f / (1.0f + expf(-gate));
        out[((size_t)t * q_heads + qh) * hd + i] = f2h(accumulator[i] / denominator * gate_scale);
      }
    }
  }
  free(accumulator);
}

/* qwen_ops.hip:768-807 */
void orc_argmax(const float* logits, size_t vocabulary, size_t stride, unsigned rows,
                const uint32_t* token_ids, uint32_t* out) {
  for (unsigned r = 0; r < rows; ++r) {
    const float* row = logits + (size_t)r * stride;
    float maximum = -INFINITY;
    uint32_t index = 0;
    for (size_t i = 0; i < vocabulary; ++i) {
      if (row[i] > maximum) {
        maximum = row[i];
        index = (uint32_t)i;
      }
    }
    out[r] = token_ids ? token_ids[index] : index;
  }
}

/* qwen_runtime.cpp:1497-1501 */
size_t orc_accept(const uint32_t* drafts, const uint32_t* targets, size_t draft_count) {
  size_t accepted = 0;
  while (accepted < draft_count && drafts[accepted] == targets[accepted]) ++accepted;
  return accepted;
}

/* Synthetic checkpoint values (the generator of gfxinfer_model_create_synthetic, restated
 * in oracle.py's synthetic_values): element i of a tensor with generator key `key` is
 * mean + n_i * (sigma * 2^-16) in fp32, n_i = the twelve 16-bit fields of
 * splitmix64(key + 3 i + j), j = 0..2, summed, plus 6 - 6 * 65536. */
static uint64_t orc_splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void orc_synthetic_values(uint64_t seed_xor_name_hash, size_t first, size_t count, float sigma,
                          float mean, float* out) {
  const uint64_t key = orc_splitmix64(seed_xor_name_hash);
  const float scale = sigma * 0x1p-16f;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)count; ++i) {
    const uint64_t index = (uint64_t)first + (uint64_t)i;
    int64_t total = 0;
    for (uint64_t j = 0; j < 3; ++j) {
      const uint64_t h = orc_splitmix64(key + 3u * index + j);
      total += (int64_t)(h & 0xFFFF) + (int64_t)((h >> 16) & 0xFFFF) + (int64_t)((h >> 32) & 0xFFFF) +
               (int64_t)(h >> 48);
    }
    const float n = (float)(total + 6 - 6 * 65536);
    const float spread = n * scale;
    out[i] = mean + spread;
  }
}
