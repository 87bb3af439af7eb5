// C entry points over the reference's own src/quantization.cpp, compiled from
// where it lies under the reference tree by oracle/Makefile into oracle/_ref/.
// TEST INFRASTRUCTURE ONLY: used to write and re-check the golden fixtures that
// pin the oracle's quantizer restatement.  Nothing here is shipped.
#include <cstring>
#include <span>

#include "gfxinfer/quantization.h"

extern "C" {

std::size_t ref_packed_row_bytes(int format, std::size_t columns) {
  return gfxinfer::packed_row_bytes(static_cast<gfxinfer::Quantization>(format), columns);
}

// quantization.cpp:163-220.  Returns the reference ErrorCode value.
int ref_quantize_group128(const float* weights, std::size_t rows, std::size_t columns,
                          int format, std::uint8_t* codes, float* scales) {
  auto result = gfxinfer::quantize_group128(
      std::span<const float>(weights, rows * columns), rows, columns,
      static_cast<gfxinfer::Quantization>(format));
  if (!result.ok()) return static_cast<int>(result.status().code());
  const auto& packed = result.value();
  std::memcpy(codes, packed.codes.data(), packed.codes.size());
  std::memcpy(scales, packed.scales.data(), packed.scales.size() * sizeof(float));
  return 0;
}

// quantization.cpp:237-251 on a packed matrix rebuilt from caller storage.
int ref_dequantize_group128(const std::uint8_t* codes, const float* scales, std::size_t rows,
                            std::size_t columns, int format, float* out) {
  gfxinfer::PackedMatrix matrix;
  matrix.rows = rows;
  matrix.columns = columns;
  matrix.format = static_cast<gfxinfer::Quantization>(format);
  const auto row_bytes = gfxinfer::packed_row_bytes(matrix.format, columns);
  matrix.codes.assign(codes, codes + rows * row_bytes);
  matrix.scales.assign(scales, scales + rows * (columns / 128));
  auto result = gfxinfer::dequantize_group128(matrix);
  if (!result.ok()) return static_cast<int>(result.status().code());
  std::memcpy(out, result.value().data(), result.value().size() * sizeof(float));
  return 0;
}

}  // extern "C"
