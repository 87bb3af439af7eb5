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

// ---- artifacts: the reference's own tiler, writer and reader (artifact.cpp,
// quantization.cpp:253-318), used to write the .gfxi fixtures the library must load and
// to check that the library's artifacts open in the reference reader. ----
#include <filesystem>
#include <string>
#include <vector>

#include "gfxinfer/artifact.h"

extern "C" {

// tile_group128_for_gfx12 on caller storage: codes (packed) + float scales in, gfx12
// tiled codes + float scales out.
int ref_tile_group128_for_gfx12(const std::uint8_t* codes, const float* scales, std::size_t rows,
                                std::size_t columns, int format, std::uint8_t* out_codes,
                                float* out_scales) {
  gfxinfer::PackedMatrix matrix;
  matrix.rows = rows;
  matrix.columns = columns;
  matrix.format = static_cast<gfxinfer::Quantization>(format);
  const auto row_bytes = gfxinfer::packed_row_bytes(matrix.format, columns);
  matrix.codes.assign(codes, codes + rows * row_bytes);
  matrix.scales.assign(scales, scales + rows * (columns / 128));
  auto tiled = gfxinfer::tile_group128_for_gfx12(matrix);
  if (!tiled.ok()) return static_cast<int>(tiled.status().code());
  std::memcpy(out_codes, tiled.value().codes.data(), tiled.value().codes.size());
  std::memcpy(out_scales, tiled.value().scales.data(), tiled.value().scales.size() * sizeof(float));
  return 0;
}

// ArtifactWriter::write with identity (arch, model, weights, recipe) and `count`
// tensors described by parallel arrays (dims: 4 per tensor).
int ref_write_artifact(const char* path, const char* arch, const char* model, const char* weights,
                       const char* recipe, std::size_t count, const char* const* names,
                       const int* dtypes, const int* quantizations, const int* ranks,
                       const std::uint64_t* dims, const void* const* data,
                       const std::uint64_t* data_bytes, const void* const* aux,
                       const std::uint64_t* aux_bytes) {
  std::vector<gfxinfer::TensorWriteRequest> requests(count);
  for (std::size_t i = 0; i < count; ++i) {
    auto& r = requests[i];
    r.name = names[i];
    r.dtype = static_cast<gfxinfer::DType>(dtypes[i]);
    r.quantization = static_cast<gfxinfer::Quantization>(quantizations[i]);
    r.dimensions.assign(dims + 4 * i, dims + 4 * i + ranks[i]);
    r.data = {static_cast<const std::byte*>(data[i]), static_cast<std::size_t>(data_bytes[i])};
    if (aux_bytes[i] != 0) {
      r.auxiliary = {static_cast<const std::byte*>(aux[i]), static_cast<std::size_t>(aux_bytes[i])};
    }
  }
  const gfxinfer::ArtifactIdentity identity{arch, model, weights, recipe};
  const auto status = gfxinfer::ArtifactWriter::write(path, identity, requests);
  return status.ok() ? 0 : static_cast<int>(status.code());
}

// ArtifactView::open: status code, and the tensor count through *tensors.
int ref_open_artifact(const char* path, int verify, std::size_t* tensors) {
  auto view = gfxinfer::ArtifactView::open(path, {.verify_checksums = verify != 0});
  if (!view.ok()) return static_cast<int>(view.status().code());
  *tensors = view.value().tensors().size();
  return 0;
}

std::uint64_t ref_crc64_ecma(const void* bytes, std::size_t count) {
  return gfxinfer::crc64_ecma({static_cast<const std::byte*>(bytes), count});
}

}  // extern "C"
