// Status/error plumbing, the gfx950 device gate and the host-side tile layout
// conversion of the C ABI.
#include "common.hpp"

#include <cstring>
#include <string>

namespace gfx950 {
namespace {
thread_local std::string g_last_error;
}

int32_t fail(int32_t code, const std::string& message) {
  g_last_error = message;
  return code;
}

int32_t ok() { return GFXI_OK; }

int32_t hip_fail(hipError_t error, const char* context) {
  return fail(GFXI_HIP_ERROR, std::string(context) + ": " + hipGetErrorString(error));
}

int32_t launch_status(const char* context) {
  const hipError_t error = hipGetLastError();
  if (error != hipSuccess) return hip_fail(error, context);
  return GFXI_OK;
}

namespace {

// Reference packed storage (src/quantization.cpp:94-150): W2 is four codes per byte
// from the low bits, W3 groups are three 16-byte bit planes, W4 is two codes per
// byte with the even column low.
int reference_packed_weight(int32_t format, const uint8_t* row, std::size_t column) {
  if (format == GFXI_W2G128) {
    const unsigned code = (row[column / 4] >> ((column & 3u) * 2u)) & 3u;
    return 2 * static_cast<int>(code) - 3;  // quantization.cpp:50
  }
  if (format == GFXI_W3G128) {
    const std::size_t group = column / kGroup, local = column % kGroup;
    unsigned code = 0;
    for (unsigned plane = 0; plane < 3; ++plane) {
      code |= ((row[group * 48 + plane * 16 + local / 8] >> (local & 7u)) & 1u) << plane;
    }
    return static_cast<int>(code) - 4;  // quantization.cpp:51
  }
  const unsigned code = (row[column / 2] >> ((column & 1u) * 4u)) & 0x0fu;
  return code >= 8u ? static_cast<int>(code) - 16 : static_cast<int>(code);  // :52-53
}

}  // namespace
}  // namespace gfx950

using namespace gfx950;

extern "C" const char* gfxinfer_last_error(void) { return g_last_error.c_str(); }

extern "C" int32_t gfxinfer_require_gfx950_device(int32_t device) {
  int count = 0;
  if (const hipError_t error = hipGetDeviceCount(&count); error != hipSuccess) {
    return hip_fail(error, "device enumeration failed");
  }
  if (device < 0 || device >= count) {
    return fail(GFXI_INVALID_ARGUMENT, "device index " + std::to_string(device) + " is out of range");
  }
  hipDeviceProp_t properties{};
  if (const hipError_t error = hipGetDeviceProperties(&properties, device); error != hipSuccess) {
    return hip_fail(error, "device properties query failed");
  }
  const std::string arch = properties.gcnArchName;
  if (arch.rfind("gfx950", 0) != 0 || properties.warpSize != 64) {
    return fail(GFXI_UNSUPPORTED, "gfxinfer_amd requires a gfx950 (MI355X) device with 64-wide "
                                  "waves; found " + arch);
  }
  return GFXI_OK;
}

extern "C" size_t gfxinfer_packed_row_bytes(int32_t format, size_t columns) {
  switch (format) {  // quantization.cpp:154-161
    case GFXI_W2G128: return (columns + 3) / 4;
    case GFXI_W3G128: return (columns * 3 + 7) / 8;
    case GFXI_W4G128: return (columns + 1) / 2;
    default: return 0;
  }
}

extern "C" int32_t gfxinfer_tile_group128_for_gfx950(int32_t format, const uint8_t* packed_codes,
                                                     const float* scales, size_t rows,
                                                     size_t columns, uint8_t* tiled_codes,
                                                     uint16_t* tiled_scales_f16) {
  if (!valid_weight_format(format)) {
    return fail(GFXI_UNSUPPORTED, "gfx950 tiling supports W2G128, W3G128 and W4G128");
  }
  if (packed_codes == nullptr || scales == nullptr || tiled_codes == nullptr ||
      tiled_scales_f16 == nullptr || rows == 0 || rows % 16 != 0 || columns == 0 ||
      columns % kGroup != 0) {
    return fail(GFXI_INVALID_ARGUMENT, "gfx950 tiling requires valid storage, N divisible by 16, "
                                       "and K divisible by 128");
  }
  const std::size_t row_bytes = gfxinfer_packed_row_bytes(format, columns);
  const std::size_t groups = columns / kGroup;
  const unsigned lb = lane_bytes(format);
#pragma omp parallel for schedule(static)
  for (long long signed_row = 0; signed_row < static_cast<long long>(rows); ++signed_row) {
    const std::size_t row = static_cast<std::size_t>(signed_row);
    const uint8_t* source = packed_codes + row * row_bytes;
    int8_t chunk[32];
    for (std::size_t group = 0; group < groups; ++group) {
      for (std::size_t kb = 0; kb < 4; ++kb) {
        for (unsigned c = 0; c < 32; ++c) {
          chunk[c] = static_cast<int8_t>(
              reference_packed_weight(format, source, group * kGroup + kb * 32 + c));
        }
        pack_lane_chunk(format, chunk,
                        tiled_codes + chunk_offset(format, row, group * kGroup + kb * 32, groups));
      }
      const __half scale = __float2half(scales[row * groups + group]);
      std::memcpy(tiled_scales_f16 + scale_offset(row, group, groups), &scale, sizeof scale);
    }
  }
  (void)lb;
  return GFXI_OK;
}

extern "C" int32_t gfxinfer_untile_group128_for_gfx950(int32_t format, const uint8_t* tiled_codes,
                                                       const uint16_t* tiled_scales_f16,
                                                       size_t rows, size_t columns,
                                                       int8_t* weights, uint16_t* scales_f16) {
  if (!valid_weight_format(format)) {
    return fail(GFXI_UNSUPPORTED, "gfx950 layout supports W2G128, W3G128 and W4G128");
  }
  if (tiled_codes == nullptr || weights == nullptr || rows == 0 || rows % 16 != 0 ||
      columns == 0 || columns % kGroup != 0) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid gfx950 untile arguments");
  }
  const std::size_t groups = columns / kGroup;
#pragma omp parallel for schedule(static)
  for (long long signed_row = 0; signed_row < static_cast<long long>(rows); ++signed_row) {
    const std::size_t row = static_cast<std::size_t>(signed_row);
    for (std::size_t column = 0; column < columns; column += 32) {
      const uint8_t* chunk = tiled_codes + chunk_offset(format, row, column, groups);
      for (unsigned c = 0; c < 32; ++c) {
        weights[row * columns + column + c] =
            static_cast<int8_t>(unpack_lane_code(format, chunk, c));
      }
    }
    if (scales_f16 != nullptr && tiled_scales_f16 != nullptr) {
      for (std::size_t group = 0; group < groups; ++group) {
        scales_f16[row * groups + group] = tiled_scales_f16[scale_offset(row, group, groups)];
      }
    }
  }
  return GFXI_OK;
}
