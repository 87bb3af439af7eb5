// .gfxi artifacts: reader, loader into the gfx950 weight arena, and writer.
//
// File format (the reference's own, src/artifact.cpp:22-67, so that artifacts move
// between the two engines): a 256-byte header, a directory of 128-byte tensor
// entries, the tensor-name string table, then payloads, each 256-byte (or more)
// aligned.  CRC-64/ECMA-182 (polynomial 0x42F0E1EBA9EA3693, MSB first, zero initial
// value, no final xor) covers the directory + names and every tensor's data.
//
// Recipes.  target_arch "gfx1200" is the reference converter's output
// (converter.cpp:345-393): codes in the gfx12 tile order [16-row tile][group][32-column
// K-step][row][fragment] and fp16 scales [tile][group][16].  That fragment order is the
// gfx950 lane order (lane = K-step * 16 + row), and W4 fragments are the same nibble
// bytes, so only W3 and W2 fragments differ: the gfx12 recipe packs the 32 codes of a
// W3 fragment sequentially (3 bits each, least significant first, code = value + 4)
// and keeps W2 fragments as the packed row bytes (four 2-bit codes per byte, lowest
// column first, code = (value + 3) / 2); the gfx950 layout re-packs both so that each
// MFMA operand register expands with one shift and mask.  target_arch "gfx950" artifacts (written here) hold the gfx950
// layout and load as plain copies.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cstring>
#include <memory>
#include <set>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "common.hpp"
#include "runtime.hpp"

namespace gfx950 {
namespace {

constexpr unsigned char kMagic[8] = {'G', 'F', 'X', 'I', '\r', '\n', 0x1a, '\n'};
constexpr uint32_t kFormatVersion = 1;  // version.h:11 kArtifactVersion
constexpr uint32_t kEndianTag = 0x01020304u;
constexpr uint64_t kFileAlignment = 256;

// On-disk structs (artifact.cpp:26-67 field order and widths).
#pragma pack(push, 1)
struct DiskHeader {
  unsigned char magic[8];
  uint32_t version;
  uint32_t header_bytes;
  uint32_t endian_tag;
  uint32_t flags;
  uint64_t directory_offset;
  uint32_t tensor_count;
  uint32_t directory_entry_bytes;
  uint64_t strings_offset;
  uint64_t strings_bytes;
  uint64_t data_offset;
  uint64_t data_bytes;
  uint64_t file_bytes;
  uint64_t manifest_crc64;
  char target_arch[16];
  char model_id[32];
  char weights_id[32];
  char recipe_id[64];
  uint8_t reserved[24];
};

struct DiskEntry {
  uint64_t name_offset;
  uint32_t name_bytes;
  uint16_t dtype;
  uint16_t quantization;
  uint16_t rank;
  uint16_t flags;
  uint32_t alignment;
  uint64_t dimensions[4];
  uint64_t data_offset;
  uint64_t data_bytes;
  uint64_t aux_offset;
  uint64_t aux_bytes;
  uint64_t data_crc64;
  uint8_t reserved[32];
};
#pragma pack(pop)
static_assert(sizeof(DiskHeader) == 256, "header is 256 bytes");
static_assert(sizeof(DiskEntry) == 128, "directory entries are 128 bytes");

// DType values (artifact.h:19-25).
constexpr uint16_t kDtypeU8 = 1, kDtypeI32 = 2, kDtypeBf16 = 4, kDtypeF32 = 5;

struct CrcTable {
  uint64_t t[8][256];
  CrcTable() {
    constexpr uint64_t poly = 0x42F0E1EBA9EA3693ull;
    for (unsigned i = 0; i < 256; ++i) {
      uint64_t v = static_cast<uint64_t>(i) << 56;
      for (int b = 0; b < 8; ++b) v = (v >> 63) ? (v << 1) ^ poly : v << 1;
      t[0][i] = v;
    }
    // t[k][i]: CRC of byte i followed by k zero bytes (slice-by-8 tables).
    for (unsigned i = 0; i < 256; ++i) {
      for (int k = 1; k < 8; ++k) t[k][i] = (t[k - 1][i] << 8) ^ t[0][t[k - 1][i] >> 56];
    }
  }
};
const CrcTable& crc_table() {
  static const CrcTable table;
  return table;
}

uint64_t crc64_update(uint64_t crc, const uint8_t* p, std::size_t n) {
  const auto& T = crc_table().t;
  while (n >= 8) {
    uint64_t w = crc ^ (static_cast<uint64_t>(p[0]) << 56 | static_cast<uint64_t>(p[1]) << 48 |
                        static_cast<uint64_t>(p[2]) << 40 | static_cast<uint64_t>(p[3]) << 32 |
                        static_cast<uint64_t>(p[4]) << 24 | static_cast<uint64_t>(p[5]) << 16 |
                        static_cast<uint64_t>(p[6]) << 8 | static_cast<uint64_t>(p[7]));
    crc = T[7][w >> 56] ^ T[6][(w >> 48) & 0xff] ^ T[5][(w >> 40) & 0xff] ^ T[4][(w >> 32) & 0xff] ^
          T[3][(w >> 24) & 0xff] ^ T[2][(w >> 16) & 0xff] ^ T[1][(w >> 8) & 0xff] ^ T[0][w & 0xff];
    p += 8;
    n -= 8;
  }
  while (n-- != 0) crc = T[0][(crc >> 56) ^ *p++] ^ (crc << 8);
  return crc;
}

bool in_file(uint64_t offset, uint64_t bytes, uint64_t file_bytes) {
  return offset <= file_bytes && bytes <= file_bytes - offset;
}

// Tensor names: [A-Za-z0-9_.-/], not absolute, no "..".
bool valid_name(const std::string& name) {
  if (name.empty() || name.front() == '/' || name.find("..") != std::string::npos) return false;
  return std::all_of(name.begin(), name.end(), [](unsigned char c) {
    return std::isalnum(c) != 0 || c == '_' || c == '-' || c == '.' || c == '/';
  });
}

template <std::size_t N>
std::string fixed(const char (&field)[N]) {
  return std::string(field, strnlen(field, N));
}

template <std::size_t N>
bool put_fixed(char (&field)[N], const std::string& value) {
  if (value.empty() || value.size() >= N) return false;
  std::memset(field, 0, N);
  std::memcpy(field, value.data(), value.size());
  return true;
}

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

}  // namespace
}  // namespace gfx950

using namespace gfx950;

struct gfxinfer_artifact {
  int fd{-1};
  const uint8_t* map{nullptr};
  std::size_t bytes{0};
  gfxinfer_artifact_identity identity{};
  std::vector<std::string> names;
  std::vector<gfxinfer_artifact_tensor> tensors;
  std::unordered_map<std::string, std::size_t> index;

  ~gfxinfer_artifact() {
    if (map != nullptr) ::munmap(const_cast<uint8_t*>(map), bytes);
    if (fd >= 0) ::close(fd);
  }
};

extern "C" uint64_t gfxinfer_crc64_ecma(uint64_t state, const void* bytes, size_t count) {
  return bytes == nullptr ? state : crc64_update(state, static_cast<const uint8_t*>(bytes), count);
}

// ArtifactView::open (artifact.cpp:264-411): the same structural checks, in the same
// spirit (a file that fails one is rejected before any payload is used).
extern "C" int32_t gfxinfer_artifact_open(const char* path, int32_t verify_checksums,
                                          gfxinfer_artifact** out) {
  return guarded([&]() -> int32_t {
    if (path == nullptr || out == nullptr) {
      return fail(GFXI_INVALID_ARGUMENT, "artifact open needs a path and an output handle");
    }
    *out = nullptr;
    auto a = std::make_unique<gfxinfer_artifact>();
    a->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (a->fd < 0) return fail(GFXI_IO_ERROR, std::string("cannot open ") + path + ": " + std::strerror(errno));
    struct stat st {};
    if (::fstat(a->fd, &st) != 0) {
      return fail(GFXI_IO_ERROR, std::string("cannot stat ") + path + ": " + std::strerror(errno));
    }
    if (st.st_size < static_cast<off_t>(sizeof(DiskHeader))) {
      return fail(GFXI_CORRUPT_ARTIFACT, "file too short to hold a .gfxi header");
    }
    a->bytes = static_cast<std::size_t>(st.st_size);
    void* m = ::mmap(nullptr, a->bytes, PROT_READ, MAP_PRIVATE, a->fd, 0);
    if (m == MAP_FAILED) {
      return fail(GFXI_IO_ERROR, std::string("cannot map ") + path + ": " + std::strerror(errno));
    }
    a->map = static_cast<const uint8_t*>(m);

    DiskHeader h;
    std::memcpy(&h, a->map, sizeof h);
    if (std::memcmp(h.magic, kMagic, sizeof kMagic) != 0) {
      return fail(GFXI_CORRUPT_ARTIFACT, "not a .gfxi file (first eight bytes differ)");
    }
    if (h.version != kFormatVersion || h.header_bytes != sizeof(DiskHeader)) {
      return fail(GFXI_UNSUPPORTED, "format version or header size this reader does not know");
    }
    if (h.endian_tag != kEndianTag) return fail(GFXI_UNSUPPORTED, "file written with the other byte order");
    if (h.directory_entry_bytes != sizeof(DiskEntry)) {
      return fail(GFXI_CORRUPT_ARTIFACT, "directory entries are not 128 bytes");
    }
    if (h.file_bytes != a->bytes) return fail(GFXI_CORRUPT_ARTIFACT, "file size differs from the size the header records");
    const uint64_t directory_bytes = static_cast<uint64_t>(h.tensor_count) * sizeof(DiskEntry);
    if (!in_file(h.directory_offset, directory_bytes, h.file_bytes) ||
        !in_file(h.strings_offset, h.strings_bytes, h.file_bytes) ||
        !in_file(h.data_offset, h.data_bytes, h.file_bytes) ||
        h.strings_offset != h.directory_offset + directory_bytes ||
        h.data_offset < h.strings_offset + h.strings_bytes) {
      return fail(GFXI_CORRUPT_ARTIFACT, "directory, name table or payload area lies outside the file or out of order");
    }
    if (verify_checksums != 0 &&
        crc64_update(0, a->map + h.directory_offset, directory_bytes + h.strings_bytes) !=
            h.manifest_crc64) {
      return fail(GFXI_CORRUPT_ARTIFACT, "CRC-64 of directory and names differs from the header");
    }
    const std::string arch = fixed(h.target_arch), model = fixed(h.model_id),
                      weights = fixed(h.weights_id), recipe = fixed(h.recipe_id);
    if (arch.empty() || model.empty() || weights.empty() || recipe.empty()) {
      return fail(GFXI_CORRUPT_ARTIFACT, "target, model, weights or recipe id is empty");
    }
    std::memcpy(a->identity.target_arch, h.target_arch, sizeof h.target_arch);
    std::memcpy(a->identity.model_id, h.model_id, sizeof h.model_id);
    std::memcpy(a->identity.weights_id, h.weights_id, sizeof h.weights_id);
    std::memcpy(a->identity.recipe_id, h.recipe_id, sizeof h.recipe_id);

    const char* strings = reinterpret_cast<const char*>(a->map + h.strings_offset);
    std::vector<std::pair<uint64_t, uint64_t>> ranges;
    a->names.reserve(h.tensor_count);
    a->tensors.reserve(h.tensor_count);
    for (uint32_t i = 0; i < h.tensor_count; ++i) {
      DiskEntry e;
      std::memcpy(&e, a->map + h.directory_offset + static_cast<uint64_t>(i) * sizeof(DiskEntry), sizeof e);
      if (e.rank > 4 || e.dtype < kDtypeU8 || e.dtype > kDtypeF32 || e.quantization > 5 ||
          e.name_bytes == 0 || !in_file(e.name_offset, e.name_bytes, h.strings_bytes)) {
        return fail(GFXI_CORRUPT_ARTIFACT, "directory entry has an impossible rank, dtype, quantization or name span");
      }
      std::string name(strings + e.name_offset, e.name_bytes);
      if (!valid_name(name) || a->index.count(name) != 0) {
        return fail(GFXI_CORRUPT_ARTIFACT, "tensor name empty, malformed or repeated: " + name);
      }
      if (e.alignment < kFileAlignment || (e.alignment & (e.alignment - 1)) != 0 ||
          e.data_offset % e.alignment != 0 || !in_file(e.data_offset, e.data_bytes, h.file_bytes) ||
          e.data_offset < h.data_offset) {
        return fail(GFXI_CORRUPT_ARTIFACT, "data payload misaligned or outside the file: " + name);
      }
      if (e.aux_bytes != 0 && (e.aux_offset % e.alignment != 0 ||
                               !in_file(e.aux_offset, e.aux_bytes, h.file_bytes) ||
                               e.aux_offset < h.data_offset)) {
        return fail(GFXI_CORRUPT_ARTIFACT, "scale payload misaligned or outside the file: " + name);
      }
      gfxinfer_artifact_tensor t{};
      t.dtype = e.dtype;
      t.quantization = e.quantization;
      t.rank = e.rank;
      t.flags = e.flags;
      t.alignment = e.alignment;
      std::memcpy(t.dimensions, e.dimensions, sizeof t.dimensions);
      t.data_offset = e.data_offset;
      t.data_bytes = e.data_bytes;
      t.aux_offset = e.aux_offset;
      t.aux_bytes = e.aux_bytes;
      t.data_crc64 = e.data_crc64;
      a->index.emplace(name, a->tensors.size());
      a->names.push_back(std::move(name));
      a->tensors.push_back(t);
      ranges.emplace_back(e.data_offset, e.data_offset + e.data_bytes);
      if (e.aux_bytes != 0) ranges.emplace_back(e.aux_offset, e.aux_offset + e.aux_bytes);
    }
    if (verify_checksums != 0) {
      // Tensors are independent: check them in parallel (one core reads ~2 GB/s).
      int bad = -1;
  #pragma omp parallel for schedule(dynamic, 1)
      for (long long i = 0; i < static_cast<long long>(a->tensors.size()); ++i) {
        const auto& t = a->tensors[static_cast<std::size_t>(i)];
        if (crc64_update(0, a->map + t.data_offset, t.data_bytes) != t.data_crc64) {
  #pragma omp critical
          bad = static_cast<int>(i);
        }
      }
      if (bad >= 0) {
        return fail(GFXI_CORRUPT_ARTIFACT, "CRC-64 of the payload differs from its entry: " + a->names[static_cast<std::size_t>(bad)]);
      }
    }
    std::sort(ranges.begin(), ranges.end());
    for (std::size_t i = 1; i < ranges.size(); ++i) {
      if (ranges[i].first < ranges[i - 1].second) {
        return fail(GFXI_CORRUPT_ARTIFACT, "two payloads share bytes");
      }
    }
    for (std::size_t i = 0; i < a->tensors.size(); ++i) a->tensors[i].name = a->names[i].c_str();
    *out = a.release();
    return ok();
  });
}

extern "C" void gfxinfer_artifact_close(gfxinfer_artifact* artifact) { delete artifact; }

extern "C" int32_t gfxinfer_artifact_get_identity(const gfxinfer_artifact* artifact,
                                                  gfxinfer_artifact_identity* out) {
  if (artifact == nullptr || out == nullptr) return fail(GFXI_INVALID_ARGUMENT, "invalid artifact query");
  *out = artifact->identity;
  return ok();
}

extern "C" size_t gfxinfer_artifact_tensor_count(const gfxinfer_artifact* artifact) {
  return artifact == nullptr ? 0 : artifact->tensors.size();
}

extern "C" int32_t gfxinfer_artifact_tensor_at(const gfxinfer_artifact* artifact, size_t index,
                                               gfxinfer_artifact_tensor* out) {
  if (artifact == nullptr || out == nullptr || index >= artifact->tensors.size()) {
    return fail(GFXI_INVALID_ARGUMENT, "artifact tensor index out of range");
  }
  *out = artifact->tensors[index];
  return ok();
}

extern "C" int32_t gfxinfer_artifact_find(const gfxinfer_artifact* artifact, const char* name,
                                          gfxinfer_artifact_tensor* out) {
  if (artifact == nullptr || name == nullptr || out == nullptr) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid artifact query");
  }
  const auto it = artifact->index.find(name);
  if (it == artifact->index.end()) return fail(GFXI_INVALID_ARGUMENT, std::string("no tensor ") + name);
  *out = artifact->tensors[it->second];
  return ok();
}

extern "C" const void* gfxinfer_artifact_bytes(const gfxinfer_artifact* artifact, uint64_t offset,
                                               uint64_t bytes) {
  if (artifact == nullptr || !in_file(offset, bytes, artifact->bytes)) return nullptr;
  return artifact->map + offset;
}

extern "C" int32_t gfxinfer_artifact_resource(const gfxinfer_artifact* artifact, const char* name,
                                              const void** data, uint64_t* bytes) {
  if (artifact == nullptr || name == nullptr || data == nullptr || bytes == nullptr) {
    return fail(GFXI_INVALID_ARGUMENT, "invalid artifact resource query");
  }
  *data = nullptr;
  *bytes = 0;
  // Resources are unquantized u8 tensors named "resources/..." (engine.cpp:32-34, 229-236).
  const auto it = artifact->index.find(name);
  if (std::string_view(name).rfind("resources/", 0) != 0 || it == artifact->index.end()) {
    return fail(GFXI_INVALID_ARGUMENT, std::string("no resource ") + name);
  }
  const gfxinfer_artifact_tensor& t = artifact->tensors[it->second];
  if (t.quantization != 0 || t.dtype != 1) {
    return fail(GFXI_INVALID_ARGUMENT, std::string(name) + " is not an unquantized u8 resource");
  }
  *data = gfxinfer_artifact_bytes(artifact, t.data_offset, t.data_bytes);
  *bytes = t.data_bytes;
  return *data != nullptr || t.data_bytes == 0 ? ok() : fail(GFXI_CORRUPT_ARTIFACT, "resource lies outside the file");
}

// ---------------------------------------------------------------------------
// Loader
// ---------------------------------------------------------------------------

namespace gfx950 {
namespace {

// One gfx12 W3 fragment (12 bytes: 32 codes of 3 bits, least significant first,
// code = value + 4; quantization.cpp:279-299) -> the gfx950 lane chunk.
void repack_w3_fragment(const uint8_t* gfx12, uint8_t* gfx950) {
  int8_t values[32];
  for (unsigned item = 0; item < 32; ++item) {
    const unsigned bit = item * 3u, byte = bit >> 3, shift = bit & 7u;
    unsigned code = static_cast<unsigned>(gfx12[byte]) >> shift;
    if (shift > 5u) code |= static_cast<unsigned>(gfx12[byte + 1]) << (8u - shift);
    values[item] = static_cast<int8_t>(static_cast<int>(code & 7u) - 4);
  }
  pack_lane_chunk(GFXI_W3G128, values, gfx950);
}

// One gfx12 W2 fragment (8 bytes: the packed row bytes of 32 columns,
// quantization.cpp:99-103, 300-307) -> the gfx950 lane chunk.
void repack_w2_fragment(const uint8_t* gfx12, uint8_t* gfx950) {
  int8_t values[32];
  for (unsigned item = 0; item < 32; ++item) {
    const unsigned code = (static_cast<unsigned>(gfx12[item / 4]) >> ((item & 3u) * 2u)) & 3u;
    values[item] = static_cast<int8_t>(2 * static_cast<int>(code) - 3);
  }
  pack_lane_chunk(GFXI_W2G128, values, gfx950);
}

void repack_fragment(int32_t format, const uint8_t* gfx12, uint8_t* gfx950) {
  if (format == GFXI_W2G128) {
    repack_w2_fragment(gfx12, gfx950);
  } else {
    repack_w3_fragment(gfx12, gfx950);
  }
}

uint64_t code_bits(int32_t format) {
  return format == GFXI_W2G128 ? 2 : (format == GFXI_W3G128 ? 3 : 4);
}

struct Staging {
  uint8_t* host{nullptr};
  std::size_t bytes{0};
  ~Staging() {
    if (host != nullptr) (void)hipHostFree(host);
  }
};

// repack_format: 0 (plain copy), or the W2 / W3 format whose gfx12 fragments are
// re-packed on the way.
int32_t upload(gfxinfer_model& m, void* device, const uint8_t* source, std::size_t bytes,
               int32_t repack_format, Staging& staging) {
  // Chunks of whole (tile, group) blocks (512 B for W2, 768 B for W3) through pinned
  // staging memory.
  constexpr std::size_t kChunk = 768u * 65536u;  // 48 MiB
  if (staging.host == nullptr) {
    if (auto e = hipHostMalloc(reinterpret_cast<void**>(&staging.host), kChunk); e != hipSuccess) {
      staging.host = nullptr;
      return hip_fail(e, "pinned staging allocation failed");
    }
    staging.bytes = kChunk;
  }
  for (std::size_t done = 0; done < bytes; done += kChunk) {
    const std::size_t n = std::min(kChunk, bytes - done);
    if (repack_format != 0) {
      const std::size_t fb = lane_bytes(repack_format);
#pragma omp parallel for schedule(static)
      for (long long f = 0; f < static_cast<long long>(n / fb); ++f) {
        repack_fragment(repack_format, source + done + static_cast<std::size_t>(f) * fb,
                        staging.host + static_cast<std::size_t>(f) * fb);
      }
    } else {
      std::memcpy(staging.host, source + done, n);
    }
    if (auto e = hipMemcpyAsync(static_cast<uint8_t*>(device) + done, staging.host, n,
                                hipMemcpyHostToDevice, m.stream);
        e != hipSuccess) {
      return hip_fail(e, "weight upload failed");
    }
    if (auto e = hipStreamSynchronize(m.stream); e != hipSuccess) return hip_fail(e, "weight upload failed");
  }
  return ok();
}

uint64_t element_count(const gfxinfer_artifact_tensor& t) {
  uint64_t n = 1;
  for (unsigned d = 0; d < t.rank; ++d) n *= t.dimensions[d];
  return t.rank == 0 ? 0 : n;
}

}  // namespace
}  // namespace gfx950

extern "C" int32_t gfxinfer_retile_gfx12_for_gfx950(int32_t format, const uint8_t* gfx12_codes,
                                                    size_t bytes, uint8_t* gfx950_codes) {
  if (gfx12_codes == nullptr || gfx950_codes == nullptr || !valid_weight_format(format) ||
      bytes % lane_bytes(format) != 0) {
    return fail(GFXI_INVALID_ARGUMENT, "gfx12 re-tiling needs W2/W3/W4 codes of whole 32-column fragments");
  }
  if (format == GFXI_W4G128) {
    std::memmove(gfx950_codes, gfx12_codes, bytes);
    return ok();
  }
  // Each fragment is read whole before its chunk is written (in place is fine).
  const std::size_t fb = lane_bytes(format);
  for (std::size_t f = 0; f < bytes / fb; ++f) repack_fragment(format, gfx12_codes + f * fb, gfx950_codes + f * fb);
  return ok();
}

// Engine::create from an artifact (engine.cpp:62-209): binds every tensor of the
// spec's converter naming, with the quantization the artifact carries (W3 or W4 for
// 2-D matrices, bf16 for the rest), plus the optional MTP draft head and its token
// ids (converter.cpp:252-302).  Accepts the reference's gfx1200 recipe (W3 fragments
// re-packed on the way in) and this library's gfx950 recipe.
extern "C" int32_t gfxinfer_model_create_from_artifact(const gfxinfer_model_spec* spec,
                                                       const char* path, int32_t verify_checksums,
                                                       int32_t device, gfxinfer_model** out) {
  return guarded([&]() -> int32_t {
    if (spec == nullptr || path == nullptr || out == nullptr) {
      return fail(GFXI_INVALID_ARGUMENT, "model loading needs a spec, a path and an output handle");
    }
    *out = nullptr;
    gfxinfer_artifact* raw = nullptr;
    if (const int32_t s = gfxinfer_artifact_open(path, verify_checksums, &raw); s != GFXI_OK) return s;
    std::unique_ptr<gfxinfer_artifact> a(raw);
    const std::string arch(a->identity.target_arch, strnlen(a->identity.target_arch, 16));
    const bool gfx12 = arch == "gfx1200";
    if (!gfx12 && arch != "gfx950") {
      return fail(GFXI_UNSUPPORTED, "artifact target is " + arch + "; expected gfx950 or gfx1200");
    }
    // The reference runtime reads gfx1200 codes as gfx12 tiles only when the recipe names
    // "tiled-v", and W3 codes as sequential 3-bit fragments only when it names "w3seq"
    // (qwen_runtime.cpp:957-960); the other layouts (row-major codes, bit-plane W3) are not
    // re-tiled here, so such files are refused rather than loaded as the wrong weights.
    const std::string recipe(a->identity.recipe_id, strnlen(a->identity.recipe_id, 64));
    const bool tiled = recipe.find("tiled-v") != std::string::npos;
    const bool sequential_w3 = recipe.find("w3seq") != std::string::npos;
    if (gfx12 && !tiled) {
      return fail(GFXI_UNSUPPORTED, "gfx1200 recipe " + recipe + " stores row-major codes; only the "
                                    "tiled recipes (\"tiled-v\") load");
    }
    std::vector<Tensor> tensors = model_tensors(*spec);
    gfxinfer_artifact_tensor head{}, ids{};
    const bool draft = a->index.count("mtp.draft_head.weight") != 0;
    if (draft) {
      (void)gfxinfer_artifact_find(a.get(), "mtp.draft_head.weight", &head);
      if (a->index.count("mtp.draft_head_token_ids") == 0) {
        return fail(GFXI_CORRUPT_ARTIFACT, "artifact has a draft head without token ids");
      }
      (void)gfxinfer_artifact_find(a.get(), "mtp.draft_head_token_ids", &ids);
      Tensor h;
      h.name = "mtp.draft_head.weight";
      h.format = GFXI_W4G128;  // replaced by the artifact's quantization below
      h.rows = head.dimensions[0];
      h.columns = head.dimensions[1];
      tensors.push_back(h);
      Tensor i;
      i.name = "mtp.draft_head_token_ids";
      i.format = kI32;
      i.rows = 1;
      i.columns = ids.dimensions[0];
      tensors.push_back(i);
    }
    // Bind and check every tensor before allocating device memory.
    std::vector<const gfxinfer_artifact_tensor*> source(tensors.size());
    for (std::size_t k = 0; k < tensors.size(); ++k) {
      Tensor& t = tensors[k];
      const auto it = a->index.find(t.name);
      if (it == a->index.end()) return fail(GFXI_CORRUPT_ARTIFACT, "artifact is missing tensor: " + t.name);
      const auto& e = a->tensors[it->second];
      source[k] = &e;
      const uint64_t count = t.rows * t.columns;
      if (t.format == kBf16) {
        if (e.quantization != 0 || e.dtype != kDtypeBf16 || element_count(e) != count ||
            e.data_bytes != count * 2) {
          return fail(GFXI_CORRUPT_ARTIFACT, "tensor " + t.name + " is not the expected bf16 shape");
        }
      } else if (t.format == kI32) {
        if (e.dtype != kDtypeI32 || e.rank != 1 || e.data_bytes != count * 4) {
          return fail(GFXI_CORRUPT_ARTIFACT, "tensor " + t.name + " is not an int32 vector");
        }
      } else {
        if (!valid_weight_format(e.quantization)) {
          return fail(GFXI_UNSUPPORTED, "tensor " + t.name + " uses a quantization the gfx950 GEMM "
                                        "does not run (W2G128, W3G128 and W4G128 only)");
        }
        t.format = e.quantization;  // the artifact's recipe decides W2, W3 or W4
        if (gfx12 && t.format == GFXI_W3G128 && !sequential_w3) {
          return fail(GFXI_UNSUPPORTED, "gfx1200 recipe " + recipe + " stores W3 tensor " + t.name +
                                        " as bit planes; only sequential W3 (\"w3seq\") loads");
        }
        const uint64_t bits = code_bits(t.format);
        if (e.dtype != kDtypeU8 || e.rank != 2 || e.dimensions[0] != t.rows ||
            e.dimensions[1] != t.columns || e.data_bytes != count * bits / 8 ||
            e.aux_bytes != t.rows * (t.columns / kGroup) * 2) {
          return fail(GFXI_CORRUPT_ARTIFACT, "tensor " + t.name + " does not match the model spec");
        }
      }
    }
    if (draft && (head.dimensions[0] != spec->mtp_draft_vocabulary || head.dimensions[1] != spec->hidden_size ||
                  ids.dimensions[0] != head.dimensions[0])) {
      return fail(GFXI_CORRUPT_ARTIFACT, "draft head shape does not match the spec's MTP vocabulary");
    }
    gfxinfer_model* m = nullptr;
    if (const int32_t s = allocate_model(*spec, device, std::move(tensors), &m); s != GFXI_OK) return s;
    Staging staging;
    int32_t status = ok();
    for (std::size_t k = 0; k < m->tensors.size() && status == GFXI_OK; ++k) {
      const Tensor& t = m->tensors[k];
      const auto& e = *source[k];
      const int32_t repack = gfx12 && (t.format == GFXI_W2G128 || t.format == GFXI_W3G128) ? t.format : 0;
      status = upload(*m, m->data(&t), a->map + e.data_offset, e.data_bytes, repack, staging);
      if (status == GFXI_OK && t.auxiliary_bytes != 0) {
        status = upload(*m, m->auxiliary(&t), a->map + e.aux_offset, e.aux_bytes, 0, staging);
      }
    }
    if (status != GFXI_OK) {
      gfxinfer_model_destroy(m);
      return status;
    }
    *out = m;
    return ok();
  });
}

// ---------------------------------------------------------------------------
// Writer (gfx950 recipe)
// ---------------------------------------------------------------------------

namespace gfx950 {
namespace {

// Shape of a tensor as the converter writes it (qwen38_spec.cpp:30-102): vectors are
// rank 1, conv1d weights [C, 1, 4], matrices [rows, columns].
void artifact_shape(const Tensor& t, DiskEntry& e) {
  const bool conv = t.name.ends_with("conv1d.weight");
  if (t.format == kI32 || (t.format == kBf16 && t.rows == 1)) {
    e.rank = 1;
    e.dimensions[0] = t.columns;
  } else if (t.format == kBf16 && conv) {
    e.rank = 3;
    e.dimensions[0] = t.rows;
    e.dimensions[1] = 1;
    e.dimensions[2] = t.columns;
  } else {
    e.rank = 2;
    e.dimensions[0] = t.rows;
    e.dimensions[1] = t.columns;
  }
}

bool write_all(int fd, const void* p, std::size_t n) {
  const auto* c = static_cast<const uint8_t*>(p);
  while (n != 0) {
    const ssize_t w = ::write(fd, c, n);
    if (w < 0 && errno == EINTR) continue;
    if (w <= 0) return false;
    c += w;
    n -= static_cast<std::size_t>(w);
  }
  return true;
}

bool write_zeros(int fd, uint64_t n) {
  static const uint8_t zeros[4096] = {};
  while (n != 0) {
    const std::size_t k = static_cast<std::size_t>(std::min<uint64_t>(n, sizeof zeros));
    if (!write_all(fd, zeros, k)) return false;
    n -= k;
  }
  return true;
}

}  // namespace
}  // namespace gfx950

extern "C" int32_t gfxinfer_model_write_artifact(const gfxinfer_model* model, const char* path,
                                                 const char* weights_id, const uint32_t* draft_rows,
                                                 size_t draft_count) {
  return guarded([&]() -> int32_t {
    if (model == nullptr || path == nullptr || weights_id == nullptr ||
        (draft_count != 0 && (draft_rows == nullptr || draft_count % 16 != 0))) {
      return fail(GFXI_INVALID_ARGUMENT, "artifact writing needs a model, a path, a weights id and "
                                         "a multiple of 16 draft rows (or none)");
    }
    if (draft_count != 0 && model->find("mtp.draft_head.weight") != nullptr) {
      return fail(GFXI_INVALID_ARGUMENT, "the model already has a draft head");
    }
    DiskHeader h{};
    std::memcpy(h.magic, kMagic, sizeof kMagic);
    h.version = kFormatVersion;
    h.header_bytes = sizeof(DiskHeader);
    h.endian_tag = kEndianTag;
    h.directory_offset = sizeof(DiskHeader);
    h.directory_entry_bytes = sizeof(DiskEntry);
    if (!put_fixed(h.target_arch, "gfx950") || !put_fixed(h.model_id, "qwen3.8-27b") ||
        !put_fixed(h.weights_id, weights_id) || !put_fixed(h.recipe_id, "gfx950-tile16x128-w3w4-bf16")) {
      return fail(GFXI_INVALID_ARGUMENT, "weights id must be 1..31 characters");
    }
    if (auto e = hipSetDevice(model->device); e != hipSuccess) return hip_fail(e, "hipSetDevice failed");
    // Host copy of the whole arena in one transfer.
    std::vector<uint8_t> arena(model->arena_bytes);
    if (auto e = hipMemcpy(arena.data(), model->arena, model->arena_bytes, hipMemcpyDeviceToHost);
        e != hipSuccess) {
      return hip_fail(e, "weight download failed");
    }
    struct Payload {
      Tensor tensor;
      const uint8_t* data;
      const uint8_t* aux;
    };
    std::vector<Payload> payloads;
    for (const Tensor& t : model->tensors) {
      payloads.push_back({t, arena.data() + t.data_offset,
                          t.auxiliary_bytes != 0 ? arena.data() + t.auxiliary_offset : nullptr});
    }
    // Draft head (converter.cpp:252-302): LM-head rows draft_rows[i] re-tiled as rows i.
    std::vector<uint8_t> head_codes, head_scales;
    std::vector<uint32_t> head_ids(draft_rows, draft_rows + draft_count);
    if (draft_count != 0) {
      const Tensor* lm = model->find("lm_head.weight");
      if (lm == nullptr) return fail(GFXI_INVALID_ARGUMENT, "model has no LM head");
      const std::size_t groups = lm->columns / kGroup, lb = lane_bytes(lm->format);
      Tensor hd;
      hd.name = "mtp.draft_head.weight";
      hd.format = lm->format;
      hd.rows = draft_count;
      hd.columns = lm->columns;
      hd.data_bytes = draft_count * lm->columns * code_bits(lm->format) / 8;
      hd.auxiliary_bytes = draft_count * groups * 2;
      head_codes.resize(hd.data_bytes);
      head_scales.resize(hd.auxiliary_bytes);
      const uint8_t* codes = arena.data() + lm->data_offset;
      const uint8_t* scales = arena.data() + lm->auxiliary_offset;
      for (std::size_t i = 0; i < draft_count; ++i) {
        const std::size_t r = draft_rows[i];
        if (r >= lm->rows) return fail(GFXI_INVALID_ARGUMENT, "draft row outside the LM head");
        for (std::size_t g = 0; g < groups; ++g) {
          for (std::size_t kb = 0; kb < 4; ++kb) {
            std::memcpy(head_codes.data() + chunk_offset(lm->format, i, g * kGroup + kb * 32, groups),
                        codes + chunk_offset(lm->format, r, g * kGroup + kb * 32, groups), lb);
          }
          std::memcpy(head_scales.data() + 2 * scale_offset(i, g, groups),
                      scales + 2 * scale_offset(r, g, groups), 2);
        }
      }
      payloads.push_back({hd, head_codes.data(), head_scales.data()});
      Tensor ids;
      ids.name = "mtp.draft_head_token_ids";
      ids.format = kI32;
      ids.rows = 1;
      ids.columns = draft_count;
      ids.data_bytes = draft_count * 4;
      payloads.push_back({ids, reinterpret_cast<const uint8_t*>(head_ids.data()), nullptr});
    }
    h.tensor_count = static_cast<uint32_t>(payloads.size());
    std::vector<DiskEntry> entries(payloads.size());
    std::string strings;
    for (std::size_t k = 0; k < payloads.size(); ++k) {
      const Tensor& t = payloads[k].tensor;
      DiskEntry& e = entries[k];
      e = {};
      e.name_offset = strings.size();
      e.name_bytes = static_cast<uint32_t>(t.name.size());
      strings += t.name;
      e.dtype = t.format == kBf16 ? kDtypeBf16 : t.format == kI32 ? kDtypeI32 : kDtypeU8;
      e.quantization = t.format > 0 ? static_cast<uint16_t>(t.format) : 0;
      e.alignment = static_cast<uint32_t>(kFileAlignment);
      artifact_shape(t, e);
      e.data_bytes = t.data_bytes;
      e.aux_bytes = t.auxiliary_bytes;
      e.data_crc64 = crc64_update(0, payloads[k].data, t.data_bytes);
    }
    const uint64_t directory_bytes = entries.size() * sizeof(DiskEntry);
    h.strings_offset = h.directory_offset + directory_bytes;
    h.strings_bytes = strings.size();
    h.data_offset = align_up(h.strings_offset + h.strings_bytes, kFileAlignment);
    uint64_t cursor = h.data_offset;
    for (DiskEntry& e : entries) {
      cursor = align_up(cursor, e.alignment);
      e.data_offset = cursor;
      cursor += e.data_bytes;
      if (e.aux_bytes != 0) {
        cursor = align_up(cursor, e.alignment);
        e.aux_offset = cursor;
        cursor += e.aux_bytes;
      }
    }
    h.file_bytes = cursor;
    h.data_bytes = cursor - h.data_offset;
    std::vector<uint8_t> manifest(directory_bytes + strings.size());
    std::memcpy(manifest.data(), entries.data(), directory_bytes);
    std::memcpy(manifest.data() + directory_bytes, strings.data(), strings.size());
    h.manifest_crc64 = crc64_update(0, manifest.data(), manifest.size());

    // Written to a temporary name, synced, then renamed into place.
    const std::string temporary = std::string(path) + ".tmp." + std::to_string(::getpid());
    const int fd = ::open(temporary.c_str(), O_WRONLY | O_CREAT | O_EXCL | O_CLOEXEC, 0644);
    if (fd < 0) return fail(GFXI_IO_ERROR, "cannot create " + temporary + ": " + std::strerror(errno));
    bool good = write_all(fd, &h, sizeof h) && write_all(fd, manifest.data(), manifest.size()) &&
                write_zeros(fd, h.data_offset - (h.strings_offset + h.strings_bytes));
    cursor = h.data_offset;
    for (std::size_t k = 0; good && k < entries.size(); ++k) {
      const DiskEntry& e = entries[k];
      good = write_zeros(fd, e.data_offset - cursor) && write_all(fd, payloads[k].data, e.data_bytes);
      cursor = e.data_offset + e.data_bytes;
      if (good && e.aux_bytes != 0) {
        good = write_zeros(fd, e.aux_offset - cursor) && write_all(fd, payloads[k].aux, e.aux_bytes);
        cursor = e.aux_offset + e.aux_bytes;
      }
    }
    good = good && ::fsync(fd) == 0;
    const int saved = errno;
    ::close(fd);
    if (!good || ::rename(temporary.c_str(), path) != 0) {
      const std::string why = std::strerror(good ? errno : saved);
      ::unlink(temporary.c_str());
      return fail(GFXI_IO_ERROR, std::string("cannot write artifact ") + path + ": " + why);
    }
    return ok();
  });
}
