// Byte-level BPE tokenizer of the Qwen tokenizer.json format and the chat prompt
// template (reference src/tokenizer.cpp, include/gfxinfer/tokenizer.h and
// src/cli/main.cpp:1037-1039).  Host code only; ICU supplies NFC normalization and
// the Unicode character classes.
//
// Encoding, as the reference: the text is cut at added tokens (the earliest match,
// the longest one at a tie); every other segment is NFC-normalized, split into
// pre-tokens by the Qwen pattern
//   (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+|\p{N}
//   | ?[^\s\p{L}\p{M}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+
// (tokenizer.cpp:143-146, anchored at each position, first alternative that matches),
// each pre-token's bytes are mapped to the GPT-2 byte alphabet, and adjacent symbols
// are merged by BPE rank until no ranked pair is left.  Here the pattern is a
// hand-written matcher over code points instead of a regex engine; \s is the Unicode
// White_Space property.  Decoding maps each piece back through the byte alphabet.
#include <unicode/normalizer2.h>
#include <unicode/uchar.h>
#include <unicode/unistr.h>

#include <algorithm>
#include <array>
#include <cstring>
#include <limits>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_map>
#include <utility>
#include <vector>

#include "common.hpp"
#include "gfxinfer_runtime.h"

namespace gfx950 {
namespace {

// UTF-8 of one code point.
void append_code_point(std::string& out, uint32_t cp) {
  if (cp < 0x80u) {
    out.push_back(static_cast<char>(cp));
  } else if (cp < 0x800u) {
    out.push_back(static_cast<char>(0xC0u | (cp >> 6)));
    out.push_back(static_cast<char>(0x80u | (cp & 0x3Fu)));
  } else if (cp < 0x10000u) {
    out.push_back(static_cast<char>(0xE0u | (cp >> 12)));
    out.push_back(static_cast<char>(0x80u | ((cp >> 6) & 0x3Fu)));
    out.push_back(static_cast<char>(0x80u | (cp & 0x3Fu)));
  } else {
    out.push_back(static_cast<char>(0xF0u | (cp >> 18)));
    out.push_back(static_cast<char>(0x80u | ((cp >> 12) & 0x3Fu)));
    out.push_back(static_cast<char>(0x80u | ((cp >> 6) & 0x3Fu)));
    out.push_back(static_cast<char>(0x80u | (cp & 0x3Fu)));
  }
}

// ---------------------------------------------------------------------------
// Minimal JSON reader: the document tree of one tokenizer.json.
// ---------------------------------------------------------------------------

struct JsonValue {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  bool boolean = false;
  double number = 0.0;
  bool integral = false;
  int64_t integer = 0;
  std::string text;
  std::vector<JsonValue> items;
  std::vector<std::pair<std::string, JsonValue>> members;

  const JsonValue* member(std::string_view key) const {
    if (kind != kObject) return nullptr;
    for (const auto& m : members) {
      if (m.first == key) return &m.second;
    }
    return nullptr;
  }
};

class JsonReader {
 public:
  JsonReader(const char* data, std::size_t size) : at_(data), end_(data + size) {}

  bool document(JsonValue& out) {
    if (!value(out, 0)) return false;
    skip_space();
    return at_ == end_ || fail("trailing characters after the JSON document");
  }
  const std::string& error() const { return error_; }

 private:
  static constexpr int kMaxDepth = 64;
  const char* at_;
  const char* end_;
  std::string error_;

  bool fail(const char* message) {
    if (error_.empty()) error_ = message;
    return false;
  }
  void skip_space() {
    while (at_ < end_ && (*at_ == ' ' || *at_ == '\t' || *at_ == '\n' || *at_ == '\r')) ++at_;
  }
  bool literal(const char* word) {
    const std::size_t n = std::strlen(word);
    if (static_cast<std::size_t>(end_ - at_) < n || std::memcmp(at_, word, n) != 0) {
      return fail("invalid JSON literal");
    }
    at_ += n;
    return true;
  }

  bool value(JsonValue& out, int depth) {
    if (depth > kMaxDepth) return fail("JSON nesting is too deep");
    skip_space();
    if (at_ == end_) return fail("unexpected end of JSON");
    switch (*at_) {
      case '{': return object(out, depth);
      case '[': return array(out, depth);
      case '"': out.kind = JsonValue::kString; return string(out.text);
      case 't': out.kind = JsonValue::kBool; out.boolean = true; return literal("true");
      case 'f': out.kind = JsonValue::kBool; out.boolean = false; return literal("false");
      case 'n': out.kind = JsonValue::kNull; return literal("null");
      default: return number(out);
    }
  }

  bool object(JsonValue& out, int depth) {
    out.kind = JsonValue::kObject;
    ++at_;
    skip_space();
    if (at_ < end_ && *at_ == '}') {
      ++at_;
      return true;
    }
    while (true) {
      skip_space();
      if (at_ == end_ || *at_ != '"') return fail("JSON object key expected");
      std::string key;
      if (!string(key)) return false;
      skip_space();
      if (at_ == end_ || *at_ != ':') return fail("':' expected in JSON object");
      ++at_;
      out.members.emplace_back(std::move(key), JsonValue{});
      if (!value(out.members.back().second, depth + 1)) return false;
      skip_space();
      if (at_ < end_ && *at_ == ',') {
        ++at_;
        continue;
      }
      if (at_ < end_ && *at_ == '}') {
        ++at_;
        return true;
      }
      return fail("',' or '}' expected in JSON object");
    }
  }

  bool array(JsonValue& out, int depth) {
    out.kind = JsonValue::kArray;
    ++at_;
    skip_space();
    if (at_ < end_ && *at_ == ']') {
      ++at_;
      return true;
    }
    while (true) {
      out.items.emplace_back();
      if (!value(out.items.back(), depth + 1)) return false;
      skip_space();
      if (at_ < end_ && *at_ == ',') {
        ++at_;
        continue;
      }
      if (at_ < end_ && *at_ == ']') {
        ++at_;
        return true;
      }
      return fail("',' or ']' expected in JSON array");
    }
  }

  bool hex4(uint32_t& out) {
    if (end_ - at_ < 4) return fail("truncated \\u escape in JSON string");
    out = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *at_++;
      out <<= 4;
      if (c >= '0' && c <= '9') out |= static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') out |= static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') out |= static_cast<uint32_t>(c - 'A' + 10);
      else return fail("invalid \\u escape in JSON string");
    }
    return true;
  }

  bool string(std::string& out) {
    ++at_;  // opening quote
    while (true) {
      if (at_ == end_) return fail("unterminated JSON string");
      const char c = *at_++;
      if (c == '"') return true;
      if (static_cast<unsigned char>(c) < 0x20u) return fail("control character in JSON string");
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (at_ == end_) return fail("unterminated JSON escape");
      const char e = *at_++;
      switch (e) {
        case '"': out.push_back('"'); break;
        case '\\': out.push_back('\\'); break;
        case '/': out.push_back('/'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          uint32_t cp = 0;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800u && cp <= 0xDBFFu) {  // high surrogate: a low one must follow
            uint32_t low = 0;
            if (end_ - at_ < 2 || at_[0] != '\\' || at_[1] != 'u') return fail("unpaired surrogate in JSON string");
            at_ += 2;
            if (!hex4(low)) return false;
            if (low < 0xDC00u || low > 0xDFFFu) return fail("unpaired surrogate in JSON string");
            cp = 0x10000u + ((cp - 0xD800u) << 10) + (low - 0xDC00u);
          } else if (cp >= 0xDC00u && cp <= 0xDFFFu) {
            return fail("unpaired surrogate in JSON string");
          }
          append_code_point(out, cp);
          break;
        }
        default: return fail("invalid escape in JSON string");
      }
    }
  }

  bool number(JsonValue& out) {
    const char* begin = at_;
    if (at_ < end_ && *at_ == '-') ++at_;
    bool digits = false, fraction = false;
    while (at_ < end_ && ((*at_ >= '0' && *at_ <= '9') || *at_ == '.' || *at_ == 'e' || *at_ == 'E' ||
                          *at_ == '+' || *at_ == '-')) {
      if (*at_ >= '0' && *at_ <= '9') digits = true;
      else fraction = true;
      ++at_;
    }
    if (!digits) return fail("invalid JSON value");
    const std::string token(begin, at_);
    char* stop = nullptr;
    out.kind = JsonValue::kNumber;
    out.number = std::strtod(token.c_str(), &stop);
    if (stop != token.c_str() + token.size()) return fail("invalid JSON number");
    if (!fraction) {
      out.integral = true;
      out.integer = std::strtoll(token.c_str(), &stop, 10);
    }
    return true;
  }
};

// ---------------------------------------------------------------------------
// UTF-8 and the GPT-2 byte alphabet.
// ---------------------------------------------------------------------------

// Next code point of well-formed UTF-8 at `at` (advanced), or false.
bool next_code_point(std::string_view text, std::size_t& at, uint32_t& cp) {
  if (at >= text.size()) return false;
  const auto lead = static_cast<unsigned char>(text[at]);
  unsigned extra = 0;
  uint32_t value = 0;
  if (lead < 0x80u) {
    cp = lead;
    ++at;
    return true;
  } else if ((lead & 0xE0u) == 0xC0u) {
    extra = 1;
    value = lead & 0x1Fu;
  } else if ((lead & 0xF0u) == 0xE0u) {
    extra = 2;
    value = lead & 0x0Fu;
  } else if ((lead & 0xF8u) == 0xF0u) {
    extra = 3;
    value = lead & 0x07u;
  } else {
    return false;
  }
  if (at + 1 + extra > text.size()) return false;
  for (unsigned i = 1; i <= extra; ++i) {
    const auto c = static_cast<unsigned char>(text[at + i]);
    if ((c & 0xC0u) != 0x80u) return false;
    value = (value << 6) | (c & 0x3Fu);
  }
  at += 1 + extra;
  cp = value;
  return true;
}

// The byte alphabet (tokenizer.cpp:68-85, 108-120): printable Latin-1 bytes stand for
// themselves, the other 68 bytes take code points 256, 257, ... in byte order.
struct ByteAlphabet {
  std::array<std::string, 256> symbol;          // byte -> UTF-8 of its code point
  std::unordered_map<uint32_t, uint8_t> byte;   // code point -> byte
  ByteAlphabet() {
    uint32_t next = 256;
    for (uint32_t b = 0; b < 256; ++b) {
      const bool printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174);
      const uint32_t cp = printable ? b : next++;
      append_code_point(symbol[b], cp);
      byte.emplace(cp, static_cast<uint8_t>(b));
    }
  }
};

const ByteAlphabet& alphabet() {
  static const ByteAlphabet table;
  return table;
}

// ---------------------------------------------------------------------------
// The pre-token pattern.
// ---------------------------------------------------------------------------

bool is_letter(uint32_t c) { return (U_GET_GC_MASK(static_cast<UChar32>(c)) & U_GC_L_MASK) != 0; }
bool is_mark(uint32_t c) { return (U_GET_GC_MASK(static_cast<UChar32>(c)) & U_GC_M_MASK) != 0; }
bool is_number(uint32_t c) { return (U_GET_GC_MASK(static_cast<UChar32>(c)) & U_GC_N_MASK) != 0; }
// \s under PCRE2_UCP (the reference's regex engine, tokenizer.cpp:143-146): \p{Z}, \h and
// \v, i.e. Unicode White_Space plus U+180E, which PCRE2 keeps in \h.
bool is_space(uint32_t c) { return c == 0x180Eu || u_isUWhiteSpace(static_cast<UChar32>(c)) != 0; }
bool is_newline(uint32_t c) { return c == '\r' || c == '\n'; }

// Case-insensitive match of an ASCII letter (s also matches U+017F, which case-folds
// to s).
bool same_letter(uint32_t c, char lower) {
  if (c == static_cast<uint32_t>(lower) || c == static_cast<uint32_t>(lower - 'a' + 'A')) return true;
  return lower == 's' && c == 0x17Fu;
}

// End (exclusive) of the pattern's match anchored at `i` of `cp`; i when nothing
// matches (every code point matches some alternative, so this does not happen).
std::size_t pretoken_end(const std::vector<uint32_t>& cp, std::size_t i) {
  const std::size_t n = cp.size();
  // 1: contractions.
  if (cp[i] == '\'') {
    static constexpr const char* kSuffixes[] = {"s", "t", "re", "ve", "m", "ll", "d"};
    for (const char* suffix : kSuffixes) {
      const std::size_t len = std::strlen(suffix);
      if (i + 1 + len > n) continue;
      bool match = true;
      for (std::size_t k = 0; k < len && match; ++k) match = same_letter(cp[i + 1 + k], suffix[k]);
      if (match) return i + 1 + len;
    }
  }
  // 2: an optional non-letter, non-number (not CR/LF) lead, then letters and marks.
  auto letters_from = [&](std::size_t j) {
    while (j < n && (is_letter(cp[j]) || is_mark(cp[j]))) ++j;
    return j;
  };
  if (!is_newline(cp[i]) && !is_letter(cp[i]) && !is_number(cp[i])) {
    const std::size_t e = letters_from(i + 1);
    if (e > i + 1) return e;
  }
  if (const std::size_t e = letters_from(i); e > i) return e;
  // 3: one number.
  if (is_number(cp[i])) return i + 1;
  // 4: an optional space, then symbols (no space, letter, mark or number), then CR/LF.
  auto symbols_from = [&](std::size_t j) {
    const std::size_t start = j;
    while (j < n && !is_space(cp[j]) && !is_letter(cp[j]) && !is_mark(cp[j]) && !is_number(cp[j])) ++j;
    if (j == start) return start;
    while (j < n && is_newline(cp[j])) ++j;
    return j;
  };
  if (cp[i] == ' ') {
    if (const std::size_t e = symbols_from(i + 1); e > i + 1) return e;
  }
  if (const std::size_t e = symbols_from(i); e > i) return e;
  // 5-7: whitespace runs.
  std::size_t run = i;
  while (run < n && is_space(cp[run])) ++run;
  if (run == i) return i;
  for (std::size_t k = run; k > i; --k) {  // 5: up to the run's last CR/LF
    if (is_newline(cp[k - 1])) return k;
  }
  if (run == n) return run;          // 6: the run ends the text
  if (run - i >= 2) return run - 1;  // 6: leave the last space to the next pre-token
  return run;                        // 7
}

// ---------------------------------------------------------------------------
// The tokenizer.
// ---------------------------------------------------------------------------

struct AddedToken {
  std::string content;
  uint32_t id;
};

}  // namespace
}  // namespace gfx950

struct gfxinfer_tokenizer {
  std::vector<std::string> pieces;                   // id -> piece
  std::unordered_map<std::string, uint32_t> ids;     // piece -> id
  std::unordered_map<std::string, uint32_t> ranks;   // "left right" -> merge rank
  std::vector<gfx950::AddedToken> added;             // longest first
};

namespace gfx950 {
namespace {

int32_t corrupt(const std::string& message) { return fail(GFXI_CORRUPT_ARTIFACT, "tokenizer JSON: " + message); }

int32_t build_tokenizer(const JsonValue& root, gfxinfer_tokenizer& t) {
  const JsonValue* model = root.member("model");
  const JsonValue* vocab = model != nullptr ? model->member("vocab") : nullptr;
  const JsonValue* merges = model != nullptr ? model->member("merges") : nullptr;
  const JsonValue* added = root.member("added_tokens");
  if (vocab == nullptr || vocab->kind != JsonValue::kObject) return corrupt("model.vocab is not an object");
  if (merges == nullptr || merges->kind != JsonValue::kArray) return corrupt("model.merges is not an array");
  if (added == nullptr || added->kind != JsonValue::kArray) return corrupt("added_tokens is not an array");
  if (const JsonValue* type = model->member("type"); type != nullptr &&
      (type->kind != JsonValue::kString || type->text != "BPE")) {
    return fail(GFXI_UNSUPPORTED, "tokenizer JSON: only BPE models are supported");
  }
  // Pieces: ids must cover 0 .. N-1 exactly once between the vocabulary and the
  // added tokens (an added token may restate a vocabulary piece's id).
  constexpr int64_t kMaxIds = int64_t{1} << 24;
  int64_t size = 0;
  auto check_id = [&](const JsonValue& v, int64_t& id) -> bool {
    if (v.kind != JsonValue::kNumber || !v.integral || v.integer < 0 || v.integer >= kMaxIds) return false;
    id = v.integer;
    size = std::max(size, id + 1);
    return true;
  };
  for (const auto& m : vocab->members) {
    int64_t id = 0;
    if (!check_id(m.second, id)) return corrupt("vocabulary id of \"" + m.first + "\" is invalid");
  }
  for (const auto& a : added->items) {
    const JsonValue* id = a.member("id");
    const JsonValue* content = a.member("content");
    int64_t value = 0;
    if (id == nullptr || !check_id(*id, value) || content == nullptr || content->kind != JsonValue::kString ||
        content->text.empty()) {
      return corrupt("added token entry is invalid");
    }
  }
  t.pieces.assign(static_cast<std::size_t>(size), std::string());
  std::vector<uint8_t> seen(static_cast<std::size_t>(size), 0);
  for (const auto& m : vocab->members) {
    const auto id = static_cast<std::size_t>(m.second.integer);
    if (seen[id] != 0) return corrupt("vocabulary id " + std::to_string(id) + " appears twice");
    seen[id] = 1;
    t.pieces[id] = m.first;
    t.ids[m.first] = static_cast<uint32_t>(id);
  }
  for (const auto& a : added->items) {
    const auto id = static_cast<std::size_t>(a.member("id")->integer);
    const std::string& content = a.member("content")->text;
    seen[id] = 1;
    t.pieces[id] = content;
    t.ids[content] = static_cast<uint32_t>(id);
    t.added.push_back({content, static_cast<uint32_t>(id)});
  }
  for (std::size_t id = 0; id < seen.size(); ++id) {
    if (seen[id] == 0) return corrupt("no piece for id " + std::to_string(id));
  }
  // Merges: "left right" strings, or [left, right] pairs (newer files).  Byte-level
  // pieces never contain U+0020, so "left right" is an unambiguous key.
  uint32_t rank = 0;
  for (const auto& m : merges->items) {
    std::string key;
    if (m.kind == JsonValue::kString) {
      const std::size_t space = m.text.find(' ');
      if (space == std::string::npos || space == 0 || space + 1 >= m.text.size() ||
          m.text.find(' ', space + 1) != std::string::npos) {
        return corrupt("merge \"" + m.text + "\" is not two pieces");
      }
      key = m.text;
    } else if (m.kind == JsonValue::kArray && m.items.size() == 2 && m.items[0].kind == JsonValue::kString &&
               m.items[1].kind == JsonValue::kString && !m.items[0].text.empty() && !m.items[1].text.empty()) {
      key = m.items[0].text + " " + m.items[1].text;
    } else {
      return corrupt("merge entry is not a string or a pair of strings");
    }
    t.ranks.emplace(std::move(key), rank++);  // a repeated pair keeps its first rank
  }
  std::stable_sort(t.added.begin(), t.added.end(),
                   [](const AddedToken& a, const AddedToken& b) { return a.content.size() > b.content.size(); });
  return GFXI_OK;
}

// NFC of a UTF-8 segment (tokenizer.cpp:122-139).
int32_t normalize(std::string_view text, std::string& out) {
  UErrorCode status = U_ZERO_ERROR;
  const icu::Normalizer2* nfc = icu::Normalizer2::getNFCInstance(status);
  if (U_FAILURE(status) || nfc == nullptr) return fail(GFXI_INTERNAL, "ICU NFC normalizer is unavailable");
  const icu::UnicodeString source = icu::UnicodeString::fromUTF8(
      icu::StringPiece(text.data(), static_cast<int32_t>(text.size())));
  icu::UnicodeString result;
  nfc->normalize(source, result, status);
  if (U_FAILURE(status)) return fail(GFXI_INVALID_ARGUMENT, "text cannot be NFC-normalized");
  out.clear();
  result.toUTF8String(out);
  return GFXI_OK;
}

// BPE of one pre-token (tokenizer.cpp:294-327): its bytes as alphabet symbols, then
// repeatedly every occurrence (left to right, not overlapping) of the best-ranked
// adjacent pair is joined.
int32_t encode_pretoken(const gfxinfer_tokenizer& t, std::string_view bytes, std::vector<uint32_t>& out) {
  const ByteAlphabet& abc = alphabet();
  std::vector<std::string> symbols;
  symbols.reserve(bytes.size());
  for (const char c : bytes) symbols.push_back(abc.symbol[static_cast<unsigned char>(c)]);
  std::string key;
  while (symbols.size() > 1) {
    uint32_t best = std::numeric_limits<uint32_t>::max();
    std::size_t best_at = 0;
    for (std::size_t i = 0; i + 1 < symbols.size(); ++i) {
      key.assign(symbols[i]).append(" ").append(symbols[i + 1]);
      const auto found = t.ranks.find(key);
      if (found != t.ranks.end() && found->second < best) {
        best = found->second;
        best_at = i;
      }
    }
    if (best == std::numeric_limits<uint32_t>::max()) break;
    const std::string left = symbols[best_at], right = symbols[best_at + 1];
    std::vector<std::string> joined;
    joined.reserve(symbols.size());
    for (std::size_t i = 0; i < symbols.size();) {
      if (i + 1 < symbols.size() && symbols[i] == left && symbols[i + 1] == right) {
        joined.push_back(left + right);
        i += 2;
      } else {
        joined.push_back(std::move(symbols[i]));
        ++i;
      }
    }
    symbols.swap(joined);
  }
  for (const auto& s : symbols) {
    const auto found = t.ids.find(s);
    if (found == t.ids.end()) return fail(GFXI_CORRUPT_ARTIFACT, "a BPE symbol is not in the vocabulary");
    out.push_back(found->second);
  }
  return GFXI_OK;
}

// One segment without added tokens: NFC, pre-tokens, BPE.
int32_t encode_segment(const gfxinfer_tokenizer& t, std::string_view segment, std::vector<uint32_t>& out) {
  if (segment.empty()) return GFXI_OK;
  std::string text;
  if (const int32_t s = normalize(segment, text); s != GFXI_OK) return s;
  std::vector<uint32_t> cp;
  std::vector<std::size_t> offset;  // byte offset of each code point, plus the end
  for (std::size_t at = 0; at < text.size();) {
    offset.push_back(at);
    uint32_t c = 0;
    if (!next_code_point(text, at, c)) return fail(GFXI_INVALID_ARGUMENT, "text is not valid UTF-8");
    cp.push_back(c);
  }
  offset.push_back(text.size());
  for (std::size_t i = 0; i < cp.size();) {
    const std::size_t e = pretoken_end(cp, i);
    if (e <= i) return fail(GFXI_INTERNAL, "the pre-tokenizer did not consume the text");
    const std::string_view piece(text.data() + offset[i], offset[e] - offset[i]);
    if (const int32_t s = encode_pretoken(t, piece, out); s != GFXI_OK) return s;
    i = e;
  }
  return GFXI_OK;
}

int32_t encode_text(const gfxinfer_tokenizer& t, std::string_view text, std::vector<uint32_t>& out) {
  std::size_t cursor = 0;
  while (cursor < text.size()) {
    std::size_t at = std::string_view::npos;
    const AddedToken* next = nullptr;
    for (const auto& a : t.added) {  // longest first: the longest wins a tie
      const std::size_t found = text.find(a.content, cursor);
      if (found < at) {
        at = found;
        next = &a;
      }
    }
    if (next == nullptr) return encode_segment(t, text.substr(cursor), out);
    if (const int32_t s = encode_segment(t, text.substr(cursor, at - cursor), out); s != GFXI_OK) return s;
    out.push_back(next->id);
    cursor = at + next->content.size();
  }
  return GFXI_OK;
}

int32_t decode_ids(const gfxinfer_tokenizer& t, const uint32_t* ids, std::size_t count, std::string& out) {
  const ByteAlphabet& abc = alphabet();
  for (std::size_t k = 0; k < count; ++k) {
    if (ids[k] >= t.pieces.size()) return fail(GFXI_INVALID_ARGUMENT, "token id is outside the vocabulary");
    const std::string& piece = t.pieces[ids[k]];
    for (std::size_t at = 0; at < piece.size();) {
      uint32_t c = 0;
      if (!next_code_point(piece, at, c)) return fail(GFXI_CORRUPT_ARTIFACT, "a tokenizer piece is not valid UTF-8");
      const auto found = abc.byte.find(c);
      if (found == abc.byte.end()) {
        return fail(GFXI_CORRUPT_ARTIFACT, "a tokenizer piece is outside the byte alphabet");
      }
      out.push_back(static_cast<char>(found->second));
    }
  }
  return GFXI_OK;
}

}  // namespace
}  // namespace gfx950

using namespace gfx950;

extern "C" int32_t gfxinfer_tokenizer_create(const void* json, size_t bytes, gfxinfer_tokenizer** out) {
  return guarded([&]() -> int32_t {
    if (out == nullptr) return fail(GFXI_INVALID_ARGUMENT, "tokenizer output pointer is null");
    *out = nullptr;
    if (json == nullptr || bytes == 0) return fail(GFXI_INVALID_ARGUMENT, "tokenizer JSON resource is empty");
    JsonValue root;
    JsonReader reader(static_cast<const char*>(json), bytes);
    if (!reader.document(root)) return fail(GFXI_CORRUPT_ARTIFACT, "tokenizer JSON: " + reader.error());
    auto tokenizer = std::make_unique<gfxinfer_tokenizer>();
    if (const int32_t s = build_tokenizer(root, *tokenizer); s != GFXI_OK) return s;
    *out = tokenizer.release();
    return GFXI_OK;
  });
}

extern "C" void gfxinfer_tokenizer_destroy(gfxinfer_tokenizer* tokenizer) { delete tokenizer; }

extern "C" size_t gfxinfer_tokenizer_vocabulary_size(const gfxinfer_tokenizer* tokenizer) {
  return tokenizer != nullptr ? tokenizer->pieces.size() : 0;
}

extern "C" int32_t gfxinfer_tokenizer_encode(const gfxinfer_tokenizer* tokenizer, const char* text, size_t length,
                                             uint32_t* ids, size_t capacity, size_t* count) {
  return guarded([&]() -> int32_t {
    if (tokenizer == nullptr || count == nullptr || (text == nullptr && length != 0) ||
        (ids == nullptr && capacity != 0)) {
      return fail(GFXI_INVALID_ARGUMENT, "tokenizer encode arguments are invalid");
    }
    std::vector<uint32_t> out;
    if (const int32_t s = encode_text(*tokenizer, std::string_view(text != nullptr ? text : "", length), out);
        s != GFXI_OK) {
      return s;
    }
    *count = out.size();
    if (const std::size_t n = std::min(out.size(), capacity); n > 0) std::copy_n(out.begin(), n, ids);
    return GFXI_OK;
  });
}

extern "C" int32_t gfxinfer_tokenizer_decode(const gfxinfer_tokenizer* tokenizer, const uint32_t* ids, size_t count,
                                             char* text, size_t capacity, size_t* length) {
  return guarded([&]() -> int32_t {
    if (tokenizer == nullptr || length == nullptr || (ids == nullptr && count != 0) ||
        (text == nullptr && capacity != 0)) {
      return fail(GFXI_INVALID_ARGUMENT, "tokenizer decode arguments are invalid");
    }
    std::string out;
    if (const int32_t s = decode_ids(*tokenizer, ids, count, out); s != GFXI_OK) return s;
    *length = out.size();
    if (const std::size_t n = std::min(out.size(), capacity); n > 0) std::memcpy(text, out.data(), n);
    return GFXI_OK;
  });
}

extern "C" int32_t gfxinfer_render_chat_prompt(const char* prompt, size_t length, char* text, size_t capacity,
                                               size_t* rendered_length) {
  return guarded([&]() -> int32_t {
    if (rendered_length == nullptr || (prompt == nullptr && length != 0) || (text == nullptr && capacity != 0)) {
      return fail(GFXI_INVALID_ARGUMENT, "chat prompt arguments are invalid");
    }
    // One user turn, then the assistant turn opened with an empty thinking block
    // (cli/main.cpp:1037-1039).
    std::string out = "<|im_start|>user\n";
    out.append(prompt != nullptr ? prompt : "", length);
    out.append("<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n");
    *rendered_length = out.size();
    if (const std::size_t n = std::min(out.size(), capacity); n > 0) std::memcpy(text, out.data(), n);
    return GFXI_OK;
  });
}
