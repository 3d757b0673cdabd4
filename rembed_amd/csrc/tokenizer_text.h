// tokenizer_text.h — text helpers shared by the host-side tokenizers
// (tokenizer.cpp: WordPiece; tokenizer_bpe.cpp: byte-level BPE): Go-style
// UTF-8 decoding, UTF-8 encoding, the Unicode classes the reference's
// tokenizers test with Go's unicode package, and the polymorphic handle
// behind rh_tokenizer_*.
#pragma once

#include <unicode/uchar.h>

#include <cstdint>
#include <string>
#include <vector>

namespace rh {
namespace text {

constexpr char32_t kReplacement = 0xFFFD;

// One rune of a UTF-8 string the way Go's `for _, r := range s` (and
// utf8.DecodeRune) decodes it: an invalid or truncated sequence, an overlong
// form, a surrogate or a value past U+10FFFF yields U+FFFD and consumes one
// byte.
inline char32_t decode_rune(const unsigned char* s, size_t n, size_t* len) {
  const unsigned char c = s[0];
  *len = 1;
  if (c < 0x80) return c;
  int need;
  char32_t r, lo;
  if (c >= 0xC2 && c <= 0xDF) {
    need = 1, r = c & 0x1F, lo = 0x80;
  } else if (c >= 0xE0 && c <= 0xEF) {
    need = 2, r = c & 0x0F, lo = 0x800;
  } else if (c >= 0xF0 && c <= 0xF4) {
    need = 3, r = c & 0x07, lo = 0x10000;
  } else {
    return kReplacement;
  }
  if ((size_t)need >= n) return kReplacement;
  for (int i = 1; i <= need; i++) {
    if ((s[i] & 0xC0) != 0x80) return kReplacement;
    r = (r << 6) | (s[i] & 0x3F);
  }
  if (r < lo || r > 0x10FFFF || (r >= 0xD800 && r <= 0xDFFF)) return kReplacement;
  *len = need + 1;
  return r;
}

inline std::vector<char32_t> decode(const char* text, size_t n) {
  std::vector<char32_t> out;
  out.reserve(n);
  const auto* s = reinterpret_cast<const unsigned char*>(text);
  for (size_t i = 0; i < n;) {
    size_t len;
    out.push_back(decode_rune(s + i, n - i, &len));
    i += len;
  }
  return out;
}

inline void append_utf8(std::string& out, char32_t r) {
  if (r < 0x80) {
    out.push_back((char)r);
  } else if (r < 0x800) {
    out.push_back((char)(0xC0 | (r >> 6)));
    out.push_back((char)(0x80 | (r & 0x3F)));
  } else if (r < 0x10000) {
    out.push_back((char)(0xE0 | (r >> 12)));
    out.push_back((char)(0x80 | ((r >> 6) & 0x3F)));
    out.push_back((char)(0x80 | (r & 0x3F)));
  } else {
    out.push_back((char)(0xF0 | (r >> 18)));
    out.push_back((char)(0x80 | ((r >> 12) & 0x3F)));
    out.push_back((char)(0x80 | ((r >> 6) & 0x3F)));
    out.push_back((char)(0x80 | (r & 0x3F)));
  }
}

inline std::string encode(const char32_t* r, size_t n) {
  std::string s;
  for (size_t i = 0; i < n; i++) append_utf8(s, r[i]);
  return s;
}

// Go's unicode.IsSpace: the Latin-1 set '\t' '\n' '\v' '\f' '\r' ' ' U+0085
// U+00A0, else the White_Space property.
inline bool is_space(char32_t r) {
  if (r <= 0xFF)
    return r == '\t' || r == '\n' || r == '\v' || r == '\f' || r == '\r' || r == ' ' ||
           r == 0x85 || r == 0xA0;
  return u_hasBinaryProperty((UChar32)r, UCHAR_WHITE_SPACE);
}

// unicode.IsLetter: general category L (Lu, Ll, Lt, Lm, Lo).
inline bool is_letter(char32_t r) {
  if (r < 0x80) return (r >= 'a' && r <= 'z') || (r >= 'A' && r <= 'Z');
  return u_isalpha((UChar32)r);
}

// unicode.IsNumber: general category N (Nd, Nl, No).
inline bool is_number(char32_t r) {
  if (r < 0x80) return r >= '0' && r <= '9';
  const int8_t t = u_charType((UChar32)r);
  return t == U_DECIMAL_DIGIT_NUMBER || t == U_LETTER_NUMBER || t == U_OTHER_NUMBER;
}

}  // namespace text
}  // namespace rh

// The handle behind rh_tokenizer_*: one tokenizer of any kind.
struct rh_tokenizer {
  virtual ~rh_tokenizer() = default;
  virtual int64_t vocab_size() const = 0;
  // The framed ids of one UTF-8 text, at most max_len (each kind applies
  // its reference's rule for a max_len below its framing).
  virtual void encode(const char* text, size_t n, int max_len, std::vector<int64_t>& ids) const = 0;
};
