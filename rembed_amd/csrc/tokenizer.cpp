// tokenizer.cpp — BERT WordPiece tokenization on the host, and the C ABI of
// every tokenizer kind (rh_tokenizer_*): text in, the int64 ids
// rh_model_embed takes out. The byte-level BPE kind is in tokenizer_bpe.cpp.
//
// Mirrors tokenizer.New / Encode (tokenizer/tokenizer.go:39-216): a vocab of
// one token per line (id = line number), HF BasicTokenizer cleaning and
// splitting, greedy longest-prefix WordPiece with "##" continuations, and
// [CLS] ... [SEP] framing truncated to max_len. Unicode properties
// (lowercase mapping, NFD, general categories, White_Space) come from ICU.
#include <unicode/normalizer2.h>
#include <unicode/uchar.h>
#include <unicode/unistr.h>

#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "rh_internal.h"
#include "tokenizer_text.h"

using namespace rh;
using namespace rh::text;

namespace {

constexpr int kMaxWordChars = 100;         // max_input_chars_per_word (tokenizer.go:24)
constexpr size_t kMaxLineBytes = 1 << 20;  // the vocab scanner's line limit (tokenizer.go:56)

// isBertPunct (tokenizer.go:81-86): the four ASCII symbol ranges, else
// Unicode category P.
bool is_bert_punct(char32_t r) {
  if (r < 0x80)
    return (r >= 33 && r <= 47) || (r >= 58 && r <= 64) || (r >= 91 && r <= 96) ||
           (r >= 123 && r <= 126);
  return u_ispunct((UChar32)r);
}

// isCJKIdeograph (tokenizer.go:91-104).
bool is_cjk(char32_t r) {
  return (r >= 0x4E00 && r <= 0x9FFF) || (r >= 0x3400 && r <= 0x4DBF) ||
         (r >= 0x20000 && r <= 0x2A6DF) || (r >= 0x2A700 && r <= 0x2B73F) ||
         (r >= 0x2B740 && r <= 0x2B81F) || (r >= 0x2B820 && r <= 0x2CEAF) ||
         (r >= 0xF900 && r <= 0xFAFF) || (r >= 0x2F800 && r <= 0x2FA1F);
}

// Cc, Cf, Co, Cs: the category-C characters the cleaning step deletes (Cn,
// unassigned, is kept; tokenizer.go:136-151).
bool is_deleted_control(char32_t r) {
  const int8_t t = u_charType((UChar32)r);
  return t == U_CONTROL_CHAR || t == U_FORMAT_CHAR || t == U_PRIVATE_USE_CHAR ||
         t == U_SURROGATE;
}

struct WordPiece final : rh_tokenizer {
  std::unordered_map<std::string, int64_t> vocab;
  bool lower = true;
  int64_t cls = 0, sep = 0, unk = 0;

  // basicTokens (tokenizer.go:110-162): lowercase + NFD when lowercasing,
  // then clean and split into words (each a UTF-8 string).
  std::vector<std::string> basic_tokens(const char* text, size_t n) const {
    std::vector<char32_t> runes = decode(text, n);
    if (lower) {
      // strings.ToLower (per-rune simple mapping; invalid bytes became
      // U+FFFD above), then norm.NFD
      icu::UnicodeString u;
      for (char32_t& r : runes) u.append((UChar32)u_tolower((UChar32)r));
      UErrorCode st = U_ZERO_ERROR;
      const icu::Normalizer2* nfd = icu::Normalizer2::getNFDInstance(st);
      if (U_FAILURE(st)) throw std::runtime_error("ICU NFD normalizer unavailable");
      const icu::UnicodeString d = nfd->normalize(u, st);
      if (U_FAILURE(st)) throw std::runtime_error("ICU NFD normalization failed");
      runes.clear();
      for (int32_t i = 0; i < d.length();) {
        const UChar32 c = d.char32At(i);
        runes.push_back((char32_t)c);
        i += U16_LENGTH(c);
      }
    }
    std::vector<std::string> out;
    std::string cur;
    auto flush = [&]() {
      if (!cur.empty()) {
        out.push_back(cur);
        cur.clear();
      }
    };
    for (char32_t r : runes) {
      if (lower && u_charType((UChar32)r) == U_NON_SPACING_MARK) continue;  // accents
      if (r == kReplacement) continue;
      if (r == '\t' || r == '\n' || r == '\r') {
        flush();
      } else if (is_deleted_control(r)) {
        continue;
      } else if (is_space(r)) {
        flush();
      } else if (is_cjk(r) || is_bert_punct(r)) {
        flush();
        std::string one;
        append_utf8(one, r);
        out.push_back(one);
      } else {
        append_utf8(cur, r);
      }
    }
    flush();
    return out;
  }

  // wordPiece (tokenizer.go:166-194): greedy longest vocab prefix, "##" for
  // continuations, the whole word [UNK] when a piece is missing or the
  // word is longer than 100 runes.
  void word_piece(const std::string& word, std::vector<int64_t>& out) const {
    const std::vector<char32_t> r = decode(word.data(), word.size());
    if ((int)r.size() > kMaxWordChars) {
      out.push_back(unk);
      return;
    }
    std::vector<int64_t> ids;
    size_t start = 0;
    std::string sub;
    while (start < r.size()) {
      size_t end = r.size();
      int64_t id = -1;
      while (start < end) {
        sub.assign(start > 0 ? "##" : "");
        for (size_t i = start; i < end; i++) append_utf8(sub, r[i]);
        auto it = vocab.find(sub);
        if (it != vocab.end()) {
          id = it->second;
          break;
        }
        end--;
      }
      if (id < 0) {
        out.push_back(unk);
        return;
      }
      ids.push_back(id);
      start = end;
    }
    out.insert(out.end(), ids.begin(), ids.end());
  }

  int64_t vocab_size() const override { return (int64_t)vocab.size(); }

  // Encode (tokenizer.go:198-216): [CLS] pieces [SEP], at most max_len ids.
  void encode(const char* text, size_t n, int max_len,
              std::vector<int64_t>& ids) const override {
    if (max_len < 2) max_len = 2;
    ids.clear();
    ids.push_back(cls);
    std::vector<int64_t> pieces;
    bool full = false;
    for (const std::string& w : basic_tokens(text, n)) {
      pieces.clear();
      word_piece(w, pieces);
      for (int64_t id : pieces) {
        if ((int)ids.size() >= max_len - 1) {
          full = true;
          break;
        }
        ids.push_back(id);
      }
      if (full) break;
    }
    ids.push_back(sep);
  }
};

}  // namespace

extern "C" {

int rh_tokenizer_wordpiece_load(const char* vocab_path, int lower_case, const char* cls_tok,
                                const char* sep_tok, const char* unk_tok, rh_tokenizer** out) {
  return api_call([&]() -> int {
    if (!vocab_path || !out) return fail(RH_ERR_INVALID, "null argument");
    *out = nullptr;
    const std::string cls = cls_tok && *cls_tok ? cls_tok : "[CLS]";
    const std::string sep = sep_tok && *sep_tok ? sep_tok : "[SEP]";
    const std::string unk = unk_tok && *unk_tok ? unk_tok : "[UNK]";
    FILE* f = fopen(vocab_path, "rb");
    if (!f) return fail(RH_ERR_INVALID, std::string("cannot open vocab ") + vocab_path);
    std::string data;
    char buf[1 << 16];
    size_t got;
    while ((got = fread(buf, 1, sizeof buf, f)) > 0) data.append(buf, got);
    const bool read_err = ferror(f) != 0;
    fclose(f);
    if (read_err) return fail(RH_ERR_INVALID, std::string("cannot read vocab ") + vocab_path);
    std::unique_ptr<WordPiece> t(new WordPiece());
    t->lower = lower_case != 0;
    // bufio.ScanLines: lines end at '\n', a trailing '\r' is dropped, a last
    // line without '\n' counts, an empty remainder after the last '\n' does
    // not; a later duplicate overrides an earlier one
    int64_t id = 0;
    for (size_t pos = 0; pos < data.size();) {
      size_t nl = data.find('\n', pos);
      const size_t end = nl == std::string::npos ? data.size() : nl;
      size_t len = end - pos;
      if (len > kMaxLineBytes) return fail(RH_ERR_INVALID, "vocab line longer than 1 MiB");
      if (len > 0 && data[pos + len - 1] == '\r') len--;
      t->vocab[data.substr(pos, len)] = id++;
      pos = nl == std::string::npos ? data.size() : nl + 1;
    }
    for (const std::string* s : {&cls, &sep, &unk})
      if (!t->vocab.count(*s))
        return fail(RH_ERR_MISSING, "vocab " + std::string(vocab_path) +
                                        " is missing the special token " + *s);
    t->cls = t->vocab[cls];
    t->sep = t->vocab[sep];
    t->unk = t->vocab[unk];
    *out = t.release();
    return RH_OK;
  });
}

int64_t rh_tokenizer_vocab_size(const rh_tokenizer* t) { return t ? t->vocab_size() : 0; }

int rh_tokenizer_encode(const rh_tokenizer* t, const char* text, size_t text_len, int max_len,
                        int64_t* ids, int capacity, int* n) {
  return api_call([&]() -> int {
    if (!t || (!text && text_len) || !ids || !n) return fail(RH_ERR_INVALID, "null argument");
    std::vector<int64_t> v;
    t->encode(text ? text : "", text_len, max_len, v);
    *n = (int)v.size();
    if ((int)v.size() > capacity)
      return fail(RH_ERR_SHAPE, "ids buffer smaller than the encoded length");
    memcpy(ids, v.data(), v.size() * sizeof(int64_t));
    return RH_OK;
  });
}

int rh_tokenizer_encode_batch(const rh_tokenizer* t, const char* const* texts,
                              const size_t* text_lens, int batch, int max_len, int64_t pad_id,
                              int64_t* ids, int32_t* lens) {
  return api_call([&]() -> int {
    if (!t || (batch > 0 && (!texts || !text_lens || !ids || !lens)) || batch < 0)
      return fail(RH_ERR_INVALID, "null argument or negative batch");
    const int stride = max_len < 2 ? 2 : max_len;
    std::vector<int64_t> v;
    for (int b = 0; b < batch; b++) {
      if (!texts[b] && text_lens[b]) return fail(RH_ERR_INVALID, "null text");
      t->encode(texts[b] ? texts[b] : "", text_lens[b], max_len, v);
      if (v.size() > (size_t)stride) return fail(RH_ERR_INVALID, "encoded row exceeds max_len");
      int64_t* row = ids + (size_t)b * stride;
      memcpy(row, v.data(), v.size() * sizeof(int64_t));
      for (size_t i = v.size(); i < (size_t)stride; i++) row[i] = pad_id;
      lens[b] = (int32_t)v.size();
    }
    return RH_OK;
  });
}

void rh_tokenizer_destroy(rh_tokenizer* t) {
  api_void([&]() { delete t; });
}

}  // extern "C"
