// tokenizer_spm.cpp — the SentencePiece Unigram tokenizer of the XLM-R
// family (multilingual-e5, paraphrase-multilingual MiniLM) on the host,
// behind rh_tokenizer_sentencepiece_load.
//
// Mirrors tokenizer/sentencepiece: a proto2 wire reader for the .model file
// (proto.go), the NMT-NFKC normalizer driven by the model's precompiled
// charsmap — a darts-clone double-array trie of replacements — plus the
// whitespace protocol (normalizer.go), Viterbi segmentation over the normal
// pieces with merged unknown runs, and HF's fairseq id space on top
// (sentencepiece.go).
#include <cfloat>
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

const char kSpaceSymbol[] = "\xE2\x96\x81";  // U+2581 LOWER ONE EIGHTH BLOCK
constexpr float kUnkPenalty = 10.0f;          // unigram_model.cc: min score - 10

// ---- proto2 wire reader (proto.go) ---------------------------------------------
struct Field {
  int number, wire;
  const uint8_t* data;  // length-delimited payload
  size_t len;
  uint64_t value;       // varint, fixed32, fixed64
};

bool uvarint(const uint8_t*& p, const uint8_t* end, uint64_t* v) {
  uint64_t x = 0;
  for (int shift = 0; shift < 64 && p < end; shift += 7) {
    const uint8_t b = *p++;
    x |= (uint64_t)(b & 0x7F) << shift;
    if (!(b & 0x80)) {
      *v = x;
      return true;
    }
  }
  return false;
}

template <class F>
void walk(const uint8_t* p, size_t n, F&& fn) {
  const uint8_t* end = p + n;
  while (p < end) {
    uint64_t tag;
    if (!uvarint(p, end, &tag)) throw std::invalid_argument("sentencepiece: bad varint tag");
    Field f{(int)(tag >> 3), (int)(tag & 7), nullptr, 0, 0};
    switch (f.wire) {
      case 0:
        if (!uvarint(p, end, &f.value)) throw std::invalid_argument("sentencepiece: bad varint");
        break;
      case 5:
        if (end - p < 4) throw std::invalid_argument("sentencepiece: short fixed32");
        f.value = (uint64_t)p[0] | ((uint64_t)p[1] << 8) | ((uint64_t)p[2] << 16) |
                  ((uint64_t)p[3] << 24);
        p += 4;
        break;
      case 1:
        if (end - p < 8) throw std::invalid_argument("sentencepiece: short fixed64");
        f.value = 0;
        for (int i = 7; i >= 0; i--) f.value = (f.value << 8) | p[i];
        p += 8;
        break;
      case 2: {
        uint64_t l;
        if (!uvarint(p, end, &l) || (uint64_t)(end - p) < l)
          throw std::invalid_argument("sentencepiece: bad length-delimited field");
        f.data = p;
        f.len = (size_t)l;
        p += l;
        break;
      }
      default:
        throw std::invalid_argument("sentencepiece: unsupported wire type");
    }
    fn(f);
  }
}

struct Piece {
  std::string text;
  float score = 0.0f;
  int kind = 1;  // 1 NORMAL 2 UNKNOWN 3 CONTROL 4 USER_DEFINED 5 UNUSED 6 BYTE
};

struct NormSpec {
  std::string charsmap;
  bool add_dummy_prefix = true, remove_extra_whitespaces = true, escape_whitespaces = true;
};

// ---- the charsmap normalizer (normalizer.go) ---------------------------------------
struct Normalizer {
  std::vector<uint32_t> units;  // darts-clone double array
  std::string blob;             // NUL-terminated replacements
  NormSpec spec;

  void init(const NormSpec& s) {
    spec = s;
    const std::string& m = s.charsmap;
    if (m.empty()) return;  // no charsmap: only the whitespace protocol
    if (m.size() < 4) throw std::invalid_argument("sentencepiece: charsmap too short");
    const uint32_t size = (uint8_t)m[0] | ((uint8_t)m[1] << 8) | ((uint8_t)m[2] << 16) |
                          ((uint32_t)(uint8_t)m[3] << 24);
    if (size % 4 || 4 + (size_t)size > m.size())
      throw std::invalid_argument("sentencepiece: charsmap trie size out of bounds");
    units.resize(size / 4);
    memcpy(units.data(), m.data() + 4, size);  // little-endian host
    blob = m.substr(4 + size);
  }

  // darts.h commonPrefixSearch: the value and length of every key that is a
  // prefix of s (a NUL in s ends the key).
  void longest_prefix(const char* s, size_t n, int* best_len, int* best_val) const {
    *best_len = 0;
    if (units.empty()) return;
    auto has_leaf = [](uint32_t u) { return (u >> 8) & 1; };
    auto value = [](uint32_t u) { return (int)(u & ((1u << 31) - 1)); };
    auto label = [](uint32_t u) { return u & ((1u << 31) | 0xFF); };
    auto offset = [](uint32_t u) { return (u >> 10) << ((u & (1u << 9)) >> 6); };
    uint32_t pos = 0;
    uint32_t unit = units[pos];
    pos ^= offset(unit);
    for (size_t i = 0; i < n; i++) {
      const uint32_t c = (uint8_t)s[i];
      if (c == 0) return;
      pos ^= c;
      if (pos >= units.size()) return;
      unit = units[pos];
      if (label(unit) != c) return;
      pos ^= offset(unit);
      if (has_leaf(unit) && pos < units.size()) {
        // the longest match wins (lengths only grow along the walk)
        *best_len = (int)(i + 1);
        *best_val = value(units[pos]);
      }
    }
  }

  std::string replacement(int v) const {
    if (v < 0 || (size_t)v >= blob.size()) return "";
    const size_t e = blob.find('\0', v);
    return blob.substr(v, e == std::string::npos ? std::string::npos : e - v);
  }

  // NormalizePrefix: the longest charsmap match maps to its replacement,
  // else one valid rune passes, else one invalid byte becomes U+FFFD.
  std::string prefix(const char* s, size_t n, size_t* consumed) const {
    int len, val = 0;
    longest_prefix(s, n, &len, &val);
    if (len == 0) {
      size_t l;
      const char32_t r = decode_rune(reinterpret_cast<const unsigned char*>(s), n, &l);
      *consumed = l;
      if (r == kReplacement && l == 1) return "\xEF\xBF\xBD";
      return std::string(s, l);
    }
    *consumed = (size_t)len;
    return replacement(val);
  }

  // Normalizer::Normalize, flow for flow.
  std::string normalize(const std::string& text) const {
    const char* s = text.data();
    size_t n = text.size();
    if (n == 0) return "";
    if (spec.remove_extra_whitespaces) {  // drop heading pieces that are " "
      while (n > 0) {
        size_t c;
        if (prefix(s, n, &c) != " ") break;
        s += c;
        n -= c;
      }
    }
    if (n == 0) return "";
    std::string out;
    out.reserve(n + 8);
    auto add_ws = [&]() {
      if (spec.escape_whitespaces) out += kSpaceSymbol;
      else out.push_back(' ');
    };
    if (spec.add_dummy_prefix) add_ws();
    bool prev_space = spec.remove_extra_whitespaces;
    while (n > 0) {
      size_t c;
      std::string sp = prefix(s, n, &c);
      size_t skip = 0;
      while (prev_space && skip < sp.size() && sp[skip] == ' ') skip++;
      if (skip < sp.size()) {
        for (size_t i = skip; i < sp.size(); i++) {
          if (spec.escape_whitespaces && sp[i] == ' ') out += kSpaceSymbol;
          else out.push_back(sp[i]);
        }
        prev_space = sp.back() == ' ';
      }
      s += c;
      n -= c;
      if (!spec.remove_extra_whitespaces) prev_space = false;
    }
    if (spec.remove_extra_whitespaces) {
      const std::string trailer = spec.escape_whitespaces ? kSpaceSymbol : " ";
      while (out.size() >= trailer.size() &&
             out.compare(out.size() - trailer.size(), trailer.size(), trailer) == 0)
        out.resize(out.size() - trailer.size());
    }
    return out;
  }
};

struct SentencePiece final : rh_tokenizer {
  Normalizer norm;
  std::unordered_map<std::string, int32_t> piece_id;  // NORMAL pieces
  std::vector<float> scores;
  int max_piece = 0;
  float unk_score = 0.0f;
  int n_pieces = 0;
  static constexpr int64_t kCls = 0, kSep = 2, kUnk = 3;  // fairseq framing

  int64_t vocab_size() const override { return n_pieces + 2; }

  // hfID (sentencepiece.go:110-121): sp <unk>/<s>/</s> to fairseq 3/0/2,
  // every other id shifted by one.
  static int64_t hf_id(int32_t sp) {
    if (sp == 0) return kUnk;
    if (sp == 1) return kCls;
    if (sp == 2) return kSep;
    return (int64_t)sp + 1;
  }

  struct Span {
    int32_t start, end, id;
  };

  // segment (sentencepiece.go:131-200): Viterbi over byte positions; an unk
  // node (score min - 10) only where no one-rune piece starts; consecutive
  // unknown spans merge.
  std::vector<Span> segment(const std::string& s) const {
    const int n = (int)s.size();
    std::vector<Span> out;
    if (n == 0) return out;
    const float neg_inf = -1e30f;
    std::vector<float> best(n + 1, neg_inf);
    std::vector<int32_t> edge(n + 1, 0), from(n + 1, -1);
    best[0] = 0.0f;
    std::string key;
    for (int i = 0; i < n; i++) {
      if (from[i] == -1 && i > 0) continue;
      const float base = best[i];
      size_t rune_len;
      decode_rune(reinterpret_cast<const unsigned char*>(s.data()) + i, n - i, &rune_len);
      bool has_single = false;
      const int limit = std::min(n, i + max_piece);
      for (int j = i + 1; j <= limit; j++) {
        key.assign(s, i, j - i);
        auto it = piece_id.find(key);
        if (it == piece_id.end()) continue;
        if (j - i == (int)rune_len) has_single = true;
        const float sc = base + scores[it->second];
        if (sc > best[j]) {
          best[j] = sc;
          edge[j] = it->second;
          from[j] = i;
        }
      }
      if (!has_single) {
        const int j = i + (int)rune_len;
        const float sc = base + unk_score;
        if (sc > best[j]) {
          best[j] = sc;
          edge[j] = 0;
          from[j] = i;
        }
      }
    }
    std::vector<Span> rev;
    for (int pos = n; pos > 0;) {
      const int f = from[pos];
      if (f < 0) return {Span{0, n, 0}};
      rev.push_back(Span{f, pos, edge[pos]});
      pos = f;
    }
    for (int i = (int)rev.size() - 1; i >= 0; i--) {
      const Span sp = rev[i];
      if (sp.id == 0 && !out.empty() && out.back().id == 0 && out.back().end == sp.start) {
        out.back().end = sp.end;
        continue;
      }
      out.push_back(sp);
    }
    return out;
  }

  // Encode (sentencepiece.go:205-241): <s> pieces </s>; the normalized text
  // is capped at (budget + 16) * max_piece bytes (on a rune start) so the
  // Viterbi work stays bounded by what the budget can use.
  void encode(const char* text, size_t n, int max_len,
              std::vector<int64_t>& ids) const override {
    ids.clear();
    ids.push_back(kCls);
    int budget = std::max(max_len - 2, 0);
    std::string s = norm.normalize(std::string(text, n));
    const size_t cap = (size_t)(budget + 16) * (size_t)max_piece;
    if (s.size() > cap) {
      size_t c = cap;
      while (c > 0 && ((unsigned char)s[c] & 0xC0) == 0x80) c--;
      s.resize(c);
    }
    for (const Span& sp : segment(s)) {
      if (budget <= 0) break;
      ids.push_back(hf_id(sp.id));
      budget--;
    }
    ids.push_back(kSep);
  }
};

}  // namespace

extern "C" {

// sentencepiece.New (tokenizer/sentencepiece/sentencepiece.go:47-103).
int rh_tokenizer_sentencepiece_load(const char* model_path, rh_tokenizer** out) {
  return api_call([&]() -> int {
    if (!model_path || !out) return fail(RH_ERR_INVALID, "null argument");
    *out = nullptr;
    try {
      FILE* f = fopen(model_path, "rb");
      if (!f) return fail(RH_ERR_INVALID, std::string("cannot open ") + model_path);
      std::string raw;
      char buf[1 << 16];
      size_t got;
      while ((got = fread(buf, 1, sizeof buf, f)) > 0) raw.append(buf, got);
      fclose(f);
      std::vector<Piece> pieces;
      NormSpec spec;
      walk(reinterpret_cast<const uint8_t*>(raw.data()), raw.size(), [&](const Field& fl) {
        if (fl.number == 1) {
          if (fl.wire != 2) throw std::invalid_argument("sentencepiece: pieces wire type");
          Piece p;
          walk(fl.data, fl.len, [&](const Field& g) {
            if (g.number == 1 && g.wire == 2) p.text.assign((const char*)g.data, g.len);
            else if (g.number == 2) {
              const uint32_t bits = (uint32_t)g.value;
              memcpy(&p.score, &bits, 4);
            } else if (g.number == 3) p.kind = (int)g.value;
          });
          pieces.push_back(std::move(p));
        } else if (fl.number == 3) {
          if (fl.wire != 2) throw std::invalid_argument("sentencepiece: normalizer wire type");
          walk(fl.data, fl.len, [&](const Field& g) {
            if (g.number == 2 && g.wire == 2) spec.charsmap.assign((const char*)g.data, g.len);
            else if (g.number == 3) spec.add_dummy_prefix = g.value != 0;
            else if (g.number == 4) spec.remove_extra_whitespaces = g.value != 0;
            else if (g.number == 5) spec.escape_whitespaces = g.value != 0;
          });
        }
      });
      if (pieces.empty())
        return fail(RH_ERR_INVALID, "sentencepiece: no pieces (not a SentencePiece model?)");
      std::unique_ptr<SentencePiece> t(new SentencePiece());
      t->norm.init(spec);
      t->n_pieces = (int)pieces.size();
      t->scores.resize(pieces.size());
      float min_score = FLT_MAX;
      for (size_t id = 0; id < pieces.size(); id++) {
        const Piece& p = pieces[id];
        t->scores[id] = p.score;
        if (p.kind == 1) {
          if (!t->piece_id.emplace(p.text, (int32_t)id).second)
            return fail(RH_ERR_INVALID, "sentencepiece: duplicate piece \"" + p.text + "\"");
          t->max_piece = std::max(t->max_piece, (int)p.text.size());
          min_score = std::min(min_score, p.score);
        } else if (p.kind != 2 && p.kind != 3) {
          // USER_DEFINED, UNUSED and BYTE pieces have matching rules this
          // tokenizer does not reproduce (sentencepiece.go:82-90)
          return fail(RH_ERR_INVALID, "sentencepiece: piece \"" + p.text +
                                          "\" has an unsupported type " +
                                          std::to_string(p.kind));
        }
      }
      if (t->max_piece == 0) return fail(RH_ERR_INVALID, "sentencepiece: no normal pieces");
      t->unk_score = min_score - kUnkPenalty;
      *out = t.release();
      return RH_OK;
    } catch (const std::invalid_argument& e) {
      return fail(RH_ERR_INVALID, e.what());
    }
  });
}

// Normalize (sentencepiece.go:244): the model's text normalization alone,
// for tests. *n receives the byte length; RH_ERR_SHAPE when it exceeds
// capacity. RH_ERR_INVALID when t is not a SentencePiece tokenizer.
int rh_tokenizer_sentencepiece_normalize(const rh_tokenizer* t, const char* text,
                                         size_t text_len, char* out, size_t capacity,
                                         size_t* n) {
  return api_call([&]() -> int {
    const auto* sp = dynamic_cast<const SentencePiece*>(t);
    if (!sp || (!text && text_len) || !n) return fail(RH_ERR_INVALID, "not a SentencePiece tokenizer");
    const std::string s = sp->norm.normalize(std::string(text ? text : "", text_len));
    *n = s.size();
    if (s.size() > capacity || (!out && !s.empty()))
      return fail(RH_ERR_SHAPE, "output buffer smaller than the normalized text");
    if (!s.empty()) memcpy(out, s.data(), s.size());
    return RH_OK;
  });
}

}  // extern "C"
