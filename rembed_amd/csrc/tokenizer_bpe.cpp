// tokenizer_bpe.cpp — byte-level BPE tokenization on the host (RoBERTa /
// GPT-2, ModernBERT, Qwen3), behind rh_tokenizer_bpe_load*, and Gemma's
// byte-fallback BPE behind rh_tokenizer_gemma_load.
//
// Mirrors tokenizer/bpe/bpe.go: text (NFC-normalized when the
// tokenizer.json declares it) is matched for added tokens leftmost-longest
// (tokenizer.json kinds only), the gaps are pre-tokenized with GPT-2's
// pattern or the Qwen pattern, each pre-token's UTF-8 bytes go through the
// bytes-to-unicode table, and adjacent symbols merge by rank (lowest first,
// leftmost among equals) until no ranked pair remains. Framing: cls ... sep
// (RoBERTa, ModernBERT) or a trailing eos alone (Qwen3), truncated so the
// suffix always survives.
#include <unicode/normalizer2.h>
#include <unicode/unistr.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <queue>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "rh_internal.h"
#include "tokenizer_text.h"

using namespace rh;
using namespace rh::text;

namespace {

// ---- a minimal JSON reader (vocab.json, tokenizer.json) ----------------------
struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;  // in file order

  const Json* get(const char* key) const {
    if (kind != Object) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char* p;
  const char* end;
  int depth = 0;

  [[noreturn]] void bad(const char* what) {
    throw std::runtime_error(std::string("tokenizer JSON: ") + what);
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  unsigned hex4() {
    if (end - p < 4) bad("short \\u escape");
    unsigned v = 0;
    for (int i = 0; i < 4; i++) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else bad("bad \\u escape");
    }
    return v;
  }
  // encoding/json's string rules: escapes decoded, a lone surrogate escape
  // becomes U+FFFD, invalid UTF-8 bytes become U+FFFD
  std::string string() {
    if (p >= end || *p != '"') bad("expected a string");
    p++;
    std::string s;
    while (true) {
      if (p >= end) bad("unterminated string");
      const unsigned char c = *p;
      if (c == '"') {
        p++;
        return s;
      }
      if (c < 0x20) bad("control character in string");
      if (c == '\\') {
        p++;
        if (p >= end) bad("unterminated escape");
        const char e = *p++;
        switch (e) {
          case '"': s.push_back('"'); break;
          case '\\': s.push_back('\\'); break;
          case '/': s.push_back('/'); break;
          case 'b': s.push_back('\b'); break;
          case 'f': s.push_back('\f'); break;
          case 'n': s.push_back('\n'); break;
          case 'r': s.push_back('\r'); break;
          case 't': s.push_back('\t'); break;
          case 'u': {
            char32_t r = hex4();
            if (r >= 0xD800 && r <= 0xDBFF) {
              if (end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                const char* save = p;
                p += 2;
                const unsigned lo = hex4();
                if (lo >= 0xDC00 && lo <= 0xDFFF) {
                  r = 0x10000 + ((r - 0xD800) << 10) + (lo - 0xDC00);
                } else {
                  p = save;  // the next escape stands alone
                  r = kReplacement;
                }
              } else {
                r = kReplacement;
              }
            } else if (r >= 0xDC00 && r <= 0xDFFF) {
              r = kReplacement;
            }
            append_utf8(s, r);
            break;
          }
          default: bad("bad escape");
        }
        continue;
      }
      size_t len;
      const char32_t r = decode_rune(reinterpret_cast<const unsigned char*>(p), end - p, &len);
      if (r == kReplacement && len == 1) append_utf8(s, kReplacement);  // invalid byte
      else s.append(p, len);
      p += len;
    }
  }
  Json value() {
    ws();
    if (p >= end) bad("unexpected end");
    Json j;
    const char c = *p;
    if (c == '{' || c == '[') {
      if (++depth > 64) bad("nesting too deep");
      const bool obj = c == '{';
      j.kind = obj ? Json::Object : Json::Array;
      p++;
      ws();
      if (p < end && *p == (obj ? '}' : ']')) {
        p++;
        depth--;
        return j;
      }
      while (true) {
        ws();
        if (obj) {
          std::string k = string();
          ws();
          if (p >= end || *p != ':') bad("expected ':'");
          p++;
          j.obj.emplace_back(std::move(k), value());
        } else {
          j.arr.push_back(value());
        }
        ws();
        if (p < end && *p == ',') {
          p++;
          continue;
        }
        if (p < end && *p == (obj ? '}' : ']')) {
          p++;
          break;
        }
        bad("expected ',' or a closing bracket");
      }
      depth--;
      return j;
    }
    if (c == '"') {
      j.kind = Json::String;
      j.str = string();
      return j;
    }
    if (end - p >= 4 && !strncmp(p, "true", 4)) {
      p += 4;
      j.kind = Json::Bool;
      j.b = true;
      return j;
    }
    if (end - p >= 5 && !strncmp(p, "false", 5)) {
      p += 5;
      j.kind = Json::Bool;
      return j;
    }
    if (end - p >= 4 && !strncmp(p, "null", 4)) {
      p += 4;
      return j;
    }
    const char* q = p;
    if (q < end && *q == '-') q++;
    while (q < end && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' ||
                       *q == '+' || *q == '-'))
      q++;
    if (q == p) bad("unexpected character");
    j.kind = Json::Number;
    j.num = std::stod(std::string(p, q));
    p = q;
    return j;
  }
};

Json parse_json_file(const char* path) {
  FILE* f = fopen(path, "rb");
  if (!f) throw std::invalid_argument(std::string("cannot open ") + path);
  std::string data;
  char buf[1 << 16];
  size_t got;
  while ((got = fread(buf, 1, sizeof buf, f)) > 0) data.append(buf, got);
  fclose(f);
  JsonParser jp{data.data(), data.data() + data.size()};
  Json j = jp.value();
  jp.ws();
  if (jp.p != jp.end) jp.bad("trailing data");
  return j;
}

int64_t json_int(const Json& j, const char* what) {
  if (j.kind != Json::Number || j.num != (double)(int64_t)j.num)
    throw std::invalid_argument(std::string("tokenizer JSON: ") + what + " is not an integer");
  return (int64_t)j.num;
}

// ---- the byte-level BPE tokenizer -------------------------------------------------
struct AddedTok {
  int64_t id;
  bool lstrip, rstrip;
};

struct Bpe final : rh_tokenizer {
  std::unordered_map<std::string, int64_t> vocab;
  std::unordered_map<std::string, int> ranks;  // key: pair_key(a, b)
  char32_t byte_enc[256];
  int64_t cls = 0, sep = 0, unk = 0;
  bool nfc = false, qwen = false, no_prefix = false;
  bool has_added = false;
  std::unordered_map<std::string, AddedTok> added;
  bool added_first[256] = {};
  int added_min = 0, added_max = 0;
  std::vector<std::pair<std::string, int64_t>> lstrip_toks;

  Bpe() {
    // byteToUnicode (bpe.go:83-99): printable Latin-1 to itself, every other
    // byte to 256 + n in byte order
    int n = 0;
    for (int b = 0; b < 256; b++) {
      const bool printable = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) ||
                             (b >= 0xAE && b <= 0xFF);
      byte_enc[b] = printable ? (char32_t)b : (char32_t)(256 + n++);
    }
  }

  static std::string pair_key(const std::string& a, const std::string& b) {
    std::string k = std::to_string(a.size());
    k.push_back(':');
    k += a;
    k += b;
    return k;
  }

  int64_t vocab_size() const override { return (int64_t)vocab.size(); }

  // GPT-2's pattern (bpe.go:311-405):
  //   's|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+
  void pre_gpt2(const std::vector<char32_t>& rs, std::vector<std::string>& out) const {
    static const char* kSuf[] = {"s", "t", "re", "ve", "m", "ll", "d"};
    const size_t n = rs.size();
    size_t i = 0;
    while (i < n) {
      const char32_t r = rs[i];
      if (r == '\'' && i + 1 < n) {  // contractions: literal, case-sensitive
        const char* m = nullptr;
        for (const char* suf : kSuf) {
          const size_t L = strlen(suf);
          bool ok = i + 1 + L <= n;
          for (size_t q = 0; ok && q < L; q++) ok = rs[i + 1 + q] == (char32_t)suf[q];
          if (ok) {
            m = suf;
            break;
          }
        }
        if (m) {
          const size_t L = strlen(m);
          out.push_back(rh::text::encode(&rs[i], 1 + L));
          i += 1 + L;
          continue;
        }
      }
      size_t j = r == ' ' ? i + 1 : i;  // only a literal space joins as " ?"
      if (j < n) {
        const char32_t c = rs[j];
        size_t k = j;
        if (is_letter(c)) {
          while (k < n && is_letter(rs[k])) k++;
        } else if (is_number(c)) {
          while (k < n && is_number(rs[k])) k++;
        } else if (!is_space(c)) {
          while (k < n && !is_space(rs[k]) && !is_letter(rs[k]) && !is_number(rs[k])) k++;
        }
        if (k > j) {
          out.push_back(rh::text::encode(&rs[i], k - i));
          i = k;
          continue;
        }
      }
      // \s+(?!\S), then \s+: rs[i] is whitespace here
      size_t k = i;
      while (k < n && is_space(rs[k])) k++;
      const size_t stop = k == n ? k : (k - i > 1 ? k - 1 : k);
      out.push_back(rh::text::encode(&rs[i], stop - i));
      i = stop;
    }
  }

  // Case-insensitive ASCII suffix letter match of strings.EqualFold over
  // the contraction letters (s t r e v m l d): simple case folding adds
  // only U+017F (long s) for 's'.
  static bool fold_eq(char32_t r, char c) {
    if (r == (char32_t)c || r == (char32_t)(c - 'a' + 'A')) return true;
    return c == 's' && r == 0x17F;
  }

  // The Qwen / GPT-NeoX pattern (bpe.go:416-519):
  //   (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}|
  //   ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+
  void pre_qwen(const std::vector<char32_t>& rs, std::vector<std::string>& out) const {
    static const char* kSuf[] = {"s", "t", "re", "ve", "m", "ll", "d"};
    auto nl = [](char32_t c) { return c == '\r' || c == '\n'; };
    const size_t n = rs.size();
    size_t i = 0;
    while (i < n) {
      const char32_t r = rs[i];
      if (r == '\'' && i + 1 < n) {
        size_t L = 0;
        for (const char* suf : kSuf) {
          const size_t sl = strlen(suf);
          bool ok = i + 1 + sl <= n;
          for (size_t q = 0; ok && q < sl; q++) ok = fold_eq(rs[i + 1 + q], suf[q]);
          if (ok) {
            L = sl;
            break;
          }
        }
        if (L) {
          out.push_back(rh::text::encode(&rs[i], 1 + L));
          i += 1 + L;
          continue;
        }
      }
      {  // [^\r\n\p{L}\p{N}]?\p{L}+
        size_t j = i;
        if (!nl(r) && !is_letter(r) && !is_number(r) && i + 1 < n && is_letter(rs[i + 1]))
          j = i + 1;
        if (j < n && is_letter(rs[j])) {
          size_t k = j;
          while (k < n && is_letter(rs[k])) k++;
          out.push_back(rh::text::encode(&rs[i], k - i));
          i = k;
          continue;
        }
      }
      if (is_number(r)) {  // \p{N}: one at a time
        out.push_back(rh::text::encode(&rs[i], 1));
        i++;
        continue;
      }
      {  //  ?[^\s\p{L}\p{N}]+[\r\n]*
        const size_t j = r == ' ' ? i + 1 : i;
        if (j < n && !is_space(rs[j]) && !is_letter(rs[j]) && !is_number(rs[j])) {
          size_t k = j;
          while (k < n && !is_space(rs[k]) && !is_letter(rs[k]) && !is_number(rs[k])) k++;
          while (k < n && nl(rs[k])) k++;
          out.push_back(rh::text::encode(&rs[i], k - i));
          i = k;
          continue;
        }
      }
      size_t k = i;
      while (k < n && is_space(rs[k])) k++;
      size_t last = n;  // \s*[\r\n]+: cut after the run's last newline
      for (size_t q = i; q < k; q++)
        if (nl(rs[q])) last = q;
      if (last != n) {
        out.push_back(rh::text::encode(&rs[i], last + 1 - i));
        i = last + 1;
        continue;
      }
      const size_t stop = k == n ? k : (k - i > 1 ? k - 1 : k);
      out.push_back(rh::text::encode(&rs[i], stop - i));
      i = stop;
    }
  }

  // bpe (bpe.go:535-590): merge the lowest-ranked adjacent pair, leftmost
  // among equal ranks, until none is ranked; candidates whose symbols
  // changed since they were queued are skipped.
  void merge(const std::vector<std::string>& start, std::vector<std::string>& out) const {
    out.clear();
    const int n = (int)start.size();
    if (n < 2) {
      out = start;
      return;
    }
    std::vector<std::string> syms = start;
    std::vector<int> next(n), prev(n);
    std::vector<char> alive(n, 1);
    for (int i = 0; i < n; i++) {
      next[i] = i + 1;
      prev[i] = i - 1;
    }
    next[n - 1] = -1;
    struct Cand {
      int rank, pos;
      std::string left, right;
      bool operator>(const Cand& o) const {
        return rank != o.rank ? rank > o.rank : pos > o.pos;
      }
    };
    std::priority_queue<Cand, std::vector<Cand>, std::greater<Cand>> heap;
    auto push = [&](int left) {
      const int right = next[left];
      if (right == -1) return;
      auto it = ranks.find(pair_key(syms[left], syms[right]));
      if (it != ranks.end()) heap.push(Cand{it->second, left, syms[left], syms[right]});
    };
    for (int i = 0; i + 1 < n; i++) push(i);
    while (!heap.empty()) {
      Cand c = heap.top();
      heap.pop();
      const int i = c.pos, j = next[i];
      if (!alive[i] || j == -1 || syms[i] != c.left || syms[j] != c.right) continue;
      syms[i] = c.left + c.right;
      alive[j] = 0;
      next[i] = next[j];
      if (next[j] != -1) prev[next[j]] = i;
      if (prev[i] != -1) push(prev[i]);
      push(i);
    }
    for (int i = 0; i != -1; i = next[i])
      if (alive[i]) out.push_back(syms[i]);
  }

  // Byte-BPE over one gap of ordinary text, appending ids while the budget
  // lasts; false once it ran out (bpe.go:673-699).
  bool emit(const std::string& gap, int& budget, std::vector<int64_t>& ids) const {
    const std::vector<char32_t> rs = decode(gap.data(), gap.size());
    std::vector<std::string> pres, start, merged;
    if (qwen) pre_qwen(rs, pres);
    else pre_gpt2(rs, pres);
    for (const std::string& pre : pres) {
      start.clear();
      for (unsigned char b : pre) {
        std::string s;
        append_utf8(s, byte_enc[b]);
        start.push_back(std::move(s));
      }
      merge(start, merged);
      for (const std::string& sym : merged) {
        if (budget <= 0) return false;
        auto it = vocab.find(sym);
        ids.push_back(it == vocab.end() ? unk : it->second);
        budget--;
      }
    }
    return true;
  }

  // byte length of the Unicode whitespace run at b[pos] (bpe.go:788-804)
  static size_t ws_run(const std::string& b, size_t pos) {
    size_t n = 0;
    while (pos + n < b.size()) {
      size_t len;
      const char32_t r =
          decode_rune(reinterpret_cast<const unsigned char*>(b.data()) + pos + n,
                      b.size() - pos - n, &len);
      if (!is_space(r)) break;
      n += len;
    }
    return n;
  }

  // matchAdded (bpe.go:748-786): the longest added-token span starting at
  // b[i] — a literal content (plus trailing whitespace when rstrip), or for
  // lstrip tokens a whitespace run followed by the content.
  bool match_added(const std::string& b, size_t i, size_t* len, int64_t* id) const {
    size_t best = 0;
    bool found = false;
    if (added_first[(unsigned char)b[i]]) {
      const size_t hi = std::min<size_t>(added_max, b.size() - i);
      for (size_t l = hi; l >= (size_t)added_min && l > 0; l--) {
        auto it = added.find(b.substr(i, l));
        if (it != added.end()) {
          size_t consumed = l;
          if (it->second.rstrip) consumed += ws_run(b, i + l);
          best = consumed;
          *id = it->second.id;
          found = true;
          break;
        }
      }
    }
    const size_t w = i + ws_run(b, i);
    if (w > i) {
      for (const auto& lt : lstrip_toks) {
        if (w + lt.first.size() <= b.size() && b.compare(w, lt.first.size(), lt.first) == 0) {
          size_t consumed = (w - i) + lt.first.size();
          if (added.at(lt.first).rstrip) consumed += ws_run(b, w + lt.first.size());
          if (consumed > best) {
            best = consumed;
            *id = lt.second;
            found = true;
          }
        }
      }
    }
    *len = best;
    return found;
  }

  // Encode (bpe.go:648-742)
  void encode(const char* text, size_t n, int max_len,
              std::vector<int64_t>& ids) const override {
    std::vector<char32_t> rs = decode(text, n);
    if (nfc) {
      icu::UnicodeString u;
      for (char32_t r : rs) u.append((UChar32)r);
      UErrorCode st = U_ZERO_ERROR;
      const icu::Normalizer2* norm = icu::Normalizer2::getNFCInstance(st);
      if (U_FAILURE(st)) throw std::runtime_error("ICU NFC normalizer unavailable");
      const icu::UnicodeString d = norm->normalize(u, st);
      if (U_FAILURE(st)) throw std::runtime_error("ICU NFC normalization failed");
      rs.clear();
      for (int32_t i = 0; i < d.length();) {
        const UChar32 c = d.char32At(i);
        rs.push_back((char32_t)c);
        i += U16_LENGTH(c);
      }
    }
    const std::string b = rh::text::encode(rs.data(), rs.size());
    ids.clear();
    int framing = 1;
    if (!no_prefix) {
      ids.push_back(cls);
      framing++;
    }
    int budget = std::max(max_len - framing, 0);
    if (!has_added) {
      emit(b, budget, ids);
    } else {
      size_t gap = 0, i = 0;
      while (i < b.size()) {
        size_t ml;
        int64_t id;
        if (!match_added(b, i, &ml, &id)) {
          i++;
          continue;
        }
        if (gap < i && !emit(b.substr(gap, i - gap), budget, ids)) {
          gap = b.size();
          break;
        }
        if (budget <= 0) {
          gap = b.size();
          break;
        }
        ids.push_back(id);
        budget--;
        i += ml;
        gap = i;
      }
      if (gap < b.size()) emit(b.substr(gap), budget, ids);
    }
    ids.push_back(sep);
  }

  int64_t lookup(const std::string& tok, const char* what) const {
    auto it = vocab.find(tok);
    if (it == vocab.end())
      throw std::invalid_argument(std::string("bpe: ") + what + " token \"" + tok +
                                  "\" is not in the vocabulary");
    return it->second;
  }
};

// parseBPEJSON (bpe.go:160-268): vocab, merges (either [["a","b"]] or
// ["a b"]), added tokens (merged into the vocab and kept for matching) and
// the NFC normalizer flag of a tokenizer.json.
std::unique_ptr<Bpe> parse_tokenizer_json(const char* path) {
  const Json j = parse_json_file(path);
  const Json* model = j.get("model");
  if (!model || model->kind != Json::Object) throw std::invalid_argument("bpe: no model");
  const Json* type = model->get("type");
  if (!type || type->kind != Json::String || type->str != "BPE")
    throw std::invalid_argument("bpe: model.type is not BPE");
  const Json* vocab = model->get("vocab");
  if (!vocab || vocab->kind != Json::Object || vocab->obj.empty())
    throw std::invalid_argument("bpe: empty model.vocab");
  std::unique_ptr<Bpe> t(new Bpe());
  for (const auto& kv : vocab->obj) t->vocab[kv.first] = json_int(kv.second, "a vocab id");
  if (const Json* norm = j.get("normalizer"))
    if (const Json* nt = norm->get("type"))
      t->nfc = nt->kind == Json::String && nt->str == "NFC";
  int amin = 1 << 30, amax = 0;
  if (const Json* at = j.get("added_tokens")) {
    if (at->kind != Json::Array) throw std::invalid_argument("bpe: added_tokens is not a list");
    for (const Json& a : at->arr) {
      const Json* content = a.get("content");
      const Json* id = a.get("id");
      if (!content || content->kind != Json::String || !id)
        throw std::invalid_argument("bpe: malformed added token");
      if (content->str.empty()) continue;
      const int64_t tid = json_int(*id, "an added token id");
      const Json* ls = a.get("lstrip");
      const Json* rs = a.get("rstrip");
      const bool lstrip = ls && ls->kind == Json::Bool && ls->b;
      const bool rstrip = rs && rs->kind == Json::Bool && rs->b;
      t->vocab[content->str] = tid;
      t->added[content->str] = AddedTok{tid, lstrip, rstrip};
      t->added_first[(unsigned char)content->str[0]] = true;
      if (lstrip) {
        // a later duplicate replaces the earlier one in the map; the list
        // keeps every lstrip entry as the reference's slice does
        t->lstrip_toks.emplace_back(content->str, tid);
      }
      amin = std::min<int>(amin, (int)content->str.size());
      amax = std::max<int>(amax, (int)content->str.size());
    }
  }
  if (amin > amax) amin = amax;
  t->added_min = amin;
  t->added_max = amax;
  t->has_added = true;
  const Json* merges = model->get("merges");
  if (!merges || merges->kind != Json::Array) throw std::invalid_argument("bpe: no merges");
  int rank = 0;
  for (const Json& m : merges->arr) {
    std::string a, b;
    if (m.kind == Json::Array) {
      if (m.arr.size() != 2 || m.arr[0].kind != Json::String || m.arr[1].kind != Json::String)
        throw std::invalid_argument("bpe: malformed merge");
      a = m.arr[0].str;
      b = m.arr[1].str;
    } else if (m.kind == Json::String) {
      const size_t sp = m.str.find(' ');
      if (sp == std::string::npos || sp == 0 || sp + 1 == m.str.size())
        throw std::invalid_argument("bpe: malformed merge \"" + m.str + "\"");
      a = m.str.substr(0, sp);
      b = m.str.substr(sp + 1);
    } else {
      throw std::invalid_argument("bpe: merges are neither [[a,b]] nor [\"a b\"]");
    }
    t->ranks[Bpe::pair_key(a, b)] = rank++;
  }
  if (rank == 0) throw std::invalid_argument("bpe: no merges");
  return t;
}

// ---- Gemma: SentencePiece-style BPE with byte fallback (tokenizer/gemma) -----------
// The ASCII space becomes U+2581 and nothing else is normalized; BPE runs
// over the whole normalized string; a rune absent from the vocab enters as
// its UTF-8 bytes, each the "<0xNN>" piece; <bos> ... <eos> framing with
// the pieces truncated to max_len - 2 (gemma.go:146-254).
struct GemmaBpe final : rh_tokenizer {
  std::unordered_map<std::string, int64_t> vocab;
  std::unordered_map<std::string, int> ranks;  // first occurrence of a pair wins
  int64_t bos = -1, eos = -1, unk = -1;

  int64_t vocab_size() const override { return (int64_t)vocab.size(); }

  void encode(const char* text, size_t n, int max_len,
              std::vector<int64_t>& ids) const override {
    // strings.ReplaceAll(text, " ", "\u2581") on the raw bytes, then the
    // runes of the result (invalid bytes read as U+FFFD)
    std::string norm;
    norm.reserve(n + 16);
    for (size_t i = 0; i < n; i++) {
      if (text[i] == ' ') norm += "\xE2\x96\x81";
      else norm.push_back(text[i]);
    }
    std::vector<std::string> syms;
    const std::vector<char32_t> rs = decode(norm.data(), norm.size());
    for (char32_t r : rs) {
      std::string s;
      append_utf8(s, r);
      if (vocab.count(s)) {
        syms.push_back(std::move(s));
        continue;
      }
      for (unsigned char b : s) {
        char piece[8];
        snprintf(piece, sizeof piece, "<0x%02X>", b);
        syms.push_back(piece);
      }
    }
    std::vector<int64_t> pieces;
    const int m = (int)syms.size();
    if (m > 0) {
      std::vector<int> next(m), prev(m);
      std::vector<char> alive(m, 1);
      for (int i = 0; i < m; i++) {
        next[i] = i + 1;
        prev[i] = i - 1;
      }
      next[m - 1] = -1;
      struct Cand {
        int rank, pos;
        std::string left, right;
        bool operator>(const Cand& o) const {
          return rank != o.rank ? rank > o.rank : pos > o.pos;
        }
      };
      std::priority_queue<Cand, std::vector<Cand>, std::greater<Cand>> heap;
      auto push = [&](int left) {
        if (left < 0) return;
        const int right = next[left];
        if (right < 0) return;
        auto it = ranks.find(Bpe::pair_key(syms[left], syms[right]));
        if (it != ranks.end()) heap.push(Cand{it->second, left, syms[left], syms[right]});
      };
      for (int i = 0; i < m; i++) push(i);
      while (!heap.empty()) {
        Cand c = heap.top();
        heap.pop();
        const int i = c.pos, j = next[i];
        if (!alive[i] || j < 0 || syms[i] != c.left || syms[j] != c.right) continue;
        syms[i] = c.left + c.right;
        alive[j] = 0;
        next[i] = next[j];
        if (next[j] >= 0) prev[next[j]] = i;
        push(prev[i]);
        push(i);
      }
      for (int i = 0; i >= 0; i = next[i]) {
        if (!alive[i]) continue;
        auto it = vocab.find(syms[i]);
        pieces.push_back(it == vocab.end() ? unk : it->second);
      }
    }
    const size_t budget = (size_t)std::max(max_len - 2, 0);
    if (pieces.size() > budget) pieces.resize(budget);
    ids.clear();
    ids.push_back(bos);
    ids.insert(ids.end(), pieces.begin(), pieces.end());
    ids.push_back(eos);
  }
};

}  // namespace

extern "C" {

// New (bpe.go:104-157): vocab.json + merges.txt, RoBERTa framing.
int rh_tokenizer_bpe_load(const char* vocab_json, const char* merges_txt, const char* cls_tok,
                          const char* sep_tok, const char* unk_tok, rh_tokenizer** out) {
  return api_call([&]() -> int {
    if (!vocab_json || !merges_txt || !cls_tok || !sep_tok || !unk_tok || !out)
      return fail(RH_ERR_INVALID, "null argument");
    *out = nullptr;
    try {
      const Json v = parse_json_file(vocab_json);
      if (v.kind != Json::Object) return fail(RH_ERR_INVALID, "bpe: vocab.json is not an object");
      std::unique_ptr<Bpe> t(new Bpe());
      for (const auto& kv : v.obj) t->vocab[kv.first] = json_int(kv.second, "a vocab id");
      FILE* f = fopen(merges_txt, "rb");
      if (!f) return fail(RH_ERR_INVALID, std::string("cannot open ") + merges_txt);
      std::string data;
      char buf[1 << 16];
      size_t got;
      while ((got = fread(buf, 1, sizeof buf, f)) > 0) data.append(buf, got);
      fclose(f);
      // bufio.ScanLines; the "#version" header and blank lines carry no merge
      int rank = 0;
      for (size_t pos = 0; pos < data.size();) {
        size_t nl = data.find('\n', pos);
        const size_t e = nl == std::string::npos ? data.size() : nl;
        size_t len = e - pos;
        if (len > 0 && data[pos + len - 1] == '\r') len--;
        const std::string line = data.substr(pos, len);
        pos = nl == std::string::npos ? data.size() : nl + 1;
        if (line.empty() || line.rfind("#version", 0) == 0) continue;
        const size_t sp = line.find(' ');
        if (sp == std::string::npos || sp == 0 || sp + 1 == line.size())
          return fail(RH_ERR_INVALID, "bpe: malformed merge line \"" + line + "\"");
        t->ranks[Bpe::pair_key(line.substr(0, sp), line.substr(sp + 1))] = rank++;
      }
      if (rank == 0) return fail(RH_ERR_INVALID, "bpe: no merges");
      t->cls = t->lookup(cls_tok, "cls");
      t->sep = t->lookup(sep_tok, "sep");
      t->unk = t->lookup(unk_tok, "unk");
      *out = t.release();
      return RH_OK;
    } catch (const std::invalid_argument& e) {
      return fail(RH_ERR_INVALID, e.what());
    }
  });
}

// NewFromTokenizerJSON (bpe.go:282-303): ModernBERT's tokenizer.json, cls
// ... sep framing, GPT-2 pre-tokenizer. NewQwenFromTokenizerJSON
// (bpe.go:305-324) when qwen is set: the Qwen pre-tokenizer and a trailing
// eos (sep_tok) alone; cls_tok and unk_tok are then unused.
int rh_tokenizer_bpe_load_json(const char* tokenizer_json, int qwen, const char* cls_tok,
                               const char* sep_tok, const char* unk_tok, rh_tokenizer** out) {
  return api_call([&]() -> int {
    if (!tokenizer_json || !sep_tok || !out || (!qwen && (!cls_tok || !unk_tok)))
      return fail(RH_ERR_INVALID, "null argument");
    *out = nullptr;
    try {
      std::unique_ptr<Bpe> t = parse_tokenizer_json(tokenizer_json);
      if (qwen) {
        t->qwen = true;
        t->no_prefix = true;
        t->sep = t->lookup(sep_tok, "eos");
        t->unk = t->sep;
      } else {
        t->cls = t->lookup(cls_tok, "cls");
        t->sep = t->lookup(sep_tok, "sep");
        t->unk = t->lookup(unk_tok, "unk");
      }
      *out = t.release();
      return RH_OK;
    } catch (const std::invalid_argument& e) {
      return fail(RH_ERR_INVALID, e.what());
    }
  });
}

// gemma.New (tokenizer/gemma/gemma.go:58-111): model.vocab, model.merges as
// [[a, b]] pairs, byte_fallback required with every "<0xNN>" piece present,
// and <bos> / <eos> / <unk> from added_tokens.
int rh_tokenizer_gemma_load(const char* tokenizer_json, rh_tokenizer** out) {
  return api_call([&]() -> int {
    if (!tokenizer_json || !out) return fail(RH_ERR_INVALID, "null argument");
    *out = nullptr;
    try {
      const Json j = parse_json_file(tokenizer_json);
      const Json* model = j.get("model");
      const Json* vocab = model ? model->get("vocab") : nullptr;
      if (!vocab || vocab->kind != Json::Object || vocab->obj.empty())
        return fail(RH_ERR_INVALID, "gemma: empty vocab");
      const Json* bf = model->get("byte_fallback");
      if (!bf || bf->kind != Json::Bool || !bf->b)
        return fail(RH_ERR_INVALID, "gemma: byte_fallback is false (required)");
      std::unique_ptr<GemmaBpe> t(new GemmaBpe());
      for (const auto& kv : vocab->obj) t->vocab[kv.first] = json_int(kv.second, "a vocab id");
      const Json* merges = model->get("merges");
      if (merges && merges->kind == Json::Array) {
        int rank = 0;
        for (const Json& m : merges->arr) {
          if (m.kind != Json::Array || m.arr.size() != 2 || m.arr[0].kind != Json::String ||
              m.arr[1].kind != Json::String)
            return fail(RH_ERR_INVALID, "gemma: a merge is not a pair");
          t->ranks.emplace(Bpe::pair_key(m.arr[0].str, m.arr[1].str), rank++);
        }
      } else if (merges && merges->kind != Json::Null) {
        return fail(RH_ERR_INVALID, "gemma: merges is not a list of pairs");
      }
      for (int b = 0; b < 256; b++) {
        char piece[8];
        snprintf(piece, sizeof piece, "<0x%02X>", b);
        if (!t->vocab.count(piece))
          return fail(RH_ERR_INVALID, std::string("gemma: byte fallback piece ") + piece +
                                          " missing from the vocab");
      }
      if (const Json* at = j.get("added_tokens"))
        for (const Json& a : at->arr) {
          const Json* c = a.get("content");
          const Json* id = a.get("id");
          if (!c || c->kind != Json::String || !id) continue;
          if (c->str == "<bos>") t->bos = json_int(*id, "an added token id");
          else if (c->str == "<eos>") t->eos = json_int(*id, "an added token id");
          else if (c->str == "<unk>") t->unk = json_int(*id, "an added token id");
        }
      if (t->bos < 0 || t->eos < 0 || t->unk < 0)
        return fail(RH_ERR_INVALID, "gemma: missing <bos>/<eos>/<unk> in added_tokens");
      *out = t.release();
      return RH_OK;
    } catch (const std::invalid_argument& e) {
      return fail(RH_ERR_INVALID, e.what());
    }
  });
}

}  // extern "C"
