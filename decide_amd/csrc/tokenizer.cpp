// Host tokenizer: ModernBERT's byte-level BPE (a HuggingFace tokenizer.json
// with NFC normalisation, the GPT-2 pre-tokenizer, added tokens and
// [CLS] $A [SEP]), as internal/tokenizer/tokenizer.go implements it:
//   Parse          tokenizer.go:60-130   vocab, merge ranks, added tokens
//   Encode         tokenizer.go:133-160  special split -> NFC -> normal split
//                                        -> preTokenize -> byteLevel -> bpe
//   splitOnTokens  tokenizer.go:168-212  leftmost-longest, lstrip / rstrip
//   preTokenize    tokenizer.go:214-272  the GPT-2 split regex, by hand
//   byteLevel      tokenizer.go:286-318  GPT-2 byte -> printable rune map
//   bpe            tokenizer.go:320-365  lowest-rank merge first, then ids
// NFC (golang.org/x/text/unicode/norm in the reference) is the Unicode
// canonical decomposition, canonical ordering and composition algorithm of
// UAX #15 over tables generated from the Unicode Character Database
// (unicode_tables.inc, gen_unicode_tables.py).
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/decide_hip.h"
#include "common.hpp"

namespace {

#include "unicode_tables.inc"

// ---------------------------------------------------------------- UTF-8
// Decodes one rune at s[i]; invalid or truncated sequences give U+FFFD and
// consume one byte (Go's utf8.DecodeRuneInString).
uint32_t decode_rune(const std::string &s, size_t i, size_t *len) {
  const unsigned char c = (unsigned char)s[i];
  const size_t n = s.size();
  if (c < 0x80) {
    *len = 1;
    return c;
  }
  auto cont = [&](size_t k) { return k < n && ((unsigned char)s[k] & 0xC0) == 0x80; };
  if (c >= 0xC2 && c <= 0xDF && cont(i + 1)) {
    *len = 2;
    return ((c & 0x1Fu) << 6) | ((unsigned char)s[i + 1] & 0x3Fu);
  }
  if (c >= 0xE0 && c <= 0xEF && cont(i + 1) && cont(i + 2)) {
    const uint32_t r = ((c & 0x0Fu) << 12) | (((unsigned char)s[i + 1] & 0x3Fu) << 6) | ((unsigned char)s[i + 2] & 0x3Fu);
    if (r >= 0x800 && !(r >= 0xD800 && r <= 0xDFFF)) {
      *len = 3;
      return r;
    }
  }
  if (c >= 0xF0 && c <= 0xF4 && cont(i + 1) && cont(i + 2) && cont(i + 3)) {
    const uint32_t r = ((c & 0x07u) << 18) | (((unsigned char)s[i + 1] & 0x3Fu) << 12) |
                       (((unsigned char)s[i + 2] & 0x3Fu) << 6) | ((unsigned char)s[i + 3] & 0x3Fu);
    if (r >= 0x10000 && r <= 0x10FFFF) {
      *len = 4;
      return r;
    }
  }
  *len = 1;
  return 0xFFFD;
}

void append_utf8(std::string &out, uint32_t r) {
  if (r < 0x80) {
    out += (char)r;
  } else if (r < 0x800) {
    out += (char)(0xC0 | (r >> 6));
    out += (char)(0x80 | (r & 0x3F));
  } else if (r < 0x10000) {
    out += (char)(0xE0 | (r >> 12));
    out += (char)(0x80 | ((r >> 6) & 0x3F));
    out += (char)(0x80 | (r & 0x3F));
  } else {
    out += (char)(0xF0 | (r >> 18));
    out += (char)(0x80 | ((r >> 12) & 0x3F));
    out += (char)(0x80 | ((r >> 6) & 0x3F));
    out += (char)(0x80 | (r & 0x3F));
  }
}

// []rune(s): one rune per valid sequence, U+FFFD per invalid byte.
std::vector<uint32_t> to_runes(const std::string &s) {
  std::vector<uint32_t> out;
  out.reserve(s.size());
  for (size_t i = 0; i < s.size();) {
    size_t l;
    out.push_back(decode_rune(s, i, &l));
    i += l;
  }
  return out;
}

// ---------------------------------------------------------------- classes
template <size_t N>
bool in_ranges(const uint32_t (&t)[N][2], uint32_t r) {
  size_t lo = 0, hi = N;
  while (lo < hi) {
    const size_t m = (lo + hi) / 2;
    if (r < t[m][0])
      hi = m;
    else if (r > t[m][1])
      lo = m + 1;
    else
      return true;
  }
  return false;
}

bool is_letter(uint32_t r) {  // unicode.IsLetter
  if (r < 0x80) return (r | 0x20) >= 'a' && (r | 0x20) <= 'z';
  return in_ranges(kLetter, r);
}
bool is_number(uint32_t r) {  // unicode.IsNumber
  if (r < 0x80) return r >= '0' && r <= '9';
  return in_ranges(kNumber, r);
}
bool is_space(uint32_t r) {  // unicode.IsSpace: the White_Space property
  switch (r) {
    case '\t': case '\n': case '\v': case '\f': case '\r': case ' ': case 0x85: case 0xA0: case 0x1680:
    case 0x2028: case 0x2029: case 0x202F: case 0x205F: case 0x3000:
      return true;
  }
  return r >= 0x2000 && r <= 0x200A;
}

// ---------------------------------------------------------------- NFC
constexpr uint32_t SBase = 0xAC00, LBase = 0x1100, VBase = 0x1161, TBase = 0x11A7;
constexpr uint32_t LCount = 19, VCount = 21, TCount = 28, NCount = VCount * TCount, SCount = LCount * NCount;

int ccc(uint32_t r) {
  if (r < 0x300) return 0;
  size_t lo = 0, hi = sizeof(kCcc) / sizeof(kCcc[0]);
  while (lo < hi) {
    const size_t m = (lo + hi) / 2;
    if (r < kCcc[m].lo)
      hi = m;
    else if (r > kCcc[m].hi)
      lo = m + 1;
    else
      return kCcc[m].ccc;
  }
  return 0;
}

const Decomp *find_decomp(uint32_t r) {
  size_t lo = 0, hi = sizeof(kDecomp) / sizeof(kDecomp[0]);
  while (lo < hi) {
    const size_t m = (lo + hi) / 2;
    if (r < kDecomp[m].cp)
      hi = m;
    else if (r > kDecomp[m].cp)
      lo = m + 1;
    else
      return &kDecomp[m];
  }
  return nullptr;
}

void decompose(uint32_t r, std::vector<uint32_t> &out) {
  if (r >= SBase && r < SBase + SCount) {  // Hangul syllable
    const uint32_t s = r - SBase;
    out.push_back(LBase + s / NCount);
    out.push_back(VBase + (s % NCount) / TCount);
    if (s % TCount) out.push_back(TBase + s % TCount);
    return;
  }
  const Decomp *d = find_decomp(r);
  if (!d) {
    out.push_back(r);
    return;
  }
  decompose(d->a, out);
  if (d->b) decompose(d->b, out);
}

uint32_t compose(uint32_t a, uint32_t b) {  // 0: none
  if (a >= LBase && a < LBase + LCount && b >= VBase && b < VBase + VCount)
    return SBase + ((a - LBase) * VCount + (b - VBase)) * TCount;
  if (a >= SBase && a < SBase + SCount && (a - SBase) % TCount == 0 && b > TBase && b < TBase + TCount)
    return a + (b - TBase);
  size_t lo = 0, hi = sizeof(kComp) / sizeof(kComp[0]);
  while (lo < hi) {
    const size_t m = (lo + hi) / 2;
    if (a < kComp[m].a || (a == kComp[m].a && b < kComp[m].b))
      hi = m;
    else if (a > kComp[m].a || b > kComp[m].b)
      lo = m + 1;
    else
      return kComp[m].c;
  }
  return 0;
}

// Leading / trailing non-starters of r's NFKD decomposition ({0, 0} for the
// code points that have none).
NonStarters non_starters(uint32_t r) {
  size_t lo = 0, hi = sizeof(kNonStarters) / sizeof(kNonStarters[0]);
  while (lo < hi) {
    const size_t m = (lo + hi) / 2;
    if (r < kNonStarters[m].cp)
      hi = m;
    else if (r > kNonStarters[m].cp)
      lo = m + 1;
    else
      return kNonStarters[m];
  }
  return NonStarters{r, 0, 0};
}

constexpr uint32_t kCgj = 0x034F;  // COMBINING GRAPHEME JOINER, a starter of class 0
constexpr int kMaxNonStarters = 30;

// NFC of UTF-8 text. Invalid bytes pass through unchanged (as x/text/norm
// leaves them) and split the text into independently normalised runs.
// Before normalising, runs of more than 30 non-starters are broken with CGJ
// (UAX #15's Stream-Safe Text Process, which x/text's NFC applies): a code
// point whose decomposition's leading non-starters would take the count of
// consecutive non-starters past 30 gets a CGJ in front of it. A code point
// whose decomposition holds no starter adds its length to the count, any
// other sets the count to its trailing non-starters; an invalid byte is a
// starter. Text below U+0300 holds no non-starter, so the fast path needs
// no count.
std::string nfc(const std::string &s) {
  bool fast = true;
  for (size_t i = 0; i < s.size() && fast;) {
    size_t l;
    const uint32_t r = decode_rune(s, i, &l);
    if (r >= kNfcStableBelow) fast = false;
    i += l;
  }
  if (fast) return s;
  std::string out;
  out.reserve(s.size());
  std::vector<uint32_t> buf;
  auto flush = [&]() {
    if (buf.empty()) return;
    // canonical ordering: stable sort of each run of non-starters by class
    for (size_t i = 1; i < buf.size(); i++) {
      const int c = ccc(buf[i]);
      if (c == 0) continue;
      size_t j = i;
      while (j > 0 && ccc(buf[j - 1]) > c) {
        std::swap(buf[j - 1], buf[j]);
        j--;
      }
    }
    // canonical composition (UAX #15)
    size_t starter = 0, w = 1;
    uint32_t starter_ch = buf[0];
    int last = ccc(starter_ch) ? 256 : 0;
    for (size_t i = 1; i < buf.size(); i++) {
      const uint32_t ch = buf[i];
      const int c = ccc(ch);
      const uint32_t comp = compose(starter_ch, ch);
      if (comp && (last < c || last == 0)) {
        buf[starter] = starter_ch = comp;
      } else {
        if (c == 0) {
          starter = w;
          starter_ch = ch;
        }
        last = c;
        buf[w++] = ch;
      }
    }
    buf.resize(w);
    for (uint32_t r : buf) append_utf8(out, r);
    buf.clear();
  };
  int run = 0;  // consecutive non-starters so far
  for (size_t i = 0; i < s.size();) {
    size_t l;
    const uint32_t r = decode_rune(s, i, &l);
    if (l == 1 && (unsigned char)s[i] >= 0x80) {  // an invalid byte
      flush();
      out += s[i];
      run = 0;
    } else {
      const NonStarters ns = non_starters(r);
      if (run + ns.lead > kMaxNonStarters) {
        buf.push_back(kCgj);
        run = 0;
      }
      decompose(r, buf);
      run = ns.lead ? run + ns.lead : ns.trail;
    }
    i += l;
  }
  flush();
  return out;
}

// ---------------------------------------------------------------- pre-tokenizer
int contraction(const std::vector<uint32_t> &rs, size_t i) {  // rs[i..] after the apostrophe
  const size_t n = rs.size();
  if (i + 1 < n && ((rs[i] == 'l' && rs[i + 1] == 'l') || (rs[i] == 'v' && rs[i + 1] == 'e') ||
                    (rs[i] == 'r' && rs[i + 1] == 'e')))
    return 2;
  if (i < n && (rs[i] == 's' || rs[i] == 't' || rs[i] == 'm' || rs[i] == 'd')) return 1;
  return 0;
}

// 's|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+
// as piece boundaries over the runes of s.
std::vector<std::string> pre_tokenize(const std::string &s) {
  const std::vector<uint32_t> rs = to_runes(s);
  const size_t n = rs.size();
  std::vector<std::string> out;
  auto emit = [&](size_t a, size_t b) {
    std::string p;
    for (size_t k = a; k < b; k++) append_utf8(p, rs[k]);
    out.push_back(std::move(p));
  };
  size_t i = 0;
  while (i < n) {
    const size_t start = i;
    const uint32_t r = rs[i];
    if (r == '\'' && i + 1 < n) {
      const int l = contraction(rs, i + 1);
      if (l > 0) {
        i += 1 + l;
        emit(start, i);
        continue;
      }
    }
    size_t j = i;
    if (r == ' ' && i + 1 < n) j = i + 1;
    if (j < n) {
      const uint32_t c = rs[j];
      int kind = 0;  // 1 letter, 2 number, 3 other
      if (is_letter(c))
        kind = 1;
      else if (is_number(c))
        kind = 2;
      else if (!is_space(c))
        kind = 3;
      if (kind) {
        size_t k = j;
        while (k < n) {
          const uint32_t x = rs[k];
          const bool ok = kind == 1 ? is_letter(x) : kind == 2 ? is_number(x) : (!is_space(x) && !is_letter(x) && !is_number(x));
          if (!ok) break;
          k++;
        }
        emit(start, k);
        i = k;
        continue;
      }
    }
    size_t k = i;
    while (k < n && is_space(rs[k])) k++;
    if (k < n && k - i > 1) k--;  // \s+(?!\S) leaves the last space to the next word
    emit(start, k);
    i = k;
  }
  return out;
}

// ---------------------------------------------------------------- byte level
struct ByteMap {
  uint32_t r[256];
  ByteMap() {
    bool have[256] = {};
    auto set = [&](int a, int b) {
      for (int x = a; x <= b; x++) {
        r[x] = (uint32_t)x;
        have[x] = true;
      }
    };
    set('!', '~');
    set(0xA1, 0xAC);
    set(0xAE, 0xFF);
    uint32_t k = 0;
    for (int x = 0; x < 256; x++)
      if (!have[x]) r[x] = 256 + k++;
  }
};
const ByteMap kBytes;

std::string pair_key(const std::string &a, const std::string &b) {
  std::string k;
  const uint32_t la = (uint32_t)a.size();
  k.append((const char *)&la, 4);
  k += a;
  k += b;
  return k;
}

// ---------------------------------------------------------------- JSON
struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal *get(const char *key) const {
    for (auto &kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char *p, *e;
  std::string err;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool fail(const char *m) {
    if (err.empty()) err = m;
    return false;
  }
  bool hex4(uint32_t *v) {
    if (e - p < 4) return fail("bad \\u escape");
    uint32_t x = 0;
    for (int i = 0; i < 4; i++) {
      const char c = p[i];
      x <<= 4;
      if (c >= '0' && c <= '9') x |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') x |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') x |= (uint32_t)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    p += 4;
    *v = x;
    return true;
  }
  bool string(std::string &out) {
    if (p >= e || *p != '"') return fail("expected string");
    p++;
    const char *run = p;
    auto flush_run = [&](const char *end) {
      // raw bytes: invalid UTF-8 becomes U+FFFD (as encoding/json does)
      std::string raw(run, end);
      for (size_t i = 0; i < raw.size();) {
        size_t l;
        const uint32_t r = decode_rune(raw, i, &l);
        (void)r;
        if (l == 1 && (unsigned char)raw[i] >= 0x80)
          append_utf8(out, 0xFFFD);
        else
          out.append(raw, i, l);
        i += l;
      }
    };
    while (true) {
      if (p >= e) return fail("unterminated string");
      const char c = *p;
      if (c == '"') {
        flush_run(p);
        p++;
        return true;
      }
      if ((unsigned char)c < 0x20) return fail("control character in string");
      if (c != '\\') {
        p++;
        continue;
      }
      flush_run(p);
      p++;
      if (p >= e) return fail("bad escape");
      const char x = *p++;
      switch (x) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t v;
          if (!hex4(&v)) return false;
          if (v >= 0xD800 && v < 0xDC00) {
            uint32_t w = 0;
            if (e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
              const char *save = p;
              p += 2;
              if (!hex4(&w)) return false;
              if (w >= 0xDC00 && w < 0xE000) {
                v = 0x10000 + ((v - 0xD800) << 10) + (w - 0xDC00);
              } else {
                p = save;
                v = 0xFFFD;
              }
            } else {
              v = 0xFFFD;
            }
          } else if (v >= 0xDC00 && v < 0xE000) {
            v = 0xFFFD;
          }
          append_utf8(out, v);
          break;
        }
        default:
          return fail("bad escape");
      }
      run = p;
    }
  }
  bool value(JVal &v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("unexpected end");
    const char c = *p;
    if (c == '{') {
      v.kind = JVal::Obj;
      p++;
      ws();
      if (p < e && *p == '}') {
        p++;
        return true;
      }
      while (true) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p >= e || *p != ':') return fail("expected ':'");
        p++;
        v.obj.emplace_back(std::move(k), JVal());
        if (!value(v.obj.back().second, depth + 1)) return false;
        ws();
        if (p < e && *p == ',') {
          p++;
          continue;
        }
        if (p < e && *p == '}') {
          p++;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = JVal::Arr;
      p++;
      ws();
      if (p < e && *p == ']') {
        p++;
        return true;
      }
      while (true) {
        v.arr.emplace_back();
        if (!value(v.arr.back(), depth + 1)) return false;
        ws();
        if (p < e && *p == ',') {
          p++;
          continue;
        }
        if (p < e && *p == ']') {
          p++;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = JVal::Str;
      return string(v.str);
    }
    if (e - p >= 4 && !std::strncmp(p, "true", 4)) {
      v.kind = JVal::Bool;
      v.b = true;
      p += 4;
      return true;
    }
    if (e - p >= 5 && !std::strncmp(p, "false", 5)) {
      v.kind = JVal::Bool;
      p += 5;
      return true;
    }
    if (e - p >= 4 && !std::strncmp(p, "null", 4)) {
      p += 4;
      return true;
    }
    if (c == '-' || (c >= '0' && c <= '9')) {
      const char *s0 = p;
      while (p < e && (*p == '-' || *p == '+' || *p == '.' || *p == 'e' || *p == 'E' || (*p >= '0' && *p <= '9'))) p++;
      v.kind = JVal::Num;
      v.num = std::strtod(std::string(s0, p).c_str(), nullptr);
      return true;
    }
    return fail("unexpected character");
  }
};

}  // namespace

struct AddedTok {
  int32_t id;
  std::string content;
  bool special, normalized, lstrip, rstrip;
};

struct dn_tokenizer {
  std::unordered_map<std::string, int32_t> vocab;
  std::unordered_map<std::string, int> ranks;  // pair_key(a, b) -> merge index
  // Id form of the merges, used when every merge's parts and result are in
  // the vocabulary (true of trained BPE files): (id a << 32 | id b) ->
  // (rank, id of a+b), and the id of each byte's symbol (-1 if absent).
  bool id_mode = false;
  std::unordered_map<uint64_t, std::pair<int, int32_t>> id_merges;
  int32_t byte_id[256];
  std::vector<AddedTok> special, normal;
  int32_t cls = 0, sep = 0, mask = 0, pad = 0;
  std::mutex mu;
  std::unordered_map<std::string, std::vector<int32_t>> cache;

  struct Seg {
    std::string text;
    const AddedTok *tok;
  };

  static std::vector<Seg> split(const std::string &s, const std::vector<AddedTok> &toks) {
    std::vector<Seg> out;
    if (s.empty()) return out;
    if (toks.empty()) {
      out.push_back({s, nullptr});
      return out;
    }
    size_t pos = 0;
    while (pos < s.size()) {
      int best = -1;
      size_t best_idx = std::string::npos;
      for (size_t i = 0; i < toks.size(); i++) {
        if (toks[i].content.empty()) continue;  // would never advance
        const size_t idx = s.find(toks[i].content, pos);
        if (idx == std::string::npos) continue;
        if (best < 0 || idx < best_idx || (idx == best_idx && toks[i].content.size() > toks[best].content.size())) {
          best = (int)i;
          best_idx = idx;
        }
      }
      if (best < 0) {
        out.push_back({s.substr(pos), nullptr});
        break;
      }
      const AddedTok &tk = toks[best];
      std::string before = s.substr(pos, best_idx - pos);
      if (tk.lstrip) before = trim_right_space(before);
      if (!before.empty()) out.push_back({before, nullptr});
      out.push_back({std::string(), &tk});
      pos = best_idx + tk.content.size();
      if (tk.rstrip) pos = skip_left_space(s, pos);
    }
    return out;
  }

  static std::string trim_right_space(const std::string &s) {
    // strings.TrimRightFunc(s, unicode.IsSpace): drop trailing space runes.
    const std::vector<uint32_t> rs = to_runes(s);
    size_t keep_bytes = s.size();
    // walk runes backwards by re-decoding from the start (runes are short)
    std::vector<size_t> starts;
    for (size_t i = 0; i < s.size();) {
      size_t l;
      decode_rune(s, i, &l);
      starts.push_back(i);
      i += l;
    }
    for (size_t k = rs.size(); k > 0; k--) {
      if (!is_space(rs[k - 1])) break;
      keep_bytes = starts[k - 1];
    }
    return s.substr(0, keep_bytes);
  }

  static size_t skip_left_space(const std::string &s, size_t pos) {
    while (pos < s.size()) {
      size_t l;
      const uint32_t r = decode_rune(s, pos, &l);
      if (!is_space(r)) break;
      pos += l;
    }
    return pos;
  }

  void bpe(const std::string &word, std::vector<int32_t> &ids) {
    {
      std::lock_guard<std::mutex> g(mu);
      auto it = cache.find(word);
      if (it != cache.end()) {
        ids.insert(ids.end(), it->second.begin(), it->second.end());
        return;
      }
    }
    if (id_mode) {
      bpe_ids(word, ids);
      return;
    }
    std::vector<std::string> parts;
    parts.reserve(word.size());
    for (unsigned char b : word) {
      std::string sym;
      append_utf8(sym, kBytes.r[b]);
      parts.push_back(std::move(sym));
    }
    while (parts.size() > 1) {
      int best_rank = 0x7fffffff, best_at = -1;
      for (size_t i = 0; i + 1 < parts.size(); i++) {
        auto it = ranks.find(pair_key(parts[i], parts[i + 1]));
        if (it != ranks.end() && it->second < best_rank) {
          best_rank = it->second;
          best_at = (int)i;
        }
      }
      if (best_at < 0) break;
      parts[best_at] += parts[best_at + 1];
      parts.erase(parts.begin() + best_at + 1);
    }
    std::vector<int32_t> out;
    for (const std::string &p : parts) {
      auto it = vocab.find(p);
      if (it != vocab.end()) {
        out.push_back(it->second);
        continue;
      }
      // No byte fallback / unknown token: emit the constituent symbols that exist.
      for (size_t i = 0; i < p.size();) {
        size_t l;
        decode_rune(p, i, &l);
        auto jt = vocab.find(p.substr(i, l));
        if (jt != vocab.end()) out.push_back(jt->second);
        i += l;
      }
    }
    ids.insert(ids.end(), out.begin(), out.end());
    std::lock_guard<std::mutex> g(mu);
    if (cache.size() > 50000) cache.clear();
    cache.emplace(word, std::move(out));
  }

  // bpe over vocabulary ids: the same merges in the same order (lowest rank
  // first, leftmost occurrence), no string building.
  void bpe_ids(const std::string &word, std::vector<int32_t> &ids) {
    {
      std::lock_guard<std::mutex> g(mu);
      auto it = cache.find(word);
      if (it != cache.end()) {
        ids.insert(ids.end(), it->second.begin(), it->second.end());
        return;
      }
    }
    std::vector<int32_t> sym;
    sym.reserve(word.size());
    for (unsigned char b : word) sym.push_back(byte_id[b]);
    while (sym.size() > 1) {
      int best_rank = 0x7fffffff, best_at = -1;
      int32_t best_id = -1;
      for (size_t i = 0; i + 1 < sym.size(); i++) {
        if (sym[i] < 0 || sym[i + 1] < 0) continue;
        auto it = id_merges.find(((uint64_t)(uint32_t)sym[i] << 32) | (uint32_t)sym[i + 1]);
        if (it != id_merges.end() && it->second.first < best_rank) {
          best_rank = it->second.first;
          best_at = (int)i;
          best_id = it->second.second;
        }
      }
      if (best_at < 0) break;
      sym[best_at] = best_id;
      sym.erase(sym.begin() + best_at + 1);
    }
    std::vector<int32_t> out;
    out.reserve(sym.size());
    for (int32_t v : sym)
      if (v >= 0) out.push_back(v);  // a symbol outside the vocabulary is dropped
    ids.insert(ids.end(), out.begin(), out.end());
    std::lock_guard<std::mutex> g(mu);
    if (cache.size() > 50000) cache.clear();
    cache.emplace(word, std::move(out));
  }

  // Decides id_mode and builds its tables.
  void build_id_merges(const std::vector<std::pair<std::string, std::string>> &merges) {
    id_mode = false;
    id_merges.clear();
    for (size_t i = 0; i < merges.size(); i++) {
      auto a = vocab.find(merges[i].first), b = vocab.find(merges[i].second),
           c = vocab.find(merges[i].first + merges[i].second);
      if (a == vocab.end() || b == vocab.end() || c == vocab.end()) {
        id_merges.clear();
        return;
      }
      id_merges.emplace(((uint64_t)(uint32_t)a->second << 32) | (uint32_t)b->second, std::make_pair((int)i, c->second));
    }
    for (int x = 0; x < 256; x++) {
      std::string sym;
      append_utf8(sym, kBytes.r[x]);
      auto it = vocab.find(sym);
      byte_id[x] = it == vocab.end() ? -1 : it->second;
    }
    id_mode = true;
  }

  std::vector<int32_t> encode(const std::string &text, bool add_special) {
    std::vector<int32_t> ids;
    if (add_special) ids.push_back(cls);
    for (const Seg &seg : split(text, special)) {
      if (seg.tok) {
        ids.push_back(seg.tok->id);
        continue;
      }
      const std::string s = nfc(seg.text);
      for (const Seg &seg2 : split(s, normal)) {
        if (seg2.tok) {
          ids.push_back(seg2.tok->id);
          continue;
        }
        for (const std::string &w : pre_tokenize(seg2.text)) bpe(w, ids);
      }
    }
    if (add_special) ids.push_back(sep);
    return ids;
  }
};

namespace {
bool jbool(const JVal *v) { return v && v->kind == JVal::Bool && v->b; }
}  // namespace

extern "C" {

int dn_tokenizer_parse(const char *json, int64_t len, dn_tokenizer **out) {
  if (!out || (!json && len > 0) || len < 0) return set_host_error(DN_INVALID_ARG, "tokenizer: bad argument");
  *out = nullptr;
  JParser jp{json, json + len, {}};
  JVal root;
  if (!jp.value(root, 0)) return set_host_error(DN_INVALID_ARG, "tokenizer: " + jp.err);
  const JVal *model = root.get("model");
  const JVal *type = model ? model->get("type") : nullptr;
  const std::string mtype = type && type->kind == JVal::Str ? type->str : "";
  if (mtype != "BPE") return set_host_error(DN_INVALID_ARG, "tokenizer: unsupported model type \"" + mtype + "\"");
  auto *t = new dn_tokenizer();
  if (const JVal *vocab = model->get("vocab")) {
    t->vocab.reserve(vocab->obj.size());
    for (auto &kv : vocab->obj) t->vocab[kv.first] = (int32_t)kv.second.num;
  }
  std::vector<std::pair<std::string, std::string>> merge_list;
  if (const JVal *merges = model->get("merges")) {
    t->ranks.reserve(merges->arr.size());
    for (size_t i = 0; i < merges->arr.size(); i++) {
      const JVal &m = merges->arr[i];
      std::string a, b;
      if (m.kind == JVal::Arr && m.arr.size() == 2 && m.arr[0].kind == JVal::Str && m.arr[1].kind == JVal::Str) {
        a = m.arr[0].str;
        b = m.arr[1].str;
      } else if (m.kind == JVal::Str) {
        const size_t sp = m.str.find(' ');
        if (sp == std::string::npos) {
          delete t;
          return set_host_error(DN_INVALID_ARG, "tokenizer: bad merge \"" + m.str + "\"");
        }
        a = m.str.substr(0, sp);
        b = m.str.substr(sp + 1);
      } else {
        delete t;
        return set_host_error(DN_INVALID_ARG, "tokenizer: bad merge " + std::to_string(i));
      }
      t->ranks.emplace(pair_key(a, b), (int)i);  // the first occurrence keeps its rank
      merge_list.emplace_back(std::move(a), std::move(b));
    }
  }
  t->build_id_merges(merge_list);
  if (const JVal *added = root.get("added_tokens")) {
    for (const JVal &a : added->arr) {
      AddedTok at;
      const JVal *id = a.get("id"), *content = a.get("content");
      at.id = id ? (int32_t)id->num : 0;
      at.content = content ? content->str : "";
      at.special = jbool(a.get("special"));
      at.normalized = jbool(a.get("normalized"));
      at.lstrip = jbool(a.get("lstrip"));
      at.rstrip = jbool(a.get("rstrip"));
      if (at.special && !at.normalized)
        t->special.push_back(at);
      else
        t->normal.push_back(at);
      if (at.content == "[CLS]") t->cls = at.id;
      if (at.content == "[SEP]") t->sep = at.id;
      if (at.content == "[MASK]") t->mask = at.id;
      if (at.content == "[PAD]") t->pad = at.id;
    }
  }
  if (t->mask == 0 || t->sep == 0 || t->cls == 0) {
    delete t;
    return set_host_error(DN_INVALID_ARG, "tokenizer: missing [CLS]/[SEP]/[MASK] added tokens");
  }
  *out = t;
  return DN_OK;
}

void dn_tokenizer_free(dn_tokenizer *t) { delete t; }

int dn_tokenizer_special_ids(const dn_tokenizer *t, int32_t *cls, int32_t *sep, int32_t *mask, int32_t *pad) {
  if (!t) return set_host_error(DN_INVALID_ARG, "tokenizer: NULL tokenizer");
  if (cls) *cls = t->cls;
  if (sep) *sep = t->sep;
  if (mask) *mask = t->mask;
  if (pad) *pad = t->pad;
  return DN_OK;
}

int dn_tokenize(dn_tokenizer *t, const char *text, int64_t len, int add_special, int32_t *ids, int64_t cap,
                int64_t *n) {
  if (!t || !n || len < 0 || (!text && len > 0) || cap < 0 || (!ids && cap > 0))
    return set_host_error(DN_INVALID_ARG, "tokenizer: bad argument");
  const std::vector<int32_t> out = t->encode(std::string(text ? text : "", (size_t)len), add_special != 0);
  *n = (int64_t)out.size();
  if ((int64_t)out.size() > cap)
    return set_host_error(DN_INVALID_ARG, "tokenizer: " + std::to_string(out.size()) + " ids do not fit in " +
                                              std::to_string(cap));
  std::copy(out.begin(), out.end(), ids);
  return DN_OK;
}

int dn_pretokenize(const char *text, int64_t len, int64_t *ends, int64_t cap, int64_t *n) {
  if (!n || len < 0 || (!text && len > 0) || cap < 0 || (!ends && cap > 0))
    return set_host_error(DN_INVALID_ARG, "tokenizer: bad argument");
  const std::vector<std::string> pieces = pre_tokenize(std::string(text ? text : "", (size_t)len));
  *n = (int64_t)pieces.size();
  if ((int64_t)pieces.size() > cap) return set_host_error(DN_INVALID_ARG, "tokenizer: output capacity too small");
  int64_t off = 0;
  for (size_t i = 0; i < pieces.size(); i++) {
    off += (int64_t)pieces[i].size();
    ends[i] = off;
  }
  return DN_OK;
}

int dn_nfc(const char *text, int64_t len, char *out, int64_t cap, int64_t *n) {
  if (!n || len < 0 || (!text && len > 0) || cap < 0 || (!out && cap > 0))
    return set_host_error(DN_INVALID_ARG, "tokenizer: bad argument");
  const std::string r = nfc(std::string(text ? text : "", (size_t)len));
  *n = (int64_t)r.size();
  if ((int64_t)r.size() > cap) return set_host_error(DN_INVALID_ARG, "tokenizer: output capacity too small");
  std::memcpy(out, r.data(), r.size());
  return DN_OK;
}

}  // extern "C"
