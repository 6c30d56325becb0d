// Byte-level BPE tokenizer and detokenizer of the Granite 3.1 models (host only), and the fixed rendering of their chat
// template. Replaces rust/moe-rt/src/tokenizador.rs: a tokenizer.json with no normaliser, the ByteLevel pre-tokenizer
// (GPT-2 pattern, no prefix space), a BPE model by merge rank (no dropout, no byte fallback, no unknown token) and the
// ByteLevel decoder; added tokens (all special, none stripped or normalised) are found in the raw text by the longest
// match at the leftmost position. Any other configuration is refused at load, instead of tokenising differently.
//
// Pre-tokenisation follows the pattern 's|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+
// (first alternative that matches wins, greedy runs, the optional space only U+0020), with \p{L}, \p{N} and \s from
// unicode_tables.h, which records exactly what the `tokenizers` library's pre-tokenizer treats as such.
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <fstream>
#include <iterator>
#include <queue>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/moert.h"
#include "json.h"
#include "unicode_tables.h"

namespace moert {
int set_error(int code, const char* fmt, ...);
}
using moert::JParser;
using moert::JVal;
using moert::set_error;

namespace {

bool in_ranges(const uint32_t (*r)[2], int n, uint32_t c) {
  int lo = 0, hi = n - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) / 2;
    if (c < r[mid][0]) hi = mid - 1;
    else if (c > r[mid][1]) lo = mid + 1;
    else return true;
  }
  return false;
}

enum Cls { SPACE = 0, LETTER = 1, NUMBER = 2, OTHER = 3 };

int cls(uint32_t c) {
  if (in_ranges(moert::kSpaceRanges, moert::kSpaceRangesCount, c)) return SPACE;
  if (in_ranges(moert::kLetterRanges, moert::kLetterRangesCount, c)) return LETTER;
  if (in_ranges(moert::kNumberRanges, moert::kNumberRangesCount, c)) return NUMBER;
  return OTHER;
}

// Code points of valid UTF-8 with the byte offset of each (offs has one more entry: the end); false on invalid UTF-8.
bool decode_utf8(const char* s, size_t n, std::vector<uint32_t>& cps, std::vector<size_t>& offs) {
  const unsigned char* p = (const unsigned char*)s;
  size_t i = 0;
  while (i < n) {
    const unsigned c = p[i];
    uint32_t cp;
    int len;
    if (c < 0x80) {
      cp = c;
      len = 1;
    } else if (c >= 0xC2 && c <= 0xDF) {
      cp = c & 0x1F;
      len = 2;
    } else if (c >= 0xE0 && c <= 0xEF) {
      cp = c & 0x0F;
      len = 3;
    } else if (c >= 0xF0 && c <= 0xF4) {
      cp = c & 0x07;
      len = 4;
    } else {
      return false;
    }
    if (i + len > n) return false;
    for (int k = 1; k < len; k++) {
      if ((p[i + k] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (p[i + k] & 0x3F);
    }
    if ((len == 3 && (cp < 0x800 || (cp >= 0xD800 && cp <= 0xDFFF))) || (len == 4 && (cp < 0x10000 || cp > 0x10FFFF)))
      return false;
    cps.push_back(cp);
    offs.push_back(i);
    i += len;
  }
  offs.push_back(n);
  return true;
}

void put_utf8(std::string& s, uint32_t cp) {
  if (cp < 0x80) {
    s += (char)cp;
  } else if (cp < 0x800) {
    s += (char)(0xC0 | (cp >> 6));
    s += (char)(0x80 | (cp & 0x3F));
  } else if (cp < 0x10000) {
    s += (char)(0xE0 | (cp >> 12));
    s += (char)(0x80 | ((cp >> 6) & 0x3F));
    s += (char)(0x80 | (cp & 0x3F));
  } else {
    s += (char)(0xF0 | (cp >> 18));
    s += (char)(0x80 | ((cp >> 12) & 0x3F));
    s += (char)(0x80 | ((cp >> 6) & 0x3F));
    s += (char)(0x80 | (cp & 0x3F));
  }
}

// Pieces of the GPT-2 pattern over cps[a, b): end indices (exclusive) of consecutive pieces covering the range.
void pretokenize(const std::vector<uint32_t>& cps, size_t a, size_t b, std::vector<size_t>& ends) {
  size_t i = a;
  while (i < b) {
    const uint32_t c = cps[i];
    // 's 't 'm 'd 're 've 'll
    if (c == '\'' && i + 1 < b) {
      const uint32_t c1 = cps[i + 1], c2 = i + 2 < b ? cps[i + 2] : 0;
      size_t len = 0;
      if (c1 == 's' || c1 == 't' || c1 == 'm' || c1 == 'd') len = 2;
      else if ((c1 == 'r' && c2 == 'e') || (c1 == 'v' && c2 == 'e') || (c1 == 'l' && c2 == 'l')) len = 3;
      if (len) {
        i += len;
        ends.push_back(i);
        continue;
      }
    }
    // an optional U+0020, then a run of letters, of numbers, or of other characters
    const size_t j = (c == ' ' && i + 1 < b) ? i + 1 : i;
    const int k = cls(cps[j]);
    if (k != SPACE) {
      size_t e = j + 1;
      while (e < b && cls(cps[e]) == k) e++;
      i = e;
      ends.push_back(i);
      continue;
    }
    // white space: \s+(?!\S) leaves the last of a run followed by a non-space to the next piece; else \s+
    size_t e = i;
    while (e < b && cls(cps[e]) == SPACE) e++;
    i = (e < b && e - i > 1) ? e - 1 : e;
    ends.push_back(i);
  }
}

// GPT-2's byte -> character map of the ByteLevel alphabet: printable bytes map to themselves, the others to U+0100
// onwards in byte order.
void byte_chars(uint32_t (&m)[256]) {
  uint32_t next = 256;
  for (uint32_t b = 0; b < 256; b++) {
    const bool printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
    m[b] = printable ? b : next++;
  }
}

bool json_false(const JVal* v) { return v && v->kind == JVal::BOOL && !v->b; }
bool json_true(const JVal* v) { return v && v->kind == JVal::BOOL && v->b; }
bool json_null(const JVal* v) { return !v || v->kind == JVal::NUL; }
bool json_str_is(const JVal* v, const char* s) { return v && v->kind == JVal::STR && v->s == s; }

}  // namespace

struct moert_tokenizer {
  std::vector<std::string> bytes;   // id -> the bytes it stands for (added tokens: their text)
  std::vector<char> has;            // id -> known (and detokenisable as bytes)
  int byte_id[256];                 // byte -> id of its one-character token, -1 (the byte is then dropped)
  std::unordered_map<uint64_t, std::pair<uint32_t, uint32_t>> merges;  // (left, right) -> (rank, merged id)
  std::vector<std::pair<std::string, uint32_t>> added;
  std::unordered_map<std::string, std::vector<uint32_t>> cache;

  static uint64_t key(uint32_t a, uint32_t b) { return ((uint64_t)a << 32) | b; }

  // BPE by merge rank over one piece's bytes: the lowest rank first, the leftmost pair among equal ranks
  void bpe(const std::string& piece, std::vector<uint32_t>& out) {
    auto hit = cache.find(piece);
    if (hit != cache.end()) {
      out.insert(out.end(), hit->second.begin(), hit->second.end());
      return;
    }
    std::vector<uint32_t> id;
    for (unsigned char b : piece)
      if (byte_id[b] >= 0) id.push_back((uint32_t)byte_id[b]);
    const size_t n = id.size();
    std::vector<size_t> nxt(n), prv(n);
    std::vector<char> live(n, 1);
    const size_t NONE = (size_t)-1;
    for (size_t i = 0; i < n; i++) {
      nxt[i] = i + 1 < n ? i + 1 : NONE;
      prv[i] = i > 0 ? i - 1 : NONE;
    }
    typedef std::pair<uint32_t, size_t> Item;  // (rank, position)
    std::priority_queue<Item, std::vector<Item>, std::greater<Item>> heap;
    auto push = [&](size_t p) {
      if (p == NONE || nxt[p] == NONE) return;
      const auto it = merges.find(key(id[p], id[nxt[p]]));
      if (it != merges.end()) heap.push({it->second.first, p});
    };
    for (size_t i = 0; i + 1 < n; i++) push(i);
    while (!heap.empty()) {
      const Item top = heap.top();
      heap.pop();
      const size_t p = top.second;
      if (!live[p] || nxt[p] == NONE) continue;
      const uint64_t k = key(id[p], id[nxt[p]]);
      const auto it = merges.find(k);
      if (it == merges.end() || it->second.first != top.first) continue;  // a stale entry (ranks name pairs uniquely)
      const size_t q = nxt[p];
      id[p] = it->second.second;
      live[q] = 0;
      nxt[p] = nxt[q];
      if (nxt[q] != NONE) prv[nxt[q]] = p;
      push(prv[p]);
      push(p);
    }
    std::vector<uint32_t> res;
    for (size_t i = 0; i != NONE && n; i = nxt[i]) res.push_back(id[i]);
    out.insert(out.end(), res.begin(), res.end());
    if (cache.size() < 50000) cache.emplace(piece, std::move(res));
  }

  void encode_plain(const char* text, const std::vector<uint32_t>& cps, const std::vector<size_t>& offs, size_t a,
                    size_t b, std::vector<uint32_t>& out) {
    std::vector<size_t> ends;
    pretokenize(cps, a, b, ends);
    size_t s = a;
    for (size_t e : ends) {
      bpe(std::string(text + offs[s], offs[e] - offs[s]), out);
      s = e;
    }
  }

  void encode(const char* text, size_t len, const std::vector<uint32_t>& cps, const std::vector<size_t>& offs,
              std::vector<uint32_t>& out) {
    size_t start = 0;  // code point index where the text not yet encoded begins
    for (size_t i = 0; i < cps.size();) {
      const std::pair<std::string, uint32_t>* best = nullptr;
      const size_t at = offs[i];
      for (const auto& a : added)
        if (a.first.size() <= len - at && std::memcmp(text + at, a.first.data(), a.first.size()) == 0 &&
            (!best || a.first.size() > best->first.size()))
          best = &a;
      if (!best) {
        i++;
        continue;
      }
      encode_plain(text, cps, offs, start, i, out);
      out.push_back(best->second);
      const size_t stop = at + best->first.size();
      while (i < cps.size() && offs[i] < stop) i++;
      start = i;
    }
    encode_plain(text, cps, offs, start, cps.size(), out);
  }
};

namespace {

int load_json(const char* json, size_t len, moert_tokenizer** out) {
  JVal j;
  std::string err;
  JParser parser(json, len);
  if (!parser.parse(j, err)) return set_error(MOERT_E_CONFIG, "tokenizer: invalid JSON: %s", err.c_str());
  if (j.kind != JVal::OBJ) return set_error(MOERT_E_CONFIG, "tokenizer: not a JSON object");
  auto unsupported = [](const char* what) {
    return set_error(MOERT_E_CONFIG, "tokenizer: tokenizer.json outside what is supported: %s", what);
  };
  if (!json_null(j.get("normalizer"))) return unsupported("a normalizer");
  const JVal* pre = j.get("pre_tokenizer");
  if (!pre || !json_str_is(pre->get("type"), "ByteLevel") || !json_false(pre->get("add_prefix_space")) ||
      !json_true(pre->get("use_regex")))
    return unsupported("pre_tokenizer other than ByteLevel{add_prefix_space: false, use_regex: true}");
  const JVal* dec = j.get("decoder");
  if (!dec || !json_str_is(dec->get("type"), "ByteLevel")) return unsupported("decoder other than ByteLevel");
  const JVal* m = j.get("model");
  if (!m || !json_str_is(m->get("type"), "BPE")) return unsupported("model other than BPE");
  if (!json_null(m->get("dropout"))) return unsupported("model.dropout");
  if (!json_null(m->get("unk_token"))) return unsupported("model.unk_token");
  for (const char* f : {"continuing_subword_prefix", "end_of_word_suffix"}) {
    const JVal* v = m->get(f);
    if (!(json_null(v) || (v->kind == JVal::STR && v->s.empty()))) return unsupported(f);
  }
  if (json_true(m->get("byte_fallback"))) return unsupported("model.byte_fallback");
  if (json_true(m->get("ignore_merges"))) return unsupported("model.ignore_merges");
  const JVal* vocab = m->get("vocab");
  if (!vocab || vocab->kind != JVal::OBJ) return unsupported("model.vocab missing");
  uint64_t max_id = 0;
  for (const auto& kv : vocab->obj) {
    if (kv.second.kind != JVal::NUM || !kv.second.is_uint || kv.second.u > UINT32_MAX)
      return set_error(MOERT_E_CONFIG, "tokenizer: invalid id for a vocabulary entry");
    max_id = std::max(max_id, kv.second.u);
  }
  std::vector<std::pair<std::string, uint32_t>> added;
  const JVal* at = j.get("added_tokens");
  if (at && at->kind == JVal::ARR) {
    for (const JVal& a : at->arr) {
      const JVal* c = a.get("content");
      const JVal* id = a.get("id");
      if (!c || c->kind != JVal::STR || !id || id->kind != JVal::NUM || !id->is_uint)
        return unsupported("an added token without content or id");
      if (!json_false(a.get("lstrip")) || !json_false(a.get("rstrip")) || !json_false(a.get("single_word")) ||
          !json_false(a.get("normalized")) || c->s.empty())
        return unsupported("an added token with lstrip / rstrip / single_word / normalized");
      if (id->u > UINT32_MAX) return unsupported("an added token id beyond u32");
      max_id = std::max(max_id, id->u);
      added.push_back({c->s, (uint32_t)id->u});
    }
  }
  // refuse sparse ids before allocating tables indexed by the largest one
  const uint64_t entries = vocab->obj.size() + added.size();
  if (max_id + 1 > entries * 2 + 1024)
    return set_error(MOERT_E_CONFIG, "tokenizer: sparse ids: largest %llu for %llu entries", (unsigned long long)max_id,
                     (unsigned long long)entries);
  uint32_t bmap[256];
  byte_chars(bmap);
  std::unordered_map<uint32_t, int> char_byte;
  for (int b = 0; b < 256; b++) char_byte[bmap[b]] = b;
  moert_tokenizer* t = new moert_tokenizer();
  const size_t size = (size_t)max_id + 1;
  t->bytes.assign(size, std::string());
  t->has.assign(size, 0);
  std::unordered_map<std::string, uint32_t> by_text;
  by_text.reserve(vocab->obj.size() * 2);
  for (const auto& kv : vocab->obj) {
    const uint32_t id = (uint32_t)kv.second.u;
    by_text[kv.first] = id;
    std::vector<uint32_t> cps;
    std::vector<size_t> offs;
    std::string bs;
    bool ok = decode_utf8(kv.first.data(), kv.first.size(), cps, offs);
    for (uint32_t c : cps) {
      const auto it = char_byte.find(c);
      if (it == char_byte.end()) {
        ok = false;
        break;
      }
      bs += (char)it->second;
    }
    if (ok) {
      t->bytes[id] = bs;
      t->has[id] = 1;
    }
  }
  for (const auto& a : added) {
    t->bytes[a.second] = a.first;
    t->has[a.second] = 1;
  }
  for (int b = 0; b < 256; b++) {
    std::string s;
    put_utf8(s, bmap[b]);
    const auto it = by_text.find(s);
    t->byte_id[b] = it == by_text.end() ? -1 : (int)it->second;
  }
  const JVal* merges = m->get("merges");
  if (!merges || merges->kind != JVal::ARR) {
    delete t;
    return unsupported("model.merges missing");
  }
  for (size_t rank = 0; rank < merges->arr.size(); rank++) {
    const JVal& mg = merges->arr[rank];
    std::string a, b;
    if (mg.kind == JVal::STR) {
      const size_t sp = mg.s.find(' ');
      if (sp == std::string::npos) {
        delete t;
        return set_error(MOERT_E_CONFIG, "tokenizer: merge %zu has no space", rank);
      }
      a = mg.s.substr(0, sp);
      b = mg.s.substr(sp + 1);
    } else if (mg.kind == JVal::ARR && mg.arr.size() == 2 && mg.arr[0].kind == JVal::STR &&
               mg.arr[1].kind == JVal::STR) {
      a = mg.arr[0].s;
      b = mg.arr[1].s;
    } else {
      delete t;
      return set_error(MOERT_E_CONFIG, "tokenizer: merge %zu is malformed", rank);
    }
    const auto ia = by_text.find(a), ib = by_text.find(b), ic = by_text.find(a + b);
    if (ia == by_text.end() || ib == by_text.end() || ic == by_text.end()) {
      delete t;
      return set_error(MOERT_E_CONFIG, "tokenizer: merge %zu uses or makes a token outside the vocabulary", rank);
    }
    // a repeated pair keeps its last rank, as the library does
    t->merges[moert_tokenizer::key(ia->second, ib->second)] = {(uint32_t)rank, ic->second};
  }
  t->added = std::move(added);
  *out = t;
  return MOERT_OK;
}

int put_out(const std::string& s, char* out, size_t max, size_t* needed) {
  if (needed) *needed = s.size();
  if (!out) return MOERT_OK;
  if (max < s.size()) return set_error(MOERT_E_RANGE, "output of %zu bytes does not fit in %zu", s.size(), max);
  std::memcpy(out, s.data(), s.size());
  return MOERT_OK;
}

// bytes -> UTF-8 text, each maximal invalid subpart replaced by U+FFFD (the Unicode recommended practice)
std::string lossy_utf8(const std::string& in) {
  const unsigned char* p = (const unsigned char*)in.data();
  const size_t n = in.size();
  std::string out;
  size_t i = 0;
  while (i < n) {
    const unsigned c = p[i];
    if (c < 0x80) {
      out += (char)c;
      i++;
      continue;
    }
    int len = 0;
    unsigned lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) len = 2;
    else if (c == 0xE0) len = 3, lo = 0xA0;
    else if (c >= 0xE1 && c <= 0xEC) len = 3;
    else if (c == 0xED) len = 3, hi = 0x9F;
    else if (c >= 0xEE && c <= 0xEF) len = 3;
    else if (c == 0xF0) len = 4, lo = 0x90;
    else if (c >= 0xF1 && c <= 0xF3) len = 4;
    else if (c == 0xF4) len = 4, hi = 0x8F;
    if (!len) {
      out += "\xEF\xBF\xBD";
      i++;
      continue;
    }
    size_t k = 1;
    while (k < (size_t)len && i + k < n) {
      const unsigned d = p[i + k];
      const unsigned l = k == 1 ? lo : 0x80, h = k == 1 ? hi : 0xBF;
      if (d < l || d > h) break;
      k++;
    }
    if (k == (size_t)len) out.append((const char*)p + i, k);
    else out += "\xEF\xBF\xBD";
    i += k;
  }
  return out;
}

}  // namespace

extern "C" {

int moert_tokenizer_from_json(const char* json, size_t len, moert_tokenizer** out) {
  if (!json || !out) return set_error(MOERT_E_CONFIG, "tokenizer: null argument");
  *out = nullptr;
  return load_json(json, len, out);
}

int moert_tokenizer_load(const char* path, moert_tokenizer** out) {
  if (!path || !out) return set_error(MOERT_E_CONFIG, "tokenizer: null argument");
  *out = nullptr;
  std::ifstream f(path, std::ios::binary);
  if (!f) return set_error(MOERT_E_CONFIG, "tokenizer: cannot read %s", path);
  const std::string raw((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  return load_json(raw.data(), raw.size(), out);
}

int moert_tokenizer_destroy(moert_tokenizer* t) {
  delete t;
  return MOERT_OK;
}

int moert_tokenizer_vocab_size(const moert_tokenizer* t, int* n) {
  if (!t || !n) return set_error(MOERT_E_CONFIG, "tokenizer: null argument");
  *n = (int)t->bytes.size();
  return MOERT_OK;
}

int moert_tokenizer_encode(moert_tokenizer* t, const char* text, size_t len, uint32_t* ids, size_t max_ids,
                           size_t* n_ids) {
  if (!t || (!text && len) || !n_ids) return set_error(MOERT_E_CONFIG, "tokenizer encode: null argument");
  std::vector<uint32_t> cps;
  std::vector<size_t> offs;
  if (!decode_utf8(text ? text : "", len, cps, offs))
    return set_error(MOERT_E_CONFIG, "tokenizer encode: the text is not valid UTF-8");
  std::vector<uint32_t> out;
  t->encode(text ? text : "", len, cps, offs, out);
  *n_ids = out.size();
  if (!ids) return MOERT_OK;
  if (max_ids < out.size()) return set_error(MOERT_E_RANGE, "tokenizer encode: %zu ids do not fit in %zu", out.size(), max_ids);
  std::copy(out.begin(), out.end(), ids);
  return MOERT_OK;
}

int moert_tokenizer_decode(const moert_tokenizer* t, const uint32_t* ids, size_t n, int lossy_text, char* out,
                           size_t max, size_t* n_bytes) {
  if (!t || (!ids && n)) return set_error(MOERT_E_CONFIG, "tokenizer decode: null argument");
  std::string s;
  for (size_t i = 0; i < n; i++) {
    if (ids[i] >= t->bytes.size() || !t->has[ids[i]])
      return set_error(MOERT_E_RANGE, "tokenizer decode: id %u outside the vocabulary", ids[i]);
    s += t->bytes[ids[i]];
  }
  return put_out(lossy_text ? lossy_utf8(s) : s, out, max, n_bytes);
}

int moert_tokenizer_pretokenize(const char* text, size_t len, size_t* ends, size_t max, size_t* n) {
  if ((!text && len) || !n) return set_error(MOERT_E_CONFIG, "pretokenize: null argument");
  std::vector<uint32_t> cps;
  std::vector<size_t> offs;
  if (!decode_utf8(text ? text : "", len, cps, offs)) return set_error(MOERT_E_CONFIG, "pretokenize: invalid UTF-8");
  std::vector<size_t> e;
  pretokenize(cps, 0, cps.size(), e);
  *n = e.size();
  if (!ends) return MOERT_OK;
  if (max < e.size()) return set_error(MOERT_E_RANGE, "pretokenize: %zu pieces do not fit in %zu", e.size(), max);
  for (size_t i = 0; i < e.size(); i++) ends[i] = offs[e[i]];
  return MOERT_OK;
}

int moert_format_date(int year, int month, int day, char* out, size_t max) {
  static const char* kMonths[12] = {"January", "February", "March",     "April",   "May",      "June",
                                    "July",    "August",   "September", "October", "November", "December"};
  if (month < 1 || month > 12) return set_error(MOERT_E_CONFIG, "date: month %d", month);
  const bool leap = (year % 4 == 0 && year % 100 != 0) || year % 400 == 0;
  const int days = month == 2 ? (leap ? 29 : 28) : (month == 4 || month == 6 || month == 9 || month == 11) ? 30 : 31;
  if (day < 1 || day > days || year < 1 || year > 9999)
    return set_error(MOERT_E_CONFIG, "date: %d-%d-%d", year, month, day);
  char buf[48];
  snprintf(buf, sizeof buf, "%s %02d, %04d", kMonths[month - 1], day, year);
  return put_out(std::string(buf) + '\0', out, max, nullptr);
}

int moert_chat_render(const int* roles, const char* const* contents, int n, int add_generation_prompt,
                      const char* date, char* out, size_t max, size_t* needed) {
  if (n < 1 || !roles || !contents) return set_error(MOERT_E_CONFIG, "chat: an empty list of messages");
  static const char* kRole[3] = {"system", "user", "assistant"};
  for (int i = 0; i < n; i++)
    if (roles[i] < 0 || roles[i] > 2 || !contents[i]) return set_error(MOERT_E_CONFIG, "chat: message %d", i);
  const std::string start = "<|start_of_role|>", end_role = "<|end_of_role|>", end = "<|end_of_text|>";
  std::string system;
  int first = 0;
  if (roles[0] == 0) {
    system = contents[0];
    first = 1;
  } else {
    system = std::string("Knowledge Cutoff Date: April 2024.\nToday's Date: ") + (date ? date : "") +
             ".\nYou are Granite, developed by IBM. You are a helpful AI assistant.";
  }
  std::string s = start + "system" + end_role + system + end + "\n";
  for (int i = first; i < n; i++) {
    s += start + kRole[roles[i]] + end_role + contents[i] + end + "\n";
    if (i + 1 == n && add_generation_prompt) s += start + "assistant" + end_role;
  }
  return put_out(s, out, max, needed);
}

}  // extern "C"
