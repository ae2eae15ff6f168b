// tokenizer.cpp — the BPE tokenizer of the Gemma family as indecis runs it
// (tokenizer/tokenizer.go: exact parity with Hugging Face `tokenizers` for
// the configurations it accepts), natively and for many texts at once, so
// that tokenization keeps up with the GPU encoder (host code).
//
// Pipeline (tokenizer.go:1-20, 557-700):
//  1. added tokens are found in the raw text, leftmost-longest, before any
//     normalisation (with their lstrip / rstrip of Unicode spaces);
//  2. each remaining segment: ' ' -> U+2581; unless the pre-tokenizer is
//     the raw Split of the original Gemma pipeline, a leading U+2581 is
//     added and the segment is split before each U+2581;
//  3. BPE on each piece: characters of the vocabulary, else byte fallback
//     (<0xXX>), else <unk> (consecutive unknowns fused); merges by
//     increasing rank, the leftmost on equal ranks;
//  4. the post-processor's template (special tokens around A, or A and B).
// Only that configuration is accepted (checkSupported, tokenizer.go:
// 329-372); anything else is rejected at load time.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <queue>
#include <sstream>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/indecis_hip.h"
#include "ixh_internal.h"

namespace {

using ixh::set_error;

int terr(const std::string &m) { return set_error(IXH_EFORMAT, m.c_str()); }

const char kMeta[] = "\xE2\x96\x81";  // U+2581, the metaspace
constexpr int kMetaLen = 3;

// ---- JSON (a document model for tokenizer.json) ---------------------------
struct JV {
  enum K { NUL, BOOL, NUM, STR, ARR, OBJ } k = NUL;
  bool b = false;
  double num = 0;
  bool is_int = false;
  long long i = 0;
  std::string s;
  std::vector<JV> a;
  std::vector<std::pair<std::string, JV>> o;
  const JV *get(const char *key) const {
    if (k != OBJ) return nullptr;
    const JV *r = nullptr;
    for (const auto &kv : o)
      if (kv.first == key) r = &kv.second;  // the last of duplicate names
    return r;
  }
  std::string str(const char *key) const {
    const JV *v = get(key);
    return v && v->k == STR ? v->s : std::string();
  }
  bool flag(const char *key) const {
    const JV *v = get(key);
    return v && v->k == BOOL && v->b;
  }
  bool null_or_missing(const char *key) const {
    const JV *v = get(key);
    return !v || v->k == NUL;
  }
};

struct JP {
  const char *p, *e;
  std::string err;
  bool fail(const char *m) {
    if (err.empty()) err = m;
    return false;
  }
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  static void put_utf8(std::string &o, unsigned c) {
    if (c < 0x80) {
      o += (char)c;
    } else if (c < 0x800) {
      o += (char)(0xC0 | (c >> 6));
      o += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      o += (char)(0xE0 | (c >> 12));
      o += (char)(0x80 | ((c >> 6) & 0x3F));
      o += (char)(0x80 | (c & 0x3F));
    } else {
      o += (char)(0xF0 | (c >> 18));
      o += (char)(0x80 | ((c >> 12) & 0x3F));
      o += (char)(0x80 | ((c >> 6) & 0x3F));
      o += (char)(0x80 | (c & 0x3F));
    }
  }
  bool hex4(unsigned &v) {
    if (e - p < 4) return fail("bad \\u escape");
    v = 0;
    for (int i = 0; i < 4; i++) {
      const char c = *p++;
      const int d = c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10 : c >= 'A' && c <= 'F' ? c - 'A' + 10 : -1;
      if (d < 0) return fail("bad \\u escape");
      v = v * 16 + (unsigned)d;
    }
    return true;
  }
  bool string(std::string &o) {
    if (p >= e || *p != '"') return fail("string expected");
    p++;
    o.clear();
    for (;;) {
      if (p >= e) return fail("unterminated string");
      const char c = *p++;
      if (c == '"') return true;
      if (c != '\\') {
        o += c;
        continue;
      }
      if (p >= e) return fail("unterminated string");
      const char x = *p++;
      switch (x) {
      case '"': o += '"'; break;
      case '\\': o += '\\'; break;
      case '/': o += '/'; break;
      case 'b': o += '\b'; break;
      case 'f': o += '\f'; break;
      case 'n': o += '\n'; break;
      case 'r': o += '\r'; break;
      case 't': o += '\t'; break;
      case 'u': {
        unsigned v;
        if (!hex4(v)) return false;
        if (v >= 0xD800 && v < 0xDC00) {  // a surrogate pair
          unsigned lo = 0;
          if (e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            if (!hex4(lo)) return false;
          }
          if (lo >= 0xDC00 && lo < 0xE000) v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
          else v = 0xFFFD;
        } else if (v >= 0xDC00 && v < 0xE000) {
          v = 0xFFFD;
        }
        put_utf8(o, v);
        break;
      }
      default: return fail("bad escape");
      }
    }
  }
  bool value(JV &v, int depth = 0) {
    if (depth > 200) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("value expected");
    const char c = *p;
    if (c == '{') {
      p++;
      v.k = JV::OBJ;
      ws();
      if (p < e && *p == '}') {
        p++;
        return true;
      }
      for (;;) {
        ws();
        std::string key;
        if (!string(key)) return false;
        ws();
        if (p >= e || *p != ':') return fail("':' expected");
        p++;
        v.o.emplace_back(std::move(key), JV());
        if (!value(v.o.back().second, depth + 1)) return false;
        ws();
        if (p < e && *p == ',') {
          p++;
          continue;
        }
        if (p < e && *p == '}') {
          p++;
          return true;
        }
        return fail("',' or '}' expected");
      }
    }
    if (c == '[') {
      p++;
      v.k = JV::ARR;
      ws();
      if (p < e && *p == ']') {
        p++;
        return true;
      }
      for (;;) {
        v.a.emplace_back();
        if (!value(v.a.back(), depth + 1)) return false;
        ws();
        if (p < e && *p == ',') {
          p++;
          continue;
        }
        if (p < e && *p == ']') {
          p++;
          return true;
        }
        return fail("',' or ']' expected");
      }
    }
    if (c == '"') {
      v.k = JV::STR;
      return string(v.s);
    }
    if (e - p >= 4 && !strncmp(p, "true", 4)) {
      p += 4;
      v.k = JV::BOOL;
      v.b = true;
      return true;
    }
    if (e - p >= 5 && !strncmp(p, "false", 5)) {
      p += 5;
      v.k = JV::BOOL;
      return true;
    }
    if (e - p >= 4 && !strncmp(p, "null", 4)) {
      p += 4;
      v.k = JV::NUL;
      return true;
    }
    const char *s = p;
    if (p < e && (*p == '-' || *p == '+')) p++;
    bool frac = false;
    while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' || *p == '+')) {
      if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
      p++;
    }
    if (p == s) return fail("value expected");
    const std::string t(s, p);
    v.k = JV::NUM;
    v.num = strtod(t.c_str(), nullptr);
    if (!frac) {
      v.is_int = true;
      v.i = strtoll(t.c_str(), nullptr, 10);
    }
    return true;
  }
};

// ---- UTF-8 as Go decodes it (unicode/utf8) --------------------------------
constexpr unsigned kRuneError = 0xFFFD;

// the rune at s[i] and its width; invalid or incomplete: (U+FFFD, 1)
inline unsigned decode_rune(const char *s, size_t n, size_t i, int *w) {
  const unsigned char b0 = (unsigned char)s[i];
  if (b0 < 0x80) {
    *w = 1;
    return b0;
  }
  auto cont = [&](size_t k, unsigned char lo, unsigned char hi) {
    return i + k < n && (unsigned char)s[i + k] >= lo && (unsigned char)s[i + k] <= hi;
  };
  if (b0 >= 0xC2 && b0 <= 0xDF) {
    if (cont(1, 0x80, 0xBF)) {
      *w = 2;
      return ((b0 & 0x1Fu) << 6) | ((unsigned char)s[i + 1] & 0x3Fu);
    }
  } else if (b0 >= 0xE0 && b0 <= 0xEF) {
    const unsigned char lo = b0 == 0xE0 ? 0xA0 : 0x80, hi = b0 == 0xED ? 0x9F : 0xBF;
    if (cont(1, lo, hi) && cont(2, 0x80, 0xBF)) {
      *w = 3;
      return ((b0 & 0x0Fu) << 12) | (((unsigned char)s[i + 1] & 0x3Fu) << 6) | ((unsigned char)s[i + 2] & 0x3Fu);
    }
  } else if (b0 >= 0xF0 && b0 <= 0xF4) {
    const unsigned char lo = b0 == 0xF0 ? 0x90 : 0x80, hi = b0 == 0xF4 ? 0x8F : 0xBF;
    if (cont(1, lo, hi) && cont(2, 0x80, 0xBF) && cont(3, 0x80, 0xBF)) {
      *w = 4;
      return ((b0 & 0x07u) << 18) | (((unsigned char)s[i + 1] & 0x3Fu) << 12) |
             (((unsigned char)s[i + 2] & 0x3Fu) << 6) | ((unsigned char)s[i + 3] & 0x3Fu);
    }
  }
  *w = 1;
  return kRuneError;
}

// the last rune of s[0:end) (utf8.DecodeLastRuneInString)
inline unsigned decode_last_rune(const char *s, size_t end, int *w) {
  const size_t lim = end >= 4 ? end - 4 : 0;
  size_t start = end - 1;
  while (start > lim && ((unsigned char)s[start] & 0xC0) == 0x80) start--;
  int ww;
  const unsigned r = decode_rune(s, end, start, &ww);
  if (start + (size_t)ww != end) {
    *w = 1;
    return kRuneError;
  }
  *w = ww;
  return r;
}

inline int encode_rune(unsigned r, char *out) {
  if (r > 0x10FFFF || (r >= 0xD800 && r < 0xE000)) r = kRuneError;
  std::string t;
  JP::put_utf8(t, r);
  memcpy(out, t.data(), t.size());
  return (int)t.size();
}

// unicode.IsSpace
inline bool is_space(unsigned r) {
  if (r <= 0xFF) return r == '\t' || r == '\n' || r == '\v' || r == '\f' || r == '\r' || r == ' ' || r == 0x85 || r == 0xA0;
  return r == 0x1680 || (r >= 0x2000 && r <= 0x200A) || r == 0x2028 || r == 0x2029 || r == 0x202F || r == 0x205F ||
         r == 0x3000;
}

// ---- the tokenizer ---------------------------------------------------------
constexpr int32_t kSeqA = -1, kSeqB = -2;

struct Added {
  std::string content;
  int32_t id;
  bool lstrip, rstrip;
};

struct Sym {
  int32_t id;
  int prev, next;
  bool merged;
  int64_t start, end;
};

struct Cand {
  int pos;
  int32_t rank, id;
  bool operator<(const Cand &o) const {  // priority_queue: the top is the smallest (rank, pos)
    return rank != o.rank ? rank > o.rank : pos > o.pos;
  }
};

}  // namespace

struct ixh_tokenizer {
  std::vector<std::string> by_id;                    // vocabulary strings ("" = absent)
  std::unordered_map<std::string, int32_t> vocab;
  std::unordered_map<uint32_t, int32_t> single;      // one-rune tokens, by rune
  std::unordered_map<uint64_t, std::pair<int32_t, int32_t>> merges;  // (a,b) -> (rank, id)
  std::vector<Added> added[256];                     // by first byte, longest first
  std::unordered_map<int32_t, std::string> names;
  int32_t size = 0, unk = 0, bos = 0, eos = 0, pad = 0;
  int32_t bytes[256];
  bool raw = false;
  std::vector<int32_t> tmpl_single, tmpl_pair;

  bool lookup_vocab(const std::string &s, int32_t *id) const {
    auto it = vocab.find(s);
    if (it == vocab.end()) return false;
    *id = it->second;
    return true;
  }
  // tokenizer.go:465-477: the vocabulary, then the added tokens
  bool lookup(const std::string &s, int32_t *id) const {
    if (lookup_vocab(s, id)) return true;
    for (int b = 0; b < 256; b++)
      for (const Added &a : added[b])
        if (a.content == s) {
          *id = a.id;
          return true;
        }
    return false;
  }
  const std::pair<int32_t, int32_t> *merge(int32_t a, int32_t b) const {
    auto it = merges.find((uint64_t)(uint32_t)a << 32 | (uint32_t)b);
    return it == merges.end() ? nullptr : &it->second;
  }
  int32_t rune_id(unsigned r, bool *ok) const {
    auto it = single.find(r);
    if (it != single.end()) {
      *ok = true;
      return it->second;
    }
    *ok = false;
    return 0;
  }

  // bpeSymbols (tokenizer.go:741-822): src (optional) gives the source
  // offset of each byte of the piece (-1: none)
  void bpe(const char *w, size_t n, const int64_t *src, std::vector<Sym> &syms) const {
    syms.clear();
    bool last_unk = false;
    for (size_t bi = 0; bi < n;) {
      int width;
      const unsigned r = decode_rune(w, n, bi, &width);
      int64_t start = -1, end = -1;
      if (src)
        for (int k = 0; k < width; k++) {
          const int64_t o = src[bi + k];
          if (o < 0) continue;
          if (start < 0 || o < start) start = o;
          end = std::max(end, o + 1);
        }
      bi += (size_t)width;
      bool ok;
      const int32_t id = rune_id(r, &ok);
      if (ok) {
        syms.push_back({id, 0, 0, false, start, end});
        last_unk = false;
        continue;
      }
      char buf[4];
      const int nb = encode_rune(r, buf);
      bool fallback = true;
      for (int k = 0; k < nb; k++)
        if (bytes[(unsigned char)buf[k]] < 0) fallback = false;
      if (fallback) {
        for (int k = 0; k < nb; k++) syms.push_back({bytes[(unsigned char)buf[k]], 0, 0, false, start, end});
        last_unk = false;
        continue;
      }
      if (last_unk) {
        Sym &l = syms.back();
        if (l.start < 0) {
          l.start = start;
          l.end = end;
        } else if (start >= 0) {
          l.start = std::min(l.start, start);
          l.end = std::max(l.end, end);
        }
      } else {
        syms.push_back({unk, 0, 0, false, start, end});
      }
      last_unk = true;
    }
    const int ns = (int)syms.size();
    for (int i = 0; i < ns; i++) {
      syms[i].prev = i - 1;
      syms[i].next = i + 1 < ns ? i + 1 : -1;
    }
    std::priority_queue<Cand> q;
    for (int i = 0; i + 1 < ns; i++)
      if (const auto *m = merge(syms[i].id, syms[i + 1].id)) q.push({i, m->first, m->second});
    while (!q.empty()) {
      const Cand top = q.top();
      q.pop();
      Sym &cur = syms[top.pos];
      if (cur.merged || cur.next < 0) continue;
      const Sym right = syms[cur.next];
      const auto *m = merge(cur.id, right.id);
      if (!m || m->second != top.id) continue;  // stale
      cur.id = top.id;
      if (cur.start < 0) {
        cur.start = right.start;
        cur.end = right.end;
      } else if (right.start >= 0) {
        cur.start = std::min(cur.start, right.start);
        cur.end = std::max(cur.end, right.end);
      }
      syms[cur.next].merged = true;
      cur.next = right.next;
      if (right.next >= 0) syms[right.next].prev = top.pos;
      if (cur.prev >= 0)
        if (const auto *mp = merge(syms[cur.prev].id, cur.id)) q.push({cur.prev, mp->first, mp->second});
      if (cur.next >= 0)
        if (const auto *mn = merge(cur.id, syms[cur.next].id)) q.push({top.pos, mn->first, mn->second});
    }
  }

  // matchAdded: the longest added token at text[i]
  const Added *match_added(const char *t, size_t n, size_t i) const {
    for (const Added &a : added[(unsigned char)t[i]])
      if (a.content.size() <= n - i && !memcmp(t + i, a.content.data(), a.content.size())) return &a;
    return nullptr;
  }

  // walkSpans (tokenizer.go:622-657)
  template <class FA, class FS>
  void walk_spans(const char *t, size_t n, FA on_added, FS on_segment) const {
    size_t start = 0, i = 0;
    while (i < n) {
      const Added *a = match_added(t, n, i);
      if (!a) {
        i++;
        continue;
      }
      size_t ms = i, me = i + a->content.size();
      if (a->lstrip)
        while (ms > start) {
          int w;
          const unsigned r = decode_last_rune(t + start, ms - start, &w);
          if (!is_space(r)) break;
          ms -= (size_t)w;
        }
      if (a->rstrip)
        while (me < n) {
          int w;
          const unsigned r = decode_rune(t, n, me, &w);
          if (!is_space(r)) break;
          me += (size_t)w;
        }
      if (ms > start) on_segment(start, ms);
      on_added(a->id, ms, me);
      start = i = me;
    }
    if (start < n) on_segment(start, n);
  }

  // walkSegmentSrc (tokenizer.go:528-574): normalise text[start:end],
  // pieces with the source offset of each byte
  template <class FW>
  void walk_segment(const char *t, size_t start, size_t end, std::string &s, std::vector<int64_t> &src,
                    FW on_piece) const {
    s.clear();
    src.clear();
    if (!raw && t[start] != ' ' && !(end - start >= (size_t)kMetaLen && !memcmp(t + start, kMeta, kMetaLen))) {
      int w;
      decode_rune(t, end, start, &w);
      s.append(kMeta, kMetaLen);
      src.push_back((int64_t)start);
      src.push_back((int64_t)(start + w - 1));
      src.push_back((int64_t)(start + w - 1));
    }
    for (size_t i = start; i < end; i++) {
      if (t[i] == ' ') {
        s.append(kMeta, kMetaLen);
        for (int k = 0; k < kMetaLen; k++) src.push_back((int64_t)i);
        continue;
      }
      s += t[i];
      src.push_back((int64_t)i);
    }
    if (raw) {
      on_piece(s.data(), s.size(), src.data());
      return;
    }
    size_t from = 0;
    for (;;) {
      const size_t next = s.find(kMeta, from + kMetaLen);
      if (next == std::string::npos) {
        on_piece(s.data() + from, s.size() - from, src.data() + from);
        return;
      }
      on_piece(s.data() + from, next - from, src.data() + from);
      from = next;
    }
  }

  // AppendOffsets (tokenizer.go:512-526); starts/ends may be null
  void encode_text(const char *t, size_t n, std::vector<int32_t> &ids, std::vector<int64_t> *starts,
                   std::vector<int64_t> *ends, std::vector<Sym> &syms, std::string &s,
                   std::vector<int64_t> &src) const {
    walk_spans(
        t, n,
        [&](int32_t id, size_t a, size_t b) {
          ids.push_back(id);
          if (starts) {
            starts->push_back((int64_t)a);
            ends->push_back((int64_t)b);
          }
        },
        [&](size_t a, size_t b) {
          walk_segment(t, a, b, s, src, [&](const char *w, size_t wn, const int64_t *ws) {
            bpe(w, wn, ws, syms);
            for (int i = syms.empty() ? -1 : 0; i >= 0; i = syms[i].next) {
              ids.push_back(syms[i].id);
              if (starts) {
                starts->push_back(syms[i].start);
                ends->push_back(syms[i].end);
              }
            }
          });
        });
  }
};

namespace {

struct Scratch {
  std::vector<Sym> syms;
  std::string s;
  std::vector<int64_t> src;
};

int specials(const std::vector<int32_t> &tm) {
  int k = 0;
  for (int32_t x : tm) k += x >= 0;
  return k;
}

void fill(const std::vector<int32_t> &tm, const std::vector<int32_t> &a, const std::vector<int32_t> &b,
          std::vector<int32_t> &out) {
  out.clear();
  for (int32_t x : tm) {
    if (x == kSeqA) out.insert(out.end(), a.begin(), a.end());
    else if (x == kSeqB) out.insert(out.end(), b.begin(), b.end());
    else out.push_back(x);
  }
}

// EncodeMax / Encode (tokenizer.go:479-495): max_len < 0 keeps everything
void encode_single(const ixh_tokenizer *t, const char *text, size_t n, int max_len, Scratch &sc,
                   std::vector<int32_t> &a, std::vector<int32_t> &out) {
  a.clear();
  t->encode_text(text, n, a, nullptr, nullptr, sc.syms, sc.s, sc.src);
  if (max_len >= 0) {
    const int budget = std::max(max_len - specials(t->tmpl_single), 0);
    if ((int)a.size() > budget) a.resize(budget);
  }
  static const std::vector<int32_t> none;
  fill(t->tmpl_single, a, none, out);
}

int parse_template(const ixh_tokenizer *t, const JV *pieces, int nseq, std::vector<int32_t> &out) {
  out.clear();
  if (!pieces || pieces->k != JV::ARR) return terr("tokenizer: template missing");
  const char *seqs[2] = {"A", "B"};
  int next = 0;
  for (const JV &p : pieces->a) {
    const JV *seq = p.get("Sequence"), *sp = p.get("SpecialToken");
    if (seq && seq->k == JV::OBJ) {
      if (next >= nseq || seq->str("id") != seqs[next]) return terr("tokenizer: template sequences out of order");
      out.push_back(kSeqA - next);
      next++;
    } else if (sp && sp->k == JV::OBJ) {
      int32_t id;
      const std::string name = sp->str("id");
      if (!t->lookup(name, &id)) return terr("tokenizer: template token \"" + name + "\" missing");
      out.push_back(id);
    } else {
      return terr("tokenizer: empty template piece");
    }
  }
  if (next != nseq) return terr("tokenizer: template without its " + std::to_string(nseq) + " sequence(s)");
  return IXH_OK;
}

// read + checkSupported + pipeline (tokenizer.go:244-372)
int build(const JV &doc, ixh_tokenizer &t) {
  if (doc.k != JV::OBJ) return terr("tokenizer: expected an object");
  const JV *model = doc.get("model");
  if (!model || model->k != JV::OBJ) return terr("tokenizer: model missing");
  // checkSupported
  if (model->str("type") != "BPE") return terr("tokenizer: model \"" + model->str("type") + "\" not supported");
  if (const JV *d = model->get("dropout"); d && d->k == JV::NUM && d->num != 0)
    return terr("tokenizer: BPE dropout not supported");
  for (const char *k : {"continuing_subword_prefix", "end_of_word_suffix"})
    if (const JV *v = model->get(k); v && v->k == JV::STR && !v->s.empty())
      return terr("tokenizer: subword prefix/suffix not supported");
  if (!model->flag("byte_fallback") || !model->flag("fuse_unk") || model->flag("ignore_merges"))
    return terr("tokenizer: expected byte_fallback=true, fuse_unk=true, ignore_merges=false");
  const JV *norm = doc.get("normalizer");
  const bool has_norm = norm && norm->k == JV::OBJ;
  if (has_norm) {
    const JV *pat = norm->get("pattern");
    if (norm->str("type") != "Replace" || !pat || pat->str("String") != " " || norm->str("content") != kMeta)
      return terr("tokenizer: normalizer not supported");
  }
  const JV *pre = doc.get("pre_tokenizer"), *post = doc.get("post_processor");
  if (!post || post->k != JV::OBJ || post->str("type") != "TemplateProcessing")
    return terr("tokenizer: expected a TemplateProcessing post-processor");
  const bool pre_obj = pre && pre->k == JV::OBJ;
  if (pre_obj && pre->str("type") == "Metaspace" && pre->str("replacement") == kMeta &&
      pre->str("prepend_scheme") == "always" && pre->flag("split")) {
    t.raw = false;
  } else if (pre_obj && pre->str("type") == "Split" && pre->get("pattern") && pre->get("pattern")->str("String") == " " &&
             pre->str("behavior") == "MergedWithPrevious" && !pre->flag("invert") && has_norm) {
    t.raw = true;
  } else {
    return terr("tokenizer: expected pre-tokenizer: Metaspace(\xE2\x96\x81, always, split) or Split(\" \", merged with previous)");
  }
  // vocabulary (decodeVocab, stream.go:98-133)
  const JV *vocab = model->get("vocab");
  if (!vocab || vocab->k != JV::OBJ) return terr("tokenizer: vocab missing");
  for (const auto &kv : vocab->o) {
    if (kv.second.k != JV::NUM || !kv.second.is_int) return terr("tokenizer: vocab: expected id for \"" + kv.first + "\"");
    const long long id = kv.second.i;
    if (id < 0 || id > (1 << 30)) return terr("tokenizer: vocab: id out of range");
    if ((size_t)id >= t.by_id.size()) t.by_id.resize((size_t)id + 1);
    t.by_id[(size_t)id] = kv.first;
  }
  // added tokens
  const JV *added = doc.get("added_tokens");
  std::vector<Added> all;
  if (added && added->k == JV::ARR)
    for (const JV &a : added->a) {
      const JV *idv = a.get("id");
      if (!idv || !idv->is_int) return terr("tokenizer: added token without id");
      if (idv->i < 0) return terr("tokenizer: id " + std::to_string(idv->i) + " negative");
      Added ad{a.str("content"), (int32_t)idv->i, a.flag("lstrip"), a.flag("rstrip")};
      if (a.flag("normalized") || a.flag("single_word") || ad.content.empty())
        return terr("tokenizer: added token \"" + ad.content + "\": normalized/single_word not supported");
      if ((size_t)ad.id >= t.by_id.size()) t.by_id.resize((size_t)ad.id + 1);
      all.push_back(ad);
    }
  t.size = (int32_t)t.by_id.size();
  for (size_t id = 0; id < t.by_id.size(); id++) {
    const std::string &s = t.by_id[id];
    if (s.empty()) continue;
    t.vocab.emplace(s, (int32_t)id);
    int w;
    const unsigned r = decode_rune(s.data(), s.size(), 0, &w);
    if ((size_t)w == s.size() && !(r == kRuneError && w == 1)) t.single.emplace(r, (int32_t)id);
  }
  for (const Added &a : all) {
    if (t.by_id[a.id] != a.content) t.names[a.id] = a.content;
    t.added[(unsigned char)a.content[0]].push_back(a);
  }
  for (auto &list : t.added)
    std::stable_sort(list.begin(), list.end(), [](const Added &x, const Added &y) { return x.content.size() > y.content.size(); });
  if (!t.lookup(model->str("unk_token"), &t.unk)) return terr("tokenizer: unk token \"" + model->str("unk_token") + "\" missing");
  if (!t.lookup("<bos>", &t.bos)) return terr("tokenizer: <bos> missing");
  if (!t.lookup("<eos>", &t.eos)) return terr("tokenizer: <eos> missing");
  if (!t.lookup("<pad>", &t.pad)) t.pad = 0;
  int rc;
  if ((rc = parse_template(&t, post->get("single"), 1, t.tmpl_single)) || (rc = parse_template(&t, post->get("pair"), 2, t.tmpl_pair)))
    return rc;
  for (int b = 0; b < 256; b++) {
    char name[8];
    snprintf(name, sizeof name, "<0x%02X>", b);
    if (!t.lookup_vocab(name, &t.bytes[b])) t.bytes[b] = -1;
  }
  // merges (decodeMerges, stream.go:135-171), rank = position
  const JV *merges = model->get("merges");
  if (merges && merges->k == JV::ARR) {
    int32_t rank = 0;
    t.merges.reserve(merges->a.size() * 2);
    for (const JV &m : merges->a) {
      std::string a, b;
      if (m.k == JV::STR) {
        const size_t sp = m.s.find(' ');
        if (sp == std::string::npos) return terr("tokenizer: invalid merge \"" + m.s + "\"");
        a = m.s.substr(0, sp);
        b = m.s.substr(sp + 1);
      } else if (m.k == JV::ARR && m.a.size() == 2 && m.a[0].k == JV::STR && m.a[1].k == JV::STR) {
        a = m.a[0].s;
        b = m.a[1].s;
      } else {
        return terr("tokenizer: merges: unexpected element");
      }
      int32_t ia, ib, im;
      if (!t.lookup_vocab(a, &ia) || !t.lookup_vocab(b, &ib) || !t.lookup_vocab(a + b, &im))
        return terr("tokenizer: merge \"" + a + "\" \"" + b + "\" out of vocabulary");
      t.merges.emplace((uint64_t)(uint32_t)ia << 32 | (uint32_t)ib, std::make_pair(rank, im));
      rank++;
    }
  }
  return IXH_OK;
}

int out_ids(const std::vector<int32_t> &ids, int32_t *out, int64_t cap, int64_t *n) {
  *n = (int64_t)ids.size();
  if (!out) return IXH_OK;
  if (cap < *n) return set_error(IXH_EINVAL, "tokenizer: output too short");
  memcpy(out, ids.data(), 4 * ids.size());
  return IXH_OK;
}

}  // namespace

extern "C" {

int ixh_tokenizer_load(const char *path, ixh_tokenizer **out) {
  if (!path || !out) return set_error(IXH_EINVAL, "tokenizer: nil argument");
  std::ifstream f(path, std::ios::binary);
  if (!f) return terr(std::string("tokenizer: open ") + path);
  std::stringstream ss;
  ss << f.rdbuf();
  const std::string data = ss.str();
  JV doc;
  JP jp{data.data(), data.data() + data.size(), {}};
  if (!jp.value(doc)) return terr("tokenizer: " + jp.err);
  jp.ws();
  if (jp.p != jp.e) return terr("tokenizer: trailing bytes after the JSON value");
  auto t = std::make_unique<ixh_tokenizer>();
  int rc;
  if ((rc = build(doc, *t))) return rc;
  *out = t.release();
  return IXH_OK;
}

void ixh_tokenizer_destroy(ixh_tokenizer *t) { delete t; }

int ixh_tokenizer_info(const ixh_tokenizer *t, int32_t *vocab_size, int32_t *bos, int32_t *eos, int32_t *pad) {
  if (!t) return set_error(IXH_EINVAL, "tokenizer: nil tokenizer");
  if (vocab_size) *vocab_size = t->size;
  if (bos) *bos = t->bos;
  if (eos) *eos = t->eos;
  if (pad) *pad = t->pad;
  return IXH_OK;
}

int ixh_tokenizer_encode(const ixh_tokenizer *t, const char *text, int64_t len, int max_len, int32_t *ids,
                         int64_t cap, int64_t *n) {
  if (!t || (!text && len > 0) || len < 0 || !n) return set_error(IXH_EINVAL, "tokenizer: bad arguments");
  Scratch sc;
  std::vector<int32_t> a, out;
  encode_single(t, text, (size_t)len, max_len, sc, a, out);
  return out_ids(out, ids, cap, n);
}

int ixh_tokenizer_encode_pair(const ixh_tokenizer *t, const char *context, int64_t clen, const char *text,
                              int64_t tlen, int max_len, int32_t *ids, int64_t cap, int64_t *n) {
  if (!t || (!context && clen > 0) || (!text && tlen > 0) || clen < 0 || tlen < 0 || !n)
    return set_error(IXH_EINVAL, "tokenizer: bad arguments");
  Scratch sc;
  std::vector<int32_t> a, b, out;
  t->encode_text(context, (size_t)clen, a, nullptr, nullptr, sc.syms, sc.s, sc.src);
  t->encode_text(text, (size_t)tlen, b, nullptr, nullptr, sc.syms, sc.s, sc.src);
  if (max_len > 0) {  // EncodePair (tokenizer.go:497-518)
    const int budget = std::max(max_len - specials(t->tmpl_pair), 0);
    if ((int)(a.size() + b.size()) > budget) {
      int keep_a = std::min((int)a.size(), budget / 3);
      const int keep_b = std::min((int)b.size(), budget - keep_a);
      keep_a = std::min((int)a.size(), budget - keep_b);
      a.resize(keep_a);
      b.resize(keep_b);
    }
  }
  fill(t->tmpl_pair, a, b, out);
  return out_ids(out, ids, cap, n);
}

int ixh_tokenizer_encode_offsets(const ixh_tokenizer *t, const char *text, int64_t len, int32_t *ids,
                                 int64_t *starts, int64_t *ends, int64_t cap, int64_t *n) {
  if (!t || (!text && len > 0) || len < 0 || !n) return set_error(IXH_EINVAL, "tokenizer: bad arguments");
  Scratch sc;
  std::vector<int32_t> a;
  std::vector<int64_t> as, ae;
  t->encode_text(text, (size_t)len, a, &as, &ae, sc.syms, sc.s, sc.src);
  // EncodeOffsets (tokenizer.go:525-540): template specials are [0, 0)
  std::vector<int32_t> out;
  std::vector<int64_t> os, oe;
  for (int32_t x : t->tmpl_single) {
    if (x == kSeqA) {
      out.insert(out.end(), a.begin(), a.end());
      os.insert(os.end(), as.begin(), as.end());
      oe.insert(oe.end(), ae.begin(), ae.end());
    } else {
      out.push_back(x);
      os.push_back(0);
      oe.push_back(0);
    }
  }
  *n = (int64_t)out.size();
  if (!ids) return IXH_OK;
  if (cap < *n) return set_error(IXH_EINVAL, "tokenizer: output too short");
  memcpy(ids, out.data(), 4 * out.size());
  if (starts) memcpy(starts, os.data(), 8 * os.size());
  if (ends) memcpy(ends, oe.data(), 8 * oe.size());
  return IXH_OK;
}

}  // extern "C"

namespace ixh {

// EncodeMax of n texts on `threads` worker threads (0: one per core), one
// id vector a text; the arguments checked as the batch entry documents.
int tokenize_texts(const ixh_tokenizer *t, const char *const *texts, const int64_t *lens, int n, int max_len,
                   int threads, std::vector<std::vector<int32_t>> &per) {
  if (!t || n < 0 || (n > 0 && (!texts || !lens))) return set_error(IXH_EINVAL, "tokenizer: bad arguments");
  for (int i = 0; i < n; i++)
    if (lens[i] < 0 || (!texts[i] && lens[i] > 0)) return set_error(IXH_EINVAL, "tokenizer: bad text");
  per.assign(n, {});
  if (n == 0) return IXH_OK;
  const int nt = std::max(1, std::min(threads > 0 ? threads : (int)std::thread::hardware_concurrency(), n));
  auto work = [&](int w) {
    Scratch sc;
    std::vector<int32_t> a;
    for (int i = w; i < n; i += nt) encode_single(t, texts[i], (size_t)lens[i], max_len, sc, a, per[i]);
  };
  std::vector<std::thread> pool;
  for (int w = 1; w < nt; w++) pool.emplace_back(work, w);
  work(0);
  for (auto &th : pool) th.join();
  return IXH_OK;
}

}  // namespace ixh

extern "C" {

int ixh_tokenizer_encode_batch(const ixh_tokenizer *t, const char *const *texts, const int64_t *lens, int n,
                               int max_len, int threads, int32_t *ids, int64_t cap, int32_t *offs) {
  if (n > 0 && !offs) return set_error(IXH_EINVAL, "tokenizer: bad arguments");
  std::vector<std::vector<int32_t>> per;
  int rc = ixh::tokenize_texts(t, texts, lens, n, max_len, threads, per);
  if (rc) return rc;
  if (offs) offs[0] = 0;
  if (n == 0) return IXH_OK;
  int64_t total = 0;
  for (int i = 0; i < n; i++) {
    total += (int64_t)per[i].size();
    if (total > INT32_MAX) return set_error(IXH_EINVAL, "tokenizer: batch over 2^31 tokens");
    offs[i + 1] = (int32_t)total;
  }
  if (!ids) return IXH_OK;
  if (cap < total) return set_error(IXH_EINVAL, "tokenizer: output too short");
  for (int i = 0; i < n; i++)
    if (!per[i].empty()) memcpy(ids + offs[i], per[i].data(), 4 * per[i].size());
  return IXH_OK;
}

}  // extern "C"
