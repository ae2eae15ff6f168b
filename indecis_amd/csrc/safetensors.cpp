// safetensors.cpp — an indecis model.safetensors straight into a model
// handle's device memory (host code; uses only the public C ABI).
//
// Format (safetensors/safetensors.go:112-243): an 8-byte little-endian
// header length n, n bytes of JSON {"name": {"dtype", "shape",
// "data_offsets": [start, end)}, "__metadata__": {...}}, then the data.
// The same checks as parseHeader / entry.bytes: n <= 100 MiB and inside
// the file; dtype F32, BF16, F16 or I8; no negative dimension; offsets
// inside the data; exactly shape-product elements.
//
// What Load (model.go:640-740) and FromTensors
// (internal/modernbert/model.go:181-234) read, without the float32 detour
// of the whole model:
//  * the embedding table in its stored format: I8 with the per-row
//    scales "indecis.embeddings.scale" (newInt8Embeddings), or BF16 with
//    the float32 rows "indecis.embeddings.exact_rows/_values"
//    (newMappedEmbeddings), uploaded as stored; F32 / F16 decoded;
//  * each layer matrix decoded to float32 one at a time and packed by
//    PackB8 (linalg/int8.go:38-77) on the host, as packs() does (infer.go:
//    184-219), then uploaded;
//  * the LayerNorm weights decoded to float32.
// Names follow transformers, with or without the "model." prefix.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/indecis_hip.h"
#include "ixh_internal.h"

namespace ixh {
namespace {

constexpr uint64_t kMaxHeader = 100ull << 20;  // maxHeader, safetensors.go:47

int efmt(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return set_error(IXH_EFORMAT, buf);
}

struct Entry {
  std::string dtype;
  std::vector<int64_t> shape;
  int64_t start = 0, end = 0;
  int64_t count() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

// ---- a small JSON reader: objects, arrays, strings, integers (the header) --
struct Json {
  const char *p, *e;
  std::string err;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool lit(char c) {
    ws();
    if (p < e && *p == c) {
      p++;
      return true;
    }
    return false;
  }
  bool str(std::string &out) {
    ws();
    if (p >= e || *p != '"') return fail("string expected");
    p++;
    out.clear();
    while (p < e && *p != '"') {
      if (*p == '\\') {
        if (++p >= e) break;
        switch (*p) {
        case 'n': out += '\n'; break;
        case 't': out += '\t'; break;
        case 'r': out += '\r'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'u': {  // \uXXXX: kept as UTF-8 for the BMP
          if (e - p < 5) return fail("bad escape");
          unsigned v = 0;
          for (int i = 1; i <= 4; i++) {
            const char c = p[i];
            v = v * 16 + (c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10
                          : c >= 'A' && c <= 'F' ? c - 'A' + 10 : 0);
          }
          if (v < 0x80) {
            out += (char)v;
          } else if (v < 0x800) {
            out += (char)(0xC0 | (v >> 6));
            out += (char)(0x80 | (v & 0x3F));
          } else {
            out += (char)(0xE0 | (v >> 12));
            out += (char)(0x80 | ((v >> 6) & 0x3F));
            out += (char)(0x80 | (v & 0x3F));
          }
          p += 4;
          break;
        }
        default: out += *p;
        }
        p++;
      } else {
        out += *p++;
      }
    }
    if (p >= e) return fail("unterminated string");
    p++;
    return true;
  }
  bool integer(int64_t &v) {
    ws();
    const char *s = p;
    bool neg = false;
    if (p < e && *p == '-') {
      neg = true;
      p++;
    }
    if (p >= e || *p < '0' || *p > '9') return fail("integer expected");
    v = 0;
    while (p < e && *p >= '0' && *p <= '9') {
      if (v > (int64_t)1 << 52) return fail("integer too large");
      v = v * 10 + (*p++ - '0');
    }
    if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) {
      p = s;
      return fail("integer expected");
    }
    if (neg) v = -v;
    return true;
  }
  // skips any value (the metadata)
  bool skip(int depth = 0) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("value expected");
    if (*p == '"') {
      std::string s;
      return str(s);
    }
    if (*p == '{' || *p == '[') {
      const char close = *p == '{' ? '}' : ']';
      const bool obj = *p == '{';
      p++;
      if (lit(close)) return true;
      do {
        if (obj) {
          std::string k;
          if (!str(k) || !lit(':')) return fail("object member expected");
        }
        if (!skip(depth + 1)) return false;
      } while (lit(','));
      return lit(close) || fail("unterminated container");
    }
    const char *s = p;
    while (p < e && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\n') p++;
    return p > s || fail("value expected");
  }
  bool fail(const char *m) {
    if (err.empty()) err = m;
    return false;
  }
};

bool parse_entry(Json &j, Entry &en) {
  if (!j.lit('{')) return j.fail("object expected");
  bool have_d = false, have_s = false, have_o = false;
  if (!j.lit('}')) {
    do {
      std::string k;
      if (!j.str(k) || !j.lit(':')) return j.fail("object member expected");
      if (k == "dtype") {
        if (!j.str(en.dtype)) return false;
        have_d = true;
      } else if (k == "shape") {
        if (!j.lit('[')) return j.fail("shape array expected");
        if (!j.lit(']')) {
          do {
            int64_t v;
            if (!j.integer(v)) return false;
            en.shape.push_back(v);
          } while (j.lit(','));
          if (!j.lit(']')) return j.fail("unterminated shape");
        }
        have_s = true;
      } else if (k == "data_offsets") {
        if (!j.lit('[') || !j.integer(en.start) || !j.lit(',') || !j.integer(en.end) || !j.lit(']'))
          return j.fail("data_offsets [start, end] expected");
        have_o = true;
      } else if (!j.skip()) {
        return false;
      }
    } while (j.lit(','));
    if (!j.lit('}')) return j.fail("unterminated object");
  }
  if (!have_d || !have_s || !have_o) return j.fail("dtype, shape and data_offsets expected");
  return true;
}

struct StFile {
  void *map = nullptr;
  size_t size = 0;
  const uint8_t *data = nullptr;  // after the header
  size_t data_size = 0;
  std::map<std::string, Entry> entries;
  ~StFile() {
    if (map) munmap(map, size);
  }
  const Entry *find(const std::string &name, std::string *found = nullptr) const {
    auto it = entries.find(name);
    if (it == entries.end()) it = entries.find("model." + name);
    if (it == entries.end()) return nullptr;
    if (found) *found = it->first;
    return &it->second;
  }
  const uint8_t *raw(const Entry &en) const { return data + en.start; }
};

int elem_size(const std::string &dt) {
  if (dt == "F32") return 4;
  if (dt == "BF16" || dt == "F16") return 2;
  if (dt == "I8") return 1;
  return 0;
}

// entry.bytes (safetensors.go:192-224)
int check_entry(const std::string &name, const Entry &en, size_t data_size) {
  for (int64_t d : en.shape)
    if (d < 0) return efmt("safetensors: %s: invalid shape", name.c_str());
  if (en.start < 0 || en.end < en.start || (uint64_t)en.end > data_size)
    return efmt("safetensors: %s: offsets [%lld, %lld) out of data bounds (%zu bytes)", name.c_str(),
                (long long)en.start, (long long)en.end, data_size);
  const int size = elem_size(en.dtype);
  if (!size) return efmt("safetensors: %s: unsupported dtype %s", name.c_str(), en.dtype.c_str());
  if (en.end - en.start != en.count() * size)
    return efmt("safetensors: %s: %lld bytes for %lld %s elements", name.c_str(),
                (long long)(en.end - en.start), (long long)en.count(), en.dtype.c_str());
  return IXH_OK;
}

int st_open(const char *path, StFile &f) {
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return efmt("safetensors: open %s: %s", path, strerror(errno));
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    close(fd);
    return efmt("safetensors: stat %s: %s", path, strerror(errno));
  }
  f.size = (size_t)sb.st_size;
  if (f.size > 0) {
    f.map = mmap(nullptr, f.size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (f.map == MAP_FAILED) {
      f.map = nullptr;
      close(fd);
      return efmt("safetensors: mmap %s: %s", path, strerror(errno));
    }
  }
  close(fd);
  const uint8_t *b = (const uint8_t *)f.map;
  if (f.size < 8) return efmt("safetensors: truncated file");
  uint64_t n = 0;
  for (int i = 7; i >= 0; i--) n = (n << 8) | b[i];
  if (n > kMaxHeader || 8 + n > f.size) return efmt("safetensors: invalid %llu-byte header", (unsigned long long)n);
  f.data = b + 8 + n;
  f.data_size = f.size - 8 - n;
  Json j{(const char *)b + 8, (const char *)b + 8 + n, {}};
  if (!j.lit('{')) return efmt("safetensors: header: object expected");
  if (!j.lit('}')) {
    do {
      std::string name;
      if (!j.str(name) || !j.lit(':')) return efmt("safetensors: header: %s", j.err.c_str());
      if (name == "__metadata__") {
        if (!j.skip()) return efmt("safetensors: metadata: %s", j.err.c_str());
        continue;
      }
      Entry en;
      if (!parse_entry(j, en)) return efmt("safetensors: %s: %s", name.c_str(), j.err.c_str());
      int rc;
      if ((rc = check_entry(name, en, f.data_size))) return rc;
      f.entries[name] = en;
    } while (j.lit(','));
    if (!j.lit('}')) return efmt("safetensors: header: unterminated object");
  }
  j.ws();
  if (j.p != j.e) return efmt("safetensors: header: trailing bytes");
  return IXH_OK;
}

uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// halfToFloat (safetensors.go:245-262)
float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 0x1f, mant = h & 0x3ff;
  uint32_t bits;
  if (ex == 0 && mant == 0) {
    bits = sign;
  } else if (ex == 0) {
    const float f = (float)mant / 1024 / 16384;
    return sign ? -f : f;
  } else if (ex == 0x1f) {
    bits = sign | 0xffu << 23 | mant << 13;
  } else {
    bits = sign | (ex + 112) << 23 | mant << 13;
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// decode (safetensors.go:226-243)
std::vector<float> decode(const StFile &f, const Entry &en) {
  const int64_t n = en.count();
  std::vector<float> out((size_t)n);
  const uint8_t *r = f.raw(en);
  if (en.dtype == "F32") {
    memcpy(out.data(), r, 4 * (size_t)n);  // little-endian host
  } else if (en.dtype == "BF16") {
    for (int64_t i = 0; i < n; i++) {
      const uint32_t bits = (uint32_t)le16(r + 2 * i) << 16;
      memcpy(&out[i], &bits, 4);
    }
  } else if (en.dtype == "F16") {
    for (int64_t i = 0; i < n; i++) out[i] = half_to_float(le16(r + 2 * i));
  } else {
    for (int64_t i = 0; i < n; i++) out[i] = (float)(int8_t)r[i];
  }
  return out;
}

int want_shape(const std::string &name, const Entry &en, std::vector<int64_t> shape) {
  if (en.shape == shape) return IXH_OK;
  auto fmt = [](const std::vector<int64_t> &s) {
    std::string t = "[";
    for (size_t i = 0; i < s.size(); i++) t += (i ? " " : "") + std::to_string(s[i]);
    return t + "]";
  };
  return efmt("modernbert: %s: shape %s, expected %s", name.c_str(), fmt(en.shape).c_str(), fmt(shape).c_str());
}

// PackB8 (linalg/int8.go:38-77) of W [n][k] (transB): per output channel
// s = f32(max|w| / 127), q = int8(Round(f64(f32(w / s)))), half away from
// zero; a zero channel keeps scale 0 and q 0.
void pack_b8(const std::vector<float> &w, int n, int k, std::vector<int8_t> &q, std::vector<float> &scale) {
  q.assign((size_t)n * k, 0);
  scale.assign(n, 0.f);
  for (int j = 0; j < n; j++) {
    const float *row = w.data() + (size_t)j * k;
    float mx = 0.f;
    for (int t = 0; t < k; t++) {
      const float a = fabsf(row[t]);
      mx = a > mx ? a : mx;
    }
    if (mx == 0.f) continue;
    const float s = mx / 127.0f;
    scale[j] = s;
    for (int t = 0; t < k; t++) {
      const float v = row[t] / s;
      q[(size_t)j * k + t] = (int8_t)std::round((double)v);
    }
  }
}

}  // namespace
}  // namespace ixh

using namespace ixh;

extern "C" int ixh_model_load_safetensors(ixh_model *m, const char *path) {
  if (!m || !path) return set_error(IXH_EINVAL, "modernbert: nil model or path");
  ixh_config cfg;
  model_config(m, &cfg);
  StFile f;
  int rc;
  if ((rc = st_open(path, f))) return rc;
  const int H = cfg.hidden, I = cfg.intermediate, V = cfg.vocab, layers = cfg.layers;
  auto need = [&](const std::string &name, std::vector<int64_t> shape, const Entry **out) {
    std::string found;
    const Entry *en = f.find(name, &found);
    if (!en) return efmt("modernbert: tensor %s missing", name.c_str());
    *out = en;
    return want_shape(name, *en, shape);
  };
  // embedding table (model.go:671-711)
  const Entry *emb;
  if ((rc = need("embeddings.tok_embeddings.weight", {V, H}, &emb))) return rc;
  if (emb->dtype == "I8") {
    const Entry *sc = f.find("indecis.embeddings.scale");
    if (!sc) return efmt("indecis: int8 table without scales");
    if ((rc = want_shape("indecis.embeddings.scale", *sc, {V}))) return rc;
    const std::vector<float> scale = decode(f, *sc);
    if ((rc = ixh_model_set_embeddings_i8(m, (const int8_t *)f.raw(*emb), scale.data()))) return rc;
  } else if (emb->dtype == "BF16") {
    std::vector<int32_t> ids;
    std::vector<float> rows;
    const Entry *er = f.find("indecis.embeddings.exact_rows");
    if (er) {
      const std::vector<float> r = decode(f, *er);
      const Entry *ev = f.find("indecis.embeddings.exact_values");
      if (!ev || ev->count() != (int64_t)r.size() * H) return efmt("indecis: malformed exact rows");
      for (float x : r) {
        if (!(x >= 0.f && x < (float)V) || x != std::floor(x)) return efmt("indecis: malformed exact rows");
        ids.push_back((int32_t)x);
      }
      rows = decode(f, *ev);
    }
    std::vector<uint16_t> table((size_t)V * H);
    memcpy(table.data(), f.raw(*emb), 2 * table.size());  // little-endian host
    if ((rc = ixh_model_set_embeddings_bf16(m, table.data(), ids.empty() ? nullptr : ids.data(),
                                            rows.empty() ? nullptr : rows.data(), (int)ids.size())))
      return rc;
  } else {
    const std::vector<float> t = decode(f, *emb);
    if ((rc = ixh_model_set_embeddings_f32(m, t.data()))) return rc;
  }
  // LayerNorm weights
  auto norm = [&](const std::string &name, int which, int layer) {
    const Entry *en;
    int r;
    if ((r = need(name, {H}, &en))) return r;
    const std::vector<float> g = decode(f, *en);
    return ixh_model_set_norm(m, which, layer, g.data());
  };
  if ((rc = norm("embeddings.norm.weight", IXH_NORM_EMB, 0)) || (rc = norm("final_norm.weight", IXH_NORM_FINAL, 0)))
    return rc;
  // layer matrices, one in float32 at a time
  std::vector<int8_t> q;
  std::vector<float> scale;
  auto matrix = [&](const std::string &name, int layer, int which, int n, int k) {
    const Entry *en;
    int r;
    if ((r = need(name, {n, k}, &en))) return r;
    const std::vector<float> w = decode(f, *en);
    pack_b8(w, n, k, q, scale);
    return ixh_model_set_matrix(m, layer, which, q.data(), scale.data(), IXH_LAYOUT_ROWS);
  };
  // in FromTensors' order, so the first missing tensor is the one it names
  for (int l = 0; l < layers; l++) {
    const std::string p = "layers." + std::to_string(l) + ".";
    if ((l > 0 && (rc = norm(p + "attn_norm.weight", IXH_NORM_ATTN, l))) ||
        (rc = matrix(p + "attn.Wqkv.weight", l, IXH_MAT_QKV, 3 * H, H)) ||
        (rc = matrix(p + "attn.Wo.weight", l, IXH_MAT_O, H, H)) ||
        (rc = norm(p + "mlp_norm.weight", IXH_NORM_MLP, l)) ||
        (rc = matrix(p + "mlp.Wi.weight", l, IXH_MAT_I, 2 * I, H)) ||
        (rc = matrix(p + "mlp.Wo.weight", l, IXH_MAT_OMLP, H, I)))
      return rc;
  }
  return IXH_OK;
}

extern "C" int ixh_safetensors_tensor(const char *path, const char *name, float *out, int64_t cap,
                                      int64_t *count) {
  if (!path || !name || !count) return set_error(IXH_EINVAL, "safetensors: nil argument");
  StFile f;
  int rc;
  if ((rc = st_open(path, f))) return rc;
  auto it = f.entries.find(name);
  if (it == f.entries.end()) return efmt("safetensors: %s: no such tensor", name);
  *count = it->second.count();
  if (!out) return IXH_OK;
  if (cap < *count) return set_error(IXH_EINVAL, "safetensors: output too short");
  const std::vector<float> v = decode(f, it->second);
  memcpy(out, v.data(), 4 * v.size());
  return IXH_OK;
}
