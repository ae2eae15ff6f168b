// host_check.cpp — the library's host-only C++ (tokenizer.cpp,
// safetensors.cpp, embed.cpp) run under AddressSanitizer + UBSan or
// ThreadSanitizer on the CPU (tests/test_sanitizers.py builds and runs
// it). No GPU is involved: the model entry points those files call are
// stubbed below and never reached.
//
//  1. the batch tokenizer on 8 worker threads, twice, against one-by-one
//     Encode of the same texts (random UTF-8, invalid bytes, empty texts);
//     8 threads encoding (plain, pair, offsets) with one shared handle;
//  2. the safetensors reader (ixh_safetensors_tensor) on a valid file,
//     then on every truncation of it, on 2,000 random corruptions of its
//     header bytes and on hand-made malformed headers: every call returns
//     (an error or a value), none reads out of bounds;
//  3. ixh_embed_normalize on random rows.
// Usage: host_check <tokenizer.json> <scratch dir>. Exit status 0 when
// every check holds (a sanitizer report aborts with a nonzero status).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "../../include/indecis_hip.h"

// ---- stubs of what the host sources link against in ixh_api.cpp ----------
namespace ixh {
thread_local std::string g_err;
int set_error(int code, const char *msg) {
  g_err = msg;
  return code;
}
void model_config(const ::ixh_model *, ::ixh_config *out) { memset(out, 0, sizeof *out); }
}  // namespace ixh
static int no_device() { return ixh::set_error(IXH_EHIP, "host_check: no device"); }
extern "C" {
const char *ixh_last_error(void) { return ixh::g_err.c_str(); }
int ixh_model_set_matrix(ixh_model *, int, int, const int8_t *, const float *, int) { return no_device(); }
int ixh_model_set_norm(ixh_model *, int, int, const float *) { return no_device(); }
int ixh_model_set_embeddings_f32(ixh_model *, const float *) { return no_device(); }
int ixh_model_set_embeddings_bf16(ixh_model *, const uint16_t *, const int32_t *, const float *, int) {
  return no_device();
}
int ixh_model_set_embeddings_i8(ixh_model *, const int8_t *, const float *) { return no_device(); }
int ixh_encode_seqs(ixh_model *, const int32_t *, const int32_t *, int, float *) { return no_device(); }
}

static int failures = 0;
#define CHECK(cond, ...)                                                  \
  do {                                                                    \
    if (!(cond)) {                                                        \
      fprintf(stderr, "host_check: %s:%d: ", __FILE__, __LINE__);        \
      fprintf(stderr, __VA_ARGS__);                                       \
      fprintf(stderr, "\n");                                              \
      failures++;                                                         \
    }                                                                     \
  } while (0)

static std::string random_text(std::mt19937 &rng) {
  static const char *words[] = {"the", " quick", " brown", "fox", " jumps", "  ", "\n", "déjà",
                                " vu", "日本語", " emoji 😀", ".", ",", "ab12", " x"};
  std::string s;
  const int n = (int)(rng() % 40);
  for (int i = 0; i < n; i++) {
    if (rng() % 17 == 0) {
      s += (char)(0x80 + rng() % 64);  // a stray continuation byte
    } else {
      s += words[rng() % (sizeof words / sizeof *words)];
    }
  }
  return s;
}

static void check_tokenizer(const char *path) {
  ixh_tokenizer *t = nullptr;
  int rc = ixh_tokenizer_load(path, &t);
  CHECK(rc == 0, "tokenizer load: %s", ixh_last_error());
  if (rc) return;
  std::mt19937 rng(7);
  std::vector<std::string> texts;
  for (int i = 0; i < 600; i++) texts.push_back(random_text(rng));
  texts.push_back("");
  const int n = (int)texts.size();
  std::vector<const char *> ptr(n);
  std::vector<int64_t> len(n);
  for (int i = 0; i < n; i++) {
    ptr[i] = texts[i].data();
    len[i] = (int64_t)texts[i].size();
  }
  // one by one
  std::vector<std::vector<int32_t>> want(n);
  for (int i = 0; i < n; i++) {
    int64_t cnt = 0;
    rc = ixh_tokenizer_encode(t, ptr[i], len[i], 64, nullptr, 0, &cnt);
    CHECK(rc == 0, "encode %d: %s", i, ixh_last_error());
    want[i].resize(cnt);
    rc = ixh_tokenizer_encode(t, ptr[i], len[i], 64, want[i].data(), cnt, &cnt);
    CHECK(rc == 0 && (size_t)cnt == want[i].size(), "encode %d again", i);
  }
  // the batch entry on 8 worker threads, twice
  for (int round = 0; round < 2; round++) {
    std::vector<int32_t> offs(n + 1);
    rc = ixh_tokenizer_encode_batch(t, ptr.data(), len.data(), n, 64, 8, nullptr, 0, offs.data());
    CHECK(rc == 0, "batch offsets: %s", ixh_last_error());
    std::vector<int32_t> ids(offs[n] + 1);
    rc = ixh_tokenizer_encode_batch(t, ptr.data(), len.data(), n, 64, 8, ids.data(), (int64_t)ids.size(),
                                    offs.data());
    CHECK(rc == 0, "batch: %s", ixh_last_error());
    for (int i = 0; i < n; i++) {
      const std::vector<int32_t> got(ids.begin() + offs[i], ids.begin() + offs[i + 1]);
      CHECK(got == want[i], "batch text %d differs", i);
    }
  }
  // 8 threads sharing the handle
  std::vector<std::thread> th;
  std::vector<int> bad(8, 0);
  for (int w = 0; w < 8; w++)
    th.emplace_back([&, w]() {
      std::vector<int32_t> ids(256);
      std::vector<int64_t> st(256), en(256);
      for (int i = w; i < n; i += 8) {
        int64_t cnt = 0;
        if (ixh_tokenizer_encode(t, ptr[i], len[i], 64, ids.data(), 256, &cnt) != 0 ||
            std::vector<int32_t>(ids.begin(), ids.begin() + cnt) != want[i])
          bad[w]++;
        if (ixh_tokenizer_encode_pair(t, ptr[i], len[i], ptr[(i + 1) % n], len[(i + 1) % n], 48, ids.data(), 256,
                                      &cnt) != 0)
          bad[w]++;
        if (len[i] < 200 && ixh_tokenizer_encode_offsets(t, ptr[i], len[i], ids.data(), st.data(), en.data(), 256,
                                                         &cnt) != 0)
          bad[w]++;
      }
    });
  for (auto &x : th) x.join();
  for (int w = 0; w < 8; w++) CHECK(bad[w] == 0, "thread %d: %d failed calls", w, bad[w]);
  ixh_tokenizer_destroy(t);
}

static void put_u64(std::string &s, uint64_t v) {
  for (int i = 0; i < 8; i++) s += (char)((v >> (8 * i)) & 0xff);
}

static bool write_file(const std::string &path, const std::string &bytes) {
  FILE *f = fopen(path.c_str(), "wb");
  if (!f) return false;
  const bool ok = fwrite(bytes.data(), 1, bytes.size(), f) == bytes.size();
  return fclose(f) == 0 && ok;
}

static int read_tensor(const std::string &path, const char *name, std::vector<float> &out) {
  int64_t count = 0;
  int rc = ixh_safetensors_tensor(path.c_str(), name, nullptr, 0, &count);
  if (rc) return rc;
  if (count < 0 || count > (1 << 20)) return -1;
  out.assign(count + 1, 0.f);
  return ixh_safetensors_tensor(path.c_str(), name, out.data(), count, &count);
}

static void check_safetensors(const std::string &dir) {
  const std::string header =
      "{\"__metadata__\":{\"format\":\"indecis\"},"
      "\"a\":{\"dtype\":\"F32\",\"shape\":[2,3],\"data_offsets\":[0,24]},"
      "\"b\":{\"dtype\":\"BF16\",\"shape\":[4],\"data_offsets\":[24,32]},"
      "\"c\":{\"dtype\":\"I8\",\"shape\":[3],\"data_offsets\":[32,35]}}";
  std::string data;
  const float a[6] = {1.f, -2.f, 3.5f, 0.f, 1e-3f, -7.f};
  data.append((const char *)a, sizeof a);
  const uint16_t b[4] = {0x3F80, 0xC040, 0x0000, 0x8000};
  data.append((const char *)b, sizeof b);
  data += (char)5;
  data += (char)-3;
  data += (char)127;
  std::string file;
  put_u64(file, header.size());
  file += header + data;
  const std::string path = dir + "/host_check.safetensors";
  CHECK(write_file(path, file), "write %s", path.c_str());
  std::vector<float> v;
  CHECK(read_tensor(path, "a", v) == 0 && v[1] == -2.f && v[5] == -7.f, "valid a: %s", ixh_last_error());
  CHECK(read_tensor(path, "b", v) == 0 && v[0] == 1.f && v[1] == -3.f, "valid b: %s", ixh_last_error());
  CHECK(read_tensor(path, "c", v) == 0 && v[1] == -3.f && v[2] == 127.f, "valid c: %s", ixh_last_error());
  // every truncation: an error, never a read past the end
  for (size_t cut = 0; cut < file.size(); cut++) {
    write_file(path, file.substr(0, cut));
    const int rc = read_tensor(path, "a", v);
    CHECK(rc != 0, "truncated at %zu read", cut);
  }
  // random corruptions of the header bytes: any result, no crash
  std::mt19937 rng(11);
  int ok = 0;
  for (int it = 0; it < 2000; it++) {
    std::string bad = file;
    const int flips = 1 + (int)(rng() % 4);
    for (int f = 0; f < flips; f++) bad[8 + rng() % header.size()] = (char)(rng() & 0xff);
    write_file(path, bad);
    for (const char *name : {"a", "b", "c"}) ok += read_tensor(path, name, v) == 0;
  }
  fprintf(stderr, "host_check: %d of 6000 corrupted reads still parsed\n", ok);
  // hand-made malformed headers
  const char *headers[] = {
      "", "{", "}", "[]", "{\"a\":", "{\"a\":{}}", "{\"a\":{\"dtype\":\"F32\"}}",
      "{\"a\":{\"dtype\":\"F32\",\"shape\":[2,3],\"data_offsets\":[24,0]}}",
      "{\"a\":{\"dtype\":\"F32\",\"shape\":[2,3],\"data_offsets\":[0,2400]}}",
      "{\"a\":{\"dtype\":\"F32\",\"shape\":[-2,3],\"data_offsets\":[0,24]}}",
      "{\"a\":{\"dtype\":\"F32\",\"shape\":[4611686018427387904,4],\"data_offsets\":[0,24]}}",
      "{\"a\":{\"dtype\":\"Q9\",\"shape\":[6],\"data_offsets\":[0,24]}}",
      "{\"a\":{\"dtype\":\"F32\",\"shape\":[6],\"data_offsets\":[0,24]}",
      "{\"\\u12",
      "{\"a\":{\"dtype\":\"F32\",\"shape\":[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[[6]]]]]]"
      "]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]]],\"data_offsets\":[0,24]}}",
  };
  for (const char *h : headers) {
    std::string bad;
    put_u64(bad, strlen(h));
    bad += h;
    bad += data;
    write_file(path, bad);
    CHECK(read_tensor(path, "a", v) != 0, "malformed header accepted: %s", h);
  }
  {
    // a name given twice: accepted, as Go's json.Unmarshal into a map
    // accepts it (safetensors.go:125-128, the later entry kept)
    const char *h = "{\"a\":{\"dtype\":\"F32\",\"shape\":[6],\"data_offsets\":[0,24]},"
                    "\"a\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,8]}}";
    std::string dup;
    put_u64(dup, strlen(h));
    dup += h;
    dup += data;
    write_file(path, dup);
    CHECK(read_tensor(path, "a", v) == 0 && v.size() == 3, "duplicate name: %s", ixh_last_error());
  }
  std::string huge;
  put_u64(huge, ~0ull);
  huge += "{}";
  write_file(path, huge);
  CHECK(read_tensor(path, "a", v) != 0, "header length 2^64-1 accepted");
  CHECK(ixh_safetensors_tensor((dir + "/absent.safetensors").c_str(), "a", nullptr, 0, nullptr) != 0,
        "absent file accepted");
  remove(path.c_str());
}

static void check_normalize() {
  std::mt19937 rng(3);
  std::normal_distribution<float> nd;
  for (int H : {1, 7, 768}) {
    std::vector<float> rows(5 * H);
    for (auto &x : rows) x = nd(rng);
    for (int k = 0; k < H; k++) rows[2 * H + k] = 0.f;  // a zero row
    CHECK(ixh_embed_normalize(rows.data(), 5, H) == 0, "normalize H=%d", H);
  }
}

int main(int argc, char **argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: host_check <tokenizer.json> <scratch dir>\n");
    return 2;
  }
  check_tokenizer(argv[1]);
  check_safetensors(argv[2]);
  check_normalize();
  if (failures) {
    fprintf(stderr, "host_check: %d checks failed\n", failures);
    return 1;
  }
  fprintf(stderr, "host_check: ok\n");
  return 0;
}
