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
//  3. ixh_embed_normalize on random rows;
//  4. host_sched.cpp: every option value through set_tuning/get_tuning;
//     pass planning and stream parts over random ragged batches (empty
//     sequences, pass boundaries, the token cap of wide models), with each
//     pass's outputs written through Outputs::at into exact-size buffers;
//     the workspace free list on 8 threads; the serving batcher's queue
//     driven by 8 client threads with a stub encode (merged batches, errors
//     handed to every request of a batch, close).
// Usage: host_check <tokenizer.json> <scratch dir>. Exit status 0 when
// every check holds (a sanitizer report aborts with a nonzero status).
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "../../include/indecis_hip.h"
#include "../../indecis_amd/csrc/host_sched.h"

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

static void check_options() {
  struct Opt {
    int id;
    int lo, hi;          // accepted range
    bool packb8;         // a PackedB8 handle takes it too
    int ixh::Tuning::*field;
  };
  const Opt opts[] = {
      {IXH_OPT_PARTS, 0, 4, false, &ixh::Tuning::parts},
      {IXH_OPT_PASS_TOKENS, 1, ixh::kMaxPassTokensOpt, false, &ixh::Tuning::pass_tokens},
      {IXH_OPT_QKV_FUSED, 0, 1, false, &ixh::Tuning::qkv_fused},
      {IXH_OPT_QKV_HEADS, 1, 2, false, &ixh::Tuning::qkv_heads},
      {IXH_OPT_GEMM, 0, 2, true, &ixh::Tuning::gemm},
      {IXH_OPT_GEMM_TILE, 0, 2, true, &ixh::Tuning::gemm_tile},
      {IXH_OPT_LN_SEG, 0, 1, false, &ixh::Tuning::ln_seg},
      {IXH_OPT_FUSE_RES, 0, 4, false, &ixh::Tuning::fuse_res},
      {IXH_OPT_FUSE_MLP, 0, 2, false, &ixh::Tuning::fuse_mlp},
      {IXH_OPT_QKV_KBLOCK, 0, 1, false, &ixh::Tuning::qkv_kblock},
  };
  for (const Opt &o : opts) {
    for (int64_t v : {(int64_t)o.lo - 1, (int64_t)o.lo, (int64_t)o.lo + 1, (int64_t)o.hi - 1, (int64_t)o.hi,
                      (int64_t)o.hi + 1, (int64_t)1 << 40, -((int64_t)1 << 40)}) {
      for (bool model : {true, false}) {
        ixh::Tuning t;
        const int before = t.*o.field;
        const int rc = ixh::set_tuning(t, o.id, v, model);
        const bool want = v >= o.lo && v <= o.hi && (model || o.packb8);
        CHECK((rc == 0) == want, "option %d value %lld model %d: rc %d", o.id, (long long)v, model, rc);
        int64_t got = -1;
        CHECK(ixh::get_tuning(t, o.id, &got) == 0, "get option %d", o.id);
        CHECK(got == (want ? v : before), "option %d value %lld read back %lld", o.id, (long long)v,
              (long long)got);
        if (!want) CHECK(strlen(ixh_last_error()) > 0, "option %d: no error text", o.id);
      }
    }
  }
  ixh::Tuning t;
  int64_t v = 0;
  CHECK(ixh::set_tuning(t, 999, 0, true) == IXH_EINVAL, "unknown option accepted");
  CHECK(ixh::get_tuning(t, 999, &v) == IXH_EINVAL, "unknown option read");
}

// Sequence lengths with runs of empty sequences and a few long ones.
static std::vector<int32_t> ragged_offs(std::mt19937 &rng, int B, int maxlen) {
  std::vector<int32_t> offs(B + 1, 0);
  for (int b = 0; b < B; b++) {
    const int kind = (int)(rng() % 8);
    const int n = kind < 2 ? 0 : kind == 7 ? (int)(rng() % (4 * maxlen + 1)) : (int)(rng() % (maxlen + 1));
    offs[b + 1] = offs[b] + n;
  }
  return offs;
}

static void check_passes() {
  // the token cap: N * max(3H, I) * 4 bytes under 2^31, at most the option's bound
  struct Shape {
    int H, I, want;
  };
  for (const Shape &s : {Shape{768, 1152, ixh::kMaxPassTokensOpt}, Shape{256, 512, ixh::kMaxPassTokensOpt},
                         Shape{384, 1152, ixh::kMaxPassTokensOpt}, Shape{2048, 5632, 87381},
                         Shape{1024, 16384, 32767}, Shape{1 << 20, 64, 170}}) {
    const int cap = ixh::pass_token_cap(s.H, s.I);
    const int64_t per = 4 * (int64_t)std::max(3 * s.H, s.I);
    CHECK(cap == s.want, "cap H %d I %d: %d, want %d", s.H, s.I, cap, s.want);
    CHECK((int64_t)cap * per < ((int64_t)1 << 31), "cap H %d I %d: %lld bytes", s.H, s.I, (long long)cap * per);
    if (cap < ixh::kMaxPassTokensOpt)
      CHECK((int64_t)(cap + 1) * per >= ((int64_t)1 << 31), "cap H %d I %d not the largest", s.H, s.I);
  }
  // check_offs
  {
    const int32_t good[4] = {0, 3, 3, 9}, first[3] = {1, 2, 3}, down[4] = {0, 4, 2, 9};
    CHECK(ixh::check_offs(good, 3) == 0, "good offsets refused");
    CHECK(ixh::check_offs(nullptr, 0) == 0, "empty batch refused");
    CHECK(ixh::check_offs(nullptr, 2) == IXH_EINVAL, "null offsets accepted");
    CHECK(ixh::check_offs(good, -1) == IXH_EINVAL, "negative batch accepted");
    CHECK(ixh::check_offs(first, 2) == IXH_EINVAL, "offs[0] != 0 accepted");
    CHECK(ixh::check_offs(down, 3) == IXH_EINVAL, "decreasing offsets accepted");
  }
  // passes of random ragged batches, outputs written through Outputs::at
  std::mt19937 rng(5);
  const int H = 3, rp = 2, rt = 5;
  for (int it = 0; it < 400; it++) {
    const int B = (int)(rng() % 60);
    std::vector<int32_t> offs = ragged_offs(rng, B, 40);
    const int N = offs[B];
    ixh::Tuning t;
    const int choices[] = {1, 2, 7, 40, 100, 1000, ixh::kMaxPassTokensOpt};
    t.pass_tokens = choices[rng() % 7];
    std::vector<int> cut;
    CHECK(ixh::plan_passes(t, 768, 1152, offs.data(), B, cut) == 0, "plan: %s", ixh_last_error());
    CHECK(cut.size() >= 2 && cut.front() == 0 && cut.back() == B, "plan ends (B %d)", B);
    for (size_t i = 0; i + 1 < cut.size(); i++) {
      const int b0 = cut[i], b1 = cut[i + 1];
      CHECK(b1 > b0 || (B == 0 && b1 == b0), "empty pass %d..%d", b0, b1);
      const int n = offs[b1] - offs[b0];
      CHECK(n <= t.pass_tokens || b1 - b0 == 1, "pass %d..%d of %d tokens over %d", b0, b1, n, t.pass_tokens);
      if (b1 < B)  // greedy: the next sequence did not fit
        CHECK(offs[b1 + 1] - offs[b0] > t.pass_tokens, "pass %d..%d cut early", b0, b1);
    }
    ixh::Outputs out;
    std::vector<float> states((size_t)N * H), pooled((size_t)B * H);
    std::vector<double> zp((size_t)B * rp), zt((size_t)N * rt);
    out.states = states.data();
    out.pooled = pooled.data();
    out.zp = zp.data();
    out.zt = zt.data();
    for (size_t i = 0; i + 1 < cut.size(); i++) {
      const int b0 = cut[i], b1 = cut[i + 1], t0 = offs[b0], n = offs[b1] - t0;
      const ixh::Outputs o = out.at(b0, t0, H, rp, rt);
      for (int k = 0; k < n * H; k++) o.states[k] += 1.f;
      for (int k = 0; k < (b1 - b0) * H; k++) o.pooled[k] += 1.f;
      for (int k = 0; k < (b1 - b0) * rp; k++) o.zp[k] += 1.0;
      for (int k = 0; k < n * rt; k++) o.zt[k] += 1.0;
    }
    bool once = true;
    for (float x : states) once &= x == 1.f;
    for (float x : pooled) once &= x == 1.f;
    for (double x : zp) once &= x == 1.0;
    for (double x : zt) once &= x == 1.0;
    CHECK(once, "passes' outputs not covered exactly once (B %d, pass_tokens %d)", B, t.pass_tokens);
    // stream parts
    for (int P = 1; P <= 4; P++) {
      std::vector<int> parts;
      ixh::split_points(offs.data(), B, P, parts);
      CHECK((int)parts.size() == P + 1 && parts[0] == 0 && parts[P] == B, "parts ends P %d", P);
      for (int p = 1; p < P; p++) {
        CHECK(parts[p] >= parts[p - 1], "parts decrease");
        const int b = parts[p];
        CHECK(b == B || (int64_t)P * offs[b] >= (int64_t)p * N, "part %d starts early", p);
        CHECK(b == parts[p - 1] || (int64_t)P * offs[b - 1] < (int64_t)p * N, "part %d starts late", p);
      }
    }
  }
  // a sequence over a wide model's cap is refused; one at it is a pass of its own
  {
    ixh::Tuning t;
    const int cap = ixh::pass_token_cap(2048, 5632);
    const int32_t over[3] = {0, 5, 5 + cap + 1}, at[4] = {0, 5, 5 + cap, 6 + cap};
    std::vector<int> cut;
    CHECK(ixh::plan_passes(t, 2048, 5632, over, 2, cut) == IXH_EINVAL, "over-long sequence accepted");
    CHECK(strstr(ixh_last_error(), "87381") != nullptr, "limit text: %s", ixh_last_error());
    CHECK(ixh::plan_passes(t, 2048, 5632, at, 3, cut) == 0 && cut == std::vector<int>({0, 1, 2, 3}),
          "sequence at the cap");
    CHECK(ixh::plan_passes(t, 768, 1152, over, 2, cut) == 0 && cut == std::vector<int>({0, 2}),
          "narrow model passes");
  }
}

static void check_free_list() {
  struct Item {
    std::atomic<int> held{0};
  };
  ixh::FreeList<Item> pool;
  std::atomic<int> made{0}, twice{0};
  std::vector<std::thread> th;
  for (int w = 0; w < 8; w++)
    th.emplace_back([&]() {
      for (int i = 0; i < 3000; i++) {
        Item *a = pool.take();
        if (!a) {
          a = new Item;
          made++;
        }
        Item *b = i % 3 == 0 ? pool.take() : nullptr;
        if (a->held.exchange(1)) twice++;
        if (b && b->held.exchange(1)) twice++;
        a->held.store(0);
        pool.put(a);
        if (b) {
          b->held.store(0);
          pool.put(b);
        }
      }
    });
  for (auto &x : th) x.join();
  std::vector<Item *> all = pool.drain();
  CHECK(twice.load() == 0, "free list handed an item out twice (%d)", twice.load());
  CHECK((int)all.size() == made.load(), "free list kept %zu of %d items", all.size(), made.load());
  for (Item *p : all) delete p;
  CHECK(pool.take() == nullptr, "drained list not empty");
}

// The batcher's queue with a stub encode: a sequence's row is (length,
// sum of ids, first id, request tag); a batch with an id of -7 fails.
static void check_batcher() {
  const int W = 4;
  std::atomic<int> passes{0};
  auto encode = [&](const int32_t *ids, const int32_t *offs, int B, float *pooled, std::string &err) -> int {
    passes++;
    bool poisoned = false;
    if (offs[0] != 0) {
      err = "stub: offsets do not start at 0";
      return IXH_EINVAL;
    }
    for (int b = 0; b < B; b++) {
      const int n = offs[b + 1] - offs[b];
      if (n < 0) {
        err = "stub: decreasing offsets";
        return IXH_EINVAL;
      }
      float sum = 0;
      for (int k = offs[b]; k < offs[b + 1]; k++) {
        sum += (float)ids[k];
        poisoned |= ids[k] == -7;
      }
      pooled[(size_t)b * W + 0] = (float)n;
      pooled[(size_t)b * W + 1] = sum;
      pooled[(size_t)b * W + 2] = n ? (float)ids[offs[b]] : -1.f;
      pooled[(size_t)b * W + 3] = n ? (float)ids[offs[b + 1] - 1] : -1.f;
    }
    std::this_thread::sleep_for(std::chrono::microseconds(200));
    if (poisoned) {
      err = "stub: poisoned batch";
      return IXH_EHIP;
    }
    return 0;
  };
  for (int workers : {1, 3}) {
    for (int max_rows : {1, 50, 65536}) {
      for (bool poison : {false, true}) {
        ixh::BatchQueue q(W, workers, max_rows, encode);
        std::atomic<int> bad{0}, submitted{0}, failed{0}, with_tokens{0};
        std::vector<std::thread> th;
        for (int c = 0; c < 8; c++)
          th.emplace_back([&, c]() {
            std::mt19937 rng(100 + c);
            for (int r = 0; r < 60; r++) {
              const int B = 1 + (int)(rng() % 5);
              std::vector<int32_t> offs = ragged_offs(rng, B, 12);
              std::vector<int32_t> ids(offs[B]);
              for (auto &x : ids) x = (int32_t)(rng() % 1000);
              const bool mine = poison && offs[B] > 0 && rng() % 10 == 0;
              if (mine) ids[rng() % ids.size()] = -7;
              std::vector<float> out((size_t)B * W, -99.f);
              std::string err;
              submitted++;
              with_tokens += offs[B] > 0;
              const int rc = q.submit(ids.data(), offs.data(), B, out.data(), err);
              if (rc) {
                failed++;
                if (rc != IXH_EHIP || err != "stub: poisoned batch" || !poison) bad++;
                continue;
              }
              if (mine) bad++;  // its own poison must fail it
              for (int b = 0; b < B; b++) {
                const int n = offs[b + 1] - offs[b];
                float sum = 0;
                for (int k = offs[b]; k < offs[b + 1]; k++) sum += (float)ids[k];
                const float *row = &out[(size_t)b * W];
                if (row[0] != (float)n || row[1] != sum || row[2] != (n ? (float)ids[offs[b]] : -1.f) ||
                    row[3] != (n ? (float)ids[offs[b + 1] - 1] : -1.f))
                  bad++;
              }
            }
          });
        for (auto &x : th) x.join();
        int64_t batches = 0, requests = 0;
        q.counts(&batches, &requests);
        CHECK(bad.load() == 0, "batcher workers %d max_rows %d poison %d: %d bad results", workers, max_rows,
              poison, bad.load());
        CHECK(requests == submitted.load(), "batcher served %lld of %d requests", (long long)requests,
              submitted.load());
        CHECK(batches <= requests && batches >= 1, "batcher passes %lld", (long long)batches);
        // max_rows 1: a pass takes requests while it holds no token, so at
        // most one request with tokens (its last)
        if (max_rows == 1) CHECK(batches >= with_tokens.load(), "max_rows 1 merged requests with tokens");
        fprintf(stderr, "host_check: batcher workers %d max_rows %d poison %d: %lld requests in %lld passes, %d failed\n",
                workers, max_rows, poison, (long long)requests, (long long)batches, failed.load());
        q.close();
        const int32_t offs[2] = {0, 1}, ids[1] = {3};
        float out[W];
        std::string err;
        CHECK(q.submit(ids, offs, 1, out, err) == IXH_EINVAL && err == "modernbert: batcher closed",
              "closed batcher accepted a request");
      }
    }
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
  check_options();
  check_passes();
  check_free_list();
  check_batcher();
  if (failures) {
    fprintf(stderr, "host_check: %d checks failed\n", failures);
    return 1;
  }
  fprintf(stderr, "host_check: ok\n");
  return 0;
}
