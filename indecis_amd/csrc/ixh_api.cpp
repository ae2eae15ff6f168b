// ixh_api.cpp — the C ABI of include/indecis_hip.h: model state on the
// GPU, a pool of (stream, workspace) pairs, and the encoder forward pass of
// internal/modernbert.(*Model).run (infer.go:304-430) as a sequence of
// gfx950 kernels on one stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/indecis_hip.h"
#include "ixh_internal.h"

using namespace ixh;

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// A failed call also leaves its error as the thread's last error, which a
// later LAUNCHCK would report as the failure of an unrelated launch: it is
// taken back here.
#define HIPCK(call)                                                                      \
  do {                                                                                   \
    hipError_t e_ = (call);                                                              \
    if (e_ != hipSuccess) {                                                              \
      (void)hipGetLastError();                                                           \
      return fail(IXH_EHIP, "modernbert: hip: %s (%s)", hipGetErrorString(e_), #call);   \
    }                                                                                    \
  } while (0)
#define LAUNCHCK(what)                                                                   \
  do {                                                                                   \
    hipError_t e_ = hipGetLastError();                                                   \
    if (e_ != hipSuccess)                                                                \
      return fail(IXH_EHIP, "modernbert: hip: %s (launch %s)", hipGetErrorString(e_), what); \
  } while (0)

inline size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

// Device buffer that grows and never shrinks.
struct DevBuf {
  void *p = nullptr;
  size_t n = 0;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  int ensure(size_t bytes) {
    if (bytes <= n) return IXH_OK;
    if (p) HIPCK(hipFree(p));
    p = nullptr;
    n = 0;
    size_t want = round_up(std::max<size_t>(bytes, 256), 256);
    HIPCK(hipMalloc(&p, want));
    n = want;
    return IXH_OK;
  }
  template <class T> T *as() const { return (T *)p; }
};

struct PinBuf {
  void *p = nullptr;
  size_t n = 0;
  ~PinBuf() {
    if (p) (void)hipHostFree(p);
  }
  int ensure(size_t bytes) {
    if (bytes <= n) return IXH_OK;
    if (p) HIPCK(hipHostFree(p));
    p = nullptr;
    n = 0;
    size_t want = round_up(std::max<size_t>(bytes, 4096), 4096);
    HIPCK(hipHostMalloc(&p, want, hipHostMallocDefault));
    n = want;
    return IXH_OK;
  }
};

struct DeviceGuard {
  int prev = -1;
  hipError_t err = hipSuccess;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    err = hipSetDevice(dev);
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};
#define DEVGUARD(dev)                                                                    \
  DeviceGuard dg_(dev);                                                                  \
  if (dg_.err != hipSuccess)                                                             \
    return fail(IXH_EHIP, "modernbert: hip: %s (hipSetDevice %d)", hipGetErrorString(dg_.err), dev);

// A quantised weight matrix on the device, padded to the GEMM tiles:
// rows to a multiple of 256 (zero channels), depth to a multiple of 64.
// q holds it row-major [np][kp] (gemm_i8, the fused QKV kernel), qk the same
// bytes K-blocked [kp/32][np][32] (gemm_as: one MFMA operand is 1 KB).
struct Mat {
  int k = 0, n = 0, kp = 0, np = 0;
  bool set = false;
  // every row d has 127 * sum_k |w[d][k]| + |128 * colsum[d]| < 2^24: then
  // for any int8 activations the reference tile acc + 128*colsum is exact
  // in float32 and f32(tile) - zc equals f32(acc) (kernels that need it
  // dequantise as f32(acc) * sb * sa)
  bool small = false;
  DevBuf q, qk, sb, zc, c128;
};

// Rows [n][k] from either layout.
std::vector<int8_t> to_rows(const int8_t *q, int k, int n, int layout) {
  std::vector<int8_t> rows((size_t)n * k);
  if (layout == IXH_LAYOUT_ROWS) {
    memcpy(rows.data(), q, rows.size());
    return rows;
  }
  const int kq = (k + 3) / 4;
  for (int j = 0; j < n; j++)
    for (int t = 0; t < k; t++)
      rows[(size_t)j * k + t] = q[(size_t)(j / 16) * kq * 64 + (t / 4) * 64 + (j % 16) * 4 + t % 4];
  return rows;
}

// Uploads rows [n][k] + scales; perm (optional) gives the source row of
// each destination row (the GeGLU interleave).
int upload_mat(Mat &M, const std::vector<int8_t> &rows, const float *scale, int k, int n,
               const std::vector<int> *perm) {
  M.k = k;
  M.n = n;
  M.kp = (int)round_up(k, 64);
  M.np = (int)round_up(n, 256);
  std::vector<int8_t> q((size_t)M.np * M.kp, 0);
  std::vector<float> sb(M.np, 0.f), zc(M.np, 0.f);
  std::vector<int32_t> c128(M.np, 0);
  M.small = true;
  for (int d = 0; d < n; d++) {
    const int s = perm ? (*perm)[d] : d;
    int32_t colsum = 0;
    int64_t l1 = 0;
    for (int t = 0; t < k; t++) {
      const int8_t v = rows[(size_t)s * k + t];
      q[(size_t)d * M.kp + t] = v;
      colsum += v;
      l1 += v < 0 ? -v : v;
    }
    // |acc| <= 127 * l1 for activations in [-127, 127]
    if (127 * l1 + 128 * (int64_t)std::abs(colsum) >= (int64_t)1 << 24) M.small = false;
    sb[d] = scale[s];
    // PackB8: zc = 128*float32(colsum) (int8.go:72-75)
    zc[d] = 128.0f * (float)colsum;
    c128[d] = 128 * colsum;
  }
  std::vector<int8_t> qk(q.size());
  for (int d = 0; d < M.np; d++)
    for (int t = 0; t < M.kp; t++)
      qk[((size_t)(t / 32) * M.np + d) * 32 + t % 32] = q[(size_t)d * M.kp + t];
  int rc;
  if ((rc = M.q.ensure(q.size())) || (rc = M.qk.ensure(qk.size())) || (rc = M.sb.ensure(sb.size() * 4)) ||
      (rc = M.zc.ensure(zc.size() * 4)) || (rc = M.c128.ensure(c128.size() * 4)))
    return rc;
  HIPCK(hipMemcpy(M.q.p, q.data(), q.size(), hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(M.qk.p, qk.data(), qk.size(), hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(M.sb.p, sb.data(), sb.size() * 4, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(M.zc.p, zc.data(), zc.size() * 4, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(M.c128.p, c128.data(), c128.size() * 4, hipMemcpyHostToDevice));
  M.set = true;
  return IXH_OK;
}

// Interleave of the Wi rows for the GeGLU epilogue: destination chunk c of
// 64 rows = GELU-input rows 32c..32c+31, then gate rows I+32c..I+32c+31.
std::vector<int> geglu_perm(int I) {
  std::vector<int> p(2 * I);
  for (int d = 0; d < 2 * I; d++) {
    const int c = d / 64, w = d % 64;
    p[d] = w < 32 ? 32 * c + w : I + 32 * c + (w - 32);
  }
  return p;
}

// The GeGLU columns computed with the fused-multiply-add GELU: the AVX2
// prefix (multiple of 16) then whole SIMD vectors (vec_simd.go:138-156).
int gelu_fma_cols(int I, int lanes) {
  int i = I & ~15;
  if (lanes > 0)
    while (i + lanes <= I) i += lanes;
  return i;
}

// ropeFor (model.go:256-277): inv = f32(1/theta^(2i/D)), angle =
// f64(f32(p)*inv), cos/sin in float64 rounded to float32.
void rope_table(double theta, int D, int rows, std::vector<float> &c, std::vector<float> &s) {
  const int half = D / 2;
  c.assign((size_t)rows * half, 0.f);
  s.assign((size_t)rows * half, 0.f);
  for (int i = 0; i < half; i++) {
    const float inv = (float)(1.0 / std::pow(theta, (double)(2 * i) / (double)D));
    for (int p = 0; p < rows; p++) {
      const double f = (double)((float)p * inv);
      c[(size_t)p * half + i] = (float)std::cos(f);
      s[(size_t)p * half + i] = (float)std::sin(f);
    }
  }
}

struct RopeTab {
  int rows = 0;
  bool user = false;
  std::shared_ptr<DevBuf> cos_t, sin_t;
};

// Decision heads resident on the device (ixh_model_set_heads): the
// pooled-row heads' weight rows end to end, then the per-token heads'.
struct HeadSet {
  int rp = 0, rt = 0;     // rows of the pooled-row heads, of the per-token heads
  DevBuf wp, bp, wt, bt;  // [rows][H] weights widened to float64 (exact), [rows] float32 biases
};

struct Workspace {
  hipStream_t stream = nullptr;
  // tabs: the pass's small host-built tables, one copy: offs [B+1], padoff
  // [B+1], blocks [2 nblocks], sequence order [B]
  DevBuf ids, tabs, pos, x, xn, qkv, xq, xqk, sa, qq, sq, kp, ks, vt, vs, ctx, g, pooled, flag;
  DevBuf cmax, gmax;  // row maxima of ctx (per head) and g (per 32 columns)
  DevBuf out_states, out_pooled, out_zp, out_zt;  // host-path staging of a pass's outputs
  PinBuf host, flag_host;
  std::vector<hipEvent_t> events;  // profiling: begin/end pairs, reused
  hipEvent_t order[2] = {nullptr, nullptr};  // cross-stream ordering (no timing)
  ~Workspace() {
    for (hipEvent_t e : events) (void)hipEventDestroy(e);
    for (hipEvent_t e : order)
      if (e) (void)hipEventDestroy(e);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

struct StatAcc {
  std::string name;
  int64_t launches = 0;
  double ms = 0, ops = 0, bytes = 0;
};

}  // namespace

struct ixh_model {
  ixh_config cfg{};
  int device = 0;
  int D = 64;
  struct Layer {
    Mat qkv, o, i, omlp;
    DevBuf attn_norm, mlp_norm;
    bool attn_norm_set = false, mlp_norm_set = false;
  };
  std::vector<Layer> layers;
  DevBuf emb_norm, final_norm;
  bool emb_norm_set = false, final_norm_set = false;
  int emb_format = -1;
  DevBuf emb_table, emb_exact_slot, emb_exact_rows, emb_i8_scale;
  std::mutex rope_mu;
  RopeTab rope[2];  // 0 local, 1 global
  std::mutex heads_mu;
  std::shared_ptr<HeadSet> heads;  // null: none set
  std::vector<std::shared_ptr<DevBuf>> rope_graveyard;
  FreeList<Workspace> pool;
  std::atomic<bool> weights_valid{true};
  std::mutex tune_mu;
  Tuning tuning;
  std::atomic<bool> profiling{false};
  std::mutex prof_mu;
  std::string prof_only;  // profile only this kernel class (empty: all)
  std::vector<StatAcc> stats;
  ~ixh_model() {
    for (Workspace *w : pool.drain()) delete w;
  }
};

struct ixh_packed_b8 {
  int device = 0;
  Mat mat;
  std::vector<int8_t> rows;  // host copy, for the GeGLU interleave
  std::vector<float> scale;
  std::mutex mu;
  Mat geglu;
  bool geglu_set = false;
  Tuning tuning;  // gemm, gemm_tile (guarded by mu)
};

namespace {

int validate_config(const ixh_config &c) {
  if (c.hidden <= 0 || c.layers <= 0 || c.heads <= 0 || c.intermediate <= 0 || c.vocab <= 0)
    return fail(IXH_EINVAL, "modernbert: invalid dimensions");
  if (c.hidden % c.heads != 0 || (c.hidden / c.heads) % 2 != 0)
    return fail(IXH_EINVAL, "modernbert: hidden_size %d incompatible with %d heads", c.hidden,
                c.heads);
  if (c.global_every <= 0 || c.local_attention <= 0)
    return fail(IXH_EINVAL, "modernbert: invalid attention windows");
  if (c.hidden / c.heads != 64)
    return fail(IXH_EINVAL, "modernbert: hip: head dimension %d not supported (64)",
                c.hidden / c.heads);
  if (c.hidden % 64 != 0 || c.intermediate % 32 != 0)
    return fail(IXH_EINVAL, "modernbert: hip: hidden %% 64 and intermediate %% 32 required");
  if (c.lanes != 0 && c.lanes != 4 && c.lanes != 8 && c.lanes != 16)
    return fail(IXH_EINVAL, "modernbert: hip: lanes %d not in {0, 4, 8, 16}", c.lanes);
  if (c.pooling != IXH_POOL_MEAN && c.pooling != IXH_POOL_CLS)
    return fail(IXH_EINVAL, "modernbert: pooling %d not supported (mean or cls)", c.pooling);
  return IXH_OK;
}

int weights_ready(const ixh_model *m) {
  if (!m->weights_valid.load())
    return fail(IXH_ESTATE, "modernbert: weights invalidated and not set again");
  for (size_t l = 0; l < m->layers.size(); l++) {
    const auto &L = m->layers[l];
    if (!L.qkv.set || !L.o.set || !L.i.set || !L.omlp.set)
      return fail(IXH_ESTATE, "modernbert: layers.%zu matrices missing", l);
    if ((l > 0 && !L.attn_norm_set) || !L.mlp_norm_set)
      return fail(IXH_ESTATE, "modernbert: layers.%zu norm weights missing", l);
  }
  if (!m->emb_norm_set || !m->final_norm_set)
    return fail(IXH_ESTATE, "modernbert: embeddings.norm or final_norm missing");
  if (m->emb_format < 0) return fail(IXH_ESTATE, "modernbert: embedding table missing");
  return IXH_OK;
}

// Tables covering at least `rows` positions, returned as device pointers
// kept alive by `hold`. The library's own tables (the ropeFor formula with
// the C library's pow/cos/sin) grow to max(rows, 512) positions as ropeFor
// does (model.go:256-277). A caller's tables (ixh_model_set_rope: Go's own
// ropeFor output) are used as given and never replaced: a batch longer
// than they are fails, and the caller uploads ropeFor(theta, n) first.
int rope_for(ixh_model *m, int global, int rows, const float **c, const float **s,
             std::vector<std::shared_ptr<DevBuf>> &hold) {
  std::lock_guard<std::mutex> lk(m->rope_mu);
  RopeTab &t = m->rope[global];
  if (t.user && t.rows < rows)
    return fail(IXH_EINVAL,
                "modernbert: hip: the %s RoPE table set by ixh_model_set_rope has %d rows, the batch "
                "needs %d (upload ropeFor(theta, %d))",
                global ? "global" : "local", t.rows, rows, rows);
  if (t.rows < rows || !t.cos_t) {
    const int size = std::max(rows, 512);
    std::vector<float> hc, hs;
    rope_table(global ? m->cfg.global_theta : m->cfg.local_theta, m->D, size, hc, hs);
    auto nc = std::make_shared<DevBuf>(), ns = std::make_shared<DevBuf>();
    int rc;
    if ((rc = nc->ensure(hc.size() * 4)) || (rc = ns->ensure(hs.size() * 4))) return rc;
    HIPCK(hipMemcpy(nc->p, hc.data(), hc.size() * 4, hipMemcpyHostToDevice));
    HIPCK(hipMemcpy(ns->p, hs.data(), hs.size() * 4, hipMemcpyHostToDevice));
    t.cos_t = nc;
    t.sin_t = ns;
    t.rows = size;
    t.user = false;
  }
  hold.push_back(t.cos_t);
  hold.push_back(t.sin_t);
  *c = t.cos_t->as<float>();
  *s = t.sin_t->as<float>();
  return IXH_OK;
}

Workspace *acquire(ixh_model *m) {
  if (Workspace *w = m->pool.take()) return w;
  Workspace *w = new Workspace();
  if (hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking) != hipSuccess) {
    delete w;
    return nullptr;
  }
  return w;
}

void release(ixh_model *m, Workspace *w) {
  m->pool.put(w);
}

struct WsGuard {
  ixh_model *m;
  Workspace *w;
  ~WsGuard() {
    if (w) release(m, w);
  }
};

__global__ void fill_u32_kernel(uint32_t *p, uint32_t v, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = v;
}
// A fill kernel rather than hipMemsetAsync: the calls around it may be
// captured into a HIP graph by the caller.
void launch_fill_u32(void *p, uint32_t v, size_t n, hipStream_t st) {
  if (n == 0) return;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
  fill_u32_kernel<<<(unsigned)blocks, 256, 0, st>>>((uint32_t *)p, v, n);
}

__global__ void check_ids_kernel(const int32_t *ids, int N, int vocab, int *flag) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < N && (ids[t] < 0 || ids[t] >= vocab)) atomicMin(flag, t);
}

// Brackets launches with HIP events when the model profiles; after the
// stream is synchronised, flush() adds the durations to the model's sums.
struct Prof {
  ixh_model *m;
  Workspace *w;
  hipStream_t st;
  bool on;
  std::string only;  // bracket only launches of this class (empty: all)
  struct Rec {
    const char *name;
    int idx;
    double ops, bytes;
  };
  std::vector<Rec> recs;
  int used = 0;
  int err = IXH_OK;

  int begin(const char *name) {
    if (!on || err || (!only.empty() && only != name)) return -1;
    if ((int)w->events.size() < 2 * (used + 1)) {
      // timing-only events: no system-scope fence (cache writeback and
      // invalidation) on record; they are read after the stream is
      // synchronised
      hipEvent_t a, b;
      if (hipEventCreateWithFlags(&a, hipEventDisableSystemFence) != hipSuccess ||
          hipEventCreateWithFlags(&b, hipEventDisableSystemFence) != hipSuccess) {
        err = fail(IXH_EHIP, "modernbert: hip: event creation failed");
        return -1;
      }
      w->events.push_back(a);
      w->events.push_back(b);
    }
    if (hipEventRecord(w->events[2 * used], st) != hipSuccess) {
      err = fail(IXH_EHIP, "modernbert: hip: event record failed");
      return -1;
    }
    return used++;
  }
  void end(int idx, const char *name, double ops, double bytes) {
    if (idx < 0) return;
    if (hipEventRecord(w->events[2 * idx + 1], st) != hipSuccess) {
      err = fail(IXH_EHIP, "modernbert: hip: event record failed");
      return;
    }
    recs.push_back({name, idx, ops, bytes});
  }
  int flush() {
    if (!on || err) return err;
    std::lock_guard<std::mutex> lk(m->prof_mu);
    for (const Rec &r : recs) {
      float ms = 0.f;
      HIPCK(hipEventElapsedTime(&ms, w->events[2 * r.idx], w->events[2 * r.idx + 1]));
      StatAcc *s = nullptr;
      for (auto &x : m->stats)
        if (x.name == r.name) s = &x;
      if (!s) {
        m->stats.push_back(StatAcc{r.name});
        s = &m->stats.back();
      }
      s->launches++;
      s->ms += ms;
      s->ops += r.ops;
      s->bytes += r.bytes;
    }
    return IXH_OK;
  }
};

// GEMM dispatch (Tuning::gemm): the A-stationary kernel (gemm_as.hip) for
// Wi + GeGLU and the plain stores unless 1, gemm_i8 for the residual GEMMs
// Wo and WoMLP. 2 runs those on the warp-specialised kernel (gemm_ws.hip)
// instead: 2-3 us faster per launch on cfg4, but the kernels around it ran
// slower and the whole pass lost 0.5-1 ms, so it is not the default.
void run_gemm(int epi, const GemmArgs &g, const Tuning &t, hipStream_t st) {
  const bool as_epi = epi == EPI_GEGLU || epi == EPI_STORE || epi == EPI_TILE;
  const bool ws_epi = epi == EPI_ACCUM || epi == EPI_ACCUM_MLP;
  if (as_epi && t.gemm != 1 && launch_gemm_as(epi, g, st)) return;
  if (ws_epi && t.gemm == 2 && launch_gemm_ws(epi, g, st)) return;
  GemmArgs gi = g;
  gi.tile_cfg = t.gemm_tile;
  launch_gemm(epi, gi, st);
}

// Parts of a batch (from kSplitTokens tokens on): Tuning::parts when set,
// else two. With the MLP block as one kernel that fills a CU, three parts
// were 1.4% slower than two on cfg4 (24.66-24.73 against 24.32-24.38 ms a
// pass, one box) and four 2%; three were also slower on eight 8,192-token
// sequences (1-2%) and on cfg3's H 256 (8%).
int split_parts(const Tuning &t, int N, int B, int H) {
  (void)N;
  (void)B;
  (void)H;
  if (t.parts > 0) return std::min(t.parts, 4);
  return 2;
}

// What a forward pass issued but has not waited for: its profiling records
// and the RoPE tables its kernels read.
struct Pending {
  std::unique_ptr<Prof> prof;
  std::vector<std::shared_ptr<DevBuf>> hold;
};

// The forward pass. ids/out are device pointers here. With `defer` the
// launches are only issued: the caller synchronises the stream, then calls
// defer->prof->flush().
int forward(ixh_model *m, const Tuning &tune, const HeadSet *heads, Workspace *w, hipStream_t st,
            const int32_t *d_ids, const int32_t *offs, int B, const Outputs &out,
            Pending *defer = nullptr) {
  // an error left by a call outside this pass (the caller's, or one this
  // library already reported) is not this pass's launch failure
  (void)hipGetLastError();
  const ixh_config &c = m->cfg;
  const int H = c.hidden, I = c.intermediate, nh = c.heads, D = m->D;
  const int N = offs[B];
  const int KpH = (int)round_up(H, 64), KpI = (int)round_up(I, 64);
  const int ldq = std::max(KpH, KpI);
  int T = 0;
  std::vector<int32_t> padoff(B + 1, 0);
  std::vector<int32_t> blocks;
  for (int b = 0; b < B; b++) {
    const int n = offs[b + 1] - offs[b];
    T = std::max(T, n);
    padoff[b + 1] = padoff[b] + (int)round_up(n, kKeyPad);
    for (int q0 = 0; q0 < n; q0 += kAttnQBlock) {
      blocks.push_back(b);
      blocks.push_back(q0);
    }
  }
  const int Npad = padoff[B];
  const int nblocks = (int)blocks.size() / 2;
  // sequences longest first (the fused QKV + prologue kernel's work order)
  std::vector<int32_t> order(B);
  for (int b = 0; b < B; b++) order[b] = b;
  std::stable_sort(order.begin(), order.end(),
                   [&](int x, int y) { return offs[x + 1] - offs[x] > offs[y + 1] - offs[y]; });
  // qkv_fused 0: QKV GEMM and attention prologue as two kernels (tests, timing)
  const bool fused = T <= kQkvSeqMax && tune.qkv_fused != 0;
  // the residual GEMMs fused with quantizeA of their input and the next
  // LayerNorm + quantizeA (gemm_res.hip), where the shapes allow it
  const bool fuse_res = tune.fuse_res != 0 && gemm_res_supported(H, KpH, m->layers[0].o.np) &&
                        gemm_res_supported(H, KpI, m->layers[0].omlp.np);
  // streamed inputs (fuse_res 2: Wo's; 3: Wo's and WoMLP's): attention
  // writes max |ctx| per (row, head), the GeGLU epilogue on gemm_as max
  // |g| per (row, 32 columns); fuse_res 1 quantises whole rows into a panel
  const bool stream_ctx = fuse_res && (tune.fuse_res == 2 || tune.fuse_res == 3) && H == KpH;
  // fuse_res 4: Wo on the whole-row kernel of 8 waves (mlp_res.hip)
  const bool wo8 = fuse_res && tune.fuse_res == 4 && wo_res_supported(H, KpH, m->layers[0].o.np) &&
                   m->layers[0].o.qk.p;
  // the whole MLP block as one kernel, where the shapes allow it: 64 rows
  // a workgroup, transposed (mlp_block.hip; fuse_mlp 2), or 32 rows
  // (mlp_res.hip; fuse_mlp 1, with the fused Wo kernel). It takes the
  // quantised mlp_norm output of whichever Wo path ran.
  const bool mlp_common = m->layers[0].i.qk.p && m->layers[0].omlp.qk.p && gelu_fma_cols(I, c.lanes) == I;
  bool mats_small = true;  // the 64-row kernel dequantises as f32(acc) * sb * sa
  for (int l = 0; l < c.layers; l++) mats_small = mats_small && m->layers[l].i.small && m->layers[l].omlp.small;
  const bool mlp_block = mlp_common && tune.fuse_mlp == 2 && mats_small &&
                         mlp_block_supported(H, I, KpH, KpI, m->layers[0].i.np);
  const bool fuse_mlp = mlp_block || (mlp_common && fuse_res && tune.fuse_mlp != 0 &&
                                      mlp_res_supported(H, I, KpH, KpI, m->layers[0].i.np));
  // the fused QKV kernel's input rows K-blocked (the weight rows then stay
  // in LDS): written so by the embedding LayerNorm and by the MLP kernel of
  // each layer
  const bool kblock = fused && fuse_mlp && tune.qkv_kblock != 0 && qkv_kblock_supported(KpH) &&
                      m->layers[0].qkv.qk.p;

  int rc;
  const size_t ntab = 2 * (size_t)(B + 1) + blocks.size() + B;
  if ((rc = w->tabs.ensure(4 * ntab)) || (rc = w->pos.ensure(4 * (size_t)N)) ||
      (rc = w->x.ensure(4 * (size_t)N * H)) || (rc = w->xn.ensure(4 * (size_t)N * H)) ||
      (!fused && (rc = w->qkv.ensure(4 * (size_t)N * 3 * H))) || (rc = w->xq.ensure((size_t)N * ldq)) ||
      (kblock && (rc = w->xqk.ensure((size_t)N * KpH))) ||
      (rc = w->sa.ensure(4 * (size_t)N)) || (rc = w->qq.ensure((size_t)N * H)) ||
      (rc = w->sq.ensure(4 * (size_t)N * nh)) || (rc = w->kp.ensure((size_t)nh * Npad * D)) ||
      (rc = w->ks.ensure(4 * (size_t)nh * Npad)) || (rc = w->vt.ensure((size_t)nh * D * Npad)) ||
      (rc = w->vs.ensure(3 * 4 * (size_t)B * nh * D)) || (rc = w->ctx.ensure(4 * (size_t)N * H)) ||
      (!fuse_mlp && (rc = w->g.ensure(4 * (size_t)N * I))) ||
      (stream_ctx && (rc = w->cmax.ensure(4 * (size_t)N * nh))) ||
      (stream_ctx && (rc = w->gmax.ensure(4 * (size_t)N * (I / 32)))))
    return rc;

  // small host-built tables through pinned memory, one copy
  if ((rc = w->host.ensure(4 * ntab))) return rc;
  int32_t *hs = (int32_t *)w->host.p;
  memcpy(hs, offs, 4 * (B + 1));
  memcpy(hs + B + 1, padoff.data(), 4 * (B + 1));
  if (!blocks.empty()) memcpy(hs + 2 * (B + 1), blocks.data(), 4 * blocks.size());
  if (B > 0) memcpy(hs + 2 * (B + 1) + blocks.size(), order.data(), 4 * (size_t)B);
  HIPCK(hipMemcpyAsync(w->tabs.p, hs, 4 * ntab, hipMemcpyHostToDevice, st));
  const int32_t *d_offs = w->tabs.as<int32_t>(), *d_padoff = d_offs + B + 1,
                *d_blocks = d_offs + 2 * (B + 1), *d_order = d_blocks + blocks.size();

  Pending local;
  Pending &pend = defer ? *defer : local;
  std::vector<std::shared_ptr<DevBuf>> &hold = pend.hold;
  const float *rc_g, *rs_g, *rc_l, *rs_l;
  if ((rc = rope_for(m, 1, T, &rc_g, &rs_g, hold)) || (rc = rope_for(m, 0, T, &rc_l, &rs_l, hold)))
    return rc;

  pend.prof.reset(new Prof{m, w, st, m->profiling.load()});
  Prof &prof = *pend.prof;
  if (prof.on) {
    std::lock_guard<std::mutex> lk(m->prof_mu);
    prof.only = m->prof_only;
  }
#define RUN(name, ops, bytes, stmt)                                                      \
  do {                                                                                   \
    const int pi_ = prof.begin(name);                                                        \
    stmt;                                                                                \
    LAUNCHCK(name);                                                                      \
    prof.end(pi_, name, (double)(ops), (double)(bytes));                                 \
  } while (0)

  // a fused kernel that refuses its arguments (a shape or option the gates
  // above let through by mistake) fails the pass instead of leaving x
  // without its residual and LayerNorm
  auto refused = [&](const char *k) {
    return fail(IXH_EINVAL, "indecis: kernel %s refused this model's shapes (H %d, I %d)", k, H, I);
  };
  // algorithmic figures: valid (query, key) pairs of local and global layers
  double keys_local = 0, keys_global = 0;
  const int Wl = c.local_attention / 2;
  for (int b = 0; b < B; b++) {
    const double n = offs[b + 1] - offs[b];
    keys_global += n * n;
    // pairs with |i - j| <= Wl: the diagonal, then n - d pairs at each
    // distance d = 1 .. min(Wl, n - 1) on both sides
    const double d = n > 0 ? std::min<double>(Wl, n - 1) : 0;
    keys_local += n + 2 * (d * n - d * (d + 1) / 2);
  }
  const double dN = N, dH = H, dI = I;
  const double row_bytes = m->emb_format == 0 ? 4 * dH : m->emb_format == 1 ? 2 * dH : dH + 4;

  float *xn = out.states ? out.states : w->xn.as<float>();
  // a part of empty sequences only: zero pooled rows (and their logits)
  if (N > 0) {
  RUN("positions", 0, 8.0 * N,
      launch_positions(d_offs, d_padoff, B, w->pos.as<int32_t>(), nullptr, st));

  // embedding gather + embeddings.norm (infer.go:361-368) -> x; layer 0's
  // QKV reads x itself (no attn_norm, infer.go:384-389): quantise it here.
  RowArgs ra{};
  ra.M = N;
  ra.H = H;
  ra.ids = d_ids;
  ra.vocab = c.vocab;
  ra.emb_format = m->emb_format;
  ra.emb_f32 = m->emb_table.as<float>();
  ra.emb_bf16 = m->emb_table.as<uint16_t>();
  ra.exact_slot = m->emb_exact_slot.as<int32_t>();
  ra.exact_rows = m->emb_exact_rows.as<float>();
  ra.emb_i8 = m->emb_table.as<int8_t>();
  ra.emb_i8_scale = m->emb_i8_scale.as<float>();
  ra.gamma = m->emb_norm.as<float>();
  ra.eps = c.norm_eps;
  ra.lanes = c.lanes;
  ra.out = w->x.as<float>();
  ra.q = w->xq.as<int8_t>();
  ra.ldq = KpH;
  ra.sa = w->sa.as<float>();
  if (kblock) {  // layer 0's QKV input, K-blocked (nothing else reads these rows)
    ra.qk = w->xqk.as<int8_t>();
    ra.qk_rows = N;
  }
  ra.seg = tune.ln_seg;
  RUN("emb_ln_quant", 0, dN * (4 + row_bytes + 4 * dH + dH + 4), launch_rownorm(ra, st));

  auto gemm = [&](int epi, const Mat &M, int Kp, float *C, int ldc, int n_valid) {
    GemmArgs g{};
    g.A = w->xq.as<int8_t>();
    g.lda = Kp;
    g.B = M.q.as<int8_t>();
    g.ldb = M.kp;
    g.Bk = M.qk.as<int8_t>();
    g.M = N;
    g.Np = M.np;
    g.Kp = M.kp;
    g.sa = w->sa.as<float>();
    g.sb = M.sb.as<float>();
    g.zc = M.zc.as<float>();
    g.c128 = M.c128.as<int32_t>();
    g.C = C;
    g.ldc = ldc;
    g.n_valid = n_valid;
    g.lanes = c.lanes;
    g.n_gelu = gelu_fma_cols(I, c.lanes);
    g.tile_cfg = tune.gemm_tile;  // the tiled GEMM's tiles, wherever it runs
    g.small = M.small;
    return g;
  };
  // GEMM HBM bytes: activations int8 + scales, weights, output (read too
  // when accumulated)
  auto gemm_bytes = [&](double k, double n, double out_cols, bool acc) {
    return dN * (k + 4) + k * n + 12 * n + dN * out_cols * 4 * (acc ? 2 : 1);
  };

  AttnArgs aa{};
  aa.qkv = w->qkv.as<float>();
  aa.H = H;
  aa.nh = nh;
  aa.N = N;
  aa.offs = d_offs;
  aa.padoff = d_padoff;
  aa.B = B;
  aa.max_n = 0;
  for (int b = 0; b < B; b++) aa.max_n = std::max(aa.max_n, offs[b + 1] - offs[b]);
  aa.scale = (float)(1.0 / std::sqrt((double)D));  // infer.go:445
  aa.lanes = c.lanes;
  aa.qq = w->qq.as<int8_t>();
  aa.sq = w->sq.as<float>();
  aa.kp = w->kp.as<int8_t>();
  aa.ks = w->ks.as<float>();
  aa.vt = w->vt.as<int8_t>();
  aa.vs = w->vs.as<float>();
  aa.kstat = aa.vs + (size_t)B * nh * D;
  aa.Npad = Npad;
  aa.blocks = d_blocks;
  aa.nblocks = nblocks;
  aa.ctx = w->ctx.as<float>();

  RowArgs ln{};
  ln.M = N;
  ln.H = H;
  ln.x = w->x.as<float>();
  ln.eps = c.norm_eps;
  ln.lanes = c.lanes;
  ln.q = w->xq.as<int8_t>();
  ln.ldq = KpH;
  ln.sa = w->sa.as<float>();
  ln.seg = tune.ln_seg;
  const double ln_bytes = dN * (4 * dH + dH + 4);

  float *const cmax = stream_ctx ? w->cmax.as<float>() : nullptr;
  aa.rmax = cmax;
  // the GeGLU maxima exist only where Wi runs on gemm_as (which writes them)
  float *gmax = nullptr;
  if (stream_ctx && tune.fuse_res == 3 && I == KpI && tune.gemm != 1 &&
      gemm_as_supported(gemm(EPI_GEGLU, m->layers[0].i, KpH, nullptr, I, I)))
    gmax = w->gmax.as<float>();
  auto res = [&](const Mat &M, const float *A, int K, const float *gamma, const float *amax, int P) {
    ResArgs r{};
    r.A = A;
    r.lda = K;
    r.K = K;
    r.amax = amax;
    r.P = P;
    r.Kp = M.kp;
    r.Bk = M.qk.as<int8_t>();
    r.Np = M.np;
    r.sb = M.sb.as<float>();
    r.zc = M.zc.as<float>();
    r.c128 = M.c128.as<int32_t>();
    r.X = w->x.as<float>();
    r.M = N;
    r.H = H;
    r.gamma = gamma;
    r.eps = c.norm_eps;
    r.Q = w->xq.as<int8_t>();
    r.ldq = KpH;
    r.SA = w->sa.as<float>();
    r.small = M.small;
    return r;
  };
  // bytes of a fused residual GEMM: input rows f32, weights, x read and
  // written, the quantised LayerNorm output
  auto res_bytes = [&](double k, bool ln_out) {
    return dN * 4 * k + k * dH + 12 * dH + dN * 8 * dH + (ln_out ? dN * (dH + 4) : 0);
  };
  bool ln_done = false;  // the attn_norm LayerNorm of this layer ran in the previous WoMLP
  for (int l = 0; l < c.layers; l++) {
    const auto &L = m->layers[l];
    const bool global = l % c.global_every == 0;  // Config.IsGlobal
    if (l > 0 && !ln_done) {
      ln.gamma = L.attn_norm.as<float>();
      RUN("ln_quant", 0, ln_bytes, launch_rownorm(ln, st));
    }
    ln_done = false;
    // QKV projection with RoPE on the queries and keys (infer.go:390-399)
    GemmArgs g = gemm(EPI_ROPE, L.qkv, KpH, w->qkv.as<float>(), 3 * H, 3 * H);
    g.rope_cos = global ? rc_g : rc_l;
    g.rope_sin = global ? rs_g : rs_l;
    g.pos = w->pos.as<int32_t>();
    g.rope_cols = 2 * H;
    g.q_cols = H;  // queries quantised per head in the epilogue
    g.qq = w->qq.as<int8_t>();
    g.sq = w->sq.as<float>();
    g.attn_scale = aa.scale;
    if (kblock) {
      g.Ak = w->xqk.as<int8_t>();
      g.ak_rows = N;
    }
    // attention (infer.go:437-518)
    aa.window = global ? -1 : c.local_attention / 2;
    if (fused) {
      // QKV GEMM and Attn8.Prepare in one kernel: int8 Q, K, V and their
      // scales are its only outputs
      RUN("gemm_qkv", 2 * dN * 3 * dH * dH,
          gemm_bytes(dH, 3 * dH, 0, false) + dN * (3 * dH + 8 * nh) + 4.0 * B * dH,
          launch_qkv_attn(g, aa, d_order, tune.qkv_heads, st));
    } else {
      RUN("gemm_qkv", 2 * dN * 3 * dH * dH,
          gemm_bytes(dH, 3 * dH, 2 * dH, false) + dN * (4 + dH + 4 * nh), launch_gemm(EPI_ROPE, g, st));
      RUN("attn_prologue", 0, dN * 2 * dH * 4 + dN * 2 * dH + 4 * dN * nh,
          launch_attn_prologue(aa, st));
    }
    const double pairs = global ? keys_global : keys_local;
    RUN(global ? "attn_global" : "attn_local", 4.0 * D * nh * pairs,
        dN * 3 * dH + 8 * dN * nh + dN * dH * 4, launch_attn_main(aa, st));
    // x += ctx . Wo^T (infer.go:403), then mlp_norm (infer.go:404-407)
    if (wo8) {
      MlpArgs wa{};
      wa.Af = w->ctx.as<float>();
      wa.lda = H;
      wa.Bo = L.o.qk.as<int8_t>();
      wa.sbo = L.o.sb.as<float>();
      wa.zco = L.o.zc.as<float>();
      wa.c128o = L.o.c128.as<int32_t>();
      wa.X = w->x.as<float>();
      wa.M = N;
      wa.H = H;
      wa.I = H;
      wa.gamma = L.mlp_norm.as<float>();
      wa.eps = c.norm_eps;
      wa.Q = w->xq.as<int8_t>();
      wa.ldq = KpH;
      wa.SA = w->sa.as<float>();
      RUN("gemm_wo_ln", 2 * dN * dH * dH, res_bytes(dH, true),
          if (!launch_wo_res(wa, c.lanes, st)) return refused("gemm_wo_ln"));
    } else if (fuse_res) {
      const ResArgs r = res(L.o, w->ctx.as<float>(), H, L.mlp_norm.as<float>(), cmax, nh);
      RUN("gemm_wo_ln", 2 * dN * dH * dH, res_bytes(dH, true),
          if (!launch_gemm_res(r, c.lanes, st)) return refused("gemm_wo_ln"));
    } else {
      RUN("quant_ctx", 0, dN * (4 * dH + dH + 4),
          launch_quant_rows(w->ctx.as<float>(), H, N, H, w->xq.as<int8_t>(), KpH, w->sa.as<float>(), st));
      g = gemm(EPI_ACCUM, L.o, KpH, w->x.as<float>(), H, H);
      RUN("gemm_wo", 2 * dN * dH * dH, gemm_bytes(dH, dH, dH, true), run_gemm(EPI_ACCUM, g, tune, st));
      ln.gamma = L.mlp_norm.as<float>();
      RUN("ln_quant", 0, ln_bytes, launch_rownorm(ln, st));
    }
    // Wi + GeGLU, x += g . WoMLP^T (infer.go:408-424)
    if (fuse_mlp) {
      // and the next layer's attn_norm, in one kernel
      const bool next = l + 1 < c.layers;
      MlpArgs ma{};
      ma.Aq = w->xq.as<int8_t>();
      ma.sa = w->sa.as<float>();
      ma.Bi = L.i.qk.as<int8_t>();
      ma.Npi = L.i.np;
      ma.sbi = L.i.sb.as<float>();
      ma.zci = L.i.zc.as<float>();
      ma.c128i = L.i.c128.as<int32_t>();
      ma.n_gelu = gelu_fma_cols(I, c.lanes);
      ma.Bo = L.omlp.qk.as<int8_t>();
      ma.Npo = L.omlp.np;
      ma.sbo = L.omlp.sb.as<float>();
      ma.zco = L.omlp.zc.as<float>();
      ma.c128o = L.omlp.c128.as<int32_t>();
      ma.X = w->x.as<float>();
      ma.M = N;
      ma.H = H;
      ma.I = I;
      ma.gamma = next ? m->layers[l + 1].attn_norm.as<float>() : nullptr;
      ma.eps = c.norm_eps;
      ma.Q = w->xq.as<int8_t>();
      ma.ldq = KpH;
      ma.SA = w->sa.as<float>();
      if (kblock && next) {
        ma.Qk = w->xqk.as<int8_t>();
        ma.qk_rows = N;
      }
      RUN("mlp_ln", 2 * dN * 2 * dI * dH + 2 * dN * dH * dI,
          dN * (dH + 4) + 3 * dI * dH + 12 * (2 * dI + dH) + dN * 8 * dH + (next ? dN * (dH + 4) : 0),
          if (!(mlp_block ? launch_mlp_block(ma, c.lanes, st) : launch_mlp_res(ma, c.lanes, st)))
            return refused("mlp_ln"));
      ln_done = next;
      continue;
    }
    g = gemm(EPI_GEGLU, L.i, KpH, w->g.as<float>(), I, I);
    g.rmax = gmax;
    g.rmax_ld = I / 32;
    RUN("gemm_wi", 2 * dN * 2 * dI * dH, gemm_bytes(dH, 2 * dI, dI, false),
        run_gemm(EPI_GEGLU, g, tune, st));
    if (fuse_res) {
      // and the next layer's attn_norm (the last layer's final_norm below
      // writes float32)
      const bool next = l + 1 < c.layers;
      const ResArgs r = res(L.omlp, w->g.as<float>(), I, next ? m->layers[l + 1].attn_norm.as<float>() : nullptr,
                            gmax, I / 32);
      RUN("gemm_womlp_ln", 2 * dN * dH * dI, res_bytes(dI, next),
          if (!launch_gemm_res(r, c.lanes, st)) return refused("gemm_womlp_ln"));
      ln_done = next;
    } else {
      RUN("quant_g", 0, dN * (4 * dI + dI + 4),
          launch_quant_rows(w->g.as<float>(), I, N, I, w->xq.as<int8_t>(), KpI, w->sa.as<float>(), st));
      g = gemm(EPI_ACCUM_MLP, L.omlp, KpI, w->x.as<float>(), H, H);
      RUN("gemm_womlp", 2 * dN * dH * dI, gemm_bytes(dI, dH, dH, true),
          run_gemm(EPI_ACCUM_MLP, g, tune, st));
    }
  }
  // final_norm (infer.go:427), then the token states, pooling (infer.go:
  // 265-287) and the heads' logits (heads.go:63-74) on the device
  {
    RowArgs r{};
    r.M = N;
    r.H = H;
    r.x = w->x.as<float>();
    r.gamma = m->final_norm.as<float>();
    r.eps = c.norm_eps;
    r.lanes = c.lanes;
    r.seg = tune.ln_seg;
    r.out = xn;
    RUN("final_norm", 0, dN * 8 * dH, launch_rownorm(r, st));
  }
  }  // N > 0
  float *pooled = out.pooled;
  if (!pooled && out.zp) {
    if ((rc = w->pooled.ensure(4 * (size_t)B * H))) return rc;
    pooled = w->pooled.as<float>();
  }
  if (pooled)
    RUN("pool", 0, dN * 4 * dH + (double)B * 4 * dH,
        launch_pool(xn, d_offs, B, N, H, c.pooling == IXH_POOL_CLS && !out.mean, pooled, st));
  if (out.zp && heads->rp > 0)
    RUN("head_pooled", 0, (double)B * (4 * dH + 8 * heads->rp),
        launch_head_logits(pooled, B, H, heads->wp.as<double>(), heads->bp.as<float>(), heads->rp, out.zp, st));
  if (out.zt && heads->rt > 0 && N > 0)
    RUN("head_tokens", 0, dN * (4 * dH + 8 * heads->rt),
        launch_head_logits(xn, N, H, heads->wt.as<double>(), heads->bt.as<float>(), heads->rt, out.zt, st));
#undef RUN
  if (defer) return prof.err;
  // tables used by queued work stay alive until the stream has run them
  HIPCK(hipStreamSynchronize(st));
  return prof.flush();
}

// Token count from which a batch is split over several streams.
constexpr int kSplitTokens = 4096;

// The batch as P parts of about equal token counts, each on its own stream
// (the caller's, then those of extra workspaces), issued back to back: the
// kernels of one part (say its GEMMs) share the CUs with those of another
// (its attention or row kernels), which are bound by other resources.
// Sequences are independent, so the results equal one pass's. Without
// extra workspaces (or for a small batch): one pass. Returns once st has
// run every part.
int forward_split(ixh_model *m, const Tuning &tune, const HeadSet *hs, Workspace *w,
                  Workspace *const *extra, int nextra, hipStream_t st, const int32_t *d_ids,
                  const int32_t *offs, int B, const Outputs &out) {
  const int N = offs[B];
  const int P = std::min(nextra + 1, B);
  if (P < 2 || N < kSplitTokens) return forward(m, tune, hs, w, st, d_ids, offs, B, out);
  // part p covers sequences [cut[p], cut[p+1]): the first starting at or
  // past p*N/P
  std::vector<int> cut;
  split_points(offs, B, P, cut);
  const int H = m->cfg.hidden;
  for (int k = 0; k < nextra; k++)
    for (int e = 0; e < 2; e++)
      if (!extra[k]->order[e]) HIPCK(hipEventCreateWithFlags(&extra[k]->order[e], hipEventDisableTiming));
  // every part follows the work queued on st so far (not the other parts;
  // delaying a part by some of the previous part's kernels gains nothing,
  // the parts drift apart by themselves)
  for (int p = 1; p < P; p++) {
    HIPCK(hipEventRecord(extra[p - 1]->order[0], st));
    HIPCK(hipStreamWaitEvent(extra[p - 1]->stream, extra[p - 1]->order[0], 0));
  }
  std::vector<Pending> pend(P);
  std::vector<std::vector<int32_t>> offp(P);
  int rc = IXH_OK;
  for (int p = 0; p < P; p++) {
    const int b0 = cut[p], b1 = cut[p + 1];
    if (b1 <= b0) continue;
    Workspace *wp = p == 0 ? w : extra[p - 1];
    hipStream_t sp = p == 0 ? st : wp->stream;
    offp[p].resize(b1 - b0 + 1);
    for (int b = b0; b <= b1; b++) offp[p][b - b0] = offs[b] - offs[b0];
    const int r = forward(m, tune, hs, wp, sp, d_ids + offs[b0], offp[p].data(), b1 - b0,
                          out.at(b0, offs[b0], H, hs->rp, hs->rt), &pend[p]);
    if (r && !rc) rc = r;
  }
  // st waits for every part whatever happened, so nothing is left queued
  for (int p = 1; p < P; p++) {
    HIPCK(hipEventRecord(extra[p - 1]->order[1], extra[p - 1]->stream));
    HIPCK(hipStreamWaitEvent(st, extra[p - 1]->order[1], 0));
  }
  HIPCK(hipStreamSynchronize(st));
  if (rc) return rc;
  for (int p = 0; p < P; p++)
    if (pend[p].prof && (rc = pend[p].prof->flush())) return rc;
  return IXH_OK;
}

// Extra workspaces for split passes, returned to the pool on scope exit.
struct ExtraWs {
  ixh_model *m;
  std::vector<Workspace *> ws;
  ExtraWs(ixh_model *model, const Tuning &t, int N, int B) : m(model) {
    const int want = N >= kSplitTokens ? split_parts(t, N, B, model->cfg.hidden) - 1 : 0;
    for (int k = 0; k < want; k++) {
      Workspace *w = acquire(m);
      if (!w) break;  // fewer parts
      ws.push_back(w);
    }
  }
  ~ExtraWs() {
    for (Workspace *w : ws) release(m, w);
  }
};

// The handle's tuning, copied once per call.
Tuning tuning_of(ixh_model *m) {
  std::lock_guard<std::mutex> lk(m->tune_mu);
  return m->tuning;
}

// The heads the call needs (an error when out asks for logits and none
// are set), kept alive by the returned pointer.
int heads_for(ixh_model *m, bool want, std::shared_ptr<HeadSet> &hs) {
  std::lock_guard<std::mutex> lk(m->heads_mu);
  hs = m->heads;
  if (want && !hs) return fail(IXH_ESTATE, "indecis: no heads set (ixh_model_set_heads)");
  if (!hs) hs = std::make_shared<HeadSet>();
  return IXH_OK;
}

// EncodeSeqs / EncodeTokens / the heads' logits from host ids into host
// outputs (what `out` points at is host memory here), pass by pass.
int encode_host(ixh_model *m, const int32_t *ids, const int32_t *offs, int B, const Outputs &out) {
  if (!m) return fail(IXH_EINVAL, "modernbert: nil model");
  int rc;
  if ((rc = check_offs(offs, B))) return rc;
  const int N = B ? offs[B] : 0;
  if (N > 0 && !ids) return fail(IXH_EINVAL, "modernbert: inconsistent batch");
  for (int t = 0; t < N; t++)
    if (ids[t] < 0 || ids[t] >= m->cfg.vocab)
      return fail(IXH_ERANGE, "modernbert: id %d out of vocabulary", ids[t]);
  std::shared_ptr<HeadSet> hsp;
  if ((rc = heads_for(m, out.zp || out.zt, hsp))) return rc;
  const HeadSet *hs = hsp.get();
  const int H = m->cfg.hidden;
  DEVGUARD(m->device);
  // empty sequences: zero pooled rows, whose logits are the biases (passes
  // overwrite the rows of the others)
  if (out.pooled && B > 0) memset(out.pooled, 0, sizeof(float) * (size_t)B * H);
  if (out.zp && hs->rp > 0 && B > 0) {
    std::vector<float> bp(hs->rp);
    HIPCK(hipMemcpy(bp.data(), hs->bp.p, 4 * (size_t)hs->rp, hipMemcpyDeviceToHost));
    for (int b = 0; b < B; b++)
      for (int r = 0; r < hs->rp; r++) out.zp[(size_t)b * hs->rp + r] = (double)bp[r];
  }
  if (N == 0) return IXH_OK;
  if ((rc = weights_ready(m))) return rc;
  const Tuning tune = tuning_of(m);
  std::vector<int> cut;
  if ((rc = plan_passes(tune, m->cfg.hidden, m->cfg.intermediate, offs, B, cut))) return rc;
  WsGuard wg{m, acquire(m)};
  Workspace *w = wg.w;
  if (!w) return fail(IXH_EHIP, "modernbert: hip: stream creation failed");
  int maxN = 0, maxB = 0;
  for (size_t i = 0; i + 1 < cut.size(); i++) {
    maxN = std::max(maxN, offs[cut[i + 1]] - offs[cut[i]]);
    maxB = std::max(maxB, cut[i + 1] - cut[i]);
  }
  ExtraWs ex(m, tune, maxN, maxB);
  hipStream_t st = w->stream;
  if ((rc = w->ids.ensure(4 * (size_t)maxN))) return rc;
  Outputs dev;
  dev.mean = out.mean;
  if (out.states) {
    if ((rc = w->out_states.ensure(4 * (size_t)maxN * H))) return rc;
    dev.states = w->out_states.as<float>();
  }
  if (out.pooled) {
    if ((rc = w->out_pooled.ensure(4 * (size_t)maxB * H))) return rc;
    dev.pooled = w->out_pooled.as<float>();
  }
  if (out.zp && hs->rp > 0) {
    if ((rc = w->out_zp.ensure(8 * (size_t)maxB * hs->rp))) return rc;
    dev.zp = w->out_zp.as<double>();
  }
  if (out.zt && hs->rt > 0) {
    if ((rc = w->out_zt.ensure(8 * (size_t)maxN * hs->rt))) return rc;
    dev.zt = w->out_zt.as<double>();
  }
  std::vector<int32_t> offp;
  for (size_t i = 0; i + 1 < cut.size(); i++) {
    const int b0 = cut[i], b1 = cut[i + 1], t0 = offs[b0], n = offs[b1] - t0;
    if (n == 0) continue;  // pooled rows and logits already set
    offp.resize(b1 - b0 + 1);
    for (int b = b0; b <= b1; b++) offp[b - b0] = offs[b] - t0;
    HIPCK(hipMemcpyAsync(w->ids.p, ids + t0, 4 * (size_t)n, hipMemcpyHostToDevice, st));
    if ((rc = forward_split(m, tune, hs, w, ex.ws.data(), (int)ex.ws.size(), st, w->ids.as<int32_t>(),
                            offp.data(), b1 - b0, dev)))
      return rc;
    const Outputs h = out.at(b0, t0, H, hs->rp, hs->rt);
    if (dev.states) HIPCK(hipMemcpyAsync(h.states, dev.states, 4 * (size_t)n * H, hipMemcpyDeviceToHost, st));
    if (dev.pooled)
      HIPCK(hipMemcpyAsync(h.pooled, dev.pooled, 4 * (size_t)(b1 - b0) * H, hipMemcpyDeviceToHost, st));
    if (dev.zp)
      HIPCK(hipMemcpyAsync(h.zp, dev.zp, 8 * (size_t)(b1 - b0) * hs->rp, hipMemcpyDeviceToHost, st));
    if (dev.zt) HIPCK(hipMemcpyAsync(h.zt, dev.zt, 8 * (size_t)n * hs->rt, hipMemcpyDeviceToHost, st));
    HIPCK(hipStreamSynchronize(st));
  }
  return IXH_OK;
}

}  // namespace

// ---- fixed scratch of the allocation-free MatMul8N (ixh_matmul8_noalloc) --
// The quantised activations and row scales of one call. Module memory: each
// GPU the library runs on holds its own copy until the process ends. Host
// code never takes the array's name as an address: scratch_ptr() resolves
// the device's copy once, with that device current.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) int8_t scratch[kNoAllocScratchBytes];

namespace {
// Per device ordinal: the scratch copy's address, and the event each call
// records after its work so that the next call's work waits for it; `order`
// keeps a call's wait, launches and record together against other threads.
struct NoAllocDev {
  std::mutex order;
  void *ptr = nullptr;
  hipEvent_t done = nullptr;
};
std::mutex g_scratch_mu;
NoAllocDev g_noalloc[64];

// With dev current: resolves the device's scratch copy and creates its
// event on first use (set-up; the entry point itself then allocates nothing).
int scratch_ptr(int dev, NoAllocDev **out) {
  if (dev < 0 || dev >= 64) return fail(IXH_EINVAL, "linalg: hip: device %d", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  NoAllocDev &d = g_noalloc[dev];
  if (!d.ptr) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(IXH_EHIP, "linalg: hip: %s (hipGetSymbolAddress scratch)", hipGetErrorString(e));
    hipEvent_t ev = nullptr;
    const hipError_t e2 = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e2 != hipSuccess) {
      (void)hipGetLastError();
      return fail(IXH_EHIP, "linalg: hip: %s (scratch event)", hipGetErrorString(e2));
    }
    d.done = ev;
    d.ptr = p;
  }
  *out = &d;
  return IXH_OK;
}
}  // namespace

namespace ixh {
int set_error(int code, const char *msg) {
  g_err = msg;
  return code;
}
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256;
  }
  std::atomic<int> &c = cache[dev & 63];
  int n = c.load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      n = 256;
    }
    c.store(n, std::memory_order_relaxed);
  }
  return n;
}
void model_config(const ixh_model *m, ixh_config *out) { *out = m->cfg; }
}  // namespace ixh

// ==== C ABI =================================================================
extern "C" {

const char *ixh_last_error(void) { return g_err.c_str(); }

int ixh_device_count(int *count) {
  if (!count) return fail(IXH_EINVAL, "ixh_device_count: nil");
  int n = 0;
  HIPCK(hipGetDeviceCount(&n));
  *count = n;
  return IXH_OK;
}

int ixh_model_create(const ixh_config *cfg, int device, ixh_model **out) {
  if (!cfg || !out) return fail(IXH_EINVAL, "modernbert: nil config");
  int rc;
  if ((rc = validate_config(*cfg))) return rc;
  int n = 0;
  HIPCK(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(IXH_EINVAL, "modernbert: hip: no device %d", device);
  auto *m = new ixh_model();
  m->cfg = *cfg;
  m->device = device;
  m->D = cfg->hidden / cfg->heads;
  m->layers.resize(cfg->layers);
  *out = m;
  return IXH_OK;
}

void ixh_model_destroy(ixh_model *m) {
  if (!m) return;
  DeviceGuard dg(m->device);
  delete m;
}

int ixh_model_set_matrix(ixh_model *m, int layer, int which, const int8_t *q, const float *scale,
                         int layout) {
  if (!m || !q || !scale) return fail(IXH_EINVAL, "modernbert: nil matrix");
  if (layer < 0 || layer >= m->cfg.layers)
    return fail(IXH_EINVAL, "modernbert: layer %d out of range", layer);
  if (layout != IXH_LAYOUT_ROWS && layout != IXH_LAYOUT_PANELS)
    return fail(IXH_EINVAL, "modernbert: layout %d", layout);
  const int H = m->cfg.hidden, I = m->cfg.intermediate;
  int k, n;
  Mat *M;
  auto &L = m->layers[layer];
  switch (which) {
  case IXH_MAT_QKV: k = H; n = 3 * H; M = &L.qkv; break;
  case IXH_MAT_O: k = H; n = H; M = &L.o; break;
  case IXH_MAT_I: k = H; n = 2 * I; M = &L.i; break;
  case IXH_MAT_OMLP: k = I; n = H; M = &L.omlp; break;
  default: return fail(IXH_EINVAL, "modernbert: matrix %d", which);
  }
  DEVGUARD(m->device);
  std::vector<int8_t> rows = to_rows(q, k, n, layout);
  std::vector<int> perm;
  if (which == IXH_MAT_I) perm = geglu_perm(I);
  return upload_mat(*M, rows, scale, k, n, which == IXH_MAT_I ? &perm : nullptr);
}

int ixh_model_set_norm(ixh_model *m, int which, int layer, const float *gamma) {
  if (!m || !gamma) return fail(IXH_EINVAL, "modernbert: nil norm");
  const int H = m->cfg.hidden;
  DevBuf *dst;
  bool *flag;
  switch (which) {
  case IXH_NORM_EMB: dst = &m->emb_norm; flag = &m->emb_norm_set; break;
  case IXH_NORM_FINAL: dst = &m->final_norm; flag = &m->final_norm_set; break;
  case IXH_NORM_ATTN:
  case IXH_NORM_MLP:
    if (layer < 0 || layer >= m->cfg.layers)
      return fail(IXH_EINVAL, "modernbert: layer %d out of range", layer);
    if (which == IXH_NORM_ATTN && layer == 0)
      return fail(IXH_EINVAL, "modernbert: layers.0 has no attn_norm");
    dst = which == IXH_NORM_ATTN ? &m->layers[layer].attn_norm : &m->layers[layer].mlp_norm;
    flag = which == IXH_NORM_ATTN ? &m->layers[layer].attn_norm_set : &m->layers[layer].mlp_norm_set;
    break;
  default: return fail(IXH_EINVAL, "modernbert: norm %d", which);
  }
  DEVGUARD(m->device);
  int rc;
  if ((rc = dst->ensure(4 * (size_t)H))) return rc;
  HIPCK(hipMemcpy(dst->p, gamma, 4 * (size_t)H, hipMemcpyHostToDevice));
  *flag = true;
  return IXH_OK;
}

int ixh_model_set_embeddings_f32(ixh_model *m, const float *table) {
  if (!m || !table) return fail(IXH_EINVAL, "modernbert: nil table");
  DEVGUARD(m->device);
  const size_t bytes = 4 * (size_t)m->cfg.vocab * m->cfg.hidden;
  int rc;
  if ((rc = m->emb_table.ensure(bytes))) return rc;
  HIPCK(hipMemcpy(m->emb_table.p, table, bytes, hipMemcpyHostToDevice));
  m->emb_format = 0;
  return IXH_OK;
}

int ixh_model_set_embeddings_bf16(ixh_model *m, const uint16_t *table, const int32_t *exact_ids,
                                  const float *exact_rows, int n_exact) {
  if (!m || !table || n_exact < 0 || (n_exact > 0 && (!exact_ids || !exact_rows)))
    return fail(IXH_EINVAL, "modernbert: nil table");
  const int V = m->cfg.vocab, H = m->cfg.hidden;
  std::vector<int32_t> slot(V, -1);
  for (int e = 0; e < n_exact; e++) {
    if (exact_ids[e] < 0 || exact_ids[e] >= V)
      return fail(IXH_EINVAL, "indecis: exact row %d out of vocabulary", exact_ids[e]);
    slot[exact_ids[e]] = e;  // embeddings.go:38-44: a later row wins
  }
  DEVGUARD(m->device);
  int rc;
  if ((rc = m->emb_table.ensure(2 * (size_t)V * H)) || (rc = m->emb_exact_slot.ensure(4 * (size_t)V)) ||
      (rc = m->emb_exact_rows.ensure(4 * (size_t)std::max(n_exact, 1) * H)))
    return rc;
  HIPCK(hipMemcpy(m->emb_table.p, table, 2 * (size_t)V * H, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(m->emb_exact_slot.p, slot.data(), 4 * (size_t)V, hipMemcpyHostToDevice));
  if (n_exact > 0)
    HIPCK(hipMemcpy(m->emb_exact_rows.p, exact_rows, 4 * (size_t)n_exact * H, hipMemcpyHostToDevice));
  m->emb_format = 1;
  return IXH_OK;
}

int ixh_model_set_embeddings_i8(ixh_model *m, const int8_t *table, const float *row_scale) {
  if (!m || !table || !row_scale) return fail(IXH_EINVAL, "modernbert: nil table");
  const int V = m->cfg.vocab, H = m->cfg.hidden;
  DEVGUARD(m->device);
  int rc;
  if ((rc = m->emb_table.ensure((size_t)V * H)) || (rc = m->emb_i8_scale.ensure(4 * (size_t)V)))
    return rc;
  HIPCK(hipMemcpy(m->emb_table.p, table, (size_t)V * H, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(m->emb_i8_scale.p, row_scale, 4 * (size_t)V, hipMemcpyHostToDevice));
  m->emb_format = 2;
  return IXH_OK;
}

int ixh_model_set_rope(ixh_model *m, int is_global, const float *cos_t, const float *sin_t,
                       int rows) {
  if (!m) return fail(IXH_EINVAL, "modernbert: nil model");
  if (!cos_t && !sin_t && rows == 0) {
    // back to the library's own tables
    std::lock_guard<std::mutex> lk(m->rope_mu);
    m->rope[is_global ? 1 : 0] = RopeTab{};
    return IXH_OK;
  }
  if (!cos_t || !sin_t || rows <= 0) return fail(IXH_EINVAL, "modernbert: nil rope table");
  DEVGUARD(m->device);
  const size_t bytes = 4 * (size_t)rows * (m->D / 2);
  auto nc = std::make_shared<DevBuf>(), ns = std::make_shared<DevBuf>();
  int rc;
  if ((rc = nc->ensure(bytes)) || (rc = ns->ensure(bytes))) return rc;
  HIPCK(hipMemcpy(nc->p, cos_t, bytes, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(ns->p, sin_t, bytes, hipMemcpyHostToDevice));
  std::lock_guard<std::mutex> lk(m->rope_mu);
  RopeTab &t = m->rope[is_global ? 1 : 0];
  t.cos_t = nc;
  t.sin_t = ns;
  t.rows = rows;
  t.user = true;
  return IXH_OK;
}

int ixh_model_invalidate(ixh_model *m) {
  if (!m) return fail(IXH_EINVAL, "modernbert: nil model");
  DEVGUARD(m->device);
  for (auto &L : m->layers) {
    L.qkv.set = L.o.set = L.i.set = L.omlp.set = false;
  }
  return IXH_OK;
}

int ixh_model_set_heads(ixh_model *m, int n, const int *rows, const int *per_token,
                        const float *const *w, const float *const *b) {
  if (!m || n < 0 || (n > 0 && (!rows || !per_token || !w || !b)))
    return fail(IXH_EINVAL, "indecis: heads: bad arguments");
  const int H = m->cfg.hidden;
  if (n == 0) {
    std::lock_guard<std::mutex> lk(m->heads_mu);
    m->heads.reset();
    return IXH_OK;
  }
  std::vector<double> wp, wt;
  std::vector<float> bp, bt;
  for (int h = 0; h < n; h++) {
    if (rows[h] <= 0 || !w[h] || !b[h]) return fail(IXH_EINVAL, "indecis: head %d: bad arguments", h);
    std::vector<double> &W = per_token[h] ? wt : wp;
    std::vector<float> &Bv = per_token[h] ? bt : bp;
    W.insert(W.end(), w[h], w[h] + (size_t)rows[h] * H);
    Bv.insert(Bv.end(), b[h], b[h] + rows[h]);
  }
  DEVGUARD(m->device);
  auto hs = std::make_shared<HeadSet>();
  hs->rp = (int)bp.size();
  hs->rt = (int)bt.size();
  int rc;
  if ((rc = hs->wp.ensure(8 * wp.size())) || (rc = hs->bp.ensure(4 * bp.size())) ||
      (rc = hs->wt.ensure(8 * wt.size())) || (rc = hs->bt.ensure(4 * bt.size())))
    return rc;
  if (!wp.empty()) {
    HIPCK(hipMemcpy(hs->wp.p, wp.data(), 8 * wp.size(), hipMemcpyHostToDevice));
    HIPCK(hipMemcpy(hs->bp.p, bp.data(), 4 * bp.size(), hipMemcpyHostToDevice));
  }
  if (!wt.empty()) {
    HIPCK(hipMemcpy(hs->wt.p, wt.data(), 8 * wt.size(), hipMemcpyHostToDevice));
    HIPCK(hipMemcpy(hs->bt.p, bt.data(), 4 * bt.size(), hipMemcpyHostToDevice));
  }
  std::lock_guard<std::mutex> lk(m->heads_mu);
  m->heads = hs;
  return IXH_OK;
}

int ixh_model_set_option(ixh_model *m, int option, int64_t value) {
  if (!m) return fail(IXH_EINVAL, "modernbert: nil model");
  std::lock_guard<std::mutex> lk(m->tune_mu);
  return set_tuning(m->tuning, option, value, true);
}

int ixh_model_get_option(ixh_model *m, int option, int64_t *value) {
  if (!m || !value) return fail(IXH_EINVAL, "modernbert: nil model");
  std::lock_guard<std::mutex> lk(m->tune_mu);
  return get_tuning(m->tuning, option, value);
}

int ixh_model_set_profiling(ixh_model *m, int on) {
  if (!m) return fail(IXH_EINVAL, "modernbert: nil model");
  std::lock_guard<std::mutex> lk(m->prof_mu);
  m->stats.clear();
  m->profiling.store(on != 0);
  return IXH_OK;
}

int ixh_model_set_profile_filter(ixh_model *m, const char *kernel_class) {
  if (!m) return fail(IXH_EINVAL, "modernbert: nil model");
  std::lock_guard<std::mutex> lk(m->prof_mu);
  m->stats.clear();
  m->prof_only = kernel_class ? kernel_class : "";
  return IXH_OK;
}

int ixh_model_profile(ixh_model *m, ixh_kernel_stat *out, int cap, int *n) {
  if (!m || !n || cap < 0 || (cap > 0 && !out)) return fail(IXH_EINVAL, "modernbert: bad arguments");
  std::lock_guard<std::mutex> lk(m->prof_mu);
  *n = (int)m->stats.size();
  for (int i = 0; i < cap && i < (int)m->stats.size(); i++) {
    const StatAcc &s = m->stats[i];
    memset(&out[i], 0, sizeof out[i]);
    snprintf(out[i].name, sizeof out[i].name, "%s", s.name.c_str());
    out[i].launches = s.launches;
    out[i].ms = s.ms;
    out[i].ops = s.ops;
    out[i].bytes = s.bytes;
  }
  return IXH_OK;
}

int ixh_encode_seqs(ixh_model *m, const int32_t *ids, const int32_t *offs, int B, float *out) {
  if (B > 0 && !out) return fail(IXH_EINVAL, "modernbert: nil output");
  Outputs o;
  o.pooled = out;
  return encode_host(m, ids, offs, B, o);
}

int ixh_encode_tokens(ixh_model *m, const int32_t *ids, const int32_t *offs, int B, float *out) {
  if (B > 0 && offs && offs[B] > 0 && !out) return fail(IXH_EINVAL, "modernbert: nil output");
  Outputs o;
  o.states = out;
  return encode_host(m, ids, offs, B, o);
}

int ixh_encode_heads(ixh_model *m, const int32_t *ids, const int32_t *offs, int B, int mean,
                     double *pooled_z, double *token_z) {
  if (!pooled_z && !token_z) return fail(IXH_EINVAL, "indecis: no output asked for");
  Outputs o;
  o.zp = pooled_z;
  o.zt = token_z;
  o.mean = mean != 0;
  return encode_host(m, ids, offs, B, o);
}

int ixh_encode_device(ixh_model *m, const int32_t *d_ids, const int32_t *offs, int B,
                      int out_kind, float *d_out, void *stream) {
  if (!m) return fail(IXH_EINVAL, "modernbert: nil model");
  if (out_kind != IXH_OUT_POOLED && out_kind != IXH_OUT_TOKENS)
    return fail(IXH_EINVAL, "modernbert: output kind %d", out_kind);
  int rc;
  if ((rc = check_offs(offs, B))) return rc;
  const int N = B ? offs[B] : 0;
  const int H = m->cfg.hidden;
  if (N > 0 && (rc = weights_ready(m))) return rc;
  const Tuning tune = tuning_of(m);
  std::vector<int> cut;
  if ((rc = plan_passes(tune, m->cfg.hidden, m->cfg.intermediate, offs, B, cut))) return rc;
  DEVGUARD(m->device);
  WsGuard wg{m, acquire(m)};
  Workspace *w = wg.w;
  if (!w) return fail(IXH_EHIP, "modernbert: hip: stream creation failed");
  hipStream_t st = stream ? (hipStream_t)stream : w->stream;
  const size_t out_elems = out_kind == IXH_OUT_TOKENS ? (size_t)N * H : (size_t)B * H;
  if (N == 0) {
    launch_fill_u32(d_out, 0u, out_elems, st);
    LAUNCHCK("fill");
    HIPCK(hipStreamSynchronize(st));
    return IXH_OK;
  }
  // ids on the device: checked by a kernel (infer.go:308-312) whose verdict
  // is read once the passes have run — no wait before them. The gather
  // clamps ids into the table, so a bad batch computes garbage that is
  // then discarded: d_out is zeroed and the reference's error returned.
  if ((rc = w->flag.ensure(4)) || (rc = w->flag_host.ensure(4))) return rc;
  const unsigned big = 0x7f7f7f7fu;  // larger than any index
  launch_fill_u32(w->flag.p, big, 1, st);
  check_ids_kernel<<<(N + 255) / 256, 256, 0, st>>>(d_ids, N, m->cfg.vocab, w->flag.as<int>());
  LAUNCHCK("check_ids");
  HIPCK(hipMemcpyAsync(w->flag_host.p, w->flag.p, 4, hipMemcpyDeviceToHost, st));
  int maxN = 0, maxB = 0;
  for (size_t i = 0; i + 1 < cut.size(); i++) {
    maxN = std::max(maxN, offs[cut[i + 1]] - offs[cut[i]]);
    maxB = std::max(maxB, cut[i + 1] - cut[i]);
  }
  ExtraWs ex(m, tune, maxN, maxB);
  HeadSet none;
  Outputs out;
  (out_kind == IXH_OUT_TOKENS ? out.states : out.pooled) = d_out;
  std::vector<int32_t> offp;
  for (size_t i = 0; i + 1 < cut.size() && !rc; i++) {
    const int b0 = cut[i], b1 = cut[i + 1], t0 = offs[b0], n = offs[b1] - t0;
    const Outputs o = out.at(b0, t0, H, 0, 0);
    if (n == 0) {
      if (o.pooled) {
        launch_fill_u32(o.pooled, 0u, (size_t)(b1 - b0) * H, st);
        LAUNCHCK("fill");
      }
      continue;
    }
    offp.resize(b1 - b0 + 1);
    for (int b = b0; b <= b1; b++) offp[b - b0] = offs[b] - t0;
    rc = forward_split(m, tune, &none, w, ex.ws.data(), (int)ex.ws.size(), st, d_ids + t0, offp.data(),
                       b1 - b0, o);
  }
  HIPCK(hipStreamSynchronize(st));  // the verdict has landed
  const unsigned bad = *(const unsigned *)w->flag_host.p;
  if (bad != big) {
    launch_fill_u32(d_out, 0u, out_elems, st);
    LAUNCHCK("fill");
    int32_t id = 0;
    HIPCK(hipMemcpyAsync(&id, d_ids + bad, 4, hipMemcpyDeviceToHost, st));
    HIPCK(hipStreamSynchronize(st));
    return fail(IXH_ERANGE, "modernbert: id %d out of vocabulary", id);
  }
  return rc;
}

int ixh_head_logits(ixh_model *m, const float *x, int T, const float *w, const float *b,
                    int rows, double *z) {
  if (!m || T < 0 || rows <= 0 || (T > 0 && (!x || !z)) || !w || !b)
    return fail(IXH_EINVAL, "indecis: head: bad arguments");
  if (T == 0) return IXH_OK;
  const int H = m->cfg.hidden;
  DEVGUARD(m->device);
  DevBuf dx, dw, db, dz;
  int rc;
  if ((rc = dx.ensure(4 * (size_t)T * H)) || (rc = dw.ensure(8 * (size_t)rows * H)) ||
      (rc = db.ensure(4 * (size_t)rows)) || (rc = dz.ensure(8 * (size_t)T * rows)))
    return rc;
  const std::vector<double> w64(w, w + (size_t)rows * H);  // widened: exact
  HIPCK(hipMemcpy(dx.p, x, 4 * (size_t)T * H, hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(dw.p, w64.data(), 8 * w64.size(), hipMemcpyHostToDevice));
  HIPCK(hipMemcpy(db.p, b, 4 * (size_t)rows, hipMemcpyHostToDevice));
  launch_head_logits(dx.as<float>(), T, H, dw.as<double>(), db.as<float>(), rows, dz.as<double>(), 0);
  LAUNCHCK("head_logits");
  HIPCK(hipDeviceSynchronize());
  HIPCK(hipMemcpy(z, dz.p, 8 * (size_t)T * rows, hipMemcpyDeviceToHost));
  return IXH_OK;
}

// ---- linalg -----------------------------------------------------------------

int ixh_packb8_create(int device, const int8_t *q, const float *scale, int k, int n, int layout,
                      ixh_packed_b8 **out) {
  if (!q || !scale || !out || k <= 0 || n <= 0) return fail(IXH_EINVAL, "linalg: PackB8: bad arguments");
  if (layout != IXH_LAYOUT_ROWS && layout != IXH_LAYOUT_PANELS)
    return fail(IXH_EINVAL, "linalg: PackB8: layout %d", layout);
  DEVGUARD(device);
  NoAllocDev *nd = nullptr;
  int src = scratch_ptr(device, &nd);  // set-up: resolve the device's scratch copy now
  if (src) return src;
  auto *b = new ixh_packed_b8();
  b->device = device;
  b->rows = to_rows(q, k, n, layout);
  b->scale.assign(scale, scale + n);
  int rc = upload_mat(b->mat, b->rows, scale, k, n, nullptr);
  if (rc) {
    delete b;
    return rc;
  }
  *out = b;
  return IXH_OK;
}

int ixh_packb8_set_option(ixh_packed_b8 *b, int option, int64_t value) {
  if (!b) return fail(IXH_EINVAL, "linalg: nil PackedB8");
  std::lock_guard<std::mutex> lk(b->mu);
  return set_tuning(b->tuning, option, value, false);
}

void ixh_packb8_destroy(ixh_packed_b8 *b) {
  if (!b) return;
  DeviceGuard dg(b->device);
  delete b;
}

namespace {
Tuning pb_tuning(ixh_packed_b8 *b) {
  std::lock_guard<std::mutex> lk(b->mu);
  return b->tuning;
}

// Uploads a [m][k] f32 with rows padded to ld = roundup(k, 4), quantises
// it into q [m][Kp] (zero padding) and sa [m] on stream st.
// Host rows a [m][k] into da [m][round_up(k, 4)] (zero padding).
int upload_rows(const float *a, int m, int k, DevBuf &da, hipStream_t st) {
  const int ld = (int)round_up(k, 4);
  int rc;
  if ((rc = da.ensure(4 * (size_t)m * ld))) return rc;
  if (ld == k) {
    HIPCK(hipMemcpyAsync(da.p, a, 4 * (size_t)m * k, hipMemcpyHostToDevice, st));
  } else {
    HIPCK(hipMemsetAsync(da.p, 0, 4 * (size_t)m * ld, st));
    HIPCK(hipMemcpy2DAsync(da.p, 4 * (size_t)ld, a, 4 * (size_t)k, 4 * (size_t)k, m,
                           hipMemcpyHostToDevice, st));
  }
  return IXH_OK;
}

// quantizeA of device rows da [m][round_up(k, 4)] into dq [m][Kp], dsa [m].
int quantize_dev(const DevBuf &da, int m, int k, int Kp, DevBuf &dq, DevBuf &dsa, hipStream_t st) {
  const int ld = (int)round_up(k, 4);
  int rc;
  if ((rc = dq.ensure((size_t)m * Kp)) || (rc = dsa.ensure(4 * (size_t)m))) return rc;
  launch_quant_rows(da.as<float>(), ld, m, ld, dq.as<int8_t>(), Kp, dsa.as<float>(), st);
  LAUNCHCK("quant_rows");
  return IXH_OK;
}

int quantize_upload(const float *a, int m, int k, int Kp, DevBuf &da, DevBuf &dq, DevBuf &dsa,
                    hipStream_t st) {
  int rc;
  if ((rc = upload_rows(a, m, k, da, st))) return rc;
  return quantize_dev(da, m, k, Kp, dq, dsa, st);
}

// The input channels MatMul8Outliers splits off (linalg/int8.go:281-316),
// from the column maxima of |A|: those above f32(ratio * mean), the mean a
// float32 sum in channel order divided by k; when more than 32 qualify, a
// selection of the first 32 places where a strictly larger maximum wins.
constexpr int kMaxOutliers = 32;  // maxOutliers, int8.go:271
std::vector<int> choose_outliers(const std::vector<float> &colmax, float ratio) {
  const int k = (int)colmax.size();
  float mean = 0.0f;
  for (int j = 0; j < k; j++) mean += colmax[j];
  mean /= (float)k;
  const float thr = ratio * mean;
  std::vector<int> out;
  for (int j = 0; j < k; j++)
    if (colmax[j] > thr) out.push_back(j);
  if ((int)out.size() > kMaxOutliers) {
    for (int i = 0; i < kMaxOutliers; i++) {
      int best = i;
      for (int x = i + 1; x < (int)out.size(); x++)
        if (colmax[out[x]] > colmax[out[best]]) best = x;
      std::swap(out[i], out[best]);
    }
    out.resize(kMaxOutliers);
  }
  return out;
}

struct TmpStream {
  hipStream_t s = nullptr;
  ~TmpStream() {
    if (s) (void)hipStreamDestroy(s);
  }
};
}  // namespace

int ixh_matmul8(ixh_packed_b8 *b, float *c, const float *a, int m, int accumulate) {
  if (!b || m < 0 || (m > 0 && (!c || !a))) return fail(IXH_EINVAL, "linalg: MatMul8: slice too short");
  if (m == 0) return IXH_OK;
  DEVGUARD(b->device);
  TmpStream ts;
  HIPCK(hipStreamCreateWithFlags(&ts.s, hipStreamNonBlocking));
  const Mat &M = b->mat;
  DevBuf da, dq, dsa, dc;
  int rc;
  if ((rc = quantize_upload(a, m, M.k, M.kp, da, dq, dsa, ts.s))) return rc;
  if ((rc = dc.ensure(4 * (size_t)m * M.n))) return rc;
  if (accumulate) HIPCK(hipMemcpyAsync(dc.p, c, 4 * (size_t)m * M.n, hipMemcpyHostToDevice, ts.s));
  GemmArgs g{};
  g.A = dq.as<int8_t>();
  g.lda = M.kp;
  g.B = M.q.as<int8_t>();
  g.ldb = M.kp;
  g.M = m;
  g.Np = M.np;
  g.Kp = M.kp;
  g.sa = dsa.as<float>();
  g.sb = M.sb.as<float>();
  g.zc = M.zc.as<float>();
  g.c128 = M.c128.as<int32_t>();
  g.C = dc.as<float>();
  g.ldc = M.n;
  g.n_valid = M.n;
  g.Bk = M.qk.as<int8_t>();
  run_gemm(accumulate ? EPI_ACCUM : EPI_STORE, g, pb_tuning(b), ts.s);
  LAUNCHCK("matmul8");
  HIPCK(hipMemcpyAsync(c, dc.p, 4 * (size_t)m * M.n, hipMemcpyDeviceToHost, ts.s));
  HIPCK(hipStreamSynchronize(ts.s));
  return IXH_OK;
}

int ixh_matmul8_noalloc(ixh_packed_b8 *b, float *d_c, int ldc, const float *d_a, int lda, int m,
                        int accumulate, void *stream) {
  if (!b || m < 0 || (m > 0 && (!d_c || !d_a))) return fail(IXH_EINVAL, "linalg: MatMul8: slice too short");
  const Mat &M = b->mat;
  if (M.k % 4 != 0 || lda < M.k || lda % 4 != 0 || ldc < M.n || ((uintptr_t)d_a & 15) ||
      ((uintptr_t)d_c & 15))
    return fail(IXH_EINVAL,
                "linalg: hip: MatMul8 without allocation needs k %% 4 == 0, lda >= k and a multiple of "
                "4, ldc >= n, 16-byte aligned buffers (k %d, n %d, lda %d, ldc %d)",
                M.k, M.n, lda, ldc);
  if (m == 0) return IXH_OK;
  const size_t qbytes = round_up((size_t)m * M.kp, 256);
  const size_t need = qbytes + 4 * (size_t)m;
  if (need > kNoAllocScratchBytes)
    return fail(IXH_EINVAL,
                "linalg: hip: MatMul8 without allocation: %d rows of depth %d need %zu bytes of "
                "scratch, over its %zu (at most %zu rows)",
                m, M.kp, need, kNoAllocScratchBytes, (kNoAllocScratchBytes - 256) / (M.kp + 4));
  DEVGUARD(b->device);
  NoAllocDev *nd = nullptr;
  int rc;
  if ((rc = scratch_ptr(b->device, &nd))) return rc;
  int8_t *dq = (int8_t *)nd->ptr;
  float *dsa = (float *)((char *)nd->ptr + qbytes);
  hipStream_t st = (hipStream_t)stream;
  // calls on this GPU run one after another whatever their streams: this
  // call's work waits for the previous call's event and records it after
  // its own (a stream under graph capture takes neither: the graph orders it)
  std::lock_guard<std::mutex> order(nd->order);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIPCK(hipStreamIsCapturing(st, &cap));
  const bool serial = cap == hipStreamCaptureStatusNone;
  if (serial) HIPCK(hipStreamWaitEvent(st, nd->done, 0));
  // quantizeA (int8.go:160-191) into the scratch: rows padded with zeros to Kp
  launch_quant_rows(d_a, lda, m, M.k, dq, M.kp, dsa, st);
  LAUNCHCK("quant_rows");
  GemmArgs g{};
  g.A = dq;
  g.lda = M.kp;
  g.B = M.q.as<int8_t>();
  g.ldb = M.kp;
  g.Bk = M.qk.as<int8_t>();
  g.M = m;
  g.Np = M.np;
  g.Kp = M.kp;
  g.sa = dsa;
  g.sb = M.sb.as<float>();
  g.zc = M.zc.as<float>();
  g.c128 = M.c128.as<int32_t>();
  g.C = d_c;
  g.ldc = ldc;
  g.n_valid = M.n;
  run_gemm(accumulate ? EPI_ACCUM : EPI_STORE, g, pb_tuning(b), st);
  LAUNCHCK("matmul8");
  if (serial) HIPCK(hipEventRecord(nd->done, st));
  return IXH_OK;
}

namespace {
// MatMul8N, optionally with MatMul8Outliers' split (ratio > 0) and a bias
// added after it (linear.apply): c[m][n] (+)= a . B (+ bias).
int matmul8_split(ixh_packed_b8 *b, float *c, const float *a, int m, int accumulate, float ratio,
                  const float *bias) {
  DEVGUARD(b->device);
  TmpStream ts;
  HIPCK(hipStreamCreateWithFlags(&ts.s, hipStreamNonBlocking));
  const Mat &M = b->mat;
  const int k = M.k, n = M.n, ld = (int)round_up(k, 4);
  DevBuf da, drest, dq, dsa, dc, dcm, dcols, dw, dbias;
  int rc;
  if ((rc = upload_rows(a, m, k, da, ts.s))) return rc;
  std::vector<int> cols;
  if (ratio > 0.f) {
    if ((rc = dcm.ensure(4 * (size_t)k))) return rc;
    HIPCK(hipMemsetAsync(dcm.p, 0, 4 * (size_t)k, ts.s));
    launch_colmax(da.as<float>(), ld, m, k, dcm.as<unsigned>(), ts.s);
    LAUNCHCK("colmax");
    std::vector<float> colmax(k);
    HIPCK(hipMemcpyAsync(colmax.data(), dcm.p, 4 * (size_t)k, hipMemcpyDeviceToHost, ts.s));
    HIPCK(hipStreamSynchronize(ts.s));
    cols = choose_outliers(colmax, ratio);
  }
  const int nc = (int)cols.size();
  if (nc > 0) {
    // the product runs on a copy of A without the chosen channels
    if ((rc = drest.ensure(4 * (size_t)m * ld)) || (rc = dcols.ensure(4 * (size_t)nc))) return rc;
    HIPCK(hipMemcpyAsync(drest.p, da.p, 4 * (size_t)m * ld, hipMemcpyDeviceToDevice, ts.s));
    HIPCK(hipMemcpyAsync(dcols.p, cols.data(), 4 * (size_t)nc, hipMemcpyHostToDevice, ts.s));
    launch_zero_cols(drest.as<float>(), ld, m, dcols.as<int>(), nc, ts.s);
    LAUNCHCK("zero_cols");
    if ((rc = quantize_dev(drest, m, k, M.kp, dq, dsa, ts.s))) return rc;
  } else if ((rc = quantize_dev(da, m, k, M.kp, dq, dsa, ts.s))) {
    return rc;
  }
  if ((rc = dc.ensure(4 * (size_t)m * n))) return rc;
  if (accumulate) HIPCK(hipMemcpyAsync(dc.p, c, 4 * (size_t)m * n, hipMemcpyHostToDevice, ts.s));
  GemmArgs g{};
  g.A = dq.as<int8_t>();
  g.lda = M.kp;
  g.B = M.q.as<int8_t>();
  g.ldb = M.kp;
  g.M = m;
  g.Np = M.np;
  g.Kp = M.kp;
  g.sa = dsa.as<float>();
  g.sb = M.sb.as<float>();
  g.zc = M.zc.as<float>();
  g.c128 = M.c128.as<int32_t>();
  g.C = dc.as<float>();
  g.ldc = n;
  g.n_valid = n;
  g.Bk = M.qk.as<int8_t>();
  run_gemm(accumulate ? EPI_ACCUM : EPI_STORE, g, pb_tuning(b), ts.s);
  LAUNCHCK("matmul8");
  std::vector<float> w;
  if (nc > 0 || bias) {
    // the split channels' dequantised weight rows: f32(q) * scale (int8.go:336-340)
    w.resize((size_t)std::max(nc, 1) * n);
    for (int t = 0; t < nc; t++)
      for (int col = 0; col < n; col++)
        w[(size_t)t * n + col] = (float)b->rows[(size_t)col * k + cols[t]] * b->scale[col];
    if ((rc = dw.ensure(4 * w.size()))) return rc;
    HIPCK(hipMemcpyAsync(dw.p, w.data(), 4 * w.size(), hipMemcpyHostToDevice, ts.s));
    if (bias) {
      if ((rc = dbias.ensure(4 * (size_t)n))) return rc;
      HIPCK(hipMemcpyAsync(dbias.p, bias, 4 * (size_t)n, hipMemcpyHostToDevice, ts.s));
    }
    launch_outlier_epilogue(dc.as<float>(), n, m, n, da.as<float>(), ld, nc ? dcols.as<int>() : nullptr, nc,
                            dw.as<float>(), bias ? dbias.as<float>() : nullptr, ts.s);
    LAUNCHCK("outlier_epilogue");
  }
  HIPCK(hipMemcpyAsync(c, dc.p, 4 * (size_t)m * n, hipMemcpyDeviceToHost, ts.s));
  HIPCK(hipStreamSynchronize(ts.s));  // w and cols outlive their copies
  return IXH_OK;
}

}  // namespace

int ixh_matmul8_outliers(ixh_packed_b8 *b, float *c, const float *a, int m, int accumulate,
                         float ratio) {
  if (!b || m < 0 || (m > 0 && (!c || !a)))
    return fail(IXH_EINVAL, "linalg: MatMul8Outliers: slice too short");
  if (m == 0 || b->mat.n == 0) return IXH_OK;
  if (!(ratio > 0.f)) return fail(IXH_EINVAL, "linalg: MatMul8Outliers: ratio %g", (double)ratio);
  return matmul8_split(b, c, a, m, accumulate, ratio, nullptr);
}

int ixh_linear8(ixh_packed_b8 *b, float *dst, const float *x, int rows, const float *bias,
                int outliers, float ratio) {
  if (!b || rows < 0 || (rows > 0 && (!dst || !x)))
    return fail(IXH_EINVAL, "siglip: linear: slice too short");
  if (rows == 0) return IXH_OK;
  if (outliers && !(ratio > 0.f)) return fail(IXH_EINVAL, "siglip: linear: ratio %g", (double)ratio);
  return matmul8_split(b, dst, x, rows, 0, outliers ? ratio : 0.f, bias);
}

int ixh_matmul8_tile(ixh_packed_b8 *b, const float *a, int m, int8_t *aq, float *sa,
                     int32_t *tile) {
  if (!b || m < 0 || (m > 0 && !a)) return fail(IXH_EINVAL, "linalg: MatMul8: slice too short");
  if (m == 0) return IXH_OK;
  DEVGUARD(b->device);
  TmpStream ts;
  HIPCK(hipStreamCreateWithFlags(&ts.s, hipStreamNonBlocking));
  const Mat &M = b->mat;
  DevBuf da, dq, dsa, dt;
  int rc;
  if ((rc = quantize_upload(a, m, M.k, M.kp, da, dq, dsa, ts.s))) return rc;
  if (tile) {
    if ((rc = dt.ensure(4 * (size_t)m * M.n))) return rc;
    GemmArgs g{};
    g.A = dq.as<int8_t>();
    g.lda = M.kp;
    g.B = M.q.as<int8_t>();
    g.ldb = M.kp;
    g.M = m;
    g.Np = M.np;
    g.Kp = M.kp;
    g.sa = dsa.as<float>();
    g.sb = M.sb.as<float>();
    g.zc = M.zc.as<float>();
    g.c128 = M.c128.as<int32_t>();
    g.Ci = dt.as<int32_t>();
    g.ldc = M.n;
    g.n_valid = M.n;
    g.Bk = M.qk.as<int8_t>();
    run_gemm(EPI_TILE, g, pb_tuning(b), ts.s);
    LAUNCHCK("matmul8_tile");
    HIPCK(hipMemcpyAsync(tile, dt.p, 4 * (size_t)m * M.n, hipMemcpyDeviceToHost, ts.s));
  }
  if (aq)
    HIPCK(hipMemcpy2DAsync(aq, (size_t)M.k, dq.p, (size_t)M.kp, (size_t)M.k, m, hipMemcpyDeviceToHost, ts.s));
  if (sa) HIPCK(hipMemcpyAsync(sa, dsa.p, 4 * (size_t)m, hipMemcpyDeviceToHost, ts.s));
  HIPCK(hipStreamSynchronize(ts.s));
  return IXH_OK;
}

int ixh_layernorm_quant(int device, const float *x, int m, int h, const float *gamma, double eps,
                        int lanes, float *out, int8_t *q, float *sa) {
  if (m < 0 || h <= 0 || (m > 0 && (!x || !gamma)) || (q && !sa))
    return fail(IXH_EINVAL, "linalg: LayerNormRow: bad arguments");
  if (h % 4 != 0) return fail(IXH_EINVAL, "linalg: hip: LayerNormRow needs rows of a multiple of 4 values");
  if (lanes != 0 && lanes != 4 && lanes != 8 && lanes != 16)
    return fail(IXH_EINVAL, "linalg: hip: lanes %d not in {0, 4, 8, 16}", lanes);
  if (m == 0) return IXH_OK;
  DEVGUARD(device);
  TmpStream ts;
  HIPCK(hipStreamCreateWithFlags(&ts.s, hipStreamNonBlocking));
  DevBuf dx, dg, dout, dq, dsa;
  int rc;
  if ((rc = dx.ensure(4 * (size_t)m * h)) || (rc = dg.ensure(4 * (size_t)h)) ||
      (rc = dout.ensure(4 * (size_t)m * h)) || (rc = dq.ensure((size_t)m * h)) ||
      (rc = dsa.ensure(4 * (size_t)m)))
    return rc;
  HIPCK(hipMemcpyAsync(dx.p, x, 4 * (size_t)m * h, hipMemcpyHostToDevice, ts.s));
  HIPCK(hipMemcpyAsync(dg.p, gamma, 4 * (size_t)h, hipMemcpyHostToDevice, ts.s));
  RowArgs r{};
  r.M = m;
  r.H = h;
  r.x = dx.as<float>();
  r.gamma = dg.as<float>();
  r.eps = eps;
  r.lanes = lanes;
  r.out = out ? dout.as<float>() : nullptr;
  r.q = q ? dq.as<int8_t>() : nullptr;
  r.ldq = h;
  r.sa = dsa.as<float>();
  launch_rownorm(r, ts.s);
  LAUNCHCK("layernorm_quant");
  if (out) HIPCK(hipMemcpyAsync(out, dout.p, 4 * (size_t)m * h, hipMemcpyDeviceToHost, ts.s));
  if (q) {
    HIPCK(hipMemcpyAsync(q, dq.p, (size_t)m * h, hipMemcpyDeviceToHost, ts.s));
    HIPCK(hipMemcpyAsync(sa, dsa.p, 4 * (size_t)m, hipMemcpyDeviceToHost, ts.s));
  }
  HIPCK(hipStreamSynchronize(ts.s));
  return IXH_OK;
}

int ixh_ln_matmul8_geglu(ixh_packed_b8 *b, const float *x, int m, const float *gamma, double eps,
                         int lanes, float *g, int32_t *tile) {
  if (!b || m < 0 || (m > 0 && (!x || !gamma || !g)))
    return fail(IXH_EINVAL, "linalg: GeluMul: bad arguments");
  const int k = b->mat.k, n = b->mat.n;
  if (n % 64 != 0) return fail(IXH_EINVAL, "linalg: hip: GeGLU needs n/2 a multiple of 32");
  if (k % 4 != 0) return fail(IXH_EINVAL, "linalg: hip: LayerNormRow needs rows of a multiple of 4 values");
  if (lanes != 0 && lanes != 4 && lanes != 8 && lanes != 16)
    return fail(IXH_EINVAL, "linalg: hip: lanes %d not in {0, 4, 8, 16}", lanes);
  if (m == 0) return IXH_OK;
  DEVGUARD(b->device);
  {
    std::lock_guard<std::mutex> lk(b->mu);
    if (!b->geglu_set) {
      std::vector<int> perm = geglu_perm(n / 2);
      int rc = upload_mat(b->geglu, b->rows, b->scale.data(), k, n, &perm);
      if (rc) return rc;
      b->geglu_set = true;
    }
  }
  TmpStream ts;
  HIPCK(hipStreamCreateWithFlags(&ts.s, hipStreamNonBlocking));
  const Mat &M = b->geglu;
  DevBuf dx, dgam, dq, dsa, dg, dt;
  int rc;
  if ((rc = dx.ensure(4 * (size_t)m * k)) || (rc = dgam.ensure(4 * (size_t)k)) ||
      (rc = dq.ensure((size_t)m * M.kp)) || (rc = dsa.ensure(4 * (size_t)m)) ||
      (rc = dg.ensure(4 * (size_t)m * (n / 2))))
    return rc;
  HIPCK(hipMemcpyAsync(dx.p, x, 4 * (size_t)m * k, hipMemcpyHostToDevice, ts.s));
  HIPCK(hipMemcpyAsync(dgam.p, gamma, 4 * (size_t)k, hipMemcpyHostToDevice, ts.s));
  RowArgs r{};
  r.M = m;
  r.H = k;
  r.x = dx.as<float>();
  r.gamma = dgam.as<float>();
  r.eps = eps;
  r.lanes = lanes;
  r.q = dq.as<int8_t>();
  r.ldq = M.kp;
  r.sa = dsa.as<float>();
  launch_rownorm(r, ts.s);
  LAUNCHCK("layernorm_quant");
  GemmArgs ga{};
  ga.A = dq.as<int8_t>();
  ga.lda = M.kp;
  ga.B = M.q.as<int8_t>();
  ga.ldb = M.kp;
  ga.M = m;
  ga.Np = M.np;
  ga.Kp = M.kp;
  ga.sa = dsa.as<float>();
  ga.sb = M.sb.as<float>();
  ga.zc = M.zc.as<float>();
  ga.c128 = M.c128.as<int32_t>();
  ga.C = dg.as<float>();
  ga.ldc = n / 2;
  ga.n_valid = n / 2;
  ga.lanes = lanes;
  ga.n_gelu = gelu_fma_cols(n / 2, lanes);
  ga.Bk = M.qk.as<int8_t>();
  run_gemm(EPI_GEGLU, ga, pb_tuning(b), ts.s);
  LAUNCHCK("geglu");
  HIPCK(hipMemcpyAsync(g, dg.p, 4 * (size_t)m * (n / 2), hipMemcpyDeviceToHost, ts.s));
  if (tile) {
    // the reference tile of the natural (un-interleaved) matrix
    const Mat &N0 = b->mat;
    if ((rc = dt.ensure(4 * (size_t)m * n))) return rc;
    GemmArgs gt = ga;
    gt.B = N0.q.as<int8_t>();
    gt.Bk = N0.qk.as<int8_t>();
    gt.Np = N0.np;
    gt.sb = N0.sb.as<float>();
    gt.zc = N0.zc.as<float>();
    gt.c128 = N0.c128.as<int32_t>();
    gt.Ci = dt.as<int32_t>();
    gt.C = nullptr;
    gt.ldc = n;
    gt.n_valid = n;
    run_gemm(EPI_TILE, gt, pb_tuning(b), ts.s);
    LAUNCHCK("geglu_tile");
    HIPCK(hipMemcpyAsync(tile, dt.p, 4 * (size_t)m * n, hipMemcpyDeviceToHost, ts.s));
  }
  HIPCK(hipStreamSynchronize(ts.s));
  return IXH_OK;
}

int ixh_attend8(int device, float *o, const float *q, const float *k, const float *v, int n, int d,
                int window, float scale, int lanes) {
  if (n < 0 || (n > 0 && (!o || !q || !k || !v))) return fail(IXH_EINVAL, "linalg: Attend8: bad arguments");
  if (d != 64) return fail(IXH_EINVAL, "linalg: hip: Attend8 head dimension %d not supported (64)", d);
  if (lanes != 0 && lanes != 4 && lanes != 8 && lanes != 16)
    return fail(IXH_EINVAL, "linalg: hip: lanes %d not in {0, 4, 8, 16}", lanes);
  if (n == 0) return IXH_OK;
  DEVGUARD(device);
  TmpStream ts;
  HIPCK(hipStreamCreateWithFlags(&ts.s, hipStreamNonBlocking));
  const int H = 64, Npad = (int)round_up(n, kKeyPad);
  std::vector<float> qkv((size_t)n * 3 * H);
  for (int j = 0; j < n; j++) {
    memcpy(&qkv[(size_t)j * 3 * H], q + (size_t)j * d, 4 * d);
    memcpy(&qkv[(size_t)j * 3 * H + H], k + (size_t)j * d, 4 * d);
    memcpy(&qkv[(size_t)j * 3 * H + 2 * H], v + (size_t)j * d, 4 * d);
  }
  std::vector<int32_t> tabs = {0, n, 0, Npad};
  std::vector<int32_t> blocks;
  for (int q0 = 0; q0 < n; q0 += kAttnQBlock) {
    blocks.push_back(0);
    blocks.push_back(q0);
  }
  DevBuf dqkv, dtabs, dblocks, dqq, dsq, dkp, dks, dvt, dvs, dctx;
  int rc;
  if ((rc = dqkv.ensure(4 * qkv.size())) || (rc = dtabs.ensure(16)) ||
      (rc = dblocks.ensure(4 * blocks.size())) || (rc = dqq.ensure((size_t)n * H)) ||
      (rc = dsq.ensure(4 * (size_t)n)) || (rc = dkp.ensure((size_t)Npad * H)) ||
      (rc = dks.ensure(4 * (size_t)Npad)) || (rc = dvt.ensure((size_t)H * Npad)) ||
      (rc = dvs.ensure(3 * 4 * H)) || (rc = dctx.ensure(4 * (size_t)n * H)))
    return rc;
  HIPCK(hipMemcpyAsync(dqkv.p, qkv.data(), 4 * qkv.size(), hipMemcpyHostToDevice, ts.s));
  HIPCK(hipMemcpyAsync(dtabs.p, tabs.data(), 16, hipMemcpyHostToDevice, ts.s));
  HIPCK(hipMemcpyAsync(dblocks.p, blocks.data(), 4 * blocks.size(), hipMemcpyHostToDevice, ts.s));
  AttnArgs aa{};
  aa.qkv = dqkv.as<float>();
  aa.H = H;
  aa.nh = 1;
  aa.N = n;
  aa.offs = dtabs.as<int32_t>();
  aa.padoff = dtabs.as<int32_t>() + 2;
  aa.B = 1;
  aa.max_n = n;
  aa.scale = scale;
  aa.window = window;
  aa.lanes = lanes;
  aa.qq = dqq.as<int8_t>();
  aa.sq = dsq.as<float>();
  aa.kp = dkp.as<int8_t>();
  aa.ks = dks.as<float>();
  aa.vt = dvt.as<int8_t>();
  aa.vs = dvs.as<float>();
  aa.kstat = aa.vs + H;
  aa.Npad = Npad;
  aa.blocks = dblocks.as<int32_t>();
  aa.nblocks = (int)blocks.size() / 2;
  aa.ctx = dctx.as<float>();
  launch_attn_quant_q(aa, ts.s);
  LAUNCHCK("attn_quant_q");
  launch_attn_prologue(aa, ts.s);
  LAUNCHCK("attn_prologue");
  launch_attn_main(aa, ts.s);
  LAUNCHCK("attn_main");
  HIPCK(hipMemcpyAsync(o, dctx.p, 4 * (size_t)n * H, hipMemcpyDeviceToHost, ts.s));
  HIPCK(hipStreamSynchronize(ts.s));
  return IXH_OK;
}


int ixh_check_exp255(int device, int64_t bad[2], float max_err[2], int64_t *undecided) {
  if (!bad || !max_err || !undecided) return fail(IXH_EINVAL, "linalg: hip: nil result");
  DEVGUARD(device);
  TmpStream ts;
  HIPCK(hipStreamCreateWithFlags(&ts.s, hipStreamNonBlocking));
  DevBuf dres;
  int rc;
  if ((rc = dres.ensure(5 * sizeof(unsigned long long)))) return rc;
  HIPCK(hipMemsetAsync(dres.p, 0, 5 * sizeof(unsigned long long), ts.s));
  // +0, then -0 .. -inf (sign bit set, exponent and mantissa up to 0x7f800000)
  launch_check_exp255(0u, 1u, dres.as<unsigned long long>(), ts.s);
  launch_check_exp255(0x80000000u, 0xff800001u, dres.as<unsigned long long>(), ts.s);
  LAUNCHCK("check_exp255");
  unsigned long long r[5];
  HIPCK(hipMemcpyAsync(r, dres.p, sizeof r, hipMemcpyDeviceToHost, ts.s));
  HIPCK(hipStreamSynchronize(ts.s));
  bad[0] = (int64_t)r[0];
  bad[1] = (int64_t)r[1];
  uint32_t e0 = (uint32_t)r[2], e1 = (uint32_t)r[3];
  memcpy(&max_err[0], &e0, 4);
  memcpy(&max_err[1], &e1, 4);
  *undecided = (int64_t)r[4];
  return IXH_OK;
}

int ixh_check_gelu(int device, int64_t bad[2]) {
  if (!bad) return fail(IXH_EINVAL, "linalg: hip: nil result");
  DEVGUARD(device);
  TmpStream ts;
  HIPCK(hipStreamCreateWithFlags(&ts.s, hipStreamNonBlocking));
  DevBuf dres;
  int rc;
  if ((rc = dres.ensure(2 * sizeof(unsigned long long)))) return rc;
  HIPCK(hipMemsetAsync(dres.p, 0, 2 * sizeof(unsigned long long), ts.s));
  launch_check_gelu(dres.as<unsigned long long>(), ts.s);
  LAUNCHCK("check_gelu");
  unsigned long long r[2];
  HIPCK(hipMemcpyAsync(r, dres.p, sizeof r, hipMemcpyDeviceToHost, ts.s));
  HIPCK(hipStreamSynchronize(ts.s));
  bad[0] = (int64_t)r[0];
  bad[1] = (int64_t)r[1];
  return IXH_OK;
}

int ixh_check_mfma_rate(int device, int iters, double *ops_per_s) {
  if (!ops_per_s || iters < 1 || iters > (1 << 22)) return fail(IXH_EINVAL, "linalg: hip: bad MFMA rate check");
  DEVGUARD(device);
  TmpStream ts;
  HIPCK(hipStreamCreateWithFlags(&ts.s, hipStreamNonBlocking));
  // four workgroups of four waves a CU: four waves a SIMD
  const int blocks = 4 * device_cus();
  DevBuf dout;
  int rc;
  if ((rc = dout.ensure((size_t)blocks * 256 * sizeof(int)))) return rc;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  HIPCK(hipEventCreate(&e0));
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return fail(IXH_EHIP, "linalg: hip: event");
  }
  launch_mfma_rate(blocks, iters, dout.as<int>(), ts.s);  // warm-up
  hipError_t e = hipEventRecord(e0, ts.s);
  if (e == hipSuccess) {
    launch_mfma_rate(blocks, iters, dout.as<int>(), ts.s);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipEventRecord(e1, ts.s);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (e != hipSuccess) return fail(IXH_EHIP, "linalg: hip: %s (MFMA rate check)", hipGetErrorString(e));
  // 32 x 32 x 32 multiply-adds = 65,536 operations an MFMA
  const double ops = (double)blocks * 4 * 4 * (double)iters * 65536.0;
  *ops_per_s = ms > 0.f ? ops / (ms * 1e-3) : 0.0;
  return IXH_OK;
}

}  // extern "C"

// ---- batching of concurrent requests ----------------------------------------
// WithBatching (model.go:136-160): the queue and its worker threads are
// BatchQueue's; a worker's merged batch runs as one encode_host pass.
struct ixh_batcher {
  std::unique_ptr<BatchQueue> q;
};

extern "C" {

int ixh_batcher_create(ixh_model *m, int workers, int max_rows, ixh_batcher **out) {
  if (!m || !out) return fail(IXH_EINVAL, "modernbert: nil model");
  if (workers <= 0) workers = 2;
  if (max_rows <= 0) max_rows = 65536;
  auto encode = [m](const int32_t *ids, const int32_t *offs, int B, float *pooled, std::string &err) {
    Outputs o;
    o.pooled = pooled;
    const int rc = encode_host(m, ids, offs, B, o);
    if (rc) err = g_err;
    return rc;
  };
  ixh_batcher *b = new ixh_batcher;
  b->q.reset(new BatchQueue(m->cfg.hidden, workers, max_rows, encode));
  *out = b;
  return IXH_OK;
}

int ixh_batcher_encode(ixh_batcher *b, const int32_t *ids, const int32_t *offs, int B, float *out) {
  if (!b) return fail(IXH_EINVAL, "modernbert: nil batcher");
  int rc;
  if ((rc = check_offs(offs, B))) return rc;
  if (B == 0) return IXH_OK;
  if ((offs[B] > 0 && !ids) || !out) return fail(IXH_EINVAL, "modernbert: inconsistent batch");
  std::string err;
  if ((rc = b->q->submit(ids, offs, B, out, err))) return fail(rc, "%s", err.c_str());
  return IXH_OK;
}

int ixh_batcher_stats(ixh_batcher *b, int64_t *batches, int64_t *requests) {
  if (!b || !batches || !requests) return fail(IXH_EINVAL, "modernbert: nil batcher");
  b->q->counts(batches, requests);
  return IXH_OK;
}

void ixh_batcher_destroy(ixh_batcher *b) { delete b; }

}  // extern "C"
