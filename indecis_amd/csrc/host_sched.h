// host_sched.h — the host-only scheduling of the C ABI, free of HIP so that
// a CPU build can run it under sanitizers: the kernel options of a handle
// (Tuning), the checks of a batch's offsets, the planning of encoder passes
// and stream parts, where a pass's outputs start, the serving batcher's
// request queue (batch.go:1-82) and the free list of per-call workspaces.
#pragma once
#include <stdint.h>

#include <condition_variable>
#include <deque>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace ixh {

// Records the calling thread's last error (ixh_last_error) and returns code.
int set_error(int code, const char *msg);

// Kernel choices of a model or PackedB8 handle (ixh_model_set_option,
// ixh_packb8_set_option). Each call copies the handle's values once, so a
// change never reaches a pass already running.
struct Tuning {
  int parts = 0;          // streams a large batch is split over: 0 auto, 1..4
  int pass_tokens = 131072;  // most tokens of one encoder pass
  int qkv_fused = 1;      // QKV GEMM fused with Attn8.Prepare (sequences <= 512 keys)
  int qkv_heads = 1;      // heads a workgroup of the fused QKV kernel: 1 or 2
  int gemm = 0;           // 0: gemm_as for Wi/stores, gemm_i8 residual; 1: gemm_i8 only;
                          // 2: as 0 with the residual GEMMs on gemm_ws
  int gemm_tile = 0;      // gemm_i8 tiles: 0 128x128/2 stages, 1 256x128/3, 2 128x128/3
  int ln_seg = 1;         // LayerNorm lanes 8/16: 1 segment kernel, 0 whole-row LDS kernel
  int fuse_res = 1;       // residual GEMMs fused with quantizeA of their input and the next LN
  int fuse_mlp = 2;       // the MLP block (Wi, GeGLU, quantizeA, WoMLP, next LN) as one kernel:
                          // 2 mlp_block (64 rows, transposed), 1 mlp_res (32 rows), 0 separate
  int qkv_kblock = 1;     // the fused QKV kernel reads its input rows K-blocked (1) or row-major (0)
};

// Upper bound of Tuning::pass_tokens.
constexpr int kMaxPassTokensOpt = 131072;

// One option of ixh_model_set_option / ixh_packb8_set_option (model_opts:
// the encoder options are allowed; a PackedB8 handle takes only the GEMM
// choices), and its read-back.
int set_tuning(Tuning &t, int option, int64_t v, bool model_opts);
int get_tuning(const Tuning &t, int option, int64_t *v);

// Most tokens one pass of a model of width H and intermediate size I
// takes, sequences included: its largest buffer, the [N][3H] float32 QKV
// projection or the [N][I] float32 GeGLU output, then stays under 2^31
// bytes, so every byte offset into a pass's buffers fits the kernels' 31-bit
// offsets. kMaxPassTokensOpt at H 768 (1.2 GB), 87,381 at H 2048.
int pass_token_cap(int H, int I);

// offs [B+1] of a batch: offs[0] 0, never decreasing (B 0: offs may be null).
int check_offs(const int32_t *offs, int B);

// Passes of whole sequences, in order, each of at most min(pass_tokens,
// pass_token_cap(H, I)) tokens (a longer sequence takes a pass of its own,
// up to that cap: a sequence over it is an error): cut[i] .. cut[i+1].
int plan_passes(const Tuning &t, int H, int I, const int32_t *offs, int B, std::vector<int> &cut);

// P stream parts of about equal token counts: part p covers sequences
// [cut[p], cut[p+1]), the first starting at or past p*N/P (a part may be
// empty). cut has P+1 entries, cut[0] 0 and cut[P] B.
void split_points(const int32_t *offs, int B, int P, std::vector<int> &cut);

// What a pass writes (null: not wanted). states [N][H] final states
// (EncodeTokens); pooled [B][H] (EncodeSeqs); zp [B][rp] pooled-row head
// logits; zt [N][rt] per-token head logits. mean: pool by the mean whatever
// the config (meanRows, spans.go:466-476).
struct Outputs {
  float *states = nullptr;
  float *pooled = nullptr;
  double *zp = nullptr, *zt = nullptr;
  int mean = 0;
  // the outputs of sequences [b0, ...) whose first token is t0, with rp
  // pooled-row and rt per-token head rows
  Outputs at(int b0, int t0, int H, int rp, int rt) const {
    Outputs o = *this;
    if (o.states) o.states += (size_t)t0 * H;
    if (o.pooled) o.pooled += (size_t)b0 * H;
    if (o.zp) o.zp += (size_t)b0 * rp;
    if (o.zt) o.zt += (size_t)t0 * rt;
    return o;
  }
};

// Items that callers take and give back (per-call workspaces); take()
// returns null when none is free, and the caller makes a new one.
template <class T>
class FreeList {
 public:
  T *take() {
    std::lock_guard<std::mutex> lk(mu_);
    if (items_.empty()) return nullptr;
    T *p = items_.back();
    items_.pop_back();
    return p;
  }
  void put(T *p) {
    std::lock_guard<std::mutex> lk(mu_);
    items_.push_back(p);
  }
  // every item, for the owner's destruction
  std::vector<T *> drain() {
    std::lock_guard<std::mutex> lk(mu_);
    std::vector<T *> all;
    all.swap(items_);
    return all;
  }

 private:
  std::mutex mu_;
  std::vector<T *> items_;
};

// WithBatching / batcher (batch.go:1-82, model.go:136-160): worker threads
// each take the first pending request and, without waiting, the requests
// already queued while the batch stays under max_rows tokens, run them as
// one encode (sequences end to end), and hand every request its pooled
// rows; an error of the encode goes to every request of the batch.
class BatchQueue {
 public:
  // encode the merged batch (ids, offs [B+1]) into pooled [B][width];
  // nonzero: an error code, with its text in err
  using Encode = std::function<int(const int32_t *ids, const int32_t *offs, int B, float *pooled,
                                   std::string &err)>;
  BatchQueue(int width, int workers, int max_rows, Encode encode);
  ~BatchQueue();  // close(), then the queued requests run and the workers end

  // Runs the request (offs already checked, B > 0) and waits for its rows
  // in out [B][width]. Nonzero: the encode's error, or IXH_EINVAL once
  // closed; its text in err.
  int submit(const int32_t *ids, const int32_t *offs, int B, float *out, std::string &err);
  // encode passes run and requests they served
  void counts(int64_t *batches, int64_t *requests);
  // refuses new requests; the queued ones still run
  void close();

 private:
  struct Req {
    const int32_t *ids;
    const int32_t *offs;
    int B, rows;
    float *out;
    int rc = 0;
    std::string err;
    bool done = false;
  };
  void work();

  const int width_, max_rows_;
  const Encode encode_;
  std::mutex mu_;
  std::condition_variable work_cv_, done_cv_;
  std::deque<Req *> queue_;
  bool stop_ = false;
  int64_t batches_ = 0, requests_ = 0;
  std::vector<std::thread> workers_;
};

}  // namespace ixh
