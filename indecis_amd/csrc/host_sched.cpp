// host_sched.cpp — the host-only scheduling of the C ABI (options, pass
// planning, the serving batcher's queue); no HIP calls, so the sanitizer
// builds of tests/sanitize run it on the CPU.
#include "host_sched.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/indecis_hip.h"

namespace ixh {
namespace {

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return set_error(code, buf);
}

}  // namespace

int set_tuning(Tuning &t, int option, int64_t v, bool model_opts) {
  auto bad = [&]() { return fail(IXH_EINVAL, "indecis: option %d: value %lld out of range", option, (long long)v); };
  switch (option) {
  case IXH_OPT_GEMM:
    if (v < 0 || v > 2) return bad();
    t.gemm = (int)v;
    return IXH_OK;
  case IXH_OPT_GEMM_TILE:
    if (v < 0 || v > 2) return bad();
    t.gemm_tile = (int)v;
    return IXH_OK;
  default: break;
  }
  if (!model_opts) return fail(IXH_EINVAL, "linalg: option %d does not apply to a PackedB8", option);
  switch (option) {
  case IXH_OPT_PARTS:
    if (v < 0 || v > 4) return bad();
    t.parts = (int)v;
    return IXH_OK;
  case IXH_OPT_PASS_TOKENS:
    if (v < 1 || v > kMaxPassTokensOpt) return bad();
    t.pass_tokens = (int)v;
    return IXH_OK;
  case IXH_OPT_QKV_FUSED:
    if (v != 0 && v != 1) return bad();
    t.qkv_fused = (int)v;
    return IXH_OK;
  case IXH_OPT_QKV_HEADS:
    if (v != 1 && v != 2) return bad();
    t.qkv_heads = (int)v;
    return IXH_OK;
  case IXH_OPT_LN_SEG:
    if (v != 0 && v != 1) return bad();
    t.ln_seg = (int)v;
    return IXH_OK;
  case IXH_OPT_FUSE_RES:
    if (v < 0 || v > 4) return bad();
    t.fuse_res = (int)v;
    return IXH_OK;
  case IXH_OPT_FUSE_MLP:
    if (v < 0 || v > 2) return bad();
    t.fuse_mlp = (int)v;
    return IXH_OK;
  case IXH_OPT_QKV_KBLOCK:
    if (v != 0 && v != 1) return bad();
    t.qkv_kblock = (int)v;
    return IXH_OK;
  default: return fail(IXH_EINVAL, "indecis: unknown option %d", option);
  }
}

int get_tuning(const Tuning &t, int option, int64_t *v) {
  switch (option) {
  case IXH_OPT_PARTS: *v = t.parts; return IXH_OK;
  case IXH_OPT_PASS_TOKENS: *v = t.pass_tokens; return IXH_OK;
  case IXH_OPT_QKV_FUSED: *v = t.qkv_fused; return IXH_OK;
  case IXH_OPT_QKV_HEADS: *v = t.qkv_heads; return IXH_OK;
  case IXH_OPT_GEMM: *v = t.gemm; return IXH_OK;
  case IXH_OPT_GEMM_TILE: *v = t.gemm_tile; return IXH_OK;
  case IXH_OPT_LN_SEG: *v = t.ln_seg; return IXH_OK;
  case IXH_OPT_FUSE_RES: *v = t.fuse_res; return IXH_OK;
  case IXH_OPT_FUSE_MLP: *v = t.fuse_mlp; return IXH_OK;
  case IXH_OPT_QKV_KBLOCK: *v = t.qkv_kblock; return IXH_OK;
  default: return fail(IXH_EINVAL, "indecis: unknown option %d", option);
  }
}

int pass_token_cap(int H, int I) {
  const int64_t per_token = 4 * (int64_t)std::max({3 * (int64_t)H, (int64_t)I, (int64_t)1});
  const int64_t cap = (((int64_t)1 << 31) - 1) / per_token;  // N * per_token < 2^31
  return (int)std::max<int64_t>(1, std::min<int64_t>(kMaxPassTokensOpt, cap));
}

int check_offs(const int32_t *offs, int B) {
  if (B < 0 || (B > 0 && !offs)) return fail(IXH_EINVAL, "modernbert: inconsistent batch");
  if (B == 0) return IXH_OK;
  if (offs[0] != 0) return fail(IXH_EINVAL, "modernbert: inconsistent batch");
  for (int b = 0; b < B; b++)
    if (offs[b + 1] < offs[b]) return fail(IXH_EINVAL, "modernbert: inconsistent batch");
  return IXH_OK;
}

// Rows do not depend on their batch (TestMatMul8RowsIndependent), so the
// results of several passes are those of one.
int plan_passes(const Tuning &t, int H, int I, const int32_t *offs, int B, std::vector<int> &cut) {
  const int cap = pass_token_cap(H, I);
  const int64_t limit = std::min(t.pass_tokens, cap);
  cut.assign(1, 0);
  for (int b = 0; b < B; b++) {
    const int n = offs[b + 1] - offs[b];
    if (n > cap)
      return fail(IXH_EINVAL, "modernbert: hip: sequence of %d tokens over the %d-token limit of a pass", n, cap);
    if (b > cut.back() && (int64_t)offs[b + 1] - offs[cut.back()] > limit) cut.push_back(b);
  }
  cut.push_back(B);
  return IXH_OK;
}

void split_points(const int32_t *offs, int B, int P, std::vector<int> &cut) {
  const int64_t N = B > 0 ? offs[B] : 0;
  cut.assign(P + 1, B);
  cut[0] = 0;
  for (int p = 1; p < P; p++) {
    int b = cut[p - 1];
    while (b < B && (int64_t)P * offs[b] < (int64_t)p * N) b++;
    cut[p] = b;
  }
}

BatchQueue::BatchQueue(int width, int workers, int max_rows, Encode encode)
    : width_(width), max_rows_(max_rows), encode_(std::move(encode)) {
  for (int i = 0; i < workers; i++) workers_.emplace_back(&BatchQueue::work, this);
}

BatchQueue::~BatchQueue() {
  close();
  for (std::thread &t : workers_) t.join();
}

void BatchQueue::close() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_ = true;
  }
  work_cv_.notify_all();
}

void BatchQueue::counts(int64_t *batches, int64_t *requests) {
  std::lock_guard<std::mutex> lk(mu_);
  *batches = batches_;
  *requests = requests_;
}

int BatchQueue::submit(const int32_t *ids, const int32_t *offs, int B, float *out, std::string &err) {
  Req r{ids, offs, B, offs[B], out};
  {
    std::unique_lock<std::mutex> lk(mu_);
    if (stop_) {
      err = "modernbert: batcher closed";
      return IXH_EINVAL;
    }
    queue_.push_back(&r);
    work_cv_.notify_one();
    done_cv_.wait(lk, [&] { return r.done; });
  }
  if (r.rc) err = r.err;
  return r.rc;
}

// batcher.work (batch.go:51-82)
void BatchQueue::work() {
  std::vector<Req *> batch;
  std::vector<int32_t> ids, offs;
  std::vector<float> pooled;
  std::string err;
  for (;;) {
    batch.clear();
    {
      std::unique_lock<std::mutex> lk(mu_);
      work_cv_.wait(lk, [&] { return stop_ || !queue_.empty(); });
      if (queue_.empty()) return;  // closed and drained
      batch.push_back(queue_.front());
      queue_.pop_front();
      int rows = batch[0]->rows;
      while (rows < max_rows_ && !queue_.empty()) {
        batch.push_back(queue_.front());
        rows += queue_.front()->rows;
        queue_.pop_front();
      }
    }
    int B = 0;
    for (Req *r : batch) B += r->B;
    offs.assign(B + 1, 0);
    ids.clear();
    int k = 0;
    for (Req *r : batch) {
      ids.insert(ids.end(), r->ids, r->ids + r->offs[r->B]);
      for (int s = 0; s < r->B; s++, k++) offs[k + 1] = offs[k] + (r->offs[s + 1] - r->offs[s]);
    }
    pooled.resize((size_t)B * width_);
    err.clear();
    const int rc = encode_(ids.data(), offs.data(), B, pooled.data(), err);
    size_t off = 0;
    for (Req *r : batch) {
      if (rc) {
        r->rc = rc;
        r->err = err;
      } else {
        memcpy(r->out, pooled.data() + off, sizeof(float) * (size_t)r->B * width_);
      }
      off += (size_t)r->B * width_;
    }
    {
      std::lock_guard<std::mutex> lk(mu_);
      for (Req *r : batch) r->done = true;
      batches_++;
      requests_ += (int64_t)batch.size();
    }
    done_cv_.notify_all();
  }
}

}  // namespace ixh
