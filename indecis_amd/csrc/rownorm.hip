// rownorm.hip — bandwidth-bound row kernels: embedding gather, LayerNorm,
// per-row int8 quantisation, pooling and decision-head logits.
//
// LayerNorm follows linalg.LayerNormRow (linalg/vec_simd.go:285-327): the
// reference keeps V float32 lane partials (V = the Go simd width of its
// host) filled sequentially, adds them in float64, and does the same for
// the fused d*d + sq. Those chains are sequential by definition, so a row
// is owned by V/4 threads, each carrying 4 lane partials with float4 loads
// (lanes == 0 is the scalar float64 build, vec_scalar.go:66-81, one thread
// per row).
#include "ixh_device.h"
#include "ixh_internal.h"

#include <algorithm>
#include <cstdlib>

namespace ixh {

namespace {

// Byte i of quantised row r: row-major q, or K-blocked qk (32-byte blocks
// of a row K-blocks apart; a 4-byte piece never straddles a block).
__device__ __forceinline__ int8_t *qbyte(const RowArgs &a, int r, int i) {
  return a.qk ? a.qk + ((size_t)(i >> 5) * a.qk_rows + r) * 32 + (i & 31) : a.q + (size_t)r * a.ldq + i;
}


struct RowSrc {
  const RowArgs &a;
  const float *f32;      // row base (f32 input, f32 table or exact row)
  const uint16_t *bf16;  // row base of a bf16 table
  const int8_t *i8;      // row base of an int8 table
  float i8s;

  __device__ RowSrc(const RowArgs &args, int r) : a(args), f32(nullptr), bf16(nullptr), i8(nullptr), i8s(0.f) {
    if (!a.ids) {
      f32 = a.x + (size_t)r * a.H;
      return;
    }
    const int id = min(max(a.ids[r], 0), a.vocab - 1);
    switch (a.emb_format) {
    case 1: {
      const int slot = a.exact_slot[id];
      if (slot >= 0)
        f32 = a.exact_rows + (size_t)slot * a.H;
      else
        bf16 = a.emb_bf16 + (size_t)id * a.H;
      break;
    }
    case 2:
      i8 = a.emb_i8 + (size_t)id * a.H;
      i8s = a.emb_i8_scale[id];
      break;
    default:
      f32 = a.emb_f32 + (size_t)id * a.H;
    }
  }
  // Four consecutive values at i (i % 4 == 0): embeddings.go:48-68.
  __device__ float4 load4(int i) const {
    if (f32) return *(const float4 *)(f32 + i);
    if (bf16) {
      const uint2 u = *(const uint2 *)(bf16 + i);
      return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                         __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    }
    const int w = *(const int *)(i8 + i);
    return make_float4((float)(int8_t)(w & 0xff) * i8s, (float)(int8_t)((w >> 8) & 0xff) * i8s,
                       (float)(int8_t)((w >> 16) & 0xff) * i8s, (float)(int8_t)(w >> 24) * i8s);
  }
  __device__ float load1(int i) const {
    if (f32) return f32[i];
    if (bf16) return __uint_as_float((unsigned)bf16[i] << 16);
    return (float)i8[i] * i8s;
  }
};

// Branch-free row source for the LDS kernel: SRC 0 f32 rows of a.x, 1 the
// f32 table, 2 the bf16 table (+ exact f32 rows), 3 the int8 table. The
// row is wave-uniform, so the only branch (bf16 vs exact) is scalar.
template <int SRC>
struct RowLoad {
  const float *f = nullptr;
  const uint16_t *h = nullptr;
  const int8_t *b = nullptr;
  float s = 0.f;
  __device__ RowLoad(const RowArgs &a, int R) {
    if constexpr (SRC == 0) {
      f = a.x + (size_t)R * a.H;
    } else {
      const int id = min(max(a.ids[R], 0), a.vocab - 1);
      if constexpr (SRC == 1) {
        f = a.emb_f32 + (size_t)id * a.H;
      } else if constexpr (SRC == 2) {
        const int slot = a.exact_slot[id];
        if (slot >= 0)
          f = a.exact_rows + (size_t)slot * a.H;
        else
          h = a.emb_bf16 + (size_t)id * a.H;
      } else {
        b = a.emb_i8 + (size_t)id * a.H;
        s = a.emb_i8_scale[id];
      }
    }
  }
  __device__ float4 load4(int i) const {
    if constexpr (SRC == 3) {
      const int w = *(const int *)(b + i);
      return make_float4((float)(int8_t)(w & 0xff) * s, (float)(int8_t)((w >> 8) & 0xff) * s,
                         (float)(int8_t)((w >> 16) & 0xff) * s, (float)(int8_t)(w >> 24) * s);
    } else if constexpr (SRC == 2) {
      if (f) return *(const float4 *)(f + i);
      const uint2 u = *(const uint2 *)(h + i);
      return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                         __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    } else {
      return *(const float4 *)(f + i);
    }
  }
};

// TPR threads per row (lanes/4), or 1 for the scalar (lanes == 0) build.
template <int TPR>
__global__ __launch_bounds__(256) void rownorm_kernel(RowArgs a) {
  const int gt = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = gt / TPR, sub = gt % TPR;
  if (r >= a.M) return;  // whole groups exit together (TPR divides 64)
  const RowSrc src(a, r);
  const int H = a.H;
  const int V = TPR * 4;
  const bool scalar = a.lanes <= 0;
  const int main_end = scalar ? 0 : (H / V) * V;

  float mean = 0.f, rstd = 1.f;
  const bool ln = a.gamma != nullptr;
  if (ln) {
    double sum = 0.0;
    if (scalar) {
      for (int i = 0; i < H; i++) sum += (double)src.load1(i);
    } else {
      float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
      for (int i = 4 * sub; i < main_end; i += V) {
        const float4 v = src.load4(i);
        p0 = p0 + v.x; p1 = p1 + v.y; p2 = p2 + v.z; p3 = p3 + v.w;
      }
      // lanes summed in float64 in lane order (vec_simd.go:294-297)
      for (int t = 0; t < TPR; t++) {
        sum += (double)__shfl(p0, t, TPR);
        sum += (double)__shfl(p1, t, TPR);
        sum += (double)__shfl(p2, t, TPR);
        sum += (double)__shfl(p3, t, TPR);
      }
      for (int i = main_end; i < H; i++) sum += (double)src.load1(i);
    }
    mean = (float)(sum / (double)H);
    double var = 0.0;
    if (scalar) {
      for (int i = 0; i < H; i++) {
        const double d = (double)(src.load1(i) - mean);
        var += d * d;
      }
    } else {
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
      for (int i = 4 * sub; i < main_end; i += V) {
        const float4 v = src.load4(i);
        const float d0 = v.x - mean, d1 = v.y - mean, d2 = v.z - mean, d3 = v.w - mean;
        s0 = __builtin_fmaf(d0, d0, s0);
        s1 = __builtin_fmaf(d1, d1, s1);
        s2 = __builtin_fmaf(d2, d2, s2);
        s3 = __builtin_fmaf(d3, d3, s3);
      }
      for (int t = 0; t < TPR; t++) {
        var += (double)__shfl(s0, t, TPR);
        var += (double)__shfl(s1, t, TPR);
        var += (double)__shfl(s2, t, TPR);
        var += (double)__shfl(s3, t, TPR);
      }
      for (int i = main_end; i < H; i++) {
        const double d = (double)(src.load1(i) - mean);
        var += d * d;
      }
    }
    rstd = (float)(1.0 / __builtin_sqrt(var / (double)H + a.eps));
  }

  // Output pass(es): o = ((x - mean) * rstd) * gamma. Each thread owns the
  // columns 4*sub + V*k (+ the tail for sub 0; every column if scalar).
  auto out_at = [&](int i, float x) -> float {
    return ln ? ((x - mean) * rstd) * a.gamma[i] : x;
  };
  const int step = scalar ? 4 : V;
  const int first = scalar ? 0 : 4 * sub;
  const int vec_end = scalar ? (H & ~3) : main_end;
  const int tail_begin = vec_end;
  const bool do_tail = scalar || sub == 0;
  float mx = 0.f;
  for (int i = first; i < vec_end; i += step) {
    const float4 v = src.load4(i);
    const float o0 = out_at(i, v.x), o1 = out_at(i + 1, v.y), o2 = out_at(i + 2, v.z),
                o3 = out_at(i + 3, v.w);
    if (a.out) *(float4 *)(a.out + (size_t)r * H + i) = make_float4(o0, o1, o2, o3);
    mx = amax(amax(amax(amax(mx, o0), o1), o2), o3);
  }
  if (do_tail)
    for (int i = tail_begin; i < H; i++) {
      const float o = out_at(i, src.load1(i));
      if (a.out) a.out[(size_t)r * H + i] = o;
      mx = amax(mx, o);
    }
  if (!a.q) return;
  for (int t = 1; t < TPR; t <<= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, t, TPR));
  // quantizeA (linalg/int8.go:160-191): scale = max/127, inv = 1/scale.
  float s = 0.f, inv = 0.f;
  if (mx != 0.f) {
    s = mx / 127.0f;
    inv = 1.0f / s;
  }
  for (int i = first; i < vec_end; i += step) {
    const float4 v = src.load4(i);
    const int q0 = q8(out_at(i, v.x), inv), q1 = q8(out_at(i + 1, v.y), inv);
    const int q2 = q8(out_at(i + 2, v.z), inv), q3 = q8(out_at(i + 3, v.w), inv);
    *(int *)qbyte(a, r, i) = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
  }
  if (do_tail) {
    for (int i = tail_begin; i < H; i++) *qbyte(a, r, i) = (int8_t)q8(out_at(i, src.load1(i)), inv);
    if (!a.qk)
      for (int i = H; i < a.ldq; i++) a.q[(size_t)r * a.ldq + i] = 0;
    a.sa[r] = s;
  }
}

// LayerNorm (+ quantisation) for lanes V in {8, 16} and H = 256*CPL with
// each wave's RPW = 64/V rows held in registers (lane t: columns
// 4*(t + 64c)) and only one 256-column segment of them in LDS at a time:
// lane (r, l) = (t / V, t % V) runs the reference's lane partial l of row r
// — x[l], x[l+V], ... added in order — segment after segment, carrying the
// partial across segments (the same additions in the same order as over
// the whole row). About 8 KB of LDS per wave instead of the whole rows, so
// four times as many waves share a CU; the output and quantisation passes
// run from the registers.
// H = 256*(CPL-1) + 128 (HALF): the last segment is 128 columns, held by
// lanes 0..31 (the others hold zeros and store nothing).
template <int V, int CPL, int SRC, bool HALF = false>
__global__ __launch_bounds__(64) void rownorm_seg_kernel(RowArgs a) {
  constexpr int RPW = 64 / V, H = 256 * CPL - (HALF ? 128 : 0), LD = 256 + V;
  __shared__ __attribute__((aligned(16))) float xs[RPW * LD];
  const int lane = threadIdx.x;
  const int grp = blockIdx.x;
  // this lane's columns of segment c exist (wave-uniform but for the half
  // segment)
  auto has = [&](int c) { return !HALF || c < CPL - 1 || lane < 32; };
  float4 x[RPW][CPL];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int R = min(grp * RPW + r, a.M - 1);  // rows past M repeat the last one
    const RowLoad<SRC> src(a, R);
#pragma unroll
    for (int c = 0; c < CPL; c++)
      x[r][c] = has(c) ? src.load4(4 * (lane + 64 * c)) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const bool ln = a.gamma != nullptr;
  const int rr = lane / V, l = lane % V;  // this lane's chain: row rr, lane partial l
  float mean = 0.f, rstd = 1.f;           // of row rr
  if (ln) {
    // sum: the chain over segment c continues from segment c-1
    float p = 0.f;
    // columns of segment c
    auto segw = [](int c) { return HALF && c == CPL - 1 ? 128 : 256; };
#pragma unroll
    for (int c = 0; c < CPL; c++) {
#pragma unroll
      for (int r = 0; r < RPW; r++) *(float4 *)&xs[r * LD + 4 * lane] = x[r][c];
      __builtin_amdgcn_wave_barrier();
      const float *xr = &xs[rr * LD + l];
#pragma unroll
      for (int k = 0; k < segw(c) / V; k++) p = p + xr[V * k];
      __builtin_amdgcn_wave_barrier();
    }
    double sum = 0.0;  // lanes in order, in float64 (vec_simd.go:294-297)
#pragma unroll
    for (int t = 0; t < V; t++) sum += (double)__shfl(p, rr * V + t);
    mean = (float)(sum / (double)H);
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; c++) {
#pragma unroll
      for (int r = 0; r < RPW; r++) *(float4 *)&xs[r * LD + 4 * lane] = x[r][c];
      __builtin_amdgcn_wave_barrier();
      const float *xr = &xs[rr * LD + l];
#pragma unroll
      for (int k = 0; k < segw(c) / V; k++) {
        const float d = xr[V * k] - mean;
        q = __builtin_fmaf(d, d, q);
      }
      __builtin_amdgcn_wave_barrier();
    }
    double var = 0.0;
#pragma unroll
    for (int t = 0; t < V; t++) var += (double)__shfl(q, rr * V + t);
    rstd = (float)(1.0 / __builtin_sqrt(var / (double)H + a.eps));
  }
  // output from the registers; every row's max |o| reduced together
  float mx[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int R = min(grp * RPW + r, a.M - 1);
    const float mu = __shfl(mean, r * V), rs = __shfl(rstd, r * V);
    mx[r] = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; c++) {
      if (!has(c)) continue;
      float4 v = x[r][c];
      if (ln) {
        const float4 g = *(const float4 *)&a.gamma[4 * (lane + 64 * c)];
        v = make_float4(((v.x - mu) * rs) * g.x, ((v.y - mu) * rs) * g.y, ((v.z - mu) * rs) * g.z,
                        ((v.w - mu) * rs) * g.w);
        x[r][c] = v;
      }
      if (a.out && grp * RPW + r < a.M) *(float4 *)(a.out + (size_t)R * H + 4 * (lane + 64 * c)) = v;
      // |o| has no NaN and no -0, so max picks the same value as the
      // reference's compare
      mx[r] = __builtin_fmaxf(mx[r], __builtin_fmaxf(__builtin_fmaxf(fabsf(v.x), fabsf(v.y)),
                                                     __builtin_fmaxf(fabsf(v.z), fabsf(v.w))));
    }
  }
  if (!a.q) return;
#pragma unroll
  for (int t = 1; t < 64; t <<= 1)
#pragma unroll
    for (int r = 0; r < RPW; r++) mx[r] = __builtin_fmaxf(mx[r], __shfl_xor(mx[r], t));
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int R = grp * RPW + r;
    if (R >= a.M) break;  // wave-uniform
    float s = 0.f, inv = 0.f;
    if (mx[r] != 0.f) {  // quantizeA (linalg/int8.go:160-191)
      s = mx[r] / 127.0f;
      inv = 1.0f / s;
    }
#pragma unroll
    for (int c = 0; c < CPL; c++) {
      if (!has(c)) continue;
      const float4 v = x[r][c];
      const int q0 = q8(v.x, inv), q1 = q8(v.y, inv), q2 = q8(v.z, inv), q3 = q8(v.w, inv);
      *(int *)qbyte(a, R, 4 * (lane + 64 * c)) = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
    }
    if (!a.qk)
      for (int i = H + lane; i < a.ldq; i += 64) a.q[(size_t)R * a.ldq + i] = 0;
    if (lane == 0) a.sa[R] = s;
  }
}

// LayerNorm (+ quantisation) for lanes V in {4, 8, 16} and H = 256*CPL:
// one wave owns RPW = 64/V rows. Lane t holds columns 4*(t + 64c) of each
// row in registers (coalesced float4 loads, every load of the wave in
// flight before the first wait) and copies them to LDS; lane (r, l) =
// (t / V, t % V) then runs the reference's lane partial l of row r —
// x[l], x[l+V], ... added in order — from LDS, so all 64 lanes carry one of
// the sequential chains. The output and quantisation passes use the
// registers. Rows are padded by V floats in LDS (conflict-free chains).
template <int V, int CPL, int SRC>
__global__ __launch_bounds__(64) void rownorm_lds_kernel(RowArgs a) {
  constexpr int RPW = 64 / V, H = 256 * CPL, LD = H + V;
  __shared__ __attribute__((aligned(16))) float xs[RPW * LD];
  __shared__ float rmean[RPW], rrstd[RPW];
  const int lane = threadIdx.x;
  const int groups = (a.M + RPW - 1) / RPW;
  // The grid holds at most as many waves as fit on the device at once; each
  // wave walks row groups blockIdx.x, + gridDim.x, ... and loads the next
  // group into registers while the current one runs from LDS.
  float4 x[RPW][CPL];
  auto load = [&](int grp) {
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      const int R = min(grp * RPW + r, a.M - 1);  // rows past M repeat the last one
      const RowLoad<SRC> src(a, R);
#pragma unroll
      for (int c = 0; c < CPL; c++) x[r][c] = src.load4(4 * (lane + 64 * c));
    }
  };
  const bool ln = a.gamma != nullptr;
  float4 g[CPL];
  if (ln) {
#pragma unroll
    for (int c = 0; c < CPL; c++) g[c] = *(const float4 *)&a.gamma[4 * (lane + 64 * c)];
  }
  int grp = blockIdx.x;
  load(grp);
  for (; grp < groups; grp += gridDim.x) {
    __syncthreads();  // the previous group's output pass is done with xs
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
      for (int c = 0; c < CPL; c++) *(float4 *)&xs[r * LD + 4 * (lane + 64 * c)] = x[r][c];
    if (grp + (int)gridDim.x < groups) load(grp + gridDim.x);
    __syncthreads();
    if (ln) {
      const int r = lane / V, l = lane % V;
      const float *xr = &xs[r * LD + l];
      float p = 0.f;
#pragma unroll
      for (int k = 0; k < H / V; k++) p = p + xr[V * k];
      double sum = 0.0;  // lanes in order, in float64 (vec_simd.go:294-297)
#pragma unroll
      for (int t = 0; t < V; t++) sum += (double)__shfl(p, r * V + t);
      const float mean = (float)(sum / (double)H);
      float q = 0.f;
#pragma unroll
      for (int k = 0; k < H / V; k++) {
        const float d = xr[V * k] - mean;
        q = __builtin_fmaf(d, d, q);
      }
      double var = 0.0;
#pragma unroll
      for (int t = 0; t < V; t++) var += (double)__shfl(q, r * V + t);
      if (l == 0) {
        rmean[r] = mean;
        rrstd[r] = (float)(1.0 / __builtin_sqrt(var / (double)H + a.eps));
      }
      __syncthreads();
    }
    // Output in three steps so the RPW wave reductions overlap: normalise
    // every row (back into LDS when it is quantised next) with its max |o|,
    // reduce the RPW maxima together, then quantise.
    float mx[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      const int R = min(grp * RPW + r, a.M - 1);  // rows past M: computed, not stored
      mx[r] = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; c++) {
        float4 *px = (float4 *)&xs[r * LD + 4 * (lane + 64 * c)];
        float4 v = *px;
        if (ln) {
          const float mean = rmean[r], rstd = rrstd[r];
          v = make_float4(((v.x - mean) * rstd) * g[c].x, ((v.y - mean) * rstd) * g[c].y,
                          ((v.z - mean) * rstd) * g[c].z, ((v.w - mean) * rstd) * g[c].w);
          if (a.q) *px = v;
        }
        if (a.out && grp * RPW + r < a.M) *(float4 *)(a.out + (size_t)R * H + 4 * (lane + 64 * c)) = v;
        // |o| has no NaN and no -0, so max picks the same value as the
        // reference's compare
        mx[r] = __builtin_fmaxf(mx[r], __builtin_fmaxf(__builtin_fmaxf(fabsf(v.x), fabsf(v.y)),
                                                       __builtin_fmaxf(fabsf(v.z), fabsf(v.w))));
      }
    }
    if (!a.q) continue;
#pragma unroll
    for (int t = 1; t < 64; t <<= 1)
#pragma unroll
      for (int r = 0; r < RPW; r++) mx[r] = __builtin_fmaxf(mx[r], __shfl_xor(mx[r], t));
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      const int R = grp * RPW + r;
      if (R >= a.M) break;  // wave-uniform
      float s = 0.f, inv = 0.f;
      if (mx[r] != 0.f) {  // quantizeA (linalg/int8.go:160-191)
        s = mx[r] / 127.0f;
        inv = 1.0f / s;
      }
#pragma unroll
      for (int c = 0; c < CPL; c++) {
        const float4 v = *(const float4 *)&xs[r * LD + 4 * (lane + 64 * c)];
        const int q0 = q8(v.x, inv), q1 = q8(v.y, inv), q2 = q8(v.z, inv), q3 = q8(v.w, inv);
        *(int *)qbyte(a, R, 4 * (lane + 64 * c)) = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
      }
      if (!a.qk)
        for (int i = H + lane; i < a.ldq; i += 64) a.q[(size_t)R * a.ldq + i] = 0;
      if (lane == 0) a.sa[R] = s;
    }
  }
}

// quantizeA on f32 rows with the row in registers (CPL float4 per lane,
// K <= 256*CPL): one wave per row, every load in flight before the max.
template <int CPL>
__global__ __launch_bounds__(256) void quant_rows_reg_kernel(const float *x, int ld, int M, int K,
                                                             int8_t *q, int ldq, float *sa) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= M) return;
  const float *row = x + (size_t)r * ld;
  float4 v[CPL];
  float mx = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; c++) {
    const int i = 4 * (lane + 64 * c);
    v[c] = i < K ? *(const float4 *)(row + i) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int c = 0; c < CPL; c++)
    mx = amax(amax(amax(amax(mx, v[c].x), v[c].y), v[c].z), v[c].w);
  for (int t = 1; t < 64; t <<= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, t));
  float s = 0.f, inv = 0.f;
  if (mx != 0.f) {
    s = mx / 127.0f;
    inv = 1.0f / s;
  }
  int8_t *qrow = q + (size_t)r * ldq;
#pragma unroll
  for (int c = 0; c < CPL; c++) {
    const int i = 4 * (lane + 64 * c);
    if (i < K) {
      const int q0 = q8(v[c].x, inv), q1 = q8(v[c].y, inv), q2 = q8(v[c].z, inv), q3 = q8(v[c].w, inv);
      *(int *)(qrow + i) = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
    }
  }
  for (int i = K + lane; i < ldq; i += 64) qrow[i] = 0;
  if (lane == 0) sa[r] = s;
}

// One wave per row: quantizeA on rows of f32 (no LayerNorm).
__global__ __launch_bounds__(256) void quant_rows_kernel(const float *x, int ld, int M, int K,
                                                         int8_t *q, int ldq, float *sa) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= M) return;
  const float *row = x + (size_t)r * ld;
  float mx = 0.f;
  for (int i = 4 * lane; i < K; i += 256) {
    const float4 v = *(const float4 *)(row + i);
    mx = amax(amax(amax(amax(mx, v.x), v.y), v.z), v.w);
  }
  for (int t = 1; t < 64; t <<= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, t));
  float s = 0.f, inv = 0.f;
  if (mx != 0.f) {
    s = mx / 127.0f;
    inv = 1.0f / s;
  }
  int8_t *qrow = q + (size_t)r * ldq;
  for (int i = 4 * lane; i < K; i += 256) {
    const float4 v = *(const float4 *)(row + i);
    const int q0 = q8(v.x, inv), q1 = q8(v.y, inv), q2 = q8(v.z, inv), q3 = q8(v.w, inv);
    *(int *)(qrow + i) = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
  }
  for (int i = K + lane; i < ldq; i += 64) qrow[i] = 0;
  if (lane == 0) sa[r] = s;
}

__global__ void positions_kernel(const int32_t *offs, const int32_t *padoff, int32_t *pos,
                                 int32_t *slot) {
  const int b = blockIdx.x;
  const int o = offs[b], n = offs[b + 1] - o, p = padoff[b];
  for (int t = threadIdx.x; t < n; t += blockDim.x) {
    pos[o + t] = t;
    if (slot) slot[o + t] = p + t;
  }
}

// infer.go:265-287: float64 sum over the sequence, in token order.
// Pooling (infer.go:265-287): the float64 sum of a column over the
// sequence's tokens in token order, over n, or the first token's row (CLS).
// Short sequences: one thread a column, its rows loaded 16 ahead of its
// in-order float64 adds.
__global__ void pool_kernel(const float *xn, const int32_t *offs, int H, int cls, float *out) {
  const int b = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= H) return;
  const int o = offs[b], n = offs[b + 1] - o;
  float *dst = out + (size_t)b * H + k;
  if (n == 0) {
    *dst = 0.f;
    return;
  }
  if (cls) {
    *dst = xn[(size_t)o * H + k];
    return;
  }
  double acc = 0.0;
  const float *col = xn + (size_t)o * H + k;
  int t = 0;
  for (; t + 16 <= n; t += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; u++) v[u] = col[(size_t)(t + u) * H];
#pragma unroll
    for (int u = 0; u < 16; u++) acc += (double)v[u];
  }
  for (; t < n; t++) acc += (double)col[(size_t)t * H];
  *dst = (float)(acc / (double)n);
}

// Long sequences (a batch averaging over 1,024 tokens a sequence): one
// workgroup of 4 waves per (sequence, 64 columns), wave 0's lane c running
// column c's chain while all four waves bring the rows in, 64 rows x 64
// columns (16 KB) a stage by direct-to-LDS buffer loads (4 rows of 256
// bytes an instruction), 8 stages in a ring and 7 in flight, so that the
// sequence streams while the chain adds (thread-per-column loads waited on
// HBM every 16 rows: 362 us for cfg5's 8 x 8,192 tokens). The chain reads
// the ring with lds_read4, 16 rows ahead of its adds, and adds whole groups
// of 16 unconditionally (the tail apart), so its only dependence is the
// float64 add itself.
constexpr int PL_R = 64, PL_S = 8, PL_STAGE = PL_R * 64 * 4;  // rows a stage, stages, bytes a stage
__device__ __forceinline__ float lds_read4(uint32_t addr) {
  float v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ float lds_read4_now(uint32_t addr) {
  float v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ void lgkm_wait16(float (&v)[16]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]),
                 "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]), "+v"(v[12]), "+v"(v[13]), "+v"(v[14]),
                 "+v"(v[15]));
}
__global__ __launch_bounds__(256) void pool_ring_kernel(const float *xn, const int32_t *offs, int H, int cls,
                                                        float *out) {
  extern __shared__ __attribute__((aligned(16))) float pring[];  // [PL_S][PL_R][64]
  const int b = blockIdx.y, c0 = 64 * blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int o = offs[b], n = offs[b + 1] - o;
  const int ncol = min(64, H - c0);
  float *dst = out + (size_t)b * H + c0 + lane;
  if (n == 0 || cls) {
    if (wave == 0 && lane < ncol) *dst = n == 0 ? 0.f : xn[(size_t)o * H + c0 + lane];
    return;
  }
  // rows of the sequence through a descriptor (rows past n read 0, never
  // added); this thread's 4 loads of a stage: rows 16 wave + 4 k + lane / 16,
  // columns 4 (lane % 16) .. + 3 (past ncol: read, never added)
  const __amdgpu_buffer_rsrc_t xr = buf_rsrc(xn + (size_t)o * H + c0, (uint32_t)(n * H * 4));
  const int ns = (n + PL_R - 1) / PL_R;
  auto issue = [&](int c) {
    // past the last stage: an offset past the descriptor's range (no
    // memory access; the count of loads in flight stays fixed)
    const int cc = min(c, ns - 1);
    const uint32_t soff = c < ns ? 0u : 0x80000000u;
    float *st = pring + (c % PL_S) * (PL_R * 64);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int r = 16 * wave + 4 * k + (lane >> 4);
      const uint32_t voff = (uint32_t)((PL_R * cc + r) * H + 4 * (lane & 15)) * 4u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(st + 256 * (4 * wave + k)), 16, voff, soff, 0, 0);
    }
  };
#pragma unroll
  for (int c = 0; c < PL_S - 1; c++) issue(c);
  double acc = 0.0;
  const uint32_t base = (uint32_t)(size_t)(lds_ptr)pring + 4u * lane;
  for (int c = 0; c < ns; c++) {
    wait_vmcnt<4 * (PL_S - 2)>();  // this thread's loads of stage c are in LDS
    lds_barrier();                 // everyone's are, and stage c - 1 is read
    issue(c + PL_S - 1);
    if (wave == 0) {
      const uint32_t st = base + (uint32_t)((c % PL_S) * PL_STAGE);
      const int rows = min(PL_R, n - PL_R * c);
      float v[16], nx[16];
#pragma unroll
      for (int i = 0; i < 16; i++) v[i] = lds_read4(st + 256u * i);
      lgkm_wait16(v);
      int r0 = 0;
      for (; r0 + 16 <= rows; r0 += 16) {
        // the next 16 rows' reads in flight while these 16 are added (past
        // the stage: rows of the ring, not added)
#pragma unroll
        for (int i = 0; i < 16; i++) nx[i] = lds_read4(st + 256u * (uint32_t)((r0 + 16 + i) & (PL_R - 1)));
#pragma unroll
        for (int i = 0; i < 16; i++) acc += (double)v[i];
        lgkm_wait16(nx);
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = nx[i];
      }
      for (int i = 0; i < rows - r0; i++) acc += (double)lds_read4_now(st + 256u * (uint32_t)(r0 + i));
    }
  }
  wait_vmcnt<0>();  // the loads past the last stage complete before the workgroup ends
  if (wave == 0 && lane < ncol) *dst = (float)(acc / (double)n);
}

// head.logits (heads.go:63-74) and the spans head (spans.go:449-459):
// z[t][r] = sum_i f64(w[r][i]) * f64(x[t][i]) in column order, + f64(b[r]).
// Each product of two float32 is exact in float64, so fma(x, w, s) rounds
// once where the reference's s + x*w does: the same bits.
//
// One workgroup of NW waves takes 64 tokens (lane = token) and rg <= NW RW
// rows: wave w the rows r0 + w + NW j, j < RW (a row past the workgroup's
// last is computed on its last row and not stored). x arrives in stages of
// 32 columns (8 KB: 64 tokens x 128 bytes) by direct-to-LDS buffer loads,
// HT_S stages in a ring, HT_S - 1 in flight; slot j of token t holds the
// token's 16-byte piece j ^ ((t >> 1) & 7), so the lanes' 16-byte reads of
// one piece fall in distinct banks. Every lane uses the same weight at a
// time, so the weights (widened to float64, exact) stay out of LDS: a
// stage's 32 weights of a row are two float64 registers whose lane l holds
// column 16 h + l % 16, loaded with the stage's x, and each FMA takes its
// weight by DPP row_newbcast (lane n of every 16-lane row, to the row) —
// no broadcast read from LDS (LDS returns 128 bytes a clock: a float64 to
// 64 lanes would cost 4 clocks an FMA) and no scalar loads (whose waits,
// one for all in flight, left the kernel at half the rate). Stages past
// the last load the last one again (the count of loads in flight stays
// fixed; nothing reads them). The ring is read by lds_read16: the
// compiler, seeing an LDS read, would wait for every direct-to-LDS load in
// flight first.
constexpr int HT_T = 64, HT_C = 32, HT_S = 4;
constexpr int HT_STAGE = HT_T * HT_C * 4;  // bytes a stage
typedef float hv4 __attribute__((ext_vector_type(4)));
// 16 bytes from LDS, outside the compiler's view (no wait is inserted for
// it or for loads in flight); lgkm_wait makes its results usable
__device__ __forceinline__ hv4 lds_read16(uint32_t addr) {
  hv4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ void lgkm_wait(hv4 (&v)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
}
// acc[j] += bcast_N(w[j]) * x for the RW rows j: v_fmac_f64 with the
// weight register as the DPP source (row_newbcast:N). The s_nop keeps two
// wait states between any VALU write of a weight register and its DPP
// read (the hardware's rule for DPP sources; the weights come from loads,
// but the compiler may copy them); one statement for the rows keeps the
// compiler from placing anything between the nop and the FMAs.
#define HT_FMA(A, W) "v_fmac_f64_dpp %" #A ", %" #W ", %[x] row_newbcast:%[n] row_mask:0xf bank_mask:0xf"
template <int N, int RW>
__device__ __forceinline__ void fmac_bc(double (&acc)[RW], const double (&w)[RW], double x) {
  if constexpr (RW == 1)
    asm volatile("s_nop 1\n\t" HT_FMA(0, 1) : "+v"(acc[0]) : "v"(w[0]), [x] "v"(x), [n] "i"(N));
  else if constexpr (RW == 2)
    asm volatile("s_nop 1\n\t" HT_FMA(0, 2) "\n\t" HT_FMA(1, 3)
                 : "+v"(acc[0]), "+v"(acc[1])
                 : "v"(w[0]), "v"(w[1]), [x] "v"(x), [n] "i"(N));
  else
    asm volatile("s_nop 1\n\t" HT_FMA(0, 3) "\n\t" HT_FMA(1, 4) "\n\t" HT_FMA(2, 5)
                 : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2])
                 : "v"(w[0]), "v"(w[1]), "v"(w[2]), [x] "v"(x), [n] "i"(N));
}
#undef HT_FMA
template <int RW, int NW>
__global__ __launch_bounds__(64 * NW) void head_logits_kernel(const float *__restrict__ x, int T, int H,
                                                              const double *__restrict__ w,
                                                              const float *__restrict__ b, int rows, int rg,
                                                              double *__restrict__ z) {
  __shared__ __attribute__((aligned(16))) float hx[HT_S * HT_T * HT_C];
  // a stage is 8 wave-wide loads (1 KB each); wave w issues loads
  // LPT w .. LPT w + LPT - 1, the ones past 7 repeating load 7 (the same
  // bytes to the same place), so every wave runs the same code
  constexpr int LPT = (HT_STAGE / 1024 + NW - 1) / NW;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t0 = blockIdx.x * HT_T, r0 = blockIdx.y * rg;
  const int nr = min(rg, rows - r0);
  const int nt = min(HT_T, T - t0);
  const int ns = H / HT_C;
  // load k of this wave: slot s = 64 q + lane of a stage (q its 1 KB
  // piece), token s / 8, global piece (s % 8) ^ ((token >> 1) & 7); through
  // a buffer descriptor over the workgroup's tokens (tokens past T read 0,
  // never stored), the lane's offset fixed in a VGPR and the stage's
  // column in the SGPR offset
  const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x + (size_t)t0 * H, (uint32_t)(nt * H * 4));
  uint32_t voff[LPT];
  int dst[LPT];
  sfor<LPT>([&](auto kv) {
    const int q = min(LPT * wave + kv.value, HT_STAGE / 1024 - 1);
    const int s = 64 * q + lane, t = s >> 3;
    voff[kv.value] = (uint32_t)(t * H + 4 * ((s & 7) ^ ((t >> 1) & 7))) * 4u;
    dst[kv.value] = 256 * q;
  });
  const double *wl[RW];  // this lane's weights: row j, column lane % 16
#pragma unroll
  for (int j = 0; j < RW; j++) wl[j] = w + (size_t)(r0 + min(wave + NW * j, nr - 1)) * H + (lane & 15);
  double wq[HT_S][2][RW];  // the ring's weights: stage slot, 16-column half, row
  auto issue = [&](auto uv, int c) {
    constexpr int u = decltype(uv)::value % HT_S;
    const int cc = HT_C * min(c, ns - 1);
    const uint32_t soff = 4u * (uint32_t)cc;
    sfor<LPT>([&](auto kv) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(hx + u * (HT_T * HT_C) + dst[kv.value]), 16,
                                               voff[kv.value], soff, 0, 0);
    });
#pragma unroll
    for (int j = 0; j < RW; j++) {
      wq[u][0][j] = wl[j][cc];
      wq[u][1][j] = wl[j][cc + 16];
    }
  };
  double acc[RW];
#pragma unroll
  for (int j = 0; j < RW; j++) acc[j] = 0.0;
  const uint32_t xl = (uint32_t)(size_t)(lds_ptr)hx + 128u * lane;  // this lane's token row, slot 0
  const int sw = (lane >> 1) & 7;
  // stage c from ring slot u: 2 + RW loads a thread in flight for each
  // later stage (LPT x pieces, 2 RW weights)
  auto stage = [&](int c, auto uv) {
    constexpr int u = decltype(uv)::value;
    wait_vmcnt<(LPT + 2 * RW) * (HT_S - 2)>();  // this thread's loads of stage c have landed
    lds_barrier();                              // everyone's are, and stage c - 1 is read
    issue(std::integral_constant<int, u + HT_S - 1>{}, c + HT_S - 1);
    const uint32_t st = xl + (uint32_t)(u * HT_STAGE);
    hv4 v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = lds_read16(st + 16u * (uint32_t)(i ^ sw));
    lgkm_wait(v);
    sfor<8>([&](auto iv) {
      constexpr int i = decltype(iv)::value, h = i / 4, n0 = 4 * (i % 4);
      const double xd[4] = {(double)v[i].x, (double)v[i].y, (double)v[i].z, (double)v[i].w};
      fmac_bc<n0>(acc, wq[u][h], xd[0]);
      fmac_bc<n0 + 1>(acc, wq[u][h], xd[1]);
      fmac_bc<n0 + 2>(acc, wq[u][h], xd[2]);
      fmac_bc<n0 + 3>(acc, wq[u][h], xd[3]);
    });
  };
  sfor<HT_S - 1>([&](auto kv) { issue(kv, kv.value); });
  // whole rounds of the ring, then the stages left
  int cb = 0;
  for (; cb + HT_S <= ns; cb += HT_S) sfor<HT_S>([&](auto uv) { stage(cb + uv.value, uv); });
  sfor<HT_S - 1>([&](auto uv) {
    if (cb + uv.value < ns) stage(cb + uv.value, uv);
  });
  wait_vmcnt<0>();  // the repeated loads past the last stage land before the workgroup ends
  if (lane < nt) {
#pragma unroll
    for (int j = 0; j < RW; j++) {
      const int r = wave + NW * j;
      if (r < nr) z[(size_t)(t0 + lane) * rows + r0 + r] = acc[j] + (double)b[r0 + r];
    }
  }
}

// Launches kern with min(work, the workgroups that fit on the device at
// once) workgroups of `threads`; the kernel strides over the rest.
template <typename Kern>
void launch_resident(Kern kern, int work, int threads, const RowArgs &a, hipStream_t s) {
  static int resident[64];  // per device; 0 until first asked
  int dev = 0;
  (void)hipGetDevice(&dev);
  int &n = resident[dev & 63];
  if (n == 0) {
    int per_cu = 0;
    (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)kern, threads, 0);
    n = std::max(1, device_cus() * per_cu);
  }
  kern<<<std::min(work, n), threads, 0, s>>>(a);
}

}  // namespace

void launch_rownorm(const RowArgs &a, hipStream_t s) {
  if (a.M <= 0) return;
  const int src = !a.ids ? 0 : a.emb_format == 0 ? 1 : a.emb_format == 1 ? 2 : 3;
  if ((a.lanes == 8 || a.lanes == 16) && a.H == 384 && a.seg != 0) {
    // a 256-column segment and a 128-column one
    const int rpw = 64 / a.lanes, groups = (a.M + rpw - 1) / rpw;
#define IXH_SEGH(VV)                                                                        \
  if (a.lanes == VV) {                                                                      \
    switch (src) {                                                                          \
    case 0: rownorm_seg_kernel<VV, 2, 0, true><<<groups, 64, 0, s>>>(a); return;           \
    case 1: rownorm_seg_kernel<VV, 2, 1, true><<<groups, 64, 0, s>>>(a); return;           \
    case 2: rownorm_seg_kernel<VV, 2, 2, true><<<groups, 64, 0, s>>>(a); return;           \
    default: rownorm_seg_kernel<VV, 2, 3, true><<<groups, 64, 0, s>>>(a); return;          \
    }                                                                                       \
  }
    IXH_SEGH(8) IXH_SEGH(16)
#undef IXH_SEGH
  }
  if (a.lanes > 0 && a.H % 256 == 0 && a.H <= 1024 && !(a.lanes == 4 && a.H > 768)) {
    const int V = a.lanes, cpl = a.H / 256, rpw = 64 / V;
    const int groups = (a.M + rpw - 1) / rpw;
#define IXH_LN(VV, CC)                                                                   \
  if (V == VV && cpl == CC) {                                                            \
    switch (src) {                                                                       \
    case 0: launch_resident(rownorm_lds_kernel<VV, CC, 0>, groups, 64, a, s); return;    \
    case 1: launch_resident(rownorm_lds_kernel<VV, CC, 1>, groups, 64, a, s); return;    \
    case 2: launch_resident(rownorm_lds_kernel<VV, CC, 2>, groups, 64, a, s); return;    \
    default: launch_resident(rownorm_lds_kernel<VV, CC, 3>, groups, 64, a, s); return;   \
    }                                                                                    \
  }
    // lanes 8 and 16: one wave per row group, rows in registers (8 KB of LDS)
#define IXH_SEG(VV, CC)                                                                  \
  if (V == VV && cpl == CC && seg) {                                                     \
    switch (src) {                                                                       \
    case 0: rownorm_seg_kernel<VV, CC, 0><<<groups, 64, 0, s>>>(a); return;             \
    case 1: rownorm_seg_kernel<VV, CC, 1><<<groups, 64, 0, s>>>(a); return;             \
    case 2: rownorm_seg_kernel<VV, CC, 2><<<groups, 64, 0, s>>>(a); return;             \
    default: rownorm_seg_kernel<VV, CC, 3><<<groups, 64, 0, s>>>(a); return;            \
    }                                                                                    \
  }
    const bool seg = a.seg != 0;  // 0: the whole-row LDS kernel
    IXH_SEG(8, 1) IXH_SEG(8, 2) IXH_SEG(8, 3) IXH_SEG(8, 4)
    IXH_SEG(16, 1) IXH_SEG(16, 2) IXH_SEG(16, 3) IXH_SEG(16, 4)
#undef IXH_SEG
    IXH_LN(4, 1) IXH_LN(4, 2) IXH_LN(4, 3)
    IXH_LN(8, 1) IXH_LN(8, 2) IXH_LN(8, 3) IXH_LN(8, 4)
    IXH_LN(16, 1) IXH_LN(16, 2) IXH_LN(16, 3) IXH_LN(16, 4)
#undef IXH_LN
  }
  const int tpr = a.lanes <= 0 ? 1 : a.lanes / 4;
  const long threads = (long)a.M * tpr;
  dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  switch (tpr) {
  case 1: rownorm_kernel<1><<<grid, block, 0, s>>>(a); break;
  case 2: rownorm_kernel<2><<<grid, block, 0, s>>>(a); break;
  case 4: rownorm_kernel<4><<<grid, block, 0, s>>>(a); break;
  }
}

void launch_quant_rows(const float *x, int ld, int M, int K, int8_t *q, int ldq, float *sa,
                       hipStream_t s) {
  if (M <= 0) return;
  const dim3 grid((M + 3) / 4);
  switch ((K + 255) / 256) {
  case 1: quant_rows_reg_kernel<1><<<grid, 256, 0, s>>>(x, ld, M, K, q, ldq, sa); break;
  case 2: quant_rows_reg_kernel<2><<<grid, 256, 0, s>>>(x, ld, M, K, q, ldq, sa); break;
  case 3: quant_rows_reg_kernel<3><<<grid, 256, 0, s>>>(x, ld, M, K, q, ldq, sa); break;
  case 4: quant_rows_reg_kernel<4><<<grid, 256, 0, s>>>(x, ld, M, K, q, ldq, sa); break;
  case 5: quant_rows_reg_kernel<5><<<grid, 256, 0, s>>>(x, ld, M, K, q, ldq, sa); break;
  case 6: quant_rows_reg_kernel<6><<<grid, 256, 0, s>>>(x, ld, M, K, q, ldq, sa); break;
  default: quant_rows_kernel<<<grid, 256, 0, s>>>(x, ld, M, K, q, ldq, sa); break;
  }
}

void launch_positions(const int32_t *offs, const int32_t *padoff, int B, int32_t *pos,
                      int32_t *slot, hipStream_t s) {
  if (B <= 0) return;
  positions_kernel<<<B, 256, 0, s>>>(offs, padoff, pos, slot);
}

void launch_pool(const float *xn, const int32_t *offs, int B, int N, int H, int cls, float *out,
                 hipStream_t s) {
  if (B <= 0) return;
  if (N / B <= 1024) {
    pool_kernel<<<dim3((H + 255) / 256, B), 256, 0, s>>>(xn, offs, H, cls, out);
    return;
  }
  constexpr int shm = PL_S * PL_STAGE;  // 128 KB
  static bool attr[64] = {};
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (!attr[dev & 63]) {
    (void)hipFuncSetAttribute((const void *)pool_ring_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, shm);
    attr[dev & 63] = true;
  }
  pool_ring_kernel<<<dim3((H + 63) / 64, B), 256, shm, s>>>(xn, offs, H, cls, out);
}

void launch_head_logits(const float *x, int T, int H, const double *w, const float *b, int rows,
                        double *z, hipStream_t s) {
  if (T <= 0 || rows <= 0) return;
  // up to 12 rows a workgroup: NW (2-4) waves of RW (1-3) rows, NW chosen
  // for the fewest chains computed (the larger NW on a tie); more rows take
  // more workgroups along y, each reading x again
  int nw = 4, rw = 3;
  if (rows < 12) {
    int best = 1 << 30;
    for (int n = 2; n <= 4; n++) {
      const int r = (rows + n - 1) / n;
      if (r <= 3 && n * r <= best) best = n * r, nw = n, rw = r;
    }
  }
  const int rg = std::min(rows, nw * rw);
  const dim3 grid((unsigned)((T + HT_T - 1) / HT_T), (unsigned)((rows + rg - 1) / rg));
  auto go = [&](auto rwc, auto nwc) {
    head_logits_kernel<decltype(rwc)::value, decltype(nwc)::value>
        <<<grid, 64 * decltype(nwc)::value, 0, s>>>(x, T, H, w, b, rows, rg, z);
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  using I4 = std::integral_constant<int, 4>;
  auto by_rw = [&](auto nwc) {
    switch (rw) {
      case 1: go(I1{}, nwc); break;
      case 2: go(I2{}, nwc); break;
      default: go(I3{}, nwc); break;
    }
  };
  switch (nw) {
    case 2: by_rw(I2{}); break;
    case 3: by_rw(I3{}); break;
    default: by_rw(I4{}); break;
  }
}

}  // namespace ixh
