// gemm_res.hip — the encoder's residual GEMMs (Wo, WoMLP) fused with the
// quantisation of their input and the LayerNorm + quantisation of their
// output.
//
// Replaces, per residual GEMM: quantizeA of its input rows (ctx, or the
// GeGLU output; linalg/int8.go:160-191), MatMul8N accumulating into x
// (infer.go:403,423; int8.go:89-155, VNNI tiles kernel_vnni_amd64.s), and
// LayerNormRow + quantizeA of the new x for the next GEMM (mlp_norm before
// Wi, the next layer's attn_norm before QKV; vec_simd.go:285-327,
// vec_scalar.go:66-81). Same arithmetic as those kernels: q*w summed in
// int32 by v_mfma_i32_32x32x32_i8, the reference tile rebuilt as
// acc + 128*colsum[n], ((f32(tile) - zc[n]) * sb[n]) * sa[m] added to x;
// the LayerNorm's V float32 lane chains in column order, combined in
// float64 in lane order.
//
// One workgroup of 4 waves owns 32 rows whole (all H output columns), so
// every step that needs a whole row stays inside it and nothing goes back
// through HBM between the steps:
//  1. the input rows are read once as float32 (ctx [N][H] or g [N][I]),
//     max |a| per row by a wave reduction, q = RNE(a * (1/s)) written to
//     an LDS panel [32][Kp] (16-byte chunks XOR-swizzled by row & 7 inside
//     128-byte groups), s kept in LDS;
//  2. the K loop: wave w owns columns QC*w .. QC*w + QC - 1 (QC = H/4) as
//     NB = QC/32 MFMA tiles; its weight fragments stream from the K-blocked
//     weights [Kp/32][Np][32] (1 KB contiguous per MFMA operand) PF steps
//     ahead, A fragments come from the panel;
//  3. dequantisation and the residual add in the MFMA layout (x read and
//     written 128 contiguous bytes per half-wave);
//  4. the LayerNorm: the row's quarters, staged in LDS row-major one after
//     the other, pass under the chain threads — thread (r, l) carries lane
//     partial l of row r (lanes 0: one float64 chain a row) — once for the
//     sum, once for the fused d*d sum;
//  5. o = ((x - mean) * rstd) * gamma in the MFMA layout, max |o| per row
//     across the waves, q8(o, 1/s) staged as bytes, stored as 16-byte rows.
// Without gamma (the last layer, whose final_norm writes float32) steps 4
// and 5 are skipped.
//
// Streamed input (STREAM, when the kernel that wrote A also wrote maxima
// of |A| over parts of each row: attention per head, the GeGLU epilogue
// per 32 columns): step 1 only reads those maxima — quantizeA's max|a| is
// their max, exactly — and the K loop brings A in K step by K step
// (32 rows x 32 columns of float32, a float4 a thread, PA steps ahead),
// quantises it and writes it to a 3-stage LDS ring read by the MFMAs, one
// barrier a step. The input rows then stream from HBM while the MFMAs run
// instead of in a bulk load before them.
#include <algorithm>

#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace gemm_res_impl {

constexpr int BM = 32;  // rows of a workgroup
constexpr int PF = 2;   // K steps of weight fragments in flight
constexpr int PA = 12;  // K steps of streamed input in flight (STREAM)

// LDS: the input panel, then the LayerNorm's staged rows: two of the
// four column quarters at a time where two workgroups a CU still fit
// (78 KB each), else one
constexpr int panel_bytes(int KT, bool stream) { return stream ? 3 * BM * 32 : BM * 32 * KT; }
constexpr int quarters_staged(int KT, int NB, bool stream) {
  return panel_bytes(KT, stream) + BM * (2 * 32 * NB + 8) * 4 <= 78 * 1024 ? 2 : 1;
}
constexpr int smem_bytes(int KT, int NB, bool stream) {
  return panel_bytes(KT, stream) + BM * (quarters_staged(KT, NB, stream) * 32 * NB + 8) * 4;
}

template <int KT, int NB, int V, bool LN, bool STREAM>
__global__ __launch_bounds__(256, 2) void gemm_res_kernel(ResArgs a) {
  constexpr int Kp = 32 * KT;
  constexpr int QC = 32 * NB;     // columns of a wave
  constexpr int H = 4 * QC;
  constexpr int QPS = quarters_staged(KT, NB, STREAM);  // column quarters a stage
  constexpr int XLD = QPS * QC + 8;  // floats per staged row (conflict-free chains)
  constexpr int CPL = (Kp + 255) / 256;  // float4 a lane per input row
  constexpr int PANEL = panel_bytes(KT, STREAM);  // ring of 3 K steps, or the whole panel
  static_assert(BM * H <= BM * XLD * 4, "the int8 output rows fit over the staged rows");
  extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
  int8_t *const panel = smem;                        // [BM][Kp] or 3 x [BM][32]
  float *const xs = (float *)(smem + PANEL);         // [BM][XLD], then [BM][H] bytes
  __shared__ float sa_s[BM];
  __shared__ float red_s[4][BM];
  __shared__ float mean_s[BM], rstd_s[BM], inv_s[BM];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  const int m0 = blockIdx.x * BM;
  const int M = a.M;

  // ---- weight fragments of the first PF K steps (independent of A) ----
  const auto brs = buf_rsrc(a.Bk, (uint32_t)a.Np * Kp);
  const uint32_t bvo = (uint32_t)fr * 32 + 16 * fh;
  const int cb = wave * QC;  // first column of this wave
  v4i bq[PF][NB];
  // The K loop takes its K steps in a rotated order, the rotation by
  // workgroup (the int32 sums are exact in any order): the 512 workgroups
  // that start together then read different weight lines from L2 at a time
  // instead of all the same ones (189 -> 180 us a launch on cfg4). The
  // streamed input's ring stays in K order.
  const int rot = STREAM ? 0 : __builtin_amdgcn_readfirstlane((int)(blockIdx.x % KT));
  auto phys = [&](int kt) { const int k = kt + rot; return k >= KT ? k - KT : k; };
  auto loadB = [&](int kt, v4i *dst) {
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)(phys(kt) * a.Np + cb + 32 * j) * 32);
      dst[j] = __builtin_amdgcn_raw_buffer_load_b128(brs, bvo, so, 0);
    }
  };
#pragma unroll
  for (int s = 0; s < PF; s++) loadB(s, bq[s]);

  // streamed input: thread t loads columns 32kt + 4(t%8) .. +3 of row t/8
  const int ar = tid >> 3, ac = 4 * (tid & 7);
  const float *asrc = a.A + (size_t)min(m0 + ar, M - 1) * a.lda + ac;  // rows past M: never stored
  float4 av[STREAM ? PA : 1];
  if constexpr (STREAM) {
#pragma unroll
    for (int s = 0; s < PA; s++)
      if (s < KT) av[s] = *(const float4 *)(asrc + 32 * s);
  }

  float inv_r = 0.f;  // STREAM: 1/s of row ar
  if constexpr (STREAM) {
    // ---- 1. the row scales from the maxima of the row's parts ----
    if (tid < BM) {
      float mx = 0.f;
      if (m0 + tid < M) {
        const float *am = a.amax + (size_t)(m0 + tid) * a.P;
        for (int p = 0; p < a.P; p++) mx = __builtin_fmaxf(mx, am[p]);
      }
      float s = 0.f, inv = 0.f;
      if (mx != 0.f) {  // quantizeA: s = max/127, inv = 1/s (int8.go:175-183)
        s = mx / 127.0f;
        inv = 1.0f / s;
      }
      sa_s[tid] = s;
      red_s[0][tid] = inv;
    }
    __syncthreads();
    inv_r = red_s[0][ar];
  } else {
  // ---- 1. quantizeA of the 32 input rows into the LDS panel ----
  // wave w: rows 8w .. 8w+7, every load in flight at once (RB rows a
  // batch); lane: columns 4(lane + 64c)
  constexpr int RB = 8 * CPL <= 24 ? 8 : 4;
#pragma unroll
  for (int half = 0; half < 8 / RB; half++) {
    float4 v[RB][CPL];
#pragma unroll
    for (int u = 0; u < RB; u++) {
      const int row = min(m0 + 8 * wave + RB * half + u, M - 1);  // rows past M: never stored
      const float *src = a.A + (size_t)row * a.lda;
#pragma unroll
      for (int c = 0; c < CPL; c++) {
        const int i = 4 * (lane + 64 * c);
        v[u][c] = i < a.K ? load_stream_f4(src + i) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int u = 0; u < RB; u++) {
      float mx = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; c++)
        mx = amax(amax(amax(amax(mx, v[u][c].x), v[u][c].y), v[u][c].z), v[u][c].w);
      mx = wave_max(mx);
      float s = 0.f, inv = 0.f;
      if (mx != 0.f) {  // quantizeA: s = max/127, inv = 1/s (int8.go:175-183)
        s = mx / 127.0f;
        inv = 1.0f / s;
      }
      const int pr = 8 * wave + RB * half + u;
      int8_t *prow = panel + pr * Kp;
#pragma unroll
      for (int c = 0; c < CPL; c++) {
        const int i = 4 * (lane + 64 * c);
        if (i < Kp) {
          const int q0 = q8(v[u][c].x, inv), q1 = q8(v[u][c].y, inv);
          const int q2 = q8(v[u][c].z, inv), q3 = q8(v[u][c].w, inv);
          const int ch = i >> 4;
          *(int *)(prow + 128 * (ch >> 3) + 16 * ((ch & 7) ^ (pr & 7)) + (i & 15)) =
              (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
        }
      }
      if (lane == 0) sa_s[pr] = s;
    }
  }
  __syncthreads();
  }  // !STREAM

  // ---- 2. the K loop ----
  v16i acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[j][r] = 0;
  if constexpr (STREAM) {
    // ring stage s: [32 rows][32 bytes]; thread t writes its 4 bytes, lane
    // (fr, fh) of a wave reads row fr, bytes 16fh .. 16fh+15
    auto put = [&](int kt) {
      const float4 v = av[kt % PA];
      const int q0 = q8(v.x, inv_r), q1 = q8(v.y, inv_r), q2 = q8(v.z, inv_r), q3 = q8(v.w, inv_r);
      *(int *)(panel + (kt % 3) * (BM * 32) + ar * 32 + ac) =
          (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
      if (kt + PA < KT) av[kt % PA] = *(const float4 *)(asrc + 32 * (kt + PA));
    };
    put(0);
    lds_barrier();
#pragma unroll
    for (int kt = 0; kt < KT; kt++) {
      // stage kt+1 is free: its last readers (step kt-2) passed the
      // barrier of step kt-1
      if (kt + 1 < KT) put(kt + 1);
      const v4i fa = *(const v4i *)(panel + (kt % 3) * (BM * 32) + fr * 32 + 16 * fh);
#pragma unroll
      for (int j = 0; j < NB; j++) acc[j] = mfma32(fa, bq[kt % PF][j], acc[j]);
      if (kt + PF < KT) loadB(kt + PF, bq[kt % PF]);
      lds_barrier();  // stage kt+1 written by every thread
    }
  } else {
  const int8_t *pa = panel + fr * Kp;
  auto loadA = [&](int kt) -> v4i {
    const int c = 2 * phys(kt) + fh;
    return *(const v4i *)(pa + 128 * (c >> 3) + 16 * ((c & 7) ^ (fr & 7)));
  };
  v4i fa = loadA(0);
#pragma unroll
  for (int kt = 0; kt < KT; kt++) {
    v4i fn = fa;
    if (kt + 1 < KT) fn = loadA(kt + 1);
#pragma unroll
    for (int j = 0; j < NB; j++) acc[j] = mfma32(fa, bq[kt % PF][j], acc[j]);
    if (kt + PF < KT) loadB(kt + PF, bq[kt % PF]);
    fa = fn;
  }
  }  // !STREAM

  // ---- 3. the reference tile, dequantised, added to x ----
  // x through a descriptor over the block's rows (rows past M read 0 and
  // are not written); lane offset in the VGPR, the row offset of register r
  // (wave-uniform) in the SGPR; every load of the wave in flight at once
  const auto xrs = buf_rsrc(a.X + (size_t)m0 * H, (uint32_t)min(M - m0, BM) * H * 4);
  auto roff = [](int r) { return (uint32_t)((8 * (r >> 2) + (r & 3)) * H * 4); };
  float x[NB][16];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const uint32_t vo = (uint32_t)(4 * fh * H + cb + 32 * j + fr) * 4;
#pragma unroll
    for (int r = 0; r < 16; r++) x[j][r] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(xrs, vo, roff(r), kStreamPolicy));
  }
  // (with the weights' bound, checked on upload, f32(acc + 128 colsum) -
  // zc is f32(acc) exactly)
  const bool small = a.small;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int col = cb + 32 * j + fr;
    const int c1 = a.c128[col];
    const float zc = a.zc[col], sb = a.sb[col];
    const uint32_t vo = (uint32_t)(4 * fh * H + col) * 4;
    if (small) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float v = ((float)acc[j][r] * sb) * sa_s[acc_row(r, lane)];
        x[j][r] = x[j][r] + v;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(x[j][r]), xrs, vo, roff(r), kStreamPolicy);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float v = deq(acc[j][r] + c1, zc, sb, sa_s[acc_row(r, lane)]);
        x[j][r] = x[j][r] + v;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(x[j][r]), xrs, vo, roff(r), kStreamPolicy);
      }
    }
  }
  if constexpr (!LN) return;

  // ---- 4. LayerNorm chains, QPS quarters at a time ----
  // chains: V > 0: BM*V of them, thread t carrying chains t and t + 256
  // (V 16); chain ch is lane partial ch % V of row ch / V. V 0: one
  // float64 chain a row, threads 0..31.
  constexpr int NCH = V > 0 ? BM * V : BM;
  constexpr int CPT = NCH > 256 ? NCH / 256 : 1;
  auto stage = [&](int q) {
    if (wave >= q && wave < q + QPS) {
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) xs[acc_row(r, lane) * XLD + (wave - q) * QC + 32 * j + fr] = x[j][r];
    }
    __syncthreads();
  };
  float p[CPT], mean[CPT], rstd[CPT];
  double pd = 0.0;
#pragma unroll
  for (int k = 0; k < CPT; k++) p[k] = 0.f;
  for (int q = 0; q < 4; q += QPS) {
    stage(q);
    if constexpr (V > 0) {
#pragma unroll
      for (int k = 0; k < CPT; k++) {
        const int ch = tid + 256 * k;
        if (ch < NCH) {
          const float *xr = xs + (ch / V) * XLD + ch % V;
#pragma unroll
          for (int e = 0; e < QPS * QC / V; e++) p[k] = p[k] + xr[V * e];
        }
      }
    } else if (tid < BM) {
      const float *xr = xs + tid * XLD;
      for (int e = 0; e < QPS * QC; e++) pd += (double)xr[e];
    }
    __syncthreads();
  }
  // lane partials in float64, in lane order (vec_simd.go:294-297)
#pragma unroll
  for (int k = 0; k < CPT; k++) {
    double sum = pd;
    if constexpr (V > 0) {
      sum = 0.0;
      const int base = lane & ~(V - 1);
#pragma unroll
      for (int t = 0; t < V; t++) sum += (double)__shfl(p[k], base + t);
    }
    mean[k] = (float)(sum / (double)H);
    p[k] = 0.f;
  }
  pd = 0.0;
  for (int q = 0; q < 4; q += QPS) {
    stage(q);
    if constexpr (V > 0) {
#pragma unroll
      for (int k = 0; k < CPT; k++) {
        const int ch = tid + 256 * k;
        if (ch < NCH) {
          const float *xr = xs + (ch / V) * XLD + ch % V;
#pragma unroll
          for (int e = 0; e < QPS * QC / V; e++) {
            const float d = xr[V * e] - mean[k];
            p[k] = __builtin_fmaf(d, d, p[k]);
          }
        }
      }
    } else if (tid < BM) {
      const float *xr = xs + tid * XLD;
      for (int e = 0; e < QPS * QC; e++) {
        const double d = (double)(xr[e] - mean[0]);
        pd += d * d;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < CPT; k++) {
    double var = pd;
    if constexpr (V > 0) {
      var = 0.0;
      const int base = lane & ~(V - 1);
#pragma unroll
      for (int t = 0; t < V; t++) var += (double)__shfl(p[k], base + t);
    }
    rstd[k] = (float)(1.0 / __builtin_sqrt(var / (double)H + a.eps));
    const int ch = tid + 256 * k;
    const bool head = V > 0 ? (ch < NCH && ch % V == 0) : tid < BM;
    if (head) {
      const int row = V > 0 ? ch / V : tid;
      mean_s[row] = mean[k];
      rstd_s[row] = rstd[k];
    }
  }
  __syncthreads();

  // ---- 5. o = ((x - mean) * rstd) * gamma, quantizeA of the row ----
  float mx[16];
#pragma unroll
  for (int r = 0; r < 16; r++) mx[r] = 0.f;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const float g = a.gamma[cb + 32 * j + fr];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = acc_row(r, lane);
      const float o = ((x[j][r] - mean_s[row]) * rstd_s[row]) * g;
      x[j][r] = o;
      mx[r] = amax(mx[r], o);
    }
  }
  // a half-wave holds one row of each register: its max by DPP (lanes 16-31
  // and 48-63 get it)
#pragma unroll
  for (int r = 0; r < 16; r++) {
    mx[r] = halfwave_max(mx[r]);
    if (fr == 16) red_s[wave][acc_row(r, lane)] = mx[r];
  }
  __syncthreads();
  // the row's scale and its inverse, once a row (quantizeA: s = max/127,
  // inv = 1/s, int8.go:175-183)
  if (tid < BM) {
    const float m = __builtin_fmaxf(__builtin_fmaxf(red_s[0][tid], red_s[1][tid]), __builtin_fmaxf(red_s[2][tid], red_s[3][tid]));
    const float sc = m != 0.f ? m / 127.0f : 0.f;
    inv_s[tid] = m != 0.f ? 1.0f / sc : 0.f;
    if (m0 + tid < M) a.SA[m0 + tid] = sc;
  }
  __syncthreads();
  int8_t *const qs = (int8_t *)xs;  // [BM][H] bytes
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int row = acc_row(r, lane);
    const float inv = inv_s[row];
#pragma unroll
    for (int j = 0; j < NB; j++) qs[row * H + cb + 32 * j + fr] = (int8_t)q8(x[j][r], inv);
  }
  __syncthreads();
  constexpr int C16 = H / 16;  // 16-byte pieces of a row
  for (int idx = tid; idx < BM * C16; idx += 256) {
    const int row = idx / C16, c = idx - row * C16;
    if (m0 + row < M) store_stream_16(a.Q + (size_t)(m0 + row) * a.ldq + 16 * c, *(const v4i *)(qs + row * H + 16 * c));
  }
  for (int idx = tid; idx < BM * (a.ldq - H); idx += 256) {
    const int row = idx / (a.ldq - H), c = H + idx - row * (a.ldq - H);
    if (m0 + row < M) a.Q[(size_t)(m0 + row) * a.ldq + c] = 0;
  }
}

template <int KT, int NB, int V, bool LN, bool STREAM>
void launch_one(const ResArgs &a, hipStream_t s) {
  const size_t shm = smem_bytes(KT, NB, STREAM);
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void *)gemm_res_kernel<KT, NB, V, LN, STREAM>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    attr = true;
  }
  gemm_res_kernel<KT, NB, V, LN, STREAM><<<(a.M + BM - 1) / BM, 256, shm, s>>>(a);
}

template <int KT, int NB, bool LN, bool STREAM>
bool launch_v(const ResArgs &a, int lanes, hipStream_t s) {
  switch (lanes) {
  case 0: launch_one<KT, NB, 0, LN, STREAM>(a, s); return true;
  case 4: launch_one<KT, NB, 4, LN, STREAM>(a, s); return true;
  case 8: launch_one<KT, NB, 8, LN, STREAM>(a, s); return true;
  case 16: launch_one<KT, NB, 16, LN, STREAM>(a, s); return true;
  default: return false;
  }
}

template <int KT, int NB>
bool launch_ln(const ResArgs &a, int lanes, hipStream_t s) {
  if (a.amax)
    return a.gamma ? launch_v<KT, NB, true, true>(a, lanes, s) : launch_v<KT, NB, false, true>(a, lanes, s);
  return a.gamma ? launch_v<KT, NB, true, false>(a, lanes, s) : launch_v<KT, NB, false, false>(a, lanes, s);
}

}  // namespace gemm_res_impl

bool gemm_res_supported(int H, int Kp, int Np) {
  // (weight rows past H, padding of the K-blocked copy, are never read)
  if (Np < H || Np % 32 != 0) return false;
  return (H == 768 && (Kp == 768 || Kp == 1152)) || (H == 384 && (Kp == 384 || Kp == 1152)) ||
         (H == 256 && (Kp == 256 || Kp == 512));
}

bool launch_gemm_res(const ResArgs &a, int lanes, hipStream_t s) {
  using namespace gemm_res_impl;
  if (a.M <= 0) return true;
  if (!gemm_res_supported(a.H, a.Kp, a.Np) || a.K > a.Kp || a.K % 4 != 0 || a.ldq < a.H) return false;
  if (a.amax && (a.K != a.Kp || a.P <= 0 || a.lda % 4 != 0)) return false;
  if (a.H == 768) return a.Kp == 768 ? launch_ln<24, 6>(a, lanes, s) : launch_ln<36, 6>(a, lanes, s);
  if (a.H == 384) return a.Kp == 384 ? launch_ln<12, 3>(a, lanes, s) : launch_ln<36, 3>(a, lanes, s);
  return a.Kp == 256 ? launch_ln<8, 2>(a, lanes, s) : launch_ln<16, 2>(a, lanes, s);
}

}  // namespace ixh
