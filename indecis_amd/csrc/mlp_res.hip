// mlp_res.hip — the encoder's whole MLP block in one kernel: Wi + GeGLU,
// quantizeA of g, WoMLP accumulated into x, and the LayerNorm +
// quantizeA of the new x for the next layer's QKV.
//
// Replaces, per layer (infer.go:408-424): MatMul8N of the mlp_norm output
// by Wi (int8.go:89-155, VNNI tiles kernel_vnni_amd64.s) with GeluMul
// (vec_simd.go:125-160), quantizeA of g (int8.go:160-191), MatMul8N by
// WoMLP into x, then the next layer's attn_norm LayerNormRow + quantizeA
// (vec_simd.go:285-327). Same arithmetic as gemm_as.hip (EPI_GEGLU) and
// gemm_res.hip: q*w summed in int32 by v_mfma_i32_32x32x32_i8, the
// reference tile rebuilt as acc + 128*colsum[n], ((f32(tile) - zc[n]) *
// sb[n]) * sa[m]; GELU in the FMA form on the columns below n_gelu, in
// the scalar form past them; the LayerNorm's V float32 lane chains in
// column order combined in float64 in lane order.
//
// One workgroup of 8 waves owns 32 rows from end to end, so g never leaves
// the CU (the separate kernels wrote it as float32 and read it back):
//  W. Wi + GeGLU: gated-column tile t (32 columns: Wi rows 64t .. 64t+31
//     for the GELU input, 64t+32 .. for the multiplier, as interleaved on
//     upload) belongs to wave t % 8. Weight fragments stream from the
//     K-blocked copy [H/32][2I][32] PF1 steps ahead across the wave's
//     tiles; A fragments come from the block's 32 input rows, staged in
//     LDS. g goes to LDS as float32 [32][I+4]; the input rows sit in the
//     columns of the last round of tiles, whose g waits in registers until
//     every wave is past its K loops;
//  Q. quantizeA of g: 16 threads a row read it into registers, max |g|
//     by a DPP reduction, q = RNE(g * (1/s)) written over g as an int8
//     panel [32][I] (16-byte chunks XOR-swizzled by row & 7 inside
//     128-byte groups), s kept in LDS;
//  M. WoMLP: wave w owns output columns QC*w .. QC*w + QC - 1 (QC = H/8)
//     as NB MFMA tiles, weight fragments from [I/32][H][32] PF2 steps
//     ahead, A fragments from the panel; meanwhile the block's x rows come
//     into LDS beside the panel by direct-to-LDS loads;
//  R. dequantisation and the residual add in the MFMA layout, into the
//     rows in LDS, written back as 16-byte pieces; the LayerNorm chains
//     over the same rows; then 16
//     threads a row: o = ((x - mean) * rstd) * gamma, max |o| by DPP, q8
//     packed into an int8 row in LDS, stored as 16-byte pieces.
// Without gamma (the last layer, whose final_norm writes float32) R stops
// after the residual. One workgroup a CU (LDS: g); rows past M read 0 and
// are never stored.
#include <algorithm>
#include <type_traits>

#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace mlp_res_impl {

constexpr int BM = 32;  // rows of a workgroup
constexpr int NW = 8;   // waves

template <int H, int I>
struct Shape {
  static constexpr int KT1 = H / 32;          // Wi K steps
  static constexpr int NG = I / 32;           // gated-column tiles
  static constexpr int KT2 = I / 32;          // WoMLP K steps
  static constexpr int NB = H / (32 * NW);    // WoMLP column tiles a wave
  static constexpr int QC = 32 * NB;          // columns a wave in M and R
  static constexpr int GLD = I + 4;           // floats a row of g in LDS
  static constexpr int XLD = H + 8;           // floats a staged row of x
  static constexpr int PF1 = 8;                     // Wi K steps in flight
  static constexpr int ACOL = 32 * (NG - NW);  // g column where the staged input rows sit
  static constexpr int PF2 = 4;                     // WoMLP K steps in flight
  // g; or the int8 panel of g (then the output rows) and x
  static constexpr int SMEM = std::max(BM * GLD * 4, BM * I + BM * XLD * 4);
  static_assert(BM * H <= BM * I, "output rows fit over the panel");
  static_assert(H % (32 * NW) == 0 && I % 64 == 0 && NG >= NW, "shape");
  // the staged input rows fit in the columns of tiles NG-NW .. NG-1: each
  // is its wave's last tile (tiles are dealt round-robin)
  static_assert(H <= 4 * 32 * NW, "staging");
  static_assert(KT1 % PF1 == 0 && KT2 % PF2 == 0, "prefetch depth");
};

// WO: the kernel for Wo instead (I = H): the block's float32 ctx rows are
// quantised into the panel (quantizeA, 16 threads a row) in place of W and
// Q; M and R are the same.
template <int H, int I, int V, bool LN, bool WO>
__global__ __launch_bounds__(512, 1) void mlp_res_kernel(MlpArgs a) {
  using S = Shape<H, I>;
  constexpr int KT1 = S::KT1, NG = S::NG, KT2 = S::KT2, NB = S::NB, QC = S::QC;
  constexpr int GLD = S::GLD, XLD = S::XLD, PF1 = S::PF1, PF2 = S::PF2, ACOL = S::ACOL;
  extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
  float *const gs = (float *)smem;  // W: g [BM][GLD]
  int8_t *const panel = smem;       // Q, M: quantised g [BM][I]
  float *const xs = (float *)(smem + BM * I);  // M, R: x [BM][XLD], past the panel
  int8_t *const qs = smem;                     // R: the int8 output rows [BM][H], over the panel
  __shared__ float sa_s[BM], sg_s[BM];
  __shared__ float mean_s[BM], rstd_s[BM];
  __shared__ __attribute__((aligned(16))) float gam_s[LN ? H : 4];  // LayerNorm weight
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  const int M = a.M, m0 = blockIdx.x * BM;
  const int rows = min(M - m0, BM);
  const uint32_t bvo = (uint32_t)fr * 32 + 16 * fh;  // lane offset in a weight fragment

  if (LN && tid < H / 4) *(float4 *)(gam_s + 4 * tid) = *(const float4 *)(a.gamma + 4 * tid);

  if constexpr (!WO) {
  // ---- W. Wi + GeGLU ----
  // weight fragments of step (k, kt): tile wave + NW k, K step kt
  const int ntile = (NG - wave + NW - 1) / NW;
  const auto wrs = buf_rsrc(a.Bi, (uint32_t)KT1 * a.Npi * 32);
  auto loadW = [&](int k, int kt, v4i *dst) {
    const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)(kt * a.Npi + 64 * (wave + NW * k)) * 32);
    dst[0] = __builtin_amdgcn_raw_buffer_load_b128(wrs, bvo, so, 0);
    dst[1] = __builtin_amdgcn_raw_buffer_load_b128(wrs, bvo + 1024, so, 0);
  };
  // the block's input rows (H bytes each, rows past M read 0) staged in
  // LDS where the last round of g tiles will go: row r at byte ACOL*4 of
  // g's row r. Every wave's last tile lies there; those g values wait in
  // registers until every wave is done with the rows.
  int8_t *const apan = (int8_t *)(gs + ACOL);
  {
    const auto ars = buf_rsrc(a.Aq + (size_t)m0 * a.ldq, (uint32_t)rows * a.ldq);
    const int ar = tid >> 4;
#pragma unroll
    for (int c = 0; c < H / 256; c++) {
      const int piece = (tid & 15) + 16 * c;  // 16-byte piece of the row
      *(v4i *)(apan + ar * GLD * 4 + 16 * piece) =
          __builtin_amdgcn_raw_buffer_load_b128(ars, (uint32_t)(ar * a.ldq + 16 * piece), 0, 0);
    }
  }
  if (tid < BM) sa_s[tid] = tid < rows ? a.sa[m0 + tid] : 0.f;
  // the first weight fragments, issued after the row loads (which the LDS
  // writes above wait for) so that they stay in flight across the barrier
  v4i bq[PF1][2];
#pragma unroll
  for (int s = 0; s < PF1; s++) loadW(0, s, bq[s]);
  lds_barrier();
  const int8_t *const afr = apan + fr * GLD * 4 + 16 * fh;  // this lane's A fragments: + 32 kt

  // the row scales of this lane's 16 accumulator rows
  float sav[16];
#pragma unroll
  for (int r = 0; r < 16; r++) sav[r] = sa_s[acc_row(r, lane)];

  // GeGLU (GeluMul, vec_simd.go:125-160; every gated column takes the FMA
  // form: n_gelu == I) of the previous tile, one accumulator row r at a
  // time, run inside the next tile's K loop so that its VALU work issues
  // while that tile's MFMAs execute
  v16i acc0, acc1, pacc0, pacc1;
  int pgc = 0, pc1a = 0, pc1b = 0;
  float pzca = 0.f, psba = 0.f, pzcb = 0.f, psbb = 0.f;
  auto geglu = [&](int r) {
    return gelu_fma(deq(pacc0[r] + pc1a, pzca, psba, sav[r])) * deq(pacc1[r] + pc1b, pzcb, psbb, sav[r]);
  };
  auto tile = [&](auto has_prev, int k) {
    constexpr bool PREV = decltype(has_prev)::value;
    // the tile's column constants, loaded before this tile's weight
    // refills: loads retire in order, so the wait for them leaves those
    // refills in flight
    const int t = wave + NW * k;
    const int ca = 64 * t + fr, cb = ca + 32;
    const int c1a = a.c128i[ca], c1b = a.c128i[cb];
    const float zca = a.zci[ca], sba = a.sbi[ca], zcb = a.zci[cb], sbb = a.sbi[cb];
    v4i fa = *(const v4i *)afr;
#pragma unroll
    for (int kt = 0; kt < KT1; kt++) {
      v4i fn = fa;
      if (kt + 1 < KT1) fn = *(const v4i *)(afr + 32 * (kt + 1));
      acc0 = mfma32(fa, bq[kt % PF1][0], kt == 0 ? v16i{} : acc0);
      acc1 = mfma32(fa, bq[kt % PF1][1], kt == 0 ? v16i{} : acc1);
      // this slot's next step: (k, kt + PF1), else the next tile's — past
      // the wave's last tile these read other weights (or, past the end
      // of the buffer, zeros) and are never used; no branch, so the waits
      // stay exact
      if (kt + PF1 < KT1) loadW(k, kt + PF1, bq[kt % PF1]);
      else loadW(k + 1, kt + PF1 - KT1, bq[kt % PF1]);
      if constexpr (PREV) {
#pragma unroll
        for (int r = 0; r < 16; r++)
          if (r * KT1 / 16 == kt) gs[acc_row(r, lane) * GLD + pgc] = geglu(r);
      }
      fa = fn;
      __builtin_amdgcn_sched_barrier(0);  // keep the refill at its step (PF1 steps in flight)
    }
    pacc0 = acc0;
    pacc1 = acc1;
    pgc = 32 * t + fr;
    pc1a = c1a;
    pc1b = c1b;
    pzca = zca;
    psba = sba;
    pzcb = zcb;
    psbb = sbb;
  };
  tile(std::false_type{}, 0);
  for (int k = 1; k < ntile; k++) tile(std::true_type{}, k);
  // the last tile's g waits in registers until every wave is done with the
  // staged rows
  float gv[16];
#pragma unroll
  for (int r = 0; r < 16; r++) gv[r] = geglu(r);
  lds_barrier();  // every wave is done with the staged rows
#pragma unroll
  for (int r = 0; r < 16; r++) gs[acc_row(r, lane) * GLD + pgc] = gv[r];
  }  // !WO

  // WoMLP weight fragments of the first PF2 K steps (independent of g): in
  // flight during Q
  const auto ors = buf_rsrc(a.Bo, (uint32_t)KT2 * H * 32);
  const int cw = wave * QC;  // first output column of this wave
  auto loadM = [&](int kt, v4i *dst) {
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)(kt * H + cw + 32 * j) * 32);
      dst[j] = __builtin_amdgcn_raw_buffer_load_b128(ors, bvo, so, 0);
    }
  };
  v4i bm[PF2][NB];
#pragma unroll
  for (int s = 0; s < PF2; s++) loadM(s, bm[s]);
  constexpr int CPR = H / 256;  // 1 KB pieces of an x row
  // the block's x rows, 1 KB pieces straight into LDS (xs, past the panel),
  // in flight through the rest of Q and the K loop — issued before the K
  // loop's weight refills, whose waits (loads retire in order) would
  // otherwise include these (rows past M load row M-1, never stored)
  auto load_x = [&] {
#pragma unroll
    for (int c = 0; c < BM * CPR / NW; c++) {
      const int q = wave + NW * c, row = q / CPR, part = q - row * CPR;
      const float *src = a.X + (size_t)(m0 + min(row, rows - 1)) * H + 256 * part + 4 * lane;
      __builtin_amdgcn_global_load_lds((glb_ptr)src, (lds_ptr)(xs + row * XLD + 256 * part), 16, 0, 0);
    }
  };
  if constexpr (WO) {
    // ---- Q. quantizeA of the ctx rows (int8.go:160-191) into the panel ----
    constexpr int QV = H / 64;  // float4 a thread
    const int qr = tid >> 4, qt = tid & 15;
    const float *arow = a.Af + (size_t)(m0 + min(qr, rows - 1)) * a.lda;  // rows past M: never stored
    float4 cv[QV];
#pragma unroll
    for (int c = 0; c < QV; c++) cv[c] = *(const float4 *)(arow + 4 * (qt + 16 * c));
    load_x();
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < QV; c++)
      mx = amax(amax(amax(amax(mx, cv[c].x), cv[c].y), cv[c].z), cv[c].w);
    mx = row16_max(mx);  // the row's 16 threads are one DPP row
    float s = 0.f, inv = 0.f;
    if (mx != 0.f) {  // quantizeA: s = max/127, inv = 1/s (int8.go:175-183)
      s = mx / 127.0f;
      inv = 1.0f / s;
    }
    if (qt == 0) sg_s[qr] = s;
    int8_t *prow = panel + qr * I;
#pragma unroll
    for (int c = 0; c < QV; c++) {
      const int i = 4 * (qt + 16 * c), ch = i >> 4;
      const int q0 = q8(cv[c].x, inv), q1 = q8(cv[c].y, inv), q2 = q8(cv[c].z, inv), q3 = q8(cv[c].w, inv);
      *(int *)(prow + 128 * (ch >> 3) + 16 * ((ch & 7) ^ (qr & 7)) + (i & 15)) =
          (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
    }
  } else {
  lds_barrier();  // g complete

  // ---- Q. quantizeA of g (int8.go:160-191) ----
  {
    constexpr int QV = I / 64;  // float4 a thread
    const int qr = tid >> 4, qt = tid & 15;
    float4 gv[QV];
#pragma unroll
    for (int c = 0; c < QV; c++) gv[c] = *(const float4 *)(gs + qr * GLD + 4 * (qt + 16 * c));
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < QV; c++)
      mx = amax(amax(amax(amax(mx, gv[c].x), gv[c].y), gv[c].z), gv[c].w);
    mx = row16_max(mx);  // the row's 16 threads are one DPP row
    float s = 0.f, inv = 0.f;
    if (mx != 0.f) {  // quantizeA: s = max/127, inv = 1/s (int8.go:175-183)
      s = mx / 127.0f;
      inv = 1.0f / s;
    }
    int pk[QV];
#pragma unroll
    for (int c = 0; c < QV; c++) {
      const int q0 = q8(gv[c].x, inv), q1 = q8(gv[c].y, inv), q2 = q8(gv[c].z, inv), q3 = q8(gv[c].w, inv);
      pk[c] = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
    }
    if (qt == 0) sg_s[qr] = s;
    lds_barrier();  // every thread holds its g: the panel goes over it
    load_x();       // g past the panel is dead now
    int8_t *prow = panel + qr * I;
#pragma unroll
    for (int c = 0; c < QV; c++) {
      const int i = 4 * (qt + 16 * c), ch = i >> 4;
      *(int *)(prow + 128 * (ch >> 3) + 16 * ((ch & 7) ^ (qr & 7)) + (i & 15)) = pk[c];
    }
  }
  }  // !WO
  lds_barrier();

  // ---- M. WoMLP ----
  // WoMLP column constants, loaded before the K loop's refills (see W)
  int c1o[NB];
  float zco[NB], sbo[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int col = cw + 32 * j + fr;
    c1o[j] = a.c128o[col];
    zco[j] = a.zco[col];
    sbo[j] = a.sbo[col];
  }
  v16i acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[j][r] = 0;
  {
    const int8_t *pa = panel + fr * I;
    auto loadA = [&](int kt) -> v4i {
      const int c = 2 * kt + fh;
      return *(const v4i *)(pa + 128 * (c >> 3) + 16 * ((c & 7) ^ (fr & 7)));
    };
    v4i f = loadA(0);
#pragma unroll
    for (int kt = 0; kt < KT2; kt++) {
      v4i fn = f;
      if (kt + 1 < KT2) fn = loadA(kt + 1);
#pragma unroll
      for (int j = 0; j < NB; j++) acc[j] = mfma32(f, bm[kt % PF2][j], acc[j]);
      if (kt + PF2 < KT2) loadM(kt + PF2, bm[kt % PF2]);
      f = fn;
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- R. the reference tile, dequantised, added to x in LDS ----
  wait_vmcnt<0>();  // this wave's x pieces landed
  lds_barrier();    // and every wave's
  {
    // every read issued before the first write: the compiler cannot tell
    // xs from the row scales, so read-add-write per element would wait on
    // LDS once per element
    float sgv[16], xv[NB][16];
#pragma unroll
    for (int r = 0; r < 16; r++) sgv[r] = sg_s[acc_row(r, lane)];
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) xv[j][r] = xs[acc_row(r, lane) * XLD + cw + 32 * j + fr];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        xs[acc_row(r, lane) * XLD + cw + 32 * j + fr] = xv[j][r] + deq(acc[j][r] + c1o[j], zco[j], sbo[j], sgv[r]);
  }
  lds_barrier();
  // x written back as 16-byte pieces of whole rows, every LDS read issued
  // before the first store
  {
    constexpr int WB = BM * (H / 4) / 512;  // pieces a thread
    static_assert(BM * (H / 4) % 512 == 0, "write-back");
    float4 wv[WB];
#pragma unroll
    for (int u = 0; u < WB; u++) {
      const int idx = tid + 512 * u, row = idx / (H / 4), c4 = idx - row * (H / 4);
      wv[u] = *(const float4 *)(xs + row * XLD + 4 * c4);
    }
#pragma unroll
    for (int u = 0; u < WB; u++) {
      const int idx = tid + 512 * u, row = idx / (H / 4), c4 = idx - row * (H / 4);
      if (row < rows) *(float4 *)(a.X + (size_t)(m0 + row) * H + 4 * c4) = wv[u];
    }
  }
  if constexpr (!LN) return;

  // LayerNorm chains over the rows in xs: V > 0: BM*V chains, thread t
  // carrying lane partial t % V of row t / V; V 0: one float64 chain a
  // row, threads 0..31
  constexpr int NCH = V > 0 ? BM * V : BM;
  static_assert(NCH <= 512 && (V == 0 || NCH % 64 == 0), "chains");
  const bool chain = tid < NCH;  // wave-uniform for V > 0
  const float *xr = V > 0 ? xs + (tid / (V > 0 ? V : 1)) * XLD + tid % (V > 0 ? V : 1) : xs + tid * XLD;
  float mean = 0.f, rstd = 0.f;
  {
    float p = 0.f;
    double pd = 0.0;
    if (chain) {
      if constexpr (V > 0) {
        // 16 reads issued before their 16 adds (the sums stay in column
        // order)
        for (int e0 = 0; e0 < H / V; e0 += 16) {
          float b[16];
#pragma unroll
          for (int u = 0; u < 16; u++) b[u] = xr[V * (e0 + u)];
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < 16; u++) p = p + b[u];
        }
      } else {
        for (int e = 0; e < H; e++) pd += (double)xr[e];
      }
    }
    // lane partials in float64, in lane order (vec_simd.go:294-297)
    double sum = pd;
    if constexpr (V > 0) {
      sum = 0.0;
      const int base = lane & ~(V - 1);
#pragma unroll
      for (int t = 0; t < V; t++) sum += (double)__shfl(p, base + t);
    }
    mean = (float)(sum / (double)H);
    p = 0.f;
    pd = 0.0;
    if (chain) {
      if constexpr (V > 0) {
        for (int e0 = 0; e0 < H / V; e0 += 16) {
          float b[16];
#pragma unroll
          for (int u = 0; u < 16; u++) b[u] = xr[V * (e0 + u)];
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < 16; u++) {
            const float d = b[u] - mean;
            p = __builtin_fmaf(d, d, p);
          }
        }
      } else {
        for (int e = 0; e < H; e++) {
          const double d = (double)(xr[e] - mean);
          pd += d * d;
        }
      }
    }
    double var = pd;
    if constexpr (V > 0) {
      var = 0.0;
      const int base = lane & ~(V - 1);
#pragma unroll
      for (int t = 0; t < V; t++) var += (double)__shfl(p, base + t);
    }
    rstd = (float)(1.0 / __builtin_sqrt(var / (double)H + a.eps));
  }
  if (chain && (V == 0 || tid % (V > 0 ? V : 1) == 0)) {
    const int row = V > 0 ? tid / (V > 0 ? V : 1) : tid;
    mean_s[row] = mean;
    rstd_s[row] = rstd;
  }
  lds_barrier();

  // o = ((x - mean) * rstd) * gamma and quantizeA of the row, from the
  // rows in xs: 16 threads a row (one DPP row), thread qt taking columns
  // 4(qt + 16c) .. +3; the int8 row goes to qs
  {
    constexpr int QV = H / 64;
    const int qr = tid >> 4, qt = tid & 15;
    const float mean = mean_s[qr], rstd = rstd_s[qr];
    const float *xrow = xs + qr * XLD;
    float4 o[QV];
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < QV; c++) {
      const int col = 4 * (qt + 16 * c);
      const float4 xv = *(const float4 *)(xrow + col), gv = *(const float4 *)(gam_s + col);
      o[c].x = ((xv.x - mean) * rstd) * gv.x;
      o[c].y = ((xv.y - mean) * rstd) * gv.y;
      o[c].z = ((xv.z - mean) * rstd) * gv.z;
      o[c].w = ((xv.w - mean) * rstd) * gv.w;
      mx = amax(amax(amax(amax(mx, o[c].x), o[c].y), o[c].z), o[c].w);
    }
    mx = row16_max(mx);
    float inv = 0.f;
    if (mx != 0.f) inv = 1.0f / (mx / 127.0f);  // quantizeA (int8.go:175-183)
#pragma unroll
    for (int c = 0; c < QV; c++) {
      const int q0 = q8(o[c].x, inv), q1 = q8(o[c].y, inv), q2 = q8(o[c].z, inv), q3 = q8(o[c].w, inv);
      *(int *)(qs + qr * H + 4 * (qt + 16 * c)) = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
    }
    if (qt == 0 && qr < rows) a.SA[m0 + qr] = mx != 0.f ? mx / 127.0f : 0.f;
  }
  lds_barrier();
  constexpr int C16 = H / 16;  // 16-byte pieces of a row
  if (a.Qk) {
    // K-blocked: 32-byte block kb of row r at (kb * qk_rows + m0 + r) * 32;
    // consecutive threads take consecutive rows of one block
    for (int idx = tid; idx < BM * C16; idx += 512) {
      const int kb = idx / (2 * BM), rem = idx - kb * 2 * BM, row = rem >> 1, p = rem & 1;
      if (row < rows)
        *(v4i *)(a.Qk + ((size_t)kb * a.qk_rows + m0 + row) * 32 + 16 * p) = *(const v4i *)(qs + row * H + 32 * kb + 16 * p);
    }
    return;
  }
  for (int idx = tid; idx < BM * C16; idx += 512) {
    const int row = idx / C16, c = idx - row * C16;
    if (row < rows) *(v4i *)(a.Q + (size_t)(m0 + row) * a.ldq + 16 * c) = *(const v4i *)(qs + row * H + 16 * c);
  }
  for (int idx = tid; idx < BM * (a.ldq - H); idx += 512) {
    const int row = idx / (a.ldq - H), c = H + idx - row * (a.ldq - H);
    if (row < rows) a.Q[(size_t)(m0 + row) * a.ldq + c] = 0;
  }
}

template <int H, int I, int V, bool LN, bool WO>
void launch_one(const MlpArgs &a, hipStream_t s) {
  constexpr size_t shm = Shape<H, I>::SMEM;
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void *)mlp_res_kernel<H, I, V, LN, WO>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    attr = true;
  }
  mlp_res_kernel<H, I, V, LN, WO><<<(a.M + BM - 1) / BM, 512, shm, s>>>(a);
}

template <int H, int I, bool LN, bool WO>
bool launch_v(const MlpArgs &a, int lanes, hipStream_t s) {
  switch (lanes) {
  case 0: launch_one<H, I, 0, LN, WO>(a, s); return true;
  case 4: launch_one<H, I, 4, LN, WO>(a, s); return true;
  case 8: launch_one<H, I, 8, LN, WO>(a, s); return true;
  case 16: launch_one<H, I, 16, LN, WO>(a, s); return true;
  default: return false;
  }
}

template <int H, int I>
bool launch_ln(const MlpArgs &a, int lanes, hipStream_t s) {
  return a.gamma ? launch_v<H, I, true, false>(a, lanes, s) : launch_v<H, I, false, false>(a, lanes, s);
}

// Every float x through both GELU forms, with gelu_div and gelu_clamp
// against IEEE division and the compare-select clamp: res[0] (FMA form),
// res[1] (scalar form) count the x whose results differ in any bit (a NaN
// result equals any NaN).
__global__ __launch_bounds__(256) void check_gelu_kernel(unsigned long long *res) {
  unsigned long long bf = 0, bs = 0;
  const unsigned long long stride = (unsigned long long)gridDim.x * 256u;
  for (unsigned long long i = blockIdx.x * 256ull + threadIdx.x; i < (1ull << 32); i += stride) {
    const float x = __uint_as_float((uint32_t)i);
    const float a = gelu_fma<true>(x), b = gelu_fma<false>(x);
    const float c = gelu_scalar<true>(x), d = gelu_scalar<false>(x);
    bf += __float_as_uint(a) != __float_as_uint(b) && !(a != a && b != b);
    bs += __float_as_uint(c) != __float_as_uint(d) && !(c != c && d != d);
  }
  for (int t = 1; t < 64; t <<= 1) {
    bf += __shfl_xor(bf, t);
    bs += __shfl_xor(bs, t);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&res[0], bf);
    atomicAdd(&res[1], bs);
  }
}

}  // namespace mlp_res_impl

void launch_check_gelu(unsigned long long *res, hipStream_t s) {
  mlp_res_impl::check_gelu_kernel<<<8192, 256, 0, s>>>(res);
}

bool mlp_res_supported(int H, int I, int KpH, int KpI, int Npi) {
  if (KpH != H || KpI != I || Npi != 2 * I) return false;
  return (H == 768 && I == 1152) || (H == 256 && I == 512);
}

bool wo_res_supported(int H, int KpH, int Np) { return KpH == H && Np == H && (H == 768 || H == 256); }

bool launch_wo_res(const MlpArgs &a, int lanes, hipStream_t s) {
  using namespace mlp_res_impl;
  if (a.M <= 0) return true;
  if (!wo_res_supported(a.H, a.H, a.H) || a.ldq < a.H || a.ldq % 16 != 0 || a.lda % 4 != 0 || !a.gamma) return false;
  if (a.H == 768) return launch_v<768, 768, true, true>(a, lanes, s);
  return launch_v<256, 256, true, true>(a, lanes, s);
}

bool launch_mlp_res(const MlpArgs &a, int lanes, hipStream_t s) {
  using namespace mlp_res_impl;
  if (a.M <= 0) return true;
  if (!mlp_res_supported(a.H, a.I, a.H, a.I, a.Npi) || a.ldq < a.H || a.ldq % 16 != 0 || a.n_gelu < a.I)
    return false;
  if (a.H == 768) return launch_ln<768, 1152>(a, lanes, s);
  return launch_ln<256, 512>(a, lanes, s);
}

}  // namespace ixh
