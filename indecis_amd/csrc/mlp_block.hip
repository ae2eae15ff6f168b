// mlp_block.hip — the encoder's whole MLP block in one kernel, 64 rows a
// workgroup, computed transposed: Wi + GeGLU, quantizeA of g, WoMLP
// accumulated into x, and the LayerNorm + quantizeA of the new x for the
// next layer's QKV.
//
// Replaces, per layer (infer.go:408-424): MatMul8N of the mlp_norm output
// by Wi (int8.go:89-155, VNNI tiles kernel_vnni_amd64.s) with GeluMul
// (vec_simd.go:125-160), quantizeA of g (int8.go:160-191), MatMul8N by
// WoMLP into x, then the next layer's attn_norm LayerNormRow + quantizeA
// (vec_simd.go:285-327, vec_scalar.go:66-81). Same arithmetic as
// mlp_res.hip: q*w summed in int32 by v_mfma_i32_32x32x32_i8, the reference
// tile rebuilt as acc + 128*colsum[n], ((f32(tile) - zc[n]) * sb[n]) *
// sa[m]; GELU in the FMA form; the LayerNorm's V float32 lane chains in
// column order combined in float64 in lane order.
//
// Why 64 rows: every Wi and WoMLP byte a workgroup reads from L2 serves
// its rows, and at 32 rows the weight traffic (2.65 MB a block at
// H 768, I 1152) bounds the block. The transposed products make the
// larger block fit: each MFMA takes the weights as its A operand (32
// channels) and the rows as its B operand (32 tokens), so an accumulator
// lane holds ONE token and 16 channels. With the weight fragment's rows
// dealt to lanes by perm32 (below), those are 16 consecutive channels,
// 16*(lane/32) + r, r = 0..15. Then
//  * a row's maximum is a lane's own maximum (plus its half-wave partner
//    and the other waves', through 2 KB of LDS);
//  * the quantised g of a lane, packed 4 values a dword, is already the
//    B operand of WoMLP for that token and K-block: the panel is written
//    and read as whole 16-byte fragments, no transpose;
//  * the per-channel constants (colsum, zc, sb, gamma) vary with r and
//    reach the lane by DPP row_newbcast folded into the VALU operation
//    that uses them, from one register a constant ("X form": lane i holds
//    channel (i % 16) + 16*(i / 32) of the tile).
//
// One workgroup of 8 waves, 64 rows, one a CU (2 waves a SIMD):
//  W. Wi + GeGLU: gated tile t (32 channels: Wi rows 64t .. 64t+31 for
//     the GELU input, 64t+32 .. for the multiplier, as interleaved on
//     upload) belongs to wave t % 8. Per K step, 2 weight fragments (PF1
//     steps ahead, across tiles) and the 2 token fragments from LDS (the
//     block's input rows staged K-blocked, fragment order), 4 MFMAs. After
//     the K loop the GeGLU runs on the 64 accumulators; the wave's last
//     HOLD tiles of g stay in registers, the earlier ones go to the
//     wave's own LDS slots (8 KB a tile). Each lane keeps max |g| of its
//     two tokens;
//  Q. the row maxima meet in LDS; each lane quantises its g (registers,
//     then its LDS slots) and writes the packed fragments to the panel
//     [I/32][2][64 lanes][16 B];
//  M. WoMLP: wave w owns output channel tiles w, w+8, w+16 (those below
//     H/32): A = WoMLP fragments (PF2 steps ahead), B = panel fragments;
//  R. dequantisation, the residual add and the store of x in registers
//     (16 consecutive floats a lane a tile); the LayerNorm chains over the
//     rows staged in LDS by channel ranges of SW columns (thread (row, l)
//     carrying lane partial l; V 0: one float64 chain a row); then o =
//     ((x - mean) * rstd) * gamma in registers, the row maxima through LDS,
//     the int8 row packed 16 bytes a lane, stored K-blocked or row-major.
// Without gamma (the last layer, whose final_norm writes float32) R stops
// after the residual. Rows past M read 0 and are never stored.
#include <algorithm>
#include <utility>

#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace mlp_block_impl {

constexpr int BM = 64;  // rows (tokens) of a workgroup
constexpr int NW = 8;   // waves

// The weight-fragment row that lane row i loads: D row i of the MFMA
// (8*(r/4) + 4*(lane/32) + r%4 for accumulator r) then holds channel
// 16*(lane/32) + r of the 32-channel group.
__device__ __forceinline__ int perm32(int i) { return 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3); }

// Lane n of each 16-lane row of v, broadcast to its row (DPP
// row_newbcast:n, gfx90a and later). With v in X form this is, in every
// lane, the constant of channel 16*(lane/32) + n. B selects one of two
// spellings of the same broadcast (mov_dpp, update_dpp) for the two token
// blocks: written once, the compiler shares one v_mov_b32_dpp between the
// blocks and can no longer fold it into either use; written twice, each
// folds into the VALU operation that uses it.
template <int N, int B = 0>
__device__ __forceinline__ int bci(int v) {
  if constexpr (B == 0) return __builtin_amdgcn_mov_dpp(v, 0x150 + N, 0xF, 0xF, true);
  else return __builtin_amdgcn_update_dpp(v, v, 0x150 + N, 0xF, 0xF, true);
}
template <int N, int B = 0>
__device__ __forceinline__ float bcf(float v) {
  return __int_as_float(bci<N, B>(__float_as_int(v)));
}

template <typename F, int... I>
__device__ __forceinline__ void sfor_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), in order
template <int N, typename F>
__device__ __forceinline__ void sfor(F &&f) {
  sfor_impl(f, std::make_integer_sequence<int, N>{});
}

// Dequantisation with the channel constants in X form (the DPP folds into
// v_add_u32, v_subrev_f32 and v_mul_f32: t + (-zc) is t - zc, signed zeros
// included).
template <int R, int B = 0>
__device__ __forceinline__ float deqx(int acc, int c1x, float zcx, float sbx, float sa) {
  return (((float)(acc + bci<R, B>(c1x)) + (-bcf<R, B>(zcx))) * bcf<R, B>(sbx)) * sa;
}

__device__ __forceinline__ int pack4(float a, float b, float c, float d, float inv) {
  const int q0 = q8(a, inv), q1 = q8(b, inv), q2 = q8(c, inv), q3 = q8(d, inv);
  return (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
}

template <int H, int I>
struct Shape {
  static constexpr int KT1 = H / 32;   // Wi K steps
  static constexpr int NG = I / 32;    // gated tiles
  static constexpr int KT2 = I / 32;   // WoMLP K steps
  static constexpr int HT = H / 32;    // output channel tiles
  static constexpr int MAXT = (NG + NW - 1) / NW;  // gated tiles of the busiest wave
  static constexpr int RT = NG % NW;               // waves with MAXT tiles (0: all)
  static constexpr int HOLD = MAXT < 3 ? MAXT : 3;  // tiles of g a wave keeps in registers
  static constexpr int SP = MAXT - HOLD;           // LDS slots of the busiest wave
  static constexpr int SLOTS = RT == 0 ? NW * SP : RT * SP + (NW - RT) * (SP > 0 ? SP - 1 : 0);
  static constexpr int NJ = (HT + NW - 1) / NW;    // output tiles of the busiest wave
  static constexpr int PF1 = 4;                    // Wi K steps in flight
  static constexpr int PF2 = 4;                    // WoMLP K steps in flight
  static constexpr int SWC = NW * 32;             // channels a stage of x: tile j of every wave
  static constexpr int XST = SWC + 8;              // floats a staged row (chains conflict-free)
  static constexpr int IN = BM * H;                // the input rows, fragment order
  static constexpr int SLOT = 2 * 16 * 64 * 4;     // one tile of g (64 tokens x 32 channels)
  static constexpr int PANEL = BM * I;
  static constexpr int XS = BM * XST * 4;
  static constexpr int SMEM = std::max(std::max(IN + SLOTS * SLOT, PANEL), XS);
  static_assert(H % 128 == 0 && I % 32 == 0, "shape: stages of whole 128-channel pieces");
  static_assert(KT1 >= PF1 && KT2 >= PF2, "prefetch depth");
  static_assert(SMEM <= 150 * 1024, "LDS");
};

template <int H, int I, int V, bool LN>
__global__ __launch_bounds__(512, 1) void mlp_block_kernel(MlpArgs a) {
  using S = Shape<H, I>;
  constexpr int KT1 = S::KT1, NG = S::NG, KT2 = S::KT2, HT = S::HT, MAXT = S::MAXT, RT = S::RT;
  constexpr int HOLD = S::HOLD, SP = S::SP, NJ = S::NJ, PF1 = S::PF1, PF2 = S::PF2;
  constexpr int SWC = S::SWC, XST = S::XST;
  extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
  int8_t *const in_s = smem;               // W: input fragments [KT1][2][64][16]
  float *const slot_s = (float *)(smem + S::IN);  // W, Q: spilled g tiles
  int8_t *const panel = smem;              // Q, M: [KT2][2][64][16]
  float *const xs = (float *)smem;         // R: a stage of the rows [BM][XST]
  __shared__ __attribute__((aligned(16))) float rmax_s[BM][NW];
  __shared__ float mean_s[BM], rstd_s[BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  const int xi = (lane & 15) + 16 * fh;  // X form: the channel this lane's constants hold
  const int M = a.M, m0 = blockIdx.x * BM;
  const int rows = min(M - m0, BM);
  const uint32_t bvo = (uint32_t)perm32(fr) * 32 + 16 * fh;  // lane offset in a weight fragment
  const int dup = __builtin_amdgcn_readfirstlane(M) >> 31;      // 0 (M >= 0), not known to be

  // ---- the block's input rows, K-blocked in fragment order: token 32b +
  // fr's bytes 32kt + 16h .. +15 at ((kt*2 + b)*64 + fr + 32h)*16 (rows
  // past M read 0) ----
  {
    constexpr int PCS = H / 16;  // 16-byte pieces a row
    const auto ars = buf_rsrc(a.Aq + (size_t)m0 * a.ldq, (uint32_t)rows * a.ldq);
    v4i v[BM * PCS / 512];
#pragma unroll
    for (int u = 0; u < BM * PCS / 512; u++) {
      const int idx = tid + 512 * u, tok = idx / PCS, p = idx - tok * PCS;
      v[u] = __builtin_amdgcn_raw_buffer_load_b128(ars, (uint32_t)(tok * a.ldq + 16 * p), 0, 0);
    }
#pragma unroll
    for (int u = 0; u < BM * PCS / 512; u++) {
      const int idx = tid + 512 * u, tok = idx / PCS, p = idx - tok * PCS;
      const int kt = p >> 1, h = p & 1, b = tok >> 5;
      *(v4i *)(in_s + ((kt * 2 + b) * 64 + (tok & 31) + 32 * h) * 16) = v[u];
    }
  }
  static_assert(BM * (H / 16) % 512 == 0, "input staging");
  // the two tokens of this lane: 32b + fr
  float sa_t[2];
#pragma unroll
  for (int b = 0; b < 2; b++) sa_t[b] = 32 * b + fr < rows ? a.sa[m0 + 32 * b + fr] : 0.f;

  // ---- W. Wi + GeGLU ----
  const int ntile = (NG - wave + NW - 1) / NW;  // MAXT or MAXT - 1
  const int skip = MAXT - ntile;                // virtual tiles this wave skips (0 or 1)
  const auto wrs = buf_rsrc(a.Bi, (uint32_t)KT1 * a.Npi * 32);
  // weight fragments of gated tile t, K step kt: the GELU-input rows and
  // the multiplier rows (past the last tile: other rows or zeros, unused)
  auto loadW = [&](int t, int kt, v4i *dst) {
    const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)(kt * a.Npi + 64 * t) * 32);
    dst[0] = __builtin_amdgcn_raw_buffer_load_b128(wrs, bvo, so, 0);
    dst[1] = __builtin_amdgcn_raw_buffer_load_b128(wrs, bvo + 1024, so, 0);
  };
  v4i wq[PF1][2];
#pragma unroll
  for (int s = 0; s < PF1; s++) loadW(wave, s, wq[s]);
  lds_barrier();  // the input fragments are in LDS

  float gh[HOLD][2][16];  // the wave's last HOLD tiles of g
  float gmx[2] = {0.f, 0.f};  // max |g| of this lane's two tokens
  sfor<MAXT>([&](auto kv) {
    constexpr int k = decltype(kv)::value;
    if (k < skip) return;  // wave-uniform
    const int t = wave + NW * (k - skip);
    // channel constants of the tile in X form (loaded before this tile's
    // refills: loads retire in order)
    const int ca = 64 * t + xi, cb = ca + 32;
    // token block 1 takes its own copy (read at ca + dup, dup == 0 but
    // opaque), so that each block's DPP broadcasts fold into their uses
    // instead of one v_mov_b32_dpp shared by both
    int c1a[2], c1b[2];
    float zca[2], sba[2], zcb[2], sbb[2];
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int o = b ? dup : 0;
      c1a[b] = a.c128i[ca + o];
      c1b[b] = a.c128i[cb + o];
      zca[b] = a.zci[ca + o];
      sba[b] = a.sbi[ca + o];
      zcb[b] = a.zci[cb + o];
      sbb[b] = a.sbi[cb + o];
    }
    v16i acc[4];  // [GELU input | multiplier][token block]
    const int8_t *bp = in_s + lane * 16;
    v4i b0 = *(const v4i *)bp, b1 = *(const v4i *)(bp + 1024);
#pragma unroll
    for (int kt = 0; kt < KT1; kt++) {
      v4i n0 = b0, n1 = b1;
      if (kt + 1 < KT1) {
        n0 = *(const v4i *)(bp + (kt + 1) * 2048);
        n1 = *(const v4i *)(bp + (kt + 1) * 2048 + 1024);
      }
      const v4i *w = wq[kt % PF1];
      acc[0] = mfma32(w[0], b0, kt == 0 ? v16i{} : acc[0]);
      acc[1] = mfma32(w[0], b1, kt == 0 ? v16i{} : acc[1]);
      acc[2] = mfma32(w[1], b0, kt == 0 ? v16i{} : acc[2]);
      acc[3] = mfma32(w[1], b1, kt == 0 ? v16i{} : acc[3]);
      // this slot's next step: this tile's, else the next tile's
      if (kt + PF1 < KT1) loadW(t, kt + PF1, wq[kt % PF1]);
      else loadW(t + NW, kt + PF1 - KT1, wq[kt % PF1]);
      b0 = n0;
      b1 = n1;
      __builtin_amdgcn_sched_barrier(0);
    }
    // GeGLU (GeluMul, vec_simd.go:125-160; every gated column takes the
    // FMA form: n_gelu == I) of token block b, channel 16*fh + r
    float g[2][16];
    sfor<2>([&](auto bv) {
      constexpr int b = decltype(bv)::value;
      sfor<16>([&](auto rv) {
        constexpr int r = decltype(rv)::value;
        const float za = deqx<r, b>(acc[b][r], c1a[b], zca[b], sba[b], sa_t[b]);
        const float zb = deqx<r, b>(acc[2 + b][r], c1b[b], zcb[b], sbb[b], sa_t[b]);
        g[b][r] = gelu_fma(za) * zb;
        gmx[b] = amax(gmx[b], g[b][r]);
      });
    });
    if constexpr (k >= MAXT - HOLD) {
#pragma unroll
      for (int b = 0; b < 2; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) gh[k - (MAXT - HOLD)][b][r] = g[b][r];
    } else {
      // the wave's LDS slot k - skip: [b][r/4][64 lanes][4]
      const int slot = RT == 0 ? wave * SP + k : (wave < RT ? wave * SP + k : RT * SP + (wave - RT) * (SP - 1) + k - 1);
      float *sp = slot_s + slot * (S::SLOT / 4) + lane * 4;
#pragma unroll
      for (int b = 0; b < 2; b++)
#pragma unroll
        for (int q = 0; q < 4; q++)
          *(float4 *)(sp + (b * 4 + q) * 256) = make_float4(g[b][4 * q], g[b][4 * q + 1], g[b][4 * q + 2], g[b][4 * q + 3]);
    }
  });

  // The x rows move between HBM and LDS in stages of SWC channels (tile j
  // of every wave), a row's stage as whole 1 KB pieces: wave w loads rows
  // 8w .. 8w+7, lane l floats 4l .. 4l+3 (rows past M read 0). Stage 0's
  // loads are issued here, ahead of Q and M, whose first waits they join.
  const auto xrs = buf_rsrc(a.X + (size_t)m0 * H, (uint32_t)rows * H * 4);
  auto load_stage = [&](int s, v4i *dst) {
#pragma unroll
    for (int u = 0; u < 8; u++)
      dst[u] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (uint32_t)(((8 * wave + u) * H + SWC * s + 4 * lane) * 4), 0, 0);
  };
  v4i xin[8];
  load_stage(0, xin);

  // WoMLP weight fragments of the first PF2 K steps (independent of g): in
  // flight during Q. Wave w's output tiles: c = w + NW*j (j < NJ, c < HT).
  const int npo = a.Npo;  // WoMLP rows a K-block (H padded on upload)
  const auto ors = buf_rsrc(a.Bo, (uint32_t)KT2 * npo * 32);
  auto loadM = [&](int kt, v4i *dst) {
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int c = min(wave + NW * j, HT - 1);  // past H/32: a valid tile, never used
      const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)(kt * npo + 32 * c) * 32);
      dst[j] = __builtin_amdgcn_raw_buffer_load_b128(ors, bvo, so, 0);
    }
  };
  v4i wm[PF2][NJ];
#pragma unroll
  for (int s = 0; s < PF2; s++) loadM(s, wm[s]);

  // ---- Q. quantizeA of g (int8.go:160-191) ----
#pragma unroll
  for (int b = 0; b < 2; b++) {
    const float m = fmax32(gmx[b], __shfl_xor(gmx[b], 32));
    if (fh == 0) rmax_s[32 * b + fr][wave] = m;
  }
  lds_barrier();  // every wave's maxima; every wave is past its K loops
  float gs[2], ginv[2];
#pragma unroll
  for (int b = 0; b < 2; b++) {
    const float4 p0 = *(const float4 *)&rmax_s[32 * b + fr][0], p1 = *(const float4 *)&rmax_s[32 * b + fr][4];
    float mx = fmax32(fmax32(fmax32(p0.x, p0.y), fmax32(p0.z, p0.w)), fmax32(fmax32(p1.x, p1.y), fmax32(p1.z, p1.w)));
    gs[b] = 0.f;
    ginv[b] = 0.f;
    if (mx != 0.f) {  // quantizeA: s = max/127, inv = 1/s (int8.go:175-183)
      gs[b] = mx / 127.0f;
      ginv[b] = 1.0f / gs[b];
    }
  }
  static_assert(NW == 8, "row maxima: two float4 a row");
  v4i qh[HOLD][2], qsp[SP > 0 ? SP : 1][2];
#pragma unroll
  for (int h = 0; h < HOLD; h++)
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int q = 0; q < 4; q++)
        qh[h][b][q] = pack4(gh[h][b][4 * q], gh[h][b][4 * q + 1], gh[h][b][4 * q + 2], gh[h][b][4 * q + 3], ginv[b]);
#pragma unroll
  for (int k = 0; k < SP; k++) {
    if (k < skip) continue;
    const int slot = RT == 0 ? wave * SP + k : (wave < RT ? wave * SP + k : RT * SP + (wave - RT) * (SP - 1) + k - 1);
    const float *sp = slot_s + slot * (S::SLOT / 4) + lane * 4;
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 v = *(const float4 *)(sp + (b * 4 + q) * 256);
        qsp[k][b][q] = pack4(v.x, v.y, v.z, v.w, ginv[b]);
      }
  }
  lds_barrier();  // every slot read: the panel goes over them
  // panel fragment (K-block t, token block b) at ((t*2 + b)*64 + lane)*16
  sfor<MAXT>([&](auto kv) {
    constexpr int k = decltype(kv)::value;
    if (k < skip) return;
    const int t = wave + NW * (k - skip);
#pragma unroll
    for (int b = 0; b < 2; b++) {
      v4i v;
      if constexpr (k >= MAXT - HOLD) v = qh[k - (MAXT - HOLD)][b];
      else v = qsp[k][b];
      *(v4i *)(panel + ((t * 2 + b) * 64 + lane) * 16) = v;
    }
  });
  lds_barrier();

  // ---- M. WoMLP ----
  int c1o[NJ][2];
  float zco[NJ][2], sbo[NJ][2];
#pragma unroll
  for (int j = 0; j < NJ; j++)
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int col = 32 * min(wave + NW * j, HT - 1) + xi + (b ? dup : 0);
      c1o[j][b] = a.c128o[col];
      zco[j][b] = a.zco[col];
      sbo[j][b] = a.sbo[col];
    }
  v16i acc[NJ][2];
  {
    const int8_t *pp = panel + lane * 16;
    v4i f0 = *(const v4i *)pp, f1 = *(const v4i *)(pp + 1024);
#pragma unroll
    for (int kt = 0; kt < KT2; kt++) {
      v4i n0 = f0, n1 = f1;
      if (kt + 1 < KT2) {
        n0 = *(const v4i *)(pp + (kt + 1) * 2048);
        n1 = *(const v4i *)(pp + (kt + 1) * 2048 + 1024);
      }
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        acc[j][0] = mfma32(wm[kt % PF2][j], f0, kt == 0 ? v16i{} : acc[j][0]);
        acc[j][1] = mfma32(wm[kt % PF2][j], f1, kt == 0 ? v16i{} : acc[j][1]);
      }
      if (kt + PF2 < KT2) loadM(kt + PF2, wm[kt % PF2]);
      f0 = n0;
      f1 = n1;
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- R. the reference tile, dequantised, added to x; the LayerNorm
  // chains ----
  // Stage s (channels SWC*s .. + SCW(s)): the rows come into xs (written as
  // loaded, 16 bytes a lane), each owning lane reads its 16 values (token
  // 32b + fr, channels 32w + 16fh + r of the stage), adds the dequantised
  // WoMLP result and writes them back; then the stage's rows go to HBM as
  // whole 1 KB pieces and the chains take its columns. Stage s + 1's loads
  // are in flight meanwhile. x keeps the new values for the variance pass
  // and the output.
  float x[NJ][2][16];
  // LayerNorm chains: V > 0: lane partial ch % V of row ch / V (thread t
  // carrying chains t + 512u); V 0: one float64 chain a row, threads 0..63
  constexpr int NCH = V > 0 ? BM * V : BM;
  constexpr int CPT = NCH > 512 ? NCH / 512 : 1;
  static_assert(V == 0 || NCH % 64 == 0, "chains: whole waves");
  float p[CPT], mean[CPT], rstd[CPT];
  double pd = 0.0;
#pragma unroll
  for (int u = 0; u < CPT; u++) p[u] = 0.f;
  // the chains over the columns of stage s in xs (pass 0: sums; 1: d*d)
  auto chains = [&](int s, int pass) {
    const int scw = min(SWC, H - SWC * s);  // channels of the stage (a multiple of 128)
    if constexpr (V > 0) {
#pragma unroll
      for (int u = 0; u < CPT; u++) {
        const int ch = tid + 512 * u;
        if (ch < NCH) {
          const float *xr = xs + (ch / V) * XST + ch % V;
          // NB reads issued before their NB adds (the sums stay in column
          // order)
          auto batch = [&](int e0, auto nb) {
            constexpr int NB = decltype(nb)::value;
            float bv[NB];
#pragma unroll
            for (int e = 0; e < NB; e++) bv[e] = xr[V * (e0 + e)];
            __builtin_amdgcn_sched_barrier(0);
            if (pass == 0) {
#pragma unroll
              for (int e = 0; e < NB; e++) p[u] = p[u] + bv[e];
            } else {
#pragma unroll
              for (int e = 0; e < NB; e++) {
                const float d = bv[e] - mean[u];
                p[u] = __builtin_fmaf(d, d, p[u]);
              }
            }
          };
          // 128 / V elements a 128-channel piece (V 4: 32, 8: 16, 16: 8)
          constexpr int NB = 128 / (V > 0 ? V : 1) < 16 ? 128 / (V > 0 ? V : 1) : 16;
          for (int e0 = 0; e0 < scw / V; e0 += NB) batch(e0, std::integral_constant<int, NB>{});
        }
      }
    } else if (tid < BM) {
      const float *xr = xs + tid * XST;
      if (pass == 0) {
        for (int e = 0; e < scw; e++) pd += (double)xr[e];
      } else {
        for (int e = 0; e < scw; e++) {
          const double d = (double)(xr[e] - mean[0]);
          pd += d * d;
        }
      }
    }
  };
  // the lane partials in float64, in lane order (vec_simd.go:294-297)
  auto combine = [&](int pass) {
#pragma unroll
    for (int u = 0; u < CPT; u++) {
      double sum = pd;
      if constexpr (V > 0) {
        sum = 0.0;
        const int base = lane & ~(V - 1);
#pragma unroll
        for (int t = 0; t < V; t++) sum += (double)__shfl(p[u], base + t);
      }
      if (pass == 0) {
        mean[u] = (float)(sum / (double)H);
        p[u] = 0.f;
      } else {
        rstd[u] = (float)(1.0 / __builtin_sqrt(sum / (double)H + a.eps));
      }
    }
    pd = 0.0;
  };
  // this wave's 16 values of stage s, token block b, in xs
  auto xs_own = [&](int b) { return xs + (32 * b + fr) * XST + 32 * wave + 16 * fh; };
#pragma unroll
  for (int s = 0; s < NJ; s++) {
    const int scw = min(SWC, H - SWC * s);
    const bool own = wave + NW * s < HT;  // wave-uniform: tile w + 8s exists
    lds_barrier();  // every wave is past the panel (M) or the previous stage's chains
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (4 * lane < scw) *(v4i *)(xs + (8 * wave + u) * XST + 4 * lane) = xin[u];
    if (s + 1 < NJ) load_stage(s + 1, xin);
    lds_barrier();
    if (own) {
      sfor<2>([&](auto bv) {
        constexpr int b = decltype(bv)::value;
        float *xo = xs_own(b);
        float4 v[4];
#pragma unroll
        for (int q = 0; q < 4; q++) v[q] = *(const float4 *)(xo + 4 * q);
        sfor<16>([&](auto rv) {
          constexpr int r = decltype(rv)::value;
          const float xv = r % 4 == 0 ? v[r / 4].x : r % 4 == 1 ? v[r / 4].y : r % 4 == 2 ? v[r / 4].z : v[r / 4].w;
          x[s][b][r] = xv + deqx<r, b>(acc[s][b][r], c1o[s][b], zco[s][b], sbo[s][b], gs[b]);
        });
#pragma unroll
        for (int q = 0; q < 4; q++)
          *(float4 *)(xo + 4 * q) = make_float4(x[s][b][4 * q], x[s][b][4 * q + 1], x[s][b][4 * q + 2], x[s][b][4 * q + 3]);
      });
    }
    lds_barrier();
    // the stage's new rows to HBM (rows past M dropped by the descriptor)
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (4 * lane < scw)
        __builtin_amdgcn_raw_buffer_store_b128(*(const v4i *)(xs + (8 * wave + u) * XST + 4 * lane), xrs,
                                               (uint32_t)(((8 * wave + u) * H + SWC * s + 4 * lane) * 4), 0, 0);
    if constexpr (LN) chains(s, 0);
  }
  if constexpr (!LN) return;
  combine(0);
  // the variance pass: the stages again, from x
#pragma unroll
  for (int s = 0; s < NJ; s++) {
    const bool own = wave + NW * s < HT;
    lds_barrier();  // the chains are past the previous stage
    if (own) {
#pragma unroll
      for (int b = 0; b < 2; b++) {
        float *xo = xs_own(b);
#pragma unroll
        for (int q = 0; q < 4; q++)
          *(float4 *)(xo + 4 * q) = make_float4(x[s][b][4 * q], x[s][b][4 * q + 1], x[s][b][4 * q + 2], x[s][b][4 * q + 3]);
      }
    }
    lds_barrier();
    chains(s, 1);
  }
  combine(1);
#pragma unroll
  for (int u = 0; u < CPT; u++) {
    const int ch = tid + 512 * u;
    const bool head = V > 0 ? (ch < NCH && ch % (V > 0 ? V : 1) == 0) : tid < BM;
    if (head) {
      const int row = V > 0 ? ch / (V > 0 ? V : 1) : tid;
      mean_s[row] = mean[u];
      rstd_s[row] = rstd[u];
    }
  }
  lds_barrier();

  // ---- o = ((x - mean) * rstd) * gamma and quantizeA of the row ----
  float gmv[NJ][2];
#pragma unroll
  for (int j = 0; j < NJ; j++)
#pragma unroll
    for (int b = 0; b < 2; b++) gmv[j][b] = a.gamma[32 * min(wave + NW * j, HT - 1) + xi + (b ? dup : 0)];
  float omx[2] = {0.f, 0.f};
  sfor<2>([&](auto bv) {
    constexpr int b = decltype(bv)::value;
    const float mu = mean_s[32 * b + fr], rs = rstd_s[32 * b + fr];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      if (wave + NW * j >= HT) continue;  // wave-uniform
      sfor<16>([&](auto rv) {
        constexpr int r = decltype(rv)::value;
        const float o = ((x[j][b][r] - mu) * rs) * bcf<r, b>(gmv[j][b]);
        x[j][b][r] = o;
        omx[b] = amax(omx[b], o);
      });
    }
  });
  // rmax_s again: every wave read the g maxima before the panel barrier
#pragma unroll
  for (int b = 0; b < 2; b++) {
    const float m = fmax32(omx[b], __shfl_xor(omx[b], 32));
    if (fh == 0) rmax_s[32 * b + fr][wave] = m;
  }
  lds_barrier();
  const int ldq = a.ldq;
#pragma unroll
  for (int b = 0; b < 2; b++) {
    const int tok = 32 * b + fr;
    const float4 p0 = *(const float4 *)&rmax_s[tok][0], p1 = *(const float4 *)&rmax_s[tok][4];
    const float mx = fmax32(fmax32(fmax32(p0.x, p0.y), fmax32(p0.z, p0.w)), fmax32(fmax32(p1.x, p1.y), fmax32(p1.z, p1.w)));
    float inv = 0.f;
    if (mx != 0.f) inv = 1.0f / (mx / 127.0f);  // quantizeA (int8.go:175-183)
    if (wave == 0 && fh == 0 && tok < rows) a.SA[m0 + tok] = mx != 0.f ? mx / 127.0f : 0.f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int c = wave + NW * j;
      if (c >= HT) continue;
      v4i pk;
#pragma unroll
      for (int q = 0; q < 4; q++) pk[q] = pack4(x[j][b][4 * q], x[j][b][4 * q + 1], x[j][b][4 * q + 2], x[j][b][4 * q + 3], inv);
      if (tok < rows) {
        if (a.Qk)  // K-blocked: 32-byte block c of row m0 + tok at (c * qk_rows + m0 + tok) * 32
          *(v4i *)(a.Qk + ((size_t)c * a.qk_rows + m0 + tok) * 32 + 16 * fh) = pk;
        else
          *(v4i *)(a.Q + (size_t)(m0 + tok) * ldq + 32 * c + 16 * fh) = pk;
      }
    }
  }
  if (!a.Qk && ldq > H) {
    for (int idx = tid; idx < BM * (ldq - H); idx += 512) {
      const int row = idx / (ldq - H), c = H + idx - row * (ldq - H);
      if (row < rows) a.Q[(size_t)(m0 + row) * ldq + c] = 0;
    }
  }
}

template <int H, int I, int V, bool LN>
void launch_one(const MlpArgs &a, hipStream_t s) {
  constexpr size_t shm = Shape<H, I>::SMEM;
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void *)mlp_block_kernel<H, I, V, LN>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    attr = true;
  }
  mlp_block_kernel<H, I, V, LN><<<(a.M + BM - 1) / BM, 512, shm, s>>>(a);
}

template <int H, int I, bool LN>
bool launch_v(const MlpArgs &a, int lanes, hipStream_t s) {
  switch (lanes) {
  case 0: launch_one<H, I, 0, LN>(a, s); return true;
  case 4: launch_one<H, I, 4, LN>(a, s); return true;
  case 8: launch_one<H, I, 8, LN>(a, s); return true;
  case 16: launch_one<H, I, 16, LN>(a, s); return true;
  default: return false;
  }
}

template <int H, int I>
bool launch_ln(const MlpArgs &a, int lanes, hipStream_t s) {
  return a.gamma ? launch_v<H, I, true>(a, lanes, s) : launch_v<H, I, false>(a, lanes, s);
}

}  // namespace mlp_block_impl

bool mlp_block_supported(int H, int I, int KpH, int KpI, int Npi) {
  if (KpH != H || KpI != I || Npi != 2 * I) return false;
  return (H == 768 && I == 1152) || (H == 384 && I == 1152) || (H == 256 && I == 512);
}

bool launch_mlp_block(const MlpArgs &a, int lanes, hipStream_t s) {
  using namespace mlp_block_impl;
  if (a.M <= 0) return true;
  if (!mlp_block_supported(a.H, a.I, a.H, a.I, a.Npi) || a.ldq < a.H || a.ldq % 16 != 0 || a.n_gelu < a.I ||
      a.Npo < a.H)
    return false;
  if (a.H == 768) return launch_ln<768, 1152>(a, lanes, s);
  if (a.H == 384) return launch_ln<384, 1152>(a, lanes, s);
  return launch_ln<256, 512>(a, lanes, s);
}

}  // namespace ixh
