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
//  * the per-channel constants (sb, gamma) vary with r and
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

// Dequantisation, ((f32(acc + 128*colsum) - zc) * sb) * sa, with sb in X
// form (the DPP folds into the v_mul_f32). The kernel runs only for
// weights whose every row has 127 * sum |w| + |128 * colsum| < 2^24 (the
// host checks on upload): then acc + 128*colsum is exact in float32 for
// any int8 activations, and so is its difference with zc = 128*colsum,
// which is acc — so f32(tile) - zc is f32(acc) bit for bit.
template <int R, int B = 0>
__device__ __forceinline__ float deqx(int acc, float sbx, float sa) {
  return ((float)acc * bcf<R, B>(sbx)) * sa;
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
  // Wi K steps in flight (the ring's slot of step kt is kt % PF1 across
  // tiles, so PF1 divides KT1)
  static constexpr int PF1 = KT1 % 3 == 0 ? 3 : 4;
  static constexpr int PF2 = 3;                    // WoMLP K steps in flight
  static constexpr int SWC = NW * 32;             // channels a stage of x: tile j of every wave
  static constexpr int XST = SWC + 8;              // floats a staged row (chains conflict-free)
  static constexpr int IN = BM * H;                // the input rows, fragment order
  static constexpr int SLOT = 2 * 16 * 64 * 4;     // one tile of g (64 tokens x 32 channels)
  static constexpr int PANEL = BM * I;
  static constexpr int XS = BM * XST * 4;
  static constexpr int SMEM = std::max(std::max(IN + SLOTS * SLOT, PANEL), (NJ > 1 ? 2 : 1) * XS);
  static_assert(H % 128 == 0 && I % 32 == 0, "shape: stages of whole 128-channel pieces");
  static_assert(KT1 >= PF1 && KT2 >= PF2 && KT1 % PF1 == 0, "prefetch depth");
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
  float *const xs = (float *)smem;         // R: stages of the rows [2][BM][XST]
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
      v[u] = __builtin_amdgcn_raw_buffer_load_b128(ars, (uint32_t)(tok * a.ldq + 16 * p), 0, kStreamPolicy);
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
  // gated tiles are dealt by wave (gw), the extra ones (NG % 8 != 0) to
  // waves 0 .. RT-1: a SIMD runs waves s and s + 4 and issues the older
  // one's instructions first (dealt to the younger wave instead, the extra
  // tile measured slower)
  const int gw = wave;
  const int ntile = (NG - gw + NW - 1) / NW;  // MAXT or MAXT - 1
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
  for (int s = 0; s < PF1; s++) loadW(gw, s, wq[s]);
  lds_barrier();  // the input fragments are in LDS

  float gh[HOLD][2][16];  // the wave's last HOLD tiles of g
  float gmx[2] = {0.f, 0.f};  // max |g| of this lane's two tokens
  // The GeGLU of a tile runs inside the next tile's K loop, a value or two
  // a K step, so that every wave issues MFMAs and VALU work together (one
  // wave alone issues VALU at about half the SIMD's rate, two waves
  // together at its full rate): pacc and psb hold the previous tile's
  // accumulators and column scales. Zero before the first tile: a wave
  // with MAXT - 1 tiles runs that GeGLU on zeros and stores nothing.
  v16i pacc[4] = {};
  float psba[2] = {0.f, 0.f}, psbb[2] = {0.f, 0.f};
  float pg[2][16];  // g of a tile bound for LDS, four values at a time
  // LDS slot of virtual tile k (k < MAXT - HOLD; the wave has it)
  auto slot_of = [&](int k) {
    return RT == 0 ? gw * SP + k : (gw < RT ? gw * SP + k : RT * SP + (gw - RT) * (SP - 1) + k - 1);
  };
  // GeGLU (GeluMul, vec_simd.go:125-160; every gated column takes the FMA
  // form: n_gelu == I) of value v of virtual tile KP: token block v / 16,
  // channel 16*fh + v % 16
  auto geglu_v = [&](auto kpv, auto vv) {
    constexpr int KP = decltype(kpv)::value, v = decltype(vv)::value, b = v / 16, r = v % 16;
    const float za = deqx<r, b>(pacc[b][r], psba[b], sa_t[b]);
    const float zb = deqx<r, b>(pacc[2 + b][r], psbb[b], sa_t[b]);
    const float g = gelu_fma(za) * zb;
    gmx[b] = amax(gmx[b], g);
    if constexpr (KP >= MAXT - HOLD) {
      gh[KP - (MAXT - HOLD)][b][r] = g;
    } else {
      pg[b][r] = g;
      if constexpr (r % 4 == 3) {
        // the wave's LDS slot: [b][r/4][64 lanes][4]
        if (KP >= skip)  // wave-uniform: the tile exists
          *(float4 *)(slot_s + slot_of(KP) * (S::SLOT / 4) + lane * 4 + (b * 4 + r / 4) * 256) =
              make_float4(pg[b][r - 3], pg[b][r - 2], pg[b][r - 1], pg[b][r]);
      }
    }
  };
  sfor<MAXT>([&](auto kv) {
    constexpr int k = decltype(kv)::value;
    if (k < skip) return;  // wave-uniform
    const int t = gw + NW * (k - skip);
    // column scales of the tile in X form (loaded before this tile's
    // refills: loads retire in order); token block 1 takes its own copy
    // (read at ca + dup, dup == 0 but opaque), so that each block's DPP
    // broadcasts fold into their uses instead of one v_mov_b32_dpp shared
    // by both
    const int ca = 64 * t + xi, cb = ca + 32;
    float sba[2], sbb[2];
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int o = b ? dup : 0;
      sba[b] = a.sbi[ca + o];
      sbb[b] = a.sbi[cb + o];
    }
    v16i acc[4];  // [GELU input | multiplier][token block]
    const int8_t *bp = in_s + lane * 16;
    v4i b0 = *(const v4i *)bp, b1 = *(const v4i *)(bp + 1024);
    sfor<KT1>([&](auto ktv) {
      constexpr int kt = decltype(ktv)::value;
      v4i n0 = b0, n1 = b1;
      if constexpr (kt + 1 < KT1) {
        n0 = *(const v4i *)(bp + (kt + 1) * 2048);
        n1 = *(const v4i *)(bp + (kt + 1) * 2048 + 1024);
      }
      const v4i *w = wq[kt % PF1];
      acc[0] = mfma32(w[0], b0, kt == 0 ? v16i{} : acc[0]);
      acc[1] = mfma32(w[0], b1, kt == 0 ? v16i{} : acc[1]);
      acc[2] = mfma32(w[1], b0, kt == 0 ? v16i{} : acc[2]);
      acc[3] = mfma32(w[1], b1, kt == 0 ? v16i{} : acc[3]);
      // this slot's next step: this tile's, else the next tile's
      if constexpr (kt + PF1 < KT1) loadW(t, kt + PF1, wq[kt % PF1]);
      else loadW(t + NW, kt + PF1 - KT1, wq[kt % PF1]);
      // the previous tile's GeGLU values of this step
      if constexpr (k >= 1) {
        sfor<32>([&](auto vv) {
          if constexpr (decltype(vv)::value * KT1 / 32 == kt) geglu_v(std::integral_constant<int, k - 1>{}, vv);
        });
      }
      b0 = n0;
      b1 = n1;
      __builtin_amdgcn_sched_barrier(0);  // keep the refill and the GeGLU values at their step
    });
#pragma unroll
    for (int q = 0; q < 4; q++) pacc[q] = acc[q];
#pragma unroll
    for (int b = 0; b < 2; b++) {
      psba[b] = sba[b];
      psbb[b] = sbb[b];
    }
  });
  // the last tile's GeGLU (every wave has virtual tile MAXT - 1)
  sfor<32>([&](auto vv) { geglu_v(std::integral_constant<int, MAXT - 1>{}, vv); });

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
    const int slot = slot_of(k);
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
    const int t = gw + NW * (k - skip);
#pragma unroll
    for (int b = 0; b < 2; b++) {
      v4i v;
      if constexpr (k >= MAXT - HOLD) v = qh[k - (MAXT - HOLD)][b];
      else v = qsp[k][b];
      *(v4i *)(panel + ((t * 2 + b) * 64 + lane) * 16) = v;
    }
  });
  lds_barrier();

  // The x rows move between HBM and LDS in stages of SWC channels (tile j
  // of every wave), a row's stage as whole 1 KB pieces: wave w loads rows
  // 8w .. 8w+7, lane l floats 4l .. 4l+3 (rows past M read 0). The first
  // two stages' loads are issued here, in flight during M, stage s + 2's
  // while stage s is processed: spread over the block, x's HBM traffic
  // does not come in one burst from every CU at once.
  const auto xrs = buf_rsrc(a.X + (size_t)m0 * H, (uint32_t)rows * H * 4);
  auto load_stage = [&](int s, v4i *dst) {
#pragma unroll
    for (int u = 0; u < 8; u++)
      dst[u] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (uint32_t)(((8 * wave + u) * H + SWC * s + 4 * lane) * 4), 0,
                                                     kStreamPolicy);
  };
  v4i xin[NJ > 1 ? 2 : 1][8];
  load_stage(0, xin[0]);
  if constexpr (NJ > 1) load_stage(1, xin[1]);

  // ---- M. WoMLP ----
  float sbo[NJ][2];
#pragma unroll
  for (int j = 0; j < NJ; j++)
#pragma unroll
    for (int b = 0; b < 2; b++) sbo[j][b] = a.sbo[32 * min(wave + NW * j, HT - 1) + xi + (b ? dup : 0)];
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
  // stage s lives in buffer s % NBUF of xs
  constexpr int NBUF = NJ > 1 ? 2 : 1;
  auto xsb = [&](int s) { return xs + (s % NBUF) * (BM * XST); };
  // the chains over the columns of stage s (pass 0: sums; 1: d*d)
  auto chains = [&](int s, int pass) {
    const int scw = min(SWC, H - SWC * s);  // channels of the stage (a multiple of 128)
    if constexpr (V > 0) {
#pragma unroll
      for (int u = 0; u < CPT; u++) {
        const int ch = tid + 512 * u;
        if (ch < NCH) {
          const float *xr = xsb(s) + (ch / V) * XST + ch % V;
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
      const float *xr = xsb(s) + tid * XST;
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
  // this wave's 16 values of stage s, token block b
  auto xs_own = [&](int s, int b) { return xsb(s) + (32 * b + fr) * XST + 32 * wave + 16 * fh; };
  auto put_own = [&](int s) {  // x of stage s from registers into its buffer
    if (wave + NW * s < HT) {
#pragma unroll
      for (int b = 0; b < 2; b++) {
        float *xo = xs_own(s, b);
#pragma unroll
        for (int q = 0; q < 4; q++)
          *(float4 *)(xo + 4 * q) = make_float4(x[s][b][4 * q], x[s][b][4 * q + 1], x[s][b][4 * q + 2], x[s][b][4 * q + 3]);
      }
    }
  };
  lds_barrier();  // every wave is past the panel (M)
  sfor<NJ>([&](auto sv) {
    constexpr int s = decltype(sv)::value;
    const int scw = min(SWC, H - SWC * s);
    const bool own = wave + NW * s < HT;  // wave-uniform: tile w + 8s exists
    // (the buffer's previous stage, s - 2, was read before stage s - 1's
    // barriers)
    float *const xb = xsb(s);
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (4 * lane < scw) *(v4i *)(xb + (8 * wave + u) * XST + 4 * lane) = xin[s % 2][u];
    if constexpr (s + 2 < NJ) load_stage(s + 2, xin[s % 2]);
    lds_barrier();
    if (own) {
      sfor<2>([&](auto bv) {
        constexpr int b = decltype(bv)::value;
        float *xo = xs_own(s, b);
        float4 v[4];
#pragma unroll
        for (int q = 0; q < 4; q++) v[q] = *(const float4 *)(xo + 4 * q);
        sfor<16>([&](auto rv) {
          constexpr int r = decltype(rv)::value;
          const float xv = r % 4 == 0 ? v[r / 4].x : r % 4 == 1 ? v[r / 4].y : r % 4 == 2 ? v[r / 4].z : v[r / 4].w;
          x[s][b][r] = xv + deqx<r, b>(acc[s][b][r], sbo[s][b], gs[b]);
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
        __builtin_amdgcn_raw_buffer_store_b128(*(const v4i *)(xb + (8 * wave + u) * XST + 4 * lane), xrs,
                                               (uint32_t)(((8 * wave + u) * H + SWC * s + 4 * lane) * 4), 0,
                                               kStreamPolicy);
    if constexpr (LN) chains(s, 0);
  });
  if constexpr (!LN) return;
  combine(0);
  // the variance pass, the stages again in column order: the last two are
  // still in their buffers, unless an earlier stage is written over one
  // (three stages: stage 0 goes over stage 2, which comes back after)
  if constexpr (NJ <= 2) {
    sfor<NJ>([&](auto sv) { chains(decltype(sv)::value, 1); });
  } else {
    static_assert(NJ == 3, "stages");
    lds_barrier();  // the sums' chains are past stage 2
    put_own(0);
    lds_barrier();
    chains(0, 1);
    chains(1, 1);
    lds_barrier();  // past stage 0's buffer
    put_own(2);
    lds_barrier();
    chains(2, 1);
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
          store_stream_16(a.Qk + ((size_t)c * a.qk_rows + m0 + tok) * 32 + 16 * fh, pk);
        else
          store_stream_16(a.Q + (size_t)(m0 + tok) * ldq + 32 * c + 16 * fh, pk);
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

// (the caller also checks that Wi and WoMLP hold the dequantisation bound
// above: Mat::small on the host)
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
