// qkv_attn.hip — the QKV projection fused with the attention prologue, for
// batches whose sequences have at most kQkvSeqMax keys.
//
// One workgroup per (sequence, head, Q|K|V) computes the 64 output columns
// of that head's Q, K or V over all rows of the sequence (the int8 GEMM of
// gemm_i8.hip: i8 MFMA, exact int32 sums, the reference's dequantisation,
// RoPE on Q and K) and finishes Attn8.Prepare (attention8.go:203-280) on
// them in place, so neither K nor V goes through HBM in float32:
//  Q: quantised per (row, head), 1/sqrt(D) folded into the scale
//     (attention8.go:211-220);
//  K: the float32 mean over the sequence — 64 sequential sums in key order
//     (AddTo, attention8.go:224-228) run by one wave over LDS slabs of 256
//     keys — then centred and quantised per key (attention8.go:240-251);
//  V: max |V| per dimension (MaxAbsTo, attention8.go:259-269), then
//     quantised per dimension and stored transposed (attention8.go:270-279).
// The outputs are those of the QKV GEMM (EPI_ROPE, queries) plus
// launch_attn_prologue: qq, sq, kp, ks, vt, vs, same layouts, same bits.
//
// Layout: NH halves of 8 waves, half f computing head NH*hp + f; in a
// half, 32-row block rb of the sequence (rb < 16) belongs to wave rb % 8,
// which holds it as 2 MFMA 32x32 tiles (the head's 64 columns). K steps of
// 64 stream A (the sequence's rows, up to 32 KB) and B (the NH heads' 64
// weight rows each, 4 KB a head) into an LDS ring with direct-to-LDS
// loads, as the GEMM does; every wave of the workgroup issues a share of
// the chunks. NH = 1: 512 threads, a 2-stage ring, two workgroups a CU.
// NH = 2: 1,024 threads, a 3-stage ring (two stages in flight), one
// workgroup a CU: each A row brought into LDS feeds two heads, so the
// sequence's rows are read 18 times instead of 36. Workgroups are dealt so
// that those of a sequence (12 heads x Q, K, V) run on one XCD and share
// its rows in L2; sequences go longest first, spread over the 8 XCDs.
//
// K-blocked input (GemmArgs::Ak, one head, KB): the rows come K-blocked,
// [Kp/32][rows][32], so a wave's A fragment (32 rows x 32 bytes) is 1 KB
// contiguous in HBM. The head's weight rows then stay in LDS for the whole
// K loop (64 rows x Kp bytes, K-blocked from the weights' K-blocked copy),
// and each wave streams its own row blocks' fragments into registers, PF
// K-blocks ahead: no ring, no barrier in the K loop, LDS read traffic of B
// only.
#include <type_traits>

#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace {

constexpr int D = 64, BK = 64, NXCD = 8;
constexpr int SEQ_MAX = kQkvSeqMax;           // 512 rows
constexpr int A_BYTES = SEQ_MAX * BK;         // A part of a stage
constexpr int KT_LD = 68;                     // floats per row of the Q/K slab
constexpr int SLAB_BYTES = 256 * KT_LD * 4;   // 256 keys
constexpr int VT_LD = 48;                     // bytes per dimension of the V^T staging tile

constexpr int cmax(int x, int y) { return x > y ? x : y; }
template <int NH>
struct Shape {
  static constexpr int NW = 8 * NH;                     // waves
  static constexpr int RING = NH == 1 ? 2 : 3;          // stages
  static constexpr int STAGE = A_BYTES + NH * D * BK;   // A + the heads' B rows
  // dynamic LDS: the ring, else one slab a half, the RoPE tables (8 KB a
  // wave) or the V^T tiles
  static constexpr int SMEM = cmax(cmax(RING * STAGE, NH * SLAB_BYTES), cmax(NW * 8192, NW * D * VT_LD));
};

// s_waitcnt vmcnt(n) for a wave-uniform n <= 3 (an immediate each).
__device__ __forceinline__ void wait_vmcnt_upto(int n) {
  if (n <= 0) wait_vmcnt<0>();
  else if (n == 1) wait_vmcnt<1>();
  else if (n == 2) wait_vmcnt<2>();
  else wait_vmcnt<3>();
}

template <int NH, bool KB>
__global__ __launch_bounds__(512 * NH, 4) void qkv_attn_kernel(GemmArgs g, AttnArgs a, const int32_t *order) {
  static_assert(!KB || NH == 1, "K-blocked input: one head a workgroup");
  using S = Shape<NH>;
  constexpr int NW = S::NW, RING = S::RING, STAGE = S::STAGE;
  extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
  __shared__ float sa_s[SEQ_MAX];
  __shared__ float red_s[NH][8][D];
  __shared__ __attribute__((aligned(16))) float stat_s[NH][D];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hf = wave >> 3, wv = wave & 7, tidh = tid & 511;  // half, wave and thread in the half
  const int fr = lane & 31, fh = lane >> 5;
  const int hgroups = a.nh / NH;
  const int per_seq = 3 * hgroups;
  const int xcd = blockIdx.x % NXCD, k = blockIdx.x / NXCD;
  const int si = xcd + NXCD * (k / per_seq);
  if (si >= a.B) return;
  const int b = order[si];
  const int part = (k % per_seq) / hgroups, h0 = NH * ((k % per_seq) % hgroups), h = h0 + hf;
  const int base = a.offs[b], n = a.offs[b + 1] - base;
  const int slot0 = a.padoff[b];  // the sequence's first key slot (K and V outputs)
  const int npad = (n + kKeyPad - 1) / kKeyPad * kKeyPad;
  const int nb = npad / 32;            // 32-row blocks stored (even, at most 16)
  const int nbc = (n + 31) / 32;       // blocks computed: a block past n is all zeros
  const int col0 = part * a.H + h * D;   // this half's head: first output column
  const int colb = part * a.H + h0 * D;  // the workgroup's first weight row
  if (n == 0) {
    if (part == 2 && tidh < D) a.vs[((size_t)b * a.nh + h) * D + tidh] = 0.f;
    return;
  }
  // Loads the K loop does not need, issued before its first stage (loads
  // retire in order, so the loop's first wait covers them): the row scales
  // (stored to LDS after the loop) and this lane's column constants.
  static_assert(SEQ_MAX <= 512, "one row scale a thread");
  const float sa_v = tid < 32 * nb ? g.sa[base + min(tid, n - 1)] : 0.f;
  float zc[2], sb[2];
  int c128[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int nc = col0 + 32 * j + fr;
    zc[j] = g.zc[nc];
    sb[j] = g.sb[nc];
    c128[j] = g.c128[nc];
  }

  // ---- int8 GEMM of the sequence's rows by the head's 64 weight rows ----
  // Stage chunks of 16 rows x 64 bytes (one wave instruction each): A
  // chunks 0 .. 2nbc-1 (rows past n load row n-1, never stored), then the
  // 4 NH B chunks (head f's at A_BYTES + f * 64 rows); chunk q is loaded by
  // wave q % NW. Lane i fills 16 bytes of its chunk: row i/4, physical
  // 16-byte column i%4 (logical (i%4) ^ swz).
  const int lrow = lane >> 2, lchunk = (lane & 3) ^ swz(lane >> 2);
  const int nchunk = 2 * nbc + 4 * NH;
  // This wave's chunks q = wave + NW c (c < nch <= MAXCH, wave-uniform):
  // the source of each lane and the LDS offset in a stage, computed once;
  // a K step then only adds kt * BK.
  constexpr int MAXCH = (2 * (SEQ_MAX / 32) + 4 * NH + NW - 1) / NW;
  static_assert(MAXCH <= 3 || RING == 2, "wait_vmcnt_upto covers 3 chunks a stage");
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int wv_u = wave_u & 7;
  const int nch = wave_u < nchunk ? (nchunk - wave_u + NW - 1) / NW : 0;
  const int8_t *csrc[MAXCH];
  int cdst[MAXCH];
#pragma unroll
  for (int c = 0; c < MAXCH; c++) {
    const int q = wave_u + NW * c;
    if (q < 2 * nbc) {
      const int row = min(16 * q + lrow, n - 1);
      csrc[c] = g.A + (size_t)(base + row) * g.lda + 16 * lchunk;
      cdst[c] = 16 * q * BK;
    } else {
      const int qb = min(q - 2 * nbc, 4 * NH - 1);  // c >= nch: never issued
      csrc[c] = g.B + (size_t)(colb + 16 * qb + lrow) * g.ldb + 16 * lchunk;
      cdst[c] = A_BYTES + 16 * qb * BK;
    }
  }
  auto issue = [&](int kt) {
    int8_t *st = smem + (kt % RING) * STAGE;
#pragma unroll
    for (int c = 0; c < MAXCH; c++)
      if (c < nch)
        __builtin_amdgcn_global_load_lds((glb_ptr)(csrc[c] + kt * BK), (lds_ptr)(st + cdst[c]), 16, 0, 0);
  };

  // (the K-blocked loop starts its sums from the MFMAs' zero operand)
  v16i acc[2][2];
  if constexpr (!KB) {
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
  }

  if constexpr (KB) {
    // the head's weight rows, resident: K-block kb's column tile j as 1 KB
    // at smem + 1024 (2 kb + j), lane l of a fragment at 16 l (row l % 32,
    // bytes 16 (l / 32) of the block), loaded as such by chunk q = 2 kb + j
    const int nkb = g.Kp / 32;
    for (int q = wave_u; q < 2 * nkb; q += NW) {
      const int8_t *src = g.Bk + ((size_t)(q >> 1) * g.Np + colb + 32 * (q & 1) + fr) * 32 + 16 * fh;
      __builtin_amdgcn_global_load_lds((glb_ptr)src, (lds_ptr)(smem + 1024 * q), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // the A loads below stay younger than these
    // this lane's A rows in K-block 0 (rows past n: row n-1, never
    // stored), a K-block further on every ak_rows rows: the lane's byte
    // offsets in the VGPRs, the K-block's in an SGPR (no address
    // arithmetic a load)
    constexpr int PF = 4;  // K-blocks in flight (nkb is a multiple of 4)
    const auto ars = buf_rsrc(g.Ak, (uint32_t)nkb * g.ak_rows * 32);
    uint32_t avo[2];
#pragma unroll
    for (int i = 0; i < 2; i++) avo[i] = (uint32_t)(base + min(32 * (wv_u + 8 * i) + fr, n - 1)) * 32 + 16 * fh;
    const uint32_t akstep = (uint32_t)g.ak_rows * 32;
    const bool two = wv_u + 8 < nbc;  // this wave's second row block
    // Both row blocks' fragments are loaded every K-block, past the last
    // K-block the last one again, whether or not the wave has a second
    // block (then row n-1: one 32-byte piece): with a load count that does
    // not depend on the wave or the step, the compiler waits for exactly
    // the fragment it needs, not for every load in flight.
    v4i fa[PF][2];
    auto loadA = [&](int kb, v4i *dst) {
      const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)min(kb, nkb - 1) * akstep);
      dst[0] = __builtin_amdgcn_raw_buffer_load_b128(ars, avo[0], so, 0);
      dst[1] = __builtin_amdgcn_raw_buffer_load_b128(ars, avo[1], so, 0);
    };
#pragma unroll
    for (int u = 0; u < PF; u++) loadA(u, fa[u]);
    wait_vmcnt<2 * PF>();  // this wave's weight chunks (older than its 2 PF A loads)
    __builtin_amdgcn_s_barrier();  // every wave's weight chunks are in LDS
    // PF K-blocks from k0; the first round's first K-block starts the sums
    auto round = [&](int k0, auto first) {
#pragma unroll
      for (int u = 0; u < PF; u++) {
        const int kb = k0 + u;
        const bool z = decltype(first)::value && u == 0;
        v4i fb[2];
#pragma unroll
        for (int j = 0; j < 2; j++) fb[j] = *(const v4i *)(smem + 1024 * (2 * kb + j) + 16 * lane);
#pragma unroll
        for (int j = 0; j < 2; j++) acc[0][j] = mfma32(fa[u][0], fb[j], z ? v16i{} : acc[0][j]);
        if (two) {
#pragma unroll
          for (int j = 0; j < 2; j++) acc[1][j] = mfma32(fa[u][1], fb[j], z ? v16i{} : acc[1][j]);
        }
        loadA(kb + PF, fa[u]);
      }
    };
    if (wv_u < nbc) {
      round(0, std::true_type{});
      for (int k0 = PF; k0 < nkb; k0 += PF) round(k0, std::false_type{});
    }
  } else {
  const int nk = g.Kp / BK;
  issue(0);
  if (RING > 2 && nk > 1) issue(1);
  for (int kt = 0; kt < nk; kt++) {
    // this step's loads landed (loads retire in order: at most the next
    // stage's nch are still in flight), every wave's too after the
    // barrier, which also ends every wave's reads of the stage issued next
    if (RING > 2 && kt + 1 < nk) wait_vmcnt_upto(nch);
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (kt + RING - 1 < nk) issue(kt + RING - 1);
    const int8_t *st = smem + (kt % RING) * STAGE;
#pragma unroll
    for (int s = 0; s < 2; s++) {
      v4i fb[2];
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int row = 64 * hf + 32 * j + fr;
        fb[j] = *(const v4i *)(st + A_BYTES + row * BK + 16 * ((2 * s + fh) ^ swz(row)));
      }
#pragma unroll
      for (int i = 0; i < 2; i++) {
        if (wv_u + 8 * i < nbc) {
          const int row = 32 * (wv_u + 8 * i) + fr;
          const v4i fa = *(const v4i *)(st + row * BK + 16 * ((2 * s + fh) ^ swz(row)));
#pragma unroll
          for (int j = 0; j < 2; j++) acc[i][j] = mfma32(fa, fb[j], acc[i][j]);
        }
      }
    }
  }
  }  // !KB
  if (tid < 32 * nb) sa_s[tid] = sa_v;
  __syncthreads();  // the ring is no longer read; the row scales are in LDS

  // ---- dequantisation (and RoPE on Q and K) in the MFMA layout ----
  // lane: columns fr and 32 + fr of the head, rows 32 rb + acc_row(r)
  // RoPE tables (cos, sin: 32 floats a position; a row's position is its
  // index in the sequence, padding rows n-1) of a block's 32 rows, staged
  // into this wave's 8 KB of the free ring by 8 direct-to-LDS loads: the
  // first block's issued before the dequantisation of both blocks, the
  // second's once the first block's are read
  float v[2][2][16];
  const bool rope = part < 2;
  const float *tab = (const float *)(smem + wave * 8192);
  auto tables = [&](int i) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int p = min(32 * (wv + 8 * i) + 8 * u + (lane >> 3), n - 1);
      const size_t off = (size_t)p * 32 + 4 * (lane & 7);
      __builtin_amdgcn_global_load_lds((glb_ptr)(g.rope_cos + off), (lds_ptr)(smem + wave * 8192 + 1024 * u), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((glb_ptr)(g.rope_sin + off), (lds_ptr)(smem + wave * 8192 + 4096 + 1024 * u), 16, 0, 0);
    }
  };
  if (rope && wv < nbc) tables(0);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    // a block past n (stored as padding keys) is not computed: its values
    // reach only rows past n, which every store below writes as zeros
    if (wv + 8 * i >= nbc) continue;
    if (g.small) {
      // the weights' bound holds (checked on upload): f32(acc + 128
      // colsum) - zc is f32(acc) exactly
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float sa = sa_s[32 * (wv + 8 * i) + acc_row(r, lane)];
        v[i][0][r] = ((float)acc[i][0][r] * sb[0]) * sa;
        v[i][1][r] = ((float)acc[i][1][r] * sb[1]) * sa;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float sa = sa_s[32 * (wv + 8 * i) + acc_row(r, lane)];
        v[i][0][r] = deq(acc[i][0][r] + c128[0], zc[0], sb[0], sa);
        v[i][1][r] = deq(acc[i][1][r] + c128[1], zc[1], sb[1], sa);
      }
    }
  }
  if (rope) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      if (wv + 8 * i >= nbc) continue;
      if (i == 1) {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt 0: this wave's reads of the first tables returned
        tables(1);
      }
      wait_vmcnt<0>();
#pragma unroll
      for (int r = 0; r < 16; r++) {
        // linalg.Rope (vec_simd.go:408-425): x1' = x1*c - x2*s, x2' = x2*c + x1*s
        const float c = tab[acc_row(r, lane) * 32 + fr], sn = tab[1024 + acc_row(r, lane) * 32 + fr];
        const float x1 = v[i][0][r], x2 = v[i][1][r];
        v[i][0][r] = x1 * c - x2 * sn;
        v[i][1][r] = x2 * c + x1 * sn;
      }
    }
  }
  __syncthreads();  // every wave is done with its tables: the ring is free again

  if (part == 2) {
    // ---- V: max |V| per dimension, scale, quantCols, V^T ----
    float vm[2] = {0.f, 0.f};
    // every row of a computed block: the rows past n in the last one are
    // row n-1 again (its A row and row scale), so they leave the maxima as
    // they are; a block past n that was not computed is left out
#pragma unroll
    for (int i = 0; i < 2; i++) {
      if (wv + 8 * i >= nbc) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        vm[0] = amax(vm[0], v[i][0][r]);
        vm[1] = amax(vm[1], v[i][1][r]);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      vm[j] = __builtin_fmaxf(vm[j], __shfl_xor(vm[j], 32));
      if (fh == 0) red_s[hf][wv][32 * j + fr] = vm[j];
    }
    __syncthreads();
    if (tidh < D) {
      float vs = 0.f;
      for (int w = 0; w < 8; w++) vs = __builtin_fmaxf(vs, red_s[hf][w][tidh]);
      float vi = 0.f;
      if (vs > 0.f) {  // attention8.go:262-269
        vs = vs / 127.0f;
        vi = 1.0f / vs;
      }
      a.vs[((size_t)b * a.nh + h) * D + tidh] = vs;
      stat_s[hf][tidh] = vi;
    }
    __syncthreads();
    const float vi0 = stat_s[hf][fr], vi1 = stat_s[hf][32 + fr];
    int8_t *vt_s = smem + wave * (D * VT_LD);  // [64 dims][32 keys] of this wave's block
    int8_t *vt = a.vt + (size_t)h * D * a.Npad + slot0;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int rb = wv + 8 * i;
      if (rb < nb) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
#pragma unroll
          for (int gq = 0; gq < 4; gq++) {
            // keys 8gq + 4fh + 0..3 of dimension 32j + fr; keys past n are
            // zero bytes (a block past n was not computed: all zero)
            int w = 0;
            if (rb < nbc) {
              int qv[4];
#pragma unroll
              for (int u = 0; u < 4; u++) qv[u] = q8(v[i][j][4 * gq + u], j ? vi1 : vi0);
              const int lim = n - (32 * rb + 8 * gq + 4 * fh);  // keys of the four still in the sequence
              const unsigned keep = lim >= 4 ? 0xffffffffu : lim <= 0 ? 0u : (1u << (8 * lim)) - 1u;
              w = (int)(((unsigned)(qv[0] & 0xff) | ((unsigned)(qv[1] & 0xff) << 8) |
                         ((unsigned)(qv[2] & 0xff) << 16) | ((unsigned)qv[3] << 24)) & keep);
            }
            *(int *)(vt_s + (32 * j + fr) * VT_LD + 8 * gq + 4 * fh) = w;
          }
        }
      }
      __syncthreads();
      if (rb < nb) {
#pragma unroll
        for (int u = 0; u < 2; u++)
          *(v4i *)(vt + (size_t)lane * a.Npad + 32 * rb + 16 * u) = *(const v4i *)(vt_s + lane * VT_LD + 16 * u);
      }
      __syncthreads();
    }
    return;
  }

  // ---- Q and K: rows through an LDS slab of 256 rows ----
  // PUT(t): this wave's block of round t (rows 256t + 32 wave ..) into the
  // slab, in the MFMA layout
  float *slab = (float *)(smem + hf * SLAB_BYTES);  // [256 rows][KT_LD], one a half
#define PUT(t)                                                    \
  if (wv + 8 * (t) < nb) {                                        \
    _Pragma("unroll") for (int r = 0; r < 16; r++) {              \
      const int lr = 32 * wv + acc_row(r, lane);                  \
      slab[lr * KT_LD + fr] = v[t][0][r];                         \
      slab[lr * KT_LD + 32 + fr] = v[t][1][r];                    \
    }                                                             \
  }
  if (part == 1) {
    // K mean over the sequence: 64 float32 chains in key order, one lane
    // a dimension
    float ksum = 0.f;
#pragma unroll
    for (int t = 0; t < 2; t++) {
      if (256 * t < n) {  // block-uniform
        PUT(t)
        __syncthreads();
        if (wv == 0) {
          // the sums stay in key order; KN slab reads are issued together
          // before their KN adds, so the chain waits on LDS once a batch
          // (KN = 8 where NH = 2 leaves fewer registers)
          constexpr int KN = NH == 1 ? 16 : 8;
          const int cnt = min(256, n - 256 * t);
          const float *col = slab + lane;
          int lr = 0;
          for (; lr + KN <= cnt; lr += KN) {
            float bt[KN];
#pragma unroll
            for (int u = 0; u < KN; u++) bt[u] = col[(lr + u) * KT_LD];
            __builtin_amdgcn_sched_barrier(0);  // every read issued before the first add
#pragma unroll
            for (int u = 0; u < KN; u++) ksum = ksum + bt[u];
          }
          for (; lr < cnt; lr++) ksum = ksum + col[lr * KT_LD];
        }
        __syncthreads();
      }
    }
    if (wv == 0) stat_s[hf][lane] = ksum * (1.0f / (float)n);  // Scale(mean, 1/n)
    __syncthreads();
  }

  // Per-row quantisation of the slab's rows (round t): two threads a row,
  // 32 values each (thread: row 16 (lane / 32) + lane % 16 of its wave's
  // 32, half (lane / 16) % 2), K centred first (quantRowAVX2 without the
  // flip, attention8.go:240-251), Q as Attn8.Prepare quantises queries
  // (attention8.go:211-220).
  int8_t *kp = a.kp + ((size_t)h * a.Npad + slot0) * D;
  float *ks = a.ks + (size_t)h * a.Npad + slot0;
  const int hh = (lane >> 4) & 1;
  const int lr = 32 * wv + 16 * (lane >> 5) + (lane & 15);
  auto quant_round = [&](int t) {
    const int row = 256 * t + lr;
    const float4 *src = (const float4 *)(slab + lr * KT_LD + 32 * hh);
    const float4 *mu = (const float4 *)(stat_s[hf] + 32 * hh);
    // the slab is read twice (max, then quantisation): fewer live registers
    auto value = [&](int c) {
      float4 x = src[c];
      if (part == 1) {
        const float4 m4 = mu[c];
        x = make_float4(x.x - m4.x, x.y - m4.y, x.z - m4.z, x.w - m4.w);
      }
      return x;
    };
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const float4 x = value(c);
      mx = amax(amax(amax(amax(mx, x.x), x.y), x.z), x.w);
    }
    mx = __builtin_fmaxf(mx, __shfl_xor(mx, 16));
    __asm__ volatile("" ::: "memory");  // keep the second read of the slab
    float sc = 0.f, inv = 0.f;
    if (mx != 0.f) {
      sc = mx / 127.0f;
      inv = 1.0f / sc;
    }
    const bool valid = row < n;
    int w[8];
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const float4 x = value(c);
      w[c] = valid ? (q8(x.x, inv) & 0xff) | ((q8(x.y, inv) & 0xff) << 8) | ((q8(x.z, inv) & 0xff) << 16) |
                         (q8(x.w, inv) << 24)
                   : 0;
    }
    const v4i lo = {w[0], w[1], w[2], w[3]}, hi = {w[4], w[5], w[6], w[7]};
    if (part == 0) {
      if (valid) {
        int8_t *dst = g.qq + (size_t)(base + row) * a.H + h * D + 32 * hh;
        *(v4i *)dst = lo;
        *(v4i *)(dst + 16) = hi;
        if (hh == 0) g.sq[(size_t)(base + row) * a.nh + h] = sc * g.attn_scale;
      }
    } else if (row < npad) {
      int8_t *dst = kp + (size_t)row * D + 32 * hh;
      *(v4i *)dst = lo;
      *(v4i *)(dst + 16) = hi;
      if (hh == 0) ks[row] = valid ? sc : 0.f;
    }
  };
  if (part == 1) {
    // the slab holds the chains' last round
    if (n > 256) {
      quant_round(1);
      __syncthreads();
      PUT(0)
      __syncthreads();
    }
    quant_round(0);
  } else {
    PUT(0)
    __syncthreads();
    quant_round(0);
    if (n > 256) {
      __syncthreads();
      PUT(1)
      __syncthreads();
      quant_round(1);
    }
  }
#undef PUT
}

}  // namespace

namespace {

// hipFuncSetAttribute once per variant: 1 set, -1 refused (that variant is
// then not used), 0 not tried yet.
template <int NH, bool KB>
bool smem_ready() {
  static int state = 0;
  if (state == 0)
    state = hipFuncSetAttribute((const void *)qkv_attn_kernel<NH, KB>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                Shape<NH>::SMEM) == hipSuccess
                ? 1
                : -1;
  return state > 0;
}

template <int NH, bool KB>
void launch_nh(const GemmArgs &g, const AttnArgs &a, const int32_t *order, hipStream_t s) {
  const int grid = NXCD * 3 * (a.nh / NH) * ((a.B + NXCD - 1) / NXCD);
  qkv_attn_kernel<NH, KB><<<grid, 512 * NH, Shape<NH>::SMEM, s>>>(g, a, order);
}

}  // namespace

bool qkv_kblock_supported(int Kp) { return Kp % 128 == 0 && Kp * 64 <= Shape<1>::SMEM; }

// One head a workgroup; two (1,024 threads) on request when the
// head count is even and the device grants the LDS. Two heads halve the
// rows brought into LDS per head, but one workgroup then fills a CU and its
// dequantisation and Attn8.Prepare phases (40% of a workgroup's time) no
// longer overlap another workgroup's K loop: slower on cfg4 (339 against
// 315 us a launch).
void launch_qkv_attn(const GemmArgs &g, const AttnArgs &a, const int32_t *order, int heads, hipStream_t s) {
  if (a.B <= 0) return;
  const bool pair = heads == 2 && a.nh % 2 == 0 && !g.Ak;
  if (pair && smem_ready<2, false>()) {
    launch_nh<2, false>(g, a, order, s);
  } else if (g.Ak) {
    (void)smem_ready<1, true>();
    launch_nh<1, true>(g, a, order, s);
  } else {
    (void)smem_ready<1, false>();
    launch_nh<1, false>(g, a, order, s);
  }
}

}  // namespace ixh
