// attention_i8.hip — int8 attention of indecis (linalg/attention8.go) on
// gfx950: QK^T and PV on i8 MFMA, the reference's full-row softmax in fp32,
// sliding-window (local) and global layers, sequences packed by offsets.
//
// Prologue, one workgroup per (sequence, head) — Attn8.Prepare
// (attention8.go:203-280): Q quantised per row with 1/sqrt(D) folded into
// its scale; K centred on its mean over the sequence (a sequential float32
// sum in key order, then times f32(1/n)) and quantised per key; V
// quantised per dimension. K is stored [head][slot][64], V transposed
// [head][d][slot]; each sequence's slots are padded with zeros to 64.
//
// Main, one workgroup per (sequence, block of 128 queries, head), 4 waves
// of 32 queries — Attn8.Attend (attention8.go:298-376). Each wave computes
// S^T = K.Q^T in 32x32 tiles (a lane holds one query, 16 keys), so the
// score tile is already the B operand of O^T = V^T.P^T. The softmax is
// the reference's two-pass one, exactly: pass 1 the row max of the valid
// scores, pass 2 e = exp(s - max) (the vector formula, or exp32 on the
// last len%V keys of a row as ExpShift does), P = RNE(255 e) as uint8,
// normalised by 1/f32(sum P). P (0..255) does not fit int8: the MFMA
// takes P - 128 and the accumulators get 128 * (sum of V over the keys of
// the tiles) added from per-chunk prefix sums, exactly. Scores need
// ((f32(tile) - kzc)*ks)*sq with the uint8 tile; tile - kzc is exactly the
// signed sum, so the kernel uses f32(sum q*k).
#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace {

constexpr int D = 64;
constexpr int CHUNK = 256;       // keys staged in LDS at a time
constexpr int KS = 80;           // LDS row stride of K (bytes)
constexpr int VS = CHUNK + 16;   // LDS row stride of V^T (bytes)

__device__ __forceinline__ float absmax16(const float4 *v) {
  float m = 0.f;
#pragma unroll
  for (int c = 0; c < 16; c++)
    m = amax(amax(amax(amax(m, v[c].x), v[c].y), v[c].z), v[c].w);
  return m;
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
  return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | (d << 24);
}

constexpr int kShortSeq = 512;   // keys one prologue workgroup holds in registers
constexpr int kStatRows = 256;   // keys per LDS slab of the long-sequence K chains
constexpr int kStatStride = kStatRows + 4;

// Statistics of a long sequence (more than kShortSeq keys) for
// Attn8.Prepare (attention8.go:224-230, 259-269), split 8 ways per
// (sequence, head): blockIdx.z 0..3 run the float32 chains of the K mean
// of 16 dimensions each, in key order (AddTo, then Scale by f32(1/n));
// blockIdx.z 4..7 take max |V| of 16 dimensions (MaxAbsTo). 4 threads own
// a key's 16 values (a float4 each), 64 keys per load. The K chains read
// their slab transposed from LDS (one dimension's keys contiguous), double
// buffered, while the next slab's loads are in flight. Writes the V scale
// to a.vs and, per (sequence, head), the K mean and 1/V scale to a.kstat.
__global__ __launch_bounds__(256) void attn_long_stats_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float kt[2][16][kStatStride];
  const int b = blockIdx.x, h = blockIdx.y, z = blockIdx.z, tid = threadIdx.x;
  const int q = tid & 3, r0 = tid >> 2;
  const bool isk = z < 4;
  const int dg = (z & 3) * 16;
  const int base = a.offs[b], n = a.offs[b + 1] - base;
  const int ld = 3 * a.H;
  const float *seq = a.qkv + (size_t)base * ld;
  const uint32_t voff = 4u * ((uint32_t)r0 * ld + (isk ? a.H : 2 * a.H) + h * D + dg + 4 * q);
  float *stat = a.kstat + ((size_t)b * a.nh + h) * 2 * D;
  const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 reg[4];
  // rows c0 .. c0+255 through a buffer descriptor of the slab's valid rows:
  // keys past the sequence read as 0
#define IXH_STAT_LOAD(c0)                                                                   \
  {                                                                                         \
    const __amdgpu_buffer_rsrc_t rs =                                                       \
        buf_rsrc(seq + (size_t)(c0) * ld, (uint32_t)min(kStatRows, n - (c0)) * ld * 4);     \
    _Pragma("unroll") for (int u = 0; u < 4; u++) reg[u] = buf_load_f4(rs, voff, 256u * u * ld); \
  }
  if (isk) {
    float ksum = 0.f;
    if (n > 0) IXH_STAT_LOAD(0)
    for (int c0 = 0, buf = 0; c0 < n; c0 += kStatRows, buf ^= 1) {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int r = r0 + 64 * u;
        kt[buf][4 * q][r] = reg[u].x;
        kt[buf][4 * q + 1][r] = reg[u].y;
        kt[buf][4 * q + 2][r] = reg[u].z;
        kt[buf][4 * q + 3][r] = reg[u].w;
      }
      __syncthreads();  // also orders the previous chain on this buffer
      if (c0 + kStatRows < n) IXH_STAT_LOAD(c0 + kStatRows)
      if (tid < 16) {
        const float *row = &kt[buf][tid][0];
        const int cnt = min(kStatRows, n - c0);
        int r = 0;
        for (; r + 4 <= cnt; r += 4) {
          const float4 v = *(const float4 *)(row + r);
          ksum = ksum + v.x;
          ksum = ksum + v.y;
          ksum = ksum + v.z;
          ksum = ksum + v.w;
        }
        for (; r < cnt; r++) ksum = ksum + row[r];
      }
    }
    if (tid < 16) stat[dg + tid] = n > 0 ? ksum * (1.0f / (float)n) : 0.f;
  } else {
    float4 vm = zero4;
    if (n > 0) IXH_STAT_LOAD(0)
    for (int c0 = 0; c0 < n; c0 += kStatRows) {
      float4 cur[4];
#pragma unroll
      for (int u = 0; u < 4; u++) cur[u] = reg[u];
      if (c0 + kStatRows < n) IXH_STAT_LOAD(c0 + kStatRows)
#pragma unroll
      for (int u = 0; u < 4; u++)
        vm = make_float4(amax(vm.x, cur[u].x), amax(vm.y, cur[u].y),
                         amax(vm.z, cur[u].z), amax(vm.w, cur[u].w));
    }
    // threads with the same q hold the same 4 dimensions: xor over r0
    for (int t = 4; t < 64; t <<= 1) {
      vm.x = __builtin_fmaxf(vm.x, __shfl_xor(vm.x, t));
      vm.y = __builtin_fmaxf(vm.y, __shfl_xor(vm.y, t));
      vm.z = __builtin_fmaxf(vm.z, __shfl_xor(vm.z, t));
      vm.w = __builtin_fmaxf(vm.w, __shfl_xor(vm.w, t));
    }
    float4 *red = (float4 *)&kt[0][0][0];  // [wave][q]
    if ((tid & 63) < 4) red[(tid >> 6) * 4 + q] = vm;
    __syncthreads();
    if (tid < 16) {
      const float *rf = (const float *)red;
      float vs = 0.f;
      for (int w = 0; w < 4; w++) vs = __builtin_fmaxf(vs, rf[w * 16 + tid]);
      float vi = 0.f;
      if (vs > 0.f) {  // attention8.go:262-269
        vs = vs / 127.0f;
        vi = 1.0f / vs;
      }
      a.vs[((size_t)b * a.nh + h) * D + dg + tid] = vs;
      stat[D + dg + tid] = vi;
    }
  }
#undef IXH_STAT_LOAD
}

// Single-read prologue: one workgroup of 512 threads per (sequence, head,
// K or V) holds up to kShortSeq keys of the 64-wide head slice in
// registers (16 float4 per thread), so K and V are read from HBM once.
// PART: a long sequence's keys in parts of kShortSeq (blockIdx.z = 2 part
// + K/V), with the K mean and 1/V scale from attn_long_stats_kernel;
// otherwise (all sequences at most kShortSeq) the statistics are computed
// here.
//  K (blockIdx.z even): row j = rg + 32u (rg = tid/16, u < 16). The 64
//    sequential float32 chains of the mean run in wave 0 over 32-row pieces
//    written to a double-buffered LDS slab (one barrier per piece); then
//    each row is centred and quantised from registers.
//  V (blockIdx.z odd): row j = 16 rg + u, so a thread holds 16 consecutive
//    keys of 4 dimensions: max |V| per dimension by a block reduction, then
//    each dimension's 16 quantised keys leave as one 16-byte store into
//    V^T.
template <bool PART>
__global__ __launch_bounds__(512, 4) void attn_prologue_rows_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float kst[2][32 * D];
  __shared__ __attribute__((aligned(16))) float red[8][D];
  __shared__ __attribute__((aligned(16))) float mean[D];
  const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int sub = tid & 15, rg = tid >> 4, wave = tid >> 6, lane = tid & 63;
  const int j0 = PART ? (int)(blockIdx.z >> 1) * kShortSeq : 0;  // first key of the part
  const int nseq = a.offs[b + 1] - a.offs[b];
  const int npseq = (nseq + kKeyPad - 1) / kKeyPad * kKeyPad;
  if (PART && j0 >= npseq) return;  // j0 < npseq implies j0 < nseq
  const int base = a.offs[b] + j0, n = min(nseq - j0, kShortSeq);
  const int slot0 = a.padoff[b] + j0;
  const int npad = min(npseq - j0, kShortSeq);
  const int H = a.H, ld = 3 * H;
  const float *stat = a.kstat + ((size_t)b * a.nh + h) * 2 * D;
  // the sequence's rows of qkv; a row is 4*ld bytes
  const __amdgpu_buffer_rsrc_t rows = buf_rsrc(a.qkv + (size_t)base * ld, (uint32_t)n * ld * 4);
  const uint32_t col = 4u * (H + h * D + 4 * sub);  // byte offset of this thread's K float4
  const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);

  if ((blockIdx.z & 1) == 0) {
    float4 kr[16];
    const uint32_t voff = (uint32_t)rg * ld * 4 + col;
#pragma unroll
    for (int u = 0; u < 16; u++) {
      const int j = rg + 32 * u;
      kr[u] = j < n ? buf_load_f4<kStreamPolicy>(rows, voff, (uint32_t)(32 * u) * ld * 4) : zero4;
    }
    // sum of K in key order (AddTo, attention8.go:224-228)
    float ksum = 0.f;
#pragma unroll
    for (int u = 0; u < 16; u++) {
      if (!PART && 32 * u < n) {  // block-uniform
        *(float4 *)&kst[u & 1][rg * D + 4 * sub] = kr[u];
        __syncthreads();
        if (wave == 0) {
          const float *col = &kst[u & 1][lane];
          const int cnt = min(32, n - 32 * u);
          if (cnt == 32) {
#pragma unroll
            for (int rr = 0; rr < 32; rr++) ksum = ksum + col[rr * D];
          } else {
            for (int rr = 0; rr < cnt; rr++) ksum = ksum + col[rr * D];
          }
        }
      }
    }
    if (wave == 0) mean[lane] = PART ? stat[lane] : n > 0 ? ksum * (1.0f / (float)n) : 0.f;  // Scale(mean, 1/n)
    __syncthreads();
    // centred rows quantised per key (quantRowAVX2 without the flip,
    // attention8.go:240-251); padding slots [n, npad) get zeros
    int8_t *kp = a.kp + ((size_t)h * a.Npad + slot0) * D;
    float *ks = a.ks + (size_t)h * a.Npad + slot0;
    const float4 mu = *(const float4 *)&mean[4 * sub];
#pragma unroll
    for (int u = 0; u < 16; u++) {
      const int j = rg + 32 * u;
      if (j < npad) {  // uniform over the 16 lanes of a row
        int kq = 0;
        float sc = 0.f;
        if (j < n) {
          const float4 c = make_float4(kr[u].x - mu.x, kr[u].y - mu.y, kr[u].z - mu.z, kr[u].w - mu.w);
          float mx = amax(amax(amax(amax(0.f, c.x), c.y), c.z), c.w);
          for (int t = 1; t < 16; t <<= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, t, 16));
          float inv = 0.f;
          if (mx != 0.f) {
            sc = mx / 127.0f;
            inv = 1.0f / sc;
          }
          kq = pack4(q8(c.x, inv), q8(c.y, inv), q8(c.z, inv), q8(c.w, inv));
        }
        *(int *)(kp + (size_t)j * D + 4 * sub) = kq;
        if (sub == 0) ks[j] = sc;
      }
    }
  } else {
    float4 vr[16];
    const uint32_t voff = (uint32_t)(16 * rg) * ld * 4 + col + 4 * H;
#pragma unroll
    for (int u = 0; u < 16; u++) {
      const int j = 16 * rg + u;
      vr[u] = j < n ? buf_load_f4<kStreamPolicy>(rows, voff, (uint32_t)u * ld * 4) : zero4;
    }
    if (PART) {
      if (tid < D) mean[tid] = stat[D + tid];
    } else {
      // max |V| per dimension (MaxAbsTo, attention8.go:259-261)
      float4 vm = zero4;
#pragma unroll
      for (int u = 0; u < 16; u++)
        vm = make_float4(amax(vm.x, vr[u].x), amax(vm.y, vr[u].y),
                         amax(vm.z, vr[u].z), amax(vm.w, vr[u].w));
      for (int t = 16; t < 64; t <<= 1) {
        vm.x = __builtin_fmaxf(vm.x, __shfl_xor(vm.x, t));
        vm.y = __builtin_fmaxf(vm.y, __shfl_xor(vm.y, t));
        vm.z = __builtin_fmaxf(vm.z, __shfl_xor(vm.z, t));
        vm.w = __builtin_fmaxf(vm.w, __shfl_xor(vm.w, t));
      }
      if (lane < 16) *(float4 *)&red[wave][4 * sub] = vm;
      __syncthreads();
      if (tid < D) {
        float vs = 0.f;
        for (int g = 0; g < 8; g++) vs = __builtin_fmaxf(vs, red[g][tid]);
        float vi = 0.f;
        if (vs > 0.f) {  // attention8.go:262-269
          vs = vs / 127.0f;
          vi = 1.0f / vs;
        }
        mean[tid] = vi;
        a.vs[((size_t)b * a.nh + h) * D + tid] = vs;
      }
    }
    __syncthreads();
    // quantCols (attention8.go:270-279), 16 keys of a dimension per store
    const float4 vi = *(const float4 *)&mean[4 * sub];
    if (16 * rg < npad) {
      int8_t *vt = a.vt + ((size_t)h * D + 4 * sub) * a.Npad + slot0 + 16 * rg;
      int w[4][4];
#pragma unroll
      for (int u = 0; u < 16; u += 4) {
        w[0][u / 4] = pack4(q8(vr[u].x, vi.x), q8(vr[u + 1].x, vi.x), q8(vr[u + 2].x, vi.x), q8(vr[u + 3].x, vi.x));
        w[1][u / 4] = pack4(q8(vr[u].y, vi.y), q8(vr[u + 1].y, vi.y), q8(vr[u + 2].y, vi.y), q8(vr[u + 3].y, vi.y));
        w[2][u / 4] = pack4(q8(vr[u].z, vi.z), q8(vr[u + 1].z, vi.z), q8(vr[u + 2].z, vi.z), q8(vr[u + 3].z, vi.z));
        w[3][u / 4] = pack4(q8(vr[u].w, vi.w), q8(vr[u + 1].w, vi.w), q8(vr[u + 2].w, vi.w), q8(vr[u + 3].w, vi.w));
      }
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const v4i o = {w[c][0], w[c][1], w[c][2], w[c][3]};
        *(v4i *)(vt + (size_t)c * a.Npad) = o;
      }
    }
  }
}

// Q per (row, head) for Attend8 callers whose queries did not come out of
// the QKV GEMM epilogue: 16 threads per row, as the prologue's K pass.
__global__ __launch_bounds__(256) void attn_quant_q_kernel(AttnArgs a) {
  const int g = blockIdx.x * 16 + (threadIdx.x >> 4), sub = threadIdx.x & 15;
  if (g >= a.N * a.nh) return;  // whole 16-lane groups leave together
  const int row = g / a.nh, h = g % a.nh;
  const float4 v = *(const float4 *)(a.qkv + (size_t)row * 3 * a.H + h * D + 4 * sub);
  float mx = amax(amax(amax(amax(0.f, v.x), v.y), v.z), v.w);
  for (int t = 1; t < 16; t <<= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, t, 16));
  float s = 0.f, inv = 0.f;
  if (mx != 0.f) {
    s = mx / 127.0f;
    inv = 1.0f / s;
  }
  *(int *)(a.qq + (size_t)row * a.H + h * D + 4 * sub) =
      pack4(q8(v.x, inv), q8(v.y, inv), q8(v.z, inv), q8(v.w, inv));
  if (sub == 0) a.sq[(size_t)row * a.nh + h] = s * a.scale;
}

// Four waves a SIMD (at most 128 VGPRs) for both layer kinds: local layers
// 116-118 us a launch on cfg4 against 129-131 at three waves a SIMD.
template <bool GLOBAL>
__global__ __launch_bounds__(256, 4) void attn_main_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t Ks[CHUNK * KS];
  __shared__ __attribute__((aligned(16))) int8_t Vs[D * VS];
  __shared__ __attribute__((aligned(16))) float kss[CHUNK];
  // per 32-key group g of the staged chunk: vpre[g][d] = 128 times the sum
  // of V over the keys of groups 0..g (int, exact: at most 128 * 256 * 127);
  // 40 KB of LDS in all, 4 workgroups per CU
  __shared__ __attribute__((aligned(16))) int vpre[CHUNK / 32][D];

  // the wave index as a scalar: the tile loops and the full-tile tests
  // that derive from it are then scalar branches, not lane masks
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // work item j = head * nblocks + entry (a sequence's query blocks are
  // consecutive entries). Workgroup L runs on XCD L % 8; each XCD takes a
  // contiguous run of items, so the query blocks of one (sequence, head)
  // run on one XCD and share its K and V in that XCD's L2.
  const int per = (a.nblocks * a.nh + 7) / 8;
  const int j = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (j >= a.nblocks * a.nh) return;  // the whole workgroup
  const int h = j / a.nblocks, ent = j - h * a.nblocks;
  const int b = a.blocks[2 * ent], Q0 = a.blocks[2 * ent + 1];
  const int base = a.offs[b], n = a.offs[b + 1] - base;
  const int slot0 = a.padoff[b];
  const int npad = (n + kKeyPad - 1) / kKeyPad * kKeyPad;
  const int H = a.H, W = a.window;
  constexpr bool global = GLOBAL;

  // this lane's query
  const int q0 = Q0 + 32 * wave;
  const int qi = q0 + (lane & 31);
  const bool qact = qi < n;
  v4i qb[2];
  {
    const v4i z = {0, 0, 0, 0};
    const int8_t *qsrc = a.qq + (size_t)(base + (qact ? qi : 0)) * H + h * D + 16 * (lane >> 5);
    qb[0] = qact ? *(const v4i *)(qsrc) : z;
    qb[1] = qact ? *(const v4i *)(qsrc + 32) : z;
  }
  const float sqv = qact ? a.sq[(size_t)(base + qi) * a.nh + h] : 0.f;
  // valid keys [cs, ce) of the query and the start of the exp32 tail
  // (ExpShift's scalar loop over the last len%V values, vec_simd.go:258-262)
  const int cs = global ? 0 : max(0, qi - W);
  const int ce = global ? n : min(n, qi + W + 1);
  const uint32_t span = (uint32_t)(ce - cs);  // > 0 for an active query
  const int V = a.lanes;
  const int ts = V > 0 ? cs + ((ce - cs) / V) * V : cs;
  // wave-wide bounds over the active queries: a tile [k0, k0+32) with
  // k0 >= cs_hi and k0+32 <= ce_lo is valid for every query
  int cs_hi = qact ? cs : 0, ce_lo = qact ? ce : 1 << 30;
  for (int t = 1; t < 64; t <<= 1) {
    cs_hi = max(cs_hi, __shfl_xor(cs_hi, t));
    ce_lo = min(ce_lo, __shfl_xor(ce_lo, t));
  }
  cs_hi = __builtin_amdgcn_readfirstlane(cs_hi);  // every lane holds the same value
  ce_lo = __builtin_amdgcn_readfirstlane(ce_lo);

  // key tiles (32 keys) of this wave and of the block
  int wt0, wt1, bk0, bk1;
  if (global) {
    wt0 = 0;
    wt1 = (n + 31) / 32;
    bk0 = 0;
    bk1 = n;
  } else {
    wt0 = max(0, q0 - W) / 32;
    wt1 = (min(n, q0 + 31 + W + 1) + 31) / 32;
    bk0 = max(0, Q0 - W) / 32 * 32;
    bk1 = min(n, Q0 + kAttnQBlock - 1 + W + 1);
  }
  if (q0 >= n) wt1 = wt0;  // idle wave (still takes part in the barriers)
  const bool one_chunk = bk1 - bk0 <= CHUNK;

  const int8_t *kglob = a.kp + ((size_t)h * a.Npad + slot0) * D;
  const float *ksglob = a.ks + (size_t)h * a.Npad + slot0;
  const int8_t *vglob = a.vt + (size_t)h * D * a.Npad + slot0;

  // Stage the chunk of keys c0 .. c0+CHUNK-1: K rows and their scales,
  // and with with_v V^T with the 8 dwords of each 32-key group permuted so
  // that lane half hf reads the keys 8*(b/4) + 4*hf + b%4 (the S^T
  // accumulator rows) as 16 contiguous bytes, plus each group's sum of V
  // per dimension. Every global load of the thread is issued before the
  // first LDS write, so the staging waits on memory once. Buffer loads:
  // keys past the sequence's slots read 0 (V^T rows continue into the next
  // sequence's slots, so those loads get an offset past the range).
  static_assert(CHUNK == 256, "one key scale a thread (256 threads)");
  constexpr int NKP = CHUNK * 4 / 256;         // 16-byte K pieces a thread
  constexpr int NVG = D * (CHUNK / 32) / 256;  // V (dimension, group) items a thread
  const auto krs = buf_rsrc(kglob, (uint32_t)npad * D);
  const auto ksrs = buf_rsrc(ksglob, (uint32_t)npad * 4);
  const auto vrs = buf_rsrc(vglob, (uint32_t)((D - 1) * a.Npad + npad));
  auto stage = [&](int c0, bool with_v) {
    // local layers: the thread's offsets are recomputed at each call from
    // an opaque copy of its index, instead of being kept in VGPRs across
    // the score loops between calls (held to 128 VGPRs, the kernel spilled
    // 8 of them: 8 KB a workgroup written to scratch)
    int tid = threadIdx.x;
    if constexpr (!GLOBAL) asm volatile("" : "+v"(tid));
    v4i kw[NKP], vlo[NVG], vhi[NVG];
#pragma unroll
    for (int i = 0; i < NKP; i++)
      kw[i] = __builtin_amdgcn_raw_buffer_load_b128(krs, (uint32_t)((c0 + (tid >> 2) + 64 * i) * D + 16 * (tid & 3)), 0, 0);
    const float kv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ksrs, (uint32_t)(c0 + tid) * 4, 0, 0));
    if (with_v) {
#pragma unroll
      for (int i = 0; i < NVG; i++) {
        const int e = tid + 256 * i, d = e / (CHUNK / 32), g = e % (CHUNK / 32);
        const uint32_t off = c0 + 32 * g < npad ? (uint32_t)(d * a.Npad + c0 + 32 * g) : 0x7fffffe0u;
        vlo[i] = __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0);
        vhi[i] = __builtin_amdgcn_raw_buffer_load_b128(vrs, off + 16, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < NKP; i++) *(v4i *)&Ks[((tid >> 2) + 64 * i) * KS + 16 * (tid & 3)] = kw[i];
    kss[tid] = kv;
    if (with_v) {
#pragma unroll
      for (int i = 0; i < NVG; i++) {
        const int e = tid + 256 * i, d = e / (CHUNK / 32), g = e % (CHUNK / 32);
        const int w[8] = {vlo[i][0], vlo[i][1], vlo[i][2], vlo[i][3], vhi[i][0], vhi[i][1], vhi[i][2], vhi[i][3]};
        const v4i o0 = {w[0], w[2], w[4], w[6]}, o1 = {w[1], w[3], w[5], w[7]};
        *(v4i *)&Vs[d * VS + 32 * g] = o0;
        *(v4i *)&Vs[d * VS + 32 * g + 16] = o1;
        int sum = 0;
#pragma unroll
        for (int u = 0; u < 8; u++) sum = __builtin_amdgcn_sdot4(w[u], 0x01010101, sum, false);
        vpre[g][d] = sum;
      }
    }
  };
  // after the barrier that follows stage_v: group sums -> prefix sums (the
  // group sums read together, then written: one wait on LDS, not one a
  // group)
  // global layers: thread d < 64 keeps 128 times the sum of V over the
  // chunks so far
  int vtot = 0;
  auto prefix_v = [&] {
    if (tid < D) {
      int gsum[CHUNK / 32];
#pragma unroll
      for (int g = 0; g < CHUNK / 32; g++) gsum[g] = vpre[g][tid];
#pragma unroll
      for (int g = 1; g < CHUNK / 32; g++) gsum[g] += gsum[g - 1];
      if constexpr (GLOBAL) {
        vtot += 128 * gsum[CHUNK / 32 - 1];  // the chunk's sum (each chunk once)
      } else {
#pragma unroll
        for (int g = 0; g < CHUNK / 32; g++) vpre[g][tid] = 128 * gsum[g];
      }
    }
    __syncthreads();
  };
  // Scores of tile t without the query scale: f32(sum q*k) * ks, in the S^T
  // layout (rows = keys 8*(r/4) + 4*(lane/32) + r%4 of the tile, column =
  // this query). The score is that times sq.
  // The integer tile of tile t (two MFMAs), then its scaled scores.
  // (Issuing tile t+1's MFMAs before tile t's VALU work was tried: no gain.)
  auto score_acc = [&](int t, int c0) {
    v16i acc = {};
    const int8_t *kr = &Ks[(t * 32 - c0 + (lane & 31)) * KS + 16 * (lane >> 5)];
    acc = mfma32(*(const v4i *)kr, qb[0], acc);
    acc = mfma32(*(const v4i *)(kr + 32), qb[1], acc);
    return acc;
  };
  auto score_scale = [&](int t, int c0, const v16i &acc, float *sv) {
    const float *kt = &kss[t * 32 - c0 + 4 * (lane >> 5)];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const float4 k4 = *(const float4 *)(kt + 8 * g);
      sv[4 * g] = (float)acc[4 * g] * k4.x;
      sv[4 * g + 1] = (float)acc[4 * g + 1] * k4.y;
      sv[4 * g + 2] = (float)acc[4 * g + 2] * k4.z;
      sv[4 * g + 3] = (float)acc[4 * g + 3] * k4.w;
    }
  };

  // ---- pass 1: row max of the valid scores ----
  // max_j f32(x_j * sq) = f32(max_j x_j * sq): rounding is monotone and
  // sq >= 0, so the query scale is applied once, to the max.
  float m = -__builtin_huge_valf();
  for (int c0 = bk0; c0 < bk1; c0 += CHUNK) {
    __syncthreads();
    stage(c0, one_chunk);
    __syncthreads();
    if (one_chunk) prefix_v();
    const int t0 = max(wt0, c0 / 32), t1 = min(wt1, (c0 + CHUNK) / 32);
    for (int t = t0; t < t1; t++) {
      float sv[16];
      score_scale(t, c0, score_acc(t, c0), sv);
      const int k0 = t * 32;
      if (k0 >= cs_hi && k0 + 32 <= ce_lo) {  // every key valid for every query
#pragma unroll
        for (int r = 0; r < 16; r++) m = __builtin_fmaxf(m, sv[r]);  // no NaN: v_max
      } else {
        // key j valid: cs <= j < ce, as one unsigned compare of j - cs
        const int jb = k0 - cs + 4 * (lane >> 5);
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const bool in = (uint32_t)(jb + 8 * (r >> 2) + (r & 3)) < span;
          m = __builtin_fmaxf(m, in ? sv[r] : -__builtin_huge_valf());
        }
      }
    }
  }
  m = __builtin_fmaxf(m, __shfl_xor(m, 32)) * sqv;

  // ---- pass 2: P = RNE(255 exp(s - m)), O^T += V^T . P^T ----
  // P (0..255) enters the MFMA as P - 128 (an int8: the byte P ^ 0x80);
  // the missing 128 * sum_j v[j][d] over every key of the tiles a wave
  // processes is the same for all its queries and is added to the
  // accumulators per chunk from the prefix sums: O stays exact.
  // P is rounded from the hardware exponential (exp255_fast) unless that
  // lands within kExp255Tol of a half-integer; there (about 1 score in 4000)
  // the reference formula decides: exp32 on the tail keys j >= ts (all keys
  // when lanes = 0), ExpShift's vector formula elsewhere.
  v16i o[2];
#pragma unroll
  for (int dt = 0; dt < 2; dt++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[dt][r] = 0;
  unsigned psum = 0;
  for (int c0 = bk0; c0 < bk1; c0 += CHUNK) {
    if (!one_chunk) {
      __syncthreads();
      stage(c0, true);
      __syncthreads();
      prefix_v();
    }
    const int t0 = max(wt0, c0 / 32), t1 = min(wt1, (c0 + CHUNK) / 32);
    if (!GLOBAL && t1 > t0) {
      // rows of this lane: dims dt*32 + 8g + 4*(lane/32) + 0..3
#pragma unroll
      for (int dt = 0; dt < 2; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int d0 = dt * 32 + 8 * g + 4 * (lane >> 5);
          const int4 hi = *(const int4 *)&vpre[t1 - 1 - c0 / 32][d0];
          const int4 lo = t0 > c0 / 32 ? *(const int4 *)&vpre[t0 - 1 - c0 / 32][d0] : int4{0, 0, 0, 0};
          o[dt][4 * g] += hi.x - lo.x;
          o[dt][4 * g + 1] += hi.y - lo.y;
          o[dt][4 * g + 2] += hi.z - lo.z;
          o[dt][4 * g + 3] += hi.w - lo.w;
        }
    }
    for (int t = t0; t < t1; t++) {
      float sv[16];
      score_scale(t, c0, score_acc(t, c0), sv);
      const int k0 = t * 32;
      const bool full = k0 >= cs_hi && k0 + 32 <= ce_lo;  // every key valid for every query
      float p[16];
      // largest distance of 255 e from its rounding: one max per score,
      // one compare per tile; the rare lanes past the tolerance recheck
      // their scores one by one
      float dev = 0.f;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        sv[r] = sv[r] * sqv - m;  // s - max, as the reference forms it
        const float y = exp255_fast(sv[r]);
        p[r] = rne(y);
        dev = __builtin_fmaxf(dev, fabsf(y - p[r]));  // no NaN here: one v_max
      }
      if (dev > 0.5f - kExp255Tol) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          if (fabsf(exp255_fast(sv[r]) - p[r]) > 0.5f - kExp255Tol) {
            const int j = k0 + acc_row(r, lane);
            const float e = (j >= ts) ? exp32_scalar(sv[r]) : exp32_simd(sv[r]);
            // QuantizeRowU8 (vec_simd.go:64-91): RNE(e*255) in [0, 255]
            p[r] = rne(e * 255.0f);
          }
        }
      }
      if (!full) {
        const int jb = k0 - cs + 4 * (lane >> 5);
#pragma unroll
        for (int r = 0; r < 16; r++) p[r] = (uint32_t)(jb + 8 * (r >> 2) + (r & 3)) < span ? p[r] : 0.0f;
      }
      unsigned pw[4];
#pragma unroll
      for (int g = 0; g < 4; g++) {
        unsigned w = 0;
#pragma unroll
        for (int u = 0; u < 4; u++) w = __builtin_amdgcn_cvt_pk_u8_f32(p[4 * g + u], u, w);
        pw[g] = w;
        psum = __builtin_amdgcn_udot4(w, 0x01010101u, psum, false);
      }
      // P - 128 as int8
      const v4i bp = {(int)(pw[0] ^ 0x80808080u), (int)(pw[1] ^ 0x80808080u),
                      (int)(pw[2] ^ 0x80808080u), (int)(pw[3] ^ 0x80808080u)};
#pragma unroll
      for (int dt = 0; dt < 2; dt++) {
        const v4i fv = *(const v4i *)&Vs[(dt * 32 + (lane & 31)) * VS + (t * 32 - c0) + 16 * (lane >> 5)];
        o[dt] = mfma32(fv, bp, o[dt]);
      }
    }
  }
  if constexpr (GLOBAL) {
    // a wave with queries takes every tile of the sequence, so its
    // correction is 128 times the sequence's sum of V (keys past it are
    // zero), added once
    // (vpre is free: its last reader, the last prefix, passed its barrier)
    if (tid < D) vpre[0][tid] = vtot;
    __syncthreads();
    if (wt1 > wt0) {
#pragma unroll
      for (int dt = 0; dt < 2; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int4 tv = *(const int4 *)&vpre[0][dt * 32 + 8 * g + 4 * (lane >> 5)];
          o[dt][4 * g] += tv.x;
          o[dt][4 * g + 1] += tv.y;
          o[dt][4 * g + 2] += tv.z;
          o[dt][4 * g + 3] += tv.w;
        }
    }
  }
  psum += __shfl_xor(psum, 32);
  // The context rows leave through LDS: each wave stages its 32 queries x
  // 64 dimensions in the free K or V staging area, then stores whole
  // 256-byte row pieces (16 lanes a query), non-temporal (the Wo kernel
  // reads them once).
  constexpr int OLD = D + 4;  // floats a staged row (conflict-free writes)
  static_assert(2 * 32 * OLD * 4 <= CHUNK * KS && 2 * 32 * OLD * 4 <= D * VS, "context staging");
  __syncthreads();  // every wave is past pass 2: Ks and Vs are free
  float *stg = (float *)(wave < 2 ? Ks : Vs) + (wave & 1) * (32 * OLD);
  const float sp = qact ? 1.0f / (float)(int)psum : 0.f;
  const float *vsd = a.vs + ((size_t)b * a.nh + h) * D;
  float mx = 0.f;  // max |ctx| of this (row, head), for the fused Wo GEMM
  // the V scales of this lane's 32 dimensions, every load issued before
  // the first store (the compiler cannot tell vs from ctx)
  float4 vsv[2][4];
#pragma unroll
  for (int dt = 0; dt < 2; dt++)
#pragma unroll
    for (int g = 0; g < 4; g++) vsv[dt][g] = *(const float4 *)&vsd[dt * 32 + acc_row(4 * g, lane)];
#pragma unroll
  for (int dt = 0; dt < 2; dt++) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d0 = dt * 32 + acc_row(4 * g, lane);
      const float4 v4 = vsv[dt][g];
      const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
      float ov[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int r = 4 * g + u;
        const int tile = o[dt][r];
        ov[u] = (((float)tile - 0.0f) * vv[u]) * sp;
        mx = __builtin_fmaxf(mx, fabsf(ov[u]));
      }
      *(float4 *)(stg + (lane & 31) * OLD + d0) = make_float4(ov[0], ov[1], ov[2], ov[3]);
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt 0: this wave's staging writes are done
  __builtin_amdgcn_wave_barrier();
  // query 4u + lane/16 of the wave, dimensions 4 (lane % 16) .. + 3
#pragma unroll
  for (int u = 0; u < 8; u++) {
    const int ql = 4 * u + (lane >> 4), qg = q0 + ql;
    const float4 v = *(const float4 *)(stg + ql * OLD + 4 * (lane & 15));
    if (qg < n)
      store_stream_16(a.ctx + (size_t)(base + qg) * H + h * D + 4 * (lane & 15),
                      v4i{__float_as_int(v.x), __float_as_int(v.y), __float_as_int(v.z), __float_as_int(v.w)});
  }
  if (a.rmax && qact) {
    mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32));  // the other 32 dimensions
    if (lane < 32) a.rmax[(size_t)(base + qi) * a.nh + h] = mx;
  }
}

// Every float v = bits -> float over [lo, hi) (v <= 0 expected): counts
// the v where exp255_fast decides the rounding (away from a half-integer by
// more than kExp255Tol) and RNE differs from the reference's
// RNE(f32(255*exp(v))), for exp32_simd (res[0]) and exp32_scalar (res[1]);
// res[2], res[3]: largest |exp255_fast - 255*exp| of each formula, as
// float bits; res[4]: number of undecided v.
__global__ __launch_bounds__(256) void check_exp255_kernel(uint32_t lo, uint32_t hi,
                                                           unsigned long long *res) {
  unsigned long long bad_v = 0, bad_s = 0, amb = 0;
  float err_v = 0.f, err_s = 0.f;
  const uint32_t stride = gridDim.x * 256u;
  for (uint32_t u = lo + blockIdx.x * 256u + threadIdx.x; u < hi && u >= lo; u += stride) {
    const float v = __uint_as_float(u);
    const float y = exp255_fast(v);
    const float p = rne(y);
    const bool decided = fabsf(y - p) <= 0.5f - kExp255Tol;
    const float yv = exp32_simd(v) * 255.0f, ys = exp32_scalar(v) * 255.0f;
    err_v = amax(err_v, y - yv);
    err_s = amax(err_s, y - ys);
    if (decided) {
      bad_v += rne(yv) != p;
      bad_s += rne(ys) != p;
    } else {
      amb++;
    }
  }
  for (int t = 1; t < 64; t <<= 1) {
    bad_v += __shfl_xor(bad_v, t);
    bad_s += __shfl_xor(bad_s, t);
    amb += __shfl_xor(amb, t);
    err_v = __builtin_fmaxf(err_v, __shfl_xor(err_v, t));
    err_s = __builtin_fmaxf(err_s, __shfl_xor(err_s, t));
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&res[0], bad_v);
    atomicAdd(&res[1], bad_s);
    atomicMax(&res[2], (unsigned long long)__float_as_uint(err_v));
    atomicMax(&res[3], (unsigned long long)__float_as_uint(err_s));
    atomicAdd(&res[4], amb);
  }
}

}  // namespace

void launch_check_exp255(uint32_t lo, uint32_t hi, unsigned long long *res, hipStream_t s) {
  if (hi <= lo) return;
  check_exp255_kernel<<<4096, 256, 0, s>>>(lo, hi, res);
}

void launch_attn_quant_q(const AttnArgs &a, hipStream_t s) {
  const long groups = (long)a.N * a.nh;
  if (groups <= 0) return;
  attn_quant_q_kernel<<<(unsigned)((groups + 15) / 16), 256, 0, s>>>(a);
}

void launch_attn_prologue(const AttnArgs &a, hipStream_t s) {
  if (a.B <= 0) return;
  if (a.max_n <= kShortSeq) {
    attn_prologue_rows_kernel<false><<<dim3(a.B, a.nh, 2), 512, 0, s>>>(a);
  } else {
    attn_long_stats_kernel<<<dim3(a.B, a.nh, 8), 256, 0, s>>>(a);
    const int parts = (a.max_n + kShortSeq - 1) / kShortSeq;
    attn_prologue_rows_kernel<true><<<dim3(a.B, a.nh, 2 * parts), 512, 0, s>>>(a);
  }
}

void launch_attn_main(const AttnArgs &a, hipStream_t s) {
  if (a.nblocks <= 0) return;
  // 8 runs of (nblocks * nh + 7) / 8 items, one an XCD (see the kernel)
  const dim3 grid(8 * ((a.nblocks * a.nh + 7) / 8));
  if (a.window < 0)
    attn_main_kernel<true><<<grid, 256, 0, s>>>(a);
  else
    attn_main_kernel<false><<<grid, 256, 0, s>>>(a);
}

}  // namespace ixh
