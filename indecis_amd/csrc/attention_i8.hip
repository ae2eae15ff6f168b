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
// normalised by 1/f32(sum P). P (0..255) does not fit int8: it is split
// as 128*(P>>7) + (P&127), two exact MFMAs. Scores need
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
    m = fmax32(m, fmax32(fmax32(fabsf(v[c].x), fabsf(v[c].y)), fmax32(fabsf(v[c].z), fabsf(v[c].w))));
  return m;
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
  return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | (d << 24);
}

__global__ __launch_bounds__(256) void attn_prologue_kernel(AttnArgs a) {
  __shared__ float mean[D];
  __shared__ float vmaxp[3][D];
  __shared__ float vinv[D];
  const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int base = a.offs[b], n = a.offs[b + 1] - base;
  const int slot0 = a.padoff[b];
  const int npad = (n + kKeyPad - 1) / kKeyPad * kKeyPad;
  const int H = a.H, ld = 3 * H;
  const float *qcol = a.qkv + (size_t)base * ld + h * D;
  const float *kcol = qcol + H;
  const float *vcol = qcol + 2 * H;

  if (tid < D) {
    // mean[d]: AddTo over the keys in order, then Scale by 1/n
    // (attention8.go:224-229).
    float m = 0.f;
    int j = 0;
    for (; j + 8 <= n; j += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = kcol[(size_t)(j + u) * ld + tid];
#pragma unroll
      for (int u = 0; u < 8; u++) m = m + v[u];
    }
    for (; j < n; j++) m = m + kcol[(size_t)j * ld + tid];
    mean[tid] = n > 0 ? m * (1.0f / (float)n) : 0.f;
  } else {
    // per-dimension max |v| (MaxAbsTo, attention8.go:259-261), 3 partials
    const int g = (tid >> 6) - 1, d = tid & 63;
    float m = 0.f;
    for (int j = g; j < n; j += 3) m = fmax32(m, fabsf(vcol[(size_t)j * ld + d]));
    vmaxp[g][d] = m;
  }
  __syncthreads();
  if (tid < D) {
    float vs = fmax32(fmax32(vmaxp[0][tid], vmaxp[1][tid]), vmaxp[2][tid]);
    float vi = 0.f;
    if (vs > 0.f) {  // attention8.go:262-269
      vs = vs / 127.0f;
      vi = 1.0f / vs;
    }
    vinv[tid] = vi;
    a.vs[((size_t)b * a.nh + h) * D + tid] = vs;
  }
  __syncthreads();

  int8_t *kp = a.kp + ((size_t)h * a.Npad + slot0) * D;
  float *ks = a.ks + (size_t)h * a.Npad + slot0;
  int8_t *vt = a.vt + (size_t)h * D * a.Npad + slot0;
  for (int j = tid; j < npad; j += 256) {
    if (j >= n) {  // zero slots up to the 64-key boundary
      v4i z = {0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < 4; c++) *(v4i *)(kp + (size_t)j * D + 16 * c) = z;
      ks[j] = 0.f;
      for (int d = 0; d < D; d++) vt[(size_t)d * a.Npad + j] = 0;
      continue;
    }
    float4 v[16];
    // Q: per row, scale*score scale (attention8.go:211-220)
    const float *qr = qcol + (size_t)j * ld;
#pragma unroll
    for (int c = 0; c < 16; c++) v[c] = *(const float4 *)(qr + 4 * c);
    float mx = absmax16(v);
    float s = 0.f, inv = 0.f;
    if (mx != 0.f) {
      s = mx / 127.0f;
      inv = 1.0f / s;
    }
    int8_t *qdst = a.qq + (size_t)(base + j) * H + h * D;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      v4i w;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const float4 f = v[4 * c + u];
        w[u] = pack4(q8(f.x, inv), q8(f.y, inv), q8(f.z, inv), q8(f.w, inv));
      }
      *(v4i *)(qdst + 16 * c) = w;
    }
    a.sq[(size_t)(base + j) * a.nh + h] = s * a.scale;
    // K: centred, per key (attention8.go:240-251)
    const float *kr = kcol + (size_t)j * ld;
#pragma unroll
    for (int c = 0; c < 16; c++) {
      const float4 f = *(const float4 *)(kr + 4 * c);
      v[c] = make_float4(f.x - mean[4 * c], f.y - mean[4 * c + 1], f.z - mean[4 * c + 2],
                         f.w - mean[4 * c + 3]);
    }
    mx = absmax16(v);
    s = 0.f;
    inv = 0.f;
    if (mx != 0.f) {
      s = mx / 127.0f;
      inv = 1.0f / s;
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      v4i w;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const float4 f = v[4 * c + u];
        w[u] = pack4(q8(f.x, inv), q8(f.y, inv), q8(f.z, inv), q8(f.w, inv));
      }
      *(v4i *)(kp + (size_t)j * D + 16 * c) = w;
    }
    ks[j] = s;
    // V: per dimension (quantCols, attention8.go:270-279), transposed
    const float *vr = vcol + (size_t)j * ld;
#pragma unroll
    for (int c = 0; c < 16; c++) {
      const float4 f = *(const float4 *)(vr + 4 * c);
      vt[(size_t)(4 * c) * a.Npad + j] = (int8_t)q8(f.x, vinv[4 * c]);
      vt[(size_t)(4 * c + 1) * a.Npad + j] = (int8_t)q8(f.y, vinv[4 * c + 1]);
      vt[(size_t)(4 * c + 2) * a.Npad + j] = (int8_t)q8(f.z, vinv[4 * c + 2]);
      vt[(size_t)(4 * c + 3) * a.Npad + j] = (int8_t)q8(f.w, vinv[4 * c + 3]);
    }
  }
}

template <bool GLOBAL>
__global__ __launch_bounds__(256) void attn_main_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t Ks[CHUNK * KS];
  __shared__ __attribute__((aligned(16))) int8_t Vs[D * VS];
  __shared__ __attribute__((aligned(16))) float kss[CHUNK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = a.blocks[2 * blockIdx.x], Q0 = a.blocks[2 * blockIdx.x + 1];
  const int h = blockIdx.y;
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
  const int V = a.lanes;
  const int ts = V > 0 ? cs + ((ce - cs) / V) * V : cs;

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

  const int8_t *kglob = a.kp + ((size_t)h * a.Npad + slot0) * D;
  const float *ksglob = a.ks + (size_t)h * a.Npad + slot0;
  const int8_t *vglob = a.vt + (size_t)h * D * a.Npad + slot0;

  auto stage_k = [&](int c0) {
    for (int e = tid; e < CHUNK * 4; e += 256) {
      const int key = e >> 2, part = e & 3;
      v4i w = {0, 0, 0, 0};
      if (c0 + key < npad) w = *(const v4i *)(kglob + (size_t)(c0 + key) * D + 16 * part);
      *(v4i *)&Ks[key * KS + 16 * part] = w;
    }
    for (int e = tid; e < CHUNK; e += 256) kss[e] = c0 + e < npad ? ksglob[c0 + e] : 0.f;
  };
  // V^T with the 8 dwords of each 32-key group permuted so that lane half
  // hf reads the keys 8*(b/4) + 4*hf + b%4 (the S^T accumulator rows) as
  // 16 contiguous bytes.
  auto stage_v = [&](int c0) {
    for (int e = tid; e < D * (CHUNK / 32); e += 256) {
      const int d = e / (CHUNK / 32), g = e % (CHUNK / 32);
      int w[8];
      if (c0 + 32 * g < npad) {
        const v4i lo = *(const v4i *)(vglob + (size_t)d * a.Npad + c0 + 32 * g);
        const v4i hi = *(const v4i *)(vglob + (size_t)d * a.Npad + c0 + 32 * g + 16);
        w[0] = lo[0]; w[1] = lo[1]; w[2] = lo[2]; w[3] = lo[3];
        w[4] = hi[0]; w[5] = hi[1]; w[6] = hi[2]; w[7] = hi[3];
      } else {
#pragma unroll
        for (int u = 0; u < 8; u++) w[u] = 0;
      }
      v4i o0 = {w[0], w[2], w[4], w[6]}, o1 = {w[1], w[3], w[5], w[7]};
      *(v4i *)&Vs[d * VS + 32 * g] = o0;
      *(v4i *)&Vs[d * VS + 32 * g + 16] = o1;
    }
  };
  auto score_tile = [&](int t, int c0) -> v16i {
    v16i acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0;
    const int8_t *kr = &Ks[(t * 32 - c0 + (lane & 31)) * KS + 16 * (lane >> 5)];
    acc = mfma32(*(const v4i *)kr, qb[0], acc);
    acc = mfma32(*(const v4i *)(kr + 32), qb[1], acc);
    return acc;
  };

  // ---- pass 1: row max of the valid scores ----
  float m = -__builtin_huge_valf();
  for (int c0 = bk0; c0 < bk1; c0 += CHUNK) {
    __syncthreads();
    stage_k(c0);
    __syncthreads();
    const int t0 = max(wt0, c0 / 32), t1 = min(wt1, (c0 + CHUNK) / 32);
    for (int t = t0; t < t1; t++) {
      const v16i acc = score_tile(t, c0);
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int j = t * 32 + acc_row(r, lane);
        const float sv = ((float)acc[r] * kss[j - c0]) * sqv;
        if (j >= cs && j < ce) m = fmax32(m, sv);
      }
    }
  }
  m = fmax32(m, __shfl_xor(m, 32));

  // ---- pass 2: P = RNE(255 exp(s - m)), O^T += V^T . P^T ----
  v16i ohi[2], olo[2];
#pragma unroll
  for (int dt = 0; dt < 2; dt++)
#pragma unroll
    for (int r = 0; r < 16; r++) ohi[dt][r] = olo[dt][r] = 0;
  int psum = 0;
  for (int c0 = bk0; c0 < bk1; c0 += CHUNK) {
    __syncthreads();
    stage_k(c0);
    stage_v(c0);
    __syncthreads();
    const int t0 = max(wt0, c0 / 32), t1 = min(wt1, (c0 + CHUNK) / 32);
    for (int t = t0; t < t1; t++) {
      const v16i acc = score_tile(t, c0);
      int hb[16], lb[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int j = t * 32 + acc_row(r, lane);
        const float sv = ((float)acc[r] * kss[j - c0]) * sqv;
        int p = 0;
        if (j >= cs && j < ce) {
          const float v = sv - m;
          float e = exp32_simd(v);
          if (j >= ts) e = exp32_scalar(v);
          p = (int)rne(e * 255.0f);  // QuantizeRowU8 (vec_simd.go:64-91)
        }
        psum += p;
        hb[r] = p >> 7;
        lb[r] = p & 127;
      }
      v4i bh, bl;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        bh[u] = pack4(hb[4 * u], hb[4 * u + 1], hb[4 * u + 2], hb[4 * u + 3]);
        bl[u] = pack4(lb[4 * u], lb[4 * u + 1], lb[4 * u + 2], lb[4 * u + 3]);
      }
#pragma unroll
      for (int dt = 0; dt < 2; dt++) {
        const v4i fv = *(const v4i *)&Vs[(dt * 32 + (lane & 31)) * VS + (t * 32 - c0) + 16 * (lane >> 5)];
        ohi[dt] = mfma32(fv, bh, ohi[dt]);
        olo[dt] = mfma32(fv, bl, olo[dt]);
      }
    }
  }
  psum += __shfl_xor(psum, 32);
  if (!qact) return;
  const float sp = 1.0f / (float)psum;
  const float *vsd = a.vs + ((size_t)b * a.nh + h) * D;
  float *orow = a.ctx + (size_t)(base + qi) * H + h * D;
#pragma unroll
  for (int dt = 0; dt < 2; dt++) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      float o[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int r = 4 * g + u;
        const int d = dt * 32 + acc_row(r, lane);
        const int tile = 128 * ohi[dt][r] + olo[dt][r];
        o[u] = (((float)tile - 0.0f) * vsd[d]) * sp;
      }
      const int d0 = dt * 32 + acc_row(4 * g, lane);
      *(float4 *)(orow + d0) = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
}

}  // namespace

void launch_attn_prologue(const AttnArgs &a, hipStream_t s) {
  if (a.B <= 0) return;
  dim3 grid(a.B, a.nh);
  attn_prologue_kernel<<<grid, 256, 0, s>>>(a);
}

void launch_attn_main(const AttnArgs &a, hipStream_t s) {
  if (a.nblocks <= 0) return;
  dim3 grid(a.nblocks, a.nh);
  if (a.window < 0)
    attn_main_kernel<true><<<grid, 256, 0, s>>>(a);
  else
    attn_main_kernel<false><<<grid, 256, 0, s>>>(a);
}

}  // namespace ixh
