// gemm_i8.hip — int8 GEMM on gfx950 i8 MFMA (v_mfma_i32_32x32x32_i8) with
// exact int32 accumulation and the reference's dequantisation fused into
// the epilogue.
//
// Replaces linalg.MatMul8N (linalg/int8.go:89-155) and its VNNI tiles
// (kernel_vnni_amd64.s:13-256). The reference multiplies uint8 activations
// q+128 by int8 weights; MFMA is signed x signed, so the kernel sums q*w and
// rebuilds the reference tile exactly as acc + 128*colsum[n] (int32), then
// rescales it with the same float32 operations in the same order:
// ((f32(tile) - zc[n]) * sb[n]) * sa[m] (+ C).
//
// Block tile 128x128, K step 64, 256 threads (4 waves, 2x2), each wave a
// 64x64 tile of 2x2 MFMA 32x32 blocks. A and B go global -> registers ->
// LDS (double buffered, rows padded to 80 bytes so the 16-byte fragment
// reads of 8 consecutive rows hit distinct banks).
#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace {

constexpr int BM = 128, BN = 128, BK = 64, LS = 80;

template <int EPI>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t As[2][BM * LS];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * LS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ntn = a.Np / BN;
  const int nt = blockIdx.x % ntn, mt = blockIdx.x / ntn;
  const int m0 = mt * BM, n0 = nt * BN;

  int lrow[2], lcol[2];
  const int8_t *ag[2], *bg[2];
  bool aok[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    int c = tid + 256 * i;
    lrow[i] = c >> 2;
    lcol[i] = (c & 3) * 16;
    aok[i] = m0 + lrow[i] < a.M;
    ag[i] = a.A + (size_t)(aok[i] ? m0 + lrow[i] : 0) * a.lda + lcol[i];
    bg[i] = a.B + (size_t)(n0 + lrow[i]) * a.ldb + lcol[i];
  }
  v4i ra[2], rb[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      v4i z = {0, 0, 0, 0};
      ra[i] = aok[i] ? *(const v4i *)(ag[i] + k0) : z;
      rb[i] = *(const v4i *)(bg[i] + k0);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      *(v4i *)&As[buf][lrow[i] * LS + lcol[i]] = ra[i];
      *(v4i *)&Bs[buf][lrow[i] * LS + lcol[i]] = rb[i];
    }
  };

  v16i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

  const int nk = a.Kp / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  const int fr = lane & 31, fk = (lane >> 5) * 16;
  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int s = 0; s < 2; s++) {
      v4i fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; i++)
        fa[i] = *(const v4i *)&As[buf][(wm * 64 + 32 * i + fr) * LS + 32 * s + fk];
#pragma unroll
      for (int j = 0; j < 2; j++)
        fb[j] = *(const v4i *)&Bs[buf][(wn * 64 + 32 * j + fr) * LS + 32 * s + fk];
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = mfma32(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds column fr of each 32x32 block ----
  const int nw = n0 + wn * 64;  // first column of the wave tile
  int ncol[2];
  float zc[2], sb[2];
  int c128[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    ncol[j] = nw + 32 * j + fr;
    zc[j] = a.zc[ncol[j]];
    sb[j] = a.sb[ncol[j]];
    c128[j] = a.c128[ncol[j]];
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int m = m0 + wm * 64 + 32 * i + acc_row(r, lane);
      if (m >= a.M) continue;
      const float sa = a.sa[m];
      if constexpr (EPI == EPI_TILE) {
#pragma unroll
        for (int j = 0; j < 2; j++)
          if (ncol[j] < a.n_valid) a.Ci[(size_t)m * a.ldc + ncol[j]] = acc[i][j][r] + c128[j];
      } else if constexpr (EPI == EPI_GEGLU) {
        // Columns nw..nw+31 hold the GELU input of gated columns
        // nw/2..nw/2+31, columns nw+32..nw+63 their multiplier
        // (Wi rows interleaved by 32 on upload; GeluMul vec_simd.go:125-160).
        const float va = deq(acc[i][0][r] + c128[0], zc[0], sb[0], sa);
        const float vb = deq(acc[i][1][r] + c128[1], zc[1], sb[1], sa);
        const int gc = nw / 2 + fr;
        if (gc < a.n_valid) {
          const float ge = gc < a.n_gelu ? gelu_fma(va) : gelu_scalar(va);
          a.C[(size_t)m * a.ldc + gc] = ge * vb;
        }
      } else if constexpr (EPI == EPI_ROPE) {
        float v0 = deq(acc[i][0][r] + c128[0], zc[0], sb[0], sa);
        float v1 = deq(acc[i][1][r] + c128[1], zc[1], sb[1], sa);
        if (nw < a.rope_cols) {
          // linalg.Rope (vec_simd.go:408-425) on the head whose 64 values
          // are this wave tile: x1' = x1*c - x2*s, x2' = x2*c + x1*s.
          const int p = a.pos[m];
          const float c = a.rope_cos[(size_t)p * 32 + fr];
          const float s = a.rope_sin[(size_t)p * 32 + fr];
          const float x1 = v0, x2 = v1;
          v0 = x1 * c - x2 * s;
          v1 = x2 * c + x1 * s;
        }
        if (nw < a.q_cols) {
          // the query head, quantised per row as Attn8.Prepare does
          // (attention8.go:211-220): the 64 values of the row are this
          // lane's two and those of the 31 other lanes of its half-wave.
          float mx = fmax32(fabsf(v0), fabsf(v1));
#pragma unroll
          for (int t = 1; t < 32; t <<= 1) mx = fmax32(mx, __shfl_xor(mx, t));
          float sc = 0.f, inv = 0.f;
          if (mx != 0.f) {
            sc = mx / 127.0f;
            inv = 1.0f / sc;
          }
          int8_t *qrow = a.qq + (size_t)m * a.q_cols + nw;
          qrow[fr] = (int8_t)q8(v0, inv);
          qrow[32 + fr] = (int8_t)q8(v1, inv);
          if (fr == 0) a.sq[(size_t)m * (a.q_cols / 64) + nw / 64] = sc * a.attn_scale;
          continue;
        }
        float *row = a.C + (size_t)m * a.ldc;
        if (ncol[0] < a.n_valid) row[ncol[0]] = v0;
        if (ncol[1] < a.n_valid) row[ncol[1]] = v1;
      } else {
        float *row = a.C + (size_t)m * a.ldc;
#pragma unroll
        for (int j = 0; j < 2; j++) {
          if (ncol[j] >= a.n_valid) continue;
          const float v = deq(acc[i][j][r] + c128[j], zc[j], sb[j], sa);
          if constexpr (EPI == EPI_ACCUM || EPI == EPI_ACCUM_MLP)
            row[ncol[j]] = row[ncol[j]] + v;
          else
            row[ncol[j]] = v;
        }
      }
    }
  }
}

}  // namespace

void launch_gemm(int epi, const GemmArgs &a, hipStream_t s) {
  if (a.M <= 0) return;
  const int mt = (a.M + BM - 1) / BM, nt = a.Np / BN;
  dim3 grid(mt * nt), block(256);
  switch (epi) {
  case EPI_STORE: gemm_i8_kernel<EPI_STORE><<<grid, block, 0, s>>>(a); break;
  case EPI_ACCUM: gemm_i8_kernel<EPI_ACCUM><<<grid, block, 0, s>>>(a); break;
  case EPI_TILE: gemm_i8_kernel<EPI_TILE><<<grid, block, 0, s>>>(a); break;
  case EPI_GEGLU: gemm_i8_kernel<EPI_GEGLU><<<grid, block, 0, s>>>(a); break;
  case EPI_ROPE: gemm_i8_kernel<EPI_ROPE><<<grid, block, 0, s>>>(a); break;
  case EPI_ACCUM_MLP: gemm_i8_kernel<EPI_ACCUM_MLP><<<grid, block, 0, s>>>(a); break;
  }
}

}  // namespace ixh
