/* vnni.c — MatMul8N (linalg/int8.go:89-155) with the reference's CPU
 * kernel shape: 6x16 tiles of VPDPBUSD (kernel_vnni_amd64.s:13-256), the
 * quantised activations as uint8 q+128 times the PackedB8 panels
 * (int8.go:30: panel p of 16 columns, quad q of 4 depths, column c, byte
 * t at p*kq*64 + q*64 + c*4 + t), the tile rescaled in registers as
 * ((f32(tile) - zc) * sb) * sa (+ C) with separate roundings
 * (kernel_vnni_amd64.s:144-232).
 *
 * TEST INFRASTRUCTURE: part of the CPU oracle library. It exists to time
 * a CPU path of the reference's class beside the GPU (bench.py's
 * cpu_baseline leg, with ixo_set_gemm(1)); the checker path is the plain
 * restatement in indecis_oracle.c, and tests/test_oracle.py checks the two
 * equal bit for bit. AVX-512 VNNI (one zmm per 16 columns) or AVX-VNNI
 * (two ymm) is chosen at run time; without either the plain loops run.
 */
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "indecis_oracle.h"

/* 0: the plain restatement; 1: VNNI tiles where the CPU has them. */
static int g_gemm = 0;
void ixo_set_gemm(int kind) { g_gemm = kind; }

/* 2: AVX-512 VNNI, 1: AVX-VNNI, 0: neither. */
int ixo_vnni_level(void) {
  __builtin_cpu_init();
  if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw")) return 2;
  if (__builtin_cpu_supports("avxvnni")) return 1;
  return 0;
}

int ixo_gemm_kind(void) { return g_gemm && ixo_vnni_level() > 0 ? ixo_vnni_level() : 0; }

/* PackB8's panel layout of w [n][k] (rows = output channels). */
static int8_t *panels_of(const int8_t *w, int k, int n, int kq) {
  const int np = (n + 15) / 16;
  int8_t *p = (int8_t *)calloc((size_t)np * kq * 64, 1);
#pragma omp parallel for schedule(static)
  for (int j = 0; j < n; j++)
    for (int t = 0; t < k; t++)
      p[(size_t)(j / 16) * kq * 64 + (t / 4) * 64 + (j % 16) * 4 + t % 4] = w[(size_t)j * k + t];
  return p;
}

/* Rows of uint8 q+128, depth padded to kq*4 with 128 (the reference's
 * padding: quantizeA fills with 128, int8.go:186-190; 128 * 0 weights). */
static uint8_t *a_u8(const int8_t *q, int ldq, int m, int k, int kq) {
  uint8_t *a = (uint8_t *)malloc((size_t)m * kq * 4 + 64);
#pragma omp parallel for schedule(static)
  for (int i = 0; i < m; i++) {
    uint8_t *r = a + (size_t)i * kq * 4;
    for (int t = 0; t < k; t++) r[t] = (uint8_t)(q[(size_t)i * ldq + t] + 128);
    for (int t = k; t < kq * 4; t++) r[t] = 128;
  }
  return a;
}

__attribute__((target("avx512f,avx512bw,avx512vnni")))
static void tiles_avx512(float *c, int ldc, const uint8_t *a, const float *sa, const int8_t *pb,
                         const float *sb, const float *zc, int m, int n, int kq, int accumulate) {
  const int np = (n + 15) / 16, mt = (m + 5) / 6;
#pragma omp parallel for schedule(dynamic) collapse(2)
  for (int it = 0; it < mt; it++)
    for (int p = 0; p < np; p++) {
      const int i0 = 6 * it, rows = m - i0 < 6 ? m - i0 : 6;
      const int8_t *bp = pb + (size_t)p * kq * 64;
      __m512i acc[6];
      for (int r = 0; r < 6; r++) acc[r] = _mm512_setzero_si512();
      for (int q = 0; q < kq; q++) {
        const __m512i b = _mm512_loadu_si512((const void *)(bp + (size_t)q * 64));
        for (int r = 0; r < rows; r++) {
          int32_t word;
          memcpy(&word, a + (size_t)(i0 + r) * kq * 4 + 4 * q, 4);
          acc[r] = _mm512_dpbusd_epi32(acc[r], _mm512_set1_epi32(word), b);
        }
      }
      const int cols = n - 16 * p < 16 ? n - 16 * p : 16;
      const __mmask16 mk = (__mmask16)((1u << cols) - 1);
      const __m512 vz = _mm512_maskz_loadu_ps(mk, zc + 16 * p);
      const __m512 vs = _mm512_maskz_loadu_ps(mk, sb + 16 * p);
      for (int r = 0; r < rows; r++) {
        __m512 v = _mm512_sub_ps(_mm512_cvtepi32_ps(acc[r]), vz);
        v = _mm512_mul_ps(v, vs);
        v = _mm512_mul_ps(v, _mm512_set1_ps(sa[i0 + r]));
        float *dst = c + (size_t)(i0 + r) * ldc + 16 * p;
        if (accumulate) v = _mm512_add_ps(_mm512_maskz_loadu_ps(mk, dst), v);
        _mm512_mask_storeu_ps(dst, mk, v);
      }
    }
}

__attribute__((target("avx2,avxvnni")))
static void tiles_avx2(float *c, int ldc, const uint8_t *a, const float *sa, const int8_t *pb,
                       const float *sb, const float *zc, int m, int n, int kq, int accumulate) {
  const int np = (n + 15) / 16, mt = (m + 5) / 6;
#pragma omp parallel for schedule(dynamic) collapse(2)
  for (int it = 0; it < mt; it++)
    for (int p = 0; p < np; p++) {
      const int i0 = 6 * it, rows = m - i0 < 6 ? m - i0 : 6;
      const int8_t *bp = pb + (size_t)p * kq * 64;
      __m256i acc[6][2];
      for (int r = 0; r < 6; r++) acc[r][0] = acc[r][1] = _mm256_setzero_si256();
      for (int q = 0; q < kq; q++) {
        const __m256i b0 = _mm256_loadu_si256((const __m256i *)(bp + (size_t)q * 64));
        const __m256i b1 = _mm256_loadu_si256((const __m256i *)(bp + (size_t)q * 64 + 32));
        for (int r = 0; r < rows; r++) {
          int32_t word;
          memcpy(&word, a + (size_t)(i0 + r) * kq * 4 + 4 * q, 4);
          const __m256i w = _mm256_set1_epi32(word);
          acc[r][0] = _mm256_dpbusd_avx_epi32(acc[r][0], w, b0);
          acc[r][1] = _mm256_dpbusd_avx_epi32(acc[r][1], w, b1);
        }
      }
      const int cols = n - 16 * p < 16 ? n - 16 * p : 16;
      for (int r = 0; r < rows; r++) {
        int32_t t[16];
        _mm256_storeu_si256((__m256i *)t, acc[r][0]);
        _mm256_storeu_si256((__m256i *)(t + 8), acc[r][1]);
        float *dst = c + (size_t)(i0 + r) * ldc + 16 * p;
        for (int j = 0; j < cols; j++) {
          const float v = (((float)t[j] - zc[16 * p + j]) * sb[16 * p + j]) * sa[i0 + r];
          dst[j] = accumulate ? dst[j] + v : v;
        }
      }
    }
}

/* The VNNI form of ixo_matmul8_deq; returns 0 when the CPU has no VNNI
 * (nothing computed). */
int ixo_matmul8_deq_vnni(float *c, int ldc, const int8_t *q, int ldq, const float *sa,
                         const int8_t *w, const float *sb, const int32_t *colsum, int m, int k,
                         int n, int accumulate) {
  const int level = ixo_vnni_level();
  if (level == 0) return 0;
  if (m <= 0 || n <= 0) return 1;
  const int kq = (k + 3) / 4;
  int8_t *pb = panels_of(w, k, n, kq);
  uint8_t *a = a_u8(q, ldq, m, k, kq);
  float *zc = (float *)malloc(sizeof(float) * (size_t)(n + 16));
  for (int j = 0; j < n; j++) zc[j] = 128.0f * (float)colsum[j]; /* PackB8, int8.go:72-75 */
  if (level == 2)
    tiles_avx512(c, ldc, a, sa, pb, sb, zc, m, n, kq, accumulate);
  else
    tiles_avx2(c, ldc, a, sa, pb, sb, zc, m, n, kq, accumulate);
  free(pb);
  free(a);
  free(zc);
  return 1;
}

/* Attn8.Attend's integer products (attention8.go:298-376) on VPDPBUSD, for
 * the timed baseline: per query, the scores of 16 keys at a time
 * (uint8 q+128 times the signed keys packed 16 a panel, minus 128 sum k:
 * the reference's kzc) and O = P.V with P (uint8) times V packed 16
 * dimensions a panel. Everything else — Attn8.Prepare, the row max,
 * ExpShift, QuantizeRowU8, the rescaling — is the restatement's own code
 * (ixo_attn_prepare, ixo_exp_shift, the same roundings), so the bits are
 * ixo_attend8's. Needs AVX-512 VNNI; returns 0 (nothing computed)
 * otherwise. */
__attribute__((target("avx512f,avx512bw,avx512vnni")))
static void attend_rows_avx512(float *o, int ldo, const int8_t *qq, const float *sq, const int8_t *kp,
                               const int32_t *kzc, const float *ks, const int8_t *vp, const float *vs,
                               int n, int window, int lanes, float *s, uint8_t *pq) {
  const int nq = (n + 15) / 16 * 4;  /* key quads of a dimension panel */
  for (int i = 0; i < n; i++) {
    int cs = 0, ce = n;
    if (window >= 0) {
      cs = i - window > 0 ? i - window : 0;
      ce = i + window + 1 < n ? i + window + 1 : n;
    }
    uint8_t qa[64];
    for (int d = 0; d < 64; d++) qa[d] = (uint8_t)(qq[(size_t)i * 64 + d] + 128);
    const int p0 = cs / 16, p1 = (ce + 15) / 16;
    for (int p = p0; p < p1; p++) {
      __m512i acc = _mm512_setzero_si512();
      const int8_t *bp = kp + (size_t)p * 16 * 64;
      for (int qd = 0; qd < 16; qd++) {
        int32_t word;
        memcpy(&word, qa + 4 * qd, 4);
        acc = _mm512_dpbusd_epi32(acc, _mm512_set1_epi32(word), _mm512_loadu_si512((const void *)(bp + 64 * qd)));
      }
      int32_t t[16];
      _mm512_storeu_si512((void *)t, _mm512_sub_epi32(acc, _mm512_loadu_si512((const void *)(kzc + 16 * p))));
      for (int c = 0; c < 16; c++) {
        const int j = 16 * p + c;
        if (j >= cs && j < ce) s[j - cs] = ((float)t[c] * ks[j]) * sq[i];
      }
    }
    const int L = ce - cs;
    float m = -__builtin_inff();
    for (int j = 0; j < L; j++) m = s[j] > m ? s[j] : m;
    ixo_exp_shift(s, L, m, lanes);
    /* P over whole key quads, zero outside [cs, ce) */
    const int q0 = cs / 4, q1 = (ce + 3) / 4;
    int32_t sum = 0;
    for (int j = 4 * q0; j < 4 * q1; j++) {
      uint8_t v = 0;
      if (j >= cs && j < ce) {
        v = (uint8_t)(int32_t)ixo_round_half_even(s[j - cs] * 255.0f);
        sum += v;
      }
      pq[j] = v;
    }
    const float sp = 1.0f / (float)sum;
    for (int dp = 0; dp < 4; dp++) {
      __m512i acc = _mm512_setzero_si512();
      const int8_t *bp = vp + (size_t)dp * nq * 64;
      for (int qd = q0; qd < q1; qd++) {
        int32_t word;
        memcpy(&word, pq + 4 * qd, 4);
        acc = _mm512_dpbusd_epi32(acc, _mm512_set1_epi32(word), _mm512_loadu_si512((const void *)(bp + 64 * qd)));
      }
      int32_t t[16];
      _mm512_storeu_si512((void *)t, acc);
      for (int c = 0; c < 16; c++) {
        const int d = 16 * dp + c;
        o[(size_t)i * ldo + d] = (((float)t[c] - 0.0f) * vs[d]) * sp;
      }
    }
  }
}

int ixo_attend8_vnni(float *o, int ldo, const float *q, const float *k, const float *v, int ld, int n,
                     int D, int window, float scale, int lanes) {
  if (ixo_vnni_level() < 2 || D != 64) return 0;
  if (n <= 0) return 1;
  const int np = (n + 15) / 16, nq = np * 4;
  int8_t *qq = (int8_t *)malloc((size_t)n * D), *kq = (int8_t *)malloc((size_t)n * D);
  int8_t *vq = (int8_t *)malloc((size_t)n * D);
  float *sq = (float *)malloc(sizeof(float) * n), *ks = (float *)calloc((size_t)np * 16, sizeof(float));
  float *vs = (float *)malloc(sizeof(float) * D), *mean = (float *)malloc(sizeof(float) * D);
  ixo_attn_prepare(q, k, v, ld, n, D, scale, qq, sq, kq, ks, vq, vs, mean);
  /* K: panel p of 16 keys, quad qd of 4 dimensions, key c, byte t */
  int8_t *kp = (int8_t *)calloc((size_t)np * 16 * 64, 1);
  int32_t *kzc = (int32_t *)calloc((size_t)np * 16, sizeof(int32_t));
  for (int j = 0; j < n; j++) {
    int32_t cs = 0;
    for (int d = 0; d < 64; d++) {
      kp[(size_t)(j / 16) * 1024 + (d / 4) * 64 + (j % 16) * 4 + d % 4] = kq[(size_t)j * 64 + d];
      cs += kq[(size_t)j * 64 + d];
    }
    kzc[j] = 128 * cs;
  }
  /* V: dimension panel dp of 16, key quad qd, dimension c, key byte t */
  int8_t *vp = (int8_t *)calloc((size_t)4 * nq * 64, 1);
  for (int j = 0; j < n; j++)
    for (int d = 0; d < 64; d++)
      vp[(size_t)(d / 16) * nq * 64 + (j / 4) * 64 + (d % 16) * 4 + j % 4] = vq[(size_t)j * 64 + d];
  float *s = (float *)malloc(sizeof(float) * (size_t)np * 16);
  uint8_t *pq = (uint8_t *)calloc((size_t)np * 16 + 4, 1);
  attend_rows_avx512(o, ldo, qq, sq, kp, kzc, ks, vp, vs, n, window, lanes, s, pq);
  free(qq); free(kq); free(vq); free(sq); free(ks); free(vs); free(mean);
  free(kp); free(kzc); free(vp); free(s); free(pq);
  return 1;
}

/* OpenMP threads of the oracle's parallel loops (the timed baseline runs
 * on all cores, then on one). */
#include <omp.h>
void ixo_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int ixo_max_threads(void) { return omp_get_max_threads(); }
