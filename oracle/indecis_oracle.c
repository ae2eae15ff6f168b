/*
 * indecis_oracle.c — CPU restatement of indecis's int8 ModernBERT encoder
 * forward pass. TEST INFRASTRUCTURE ONLY: the checker of the HIP path,
 * never part of it (see indecis_oracle.h).
 *
 * Compile with -ffp-contract=off, no -ffast-math: every float operation
 * below is rounded exactly where the reference rounds it.
 */
#include "indecis_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- scalar building blocks ------------------------------------------- */

static inline float fmax32(float a, float b) { return b > a ? b : a; }
static inline float fmin32(float a, float b) { return b < a ? b : a; }

static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* linalg/int8.go:207-210: (v + 1.5*2^23) - 1.5*2^23, RNE for |v| < 2^22. */
float ixo_round_half_even(float v) {
  const float magic = 12582912.0f;
  return (v + magic) - magic;
}

/* linalg/fastmath.go:36-52 (Cephes expf, separate roundings). */
float ixo_exp32(float x) {
  if (x < -87.3f) return 0.0f;
  x = fmin32(x, 88.7f);
  float n = ixo_round_half_even(x * 1.44269504088896341f);
  float r = x - n * 0.693359375f - n * -2.12194440e-4f;
  float p = 1.9875691500e-4f;
  p = p * r + 1.3981999507e-3f;
  p = p * r + 8.3334519073e-3f;
  p = p * r + 4.1665795894e-2f;
  p = p * r + 1.6666665459e-1f;
  p = p * r + 5.0000001201e-1f;
  float y = p * r * r + r + 1.0f;
  return y * bits_f32((uint32_t)((int32_t)n + 127) << 23);
}

/* One lane of ExpShift's vector body, linalg/vec_simd.go:235-248: v is
 * x - m; the range reduction and polynomial use fused multiply-adds. */
float ixo_exp_simd(float v) {
  int under = v < -87.3f;
  v = fmin32(fmax32(v, -87.3f), 88.7f);
  const float magic = 12582912.0f;
  float n = fmaf(v, 1.44269504088896341f, magic) - magic;
  float r = fmaf(n, -0.693359375f, v);
  r = fmaf(n, 2.12194440e-4f, r);
  float p = fmaf(r, 1.9875691500e-4f, 1.3981999507e-3f);
  p = fmaf(r, p, 8.3334519073e-3f);
  p = fmaf(r, p, 4.1665795894e-2f);
  p = fmaf(r, p, 1.6666665459e-1f);
  p = fmaf(r, p, 5.0000001201e-1f);
  float y = fmaf(p * r, r, r) + 1.0f;
  float pw = bits_f32((uint32_t)((int32_t)n + 127) << 23);
  return under ? 0.0f : y * pw;
}

/* GELU (erf) as geluMulAVX2 computes it, linalg/gelu_amd64.s:173-195 (the
 * same operations as the portable body, vec_simd.go:139-155). */
float ixo_gelu_fma(float x) {
  float t = x * 0.7071067811865476f;
  t = fmin32(fmax32(t, -4.0f), 4.0f);
  float t2 = t * t;
  float p = fmaf(t2, -2.72614225801306e-10f, 2.77068142495902e-08f);
  p = fmaf(t2, p, -2.10102402082508e-06f);
  p = fmaf(t2, p, -5.69250639462346e-05f);
  p = fmaf(t2, p, -7.34990630326855e-04f);
  p = fmaf(t2, p, -2.95459980854025e-03f);
  p = fmaf(t2, p, -1.60960333262415e-02f);
  p = p * t;
  float q = fmaf(t2, -1.45660718464996e-05f, -2.13374055278905e-04f);
  q = fmaf(t2, q, -1.68282697438203e-03f);
  q = fmaf(t2, q, -7.37332916720468e-03f);
  q = fmaf(t2, q, -1.42647390514189e-02f);
  return (0.5f * x) * (1.0f + p / q);
}

/* geluScalar / erf32, linalg/fastmath.go:9-26 (separate roundings). */
float ixo_gelu_scalar(float x) {
  float e = x * 0.7071067811865476f;
  e = fmin32(fmax32(e, -4.0f), 4.0f);
  float x2 = e * e;
  float p = x2 * -2.72614225801306e-10f + 2.77068142495902e-08f;
  p = x2 * p + -2.10102402082508e-06f;
  p = x2 * p + -5.69250639462346e-05f;
  p = x2 * p + -7.34990630326855e-04f;
  p = x2 * p + -2.95459980854025e-03f;
  p = x2 * p + -1.60960333262415e-02f;
  p *= e;
  float q = x2 * -1.45660718464996e-05f + -2.13374055278905e-04f;
  q = x2 * q + -1.68282697438203e-03f;
  q = x2 * q + -7.37332916720468e-03f;
  q = x2 * q + -1.42647390514189e-02f;
  float erf = p / q;
  return 0.5f * x * (1.0f + erf);
}

/* ---- linalg-level operations ------------------------------------------- */

/* linalg/int8.go:38-77. Rounding: math.Round (half away from zero) of the
 * float32 quotient w/s, widened to float64. */
void ixo_pack_b8(const float *b, int k, int n, int transB, int8_t *q,
                 float *scale, int32_t *colsum) {
  for (int j = 0; j < n; j++) {
    float mx = 0.0f;
    for (int t = 0; t < k; t++) {
      float w = transB ? b[(size_t)j * k + t] : b[(size_t)t * n + j];
      mx = fmax32(mx, fabsf(w));
    }
    scale[j] = 0.0f;
    colsum[j] = 0;
    memset(q + (size_t)j * k, 0, (size_t)k);
    if (mx == 0.0f) continue;
    float s = mx / 127.0f;
    scale[j] = s;
    int32_t cs = 0;
    for (int t = 0; t < k; t++) {
      float w = transB ? b[(size_t)j * k + t] : b[(size_t)t * n + j];
      int8_t v = (int8_t)(int)round((double)(w / s));
      q[(size_t)j * k + t] = v;
      cs += v;
    }
    colsum[j] = cs;
  }
}

void ixo_b8_to_panels(const int8_t *q, int k, int n, int8_t *panels) {
  int kq = (k + 3) / 4;
  int np = (n + 15) / 16;
  memset(panels, 0, (size_t)np * kq * 64);
  for (int j = 0; j < n; j++)
    for (int t = 0; t < k; t++)
      panels[(size_t)(j / 16) * kq * 64 + (t / 4) * 64 + (j % 16) * 4 + t % 4] =
          q[(size_t)j * k + t];
}

/* linalg/int8.go:160-191 (Go path) == quant_amd64.s:23-121 (AVX2 path,
 * mean 0, flip): scale = max/127 (VDIVSS), inv = 1/scale (VDIVSS),
 * q = RNE(x*inv) (VCVTPS2DQ / roundHalfEven). A zero row gets scale 0 and
 * q = 0 (the reference fills 128, i.e. 0 after the offset). */
void ixo_quantize_rows(const float *a, int lda, int m, int k, int8_t *q,
                       int ldq, float *sa) {
#pragma omp parallel for schedule(static)
  for (int i = 0; i < m; i++) {
    const float *x = a + (size_t)i * lda;
    int8_t *row = q + (size_t)i * ldq;
    float mx = 0.0f;
    for (int t = 0; t < k; t++) mx = fmax32(mx, fabsf(x[t]));
    sa[i] = 0.0f;
    if (mx == 0.0f) {
      memset(row, 0, (size_t)k);
      continue;
    }
    float s = mx / 127.0f;
    float inv = 1.0f / s;
    sa[i] = s;
    for (int t = 0; t < k; t++)
      row[t] = (int8_t)(int32_t)ixo_round_half_even(x[t] * inv);
  }
}

static int32_t dot_i8(const int8_t *a, const int8_t *b, int k) {
  int32_t s = 0;
  for (int t = 0; t < k; t++) s += (int32_t)a[t] * (int32_t)b[t];
  return s;
}

void ixo_matmul8_tile(const int8_t *q, int ldq, const int8_t *w, int k,
                      int m, int n, int32_t *tile) {
#pragma omp parallel for schedule(static)
  for (int i = 0; i < m; i++) {
    const int8_t *a = q + (size_t)i * ldq;
    for (int j = 0; j < n; j++) {
      const int8_t *b = w + (size_t)j * k;
      int32_t s = 0;
      for (int t = 0; t < k; t++) s += ((int32_t)a[t] + 128) * (int32_t)b[t];
      tile[(size_t)i * n + j] = s;
    }
  }
}

/* The 6x16 VNNI tile rescaled in registers, kernel_vnni_amd64.s:144-232:
 * VCVTDQ2PS, VSUBPS zc, VMULPS sb, VMULPS sa, then VADDPS C. The integer
 * tile is sum (q+128)*w = sum q*w + 128*colsum (exact in int32). */
void ixo_matmul8_deq(float *c, int ldc, const int8_t *q, int ldq,
                     const float *sa, const int8_t *w, const float *sb,
                     const int32_t *colsum, int m, int k, int n,
                     int accumulate) {
  /* the timed CPU baseline's VNNI tiles (vnni.c), when selected */
  if (ixo_gemm_kind() && ixo_matmul8_deq_vnni(c, ldc, q, ldq, sa, w, sb, colsum, m, k, n, accumulate))
    return;
#pragma omp parallel for schedule(static)
  for (int i = 0; i < m; i++) {
    const int8_t *a = q + (size_t)i * ldq;
    float *ci = c + (size_t)i * ldc;
    for (int j = 0; j < n; j++) {
      int32_t tile = dot_i8(a, w + (size_t)j * k, k) + 128 * colsum[j];
      float zc = 128.0f * (float)colsum[j];
      float v = (((float)tile - zc) * sb[j]) * sa[i];
      ci[j] = accumulate ? ci[j] + v : v;
    }
  }
}

void ixo_matmul8(float *c, int ldc, const float *a, int lda, const int8_t *w,
                 const float *sb, const int32_t *colsum, int m, int k, int n,
                 int accumulate) {
  int8_t *q = (int8_t *)malloc((size_t)m * k + 1);
  float *sa = (float *)malloc(sizeof(float) * (size_t)(m + 1));
  ixo_quantize_rows(a, lda, m, k, q, k, sa);
  ixo_matmul8_deq(c, ldc, q, k, sa, w, sb, colsum, m, k, n, accumulate);
  free(q);
  free(sa);
}

/* linalg/int8.go:272-349. */
int ixo_matmul8_outliers(float *c, int ldc, const float *a, int lda, const int8_t *w,
                         const float *sb, const int32_t *colsum, int m, int k, int n,
                         int accumulate, float ratio, int *cols) {
  if (m == 0 || n == 0) return 0;
  /* column maxima of |a| (abs32 clears the sign bit, int8.go:203) */
  float *colmax = (float *)calloc((size_t)k + 1, sizeof(float));
  for (int i = 0; i < m; i++)
    for (int j = 0; j < k; j++) {
      const float v = fabsf(a[(size_t)i * lda + j]);
      colmax[j] = fmax32(colmax[j], v);
    }
  float mean = 0.0f; /* float32, in channel order (int8.go:289-293) */
  for (int j = 0; j < k; j++) mean += colmax[j];
  mean /= (float)k;
  const float thr = ratio * mean;
  int *out = (int *)malloc(sizeof(int) * ((size_t)k + 1));
  int nout = 0;
  for (int j = 0; j < k; j++)
    if (colmax[j] > thr) out[nout++] = j;
  if (nout == 0) {
    free(colmax);
    free(out);
    ixo_matmul8(c, ldc, a, lda, w, sb, colsum, m, k, n, accumulate);
    return 0;
  }
  if (nout > 32) {
    /* keep the largest: selection of the first 32 places, a strictly larger
     * maximum wins (int8.go:304-316) */
    for (int i = 0; i < 32; i++) {
      int best = i;
      for (int x = i + 1; x < nout; x++)
        if (colmax[out[x]] > colmax[out[best]]) best = x;
      const int t = out[i];
      out[i] = out[best];
      out[best] = t;
    }
    nout = 32;
  }
  float *rest = (float *)malloc(sizeof(float) * ((size_t)m * k + 1));
  for (int i = 0; i < m; i++) {
    memcpy(rest + (size_t)i * k, a + (size_t)i * lda, sizeof(float) * (size_t)k);
    for (int t = 0; t < nout; t++) rest[(size_t)i * k + out[t]] = 0.0f;
  }
  ixo_matmul8(c, ldc, rest, k, w, sb, colsum, m, k, n, accumulate);
  float *wd = (float *)malloc(sizeof(float) * ((size_t)n + 1));
  for (int t = 0; t < nout; t++) {
    const int j = out[t];
    for (int col = 0; col < n; col++) wd[col] = (float)w[(size_t)col * k + j] * sb[col];
    for (int i = 0; i < m; i++) {
      const float x = a[(size_t)i * lda + j];
      float *ci = c + (size_t)i * ldc;
      for (int col = 0; col < n; col++) {
        const float p = x * wd[col]; /* separate rounding: no FMA (gc, amd64) */
        ci[col] = ci[col] + p;
      }
    }
    if (cols) cols[t] = j;
  }
  free(wd);
  free(rest);
  free(colmax);
  free(out);
  return nout;
}

/* internal/siglip/encoder.go:36-49. */
void ixo_linear8(float *dst, const float *x, const int8_t *w, const float *sb,
                 const int32_t *colsum, int rows, int k, int n, const float *bias,
                 int outliers, float ratio) {
  if (outliers)
    ixo_matmul8_outliers(dst, n, x, k, w, sb, colsum, rows, k, n, 0, ratio, NULL);
  else
    ixo_matmul8(dst, n, x, k, w, sb, colsum, rows, k, n, 0);
  if (bias)
    for (int r = 0; r < rows; r++)
      for (int col = 0; col < n; col++) dst[(size_t)r * n + col] = dst[(size_t)r * n + col] + bias[col];
}

/* linalg/vec_simd.go:285-327 (lanes V > 0): float32 lane partials of the
 * sum, added in float64; float32 lane partials of fma(d, d, sq); float64
 * tail. lanes == 0: vec_scalar.go:66-81. */
void ixo_layernorm_row(float *o, const float *x, const float *gamma, int n,
                       double eps, int lanes) {
  if (lanes <= 0) {
    double sum = 0.0;
    for (int i = 0; i < n; i++) sum += (double)x[i];
    float mean = (float)(sum / (double)n);
    double var = 0.0;
    for (int i = 0; i < n; i++) {
      double d = (double)(x[i] - mean);
      var += d * d;
    }
    float rstd = (float)(1.0 / sqrt(var / (double)n + eps));
    for (int i = 0; i < n; i++) o[i] = (x[i] - mean) * rstd * gamma[i];
    return;
  }
  int V = lanes;
  float acc[16] = {0};
  int i = 0;
  for (; i + V <= n; i += V)
    for (int l = 0; l < V; l++) acc[l] = acc[l] + x[i + l];
  double sum = 0.0;
  for (int l = 0; l < V; l++) sum += (double)acc[l];
  for (; i < n; i++) sum += (double)x[i];
  float mean = (float)(sum / (double)n);
  float sq[16] = {0};
  i = 0;
  for (; i + V <= n; i += V)
    for (int l = 0; l < V; l++) {
      float d = x[i + l] - mean;
      sq[l] = fmaf(d, d, sq[l]);
    }
  double var = 0.0;
  for (int l = 0; l < V; l++) var += (double)sq[l];
  for (; i < n; i++) {
    double d = (double)(x[i] - mean);
    var += d * d;
  }
  float rstd = (float)(1.0 / sqrt(var / (double)n + eps));
  for (i = 0; i < n; i++) o[i] = ((x[i] - mean) * rstd) * gamma[i];
}

/* GeluMul: the AVX2 kernel covers the multiple-of-16 prefix
 * (kernel_amd64.go:151-160), the SIMD body the next multiples of V, the
 * scalar geluScalar the rest (vec_simd.go:138-159; vec_scalar.go:44-48). */
void ixo_gelu_mul(float *o, const float *a, const float *b, int n, int lanes) {
  int i = n & ~15;
  if (lanes > 0)
    while (i + lanes <= n) i += lanes;
  for (int t = 0; t < i; t++) o[t] = ixo_gelu_fma(a[t]) * b[t];
  for (int t = i; t < n; t++) o[t] = ixo_gelu_scalar(a[t]) * b[t];
}

/* linalg/vec_simd.go:220-264: the vector body on the first n - n%V
 * values, exp32 on the tail; the returned sum as the reference adds it. */
float ixo_exp_shift(float *x, int n, float m, int lanes) {
  if (lanes <= 0) {
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
      float e = ixo_exp32(x[i] - m);
      x[i] = e;
      sum += e;
    }
    return sum;
  }
  int V = lanes;
  float acc[16] = {0};
  int i = 0;
  for (; i + V <= n; i += V)
    for (int l = 0; l < V; l++) {
      float e = ixo_exp_simd(x[i + l] - m);
      x[i + l] = e;
      acc[l] = acc[l] + e;
    }
  float sum = 0.0f;
  for (int l = 0; l < V; l++) sum += acc[l];
  for (; i < n; i++) {
    float e = ixo_exp32(x[i] - m);
    x[i] = e;
    sum += e;
  }
  return sum;
}

/* linalg/vec_simd.go:64-91: the vector body rounds x*inv (a product, then
 * the magic-number add and subtract, each rounded) V values at a time and
 * sums them in int32 lanes; the tail rounds roundHalfEven(x*inv) — the same
 * operations, so with no fused multiply-add in the tail every element has
 * the same formula (vec_scalar.go:23-31 for lanes == 0). The int32 sum is
 * exact in any order (at most 255 n). */
int32_t ixo_quantize_row_u8(uint8_t *dst, const float *x, int n, float inv, int lanes) {
  (void)lanes;
  int32_t sum = 0;
  for (int i = 0; i < n; i++) {
    const int32_t q = (int32_t)ixo_round_half_even(x[i] * inv);
    dst[i] = (uint8_t)q;
    sum += q;
  }
  return sum;
}

/* internal/modernbert/model.go:266-274. */
void ixo_rope_table(double theta, int D, int rows, float *cos_t, float *sin_t) {
  int half = D / 2;
  for (int i = 0; i < half; i++) {
    float inv = (float)(1.0 / pow(theta, (double)(2 * i) / (double)D));
    for (int p = 0; p < rows; p++) {
      double f = (double)((float)p * inv);
      cos_t[(size_t)p * half + i] = (float)cos(f);
      sin_t[(size_t)p * half + i] = (float)sin(f);
    }
  }
}

/* linalg/vec_simd.go:408-425: x1' = x1*c - x2*s, x2' = x2*c + x1*s. */
void ixo_rope(float *x, const float *cos_t, const float *sin_t, int half) {
  for (int i = 0; i < half; i++) {
    float a = x[i], b = x[i + half];
    x[i] = a * cos_t[i] - b * sin_t[i];
    x[i + half] = b * cos_t[i] + a * sin_t[i];
  }
}

/* Quantises c = x - mean like quantRowAVX2 (quant_amd64.s:23-121) without
 * the flip: returns the scale (0 for a zero row, q then all 0). */
static float quant_row_centered(const float *x, const float *mean, int D,
                                int8_t *q) {
  float mx = 0.0f;
  for (int d = 0; d < D; d++) mx = fmax32(mx, fabsf(x[d] - (mean ? mean[d] : 0.0f)));
  if (mx == 0.0f) {
    memset(q, 0, (size_t)D);
    return 0.0f;
  }
  float s = mx / 127.0f;
  float inv = 1.0f / s;
  for (int d = 0; d < D; d++) {
    float c = x[d] - (mean ? mean[d] : 0.0f);
    q[d] = (int8_t)(int32_t)ixo_round_half_even(c * inv);
  }
  return s;
}

/* Attn8.Prepare, AVX2 path (attention8.go:203-280) — the same values as the
 * Go path (attention8.go:99-198): Q per row with the score scale folded
 * into sq; K centred on its mean (sequential float32 AddTo, then Scale by
 * 1/n) and quantised per key; V quantised per dimension. */
void ixo_attn_prepare(const float *q, const float *k, const float *v, int ld,
                      int n, int D, float scale, int8_t *qq, float *sq,
                      int8_t *kq, float *ks, int8_t *vq, float *vs,
                      float *kmean) {
  for (int i = 0; i < n; i++) {
    float s = quant_row_centered(q + (size_t)i * ld, NULL, D, qq + (size_t)i * D);
    sq[i] = s == 0.0f ? 0.0f : s * scale;
  }
  float *mean = kmean;
  for (int d = 0; d < D; d++) mean[d] = 0.0f;
  for (int j = 0; j < n; j++)
    for (int d = 0; d < D; d++) mean[d] = mean[d] + k[(size_t)j * ld + d];
  float inv_n = 1.0f / (float)n;
  for (int d = 0; d < D; d++) mean[d] = mean[d] * inv_n;
  for (int j = 0; j < n; j++)
    ks[j] = quant_row_centered(k + (size_t)j * ld, mean, D, kq + (size_t)j * D);
  float vinv[512];
  for (int d = 0; d < D; d++) {
    float mx = 0.0f;
    for (int j = 0; j < n; j++) mx = fmax32(mx, fabsf(v[(size_t)j * ld + d]));
    vs[d] = mx;
    vinv[d] = 0.0f;
    if (vs[d] > 0.0f) {
      vs[d] = vs[d] / 127.0f;
      vinv[d] = 1.0f / vs[d];
    }
  }
  for (int j = 0; j < n; j++)
    for (int d = 0; d < D; d++)
      vq[(size_t)j * D + d] =
          (int8_t)(int32_t)ixo_round_half_even(v[(size_t)j * ld + d] * vinv[d]);
}

/* Attn8.Attend (attention8.go:298-376), query by query: the result of a
 * query depends only on its own valid keys (TestAttn8Ranges), so the
 * 48-query blocks of the reference need not be reproduced. */
void ixo_attend8(float *o, int ldo, const float *q, const float *k,
                 const float *v, int ld, int n, int D, int window,
                 float scale, int lanes) {
  if (n <= 0) return;
  /* the timed CPU baseline's VNNI products (vnni.c), when selected */
  if (ixo_gemm_kind() && ixo_attend8_vnni(o, ldo, q, k, v, ld, n, D, window, scale, lanes)) return;
  int8_t *qq = (int8_t *)malloc((size_t)n * D);
  int8_t *kq = (int8_t *)malloc((size_t)n * D);
  int8_t *vq = (int8_t *)malloc((size_t)n * D);
  float *sq = (float *)malloc(sizeof(float) * n);
  float *ks = (float *)malloc(sizeof(float) * n);
  float *vs = (float *)malloc(sizeof(float) * D);
  float *mean = (float *)malloc(sizeof(float) * D);
  ixo_attn_prepare(q, k, v, ld, n, D, scale, qq, sq, kq, ks, vq, vs, mean);
  float *s = (float *)malloc(sizeof(float) * n);
  int32_t *pq = (int32_t *)malloc(sizeof(int32_t) * n);
  for (int i = 0; i < n; i++) {
    int cs = 0, ce = n;
    if (window >= 0) {
      cs = i - window > 0 ? i - window : 0;
      ce = i + window + 1 < n ? i + window + 1 : n;
    }
    int L = ce - cs;
    /* S = ((f32(tile) - kzc) * ks) * sq; tile - kzc = sum qq*kq exactly. */
    for (int j = cs; j < ce; j++) {
      int32_t acc = dot_i8(qq + (size_t)i * D, kq + (size_t)j * D, D);
      s[j - cs] = ((float)acc * ks[j]) * sq[i];
    }
    float m = -INFINITY;
    for (int j = 0; j < L; j++) m = fmax32(m, s[j]);
    ixo_exp_shift(s, L, m, lanes);
    /* QuantizeRowU8(prow, valid, 255), vec_simd.go:64-91. */
    int32_t sum = 0;
    for (int j = 0; j < L; j++) {
      pq[j] = (int32_t)ixo_round_half_even(s[j] * 255.0f);
      sum += pq[j];
    }
    float sp = 1.0f / (float)sum;
    for (int d = 0; d < D; d++) {
      int32_t tile = 0;
      for (int j = 0; j < L; j++) tile += pq[j] * (int32_t)vq[(size_t)(cs + j) * D + d];
      o[(size_t)i * ldo + d] = (((float)tile - 0.0f) * vs[d]) * sp;
    }
  }
  free(qq); free(kq); free(vq); free(sq); free(ks); free(vs); free(mean);
  free(s); free(pq);
}

/* Attn8.Attend (attention8.go:298-376) blocked as the reference blocks it:
 * queries [i0, i1) in blocks of 48 (AttnBlock, :26); a block's scores over
 * whole 16-key panels [c0, c1) covering its windows (:313-316), the
 * padding keys of the last panel scoring 0; per row the valid keys
 * (:345-348), ExpShift over them, QuantizeRowU8 and 1/sum P (:349-355);
 * P.V over the block's panels, the other keys' weights 0 (:358-373). Row i
 * goes to o[(i - i0)*ldo]. Test infrastructure: it checks the per-query
 * restatement ixo_attend8 (TestAttn8Ranges). plant != 0 plants a mistake
 * the tests must catch: 1 an exclusive window bound (|i - j| < window),
 * 2 the weights normalised by 1/(255 * sum e) instead of 1/sum P. */
void ixo_attend8_blocked(float *o, int ldo, const float *q, const float *k,
                         const float *v, int ld, int n, int D, int i0, int i1,
                         int window, float scale, int lanes, int plant) {
  if (n <= 0 || i0 >= i1) return;
  enum { BLOCK = 48, PANEL = 16 };
  const int npad = (n + PANEL - 1) / PANEL * PANEL;
  int8_t *qq = (int8_t *)malloc((size_t)n * D);
  int8_t *kq = (int8_t *)calloc((size_t)npad * D, 1);
  int8_t *vq = (int8_t *)calloc((size_t)npad * D, 1);
  float *sq = (float *)malloc(sizeof(float) * n);
  float *ks = (float *)calloc(npad, sizeof(float));
  float *vs = (float *)malloc(sizeof(float) * D);
  float *mean = (float *)malloc(sizeof(float) * D);
  ixo_attn_prepare(q, k, v, ld, n, D, scale, qq, sq, kq, ks, vq, vs, mean);
  float *s = (float *)malloc(sizeof(float) * BLOCK * npad);
  int32_t *p = (int32_t *)malloc(sizeof(int32_t) * BLOCK * npad);
  float sp[BLOCK];
  for (int b0 = i0; b0 < i1; b0 += BLOCK) {
    const int b1 = b0 + BLOCK < i1 ? b0 + BLOCK : i1;
    int c0 = 0, c1 = npad;
    if (window >= 0) {
      c0 = (b0 - window > 0 ? b0 - window : 0) / PANEL * PANEL;
      int e = (b1 - 1 + window + 1 + PANEL - 1) / PANEL * PANEL;
      c1 = e < npad ? e : npad;
    }
    const int W = c1 - c0;
    for (int i = b0; i < b1; i++)
      for (int j = c0; j < c1; j++) {
        int32_t acc = dot_i8(qq + (size_t)i * D, kq + (size_t)j * D, D);
        s[(i - b0) * W + j - c0] = ((float)acc * ks[j]) * sq[i];
      }
    for (int i = b0; i < b1; i++) {
      float *row = s + (size_t)(i - b0) * W;
      int32_t *prow = p + (size_t)(i - b0) * W;
      int cs = 0, ce = (n < c1 ? n : c1) - c0;
      if (window >= 0) {
        const int w = plant == 1 ? window - 1 : window;
        cs = i - w - c0 > 0 ? i - w - c0 : 0;
        ce = (i + w + 1 < n ? i + w + 1 : n) - c0;
      }
      float mx = -INFINITY;
      for (int j = cs; j < ce; j++) mx = fmax32(mx, row[j]);
      const float esum = ixo_exp_shift(row + cs, ce - cs, mx, lanes);
      int32_t sum = 0;
      for (int j = 0; j < W; j++) {
        prow[j] = j >= cs && j < ce ? (int32_t)ixo_round_half_even(row[j] * 255.0f) : 0;
        sum += prow[j];
      }
      sp[i - b0] = plant == 2 ? 1.0f / (255.0f * esum) : 1.0f / (float)sum;
    }
    for (int i = b0; i < b1; i++)
      for (int d = 0; d < D; d++) {
        int32_t tile = 0;
        for (int j = 0; j < W; j++) tile += p[(size_t)(i - b0) * W + j] * (int32_t)vq[(size_t)(c0 + j) * D + d];
        o[(size_t)(i - i0) * ldo + d] = (((float)tile - 0.0f) * vs[d]) * sp[i - b0];
      }
  }
  free(qq); free(kq); free(vq); free(sq); free(ks); free(vs); free(mean); free(s); free(p);
}

/* ---- encoder ------------------------------------------------------------ */

static uint32_t u16_le(const uint16_t *p) { return (uint32_t)*p; }

void ixo_embed_row(const ixo_model *m, int32_t id, float *dst) {
  int H = m->hidden;
  switch (m->emb_format) {
  case IXO_EMB_I8: {
    const int8_t *raw = m->emb_i8 + (size_t)id * H;
    float s = m->emb_i8_scale[id];
    for (int j = 0; j < H; j++) dst[j] = (float)raw[j] * s;
    return;
  }
  case IXO_EMB_BF16: {
    /* newMappedEmbeddings fills a map in row order (embeddings.go:38-44):
     * of two rows for one id, the later one is read */
    for (int e = m->emb_n_exact - 1; e >= 0; e--)
      if (m->emb_exact_ids[e] == id) {
        memcpy(dst, m->emb_exact_rows + (size_t)e * H, sizeof(float) * H);
        return;
      }
    const uint16_t *raw = m->emb_bf16 + (size_t)id * H;
    for (int j = 0; j < H; j++) dst[j] = bits_f32(u16_le(raw + j) << 16);
    return;
  }
  default:
    memcpy(dst, m->emb_f32 + (size_t)id * H, sizeof(float) * H);
  }
}

int ixo_encode(const ixo_model *m, const int32_t *ids, const int32_t *offs,
               int B, float *hidden) {
  const int H = m->hidden, I = m->intermediate, nh = m->heads, D = H / nh;
  const int half = D / 2;
  const int N = offs[B];
  for (int t = 0; t < N; t++)
    if (ids[t] < 0 || ids[t] >= m->vocab) return -1;
  if (N == 0) return 0;
  float *x = (float *)malloc(sizeof(float) * (size_t)N * H);
  float *xn = hidden;
  float *qkv = (float *)malloc(sizeof(float) * (size_t)N * 3 * H);
  float *ctx = (float *)malloc(sizeof(float) * (size_t)N * H);
  float *z = (float *)malloc(sizeof(float) * (size_t)N * 2 * I);
  float *g = (float *)malloc(sizeof(float) * (size_t)N * I);
  int32_t *pos = (int32_t *)malloc(sizeof(int32_t) * (size_t)N);
  int32_t *colsum = (int32_t *)malloc(sizeof(int32_t) * (size_t)(3 * H + 2 * I + H));
  for (int b = 0; b < B; b++)
    for (int t = offs[b]; t < offs[b + 1]; t++) pos[t] = t - offs[b];

  /* infer.go:361-368 */
#pragma omp parallel for schedule(static)
  for (int r = 0; r < N; r++) {
    ixo_embed_row(m, ids[r], xn + (size_t)r * H);
    ixo_layernorm_row(x + (size_t)r * H, xn + (size_t)r * H, m->emb_norm, H,
                      m->norm_eps, m->lanes);
  }
  const float scale = (float)(1.0 / sqrt((double)D));
  for (int l = 0; l < m->layers; l++) {
    const int8_t *wqkv = m->wqkv_q + (size_t)l * 3 * H * H;
    const int8_t *wo = m->wo_q + (size_t)l * H * H;
    const int8_t *wi = m->wi_q + (size_t)l * 2 * I * H;
    const int8_t *womlp = m->womlp_q + (size_t)l * H * I;
    const float *sqkv = m->wqkv_s + (size_t)l * 3 * H, *so = m->wo_s + (size_t)l * H;
    const float *si = m->wi_s + (size_t)l * 2 * I, *somlp = m->womlp_s + (size_t)l * H;
    int global = (l % m->global_every) == 0;
    int window = global ? -1 : m->local_attention / 2;
    const float *ct = global ? m->rope_cos_global : m->rope_cos_local;
    const float *st = global ? m->rope_sin_global : m->rope_sin_local;

    /* infer.go:384-390: layer 0 has no attn_norm, QKV reads x. */
    const float *in = x;
    if (l > 0) {
#pragma omp parallel for schedule(static)
      for (int r = 0; r < N; r++)
        ixo_layernorm_row(xn + (size_t)r * H, x + (size_t)r * H,
                          m->attn_norm + (size_t)l * H, H, m->norm_eps, m->lanes);
      in = xn;
    }
    for (int j = 0; j < 3 * H; j++) colsum[j] = 0;
    for (int j = 0; j < 3 * H; j++)
      for (int t = 0; t < H; t++) colsum[j] += wqkv[(size_t)j * H + t];
    ixo_matmul8(qkv, 3 * H, in, H, wqkv, sqkv, colsum, N, H, 3 * H, 0);
    /* infer.go:391-399 */
#pragma omp parallel for schedule(static)
    for (int r = 0; r < N; r++)
      for (int h = 0; h < 2 * nh; h++)
        ixo_rope(qkv + (size_t)r * 3 * H + (size_t)h * D, ct + (size_t)pos[r] * half,
                 st + (size_t)pos[r] * half, half);
    /* infer.go:484-518 */
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int b = 0; b < B; b++)
      for (int h = 0; h < nh; h++) {
        int off = offs[b], n = offs[b + 1] - offs[b];
        if (n == 0) continue;
        const float *rows = qkv + (size_t)off * 3 * H;
        ixo_attend8(ctx + (size_t)off * H + (size_t)h * D, H, rows + (size_t)h * D,
                    rows + H + (size_t)h * D, rows + 2 * H + (size_t)h * D, 3 * H, n,
                    D, window, scale, m->lanes);
      }
    /* infer.go:403 */
    for (int j = 0; j < H; j++) {
      colsum[j] = 0;
      for (int t = 0; t < H; t++) colsum[j] += wo[(size_t)j * H + t];
    }
    ixo_matmul8(x, H, ctx, H, wo, so, colsum, N, H, H, 1);
    /* infer.go:404-406 */
#pragma omp parallel for schedule(static)
    for (int r = 0; r < N; r++)
      ixo_layernorm_row(xn + (size_t)r * H, x + (size_t)r * H,
                        m->mlp_norm + (size_t)l * H, H, m->norm_eps, m->lanes);
    /* infer.go:414-424 */
    for (int j = 0; j < 2 * I; j++) {
      colsum[j] = 0;
      for (int t = 0; t < H; t++) colsum[j] += wi[(size_t)j * H + t];
    }
    ixo_matmul8(z, 2 * I, xn, H, wi, si, colsum, N, H, 2 * I, 0);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < N; r++)
      ixo_gelu_mul(g + (size_t)r * I, z + (size_t)r * 2 * I, z + (size_t)r * 2 * I + I,
                   I, m->lanes);
    for (int j = 0; j < H; j++) {
      colsum[j] = 0;
      for (int t = 0; t < I; t++) colsum[j] += womlp[(size_t)j * I + t];
    }
    ixo_matmul8(x, H, g, I, womlp, somlp, colsum, N, I, H, 1);
  }
  /* infer.go:427 */
#pragma omp parallel for schedule(static)
  for (int r = 0; r < N; r++)
    ixo_layernorm_row(xn + (size_t)r * H, x + (size_t)r * H, m->final_norm, H,
                      m->norm_eps, m->lanes);
  free(x); free(qkv); free(ctx); free(z); free(g); free(pos); free(colsum);
  return 0;
}

/* infer.go:265-287 */
void ixo_pool(const float *hidden, const int32_t *offs, int B, int H, int cls,
              float *out) {
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; b++) {
    int n = offs[b + 1] - offs[b];
    float *o = out + (size_t)b * H;
    if (n == 0) {
      for (int k = 0; k < H; k++) o[k] = 0.0f;
      continue;
    }
    if (cls) {
      memcpy(o, hidden + (size_t)offs[b] * H, sizeof(float) * H);
      continue;
    }
    for (int k = 0; k < H; k++) {
      double acc = 0.0;
      for (int t = offs[b]; t < offs[b + 1]; t++) acc += (double)hidden[(size_t)t * H + k];
      o[k] = (float)(acc / (double)n);
    }
  }
}

/* heads.go:63-74 */
void ixo_head_logits(const float *x, int T, int H, const float *w,
                     const float *b, int rows, double *z) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; t++)
    for (int r = 0; r < rows; r++) {
      double s = 0.0;
      for (int i = 0; i < H; i++)
        s += (double)w[(size_t)r * H + i] * (double)x[(size_t)t * H + i];
      z[(size_t)t * rows + r] = s + (double)b[r];
    }
}
