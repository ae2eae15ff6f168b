/*
 * indecis_oracle.h — CPU restatement of indecis's int8 ModernBERT encoder
 * forward pass (the Go reference at Bornholm/indecis), used as the checker
 * of the HIP implementation.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (indecis_amd/) links,
 * loads or calls this code. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the thing results are
 * compared against (or, for cpu_baseline, timed beside the GPU).
 *
 * Every function restates one reference function, cited file:line, with
 * the same float32/float64 operations in the same order: explicit fmaf()
 * where the reference fuses (Go SIMD MulAdd, VFMADD), separate roundings
 * where it does not. Scalar Go code is taken to be unfused: the reference
 * is built at GOAMD64 v1 or v2 (Go's default is v1), where the compiler
 * has no FMA instruction for scalar float code. The Go specification lets
 * an implementation fuse x*y + z, and from GOAMD64 v3 the instruction is
 * there: a v3 build may round exp32, roundHalfEven(x*inv) in quantizeA's
 * and QuantizeRowU8's scalar tails, and the scalar LayerNorm's d*d sum
 * differently (tests/golden/go_semantics.json holds vectors that tell).
 * Build with -ffp-contract=off and without -ffast-math.
 *
 * `lanes` is the Go simd vector length V of the reference host: 0 for a
 * build without GOEXPERIMENT=simd (vec_scalar.go), 4 (SSE/Neon), 8 (AVX2)
 * or 16 (AVX-512). It changes LayerNormRow's partial sums and which
 * elements of an ExpShift row use the scalar exp32 formula.
 */
#ifndef INDECIS_ORACLE_H
#define INDECIS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar building blocks ------------------------------------------- */
float ixo_round_half_even(float v);                 /* linalg/int8.go:207-210 */
float ixo_exp32(float x);                           /* linalg/fastmath.go:36-52 */
float ixo_exp_simd(float v);                        /* linalg/vec_simd.go:235-248 (one lane) */
float ixo_gelu_fma(float x);                        /* linalg/gelu_amd64.s:173-195 */
float ixo_gelu_scalar(float x);                     /* linalg/fastmath.go:9-26 */

/* ---- linalg-level operations ------------------------------------------- */
/* PackB8 (linalg/int8.go:38-77): q is written [n][k] (row j = output
 * channel j, its k depths contiguous), not in the reference's panel order;
 * colsum[j] = sum of q[j][:]. */
void ixo_pack_b8(const float *b, int k, int n, int transB, int8_t *q,
                 float *scale, int32_t *colsum);
/* Reorders q [n][k] into the reference panel layout
 * data[p*kq*64 + qd*64 + c*4 + t] (linalg/int8.go:30,65-68). */
void ixo_b8_to_panels(const int8_t *q, int k, int n, int8_t *panels);

/* quantizeA (linalg/int8.go:160-191, quant_amd64.s:23-121): per row,
 * scale = max|x|/127, q = RNE(x * (1/scale)). q is signed int8 (the
 * reference stores q+128 as uint8). */
void ixo_quantize_rows(const float *a, int lda, int m, int k, int8_t *q,
                       int ldq, float *sa);

/* The reference integer tile (microKernel8Go, linalg/int8.go:214-227) over
 * whole matrices: tile[i][j] = sum_k (q[i][k]+128) * w[j][k]. */
void ixo_matmul8_tile(const int8_t *q, int ldq, const int8_t *w, int k,
                      int m, int n, int32_t *tile);

/* MatMul8N (linalg/int8.go:89-155) given the quantised operands:
 * c[i][j] (+)= ((f32(tile) - 128*colsum[j]) * sb[j]) * sa[i]
 * (kernel_vnni_amd64.s:144-232, Dequantize vec_simd.go:99-119). */
void ixo_matmul8_deq(float *c, int ldc, const int8_t *q, int ldq,
                     const float *sa, const int8_t *w, const float *sb,
                     const int32_t *colsum, int m, int k, int n,
                     int accumulate);

/* MatMul8N from float activations: quantizeA then ixo_matmul8_deq. */
void ixo_matmul8(float *c, int ldc, const float *a, int lda, const int8_t *w,
                 const float *sb, const int32_t *colsum, int m, int k, int n,
                 int accumulate);

/* MatMul8Outliers (linalg/int8.go:272-349): the input channels whose
 * column max |a| exceeds f32(ratio * mean of the column maxima) — the 32
 * largest when more — are zeroed in a copy of a, MatMul8N runs on the
 * copy, then each such channel j (in the chosen order) adds
 * a[i][j] * f32(w[col][j] * sb[col]) to c[i][col]. Writes the chosen
 * channels to cols (room for 32) and returns their number. */
int ixo_matmul8_outliers(float *c, int ldc, const float *a, int lda, const int8_t *w,
                         const float *sb, const int32_t *colsum, int m, int k, int n,
                         int accumulate, float ratio, int *cols);

/* linear.apply (internal/siglip/encoder.go:36-49): MatMul8Outliers (ratio)
 * or MatMul8N (outliers == 0) into dst, then AddTo(dst row, bias) when
 * bias is not NULL (vec_scalar.go:97-101). */
void ixo_linear8(float *dst, const float *x, const int8_t *w, const float *sb,
                 const int32_t *colsum, int rows, int k, int n, const float *bias,
                 int outliers, float ratio);

/* LayerNormRow (linalg/vec_simd.go:285-327; lanes==0: vec_scalar.go:66-81). */
void ixo_layernorm_row(float *o, const float *x, const float *gamma, int n,
                       double eps, int lanes);

/* GeluMul (linalg/vec_simd.go:125-160 with the AVX2 prefix of
 * kernel_amd64.go:151-160): o[i] = gelu(a[i]) * b[i]. */
void ixo_gelu_mul(float *o, const float *a, const float *b, int n, int lanes);

/* ExpShift (linalg/vec_simd.go:220-264; lanes==0: vec_scalar.go:50-58). */
float ixo_exp_shift(float *x, int n, float m, int lanes);

/* QuantizeRowU8 (linalg/vec_simd.go:64-91; lanes==0: vec_scalar.go:23-31):
 * dst[i] = uint8(RNE(x[i]*inv)), the sum of the rounded values. */
int32_t ixo_quantize_row_u8(uint8_t *dst, const float *x, int n, float inv, int lanes);

/* ropeFor (internal/modernbert/model.go:256-277): cos/sin [rows][D/2]. */
void ixo_rope_table(double theta, int D, int rows, float *cos_t, float *sin_t);
/* Rope (linalg/vec_simd.go:408-425), in place on 2*half values. */
void ixo_rope(float *x, const float *cos_t, const float *sin_t, int half);

/* Attend8 = Attn8.Prepare + Attn8.Attend (linalg/attention8.go:70-376):
 * o[i*ldo + d] for n queries of D values, q/k/v rows ld floats apart.
 * window < 0: global; else |i-j| <= window. */
void ixo_attend8(float *o, int ldo, const float *q, const float *k,
                 const float *v, int ld, int n, int D, int window,
                 float scale, int lanes);

/* The CPU baseline's GEMM (vnni.c): ixo_set_gemm(1) makes MatMul8N use
 * 6x16 VPDPBUSD tiles (AVX-512 VNNI or AVX-VNNI, chosen at run time; the
 * same bits); 0 (default) the plain restatement. ixo_vnni_level: 2
 * AVX-512 VNNI, 1 AVX-VNNI, 0 none; ixo_gemm_kind: the level in use. */
void ixo_set_gemm(int kind);
int ixo_vnni_level(void);
int ixo_gemm_kind(void);
int ixo_matmul8_deq_vnni(float *c, int ldc, const int8_t *q, int ldq, const float *sa,
                         const int8_t *w, const float *sb, const int32_t *colsum, int m, int k,
                         int n, int accumulate);
void ixo_set_threads(int n);
int ixo_max_threads(void);
int ixo_attend8_vnni(float *o, int ldo, const float *q, const float *k, const float *v, int ld, int n,
                     int D, int window, float scale, int lanes);

/* Attn8.Attend blocked as the reference blocks it (48 queries, 16-key
 * panels), queries [i0, i1) into o[(i - i0)*ldo]; plant 1 or 2 plants a
 * mistake (exclusive window bound; 1/(255 sum e) normalisation). */
void ixo_attend8_blocked(float *o, int ldo, const float *q, const float *k,
                         const float *v, int ld, int n, int D, int i0, int i1,
                         int window, float scale, int lanes, int plant);

/* Attn8.Prepare outputs (attention8.go:203-280), for checking the GPU
 * attention prologue: qq [n][D] signed, sq [n]; kq [n][D] signed
 * (centred), ks [n]; vq [n][D] signed, vs [D]; kmean [D]. */
void ixo_attn_prepare(const float *q, const float *k, const float *v, int ld,
                      int n, int D, float scale, int8_t *qq, float *sq,
                      int8_t *kq, float *ks, int8_t *vq, float *vs,
                      float *kmean);

/* ---- encoder ------------------------------------------------------------ */
enum { IXO_EMB_F32 = 0, IXO_EMB_BF16 = 1, IXO_EMB_I8 = 2 };

typedef struct {
  int hidden, layers, heads, intermediate, vocab;
  double norm_eps;
  int global_every;    /* Config.GlobalEvery */
  int local_attention; /* Config.LocalAttention: window = local_attention/2 */
  int lanes;
  /* weights, layer-major, quantised as PackB8 does: q [n][k], scale [n] */
  const int8_t *wqkv_q;  const float *wqkv_s;   /* [L][3H][H], [L][3H] */
  const int8_t *wo_q;    const float *wo_s;     /* [L][H][H],  [L][H]  */
  const int8_t *wi_q;    const float *wi_s;     /* [L][2I][H], [L][2I] */
  const int8_t *womlp_q; const float *womlp_s;  /* [L][H][I],  [L][H]  */
  const float *attn_norm;  /* [L][H], row 0 unused (layer 0 has none) */
  const float *mlp_norm;   /* [L][H] */
  const float *emb_norm;   /* [H] */
  const float *final_norm; /* [H] */
  int emb_format;
  const float *emb_f32;    /* [V][H] */
  const uint16_t *emb_bf16;/* [V][H] */
  const int32_t *emb_exact_ids; const float *emb_exact_rows; int emb_n_exact;
  const int8_t *emb_i8; const float *emb_i8_scale; /* [V][H], [V] */
  /* RoPE tables [rope_rows][D/2] for the global and local thetas */
  const float *rope_cos_global, *rope_sin_global;
  const float *rope_cos_local, *rope_sin_local;
  int rope_rows;
} ixo_model;

/* Embedding row (internal/modernbert/infer.go:52-59, embeddings.go:48-68). */
void ixo_embed_row(const ixo_model *m, int32_t id, float *dst);

/* run (internal/modernbert/infer.go:304-430): final states [N][H] of the
 * sequences laid end to end (offs[B] = N). Returns 0, or -1 for an id out
 * of the vocabulary (infer.go:308-312). */
int ixo_encode(const ixo_model *m, const int32_t *ids, const int32_t *offs,
               int B, float *hidden);

/* Pooling (infer.go:265-287): mean (float64 accumulation) or first token. */
void ixo_pool(const float *hidden, const int32_t *offs, int B, int H, int cls,
              float *out);

/* head.logits (heads.go:63-74): z[t][r] = sum_i f64(w[r][i])*f64(x[t][i]) + f64(b[r]). */
void ixo_head_logits(const float *x, int T, int H, const float *w,
                     const float *b, int rows, double *z);

#ifdef __cplusplus
}
#endif
#endif
