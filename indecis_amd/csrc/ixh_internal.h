// ixh_internal.h — kernel launchers shared by the C-ABI (ixh_api.cpp) and
// the kernel sources. Host-side only types; no torch, no reference code.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "host_sched.h"

struct ixh_model;   // include/indecis_hip.h
struct ixh_config;
struct ixh_tokenizer;

namespace ixh {

// Compute units of the current device (cached per device; 256 if the query
// fails), for grids of resident workgroups.
int device_cus();

// ---- int8 GEMM ----------------------------------------------------------
// C = epilogue(A . B^T): A int8 [M][lda] (signed activations, zero
// padding to Kp), B int8 [Np][ldb] (weights, one row per output channel,
// zero padding), Kp a multiple of 64, Np a multiple of 128.
enum GemmEpi {
  EPI_STORE = 0,   // C[m][n] = deq
  EPI_ACCUM = 1,   // C[m][n] += deq            (Wo, WoMLP residual)
  EPI_TILE = 2,    // Ci[m][n] = reference int32 tile (tests)
  EPI_GEGLU = 3,   // G[m][j] = gelu(deq a)*deq b, B rows interleaved by 32
  EPI_ROPE = 4,    // C[m][n] = deq, RoPE on columns < rope_cols
  EPI_ACCUM_MLP = 5,  // EPI_ACCUM as a kernel of its own (WoMLP), for profiles
};

struct GemmArgs {
  const int8_t *A;
  int lda;
  const int8_t *B;
  int ldb;
  const int8_t *Bk;      // the same weights K-blocked [Kp/32][Np][32] (gemm_as), or nullptr
  int M, Np, Kp;
  const float *sa;       // [M]
  const float *sb;       // [Np]
  const float *zc;       // [Np] 128*colsum as float
  const int32_t *c128;   // [Np] 128*colsum
  float *C;              // EPI_STORE/ACCUM/ROPE: [M][ldc]; EPI_GEGLU: [M][ldc] gated
  int ldc;
  int32_t *Ci;           // EPI_TILE
  int n_valid;           // output columns stored (of the B rows; GEGLU: gated cols)
  // EPI_ROPE
  const float *rope_cos, *rope_sin;  // [rows][32]
  const int32_t *pos;                // [M]
  int rope_cols;                     // columns < rope_cols are rotated (2H)
  int lanes;                         // Go simd width, for the GeGLU tail rule
  int n_gelu;                        // GEGLU: I (gated width), for the tail rule
  // EPI_ROPE: columns < q_cols are the queries, quantised per (row, head)
  // into qq [M][q_cols] and sq [M][q_cols/64] (times attn_scale) instead
  // of being stored in C
  int q_cols;
  int8_t *qq;
  float *sq;
  float attn_scale;
  int tile_cfg;  // gemm_i8: 0: 128x128 tiles, 2 LDS stages; 1: 256x128, 3; 2: 128x128, 3
  // every weight row has 127 * sum|w| + |128 * colsum| < 2^24: the
  // reference's f32(acc + 128*colsum) - zc is then f32(acc) for any int8
  // activations, and kernels that read this may dequantise as
  // f32(acc) * sb * sa (the fused QKV kernel does)
  int small = 0;
  // EPI_GEGLU on gemm_as: when not null, rmax[m][c] = max |G[m][32c .. 32c+31]|
  // for c < rmax_ld (the row maxima the fused residual GEMM quantises by)
  float *rmax = nullptr;
  int rmax_ld = 0;
  // fused QKV kernel: when not null, A K-blocked as [Kp/32][ak_rows][32]
  // (32 bytes of a row per K-block, a sequence's rows contiguous)
  const int8_t *Ak = nullptr;
  int ak_rows = 0;
};

void launch_gemm(int epi, const GemmArgs &a, hipStream_t s);

// The A-stationary GEMM (gemm_as.hip) for EPI_STORE/ACCUM/ACCUM_MLP/TILE/
// GEGLU: needs Bk, Np a multiple of 256 and Kp one of 256, 512, 768, 1152;
// returns false (nothing launched) otherwise.
bool gemm_as_supported(const GemmArgs &a);
bool launch_gemm_as(int epi, const GemmArgs &a, hipStream_t s);
// The warp-specialised GEMM (gemm_ws.hip): same operands and conditions as
// gemm_as; MFMA waves and epilogue waves hand blocks over through LDS.
bool launch_gemm_ws(int epi, const GemmArgs &a, hipStream_t s);

// The residual GEMMs fused with the quantisation of their input and the
// LayerNorm + quantisation of their output (gemm_res.hip): X[m][:H] +=
// deq(quantizeA(A[m][:K]) . B^T), then, with gamma, Q/SA = quantizeA(
// LayerNorm(X[m], gamma)). Needs Np >= H (a multiple of 32) and (H, Kp)
// one of (768, 768), (768, 1152), (384, 384), (384, 1152), (256, 256),
// (256, 512); returns false (nothing launched) otherwise.
struct ResArgs {
  const float *A;        // [M][lda] float32 input rows, K valid columns (K % 4 == 0)
  int lda, K, Kp;
  // when not null: amax[m][p] (p < P) are maxima of |A[m]| over parts of
  // the row that together cover it (written by the kernel that wrote A):
  // the rows are then quantised K step by K step inside the K loop
  const float *amax;
  int P;
  const int8_t *Bk;      // weights K-blocked [Kp/32][Np][32]
  int Np;
  const float *sb, *zc;  // [Np]
  const int32_t *c128;   // [Np]
  float *X;              // [M][H] residual, updated in place
  int M, H;
  const float *gamma;    // [H] LayerNorm weight of the new x, or nullptr (no LayerNorm)
  double eps;
  int8_t *Q;             // [M][ldq] quantised LayerNorm output
  int ldq;
  float *SA;             // [M] its scales
  // when not null, Q is written K-blocked here instead ([H/32][qk_rows][32],
  // the fused QKV kernel's K-blocked input)
  int8_t *Qk = nullptr;
  int qk_rows = 0;
  int small = 0;  // the weights' dequantisation bound holds (GemmArgs::small)
};
bool gemm_res_supported(int H, int Kp, int Np);
bool launch_gemm_res(const ResArgs &a, int lanes, hipStream_t s);

// The MLP block in one kernel (mlp_res.hip): X[m][:H] += deq(quantizeA(
// GeGLU(deq(Aq[m] . Wi^T))) . WoMLP^T), then, with gamma, Q/SA =
// quantizeA(LayerNorm(X[m], gamma)). Aq/sa and Q/SA may be the same
// buffers: a workgroup reads its rows before it writes them. Needs (H, I)
// one of (768, 1152), (256, 512), unpadded, and every gated column in the
// FMA-form GELU (n_gelu == I); returns false (nothing launched) otherwise.
struct MlpArgs {
  const float *Af;       // launch_wo_res: [M][lda] float32 ctx rows
  int lda;
  const int8_t *Aq;      // [M][ldq] quantised mlp_norm rows (H bytes valid)
  const float *sa;       // [M] their scales
  const int8_t *Bi;      // Wi K-blocked [H/32][Npi][32], rows interleaved by 32
  int Npi;               // 2I
  const float *sbi, *zci;  // [Npi]
  const int32_t *c128i;    // [Npi]
  int n_gelu;            // gated columns below it take the FMA-form GELU (must be I)
  const int8_t *Bo;      // WoMLP K-blocked [I/32][Npo][32]
  int Npo = 0;           // its rows a K-block (H padded; 0: H)
  const float *sbo, *zco;  // [H]
  const int32_t *c128o;    // [H]
  float *X;              // [M][H] residual, updated in place
  int M, H, I;
  const float *gamma;    // [H] LayerNorm weight of the new x, or nullptr
  double eps;
  int8_t *Q;             // [M][ldq] quantised LayerNorm output
  int ldq;
  float *SA;             // [M] its scales
  // when not null, Q is written K-blocked here instead ([H/32][qk_rows][32],
  // the fused QKV kernel's K-blocked input)
  int8_t *Qk = nullptr;
  int qk_rows = 0;
};
bool mlp_res_supported(int H, int I, int KpH, int KpI, int Npi);
bool launch_mlp_res(const MlpArgs &a, int lanes, hipStream_t s);
// The MLP block 64 rows a workgroup with transposed products
// (mlp_block.hip): same arguments and results as launch_mlp_res; needs
// (H, I) one of (768, 1152), (384, 1152), (256, 512), unpadded, and
// n_gelu == I; returns false (nothing launched) otherwise. The caller
// also guarantees the dequantisation bound of both matrices: every row
// has 127 * sum |w| + |128 * colsum| < 2^24 (the kernel dequantises as
// f32(acc) * sb * sa, which equals the reference's order then).
bool mlp_block_supported(int H, int I, int KpH, int KpI, int Npi);
bool launch_mlp_block(const MlpArgs &a, int lanes, hipStream_t s);
// The same kernel for Wo (mlp_res.hip, WO mode): X[m] += deq(quantizeA(
// Af[m][:H]) . Wo^T), then Q/SA = quantizeA(LayerNorm(X[m], gamma)); Bo,
// sbo, zco, c128o are Wo's (K-blocked [H/32][H][32]). Needs H 768 or 256,
// unpadded, and gamma.
bool wo_res_supported(int H, int KpH, int Np);
bool launch_wo_res(const MlpArgs &a, int lanes, hipStream_t s);

// ---- host helpers (ixh_api.cpp) ---------------------------------------------
// Sets the calling thread's ixh_last_error message; returns code.
int set_error(int code, const char *msg);
// EncodeMax of n texts on worker threads, one id vector a text (tokenizer.cpp).
int tokenize_texts(const ixh_tokenizer *t, const char *const *texts, const int64_t *lens, int n, int max_len,
                   int threads, std::vector<std::vector<int32_t>> &per);
// The config a model handle was created with.
void model_config(const ::ixh_model *m, ::ixh_config *out);

// ---- MatMul8Outliers / linear.apply (outliers.hip) --------------------------
// out[j] |= bits of max_i |a[i][j]| (out zeroed first)
void launch_colmax(const float *a, int ld, int m, int k, unsigned *out, hipStream_t s);
// a[i][cols[t]] = 0
void launch_zero_cols(float *a, int ld, int m, const int *cols, int ncols, hipStream_t s);
// c[i][col] = (c + a[i][cols[0]] * w[0][col] + ...) + bias[col] (bias may be null)
void launch_outlier_epilogue(float *c, int ldc, int m, int n, const float *a, int lda, const int *cols,
                             int ncols, const float *w, const float *bias, hipStream_t s);

// ---- row kernels ----------------------------------------------------------
struct RowArgs {
  int M, H;
  const float *x;          // [M][H] input (unless gather)
  // gather (embedding row, internal/modernbert/infer.go:52-59)
  const int32_t *ids;
  int vocab;               // ids are clamped into [0, vocab) (a bad batch's result is discarded)
  int emb_format;          // 0 f32, 1 bf16 (+exact rows), 2 int8 (+row scale)
  const float *emb_f32;
  const uint16_t *emb_bf16;
  const int32_t *exact_slot; // [V] -1 or index into exact_rows
  const float *exact_rows;
  const int8_t *emb_i8;
  const float *emb_i8_scale;
  const float *gamma;      // LayerNorm weight, nullptr: no LayerNorm
  double eps;
  int lanes;
  float *out;              // [M][H] f32 result, or nullptr
  int8_t *q;               // [M][ldq] quantised result, or nullptr
  int ldq;
  float *sa;               // [M]
  int seg = 1;             // lanes 8/16: segment kernel (1) or whole-row LDS kernel (0)
  // when not null (with q), the quantised rows go here K-blocked instead,
  // [H/32][qk_rows][32] (H a multiple of 32; nothing is written to q)
  int8_t *qk = nullptr;
  int qk_rows = 0;
};
void launch_rownorm(const RowArgs &a, hipStream_t s);

// Per-row int8 quantisation (quantizeA) of f32 rows [M][ld] into [M][ldq].
void launch_quant_rows(const float *x, int ld, int M, int K, int8_t *q, int ldq,
                       float *sa, hipStream_t s);

// Token positions and padded key slots from cumulative offsets.
void launch_positions(const int32_t *offs, const int32_t *padoff, int B,
                      int32_t *pos, int32_t *slot, hipStream_t s);

// Mean (float64 accumulation) or first-token pooling, [B][H]; N is the
// batch's token count (it sizes the kernel's ring).
void launch_pool(const float *xn, const int32_t *offs, int B, int N, int H, int cls,
                 float *out, hipStream_t s);

// head.logits (heads.go:63-74) over T rows.
void launch_head_logits(const float *x, int T, int H, const double *w,
                        const float *b, int rows, double *z, hipStream_t s);

// ---- attention ------------------------------------------------------------
struct AttnArgs {
  const float *qkv;        // [N][3H], RoPE applied
  int H, nh, N;
  const int32_t *offs;     // [B+1]
  const int32_t *padoff;   // [B+1] start of each sequence's key slots
  int B;
  int max_n;               // longest sequence (picks the prologue variant)
  float scale;             // 1/sqrt(D)
  int window;              // <0 global
  int lanes;
  // prologue outputs / main inputs
  int8_t *qq;              // [N][H]
  float *sq;               // [N][nh]
  int8_t *kp;              // [nh][Npad][64]
  float *ks;               // [nh][Npad]
  int8_t *vt;              // [nh][64][Npad]
  float *vs;               // [B][nh][64]
  float *kstat;            // [B][nh][2][64] K mean, 1/V scale (sequences over 512 keys)
  int Npad;
  const int32_t *blocks;   // [nblocks][2]: (sequence, first query)
  int nblocks;
  float *ctx;              // [N][H]
  float *rmax = nullptr;   // when not null: [N][nh] max |ctx| of each (row, head)
};
void launch_attn_quant_q(const AttnArgs &a, hipStream_t s);
void launch_attn_prologue(const AttnArgs &a, hipStream_t s);
void launch_attn_main(const AttnArgs &a, hipStream_t s);
// exp255_fast against the reference exponentials over float bits [lo, hi):
// res[5] (zeroed by the caller) = {bad simd, bad scalar, max err simd bits,
// max err scalar bits, undecided}
void launch_check_exp255(uint32_t lo, uint32_t hi, unsigned long long *res, hipStream_t s);
void launch_check_gelu(unsigned long long *res, hipStream_t s);
// blocks workgroups of 4 waves, each wave 4 * iters int8 MFMAs 32x32x32;
// out: blocks * 256 ints (checksums)
void launch_mfma_rate(int blocks, int iters, int *out, hipStream_t s);

constexpr int kAttnQBlock = 128;  // queries per workgroup (4 waves x 32)
constexpr int kKeyPad = 64;       // key slots of a sequence are padded to this

// The QKV projection fused with the attention prologue (qkv_attn.hip), for
// batches whose sequences have at most kQkvSeqMax keys: g as for the
// EPI_ROPE GEMM (A, sa, B, sb, zc, c128, Kp, rope tables, pos, qq, sq,
// attn_scale; C unused), a as for launch_attn_prologue (qkv unused);
// order[B]: the sequences, longest first; heads: per workgroup, 1 or 2
// (2 only for an even head count where the device grants the LDS).
constexpr int kQkvSeqMax = 512;
void launch_qkv_attn(const GemmArgs &g, const AttnArgs &a, const int32_t *order, int heads, hipStream_t s);
// The fused QKV kernel's K-blocked input ([Kp/32][rows][32]): supported
// for Kp a multiple of 128 whose weight rows fit in its LDS.
bool qkv_kblock_supported(int Kp);

}  // namespace ixh
