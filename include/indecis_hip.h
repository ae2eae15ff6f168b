/*
 * indecis_hip.h — C ABI of the MI355X (gfx950) int8 ModernBERT encoder.
 *
 * This is the drop-in boundary for indecis's int8 encoder forward pass:
 * the body of internal/modernbert.(*Model).run (infer.go:304-430) and the
 * linalg entry points it calls. A cgo file built under the `rocm` tag
 * binds these functions; EncodeSeqs, EncodeTokens and
 * Encode keep their Go signatures, so model.go:425, batch.go:71,
 * spans.go:423, distill.go:121 and open.go:131 switch with no change.
 *
 * Conventions: plain pointers and sizes, no GPU types in signatures. Host
 * pointers are borrowed for the call only. Every function returns 0 on
 * success or a nonzero IXH_E* code; ixh_last_error() then gives the
 * message of the calling thread's last failure, worded as the reference
 * words its errors where it has one ("modernbert: id 5 out of
 * vocabulary"). Model handles are safe to share between threads once
 * their weights are set: each call takes its own stream and workspace
 * from a pool (the reference's workspaces, infer.go:229-235,342-346).
 */
#ifndef INDECIS_HIP_H
#define INDECIS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  IXH_OK = 0,
  IXH_EINVAL = 1,   /* bad argument (the reference panics or errors) */
  IXH_ERANGE = 2,   /* id out of vocabulary (infer.go:310-312) */
  IXH_ESTATE = 3,   /* weights missing (infer.go:170-182) */
  IXH_EHIP = 4,     /* HIP runtime error ("modernbert: hip: ...") */
  IXH_ENOMEM = 5,
  IXH_EFORMAT = 6,  /* unreadable or malformed weights file (safetensors.go:112-224) */
};

/* modernbert.Config (internal/modernbert/model.go:26-49) plus the Go simd
 * vector width of the host whose results are reproduced. */
typedef struct ixh_config {
  int hidden;          /* hidden_size */
  int layers;          /* num_hidden_layers */
  int heads;           /* num_attention_heads (head dim must be 64) */
  int intermediate;    /* intermediate_size */
  int vocab;           /* vocab_size */
  double norm_eps;     /* norm_eps */
  int global_every;    /* global_attn_every_n_layers (IsGlobal: l%n == 0) */
  int local_attention; /* local_attention; window = local_attention/2 */
  double global_theta; /* global_rope_theta */
  double local_theta;  /* local_rope_theta */
  int pooling;         /* IXH_POOL_MEAN or IXH_POOL_CLS (Config.CLS) */
  int lanes;           /* Go simd V: 0 (no simd build), 4, 8 or 16 */
} ixh_config;

enum { IXH_POOL_MEAN = 0, IXH_POOL_CLS = 1 };
enum { IXH_MAT_QKV = 0, IXH_MAT_O = 1, IXH_MAT_I = 2, IXH_MAT_OMLP = 3 };
enum { IXH_NORM_EMB = 0, IXH_NORM_ATTN = 1, IXH_NORM_MLP = 2, IXH_NORM_FINAL = 3 };
/* Weight layouts: rows = q[n][k] (row j is output channel j, the
 * transformers [out, in] layout PackB8 reads with transB); panels = the
 * PackedB8.data order p*kq*64 + q*64 + c*4 + t (linalg/int8.go:30). */
enum { IXH_LAYOUT_ROWS = 0, IXH_LAYOUT_PANELS = 1 };
enum { IXH_OUT_POOLED = 0, IXH_OUT_TOKENS = 1 };

typedef struct ixh_model ixh_model;
typedef struct ixh_packed_b8 ixh_packed_b8;

/* Message of this thread's last failure ("" if none). */
const char *ixh_last_error(void);

/* Number of visible GPUs. */
int ixh_device_count(int *count);

/* ---- model (internal/modernbert) -------------------------------------- */

/* Replaces modernbert.FromTensors + packs() (model.go:181-234,
 * infer.go:184-219) for the int8 path: creates an empty model on device;
 * the set_* calls upload what PackB8 and the tensors hold. */
int ixh_model_create(const ixh_config *cfg, int device, ixh_model **out);
void ixh_model_destroy(ixh_model *m);

/* One packed int8 matrix of a layer (packedLayer, infer.go:84-87,
 * 209-216): q int8 and the per-output-channel scale of PackedB8
 * (int8.go:27-34); colsum is derived from q. Shapes: QKV [3H][H], O [H][H],
 * I [2I][H] (GELU input rows then gate rows, model.go:96), OMLP [H][I]. */
int ixh_model_set_matrix(ixh_model *m, int layer, int which, const int8_t *q,
                         const float *scale, int layout);

/* LayerNorm weights (no bias): EMB and FINAL ignore layer; ATTN of layer 0
 * does not exist (model.go:92) and is rejected. */
int ixh_model_set_norm(ixh_model *m, int which, int layer, const float *gamma);

/* Embedding table (embRow infer.go:52-59, mappedEmbeddings.Row
 * embeddings.go:48-68): float32 [V][H]; or bf16 [V][H] with n_exact float32
 * rows overriding ids exact_ids; or int8 [V][H] with one scale per row. */
int ixh_model_set_embeddings_f32(ixh_model *m, const float *table);
int ixh_model_set_embeddings_bf16(ixh_model *m, const uint16_t *table,
                                  const int32_t *exact_ids,
                                  const float *exact_rows, int n_exact);
int ixh_model_set_embeddings_i8(ixh_model *m, const int8_t *table,
                                const float *row_scale);

/* Every weight of the model from an indecis model.safetensors (Load,
 * model.go:640-740; FromTensors names, internal/modernbert/model.go:
 * 181-234, "model." prefix accepted): the embedding table uploaded in its
 * stored format (I8 + "indecis.embeddings.scale", BF16 + the exact rows,
 * or F32/F16 decoded), each layer matrix decoded (F32, BF16, F16, I8) and
 * packed by PackB8 (linalg/int8.go:38-77) on the host one at a time, the
 * LayerNorm weights decoded. The file is memory-mapped and checked as
 * safetensors.Parse checks it (IXH_EFORMAT and its message otherwise);
 * shapes must match the handle's config. */
int ixh_model_load_safetensors(ixh_model *m, const char *path);

/* safetensors.File.Tensor (safetensors.go:160-173): tensor `name` of the
 * file decoded to float32 (BF16 and F16 widened, I8 as integers) into out
 * (room for cap floats); *count receives its element count (out may be
 * NULL to ask only for it). Host only: no GPU is touched. */
int ixh_safetensors_tensor(const char *path, const char *name, float *out,
                           int64_t cap, int64_t *count);

/* ---- tokenizer (host only: no GPU is touched) --------------------------- */

/* The Gemma-family BPE tokenizer of tokenizer/tokenizer.go (exact parity
 * with Hugging Face tokenizers for the configurations it accepts). Load
 * (tokenizer.go:80-94, the tokenizer.json path; configurations the
 * reference rejects are rejected with its messages, IXH_EFORMAT). The
 * handle is immutable: any number of threads may encode with it. */
typedef struct ixh_tokenizer ixh_tokenizer;
int ixh_tokenizer_load(const char *path, ixh_tokenizer **out);
void ixh_tokenizer_destroy(ixh_tokenizer *t);
/* VocabSize, BosID, EosID, PadID (tokenizer.go:443-461); any may be NULL. */
int ixh_tokenizer_info(const ixh_tokenizer *t, int32_t *vocab_size,
                       int32_t *bos, int32_t *eos, int32_t *pad);
/* Encode (max_len < 0) or EncodeMax (tokenizer.go:479-495) of text[len]
 * (UTF-8, invalid bytes as Go reads them): *n ids, written to ids when it
 * is not NULL (room for cap). */
int ixh_tokenizer_encode(const ixh_tokenizer *t, const char *text,
                         int64_t len, int max_len, int32_t *ids, int64_t cap,
                         int64_t *n);
/* EncodePair (tokenizer.go:497-518): the pair template, max_len > 0
 * truncating the context before the text (0: no limit, as there). */
int ixh_tokenizer_encode_pair(const ixh_tokenizer *t, const char *context,
                              int64_t clen, const char *text, int64_t tlen,
                              int max_len, int32_t *ids, int64_t cap,
                              int64_t *n);
/* EncodeOffsets (tokenizer.go:525-540): ids and the byte span
 * [starts[i], ends[i]) of each in text (template specials: [0, 0)). */
int ixh_tokenizer_encode_offsets(const ixh_tokenizer *t, const char *text,
                                 int64_t len, int32_t *ids, int64_t *starts,
                                 int64_t *ends, int64_t cap, int64_t *n);
/* No reference counterpart (the reference tokenizes one text per call,
 * model.go:202-210): EncodeMax of n texts on `threads` threads (0: one per
 * core; max_len < 0: Encode), laid end to end in ids (room for cap) with
 * offs[n+1] cumulative —
 * the ids/offs of ixh_encode_seqs. With ids NULL, or cap below the total,
 * only offs is filled (the latter returns IXH_EINVAL). */
int ixh_tokenizer_encode_batch(const ixh_tokenizer *t,
                               const char *const *texts, const int64_t *lens,
                               int n, int max_len, int threads, int32_t *ids,
                               int64_t cap, int32_t *offs);

/* Model.Embed (open.go:118-155): each text through EncodeMax(text,
 * max_len), the encoder's pooled row, scaled to norm 1 by
 * float32(1 / sqrt(max(sum of float64 squares, 1e-24))): out [n][H]. The
 * tokenizer runs on `threads` host threads (0: one per core). The
 * reference's embedding cache (WithEmbedCache) stays with the caller. */
int ixh_embed_texts(ixh_model *m, const ixh_tokenizer *t,
                    const char *const *texts, const int64_t *lens, int n,
                    int max_len, int threads, float *out);
/* The normalisation of Model.embed (open.go:134-146) on n rows of H
 * floats, in place (host only). */
int ixh_embed_normalize(float *rows, int n, int H);

/* Optional: RoPE tables as Go's ropeFor computes them (model.go:256-277),
 * cos/sin [rows][head_dim/2], for the global (is_global=1) or local theta.
 * They are used as given and never replaced: a batch whose longest
 * sequence exceeds `rows` fails (IXH_EINVAL) until the caller uploads
 * ropeFor(theta, n) for it. Without them (or after a call with NULL, NULL,
 * 0) the library computes the same formula with the C library's
 * pow/cos/sin, growing the tables to max(n, 512) rows as ropeFor does. */
int ixh_model_set_rope(ixh_model *m, int is_global, const float *cos_t,
                       const float *sin_t, int rows);

/* Kernel and pass choices of a model handle (no counterpart in the
 * reference, whose only knob is the worker count, linalg.SetWorkers).
 * Results never depend on them (the tests check every choice against the
 * oracle); they only move time. Each call reads the handle's values once. */
enum {
  IXH_OPT_PARTS = 0,       /* streams a large batch is split over: 0 auto (default), 1..4 */
  IXH_OPT_PASS_TOKENS = 1, /* most tokens of one pass, 1..131072 (default): larger
                              batches run as several passes of whole sequences */
  IXH_OPT_QKV_FUSED = 2,   /* 1 (default): QKV GEMM fused with Attn8.Prepare for
                              sequences <= 512 keys; 0: two kernels */
  IXH_OPT_QKV_HEADS = 3,   /* heads a workgroup of the fused QKV kernel: 1 (default) or 2 */
  IXH_OPT_GEMM = 4,        /* 0 (default): A-stationary GEMM for Wi and plain stores;
                              1: the tiled GEMM only; 2: as 0, residual GEMMs warp-specialised */
  IXH_OPT_GEMM_TILE = 5,   /* tiled GEMM: 0 (default) 128x128 2 stages, 1 256x128 3, 2 128x128 3 */
  IXH_OPT_LN_SEG = 6,      /* LayerNorm at lanes 8/16: 1 (default) segment kernel, 0 whole-row */
  IXH_OPT_FUSE_RES = 7,    /* 1 (default): Wo and WoMLP fused with the quantisation of their
                              input and the next LayerNorm + quantisation; 2: Wo's input
                              streamed in its K loop (attention writes row maxima); 3: also
                              WoMLP's (the GeGLU epilogue writes them); 4: Wo on the
                              whole-row kernel of 8 waves; 0: separate kernels */
  IXH_OPT_FUSE_MLP = 8,    /* Wi, GeGLU, the quantisation of g, WoMLP and the next LayerNorm +
                              quantisation as one kernel: 2 (default) 64 rows a workgroup,
                              transposed products (hidden 768, 384 or 256); 1: 32 rows a
                              workgroup (hidden 768 or 256, needs FUSE_RES != 0); 0: Wi and
                              WoMLP as chosen by FUSE_RES */
  IXH_OPT_QKV_KBLOCK = 9,  /* 1 (default): the fused QKV kernel reads its input rows K-blocked
                              (written so by the MLP kernel and the embedding LayerNorm) and
                              keeps the head's weight rows in LDS (needs FUSE_MLP); 0:
                              row-major rows through an LDS ring */
};
int ixh_model_set_option(ixh_model *m, int option, int64_t value);
int ixh_model_get_option(ixh_model *m, int option, int64_t *value);

/* Drops the uploaded weights (Invalidate/SetInt8, infer.go:95-135): the
 * next encode fails with IXH_ESTATE until they are set again. */
int ixh_model_invalidate(ixh_model *m);

/* EncodeSeqs (infer.go:261-289): ids of B sequences laid end to end,
 * offs[B+1] cumulative (offs[0] = 0), out [B][H] pooled (mean or CLS).
 * A batch over the pass size (IXH_OPT_PASS_TOKENS) runs as several passes
 * of whole sequences; a single sequence over 131072 tokens is refused. */
int ixh_encode_seqs(ixh_model *m, const int32_t *ids, const int32_t *offs,
                    int B, float *out);
/* EncodeTokens (infer.go:293-299): out [offs[B]][H] final states. */
int ixh_encode_tokens(ixh_model *m, const int32_t *ids, const int32_t *offs,
                      int B, float *out);
/* Either of the above (out_kind IXH_OUT_POOLED or IXH_OUT_TOKENS) with ids
 * and out already in device memory of the model's GPU (offs stays on the
 * host), on `stream` (a hipStream_t, or NULL for the workspace's own
 * stream). Ids are checked on the device. Returns when the work is done. */
int ixh_encode_device(ixh_model *m, const int32_t *d_ids, const int32_t *offs,
                      int B, int out_kind, float *d_out, void *stream);

/* WithBatching (model.go:136-160) and its batcher (batch.go:1-82): requests
 * from concurrent callers are grouped into one encode pass. `workers`
 * threads each take the first pending request and, without waiting, those
 * already queued while the batch stays under `max_rows` tokens; the
 * sequences go end to end and each request gets its pooled rows. An error
 * of the pass (an id out of vocabulary) is returned to every request of
 * that batch. workers <= 0: 2; max_rows <= 0: 65536 (the reference's CPU
 * default, 512, is far below what fills the GPU). */
typedef struct ixh_batcher ixh_batcher;
int ixh_batcher_create(ixh_model *m, int workers, int max_rows, ixh_batcher **out);
/* batcher.encode (batch.go:32-49): EncodeSeqs's arguments; blocks until
 * the request's pooled rows [B][H] are in out. Thread-safe. */
int ixh_batcher_encode(ixh_batcher *b, const int32_t *ids, const int32_t *offs,
                       int B, float *out);
/* Passes run and requests served so far (no counterpart in the reference;
 * for tests and serving metrics). */
int ixh_batcher_stats(ixh_batcher *b, int64_t *batches, int64_t *requests);
/* Waits for queued requests, stops the workers, frees the batcher. The
 * model must outlive it. */
void ixh_batcher_destroy(ixh_batcher *b);

/* Per-kernel timing (no counterpart in the reference, whose profiling is Go
 * pprof around the whole call, tools/infbench/main.go:71-88): when on,
 * every kernel of an encode is bracketed by HIP events on its stream and
 * its duration, algorithmic int8 ops (GEMM and attention MFMA work, 2 per
 * multiply-add) and algorithmic HBM bytes are summed per kernel class.
 * Turning it on or off clears the sums. */
typedef struct ixh_kernel_stat {
  char name[48];    /* kernel class, e.g. "gemm_wi" */
  int64_t launches;
  double ms;        /* summed event-measured durations */
  double ops;       /* summed algorithmic int8 ops */
  double bytes;     /* summed algorithmic HBM bytes */
} ixh_kernel_stat;
int ixh_model_set_profiling(ixh_model *m, int on);
/* Restricts the timing to launches of one kernel class (NULL or "": every
 * launch), so that a timed run carries two events per launch of that class
 * only. Clears the sums. */
int ixh_model_set_profile_filter(ixh_model *m, const char *kernel_class);
/* Copies up to cap class records into out; *n receives the number of
 * classes. */
int ixh_model_profile(ixh_model *m, ixh_kernel_stat *out, int cap, int *n);

/* The model's decision heads, resident on its GPU (newHead/head.logits,
 * heads.go:29-74): head h has rows[h] weight rows w[h] [rows[h]][H] and
 * biases b[h] [rows[h]]; per_token[h] != 0 marks a Spans head, whose
 * logits are taken of every token's state (spans.go:449-459), 0 a head of
 * the pooled row. n = 0 removes them. Thread-safe; a pass in flight keeps
 * the heads it started with. */
int ixh_model_set_heads(ixh_model *m, int n, const int *rows,
                        const int *per_token, const float *const *w,
                        const float *const *b);
/* infer's GPU half (spans.go:369-470, model.go:316-330) for a group of
 * sequences (EncodeSeqs's ids/offs): the encoder pass, then on the device
 *   pooled_z [B][Rp]: for each sequence the logits of the pooled-row heads
 *     in order (Rp = the sum of their rows), z = sum_i f64(w) f64(x) + b,
 *     on the pooled row of EncodeSeqs (the config's pooling) or, with
 *     mean != 0, on the mean of its states (meanRows, spans.go:466-476, as
 *     infer pools for a model with Spans questions);
 *   token_z [N][Rt]: each token's logits of the per-token heads.
 * Either output may be NULL (not computed). Batches over the pass size run
 * as several passes; only the logits leave the GPU. */
int ixh_encode_heads(ixh_model *m, const int32_t *ids, const int32_t *offs,
                     int B, int mean, double *pooled_z, double *token_z);

/* head.logits (heads.go:63-74) on host rows: z[t][r] = sum_i
 * f64(w[r][i]) f64(x[t][i]) + f64(b[r]), computed on the model's GPU. */
int ixh_head_logits(ixh_model *m, const float *x, int T, const float *w,
                    const float *b, int rows, double *z);

/* ---- linalg ------------------------------------------------------------- */

/* A PackedB8 on device (linalg/int8.go:27-77): k x n, from q and scale as
 * for ixh_model_set_matrix. */
int ixh_packb8_create(int device, const int8_t *q, const float *scale, int k,
                      int n, int layout, ixh_packed_b8 **out);
void ixh_packb8_destroy(ixh_packed_b8 *b);
/* IXH_OPT_GEMM / IXH_OPT_GEMM_TILE for the linalg calls on this handle. */
int ixh_packb8_set_option(ixh_packed_b8 *b, int option, int64_t value);

/* MatMul8N (linalg/int8.go:89-155): c[m][n] (+)= a[m][k] . B, a quantised
 * per row as quantizeA does. Host buffers. */
int ixh_matmul8(ixh_packed_b8 *b, float *c, const float *a, int m,
                int accumulate);

/* MatMul8N on device buffers that allocates nothing. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, serving loops or harnesses that forbid hipMalloc). d_a [m][lda]
 * and d_c [m][ldc] float32 in the memory of b's GPU, 16-byte aligned;
 * k % 4 == 0, lda >= k and a multiple of 4, ldc >= n. The quantised
 * activations and their scales go to a fixed scratch array of 32 MiB per
 * GPU (module memory, held until the process ends): m * (round_up(k, 64) +
 * 4) bytes (plus alignment) must fit, else IXH_EINVAL with the limit. The
 * work is queued on `stream` (a hipStream_t; NULL: the null stream) and
 * the call returns without waiting. Every call on a GPU shares that GPU's
 * scratch, so calls on one GPU run one after another on the device: each
 * call's work waits, on its stream, for the previous call's (an event per
 * GPU, made when the first PackedB8 of that GPU is created, recorded after
 * every call), whichever streams or threads issue them. A call on a stream
 * under graph capture neither waits nor records: the graph orders it, so
 * two captured calls must not sit on parallel branches. */
int ixh_matmul8_noalloc(ixh_packed_b8 *b, float *d_c, int ldc, const float *d_a,
                        int lda, int m, int accumulate, void *stream);

/* MatMul8Outliers (linalg/int8.go:272-349), the LLM.int8() decomposition:
 * the input channels whose column max |a| exceeds ratio times the mean of
 * the column maxima (the 32 largest when more) are zeroed in a copy of a,
 * MatMul8N runs on the copy, and each such channel then adds
 * a[i][j] * (q[col][j] * scale[col]) to c[i][col] in float32. ratio > 0.
 * Host buffers. */
int ixh_matmul8_outliers(ixh_packed_b8 *b, float *c, const float *a, int m,
                         int accumulate, float ratio);

/* siglip linear.apply (internal/siglip/encoder.go:36-49): dst[rows][n] =
 * x . B through MatMul8Outliers (outliers != 0, ratio > 0) or MatMul8N,
 * then AddTo(dst row, bias) when bias is not NULL. Host buffers. */
int ixh_linear8(ixh_packed_b8 *b, float *dst, const float *x, int rows,
                const float *bias, int outliers, float ratio);

/* The integers MatMul8N works with, for bit-exact checks: the quantised
 * activations (signed, i.e. the reference's uint8 minus 128) aq[m][k],
 * their scales sa[m], and the reference tile (microKernel8Go,
 * int8.go:214-227) tile[m][n] = sum (aq+128)*q. */
int ixh_matmul8_tile(ixh_packed_b8 *b, const float *a, int m, int8_t *aq,
                     float *sa, int32_t *tile);

/* LayerNormRow (linalg/vec_simd.go:285-327) of m rows of h values, then,
 * if q is not NULL, quantizeA of the result (q[m][h] signed, sa[m]) — the
 * fused LN + quantisation of the encoder. out may be NULL. */
int ixh_layernorm_quant(int device, const float *x, int m, int h,
                        const float *gamma, double eps, int lanes, float *out,
                        int8_t *q, float *sa);

/* LN + quantizeA + MatMul8N + GeluMul (infer.go:404-418): the fused Wi
 * step. g[m][n/2] = gelu(z[:, :n/2]) * z[:, n/2:] with z = LN(x) . B
 * (B is k x n, n/2 a multiple of 32); also the int32 tile if not NULL. */
int ixh_ln_matmul8_geglu(ixh_packed_b8 *b, const float *x, int m,
                         const float *gamma, double eps, int lanes, float *g,
                         int32_t *tile);

/* Attend8 (linalg/attention8.go:70-73): o[n][64] = attention of q over k, v
 * (n x 64 each), window < 0 global, scores scaled by scale. */
int ixh_attend8(int device, float *o, const float *q, const float *k,
                const float *v, int n, int d, int window, float scale,
                int lanes);

/* Self-check of the attention kernels' softmax rounding (no counterpart in
 * the reference; for tests and deployment checks). The kernels round
 * 255*exp(s - max) with the device's base-2 exponential and fall back to
 * the reference's exp32 formulas where the value is within a tolerance of
 * a rounding boundary. For every float v in [-inf, -0] and +0 this counts
 * the v where that shortcut would round differently from the reference:
 * bad[0] for the vector formula (ExpShift's SIMD body), bad[1] for the
 * scalar exp32; both must be 0. max_err[0..1]: the largest distance of the
 * shortcut from 255*exp(v) of each formula; *undecided: how many v take the
 * fallback. */
int ixh_check_exp255(int device, int64_t bad[2], float max_err[2], int64_t *undecided);

/* Check of the device GELU (no counterpart in the reference, which computes
 * GeluMul with IEEE division, linalg/gelu_amd64.s:173-195 and
 * fastmath.go:9-26): the kernels divide by Markstein's FMA sequence and
 * clamp with v_med3. For every one of the 2^32 float inputs this counts the
 * x whose GELU differs in any bit from the IEEE-division form: bad[0] for
 * the FMA form, bad[1] for the scalar form; both must be 0. */
int ixh_check_gelu(int device, int64_t bad[2]);

/* Rate check of the int8 matrix cores (no counterpart in the reference; the
 * scale of the roofline figures): every wave of four a SIMD issues
 * 4 * iters v_mfma_i32_32x32x32_i8 back to back from registers (iters in
 * 1 .. 2^22). *ops_per_s: int8 operations (two a multiply-add) a second
 * over the timed launch, to set against the 5.0e15 dense peak. */
int ixh_check_mfma_rate(int device, int iters, double *ops_per_s);

#ifdef __cplusplus
}
#endif
#endif
