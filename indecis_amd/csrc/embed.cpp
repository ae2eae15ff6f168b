// embed.cpp — Model.Embed (open.go:118-155): texts to embeddings of norm
// 1, the tokenizer and the encoder of this library in one call (host code
// around ixh_encode_seqs).
//
// The reference tokenizes each text with EncodeMax(text, maxLen), encodes
// the id lists in groups of 32 sorted by length (forEachPooled,
// model.go:391-417) and scales each pooled row by
// float32(1 / sqrt(max(sum of float64 squares, 1e-24))). A row does not
// depend on the other sequences of its pass, so the whole list goes
// through one pass here (the encoder orders sequences itself).
#include <algorithm>
#include <cmath>
#include <vector>

#include "../../include/indecis_hip.h"
#include "ixh_internal.h"

extern "C" {

int ixh_embed_normalize(float *rows, int n, int H) {
  if (n < 0 || H <= 0 || (n > 0 && !rows)) return ixh::set_error(IXH_EINVAL, "indecis: bad arguments");
  for (int i = 0; i < n; i++) {
    float *x = rows + (size_t)i * H;
    double s = 0;
    for (int j = 0; j < H; j++) s += (double)x[j] * (double)x[j];
    const float inv = (float)(1 / std::sqrt(std::max(s, 1e-24)));
    for (int j = 0; j < H; j++) x[j] = x[j] * inv;
  }
  return IXH_OK;
}

int ixh_embed_texts(ixh_model *m, const ixh_tokenizer *t, const char *const *texts, const int64_t *lens, int n,
                    int max_len, int threads, float *out) {
  if (!m || !t) return ixh::set_error(IXH_EINVAL, "indecis: nil model or tokenizer");
  if (n > 0 && !out) return ixh::set_error(IXH_EINVAL, "indecis: bad arguments");
  std::vector<std::vector<int32_t>> per;
  int rc = ixh::tokenize_texts(t, texts, lens, n, max_len, threads, per);
  if (rc) return rc;
  if (n == 0) return IXH_OK;
  std::vector<int32_t> offs(n + 1, 0);
  for (int i = 0; i < n; i++) {
    const int64_t next = (int64_t)offs[i] + (int64_t)per[i].size();
    if (next > INT32_MAX) return ixh::set_error(IXH_EINVAL, "indecis: batch over 2^31 tokens");
    offs[i + 1] = (int32_t)next;
  }
  std::vector<int32_t> ids(offs[n]);
  for (int i = 0; i < n; i++)
    if (!per[i].empty()) std::copy(per[i].begin(), per[i].end(), ids.begin() + offs[i]);
  if ((rc = ixh_encode_seqs(m, ids.data(), offs.data(), n, out))) return rc;
  ixh_config c;
  ixh::model_config(m, &c);
  return ixh_embed_normalize(out, n, c.hidden);
}

}  // extern "C"
