// outliers.hip — the LLM.int8() decomposition of linalg.MatMul8Outliers
// (linalg/int8.go:272-349) and the bias of siglip's linear.apply
// (internal/siglip/encoder.go:36-49), around the int8 GEMM:
//  * column maxima of |A| (order-free, so an atomic max of the float bits:
//    |x| is never negative);
//  * the chosen input channels zeroed in a copy of A before quantizeA;
//  * after the GEMM, per output element, the chosen channels' products
//    a[i][j] * f32(q[col][j] * sb[col]) added one by one in the chosen
//    order (product and sum rounded separately, as gc computes
//    ci[col] += x * wv for amd64 at GOAMD64 v1/v2, which has no scalar
//    FMA), then the bias (AddTo, vec_scalar.go:97-101).
// The channel choice itself (a float32 mean in channel order, a partial
// selection of the 32 largest) runs on the host over the k maxima.
#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace {

constexpr int kColRows = 256;  // rows per workgroup of the column-max kernel

__global__ __launch_bounds__(256) void colmax_kernel(const float *a, int ld, int m, int k,
                                                     unsigned *out) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= k) return;
  const int r0 = blockIdx.y * kColRows, r1 = min(m, r0 + kColRows);
  float mx = 0.f;
  for (int i = r0; i < r1; i++) mx = fmax32(mx, fabsf(a[(size_t)i * ld + j]));
  atomicMax(out + j, __float_as_uint(mx));
}

__global__ __launch_bounds__(256) void zero_cols_kernel(float *a, int ld, int m, const int *cols,
                                                        int ncols) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long)m * ncols) return;
  const int i = (int)(e / ncols), t = (int)(e % ncols);
  a[(size_t)i * ld + cols[t]] = 0.f;
}

__global__ __launch_bounds__(256) void outlier_epilogue_kernel(float *c, int ldc, int m, int n,
                                                               const float *a, int lda,
                                                               const int *cols, int ncols,
                                                               const float *w, const float *bias) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long)m * n) return;
  const int i = (int)(e / n), col = (int)(e % n);
  float v = c[(size_t)i * ldc + col];
  const float *ar = a + (size_t)i * lda;
  for (int t = 0; t < ncols; t++) {
    const float p = ar[cols[t]] * w[(size_t)t * n + col];
    v = v + p;
  }
  if (bias) v = v + bias[col];
  c[(size_t)i * ldc + col] = v;
}

}  // namespace

void launch_colmax(const float *a, int ld, int m, int k, unsigned *out, hipStream_t s) {
  if (m <= 0 || k <= 0) return;
  const dim3 grid((k + 255) / 256, (m + kColRows - 1) / kColRows);
  colmax_kernel<<<grid, 256, 0, s>>>(a, ld, m, k, out);
}

void launch_zero_cols(float *a, int ld, int m, const int *cols, int ncols, hipStream_t s) {
  const long total = (long)m * ncols;
  if (total <= 0) return;
  zero_cols_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(a, ld, m, cols, ncols);
}

void launch_outlier_epilogue(float *c, int ldc, int m, int n, const float *a, int lda, const int *cols,
                             int ncols, const float *w, const float *bias, hipStream_t s) {
  const long total = (long)m * n;
  if (total <= 0) return;
  outlier_epilogue_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(c, ldc, m, n, a, lda, cols,
                                                                          ncols, w, bias);
}

}  // namespace ixh
