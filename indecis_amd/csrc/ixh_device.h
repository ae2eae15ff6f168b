// ixh_device.h — device-side numerics shared by the gfx950 kernels.
//
// Every float operation here is rounded where the reference rounds it
// (the sources are compiled with -ffp-contract=off): __builtin_fmaf where
// the reference fuses (Go SIMD MulAdd, VFMADD213PS), separate operations
// where it does not. IEEE division (HIP's default correctly rounded f32
// divide; the GELU's own division, gelu_div, gives the same GELU results
// on every input) and RNE conversions throughout.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace ixh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// 32x32x32 int8 MFMA (gfx950): D[i][j] = sum_k A[i][k] B[k][j] + C.
// Lane l supplies row i = l%32 of A and column j = l%32 of B, 16 bytes
// each, over the same 16 values of k (lanes 0-31 one half of k, 32-63 the
// other). D: lane l holds column j = l%32, rows 8*(r/4) + 4*(l/32) + r%4
// for r = 0..15.
__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int acc_row(int r, int lane) {
  return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

__device__ __forceinline__ float fmax32(float a, float b) { return b > a ? b : a; }

// max(m, |v|) for a running maximum of absolute values started at 0 (so m
// is never NaN): v_max_f32 (IEEE maxNum) returns the operand that is not
// NaN, which is fmax32(m, |v|) — Go's `if v > m { m = v }` — in one
// instruction (two of them fuse into v_max3_f32) instead of a compare and
// a select. For inputs without NaN every order of the maxima gives the
// same value; NaN inputs are not reproduced lane by lane from the
// reference's VMAXPS registers (neither are they by the compare form).
__device__ __forceinline__ float amax(float m, float v) { return __builtin_fmaxf(m, __builtin_fabsf(v)); }
__device__ __forceinline__ float fmin32(float a, float b) { return b < a ? b : a; }

// roundHalfEven (linalg/int8.go:207-210) == VCVTPS2DQ for |v| < 2^22.
__device__ __forceinline__ float rne(float v) { return __builtin_rintf(v); }

// RNE(x * inv) as int8 (QuantizeRow / quantRowAVX2 / quantColsAVX2).
__device__ __forceinline__ int q8(float x, float inv) { return (int)rne(x * inv); }

// exp32 (linalg/fastmath.go:36-52): separate roundings.
__device__ __forceinline__ float exp32_scalar(float x) {
  if (x < -87.3f) return 0.0f;
  x = fmin32(x, 88.7f);
  float n = rne(x * 1.44269504088896341f);
  float r = x - n * 0.693359375f - n * -2.12194440e-4f;
  float p = 1.9875691500e-4f;
  p = p * r + 1.3981999507e-3f;
  p = p * r + 8.3334519073e-3f;
  p = p * r + 4.1665795894e-2f;
  p = p * r + 1.6666665459e-1f;
  p = p * r + 5.0000001201e-1f;
  float y = p * r * r + r + 1.0f;
  return y * __int_as_float(((int)n + 127) << 23);
}

// One lane of ExpShift's vector body (linalg/vec_simd.go:235-248).
__device__ __forceinline__ float exp32_simd(float v) {
  bool under = v < -87.3f;
  v = fmin32(fmax32(v, -87.3f), 88.7f);
  const float magic = 12582912.0f;
  float n = __builtin_fmaf(v, 1.44269504088896341f, magic) - magic;
  float r = __builtin_fmaf(n, -0.693359375f, v);
  r = __builtin_fmaf(n, 2.12194440e-4f, r);
  float p = __builtin_fmaf(r, 1.9875691500e-4f, 1.3981999507e-3f);
  p = __builtin_fmaf(r, p, 8.3334519073e-3f);
  p = __builtin_fmaf(r, p, 4.1665795894e-2f);
  p = __builtin_fmaf(r, p, 1.6666665459e-1f);
  p = __builtin_fmaf(r, p, 5.0000001201e-1f);
  float y = __builtin_fmaf(p * r, r, r) + 1.0f;
  float pw = __int_as_float(((int)n + 127) << 23);
  return under ? 0.0f : y * pw;
}

// Cache policy of the buffer loads and stores of data a kernel streams
// (read or written once: activations, the residual rows): nt, the
// non-temporal hint, so that they do not displace the weights that every
// workgroup rereads from L2. The weights keep the default policy. Only for
// accesses whose wave instruction covers whole 128-byte lines: on stores
// of 16 bytes a row (the QKV kernel's K and Q rows, attention's context)
// the hint made those kernels 6% and 12% slower; on the final LayerNorm's
// output, which pooling reads next, 76 -> 87 us.
constexpr int kStreamPolicy = 2;
typedef float f4v __attribute__((ext_vector_type(4)));
// a float4 of streamed data through a plain pointer (global_load ... nt)
__device__ __forceinline__ float4 load_stream_f4(const float *p) {
  const f4v t = __builtin_nontemporal_load((const f4v *)p);
  return make_float4(t.x, t.y, t.z, t.w);
}
// 16 bytes of streamed output through a plain pointer (global_store ... nt)
__device__ __forceinline__ void store_stream_16(void *p, v4i v) { __builtin_nontemporal_store(v, (v4i *)p); }

// Buffer resource over `bytes` bytes from p (gfx9 descriptor word 3), for
// loads that share one VGPR offset and step by a wave-uniform SGPR offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}
template <int POLICY = 0>
__device__ __forceinline__ float4 buf_load_f4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const v4i t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, POLICY);
  return make_float4(__int_as_float(t[0]), __int_as_float(t[1]), __int_as_float(t[2]),
                     __int_as_float(t[3]));
}

// 255*exp(v) from the hardware base-2 exponential (v_exp_f32): fma(v,
// log2 e, log2 255), then 2^x. Used only to round: where it lies more than
// kExp255Tol from a half-integer, RNE of it equals RNE(f32(255*exp32(v)))
// for both reference formulas (exp32_simd and exp32_scalar), for every
// float v <= 0 — ixh_check_exp255 verifies this on the device, float by
// float. Elsewhere the caller evaluates the reference formula. The largest
// |exp255_fast - 255*exp32| over those floats is 7.63e-5 (5 ulp at 255);
// the tolerance is 1.6 times that.
constexpr float kExp255Tol = 1.0f / 8192;
__device__ __forceinline__ float exp255_fast(float v) {
  return __builtin_amdgcn_exp2f(__builtin_fmaf(v, 1.44269504088896341f, 7.99435343685885793f));
}

// p / q for the GELU's rational erf: the hardware reciprocal (v_rcp_f32)
// times p, corrected once by the exact remainder fma(-q, y, p) (Markstein's
// FMA-based division, one step). Here q, the denominator polynomial on t*t
// in [0, 16], lies in [-2.4, -0.0142] and |p| <= |q|, so no operand needs
// the range scaling of the general IEEE sequence. The quotient may differ
// from the correctly rounded p / q in its last bit; the GELU result
// 0.5x(1 + p/q) does not: ixh_check_gelu verifies, for every float input of
// both GELU forms, that it equals the GELU with IEEE division (a refined
// reciprocal and a second correction change none of those results; with no
// correction about 15 million inputs differ).
__device__ __forceinline__ float gelu_div(float p, float q) {
  const float r = __builtin_amdgcn_rcpf(q);
  const float y = p * r;
  return __builtin_fmaf(__builtin_fmaf(-q, y, p), r, y);
}

// clamp of the GELU argument to [-4, 4] (VMAXPS/VMINPS in the reference):
// v_med3 gives the same value for every non-NaN t, and a NaN t comes only
// from a NaN x, whose GELU is NaN through 0.5*x either way.
__device__ __forceinline__ float gelu_clamp(float t) { return __builtin_amdgcn_fmed3f(t, -4.0f, 4.0f); }

// GELU (erf) of geluMulAVX2 (linalg/gelu_amd64.s:173-195). FAST: gelu_div
// and gelu_clamp; false: IEEE division and the compare-select clamp (the
// form ixh_check_gelu compares against).
template <bool FAST = true>
__device__ __forceinline__ float gelu_fma(float x) {
  float t = x * 0.7071067811865476f;
  t = FAST ? gelu_clamp(t) : fmin32(fmax32(t, -4.0f), 4.0f);
  float t2 = t * t;
  float p = __builtin_fmaf(t2, -2.72614225801306e-10f, 2.77068142495902e-08f);
  p = __builtin_fmaf(t2, p, -2.10102402082508e-06f);
  p = __builtin_fmaf(t2, p, -5.69250639462346e-05f);
  p = __builtin_fmaf(t2, p, -7.34990630326855e-04f);
  p = __builtin_fmaf(t2, p, -2.95459980854025e-03f);
  p = __builtin_fmaf(t2, p, -1.60960333262415e-02f);
  p = p * t;
  float q = __builtin_fmaf(t2, -1.45660718464996e-05f, -2.13374055278905e-04f);
  q = __builtin_fmaf(t2, q, -1.68282697438203e-03f);
  q = __builtin_fmaf(t2, q, -7.37332916720468e-03f);
  q = __builtin_fmaf(t2, q, -1.42647390514189e-02f);
  return (0.5f * x) * (1.0f + (FAST ? gelu_div(p, q) : p / q));
}

// geluScalar (linalg/fastmath.go:9-26): separate roundings.
template <bool FAST = true>
__device__ __forceinline__ float gelu_scalar(float x) {
  float e = x * 0.7071067811865476f;
  e = FAST ? gelu_clamp(e) : fmin32(fmax32(e, -4.0f), 4.0f);
  float x2 = e * e;
  float p = x2 * -2.72614225801306e-10f + 2.77068142495902e-08f;
  p = x2 * p + -2.10102402082508e-06f;
  p = x2 * p + -5.69250639462346e-05f;
  p = x2 * p + -7.34990630326855e-04f;
  p = x2 * p + -2.95459980854025e-03f;
  p = x2 * p + -1.60960333262415e-02f;
  p = p * e;
  float q = x2 * -1.45660718464996e-05f + -2.13374055278905e-04f;
  q = x2 * q + -1.68282697438203e-03f;
  q = x2 * q + -7.37332916720468e-03f;
  q = x2 * q + -1.42647390514189e-02f;
  return 0.5f * x * (1.0f + (FAST ? gelu_div(p, q) : p / q));
}

// Direct-to-LDS loads (global_load_lds_dwordx4): pointer types, and the
// XOR swizzle of the four 16-byte chunks of a 64-byte LDS row, by
// (row >> 1) & 3, so 16-byte fragment reads of consecutive rows fall in
// distinct banks.
typedef __attribute__((address_space(3))) void *lds_ptr;
typedef const __attribute__((address_space(1))) void *glb_ptr;
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 3; }

// s_waitcnt with only the vector-memory count (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier for LDS only: this wave's LDS accesses complete
// (lgkmcnt 0), then s_barrier; the wave's global loads stay in flight
// (__syncthreads would wait for them too).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt 63, expcnt 7, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Max of x over each 16-lane row of the wave (DPP row_ror 8, 4, 2, 1):
// every lane gets its row's max. x must not be NaN.
__device__ __forceinline__ float row16_max(float x) {
  int v = __float_as_int(x);
  v = __float_as_int(__builtin_fmaxf(__int_as_float(v),
                                     __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false))));
  v = __float_as_int(__builtin_fmaxf(__int_as_float(v),
                                     __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false))));
  v = __float_as_int(__builtin_fmaxf(__int_as_float(v),
                                     __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x122, 0xF, 0xF, false))));
  v = __float_as_int(__builtin_fmaxf(__int_as_float(v),
                                     __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x121, 0xF, 0xF, false))));
  return __int_as_float(v);
}

// Max of x over the 32 lanes of each half-wave (lanes 0-31, 32-63) with
// DPP: rotations inside each 16-lane row, then row 0 (2) into row 1 (3) by
// row_bcast:15. The result is in lanes 16-31 and 48-63. x must not be NaN.
__device__ __forceinline__ float halfwave_max(float x) {
  int v = __float_as_int(x);
  v = __float_as_int(__builtin_fmaxf(__int_as_float(v),
                                     __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false))));
  v = __float_as_int(__builtin_fmaxf(__int_as_float(v),
                                     __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false))));
  v = __float_as_int(__builtin_fmaxf(__int_as_float(v),
                                     __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x122, 0xF, 0xF, false))));
  v = __float_as_int(__builtin_fmaxf(__int_as_float(v),
                                     __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x121, 0xF, 0xF, false))));
  // rows 1 and 3 take the max with lane 15 of the row before; rows 0 and
  // 2 keep their value (old = v)
  v = __float_as_int(__builtin_fmaxf(__int_as_float(v),
                                     __int_as_float(__builtin_amdgcn_update_dpp(v, v, 0x142, 0xA, 0xF, false))));
  return __int_as_float(v);
}

// Max of x over the whole wave, in every lane (DPP within the half-waves,
// then their two maxima read from lanes 31 and 63). x must not be NaN.
__device__ __forceinline__ float wave_max(float x) {
  const int h = __float_as_int(halfwave_max(x));
  return __builtin_fmaxf(__int_as_float(__builtin_amdgcn_readlane(h, 31)),
                         __int_as_float(__builtin_amdgcn_readlane(h, 63)));
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), in
// order: a loop whose index is a constant in every body (register arrays
// indexed by it stay in registers).
template <typename F, int... I>
__device__ __forceinline__ void sfor_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sfor(F &&f) {
  sfor_impl(f, std::make_integer_sequence<int, N>{});
}

// Dequantisation of one int8 GEMM result (kernel_vnni_amd64.s:144-200):
// f32(tile) - zc, times sb, times sa — tile being the reference's
// unsigned-offset integer sum.
__device__ __forceinline__ float deq(int tile, float zc, float sb, float sa) {
  return (((float)tile - zc) * sb) * sa;
}

}  // namespace ixh
