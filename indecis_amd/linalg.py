"""Host-side mirror of indecis's linalg int8 entry points on the GPU
(linalg/int8.go, linalg/vec_simd.go, linalg/attention8.go), through the C
ABI. Arguments keep the reference's meaning: B operands are PackedB8
(per-output-channel int8 weights), activations float32 rows.
"""
import ctypes as C

import numpy as np

from . import _lib
from .modernbert import pack_b8  # noqa: F401  (PackB8 lives with the weights)


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


class PackedB8:
    """PackedB8 (int8.go:27-34) resident on a GPU: k x n, built from the
    quantised weights q [n][k] and their scales (what PackB8 computes)."""

    def __init__(self, q, scale, device=0, layout=_lib.LAYOUT_ROWS, k=None, n=None):
        q = np.ascontiguousarray(q, np.int8)
        scale = np.ascontiguousarray(scale, np.float32)
        if layout == _lib.LAYOUT_ROWS:
            n, k = q.shape
        self.k, self.n = k, n
        self.device = device
        h = C.c_void_p()
        _lib.check(_lib.lib().ixh_packb8_create(device, _ptr(q), _ptr(scale), k, n, layout, C.byref(h)))
        self._h = h

    def set_option(self, name, value):
        """The GEMM kernel choice for calls on this handle
        (ixh_packb8_set_option): "gemm" or "gemm_tile"."""
        _lib.check(_lib.lib().ixh_packb8_set_option(self._h, _lib.OPTIONS[name], int(value)))

    def close(self):
        if self._h:
            _lib.lib().ixh_packb8_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matmul8(c, a, b, m, accumulate=False):
    """MatMul8N (int8.go:89-155): c[m][n] (+)= a[m][k] . B, in place."""
    if c.dtype != np.float32 or not c.flags.c_contiguous:
        raise ValueError("linalg: MatMul8: c must be contiguous float32")
    if a.size < m * b.k or c.size < m * b.n:
        raise ValueError("linalg: MatMul8: slice too short")
    a = np.ascontiguousarray(a, np.float32)
    _lib.check(_lib.lib().ixh_matmul8(b._h, _ptr(c), _ptr(a), m, 1 if accumulate else 0))
    return c


def matmul8_outliers(c, a, b, m, accumulate=False, ratio=6.0):
    """MatMul8Outliers (int8.go:272-349): c[m][n] (+)= a[m][k] . B with the
    LLM.int8() split of massive input channels, in place."""
    if c.dtype != np.float32 or not c.flags.c_contiguous:
        raise ValueError("linalg: MatMul8Outliers: c must be contiguous float32")
    if a.size < m * b.k or c.size < m * b.n:
        raise ValueError("linalg: MatMul8Outliers: slice too short")
    a = np.ascontiguousarray(a, np.float32)
    _lib.check(_lib.lib().ixh_matmul8_outliers(b._h, _ptr(c), _ptr(a), m, 1 if accumulate else 0,
                                               float(ratio)))
    return c


def linear8(x, b, bias=None, outliers=False, ratio=6.0):
    """siglip linear.apply (encoder.go:36-49): x[rows][k] . B (+ bias)."""
    x = np.ascontiguousarray(x, np.float32)
    rows = x.shape[0]
    if x.shape[1] != b.k:
        raise ValueError("siglip: linear: slice too short")
    dst = np.zeros((rows, b.n), np.float32)
    bias_c = None if bias is None else np.ascontiguousarray(bias, np.float32)
    if bias_c is not None and bias_c.size < b.n:
        raise ValueError("siglip: linear: bias too short")
    _lib.check(_lib.lib().ixh_linear8(b._h, _ptr(dst), _ptr(x), rows,
                                      None if bias_c is None else _ptr(bias_c),
                                      1 if outliers else 0, float(ratio)))
    return dst


def matmul8_tile(a, b):
    """The integers of MatMul8N: (aq signed [m][k], sa [m], tile [m][n])
    with tile = sum (aq+128)*q as microKernel8Go computes it."""
    a = np.ascontiguousarray(a, np.float32)
    m = a.shape[0]
    aq = np.zeros((m, b.k), np.int8)
    sa = np.zeros(m, np.float32)
    tile = np.zeros((m, b.n), np.int32)
    _lib.check(_lib.lib().ixh_matmul8_tile(b._h, _ptr(a), m, _ptr(aq), _ptr(sa), _ptr(tile)))
    return aq, sa, tile


def layernorm_quant(x, gamma, eps=1e-5, lanes=8, device=0, want_out=True, want_q=True):
    """LayerNormRow (vec_simd.go:285-327) of each row, then quantizeA of
    the result: (out [m][h] | None, q [m][h] | None, sa [m] | None)."""
    x = np.ascontiguousarray(x, np.float32)
    m, h = x.shape
    g = np.ascontiguousarray(gamma, np.float32)
    out = np.zeros((m, h), np.float32) if want_out else None
    q = np.zeros((m, h), np.int8) if want_q else None
    sa = np.zeros(m, np.float32) if want_q else None
    _lib.check(_lib.lib().ixh_layernorm_quant(
        device, _ptr(x), m, h, _ptr(g), eps, lanes,
        _ptr(out) if want_out else None, _ptr(q) if want_q else None, _ptr(sa) if want_q else None))
    return out, q, sa


def ln_matmul8_geglu(x, gamma, b, eps=1e-5, lanes=8, want_tile=True):
    """LayerNormRow, quantizeA, MatMul8N, GeluMul (infer.go:404-418) in
    one call: (g [m][n/2], tile [m][n] | None)."""
    x = np.ascontiguousarray(x, np.float32)
    m = x.shape[0]
    g = np.zeros((m, b.n // 2), np.float32)
    tile = np.zeros((m, b.n), np.int32) if want_tile else None
    gam = np.ascontiguousarray(gamma, np.float32)
    _lib.check(_lib.lib().ixh_ln_matmul8_geglu(b._h, _ptr(x), m, _ptr(gam), eps, lanes, _ptr(g),
                                               _ptr(tile) if want_tile else None))
    return g, tile


def attend8(q, k, v, window=-1, scale=0.125, lanes=8, device=0):
    """Attend8 (attention8.go:70-73) on [n][64] float32 operands."""
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    n, d = q.shape
    o = np.zeros((max(n, 1), d), np.float32)
    _lib.check(_lib.lib().ixh_attend8(device, _ptr(o), _ptr(q), _ptr(k), _ptr(v), n, d, window,
                                      float(scale), lanes))
    return o[:n]


def check_exp255(device=0):
    """Runs the device self-check of the attention softmax rounding over
    every float v <= 0: returns (bad_simd, bad_scalar, max_err_simd,
    max_err_scalar, undecided). bad_* must be 0."""
    bad = (C.c_int64 * 2)()
    err = (C.c_float * 2)()
    und = C.c_int64()
    _lib.check(_lib.lib().ixh_check_exp255(device, bad, err, C.byref(und)))
    return int(bad[0]), int(bad[1]), float(err[0]), float(err[1]), int(und.value)


def check_mfma_rate(device=0, iters=20000):
    """int8 operations a second that the device's matrix cores sustain when
    every wave issues v_mfma_i32_32x32x32_i8 back to back from registers."""
    r = C.c_double()
    _lib.check(_lib.lib().ixh_check_mfma_rate(device, iters, C.byref(r)))
    return float(r.value)


def check_gelu(device=0):
    """Runs the device self-check of the GELU's division and clamp over
    every float input: returns (bad_fma_form, bad_scalar_form); both must
    be 0."""
    bad = (C.c_int64 * 2)()
    _lib.check(_lib.lib().ixh_check_gelu(device, bad))
    return int(bad[0]), int(bad[1])
