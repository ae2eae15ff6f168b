"""ctypes bindings of the CPU oracle (indecis_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker of the HIP path (never as the
thing measured or shipped). Each wrapper restates the reference function
cited in indecis_oracle.h.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(HERE, "liboracle.so")
_lib = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")

EMB_F32, EMB_BF16, EMB_I8 = 0, 1, 2


class IxoModel(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("layers", C.c_int), ("heads", C.c_int),
        ("intermediate", C.c_int), ("vocab", C.c_int),
        ("norm_eps", C.c_double),
        ("global_every", C.c_int), ("local_attention", C.c_int), ("lanes", C.c_int),
        ("wqkv_q", C.c_void_p), ("wqkv_s", C.c_void_p),
        ("wo_q", C.c_void_p), ("wo_s", C.c_void_p),
        ("wi_q", C.c_void_p), ("wi_s", C.c_void_p),
        ("womlp_q", C.c_void_p), ("womlp_s", C.c_void_p),
        ("attn_norm", C.c_void_p), ("mlp_norm", C.c_void_p),
        ("emb_norm", C.c_void_p), ("final_norm", C.c_void_p),
        ("emb_format", C.c_int),
        ("emb_f32", C.c_void_p), ("emb_bf16", C.c_void_p),
        ("emb_exact_ids", C.c_void_p), ("emb_exact_rows", C.c_void_p), ("emb_n_exact", C.c_int),
        ("emb_i8", C.c_void_p), ("emb_i8_scale", C.c_void_p),
        ("rope_cos_global", C.c_void_p), ("rope_sin_global", C.c_void_p),
        ("rope_cos_local", C.c_void_p), ("rope_sin_local", C.c_void_p),
        ("rope_rows", C.c_int),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            from oracle import build as _b
            _b.build()
        L = C.CDLL(_SO)
        L.ixo_round_half_even.argtypes = [C.c_float]
        L.ixo_round_half_even.restype = C.c_float
        L.ixo_exp32.argtypes = [C.c_float]
        L.ixo_exp32.restype = C.c_float
        L.ixo_exp_simd.argtypes = [C.c_float]
        L.ixo_exp_simd.restype = C.c_float
        L.ixo_gelu_fma.argtypes = [C.c_float]
        L.ixo_gelu_fma.restype = C.c_float
        L.ixo_gelu_scalar.argtypes = [C.c_float]
        L.ixo_gelu_scalar.restype = C.c_float
        L.ixo_pack_b8.argtypes = [f32p, C.c_int, C.c_int, C.c_int, i8p, f32p, i32p]
        L.ixo_b8_to_panels.argtypes = [i8p, C.c_int, C.c_int, i8p]
        L.ixo_quantize_rows.argtypes = [f32p, C.c_int, C.c_int, C.c_int, i8p, C.c_int, f32p]
        L.ixo_matmul8_tile.argtypes = [i8p, C.c_int, i8p, C.c_int, C.c_int, C.c_int, i32p]
        L.ixo_matmul8_deq.argtypes = [f32p, C.c_int, i8p, C.c_int, f32p, i8p, f32p, i32p,
                                      C.c_int, C.c_int, C.c_int, C.c_int]
        L.ixo_matmul8.argtypes = [f32p, C.c_int, f32p, C.c_int, i8p, f32p, i32p,
                                  C.c_int, C.c_int, C.c_int, C.c_int]
        L.ixo_matmul8_outliers.argtypes = [f32p, C.c_int, f32p, C.c_int, i8p, f32p, i32p, C.c_int,
                                           C.c_int, C.c_int, C.c_int, C.c_float, i32p]
        L.ixo_matmul8_outliers.restype = C.c_int
        L.ixo_linear8.argtypes = [f32p, f32p, i8p, f32p, i32p, C.c_int, C.c_int, C.c_int,
                                  C.c_void_p, C.c_int, C.c_float]
        L.ixo_layernorm_row.argtypes = [f32p, f32p, f32p, C.c_int, C.c_double, C.c_int]
        L.ixo_gelu_mul.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int]
        L.ixo_exp_shift.argtypes = [f32p, C.c_int, C.c_float, C.c_int]
        L.ixo_exp_shift.restype = C.c_float
        L.ixo_quantize_row_u8.argtypes = [C.POINTER(C.c_uint8), f32p, C.c_int, C.c_float, C.c_int]
        L.ixo_quantize_row_u8.restype = C.c_int32
        L.ixo_rope_table.argtypes = [C.c_double, C.c_int, C.c_int, f32p, f32p]
        L.ixo_rope.argtypes = [f32p, f32p, f32p, C.c_int]
        L.ixo_attend8.argtypes = [f32p, C.c_int, f32p, f32p, f32p, C.c_int, C.c_int,
                                  C.c_int, C.c_int, C.c_float, C.c_int]
        L.ixo_attend8_blocked.argtypes = [C.c_void_p, C.c_int, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int,
                                          C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, C.c_int]
        L.ixo_attn_prepare.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_float,
                                       i8p, f32p, i8p, f32p, i8p, f32p, f32p]
        L.ixo_encode.argtypes = [C.POINTER(IxoModel), i32p, i32p, C.c_int, f32p]
        L.ixo_encode.restype = C.c_int
        L.ixo_pool.argtypes = [f32p, i32p, C.c_int, C.c_int, C.c_int, f32p]
        L.ixo_embed_row.argtypes = [C.POINTER(IxoModel), C.c_int32, f32p]
        L.ixo_set_gemm.argtypes = [C.c_int]
        L.ixo_set_gemm.restype = None
        L.ixo_vnni_level.restype = C.c_int
        L.ixo_gemm_kind.restype = C.c_int
        L.ixo_set_threads.argtypes = [C.c_int]
        L.ixo_set_threads.restype = None
        L.ixo_max_threads.restype = C.c_int
        L.ixo_head_logits.argtypes = [f32p, C.c_int, C.c_int, f32p, f32p, C.c_int, f64p]
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- scalar ---------------------------------------------------------------
def round_half_even(v):
    return lib().ixo_round_half_even(float(v))


def exp32(v):
    return lib().ixo_exp32(float(v))


def exp_simd(v):
    return lib().ixo_exp_simd(float(v))


def gelu_fma(v):
    return lib().ixo_gelu_fma(float(v))


def gelu_scalar(v):
    return lib().ixo_gelu_scalar(float(v))


# ---- linalg ---------------------------------------------------------------
def pack_b8(b, k, n, transB=True):
    """PackB8 (linalg/int8.go:38-77) -> (q [n,k] int8, scale [n], colsum [n])."""
    b = _c(b, np.float32).reshape(-1)
    q = np.zeros((n, k), np.int8)
    s = np.zeros(n, np.float32)
    cs = np.zeros(n, np.int32)
    lib().ixo_pack_b8(b, k, n, 1 if transB else 0, q, s, cs)
    return q, s, cs


def b8_to_panels(q):
    n, k = q.shape
    kq = (k + 3) // 4
    out = np.zeros(((n + 15) // 16) * kq * 64, np.int8)
    lib().ixo_b8_to_panels(_c(q, np.int8), k, n, out)
    return out


def quantize_rows(a):
    """quantizeA (linalg/int8.go:160-191) -> (q signed [m,k], sa [m])."""
    a = _c(a, np.float32)
    m, k = a.shape
    q = np.zeros((m, k), np.int8)
    sa = np.zeros(m, np.float32)
    if m:
        lib().ixo_quantize_rows(a, k, m, k, q, k, sa)
    return q, sa


def matmul8_tile(q, w):
    """Reference integer tile: sum (q+128)*w (microKernel8Go)."""
    q = _c(q, np.int8)
    w = _c(w, np.int8)
    m, k = q.shape
    n = w.shape[0]
    t = np.zeros((m, n), np.int32)
    lib().ixo_matmul8_tile(q, k, w, k, m, n, t)
    return t


def matmul8(a, wq, sb, colsum, c=None, accumulate=False):
    """MatMul8N (linalg/int8.go:89-155): c (+)= deq(quant(a) . wq^T)."""
    a = _c(a, np.float32)
    m, k = a.shape
    n = wq.shape[0]
    out = np.zeros((m, n), np.float32) if c is None else _c(c, np.float32).copy()
    if m:
        lib().ixo_matmul8(out, n, a, k, _c(wq, np.int8), _c(sb, np.float32),
                          _c(colsum, np.int32), m, k, n, 1 if accumulate else 0)
    return out


def matmul8_outliers(a, wq, sb, colsum, ratio, c=None, accumulate=False):
    """MatMul8Outliers (linalg/int8.go:272-349): (c, chosen input channels)."""
    a = _c(a, np.float32)
    m, k = a.shape
    n = wq.shape[0]
    out = np.zeros((m, n), np.float32) if c is None else _c(c, np.float32).copy()
    cols = np.zeros(32, np.int32)
    nout = lib().ixo_matmul8_outliers(out, n, a, k, _c(wq, np.int8), _c(sb, np.float32),
                                      _c(colsum, np.int32), m, k, n, 1 if accumulate else 0,
                                      float(ratio), cols)
    return out, cols[:nout].copy()


def linear8(x, wq, sb, colsum, bias=None, outliers=False, ratio=6.0):
    """siglip linear.apply (encoder.go:36-49): x . W^T (+ bias)."""
    x = _c(x, np.float32)
    rows, k = x.shape
    n = wq.shape[0]
    dst = np.zeros((rows, n), np.float32)
    if rows:
        keep = _c(bias, np.float32) if bias is not None else None  # alive during the call
        bptr = keep.ctypes.data if keep is not None else None
        lib().ixo_linear8(dst, x, _c(wq, np.int8), _c(sb, np.float32), _c(colsum, np.int32), rows, k, n,
                          bptr, 1 if outliers else 0, float(ratio))
    return dst


def matmul8_deq(q, sa, wq, sb, colsum, c=None, accumulate=False):
    q = _c(q, np.int8)
    m, k = q.shape
    n = wq.shape[0]
    out = np.zeros((m, n), np.float32) if c is None else _c(c, np.float32).copy()
    lib().ixo_matmul8_deq(out, n, q, k, _c(sa, np.float32), _c(wq, np.int8),
                          _c(sb, np.float32), _c(colsum, np.int32), m, k, n,
                          1 if accumulate else 0)
    return out


def layernorm_rows(x, gamma, eps=1e-5, lanes=8):
    x = _c(x, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    o = np.empty_like(x2)
    g = _c(gamma, np.float32)
    for r in range(x2.shape[0]):
        row = np.empty(x2.shape[1], np.float32)
        lib().ixo_layernorm_row(row, np.ascontiguousarray(x2[r]), g, x2.shape[1], eps, lanes)
        o[r] = row
    return o.reshape(x.shape)


def gelu_mul(a, b, lanes=8):
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    a2, b2 = a.reshape(-1, a.shape[-1]), b.reshape(-1, b.shape[-1])
    o = np.empty_like(a2)
    for r in range(a2.shape[0]):
        row = np.empty(a2.shape[1], np.float32)
        lib().ixo_gelu_mul(row, np.ascontiguousarray(a2[r]), np.ascontiguousarray(b2[r]),
                           a2.shape[1], lanes)
        o[r] = row
    return o.reshape(a.shape)


def exp_shift(x, m, lanes=8):
    x = _c(x, np.float32).copy()
    s = lib().ixo_exp_shift(x, x.size, float(m), lanes)
    return x, s


def quantize_row_u8(x, inv, lanes=8):
    x = _c(x, np.float32)
    dst = np.zeros(x.size, np.uint8)
    s = lib().ixo_quantize_row_u8(dst.ctypes.data_as(C.POINTER(C.c_uint8)), x, x.size, float(inv), lanes)
    return dst, int(s)


def rope_table(theta, D, rows):
    half = D // 2
    c = np.zeros((rows, half), np.float32)
    s = np.zeros((rows, half), np.float32)
    lib().ixo_rope_table(float(theta), D, rows, c, s)
    return c, s


def rope(x, cos_row, sin_row):
    x = _c(x, np.float32).copy()
    lib().ixo_rope(x, _c(cos_row, np.float32), _c(sin_row, np.float32), x.size // 2)
    return x


def attend8(q, k, v, window=-1, scale=0.125, lanes=8):
    """Attend8 (linalg/attention8.go:70-73) on [n, D] operands."""
    q, k, v = (_c(t, np.float32) for t in (q, k, v))
    n, D = q.shape
    o = np.zeros((n, D), np.float32)
    if n:
        lib().ixo_attend8(o, D, q, k, v, D, n, D, window, scale, lanes)
    return o


def set_gemm(kind):
    """MatMul8N of the oracle: 0 the plain restatement (the checker), 1 the
    VPDPBUSD tiles of vnni.c where the CPU has VNNI (the timed baseline).
    Returns the VNNI level in use (2 AVX-512, 1 AVX-VNNI, 0 plain)."""
    lib().ixo_set_gemm(int(kind))
    return lib().ixo_gemm_kind()


def attend8_blocked(o, off, ldo, q, k, v, i0, i1, window=-1, scale=0.125, lanes=8, plant=0):
    """Attn8.Attend as the reference blocks it, queries [i0, i1) written to
    the float32 array o from element `off` on, rows ldo apart."""
    q, k, v = (_c(t, np.float32) for t in (q, k, v))
    n, D = q.shape
    assert o.dtype == np.float32 and o.flags.c_contiguous
    assert off + (i1 - i0 - 1) * ldo + D <= o.size
    lib().ixo_attend8_blocked(o.ctypes.data + 4 * off, ldo, q, k, v, D, n, D, i0, i1, window, scale, lanes, plant)


def attn_prepare(q, k, v, scale=0.125):
    q, k, v = (_c(t, np.float32) for t in (q, k, v))
    n, D = q.shape
    out = dict(qq=np.zeros((n, D), np.int8), sq=np.zeros(n, np.float32),
               kq=np.zeros((n, D), np.int8), ks=np.zeros(n, np.float32),
               vq=np.zeros((n, D), np.int8), vs=np.zeros(D, np.float32),
               kmean=np.zeros(D, np.float32))
    lib().ixo_attn_prepare(q, k, v, D, n, D, scale, out["qq"], out["sq"], out["kq"],
                           out["ks"], out["vq"], out["vs"], out["kmean"])
    return out


# ---- encoder --------------------------------------------------------------
class OracleModel:
    """Holds the numpy weights of a model (see indecis_amd.modernbert.Weights)
    and runs the oracle encoder on them."""

    def __init__(self, w, lanes=8):
        self.w = w
        self.lanes = lanes
        cfg = w.cfg
        self._keep = []
        m = IxoModel()
        m.hidden, m.layers, m.heads = cfg.hidden, cfg.layers, cfg.heads
        m.intermediate, m.vocab = cfg.intermediate, cfg.vocab
        m.norm_eps = cfg.norm_eps
        m.global_every, m.local_attention, m.lanes = cfg.global_every, cfg.local_attention, lanes

        def ptr(a, dt):
            a = np.ascontiguousarray(a, dtype=dt)
            self._keep.append(a)
            return a.ctypes.data

        m.wqkv_q, m.wqkv_s = ptr(w.wqkv_q, np.int8), ptr(w.wqkv_s, np.float32)
        m.wo_q, m.wo_s = ptr(w.wo_q, np.int8), ptr(w.wo_s, np.float32)
        m.wi_q, m.wi_s = ptr(w.wi_q, np.int8), ptr(w.wi_s, np.float32)
        m.womlp_q, m.womlp_s = ptr(w.womlp_q, np.int8), ptr(w.womlp_s, np.float32)
        m.attn_norm, m.mlp_norm = ptr(w.attn_norm, np.float32), ptr(w.mlp_norm, np.float32)
        m.emb_norm, m.final_norm = ptr(w.emb_norm, np.float32), ptr(w.final_norm, np.float32)
        m.emb_format = w.emb_format
        if w.emb_format == EMB_F32:
            m.emb_f32 = ptr(w.emb_f32, np.float32)
        elif w.emb_format == EMB_BF16:
            m.emb_bf16 = ptr(w.emb_bf16, np.uint16)
            m.emb_n_exact = len(w.emb_exact_ids)
            m.emb_exact_ids = ptr(w.emb_exact_ids, np.int32)
            m.emb_exact_rows = ptr(w.emb_exact_rows, np.float32)
        else:
            m.emb_i8 = ptr(w.emb_i8, np.int8)
            m.emb_i8_scale = ptr(w.emb_i8_scale, np.float32)
        self.m = m
        self._ptr = ptr
        self._rope(w.rope_rows)

    def _rope(self, rows):
        """ropeFor tables covering max(rows, 512) positions (model.go:256-277)."""
        cfg, m, ptr = self.w.cfg, self.m, self._ptr
        rows = max(rows, 512)
        D = cfg.hidden // cfg.heads
        cg, sg = rope_table(cfg.global_theta, D, rows)
        cl, sl = rope_table(cfg.local_theta, D, rows)
        m.rope_cos_global, m.rope_sin_global = ptr(cg, np.float32), ptr(sg, np.float32)
        m.rope_cos_local, m.rope_sin_local = ptr(cl, np.float32), ptr(sl, np.float32)
        m.rope_rows = rows

    def set_rope(self, cos_g, sin_g, cos_l, sin_l):
        """RoPE tables given by a caller ([rows][D/2] each, as ropeFor
        returns them, model.go:256-277), used as they are for batches of
        up to `rows` tokens."""
        m, ptr = self.m, self._ptr
        rows = min(len(cos_g), len(sin_g), len(cos_l), len(sin_l))
        m.rope_cos_global, m.rope_sin_global = ptr(cos_g, np.float32), ptr(sin_g, np.float32)
        m.rope_cos_local, m.rope_sin_local = ptr(cos_l, np.float32), ptr(sin_l, np.float32)
        m.rope_rows = rows

    def embed_row(self, id_):
        """embRow (infer.go:52-59, embeddings.go:48-68): the table row of id."""
        out = np.zeros(self.w.cfg.hidden, np.float32)
        lib().ixo_embed_row(C.byref(self.m), int(id_), out)
        return out

    def encode_tokens(self, seqs):
        """EncodeTokens (infer.go:293-299): [N, H] final states."""
        ids = np.concatenate([np.asarray(s, np.int32) for s in seqs]) if seqs else np.zeros(0, np.int32)
        offs = np.zeros(len(seqs) + 1, np.int32)
        offs[1:] = np.cumsum([len(s) for s in seqs])
        N = int(offs[-1])
        T = max((len(s) for s in seqs), default=0)
        if T > self.m.rope_rows:
            self._rope(T)
        H = self.w.cfg.hidden
        out = np.zeros((max(N, 1), H), np.float32)
        rc = lib().ixo_encode(C.byref(self.m), _c(ids, np.int32) if N else np.zeros(1, np.int32),
                              offs, len(seqs), out)
        if rc != 0:
            raise ValueError("modernbert: id out of vocabulary")
        return out[:N], offs

    def encode_seqs(self, seqs):
        """EncodeSeqs (infer.go:261-289): [B, H] pooled."""
        hidden, offs = self.encode_tokens(seqs)
        return pool(hidden, offs, self.w.cfg.hidden, self.w.cfg.pooling == "cls")


def pool(hidden, offs, H, cls=False):
    B = len(offs) - 1
    out = np.zeros((B, H), np.float32)
    h = _c(hidden, np.float32) if hidden.size else np.zeros((1, H), np.float32)
    lib().ixo_pool(h, _c(offs, np.int32), B, H, 1 if cls else 0, out)
    return out


def head_logits(x, w, b):
    x = _c(x, np.float32)
    T, H = x.shape
    rows = w.shape[0]
    z = np.zeros((T, rows), np.float64)
    lib().ixo_head_logits(x, T, H, _c(w, np.float32), _c(b, np.float32), rows, z)
    return z


def embed_normalize(rows):
    """Model.embed's scaling (open.go:134-146): per row, n = the float64
    sum of float64 squares in column order, inv = float32(1 / sqrt(max(n,
    1e-24))), each value times inv in float32. np.cumsum adds in order."""
    x = np.asarray(rows, np.float32)
    out = np.empty_like(x)
    for i, r in enumerate(x):
        d = r.astype(np.float64)
        n = float(np.cumsum(d * d)[-1]) if r.size else 0.0
        inv = np.float32(1.0 / np.sqrt(max(n, 1e-24)))
        out[i] = r * inv
    return out
