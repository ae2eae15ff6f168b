"""Host-side mirror of indecis's internal/modernbert inference API, backed by
the gfx950 library through its C ABI (include/indecis_hip.h).

Config mirrors modernbert.Config (internal/modernbert/model.go:26-80);
Model.encode_seqs / encode_tokens / encode mirror EncodeSeqs / EncodeTokens
/ Encode (infer.go:244-299) with the same argument meaning and the same
errors ("modernbert: id N out of vocabulary", "modernbert: inconsistent
batch"). Weights holds a model's int8 matrices as PackB8 leaves them
(int8.go:38-77); Weights.random builds the seeded random-init models the
parity tests and the benchmark use.
"""
import ctypes as C
import dataclasses
import json

import numpy as np

from . import _lib

EMB_F32, EMB_BF16, EMB_I8 = 0, 1, 2


@dataclasses.dataclass
class Config:
    """modernbert.Config (model.go:26-49)."""
    hidden: int
    layers: int
    heads: int
    intermediate: int
    vocab: int
    norm_eps: float = 1e-5
    global_every: int = 3
    local_attention: int = 128
    global_theta: float = 160000.0
    local_theta: float = 10000.0
    pooling: str = "mean"
    pad_id: int = 0
    activation: str = "gelu"

    def head_dim(self):
        return self.hidden // self.heads

    def is_global(self, layer):
        """IsGlobal (model.go:59)."""
        return layer % self.global_every == 0

    def window(self):
        """Window (model.go:62): half of the local attention width."""
        return self.local_attention // 2

    def cls(self):
        return self.pooling == "cls"

    def validate(self):
        """validate (model.go:64-80)."""
        if min(self.hidden, self.layers, self.heads, self.intermediate, self.vocab) <= 0:
            raise ValueError("modernbert: invalid dimensions")
        if self.hidden % self.heads != 0 or self.head_dim() % 2 != 0:
            raise ValueError(f"modernbert: hidden_size {self.hidden} incompatible with {self.heads} heads")
        if self.global_every <= 0 or self.local_attention <= 0:
            raise ValueError("modernbert: invalid attention windows")
        if self.activation != "gelu":
            raise ValueError(f'modernbert: activation "{self.activation}" not supported')
        if self.pooling not in ("", "mean", "cls"):
            raise ValueError(f'modernbert: pooling "{self.pooling}" not supported')

    @classmethod
    def from_json(cls, text):
        """config.json fields read by Load (model.go:124-144)."""
        d = json.loads(text)
        if d.get("attention_bias") or d.get("mlp_bias") or d.get("norm_bias"):
            raise ValueError("modernbert: biases are not supported")
        return cls(hidden=d["hidden_size"], layers=d["num_hidden_layers"],
                   heads=d["num_attention_heads"], intermediate=d["intermediate_size"],
                   vocab=d["vocab_size"], norm_eps=d.get("norm_eps", 1e-5),
                   global_every=d["global_attn_every_n_layers"],
                   local_attention=d["local_attention"],
                   global_theta=d.get("global_rope_theta", 160000.0),
                   local_theta=d.get("local_rope_theta", 10000.0),
                   pooling=d.get("classifier_pooling", "") or "mean",
                   pad_id=d.get("pad_token_id", 0),
                   activation=d.get("hidden_activation", "gelu"))


# The BASELINE.json shapes.
SMALL = Config(hidden=256, layers=6, heads=4, intermediate=512, vocab=32768)
BASE = Config(hidden=768, layers=22, heads=12, intermediate=1152, vocab=50368)


def pack_b8(w, transB=True):
    """PackB8 (linalg/int8.go:38-77) of op(B) k x n: per output channel j,
    s = max|w|/127 (float32), q = math.Round(float64(float32(w/s))) (half
    away from zero). Returns q [n][k] int8, scale [n] float32."""
    w = np.asarray(w, np.float32)
    wt = w if transB else w.T          # [n][k]
    mx = np.abs(wt).max(axis=1)
    s = (mx / np.float32(127)).astype(np.float32)
    safe = np.where(s == 0, np.float32(1), s).astype(np.float32)
    x = (wt / safe[:, None]).astype(np.float32).astype(np.float64)
    q = np.trunc(x + np.copysign(0.5, x))
    q = np.where(s[:, None] == 0, 0, q).astype(np.int8)
    return np.ascontiguousarray(q), np.where(mx == 0, np.float32(0), s).astype(np.float32)


class Weights:
    """The tensors a model needs on the int8 path, layer-major:
    wqkv_q [L][3H][H], wo_q [L][H][H], wi_q [L][2I][H] (GELU-input rows then
    gate rows, model.go:96), womlp_q [L][H][I] int8 with one float32 scale
    per output channel; LayerNorm weights; the embedding table."""

    def __init__(self, cfg, rope_rows=512):
        self.cfg = cfg
        self.rope_rows = rope_rows
        self.emb_format = EMB_F32
        self.emb_f32 = None
        self.emb_bf16 = None
        self.emb_exact_ids = np.zeros(0, np.int32)
        self.emb_exact_rows = np.zeros((0, cfg.hidden), np.float32)
        self.emb_i8 = None
        self.emb_i8_scale = None

    @staticmethod
    def random(cfg, seed=0, emb_format=EMB_F32, weight_scale=(2e-4, 6e-4), n_exact=8):
        """Seeded random-init model: int8 weights U[-127, 127] with scales
        U(weight_scale) (an effective std of about 0.015-0.045), LayerNorm
        weights U(0.9, 1.1), embeddings N(0, 1) in the requested format."""
        rng = np.random.default_rng(seed)
        H, I, L, V = cfg.hidden, cfg.intermediate, cfg.layers, cfg.vocab
        w = Weights(cfg)

        def mat(n, k):
            q = rng.integers(-127, 128, size=(L, n, k), dtype=np.int8)
            s = rng.uniform(*weight_scale, size=(L, n)).astype(np.float32)
            return q, s

        w.wqkv_q, w.wqkv_s = mat(3 * H, H)
        w.wo_q, w.wo_s = mat(H, H)
        w.wi_q, w.wi_s = mat(2 * I, H)
        w.womlp_q, w.womlp_s = mat(H, I)
        w.attn_norm = rng.uniform(0.9, 1.1, size=(L, H)).astype(np.float32)
        w.mlp_norm = rng.uniform(0.9, 1.1, size=(L, H)).astype(np.float32)
        w.emb_norm = rng.uniform(0.9, 1.1, size=H).astype(np.float32)
        w.final_norm = rng.uniform(0.9, 1.1, size=H).astype(np.float32)
        emb = rng.standard_normal((V, H), dtype=np.float32)
        w.set_embeddings(emb, emb_format, rng=rng, n_exact=n_exact)
        return w

    def set_embeddings(self, emb, fmt, rng=None, n_exact=8):
        """Stores a float32 table in one of the three formats the reference
        reads (embeddings.go:24-68): float32; bf16 (truncated) plus n_exact
        float32 rows that override their ids; int8 with a scale per row."""
        emb = np.ascontiguousarray(emb, np.float32)
        self.emb_format = fmt
        if fmt == EMB_F32:
            self.emb_f32 = emb
        elif fmt == EMB_BF16:
            self.emb_bf16 = (emb.view(np.uint32) >> 16).astype(np.uint16)
            rng = rng or np.random.default_rng(0)
            ids = rng.choice(emb.shape[0], size=min(n_exact, emb.shape[0]), replace=False)
            self.emb_exact_ids = np.sort(ids).astype(np.int32)
            self.emb_exact_rows = emb[self.emb_exact_ids] * np.float32(1.25)
        elif fmt == EMB_I8:
            mx = np.abs(emb).max(axis=1)
            s = (mx / np.float32(127)).astype(np.float32)
            safe = np.where(s == 0, np.float32(1), s)
            self.emb_i8 = np.clip(np.rint(emb / safe[:, None]), -127, 127).astype(np.int8)
            self.emb_i8_scale = s
        else:
            raise ValueError(f"embedding format {fmt}")


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def _offsets(seqs):
    offs = np.zeros(len(seqs) + 1, np.int32)
    if seqs:
        offs[1:] = np.cumsum([len(s) for s in seqs])
    ids = (np.concatenate([np.asarray(s, np.int32) for s in seqs])
           if seqs and offs[-1] > 0 else np.zeros(1, np.int32))
    return np.ascontiguousarray(ids, np.int32), offs


class Model:
    """modernbert.Model on the int8 path, its weights resident on one GPU."""

    def __init__(self, weights, device=0, lanes=8, cfg=None):
        self.cfg = cfg = weights.cfg if weights is not None else cfg
        cfg.validate()
        self.lanes = lanes
        L = _lib.lib()
        c = _lib.IxhConfig(
            hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads,
            intermediate=cfg.intermediate, vocab=cfg.vocab, norm_eps=cfg.norm_eps,
            global_every=cfg.global_every, local_attention=cfg.local_attention,
            global_theta=cfg.global_theta, local_theta=cfg.local_theta,
            pooling=_lib.POOL_CLS if cfg.cls() else _lib.POOL_MEAN, lanes=lanes)
        h = C.c_void_p()
        _lib.check(L.ixh_model_create(C.byref(c), device, C.byref(h)))
        self._h = h
        self._L = L
        self.device = device
        if weights is not None:
            self.upload(weights)

    @classmethod
    def open(cls, cfg, path, device=0, lanes=8):
        """Load (model.go:640-740) of an indecis model.safetensors straight
        into device memory: see load_safetensors."""
        m = cls(None, device=device, lanes=lanes, cfg=cfg)
        try:
            m.load_safetensors(path)
        except Exception:
            m.close()
            raise
        return m

    def load_safetensors(self, path):
        """Every weight from a model.safetensors (ixh_model_load_safetensors):
        the embedding table in its stored format, each layer matrix packed
        by PackB8 on the host, the LayerNorm weights."""
        _lib.check(self._L.ixh_model_load_safetensors(self._h, str(path).encode()))

    def upload(self, w):
        """packs() (infer.go:184-219): uploads every matrix and table."""
        L, h, cfg = self._L, self._h, self.cfg
        for l in range(cfg.layers):
            for which, q, s in ((_lib.MAT_QKV, w.wqkv_q, w.wqkv_s), (_lib.MAT_O, w.wo_q, w.wo_s),
                                (_lib.MAT_I, w.wi_q, w.wi_s), (_lib.MAT_OMLP, w.womlp_q, w.womlp_s)):
                qa = np.ascontiguousarray(q[l], np.int8)
                sa = np.ascontiguousarray(s[l], np.float32)
                _lib.check(L.ixh_model_set_matrix(h, l, which, _ptr(qa), _ptr(sa), _lib.LAYOUT_ROWS))
            if l > 0:
                g = np.ascontiguousarray(w.attn_norm[l], np.float32)
                _lib.check(L.ixh_model_set_norm(h, _lib.NORM_ATTN, l, _ptr(g)))
            g = np.ascontiguousarray(w.mlp_norm[l], np.float32)
            _lib.check(L.ixh_model_set_norm(h, _lib.NORM_MLP, l, _ptr(g)))
        for which, g in ((_lib.NORM_EMB, w.emb_norm), (_lib.NORM_FINAL, w.final_norm)):
            g = np.ascontiguousarray(g, np.float32)
            _lib.check(L.ixh_model_set_norm(h, which, 0, _ptr(g)))
        if w.emb_format == EMB_F32:
            _lib.check(L.ixh_model_set_embeddings_f32(h, _ptr(w.emb_f32)))
        elif w.emb_format == EMB_BF16:
            ids = np.ascontiguousarray(w.emb_exact_ids, np.int32)
            rows = np.ascontiguousarray(w.emb_exact_rows, np.float32)
            _lib.check(L.ixh_model_set_embeddings_bf16(h, _ptr(w.emb_bf16), _ptr(ids), _ptr(rows), len(ids)))
        else:
            _lib.check(L.ixh_model_set_embeddings_i8(h, _ptr(w.emb_i8), _ptr(w.emb_i8_scale)))

    def set_rope(self, is_global, cos_t, sin_t):
        """Go's ropeFor tables (model.go:256-277), [rows][D/2]."""
        c = np.ascontiguousarray(cos_t, np.float32)
        s = np.ascontiguousarray(sin_t, np.float32)
        _lib.check(self._L.ixh_model_set_rope(self._h, 1 if is_global else 0, _ptr(c), _ptr(s), c.shape[0]))

    def reset_rope(self, is_global):
        """Back to the library's own RoPE tables (the ropeFor formula)."""
        _lib.check(self._L.ixh_model_set_rope(self._h, 1 if is_global else 0, None, None, 0))

    def set_option(self, name, value):
        """A kernel or pass choice (ixh_model_set_option): parts,
        pass_tokens, qkv_fused, qkv_heads, gemm, gemm_tile, ln_seg.
        Results never depend on it."""
        _lib.check(self._L.ixh_model_set_option(self._h, _lib.OPTIONS[name], int(value)))

    def option(self, name):
        v = C.c_int64(0)
        _lib.check(self._L.ixh_model_get_option(self._h, _lib.OPTIONS[name], C.byref(v)))
        return v.value

    def set_heads(self, heads):
        """The decision heads on the device (ixh_model_set_heads): a list
        of (w [rows, H], b [rows], per_token) in order; [] removes them."""
        n = len(heads)
        ws = [np.ascontiguousarray(w, np.float32) for w, _, _ in heads]
        bs = [np.ascontiguousarray(b, np.float32) for _, b, _ in heads]
        rows = np.array([w.shape[0] for w in ws] or [0], np.int32)
        tok = np.array([1 if t else 0 for _, _, t in heads] or [0], np.int32)
        wp = (C.c_void_p * max(n, 1))(*[w.ctypes.data for w in ws])
        bp = (C.c_void_p * max(n, 1))(*[b.ctypes.data for b in bs])
        _lib.check(self._L.ixh_model_set_heads(self._h, n, _ptr(rows), _ptr(tok), C.cast(wp, C.c_void_p),
                                               C.cast(bp, C.c_void_p)))
        self._heads = [(w.shape[0], bool(t)) for (w, _, t) in zip(ws, bs, [h[2] for h in heads])]

    def encode_heads(self, seqs, mean=False, pooled=True, tokens=True):
        """infer's GPU half (ixh_encode_heads): (pooled_z [B, Rp] or None,
        token_z [N, Rt] or None), the logits of the pooled-row heads and of
        the per-token heads, in the order they were set."""
        heads = getattr(self, "_heads", [])
        rp = sum(r for r, t in heads if not t)
        rt = sum(r for r, t in heads if t)
        ids, offs = _offsets(seqs)
        B, N = len(seqs), int(offs[-1])
        zp = np.zeros((max(B, 1), max(rp, 1)), np.float64) if pooled and rp else None
        zt = np.zeros((max(N, 1), max(rt, 1)), np.float64) if tokens and rt else None
        _lib.check(self._L.ixh_encode_heads(self._h, _ptr(ids), _ptr(offs), B, 1 if mean else 0,
                                            _ptr(zp) if zp is not None else None,
                                            _ptr(zt) if zt is not None else None))
        return (zp[:B, :rp] if zp is not None else None), (zt[:N, :rt] if zt is not None else None)

    def invalidate(self):
        """Invalidate (infer.go:95-100)."""
        _lib.check(self._L.ixh_model_invalidate(self._h))

    def encode_seqs(self, seqs):
        """EncodeSeqs (infer.go:261-289): [B, H] pooled embeddings."""
        ids, offs = _offsets(seqs)
        out = np.zeros((max(len(seqs), 1), self.cfg.hidden), np.float32)
        _lib.check(self._L.ixh_encode_seqs(self._h, _ptr(ids), _ptr(offs), len(seqs), _ptr(out)))
        return out[:len(seqs)]

    def embed(self, tokenizer, texts, max_len=256, threads=0):
        """Model.Embed (open.go:118-155): [n, H] embeddings of norm 1, each
        text through EncodeMax(text, max_len) (max_len 256 as Open sets
        it, model.go:265) on `threads` host threads, then the encoder."""
        bs = [t.encode("utf-8") if isinstance(t, str) else bytes(t) for t in texts]
        n = len(bs)
        arr = (C.c_char_p * max(n, 1))(*bs)
        lens = np.array([len(b) for b in bs] or [0], np.int64)
        out = np.zeros((max(n, 1), self.cfg.hidden), np.float32)
        _lib.check(self._L.ixh_embed_texts(self._h, tokenizer._h, C.cast(arr, C.c_void_p), _ptr(lens), n,
                                           max_len, threads, _ptr(out)))
        return out[:n]

    def encode_tokens(self, seqs):
        """EncodeTokens (infer.go:293-299): [sum of lengths, H]."""
        ids, offs = _offsets(seqs)
        N = int(offs[-1])
        out = np.zeros((max(N, 1), self.cfg.hidden), np.float32)
        _lib.check(self._L.ixh_encode_tokens(self._h, _ptr(ids), _ptr(offs), len(seqs), _ptr(out)))
        return out[:N]

    def encode(self, ids, lens, T):
        """Encode (infer.go:244-253): a batch right-padded to T tokens
        (IDs [B*T], Lens [B]); padding never reaches the GPU."""
        ids = np.asarray(ids, np.int32)
        if ids.size != len(lens) * T:
            raise ValueError("modernbert: inconsistent batch")
        return self.encode_seqs([ids[i * T:i * T + n] for i, n in enumerate(lens)])

    def encode_device(self, ids_ptr, offs, out_ptr, kind=_lib.OUT_POOLED, stream=None):
        """ixh_encode_device: ids and out are device pointers (ints)."""
        offs = np.ascontiguousarray(offs, np.int32)
        _lib.check(self._L.ixh_encode_device(self._h, C.c_void_p(ids_ptr), _ptr(offs), len(offs) - 1,
                                             kind, C.c_void_p(out_ptr),
                                             C.c_void_p(stream) if stream else None))

    def set_profiling(self, on, only=None):
        """Per-kernel HIP-event timing of every encode (clears the sums);
        `only` restricts it to one kernel class."""
        _lib.check(self._L.ixh_model_set_profile_filter(self._h, (only or "").encode()))
        _lib.check(self._L.ixh_model_set_profiling(self._h, 1 if on else 0))

    def profile(self):
        """{kernel class: dict(launches, ms, ops, bytes)} summed since
        profiling was turned on."""
        n = C.c_int(0)
        _lib.check(self._L.ixh_model_profile(self._h, None, 0, C.byref(n)))
        arr = (_lib.IxhKernelStat * max(n.value, 1))()
        _lib.check(self._L.ixh_model_profile(self._h, arr, n.value, C.byref(n)))
        return {a.name.decode(): dict(launches=a.launches, ms=a.ms, ops=a.ops, bytes=a.bytes)
                for a in arr[:n.value]}

    def head_logits(self, x, w, b):
        """head.logits (heads.go:63-74) of rows x: [T, rows] float64."""
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        z = np.zeros((max(x.shape[0], 1), w.shape[0]), np.float64)
        _lib.check(self._L.ixh_head_logits(self._h, _ptr(x), x.shape[0], _ptr(w), _ptr(b), w.shape[0], _ptr(z)))
        return z[:x.shape[0]]

    def close(self):
        if self._h:
            self._L.ixh_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Batcher:
    """WithBatching (model.go:136-160) / batcher (batch.go): encode_seqs
    calls from concurrent threads are grouped into single encode passes of
    up to max_rows tokens by `workers` native threads (0: library
    defaults, 2 workers and 65536 tokens). The model must outlive it."""

    def __init__(self, model, workers=0, max_rows=0):
        self.model = model
        self._L = model._L
        h = C.c_void_p()
        _lib.check(self._L.ixh_batcher_create(model._h, workers, max_rows, C.byref(h)))
        self._h = h

    def encode_seqs(self, seqs):
        """batcher.encode (batch.go:32-49): [B, H] pooled embeddings; an
        error of the pass the request joined is raised here."""
        ids, offs = _offsets(seqs)
        out = np.zeros((max(len(seqs), 1), self.model.cfg.hidden), np.float32)
        _lib.check(self._L.ixh_batcher_encode(self._h, _ptr(ids), _ptr(offs), len(seqs), _ptr(out)))
        return out[:len(seqs)]

    def stats(self):
        """(passes run, requests served) so far."""
        b, r = C.c_int64(0), C.c_int64(0)
        _lib.check(self._L.ixh_batcher_stats(self._h, C.byref(b), C.byref(r)))
        return b.value, r.value

    def close(self):
        if self._h:
            self._L.ixh_batcher_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
