"""Float64 restatement of indecis's float ModernBERT forward pass
(internal/modernbert/forward.go:67-200, ops.go:19-44), used to pin the int8
oracle the way the reference pins its int8 path: TestEncodeInt8
(internal/modernbert/infer_test.go:195-222) requires a cosine >= 0.99
between the int8 and float pooled embeddings. Test infrastructure only.

Weights are the dequantised int8 matrices (q * scale), so the two paths
see the same model; everything here is float64 and shares no code with
the C oracle.
"""
import math

import numpy as np


def layer_norm(x, gamma, eps):
    """layerNorm (ops.go:19-44), no bias."""
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * gamma


def gelu(x):
    """Exact GELU (erf)."""
    v = np.vectorize(math.erf)
    return 0.5 * x * (1.0 + v(x / math.sqrt(2.0)))


def rope_tables(theta, D, n):
    """ropeFor (model.go:256-277) in float64."""
    half = D // 2
    inv = 1.0 / theta ** (np.arange(half) * 2.0 / D)
    ang = np.arange(n)[:, None] * inv[None, :]
    return np.cos(ang), np.sin(ang)


def apply_rope(x, c, s):
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def forward_tokens(w, seq, gelu_on_gate=False):
    """Final states [n, H] of one sequence (forward.go Forward, one row of
    the batch). gelu_on_gate plants a mistake (GELU on the wrong half) for
    the sensitivity test."""
    cfg = w.cfg
    H, I, nh = cfg.hidden, cfg.intermediate, cfg.heads
    D = H // nh
    seq = np.asarray(seq)
    n = len(seq)
    if w.emb_format != 0:
        raise ValueError("float reference reads the float32 table")
    x = w.emb_f32[seq].astype(np.float64)
    x = layer_norm(x, w.emb_norm.astype(np.float64), cfg.norm_eps)
    for l in range(cfg.layers):
        wq = w.wqkv_q[l].astype(np.float64) * w.wqkv_s[l][:, None]
        wo = w.wo_q[l].astype(np.float64) * w.wo_s[l][:, None]
        wi = w.wi_q[l].astype(np.float64) * w.wi_s[l][:, None]
        wm = w.womlp_q[l].astype(np.float64) * w.womlp_s[l][:, None]
        h_in = x if l == 0 else layer_norm(x, w.attn_norm[l].astype(np.float64), cfg.norm_eps)
        qkv = h_in @ wq.T
        glob = l % cfg.global_every == 0
        theta = cfg.global_theta if glob else cfg.local_theta
        c, s = rope_tables(theta, D, n)
        ctx = np.zeros((n, H))
        scale = 1.0 / math.sqrt(D)
        i = np.arange(n)
        mask = np.ones((n, n), bool) if glob else (np.abs(i[:, None] - i[None, :]) <= cfg.local_attention // 2)
        for hd in range(nh):
            q = apply_rope(qkv[:, hd * D:(hd + 1) * D], c, s)
            k = apply_rope(qkv[:, H + hd * D:H + (hd + 1) * D], c, s)
            v = qkv[:, 2 * H + hd * D:2 * H + (hd + 1) * D]
            sc = (q @ k.T) * scale
            sc = np.where(mask, sc, -np.inf)
            sc = sc - sc.max(axis=1, keepdims=True)
            p = np.exp(sc)
            p /= p.sum(axis=1, keepdims=True)
            ctx[:, hd * D:(hd + 1) * D] = p @ v
        x = x + ctx @ wo.T
        z = layer_norm(x, w.mlp_norm[l].astype(np.float64), cfg.norm_eps) @ wi.T
        a, g = z[:, :I], z[:, I:]
        if gelu_on_gate:
            a, g = g, a
        x = x + (gelu(a) * g) @ wm.T
    return layer_norm(x, w.final_norm.astype(np.float64), cfg.norm_eps)


def pooled(w, seq, **kw):
    return forward_tokens(w, seq, **kw).mean(axis=0)
