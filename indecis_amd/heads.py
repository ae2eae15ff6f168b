"""Decision heads on the pooled or per-token states (root package of
indecis: heads.go, spans.go). Logits are computed on the GPU in float64
(Model.head_logits); turning them into answers is host float64 work, as in
the reference: sigmoid/softmax (heads.go:125-223) and the spans
log-softmax (spans.go:293-311).
"""
import numpy as np


def span_tag_count(types):
    """spanTagCount (spans.go:125): outside + begin/inside per type."""
    return 1 + 2 * types


def sigmoid(z):
    """heads.go:189-195 (stable for both signs)."""
    z = np.asarray(z, np.float64)
    out = np.empty_like(z)
    pos = z >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-z[pos]))
    e = np.exp(z[~pos])
    out[~pos] = e / (1.0 + e)
    return out


def softmax(z):
    """heads.go:208-223, over the last axis."""
    z = np.asarray(z, np.float64)
    p = np.exp(z - z.max(axis=-1, keepdims=True))
    return p / p.sum(axis=-1, keepdims=True)


def log_softmax(z, temperature=1.0):
    """logSoftmax (spans.go:293-311)."""
    if temperature <= 0:
        temperature = 1.0
    zt = np.asarray(z, np.float64) / temperature
    mx = zt.max(axis=-1, keepdims=True)
    lse = mx + np.log(np.exp(zt - mx).sum(axis=-1, keepdims=True))
    return zt - lse


def random_head(rows, hidden, rng):
    """newHead (heads.go:29-48): w ~ N(0, 0.02), b = 0."""
    w = (rng.standard_normal((rows, hidden)) * 0.02).astype(np.float32)
    return w, np.zeros(rows, np.float32)
