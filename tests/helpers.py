"""Shared inputs of the tests: the BASELINE.json configurations as seeded
random-init models and seeded id batches."""
import numpy as np

from indecis_amd.modernbert import BASE, SMALL, Config, Weights

CLS_ID, SEP_ID = 1, 2  # special ids (< 5) used as CLS and SEP in cfg2


def small_cfg(**kw):
    c = Config(**{**SMALL.__dict__, **kw})
    return c


def base_cfg(**kw):
    return Config(**{**BASE.__dict__, **kw})


def bekko_cfg(**kw):
    """The reference's own int8 backbone width, bekko-embedding-v1-a8m:
    hidden 384 (6 heads of 64), MLP 2 x 1152 (linalg/gemm_test.go:104-105)."""
    return Config(**{**BASE.__dict__, "hidden": 384, "heads": 6, "intermediate": 1152,
                     "vocab": 32768, **kw})


def ids_cfg2(rng, B=64, T=15, vocab=32768):
    """cfg2: B x T tokens, ids uniform in [5, vocab), CLS first, SEP last."""
    seqs = []
    for _ in range(B):
        s = rng.integers(5, vocab, size=T, dtype=np.int32)
        s[0], s[-1] = CLS_ID, SEP_ID
        seqs.append(s)
    return seqs


def ids_uniform_lengths(rng, B, lo, hi, vocab):
    """Lengths uniform in [lo, hi], ids uniform over the vocabulary."""
    lens = rng.integers(lo, hi + 1, size=B)
    return [rng.integers(0, vocab, size=int(n), dtype=np.int32) for n in lens]


def f32_bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def mismatch_report(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    if a.shape != b.shape:
        return f"shape {a.shape} vs {b.shape}"
    d = a.view(np.uint32) != b.view(np.uint32)
    n = int(d.sum())
    if n == 0:
        return "identical"
    idx = np.argwhere(d)[:5]
    diff = np.abs(a.astype(np.float64) - b.astype(np.float64))
    return (f"{n}/{a.size} differ, max abs {diff.max():.3g}, mean abs {diff.mean():.3g}, "
            f"first at {idx.tolist()}: {[float(a[tuple(i)]) for i in idx]} vs {[float(b[tuple(i)]) for i in idx]}")
