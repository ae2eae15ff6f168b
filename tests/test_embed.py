"""Model.Embed's normalisation (open.go:134-146) on the CPU: the oracle's
restatement pinned by closed forms and invariants, and the library's host
routine (ixh_embed_normalize) equal to it bit for bit."""
import ctypes as C

import numpy as np
import pytest

from indecis_amd import _lib
from oracle import oracle as orc


def _lib_normalize(x):
    x = np.ascontiguousarray(x, np.float32).copy()
    _lib.check(_lib.lib().ixh_embed_normalize(x.ctypes.data_as(C.c_void_p), x.shape[0], x.shape[1]))
    return x


def test_closed_forms():
    """3-4-5: the scale is float32(1/5) and each value is rounded once;
    a zero row stays zero (the 1e-24 floor); one nonzero value becomes +-1."""
    got = orc.embed_normalize(np.array([[3, 4], [0, 0], [0, -7.5]], np.float32))
    inv = np.float32(0.2)
    assert got[0].tolist() == [np.float32(3) * inv, np.float32(4) * inv]
    assert got[1].tolist() == [0.0, 0.0]
    assert got[2].tolist() == [0.0, -1.0]


def test_invariants_and_planted_mistake():
    """Scaling a row by 2^k leaves the output bits unchanged (every step is
    exact under it); norms are 1 within float32 rounding; summing the
    squares in float32 (a plausible slip) changes some rows' bits, which
    the float64 sum of the reference does not."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((400, 768)) * rng.uniform(0.01, 30, (400, 1))).astype(np.float32)
    y = orc.embed_normalize(x)
    assert np.array_equal(orc.embed_normalize(x * np.float32(2 ** 20)), y)
    assert np.array_equal(orc.embed_normalize(x * np.float32(2 ** -20)), y)
    assert np.abs(np.sqrt((y.astype(np.float64) ** 2).sum(1)) - 1).max() < 1e-6
    bad = np.empty_like(x)
    for i, r in enumerate(x):
        n32 = np.float32(0)
        for v in r:
            n32 = np.float32(n32 + v * v)
        bad[i] = r * np.float32(1 / np.sqrt(np.float64(n32)))
    assert not np.array_equal(bad, y)


@pytest.mark.parametrize("n,H", [(1, 768), (37, 256), (5, 1)])
def test_library_equals_oracle(n, H):
    """ixh_embed_normalize (host code) against the oracle, bit for bit,
    including a zero row and rows of large and tiny magnitude."""
    rng = np.random.default_rng(n * 7 + H)
    x = (rng.standard_normal((n, H)) * rng.uniform(1e-3, 1e3, (n, 1))).astype(np.float32)
    x[0] = 0
    assert np.array_equal(_lib_normalize(x), orc.embed_normalize(x))


def test_embed_argument_errors():
    """Nil model / tokenizer are refused before any GPU call."""
    with pytest.raises(_lib.IxhError, match="nil model or tokenizer"):
        _lib.check(_lib.lib().ixh_embed_texts(None, None, None, None, 0, 16, 0, None))
    with pytest.raises(_lib.IxhError, match="bad arguments"):
        _lib.check(_lib.lib().ixh_embed_normalize(None, 3, 4))
