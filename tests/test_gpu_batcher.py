"""WithBatching on the GPU (batch.go, model.go:136-160): requests from
concurrent callers grouped into single encode passes, through the C ABI
(ixh_batcher_*). Each request must get exactly what EncodeSeqs gives it
alone (the pass is the same computation, sequences being independent:
forward_test.go:141-160), and an error of a pass reaches its requests."""
import threading

import numpy as np
import pytest

from helpers import f32_bits_equal, ids_uniform_lengths, mismatch_report, small_cfg
from indecis_amd import _lib
from indecis_amd.modernbert import Batcher, Model, Weights
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

_pair = {}


def pair():
    if not _pair:
        cfg = small_cfg(layers=2)
        w = Weights.random(cfg, seed=31)
        _pair["v"] = (cfg, Model(w, lanes=8), orc.OracleModel(w, lanes=8))
    return _pair["v"]


def _run_clients(bat, reqs, clients):
    got, errs = [None] * len(reqs), [None] * len(reqs)

    def client(k):
        for i in range(k, len(reqs), clients):
            try:
                got[i] = bat.encode_seqs(reqs[i])
            except _lib.IxhError as e:
                errs[i] = e

    ts = [threading.Thread(target=client, args=(k,)) for k in range(clients)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=300)
    return got, errs


@pytest.mark.parametrize("workers,max_rows", [(1, 0), (2, 700)])
def test_batcher_equals_encode_seqs(workers, max_rows):
    """48 requests of 1-3 sequences (1-200 tokens) from 8 threads: every
    pooled row equals the request's own EncodeSeqs, and one equals the
    oracle."""
    cfg, gpu, ora = pair()
    rng = np.random.default_rng(32 + workers)
    reqs = [ids_uniform_lengths(rng, int(rng.integers(1, 4)), 1, 200, cfg.vocab) for _ in range(48)]
    want = [gpu.encode_seqs(r) for r in reqs]
    bat = Batcher(gpu, workers=workers, max_rows=max_rows)
    got, errs = _run_clients(bat, reqs, 8)
    passes, served = bat.stats()
    bat.close()
    assert all(e is None for e in errs), errs
    assert served == len(reqs) and 1 <= passes <= served
    print(f"{served} requests in {passes} passes")
    for g, w in zip(got, want):
        assert f32_bits_equal(g, w), mismatch_report(g, w)
    assert f32_bits_equal(got[0], ora.encode_seqs(reqs[0]))


def test_batcher_errors():
    """An id out of vocabulary fails its pass with the reference's message
    (infer.go:311); concurrent requests either succeed exactly or, if they
    shared that pass, get the same error (batch.go:76-79). The batcher keeps
    serving afterwards."""
    cfg, gpu, _ = pair()
    bat = Batcher(gpu, workers=1)
    with pytest.raises(_lib.IxhError, match="modernbert: id 40000 out of vocabulary"):
        bat.encode_seqs([np.array([1, 40000, 2], np.int32)])
    assert bat.encode_seqs([]).shape == (0, cfg.hidden)
    rng = np.random.default_rng(33)
    reqs = [ids_uniform_lengths(rng, 2, 1, 64, cfg.vocab) for _ in range(24)]
    for i in (3, 11, 19):
        reqs[i] = [np.array([5, cfg.vocab + 7], np.int32)]
    got, errs = _run_clients(bat, reqs, 6)
    for i, r in enumerate(reqs):
        if i in (3, 11, 19):
            assert errs[i] is not None and f"id {cfg.vocab + 7} out of vocabulary" in str(errs[i])
        elif errs[i] is not None:
            assert f"id {cfg.vocab + 7} out of vocabulary" in str(errs[i])
        else:
            assert f32_bits_equal(got[i], gpu.encode_seqs(r))
    good = ids_uniform_lengths(rng, 3, 1, 64, cfg.vocab)
    assert f32_bits_equal(bat.encode_seqs(good), gpu.encode_seqs(good))
    bat.close()
