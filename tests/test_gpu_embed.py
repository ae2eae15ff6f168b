"""Model.Embed (open.go:118-155) through ixh_embed_texts: the native
tokenizer's EncodeMax, the encoder and the normalisation equal the oracle
(the same ids through OracleModel.encode_seqs, then the oracle's
normalisation), bit for bit."""
import json
import os

import numpy as np
import pytest

from helpers import small_cfg
from indecis_amd.modernbert import Model, Weights
from indecis_amd.tokenizer import Tokenizer
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOK = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tokenizer", "tokenizer.json")


def _texts():
    rng = np.random.default_rng(3)
    pool = [json.loads(line)["text"] for line in open(os.path.join(os.path.dirname(TOK), "tokenizer_cases.jsonl"),
                                                      encoding="utf-8")]
    texts = [pool[int(i)] for i in rng.integers(0, len(pool), 30)]
    texts += ["", "a", " ".join(pool[:80])]  # empty, one letter, a text past max_len
    return texts


@pytest.mark.parametrize("max_len", [256, 16])
def test_embed_equals_oracle(max_len):
    cfg = small_cfg(layers=3)
    w = Weights.random(cfg, seed=12)
    tok = Tokenizer(TOK)
    assert tok.vocab_size <= cfg.vocab
    gpu, ora = Model(w, lanes=8), orc.OracleModel(w, lanes=8)
    texts = _texts()
    got = gpu.embed(tok, texts, max_len=max_len, threads=4)
    seqs = [tok.encode(t, max_len=max_len) for t in texts]
    assert max(len(s) for s in seqs) == max_len
    want = orc.embed_normalize(ora.encode_seqs(seqs))
    gpu.close()
    assert got.shape == want.shape and np.array_equal(got.view(np.uint32), want.view(np.uint32))

