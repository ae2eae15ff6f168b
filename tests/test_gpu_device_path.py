"""The device-buffer entry point (ixh_encode_device: ids already in HBM,
output left there — the path bench.py times) against the host-buffer one
(EncodeSeqs / EncodeTokens, infer.go:244-299), bit for bit, and its error
path: the id check runs on the device and is read after the pass, so a bad
id must still give the reference's message (infer.go:311), a zeroed output,
and leave the next call exact. Device buffers come from torch."""
import numpy as np
import pytest

from helpers import f32_bits_equal, ids_uniform_lengths, mismatch_report, small_cfg
from indecis_amd import _lib
from indecis_amd.modernbert import Model, Weights

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _offs(seqs):
    offs = np.zeros(len(seqs) + 1, np.int32)
    offs[1:] = np.cumsum([len(s) for s in seqs])
    return offs


def _run(gpu, seqs, kind, hidden):
    offs = _offs(seqs)
    ids = torch.from_numpy(np.concatenate(seqs).astype(np.int32)).to("cuda")
    rows = len(seqs) if kind == _lib.OUT_POOLED else int(offs[-1])
    out = torch.full((rows, hidden), 7.0, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    gpu.encode_device(ids.data_ptr(), offs, out.data_ptr(), kind, stream)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("split", [1, 2])
def test_device_path_equals_host_path(split):
    cfg = small_cfg()
    w = Weights.random(cfg, seed=21)
    gpu = Model(w, lanes=8)
    gpu.set_option("parts", split)
    rng = np.random.default_rng(21)
    # above the two-part threshold (4,096 tokens) when split = 2
    seqs = ids_uniform_lengths(rng, 40, 1, 300, cfg.vocab)
    got = _run(gpu, seqs, _lib.OUT_POOLED, cfg.hidden)
    want = gpu.encode_seqs(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    got = _run(gpu, seqs, _lib.OUT_TOKENS, cfg.hidden)
    want = gpu.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    gpu.close()


@pytest.mark.parametrize("bad", [40000, -1, 2**31 - 1])
@pytest.mark.parametrize("kind", [_lib.OUT_POOLED, _lib.OUT_TOKENS])
def test_device_path_bad_id(bad, kind):
    cfg = small_cfg(layers=2)
    w = Weights.random(cfg, seed=22)
    gpu = Model(w, lanes=8)
    rng = np.random.default_rng(22)
    seqs = ids_uniform_lengths(rng, 6, 1, 90, cfg.vocab)
    seqs[3] = np.concatenate([seqs[3], np.array([bad, 5], np.int32)])
    offs = _offs(seqs)
    ids = torch.from_numpy(np.concatenate(seqs)).to("cuda")
    rows = len(seqs) if kind == _lib.OUT_POOLED else int(offs[-1])
    out = torch.full((rows, cfg.hidden), 7.0, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    with pytest.raises(_lib.IxhError, match=f"modernbert: id {bad} out of vocabulary"):
        gpu.encode_device(ids.data_ptr(), offs, out.data_ptr(), kind, stream)
    torch.cuda.synchronize()
    assert not out.cpu().numpy().any()
    # the model and its workspaces are fine afterwards
    seqs[3] = seqs[3][:-2]
    got = _run(gpu, seqs, kind, cfg.hidden)
    want = gpu.encode_seqs(seqs) if kind == _lib.OUT_POOLED else gpu.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    gpu.close()
