"""GPU parity of the ABI branches a Go binding relies on, through the C ABI:
CLS pooling (infer.go:264-273), PackedB8 panel uploads (int8.go:30,
65-68), a caller's RoPE tables (ropeFor, model.go:256-277), batches over
the pass size, the decision heads on the device (heads.go:63-74,
spans.go:369-470) and cfg5's 8,192-key sequences (attention8.go:298-376),
each against the CPU oracle bit for bit; and a device allocation that
fails, as a clean error."""
import ctypes as C

import numpy as np
import pytest

from helpers import base_cfg, f32_bits_equal, ids_uniform_lengths, mismatch_report, small_cfg
from indecis_amd import _lib, heads, linalg
from indecis_amd.modernbert import Model, Weights
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _pair(cfg, seed, lanes=8):
    w = Weights.random(cfg, seed=seed)
    return w, Model(w, lanes=lanes), orc.OracleModel(w, lanes=lanes)


def test_cls_pooling():
    """Config.Pooling "cls": EncodeSeqs returns each sequence's first-token
    state (infer.go:264-273); an empty sequence gives a zero row."""
    cfg = small_cfg(layers=3, pooling="cls")
    w, gpu, ora = _pair(cfg, seed=41)
    rng = np.random.default_rng(41)
    seqs = ids_uniform_lengths(rng, 12, 1, 200, cfg.vocab)
    seqs.insert(4, np.zeros(0, np.int32))
    got = gpu.encode_seqs(seqs)
    want = ora.encode_seqs(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    states, offs = ora.encode_tokens(seqs)
    for b, s in enumerate(seqs):
        first = states[offs[b]] if len(s) else np.zeros(cfg.hidden, np.float32)
        assert f32_bits_equal(got[b], first)
    # the mean differs: the branch taken is the CLS one
    mean = orc.pool(states, offs, cfg.hidden, cls=False)
    assert not np.array_equal(got[0], mean[0])
    gpu.close()


@pytest.mark.parametrize("pooling", ["mean", "cls"])
def test_pool_long_sequences(pooling):
    """Pooling (infer.go:265-287) on the long-sequence path (a pass whose
    sequences average over 1,024 tokens: one workgroup per 64 columns
    streaming the rows through a ring): sequences of 2,000, 1, 0 and 1,300
    tokens, as one part, mean and CLS, equal the oracle bit for bit."""
    cfg = small_cfg(layers=1, pooling=pooling)
    w, gpu, ora = _pair(cfg, seed=49)
    gpu.set_option("parts", 1)
    rng = np.random.default_rng(49)
    seqs = [rng.integers(0, cfg.vocab, size=n, dtype=np.int32) for n in (2000, 1, 0, 1300)]
    got = gpu.encode_seqs(seqs)
    want = ora.encode_seqs(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    assert not got[2].any()
    gpu.close()


def test_panels_upload_equals_rows():
    """ixh_model_set_matrix with IXH_LAYOUT_PANELS (PackedB8.data, int8.go:30)
    gives the model uploaded by rows, bit for bit."""
    cfg = small_cfg(layers=2)
    w, gpu, ora = _pair(cfg, seed=42)
    rng = np.random.default_rng(42)
    seqs = ids_uniform_lengths(rng, 6, 1, 150, cfg.vocab)
    want = gpu.encode_tokens(seqs)
    L, h = gpu._L, gpu._h
    for l in range(cfg.layers):
        for which, q, s in ((_lib.MAT_QKV, w.wqkv_q, w.wqkv_s), (_lib.MAT_O, w.wo_q, w.wo_s),
                            (_lib.MAT_I, w.wi_q, w.wi_s), (_lib.MAT_OMLP, w.womlp_q, w.womlp_s)):
            p = orc.b8_to_panels(q[l])
            sc = np.ascontiguousarray(s[l], np.float32)
            _lib.check(L.ixh_model_set_matrix(h, l, which, p.ctypes.data, sc.ctypes.data,
                                              _lib.LAYOUT_PANELS))
    got = gpu.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    ref, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, ref), mismatch_report(got, ref)
    gpu.close()


@pytest.mark.parametrize("k,n", [(70, 40), (257, 19), (768, 2304), (1151, 33)])
def test_panels_packb8_equals_rows(k, n):
    """ixh_packb8_create from panels (k not a multiple of 4, n not one of
    16: padded quads and panels) equals the handle built from rows:
    quantised activations, reference tile and floats."""
    rng = np.random.default_rng(k * 7 + n)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    p = orc.b8_to_panels(q)
    assert p.size == ((n + 15) // 16) * ((k + 3) // 4) * 64
    br = linalg.PackedB8(q, s)
    bp = linalg.PackedB8(p, s, layout=_lib.LAYOUT_PANELS, k=k, n=n)
    a = rng.standard_normal((37, k)).astype(np.float32)
    r1, r2 = linalg.matmul8_tile(a, br), linalg.matmul8_tile(a, bp)
    for x, y in zip(r1, r2):
        assert np.array_equal(x, y)
    aq, _ = orc.quantize_rows(a)
    assert np.array_equal(r2[2], orc.matmul8_tile(aq, q))
    c0 = rng.standard_normal((37, n)).astype(np.float32)
    got = linalg.matmul8(c0.copy(), a, bp, 37, accumulate=True)
    colsum = q.astype(np.int32).sum(axis=1).astype(np.int32)
    ref = orc.matmul8(a, q, s, colsum, c=c0, accumulate=True)
    assert f32_bits_equal(got, ref), mismatch_report(got, ref)


def _ulp(t, sign):
    return np.nextafter(t, np.float32(np.inf) if sign > 0 else np.float32(-np.inf)).astype(np.float32)


def test_caller_rope_tables_used_past_512():
    """ixh_model_set_rope: the caller's tables are used as given (Go's own
    ropeFor bits), also for positions past 512. Tables whose entries are
    moved by one ulp (alternating up/down by position and dimension) give
    the oracle's result on the same tables for a 700-token sequence; grossly
    different tables change the result (they are read); a batch longer
    than the tables fails until longer ones are uploaded."""
    cfg = small_cfg(layers=3)
    w, gpu, ora = _pair(cfg, seed=43)
    D = cfg.head_dim()
    rows = 760
    tabs = []
    for theta in (cfg.global_theta, cfg.local_theta):
        c, s = orc.rope_table(theta, D, rows)
        sign = np.where((np.arange(rows)[:, None] + np.arange(D // 2)[None, :]) % 2 == 0, 1, -1)
        c = np.where(sign > 0, _ulp(c, 1), _ulp(c, -1)).astype(np.float32)
        s = np.where(sign > 0, _ulp(s, -1), _ulp(s, 1)).astype(np.float32)
        tabs.append((np.ascontiguousarray(c), np.ascontiguousarray(s)))
    rng = np.random.default_rng(43)
    seqs = [rng.integers(0, cfg.vocab, size=700, dtype=np.int32),
            rng.integers(0, cfg.vocab, size=90, dtype=np.int32)]
    default = gpu.encode_tokens(seqs)
    gpu.set_rope(True, *tabs[0])
    gpu.set_rope(False, *tabs[1])
    got = gpu.encode_tokens(seqs)
    ora.set_rope(tabs[0][0], tabs[0][1], tabs[1][0], tabs[1][1])
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    # the oracle's own tables give the library's default result
    ref = orc.OracleModel(w, lanes=8).encode_tokens(seqs)[0]
    assert f32_bits_equal(default, ref), mismatch_report(default, ref)
    # tables that differ grossly past 512 change the rows there: read, not rebuilt
    gross = [(np.ascontiguousarray(np.where(np.arange(rows)[:, None] >= 512, s, c)),
              np.ascontiguousarray(np.where(np.arange(rows)[:, None] >= 512, c, s))) for c, s in tabs]
    gpu.set_rope(True, *gross[0])
    gpu.set_rope(False, *gross[1])
    g2 = gpu.encode_tokens(seqs)
    # layer 0 is global: every row of the long sequence moves; the short
    # sequence (positions < 90) does not
    assert not np.array_equal(g2[:700], got[:700]) and f32_bits_equal(g2[700:], got[700:])
    # a batch longer than the caller's tables is refused, not silently rebuilt
    longer = [rng.integers(0, cfg.vocab, size=rows + 1, dtype=np.int32)]
    with pytest.raises(_lib.IxhError, match="RoPE table set by ixh_model_set_rope has 760 rows"):
        gpu.encode_tokens(longer)
    gpu.reset_rope(True)
    gpu.reset_rope(False)
    assert f32_bits_equal(gpu.encode_tokens(seqs), default)
    gpu.encode_tokens(longer)  # the library's own tables grow again
    gpu.close()


def test_batches_over_the_pass_size():
    """Option pass_tokens: a batch larger than it runs as passes of whole
    sequences (a sequence longer than it takes a pass alone); the results
    equal one pass's, through the host and the device entry points, and a
    sequence over 131072 tokens is refused before any work."""
    torch = pytest.importorskip("torch")
    cfg = small_cfg(layers=2)
    w, gpu, ora = _pair(cfg, seed=44)
    rng = np.random.default_rng(44)
    seqs = ids_uniform_lengths(rng, 30, 0, 300, cfg.vocab)
    seqs.insert(3, rng.integers(0, cfg.vocab, size=900, dtype=np.int32))
    one_t, one_p = gpu.encode_tokens(seqs), gpu.encode_seqs(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(one_t, want), mismatch_report(one_t, want)
    gpu.set_option("pass_tokens", 700)
    assert f32_bits_equal(gpu.encode_tokens(seqs), one_t)
    assert f32_bits_equal(gpu.encode_seqs(seqs), one_p)
    offs = np.zeros(len(seqs) + 1, np.int32)
    offs[1:] = np.cumsum([len(s) for s in seqs])
    ids = torch.from_numpy(np.concatenate(seqs).astype(np.int32)).to("cuda")
    for kind, rows, ref in ((_lib.OUT_TOKENS, int(offs[-1]), one_t), (_lib.OUT_POOLED, len(seqs), one_p)):
        out = torch.full((rows, cfg.hidden), 7.0, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        gpu.encode_device(ids.data_ptr(), offs, out.data_ptr(), kind, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert f32_bits_equal(out.cpu().numpy(), ref)
    with pytest.raises(_lib.IxhError, match="out of range"):
        gpu.set_option("pass_tokens", 131073)
    huge = [np.zeros(131073, np.int32)]
    with pytest.raises(_lib.IxhError, match="sequence of 131073 tokens over the 131072-token limit"):
        gpu.encode_seqs(huge)
    gpu.close()


def _decision_heads(cfg, rng):
    hc = heads.random_head(8, cfg.hidden, rng)
    hn = heads.random_head(1, cfg.hidden, rng)
    hs = heads.random_head(heads.span_tag_count(4), cfg.hidden, rng)
    bias = [rng.standard_normal(r).astype(np.float32) for r in (8, 1, 9)]
    return [(hc[0], bias[0], False), (hs[0], bias[2], True), (hn[0], bias[1], False)]


@pytest.mark.parametrize("pooling,mean", [("mean", False), ("cls", False), ("cls", True)])
def test_heads_on_device(pooling, mean):
    """ixh_encode_heads: a Choice-8 and a Noul head on the pooled row and a
    Spans head (9 labels) on every token, computed after final_norm on the
    device, equal head.logits (heads.go:63-74) of the oracle's pooled rows
    and states; mean=1 pools by the mean whatever the config (meanRows,
    spans.go:466-476); an empty sequence's pooled logits are the biases."""
    cfg = small_cfg(layers=2, pooling=pooling)
    w, gpu, ora = _pair(cfg, seed=45)
    rng = np.random.default_rng(45)
    hl = _decision_heads(cfg, rng)
    gpu.set_heads(hl)
    seqs = ids_uniform_lengths(rng, 24, 16, 256, cfg.vocab)
    seqs.insert(5, np.zeros(0, np.int32))
    zp, zt = gpu.encode_heads(seqs, mean=mean)
    states, offs = ora.encode_tokens(seqs)
    pooled = orc.pool(states, offs, cfg.hidden, cls=(pooling == "cls" and not mean))
    wp = np.concatenate([hl[0][0], hl[2][0]])
    bp = np.concatenate([hl[0][1], hl[2][1]])
    assert np.array_equal(zp, orc.head_logits(pooled, wp, bp))
    assert np.array_equal(zp[5], bp.astype(np.float64))
    assert np.array_equal(zt, orc.head_logits(states, hl[1][0], hl[1][1]))
    # the same with a pass size that cuts the batch
    gpu.set_option("pass_tokens", 1000)
    zp2, zt2 = gpu.encode_heads(seqs, mean=mean)
    assert np.array_equal(zp2, zp) and np.array_equal(zt2, zt)
    gpu.set_heads([])
    ids = np.concatenate(seqs).astype(np.int32)
    z = np.zeros((len(seqs), 16), np.float64)
    with pytest.raises(_lib.IxhError, match="no heads set"):
        _lib.check(gpu._L.ixh_encode_heads(gpu._h, ids.ctypes.data, offs.ctypes.data, len(seqs), 0,
                                           z.ctypes.data, None))
    gpu.close()


@pytest.mark.parametrize("hidden", [256, 768])
def test_head_logits_kernel_shapes(hidden):
    """head.logits (heads.go:63-74) on the device (ixh_head_logits): the
    float64 sums in column order for row counts within and past one
    workgroup's 12 rows (every shape of 2-4 waves of 1-3 rows), token
    counts around its 64 tokens, and rows with large, tiny and cancelling
    values, equal the oracle's bit for bit."""
    cfg = small_cfg(layers=1) if hidden == 256 else base_cfg(layers=1)
    w, gpu, _ = _pair(cfg, seed=48)
    rng = np.random.default_rng(48)
    for T, rows in ((1, 1), (63, 9), (64, 12), (65, 13), (1000, 30), (130, 4), (129, 2), (200, 3), (70, 5),
                    (257, 7), (4099, 9)):
        x = rng.standard_normal((T, hidden)).astype(np.float32)
        x[0, :8] = [3e38, -3e38, 1e-38, -1e-38, 1.0, -1.0, 65504.0, 1e-7]
        hw = (rng.standard_normal((rows, hidden)) * 0.02).astype(np.float32)
        hb = rng.standard_normal(rows).astype(np.float32)
        z = gpu.head_logits(x, hw, hb)
        assert np.array_equal(z, orc.head_logits(x, hw, hb)), (T, rows)
    gpu.close()


def test_cfg5_long_sequence_exact():
    """cfg5's length: one 8,192-token sequence and a short one at base width
    through 3 layers (global, local, local): the statistics kernel and 16
    prologue parts of 512 keys, 64 query blocks over 8,192 keys, the
    65,536-key-slot workspace; token states and the 9-label spans logits
    (EncodeTokens + the spans head, infer.go:484-518, spans.go:449-459) and
    the mean-pooled row equal the oracle's bit for bit."""
    cfg = base_cfg(layers=3)
    w, gpu, ora = _pair(cfg, seed=46)
    rng = np.random.default_rng(46)
    seqs = [rng.integers(0, cfg.vocab, size=8192, dtype=np.int32),
            rng.integers(0, cfg.vocab, size=77, dtype=np.int32)]
    hs = heads.random_head(heads.span_tag_count(4), cfg.hidden, rng)
    gpu.set_heads([(hs[0], hs[1], True)])
    _, zt = gpu.encode_heads(seqs, pooled=False)
    got = gpu.encode_tokens(seqs)
    pooled = gpu.encode_seqs(seqs)
    want, offs = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    assert np.array_equal(zt, orc.head_logits(want, hs[0], hs[1]))
    assert f32_bits_equal(pooled, orc.pool(want, offs, cfg.hidden))
    gpu.close()


def test_option_values_checked():
    cfg = small_cfg(layers=1)
    w, gpu, _ = _pair(cfg, seed=47)
    for name, bad in (("parts", 5), ("qkv_heads", 3), ("gemm", 3), ("gemm_tile", -1), ("pass_tokens", 0),
                      ("fuse_res", 5), ("fuse_mlp", 3), ("qkv_kblock", 2)):
        with pytest.raises(_lib.IxhError, match="out of range"):
            gpu.set_option(name, bad)
    gpu.set_option("parts", 2)
    assert gpu.option("parts") == 2
    gpu.close()


def test_bf16_exact_rows_later_wins():
    """A bf16 table whose exact rows name one id twice: the later row is
    read (newMappedEmbeddings fills a map in row order, embeddings.go:38-44),
    on the GPU as in the oracle."""
    from indecis_amd.modernbert import EMB_BF16
    cfg = small_cfg(layers=1)
    w = Weights.random(cfg, seed=48, emb_format=EMB_BF16)
    rng = np.random.default_rng(48)
    w.emb_exact_ids = np.array([5, 9, 5], np.int32)
    w.emb_exact_rows = rng.standard_normal((3, cfg.hidden)).astype(np.float32)
    gpu, ora = Model(w, lanes=8), orc.OracleModel(w, lanes=8)
    seqs = [np.array([5, 9, 5, 11], np.int32), rng.integers(0, cfg.vocab, size=30, dtype=np.int32)]
    got = gpu.encode_tokens(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    gpu.close()


def test_failed_allocation_is_a_clean_error():
    """A device allocation that cannot succeed — the embedding table of a
    model whose vocabulary needs more bytes than the GPU has — fails with the
    library's HIP error and message (nothing is launched, the host table is
    not read), and leaves nothing behind: encodes on a working model before
    and after it give the oracle's bits."""
    import dataclasses
    import torch
    cfg = small_cfg(layers=1)
    w, gpu, ora = _pair(cfg, seed=49)
    rng = np.random.default_rng(49)
    seqs = [rng.integers(0, cfg.vocab, size=n, dtype=np.int32) for n in (40, 7)]
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(gpu.encode_tokens(seqs), want)
    big = dataclasses.replace(cfg, vocab=700_000_000)
    need = 4 * big.vocab * big.hidden
    total = torch.cuda.get_device_properties(0).total_memory
    if need <= 2 * total:
        pytest.skip(f"the device holds {total} bytes: the table would fit")
    huge = Model(None, cfg=big, lanes=8)
    tiny = np.zeros(16, np.float32)  # never read: the allocation fails first
    with pytest.raises(_lib.IxhError, match="out of memory|hip:"):
        _lib.check(_lib.lib().ixh_model_set_embeddings_f32(huge._h, tiny.ctypes.data_as(C.c_void_p)))
    huge.close()
    assert f32_bits_equal(gpu.encode_tokens(seqs), want)
    gpu.close()
