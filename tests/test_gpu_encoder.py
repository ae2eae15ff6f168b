"""GPU parity of the whole int8 encoder (modernbert.run, infer.go:304-430)
against the CPU oracle, through the C ABI, on the BASELINE.json
configurations (reduced batches where the oracle would take minutes), plus
the reference's invariants at full size."""
import concurrent.futures as cf
import contextlib

import numpy as np
import pytest

from helpers import (base_cfg, bekko_cfg, f32_bits_equal, ids_cfg2, ids_uniform_lengths, mismatch_report,
                     small_cfg)
from indecis_amd import _lib, heads
from indecis_amd.modernbert import EMB_BF16, EMB_F32, EMB_I8, Model, Weights
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

_models = {}


@contextlib.contextmanager
def options(gpu, **kw):
    """Sets model options for a block, then restores them (the models are
    shared between tests)."""
    old = {k: gpu.option(k) for k in kw}
    try:
        for k, v in kw.items():
            gpu.set_option(k, v)
        yield
    finally:
        for k, v in old.items():
            gpu.set_option(k, v)


def model_pair(cfg, seed=0, emb_format=EMB_F32, lanes=8):
    key = (tuple(cfg.__dict__.values()), seed, emb_format, lanes)
    if key not in _models:
        w = Weights.random(cfg, seed=seed, emb_format=emb_format)
        _models[key] = (w, Model(w, lanes=lanes), orc.OracleModel(w, lanes=lanes))
    return _models[key]


def test_cfg2_pooled_and_heads():
    """cfg2: small encoder, 64 x 15 tokens, mean pooling, an 8-way choice
    head and a yes/no head."""
    cfg = small_cfg()
    w, gpu, ora = model_pair(cfg)
    rng = np.random.default_rng(2)
    seqs = ids_cfg2(rng)
    got = gpu.encode_seqs(seqs)
    want = ora.encode_seqs(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    hw, hb = heads.random_head(8, cfg.hidden, rng)
    nw, nb = heads.random_head(1, cfg.hidden, rng)
    z = gpu.head_logits(got, hw, hb)
    zr = orc.head_logits(want, hw, hb)
    assert np.array_equal(z, zr)
    p = heads.softmax(z)
    assert np.allclose(p.sum(axis=1), 1.0)
    zn = gpu.head_logits(got, nw, nb)
    assert np.array_equal(zn, orc.head_logits(want, nw, nb))


def test_cfg3_tokens_and_spans():
    """cfg3 (reduced batch): lengths U[16,256], token states and a 9-label
    spans head on every token; the padded Encode form equals EncodeSeqs."""
    cfg = small_cfg()
    w, gpu, ora = model_pair(cfg)
    rng = np.random.default_rng(3)
    seqs = ids_uniform_lengths(rng, 24, 16, 256, cfg.vocab)
    got = gpu.encode_tokens(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    sw, sb = heads.random_head(heads.span_tag_count(4), cfg.hidden, rng)
    assert np.array_equal(gpu.head_logits(got, sw, sb), orc.head_logits(want, sw, sb))
    T = 256
    ids = np.zeros(len(seqs) * T, np.int32)
    for i, s in enumerate(seqs):
        ids[i * T:i * T + len(s)] = s
    pooled = gpu.encode(ids, [len(s) for s in seqs], T)
    assert f32_bits_equal(pooled, ora.encode_seqs(seqs))


@pytest.mark.parametrize("emb_format", [EMB_BF16, EMB_I8])
def test_embedding_formats(emb_format):
    cfg = small_cfg(layers=2)
    w, gpu, ora = model_pair(cfg, seed=5, emb_format=emb_format)
    rng = np.random.default_rng(4)
    seqs = ids_uniform_lengths(rng, 6, 1, 40, cfg.vocab)
    if emb_format == EMB_BF16:
        seqs.append(np.asarray(w.emb_exact_ids, np.int32))  # exact rows used
    got = gpu.encode_tokens(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("lanes", [0, 4, 16])
def test_lanes_variants(lanes):
    cfg = small_cfg(layers=3)
    w, gpu, ora = model_pair(cfg, seed=6, lanes=lanes)
    rng = np.random.default_rng(lanes + 10)
    seqs = ids_uniform_lengths(rng, 5, 1, 200, cfg.vocab)
    got = gpu.encode_seqs(seqs)
    want = ora.encode_seqs(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)


def test_base_shape_exact():
    """The ModernBERT-base shape of cfg4 (H 768, 22 layers, 12 heads, I 1152)
    on a few sequences of lengths U[64, 512]."""
    cfg = base_cfg()
    w, gpu, ora = model_pair(cfg, seed=7)
    rng = np.random.default_rng(8)
    seqs = ids_uniform_lengths(rng, 3, 64, 512, cfg.vocab)
    got = gpu.encode_tokens(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)


def test_long_context_exact():
    """cfg5-style long sequence (global attention over 2,100 keys, local
    window elsewhere), base width with 4 layers (global, local, local,
    global)."""
    cfg = base_cfg(layers=4)
    w, gpu, ora = model_pair(cfg, seed=9)
    rng = np.random.default_rng(10)
    seqs = [rng.integers(0, cfg.vocab, size=2100, dtype=np.int32),
            rng.integers(0, cfg.vocab, size=333, dtype=np.int32)]
    got = gpu.encode_tokens(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)


def test_batch_equals_single():
    """A sequence's states do not depend on its batch (forward_test.go:141-160,
    TestMatMul8RowsIndependent)."""
    cfg = small_cfg()
    w, gpu, _ = model_pair(cfg)
    rng = np.random.default_rng(11)
    seqs = ids_uniform_lengths(rng, 40, 1, 300, cfg.vocab)
    allt = gpu.encode_tokens(seqs)
    off = 0
    for s in seqs[:8]:
        one = gpu.encode_tokens([s])
        assert f32_bits_equal(one, allt[off:off + len(s)])
        off += len(s)


def test_errors_and_empty():
    cfg = small_cfg(layers=1)
    w, gpu, _ = model_pair(cfg)
    with pytest.raises(_lib.IxhError, match="modernbert: id 40000 out of vocabulary"):
        gpu.encode_seqs([np.array([1, 40000, 2], np.int32)])
    with pytest.raises(_lib.IxhError, match="modernbert: id -1 out of vocabulary"):
        gpu.encode_seqs([np.array([-1], np.int32)])
    with pytest.raises(ValueError, match="inconsistent batch"):
        gpu.encode(np.zeros(5, np.int32), [2, 2], 2)
    out = gpu.encode_seqs([np.zeros(0, np.int32), np.array([3, 4], np.int32)])
    assert np.all(out[0] == 0) and np.any(out[1] != 0)
    assert gpu.encode_seqs([]).shape == (0, cfg.hidden)
    assert gpu.encode_tokens([np.zeros(0, np.int32)]).shape == (0, cfg.hidden)


def test_concurrent_inference():
    """TestConcurrentInference (concurrency_test.go:12-70): 8 threads on one
    model give the sequential results."""
    cfg = small_cfg(layers=2)
    w, gpu, _ = model_pair(cfg)
    rng = np.random.default_rng(12)
    batches = [ids_uniform_lengths(rng, 4, 1, 120, cfg.vocab) for _ in range(16)]
    want = [gpu.encode_seqs(b) for b in batches]
    with cf.ThreadPoolExecutor(8) as ex:
        got = list(ex.map(gpu.encode_seqs, batches))
    for g, wnt in zip(got, want):
        assert f32_bits_equal(g, wnt)


def test_invalidate_requires_upload():
    cfg = small_cfg(layers=1)
    w = Weights.random(cfg, seed=13)
    m = Model(w)
    seq = [np.array([5, 6, 7], np.int32)]
    before = m.encode_seqs(seq)
    m.invalidate()
    with pytest.raises(_lib.IxhError) as e:
        m.encode_seqs(seq)
    assert e.value.code == _lib.IXH_ESTATE
    m.upload(w)
    assert f32_bits_equal(m.encode_seqs(seq), before)
    m.close()


@pytest.mark.parametrize("longest", [512, 513, 1025])
def test_prologue_edge_lengths(longest):
    """Sequence lengths around the attention prologue's 32-key pieces and
    64-slot padding, with the longest at 512 (single-read prologue) or 513
    and 1025 (statistics kernel, then 512-key parts; the last part of the
    longest holds 1 key, and the short sequences of the batch have no
    second part)."""
    cfg = small_cfg()
    w, gpu, ora = model_pair(cfg, seed=11)
    rng = np.random.default_rng(longest)
    seqs = [rng.integers(0, cfg.vocab, size=n, dtype=np.int32)
            for n in (1, 31, 32, 33, 64, 65, 127, longest, 0, 2)]
    got = gpu.encode_tokens(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)


def test_unfused_qkv_path_exact():
    """Option qkv_fused 0: a batch of short sequences through the QKV GEMM
    (float32 K, V) and the separate attention prologue, the path every
    batch with a sequence over 512 keys takes, equals the oracle too."""
    cfg = small_cfg(layers=3)
    w, gpu, ora = model_pair(cfg, seed=23)
    rng = np.random.default_rng(23)
    seqs = [rng.integers(0, cfg.vocab, size=n, dtype=np.int32) for n in (1, 33, 64, 65, 300, 512, 0, 7)]
    with options(gpu, qkv_fused=0):
        got = gpu.encode_tokens(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("parts", [2, 3])
def test_split_streams_exact(parts):
    """A batch of at least 4,096 tokens runs as parts on as many streams
    (forward_split; option parts, default 2 here); token states and pooled
    output equal the oracle's, with an empty sequence last (a part of
    empty sequences only)."""
    cfg = small_cfg(layers=3)
    w, gpu, ora = model_pair(cfg, seed=21)
    rng = np.random.default_rng(21)
    seqs = ids_uniform_lengths(rng, 40, 64, 256, cfg.vocab) + [np.zeros(0, np.int32)]
    assert sum(len(s) for s in seqs) >= 4096
    with options(gpu, parts=parts):
        got = gpu.encode_tokens(seqs)
        pooled = gpu.encode_seqs(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    assert f32_bits_equal(pooled, ora.encode_seqs(seqs))


@pytest.mark.parametrize("nheads", [2, 1])
def test_qkv_heads_per_workgroup(nheads):
    """The fused QKV kernel with two heads a workgroup (option qkv_heads 2:
    1,024 threads, a 3-stage ring) and with one (the default), at lengths
    around its 32-row blocks and the 256-row slab, up to 512."""
    cfg = base_cfg(layers=2)
    w, gpu, ora = model_pair(cfg, seed=31)
    rng = np.random.default_rng(31)
    seqs = [rng.integers(0, cfg.vocab, size=n, dtype=np.int32)
            for n in (1, 31, 32, 33, 255, 256, 257, 300, 511, 512, 0, 64)]
    with options(gpu, qkv_heads=nheads):
        got = gpu.encode_tokens(seqs)
        pooled = gpu.encode_seqs(seqs)
    want, _ = ora.encode_tokens(seqs)
    assert f32_bits_equal(got, want), mismatch_report(got, want)
    assert f32_bits_equal(pooled, ora.encode_seqs(seqs))


@pytest.mark.parametrize("shape,lanes", [("small", 0), ("small", 4), ("small", 8), ("small", 16),
                                         ("base", 8), ("base", 16), ("base", 0), ("bekko", 8), ("bekko", 0)])
def test_fused_residual_gemms(shape, lanes):
    """Option fuse_res: Wo and WoMLP fused with quantizeA of their input rows
    and the next LayerNorm + quantizeA (gemm_res.hip), the input quantised
    into a whole-row panel first (1, the default) or streamed in the K
    loop from the producers' row maxima (2: Wo's, from attention's maxima
    per head; 3: also WoMLP's, from the GeGLU epilogue's maxima per 32
    columns), or Wo on the 8-wave whole-row kernel (4, mlp_res.hip), with
    and without the MLP kernel, give the separate kernels' bits (0) and the
    oracle's, for
    every lane width of the LayerNorm chains, at the three model widths
    (at hidden 384 the 8-wave Wo kernel does not apply: option 4 takes the
    panel kernel), with row counts that leave a partial 32-row block and a
    last layer without LayerNorm; also with Wi on gemm_i8 (option gemm 1:
    no GeGLU maxima, so WoMLP takes the panel while Wo streams)."""
    cfg = _shape_cfg(shape, 3 if shape == "small" else 2)
    w, gpu, ora = model_pair(cfg, seed=71, lanes=lanes)
    rng = np.random.default_rng(71 + lanes)
    seqs = ids_uniform_lengths(rng, 7, 1, 300, cfg.vocab)
    if sum(len(s) for s in seqs) % 32 == 0:
        seqs.append(rng.integers(0, cfg.vocab, size=5, dtype=np.int32))
    want, _ = ora.encode_tokens(seqs)
    for mode, gemm, mlp in ((1, 0, 1), (1, 0, 0), (2, 0, 0), (3, 0, 0), (0, 0, 0), (3, 1, 0), (2, 0, 1),
                            (4, 0, 1), (4, 0, 0), (1, 0, 2), (0, 0, 2), (4, 0, 2)):
        with options(gpu, fuse_res=mode, gemm=gemm, fuse_mlp=mlp):
            got = gpu.encode_tokens(seqs)
        assert f32_bits_equal(got, want), (mode, gemm, mlp, mismatch_report(got, want))


def _shape_cfg(shape, layers):
    return {"small": small_cfg, "base": base_cfg, "bekko": bekko_cfg}[shape](layers=layers)


@pytest.mark.parametrize("shape,kernel", [("small", 1), ("base", 1), ("small", 2), ("base", 2),
                                          ("bekko", 2)])
def test_fused_mlp_block_rows(shape, kernel):
    """Option fuse_mlp: the MLP block as one kernel (Wi, GeGLU, quantizeA
    of g, WoMLP, the next LayerNorm + quantizeA), one workgroup per 32 rows
    (1, mlp_res.hip) or per 64 rows with transposed products (2,
    mlp_block.hip), gives the oracle's bits at row counts below, at and
    around its row blocks, and equals the separate kernels (fuse_mlp 0) on
    a batch of 4,000 rows."""
    cfg = _shape_cfg(shape, 2)
    w, gpu, ora = model_pair(cfg, seed=73, lanes=8)
    rng = np.random.default_rng(73)
    with options(gpu, fuse_mlp=kernel):
        for n in (1, 31, 32, 33, 63, 64, 65, 97, 128, 129):
            seqs = [rng.integers(0, cfg.vocab, size=n, dtype=np.int32)]
            got = gpu.encode_tokens(seqs)
            want, _ = ora.encode_tokens(seqs)
            assert f32_bits_equal(got, want), (n, mismatch_report(got, want))
        seqs = ids_uniform_lengths(rng, 16, 150, 350, cfg.vocab)
        fused = gpu.encode_tokens(seqs)
    with options(gpu, fuse_mlp=0):
        separate = gpu.encode_tokens(seqs)
    assert f32_bits_equal(fused, separate), mismatch_report(fused, separate)


@pytest.mark.parametrize("lanes", [0, 4, 8, 16])
def test_mlp_block_lanes(lanes):
    """The 64-row MLP kernel (fuse_mlp 2) for every lane width of the
    LayerNorm chains (float32 lane partials in two column stages at hidden
    768, or one float64 chain a row), and the last layer without
    LayerNorm, against the oracle, at both model widths of BASELINE.json."""
    for shape, layers in (("small", 3), ("base", 2)):
        cfg = _shape_cfg(shape, layers)
        w, gpu, ora = model_pair(cfg, seed=79, lanes=lanes)
        rng = np.random.default_rng(79 + lanes)
        seqs = ids_uniform_lengths(rng, 9, 1, 300, cfg.vocab)
        want, _ = ora.encode_tokens(seqs)
        with options(gpu, fuse_mlp=2):
            got = gpu.encode_tokens(seqs)
        assert f32_bits_equal(got, want), (shape, mismatch_report(got, want))


@pytest.mark.parametrize("which", ["wi", "womlp", "wqkv", "wo"])
def test_deq_bound_fallback(which):
    """A weight row past the dequantisation bound (127 * sum|w| + |128 *
    colsum| >= 2^24: a row of 127s) makes the kernels that dequantise as
    f32(acc) * sb * sa take the reference's order for that matrix (the
    64-row MLP kernel hands the block to the exact kernels; the fused QKV
    and Wo kernels switch their epilogue); the result is the oracle's
    either way."""
    for shape in ("small", "base"):
        cfg = _shape_cfg(shape, 2)
        w = Weights.random(cfg, seed=89)
        m = {"wi": w.wi_q, "womlp": w.womlp_q, "wqkv": w.wqkv_q, "wo": w.wo_q}[which]
        m[0, 3, :] = 127
        gpu, ora = Model(w, lanes=8), orc.OracleModel(w, lanes=8)
        rng = np.random.default_rng(89)
        seqs = ids_uniform_lengths(rng, 6, 1, 200, cfg.vocab)
        want, _ = ora.encode_tokens(seqs)
        for mlp in (2, 1):
            with options(gpu, fuse_mlp=mlp):
                got = gpu.encode_tokens(seqs)
            assert f32_bits_equal(got, want), (shape, mlp, mismatch_report(got, want))
        gpu.close()


@pytest.mark.parametrize("lanes", [8, 16])
def test_bekko_width_exact(lanes):
    """The reference's own backbone width (bekko a8m: hidden 384, 6 heads,
    MLP 2 x 1152; linalg/gemm_test.go:104-105) through the whole encoder,
    with the fused kernels on (the 64-row MLP kernel, the fused QKV and
    residual kernels, the LayerNorm segment kernel with a 128-column
    segment) and off, pooled and per token, against the oracle."""
    cfg = bekko_cfg(layers=3)
    w, gpu, ora = model_pair(cfg, seed=83, lanes=lanes)
    rng = np.random.default_rng(83)
    seqs = ids_uniform_lengths(rng, 12, 1, 400, cfg.vocab)
    want, _ = ora.encode_tokens(seqs)
    for mlp, res, qkv, seg in ((2, 1, 1, 1), (0, 0, 0, 1), (2, 0, 0, 1), (1, 1, 1, 1), (2, 1, 1, 0)):
        with options(gpu, fuse_mlp=mlp, fuse_res=res, qkv_fused=qkv, ln_seg=seg):
            got = gpu.encode_tokens(seqs)
            pooled = gpu.encode_seqs(seqs)
        assert f32_bits_equal(got, want), ((mlp, res, qkv, seg), mismatch_report(got, want))
        assert f32_bits_equal(pooled, ora.encode_seqs(seqs)), (mlp, res, qkv, seg)


@pytest.mark.parametrize("shape", ["small", "base"])
def test_qkv_kblock_input_exact(shape):
    """Option qkv_kblock: the fused QKV kernel reading its input rows
    K-blocked ([K/32][N][32], written so by the MLP kernel and by the
    embedding LayerNorm) with the head's weight rows resident in LDS gives
    the oracle's bits, in one part and in two, and so does the row-major
    ring (qkv_kblock 0)."""
    cfg = small_cfg(layers=3) if shape == "small" else base_cfg(layers=2)
    w, gpu, ora = model_pair(cfg, seed=77, lanes=8)
    rng = np.random.default_rng(77)
    seqs = ids_uniform_lengths(rng, 24, 1, 512, cfg.vocab)
    want, _ = ora.encode_tokens(seqs)
    for kb, parts in ((1, 1), (1, 2), (0, 1)):
        with options(gpu, qkv_kblock=kb, parts=parts):
            got = gpu.encode_tokens(seqs)
        assert f32_bits_equal(got, want), (kb, parts, mismatch_report(got, want))
    # the edges of the row blocks (32 rows, one or two a wave: 256), of the
    # K mean's read batches (16 rows, taken two at a time) and of the fused
    # kernel's limit (512 keys)
    edges = [rng.integers(0, cfg.vocab, size=n, dtype=np.int32)
             for n in (1, 15, 16, 17, 31, 32, 33, 47, 48, 49, 255, 256, 257, 271, 272, 273, 288,
                       303, 511, 512)]
    want, _ = ora.encode_tokens(edges)
    with options(gpu, qkv_kblock=1, parts=1):
        got = gpu.encode_tokens(edges)
    assert f32_bits_equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("lanes", [8, 16])
def test_ln_whole_row_kernel(lanes):
    """Option ln_seg 0: the row LayerNorms of lane widths 8 and 16 (the
    embedding one, which also writes the QKV input K-blocked, and the final
    one) on the whole-row LDS kernel instead of the segment kernel give the
    oracle's bits, with the K-blocked QKV input and without it."""
    cfg = small_cfg(layers=2)
    w, gpu, ora = model_pair(cfg, seed=9, lanes=lanes)
    rng = np.random.default_rng(90 + lanes)
    seqs = ids_uniform_lengths(rng, 6, 1, 300, cfg.vocab)
    want, _ = ora.encode_tokens(seqs)
    for kb in (1, 0):
        with options(gpu, ln_seg=0, qkv_kblock=kb):
            got = gpu.encode_tokens(seqs)
        assert f32_bits_equal(got, want), (kb, mismatch_report(got, want))
