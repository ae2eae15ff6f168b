"""GPU parity of the linalg-level kernels against the CPU oracle, through
the C ABI: quantised activations and int32 accumulators bit-exact, float
outputs bit-exact (the kernels reproduce the reference's roundings)."""
import numpy as np
import pytest

from helpers import f32_bits_equal, ids_uniform_lengths, mismatch_report, small_cfg
from indecis_amd import linalg
from indecis_amd.modernbert import Model, Weights
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _weights(rng, n, k, kind="random"):
    if kind == "max":
        q = np.full((n, k), 127, np.int8)
    elif kind == "mixed":
        q = np.where((np.arange(n * k).reshape(n, k) // 3) % 2 == 0, -127, 127).astype(np.int8)
    else:
        q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    return q, s


def test_cfg1_fused_op():
    """BASELINE cfg1: X [256x256] N(0,1), gamma U(0.9,1.1), LN eps 1e-5,
    per-row quantisation, W int8 [256 x 1024] U[-127,127], scales
    U(1e-3,1e-2), dequant + GeGLU (GELU on the first 512, infer.go:418)."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((256, 256)).astype(np.float32)
    gamma = rng.uniform(0.9, 1.1, 256).astype(np.float32)
    q, s = _weights(rng, 1024, 256)
    b = linalg.PackedB8(q, s)
    for lanes in (8, 16, 0):
        xn_ref = orc.layernorm_rows(x, gamma, 1e-5, lanes)
        aq_ref, sa_ref = orc.quantize_rows(xn_ref)
        tile_ref = orc.matmul8_tile(aq_ref, q)
        colsum = q.astype(np.int32).sum(axis=1).astype(np.int32)
        z_ref = orc.matmul8_deq(aq_ref, sa_ref, q, s, colsum)
        g_ref = orc.gelu_mul(z_ref[:, :512], z_ref[:, 512:], lanes)
        out, aq, sa = linalg.layernorm_quant(x, gamma, 1e-5, lanes)
        assert f32_bits_equal(out, xn_ref), mismatch_report(out, xn_ref)
        assert np.array_equal(aq, aq_ref)
        assert f32_bits_equal(sa, sa_ref)
        g, tile = linalg.ln_matmul8_geglu(x, gamma, b, 1e-5, lanes)
        assert np.array_equal(tile, tile_ref)
        assert f32_bits_equal(g, g_ref), mismatch_report(g, g_ref)


@pytest.mark.parametrize("kind", ["random", "max", "mixed"])
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (6, 4, 16), (7, 384, 1152), (15, 1152, 384),
                                   (33, 301, 17), (130, 768, 2304), (257, 70, 40)])
def test_matmul8_tile_exact(m, k, n, kind):
    """microKernel8 == microKernel8Go (kernel_test.go:76-95): the GPU's
    reference tile and quantised activations equal the oracle's."""
    rng = np.random.default_rng(m * 7919 + k * 31 + n)
    a = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    if kind == "max":
        a[:] = np.abs(a) + 1
    q, s = _weights(rng, n, k, kind)
    b = linalg.PackedB8(q, s)
    aq, sa, tile = linalg.matmul8_tile(a, b)
    aq_ref, sa_ref = orc.quantize_rows(a)
    assert np.array_equal(aq, aq_ref)
    assert f32_bits_equal(sa, sa_ref)
    assert np.array_equal(tile, orc.matmul8_tile(aq_ref, q))


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("m,k,n", [(1, 64, 128), (13, 70, 40), (100, 768, 768), (300, 1152, 768)])
def test_matmul8_float_exact(m, k, n, accumulate):
    """MatMul8N: c (+)= ((f32(tile) - zc)*sb)*sa bit for bit."""
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    a[min(2, m - 1)] = 0.0  # a zero row: scale 0
    q, s = _weights(rng, n, k)
    b = linalg.PackedB8(q, s)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    colsum = q.astype(np.int32).sum(axis=1).astype(np.int32)
    ref = orc.matmul8(a, q, s, colsum, c=c0, accumulate=accumulate)
    c = c0.copy()
    linalg.matmul8(c, a, b, m, accumulate)
    assert f32_bits_equal(c, ref), mismatch_report(c, ref)


def test_matmul8_rows_independent():
    """TestMatMul8RowsIndependent (int8_test.go:149-171)."""
    rng = np.random.default_rng(3)
    m, k, n = 13, 70, 40
    a = rng.standard_normal((m, k)).astype(np.float32)
    q, s = _weights(rng, n, k)
    b = linalg.PackedB8(q, s)
    allc = np.zeros((m, n), np.float32)
    linalg.matmul8(allc, a, b, m)
    for i in range(m):
        one = np.zeros((1, n), np.float32)
        linalg.matmul8(one, a[i:i + 1].copy(), b, 1)
        assert f32_bits_equal(one[0], allc[i])


@pytest.mark.parametrize("lanes", [0, 4, 8, 16])
@pytest.mark.parametrize("m,h", [(1, 4), (7, 36), (64, 256), (33, 384), (300, 768), (5, 1152)])
def test_layernorm_quant_exact(m, h, lanes):
    rng = np.random.default_rng(m * h + lanes)
    x = (rng.standard_normal((m, h)) * 3 + 0.5).astype(np.float32)
    gamma = rng.uniform(0.9, 1.1, h).astype(np.float32)
    ref = orc.layernorm_rows(x, gamma, 1e-5, lanes)
    q_ref, sa_ref = orc.quantize_rows(ref)
    out, q, sa = linalg.layernorm_quant(x, gamma, 1e-5, lanes)
    assert f32_bits_equal(out, ref), mismatch_report(out, ref)
    assert np.array_equal(q, q_ref)
    assert f32_bits_equal(sa, sa_ref)


@pytest.mark.parametrize("lanes", [8, 16, 0])
@pytest.mark.parametrize("window", [-1, 8, 64])
@pytest.mark.parametrize("n", [1, 5, 17, 48, 100, 259, 300, 600, 1025, 2600])
def test_attend8_exact(n, window, lanes):
    """Attend8 on the GPU == the oracle's restatement, bit for bit, with the
    inputs of TestAttend8 (attention8_test.go:50-68)."""
    rng = np.random.default_rng(n * 100 + window + 7 * lanes)
    D = 64
    q = (rng.standard_normal((n, D)) * 2).astype(np.float32)
    k = (rng.standard_normal((n, D)) * 2).astype(np.float32) + (np.arange(n * D) % D % 7).reshape(n, D).astype(np.float32)
    v = rng.standard_normal((n, D)).astype(np.float32)
    ref = orc.attend8(q, k, v, window, 0.125, lanes)
    o = linalg.attend8(q, k, v, window, 0.125, lanes)
    assert f32_bits_equal(o, ref), mismatch_report(o, ref)


@pytest.mark.parametrize("lanes", [8, 0])
@pytest.mark.parametrize("window", [100, 300])
@pytest.mark.parametrize("n", [300, 1025])
def test_attend8_wide_window_exact(n, window, lanes):
    """Sliding windows wider than 64 keys a side: a workgroup's 128 queries
    then need more than one staged chunk of 256 keys, so pass 2 stages K
    and V again chunk by chunk (a path the encoder's window of 64 keys a
    side never takes). Bit for bit against the oracle."""
    rng = np.random.default_rng(n * 100 + window + 7 * lanes + 1)
    D = 64
    q = (rng.standard_normal((n, D)) * 2).astype(np.float32)
    k = (rng.standard_normal((n, D)) * 2).astype(np.float32) + (np.arange(n * D) % D % 7).reshape(n, D).astype(np.float32)
    v = rng.standard_normal((n, D)).astype(np.float32)
    ref = orc.attend8(q, k, v, window, 0.125, lanes)
    o = linalg.attend8(q, k, v, window, 0.125, lanes)
    assert f32_bits_equal(o, ref), mismatch_report(o, ref)


@pytest.mark.parametrize("tile_cfg", [0, 1, 2])
def test_gemm_tile_configs(tile_cfg):
    """The gemm_i8 kernel alone (option gemm 1) in its default 128x128 and
    its 256x128 / 3-stage and 128x128 / 3-stage tile configurations
    (option gemm_tile) gives the oracle's reference tile and floats, on
    ragged shapes that leave partial M tiles and padded N and K."""
    rng = np.random.default_rng(tile_cfg)
    for m, k, n in [(7, 384, 1152), (257, 70, 40), (300, 1152, 768), (1000, 768, 2304)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        q, s = _weights(rng, n, k)
        b = linalg.PackedB8(q, s)
        b.set_option("gemm", 1)
        b.set_option("gemm_tile", tile_cfg)
        aq, sa, tile = linalg.matmul8_tile(a, b)
        aq_ref, sa_ref = orc.quantize_rows(a)
        assert np.array_equal(tile, orc.matmul8_tile(aq_ref, q))
        c0 = rng.standard_normal((m, n)).astype(np.float32)
        colsum = q.astype(np.int32).sum(axis=1).astype(np.int32)
        ref = orc.matmul8(a, q, s, colsum, c=c0, accumulate=True)
        got = linalg.matmul8(c0.copy(), a, b, m, accumulate=True)
        assert f32_bits_equal(got, ref), mismatch_report(got, ref)
    # the whole encoder (RoPE/Q-quant, GeGLU and residual epilogues)
    cfg = small_cfg()
    w = Weights.random(cfg, seed=5)
    gpu, ora = Model(w, lanes=8), orc.OracleModel(w, lanes=8)
    gpu.set_option("gemm", 1)
    gpu.set_option("gemm_tile", tile_cfg)
    seqs = ids_uniform_lengths(rng, 5, 1, 300, cfg.vocab)
    got = gpu.encode_tokens(seqs)
    want, _ = ora.encode_tokens(seqs)
    gpu.close()
    assert f32_bits_equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("kind", ["random", "max", "mixed"])
@pytest.mark.parametrize("m,k,n", [(1, 768, 256), (63, 256, 768), (65, 512, 1000), (130, 256, 1024),
                                   (1000, 768, 2304), (3001, 1152, 768)])
def test_gemm_as_exact(m, k, n, kind):
    """The A-stationary GEMM (gemm_as.hip: the default wherever K is 256,
    512, 768 or 1152) gives the oracle's reference tile and floats, stored
    and accumulated: partial 64-row M-blocks, N padded to 256, runs of
    units that cross M-blocks, the largest tiles (all weights 127)."""
    rng = np.random.default_rng(m * 13 + k + n)
    a = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    if kind == "max":
        a[:] = np.abs(a) + 1
    q, s = _weights(rng, n, k, kind)
    b = linalg.PackedB8(q, s)
    aq, sa, tile = linalg.matmul8_tile(a, b)
    aq_ref, sa_ref = orc.quantize_rows(a)
    assert np.array_equal(aq, aq_ref)
    assert np.array_equal(tile, orc.matmul8_tile(aq_ref, q))
    colsum = q.astype(np.int32).sum(axis=1).astype(np.int32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    for acc in (False, True):
        ref = orc.matmul8(a, q, s, colsum, c=c0, accumulate=acc)
        got = linalg.matmul8(c0.copy(), a, b, m, accumulate=acc)
        assert f32_bits_equal(got, ref), mismatch_report(got, ref)


@pytest.mark.parametrize("gemm", [1, 2])
def test_encoder_gemm_kernel_choices(gemm):
    """Option gemm: the whole encoder on gemm_i8 alone (1: Wi + GeGLU and
    the residual GEMMs included), or with the warp-specialised kernel for
    the residual GEMMs (2), equals the oracle too."""
    cfg = small_cfg()
    w = Weights.random(cfg, seed=9)
    gpu, ora = Model(w, lanes=8), orc.OracleModel(w, lanes=8)
    gpu.set_option("gemm", gemm)
    rng = np.random.default_rng(9)
    seqs = ids_uniform_lengths(rng, 5, 1, 300, cfg.vocab)
    got = gpu.encode_tokens(seqs)
    want, _ = ora.encode_tokens(seqs)
    gpu.close()
    assert f32_bits_equal(got, want), mismatch_report(got, want)


@pytest.mark.parametrize("kind", ["random", "max"])
@pytest.mark.parametrize("m,k,n", [(1, 768, 256), (64, 256, 256), (65, 512, 768), (700, 1152, 768),
                                   (3001, 768, 768), (4100, 1152, 768)])
def test_gemm_ws_accumulate_exact(m, k, n, kind):
    """The warp-specialised GEMM (gemm_ws.hip, option gemm 2: MatMul8N with
    accumulate, int8.go:89-155, as the residual GEMMs run it) adds the oracle's
    floats to C bit for bit: partial 64-row M-blocks, one-row inputs, runs
    of units that cross M-blocks, all weights 127. Each shape runs three
    times on the same inputs: the MFMA and epilogue waves hand blocks over
    through LDS, and every call must give the same bits."""
    rng = np.random.default_rng(m * 17 + k + 3 * n)
    a = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    if kind == "max":
        a[:] = np.abs(a) + 1
    q, s = _weights(rng, n, k, kind)
    b = linalg.PackedB8(q, s)
    b.set_option("gemm", 2)
    colsum = q.astype(np.int32).sum(axis=1).astype(np.int32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    ref = orc.matmul8(a, q, s, colsum, c=c0, accumulate=True)
    for _ in range(3):
        got = linalg.matmul8(c0.copy(), a, b, m, accumulate=True)
        assert f32_bits_equal(got, ref), mismatch_report(got, ref)


def _outlier_inputs(case, rng):
    if case == "reference":  # TestMatMul8Outliers (int8_test.go:98-118)
        m, k, n = 64, 3072, 96
        a = rng.standard_normal((m, k)).astype(np.float32)
        a[:, 1038] = 1000 * rng.standard_normal(m).astype(np.float32)
        a[:, 7] = 150
        b = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
        q, s, cs = orc.pack_b8(b, k, n, transB=False)
        return a, q, s, cs
    m, k, n = {"many": (33, 1000, 300), "ties": (9, 1000, 40), "none": (70, 768, 256),
               "large": (3000, 768, 768), "one_row": (1, 1152, 768)}[case]
    a = rng.standard_normal((m, k)).astype(np.float32)
    if case == "many":
        for j in rng.choice(k, 45, replace=False):
            a[:, j] *= float(rng.uniform(400, 2000))
    elif case == "ties":
        for j in range(40):
            a[:, 3 * j] = 5000.0 * np.sign(a[:, 3 * j] + 1e-3)
        a[0, [1, 4, 7, 10, 13]] = [8000, 7000, 8000, 6000, 7500]
    elif case in ("large", "one_row"):
        a[:, [5, 300, 700]] *= 250
    q, s, cs = orc.pack_b8(rng.standard_normal((n, k)).astype(np.float32), k, n)
    return a, q, s, cs


@pytest.mark.parametrize("case", ["reference", "many", "ties", "none", "large", "one_row"])
def test_matmul8_outliers_exact(case):
    """MatMul8Outliers on the GPU (column maxima, the host's channel choice,
    the int8 product of the zeroed copy, the float32 adds of the split
    channels) equals the oracle bit for bit, stored and accumulated; with
    no channel over the bar it is MatMul8N's result."""
    rng = np.random.default_rng(["reference", "many", "ties", "none", "large", "one_row"].index(case) + 3)
    a, q, s, cs = _outlier_inputs(case, rng)
    m, n = a.shape[0], q.shape[0]
    b = linalg.PackedB8(q, s)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    for acc in (False, True):
        want, cols = orc.matmul8_outliers(a, q, s, cs, 6.0, c=c0, accumulate=acc)
        got = linalg.matmul8_outliers(c0.copy(), a, b, m, accumulate=acc, ratio=6.0)
        assert f32_bits_equal(got, want), mismatch_report(got, want)
    if case == "none":
        assert len(cols) == 0
        plain = linalg.matmul8(c0.copy(), a, b, m, accumulate=True)
        assert f32_bits_equal(got, plain)
    elif case in ("many", "ties"):
        assert len(cols) == 32


@pytest.mark.parametrize("outliers", [False, True])
@pytest.mark.parametrize("with_bias", [False, True])
def test_linear8_exact(outliers, with_bias):
    """siglip linear.apply (encoder.go:36-49) on the GPU: the product (split
    or not), then the bias, equal to the oracle bit for bit."""
    rng = np.random.default_rng(10 + outliers + 2 * with_bias)
    rows, k, n = 729, 768, 3072  # SigLIP-base fc1 over one image's 27x27 patches
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[:, [11, 400]] *= 300
    q, s, cs = orc.pack_b8(rng.standard_normal((n, k)).astype(np.float32), k, n)
    bias = rng.standard_normal(n).astype(np.float32) if with_bias else None
    want = orc.linear8(x, q, s, cs, bias, outliers, 6.0)
    got = linalg.linear8(x, linalg.PackedB8(q, s), bias, outliers, 6.0)
    assert f32_bits_equal(got, want), mismatch_report(got, want)


def test_exp255_shortcut_every_float():
    """The attention kernels round 255*exp(v) from the hardware exponential
    and fall back to the reference formulas (ExpShift's vector body and
    exp32, vec_simd.go:235-262) only near a rounding boundary. Over every
    float v <= 0 the shortcut must never round differently from either
    formula; its distance from them stays below the margin (2^-13, the
    kernels' kExp255Tol; measured 7.63e-5)."""
    bad_v, bad_s, err_v, err_s, undecided = linalg.check_exp255()
    assert bad_v == 0 and bad_s == 0, (bad_v, bad_s)
    assert err_v < 2.0 ** -13 and err_s < 2.0 ** -13, (err_v, err_s)
    print(f"max |fast - ref|: simd {err_v:.3g}, scalar {err_s:.3g}; undecided floats {undecided}")


def test_gelu_division_every_float():
    """The kernels' GELU divides with the hardware reciprocal and one
    exact-remainder FMA correction (Markstein's method, one step) and clamps
    with v_med3 instead of IEEE division and compare-select. Over all 2^32
    float inputs both GELU forms (geluMulAVX2's FMA form, geluScalar;
    gelu_amd64.s:173-195, fastmath.go:9-26) must give the IEEE-division
    result in every bit."""
    bad_fma, bad_scalar = linalg.check_gelu()
    assert bad_fma == 0 and bad_scalar == 0, (bad_fma, bad_scalar)


def test_mfma_rate_check():
    """ixh_check_mfma_rate: int8 MFMAs issued back to back from registers
    run at a sizeable fraction of the 5.0e15 dense peak, never above it."""
    r = linalg.check_mfma_rate(0, iters=20000)
    assert 0.2 * 5.0e15 < r < 1.05 * 5.0e15, r
