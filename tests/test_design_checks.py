"""CPU checks behind design decisions that rest on the data rather than on
the reference: each computes, from committed code, the figure that decided
whether a kernel variant was worth building."""
import math

import numpy as np

import float_reference as fref
from indecis_amd.modernbert import BASE, Weights


def test_attention_tiles_skippable_by_p_zero():
    """Attention pass 2 could skip a (32-query, 32-key) tile whose every
    score has s - max < ln(0.5/255) = -6.2344 (P = RNE(255 exp(s - max)) is
    then 0 for all of them, exactly). On the benchmark's model (cfg4's
    random-init weights, seed 4) and its first sequences, layer 0 (global),
    scores in the float64 approximation (int8 rounding moves s by far less
    than the margin used): fewer than 1 in 1,000 tiles qualify, so the
    skip would cost its test on every tile and save almost nothing."""
    cfg = BASE
    w = Weights.random(cfg, seed=4)  # the weights bench.py's cfg4 uses
    rng = np.random.default_rng(20261201)  # bench.make_inputs' generator
    lens = rng.integers(64, 513, size=256)
    seqs = [rng.integers(0, cfg.vocab, size=int(n), dtype=np.int32) for n in lens][:6]
    H, nh = cfg.hidden, cfg.heads
    D = H // nh
    wq = w.wqkv_q[0].astype(np.float64) * w.wqkv_s[0][:, None]
    tiles = skippable = 0
    gaps = []
    for seq in seqs:
        n = len(seq)
        x = fref.layer_norm(w.emb_f32[seq].astype(np.float64), w.emb_norm.astype(np.float64), cfg.norm_eps)
        qkv = x @ wq.T
        c, s = fref.rope_tables(cfg.global_theta, D, n)
        for hd in range(nh):
            q = fref.apply_rope(qkv[:, hd * D:(hd + 1) * D], c, s)
            k = fref.apply_rope(qkv[:, H + hd * D:H + (hd + 1) * D], c, s)
            sc = (q @ k.T) / math.sqrt(D)
            sc = sc - sc.max(axis=1, keepdims=True)
            gaps.append(sc.ravel())
            for i0 in range(0, n, 32):
                for j0 in range(0, n, 32):
                    tiles += 1
                    skippable += bool((sc[i0:i0 + 32, j0:j0 + 32] < -6.3).all())
    p1 = float(np.percentile(np.concatenate(gaps), 1))
    print(f"tiles {tiles}, skippable {skippable}, 1st percentile of s - max {p1:.2f}")
    assert tiles > 2000
    assert skippable * 1000 < tiles
    assert p1 > -6.2344


def test_pass1_tile_bound_skips_few():
    """Attention pass 1 could skip a 32-key tile whose score bound
    f32(max acc * max ks) lies under the running maximum of every query of
    the wave (rounding is monotone, so the maximum stays exact). Simulated
    with Gaussian int8 queries and keys (D 64) and key scales varying by
    +-20%, tiles in key order as the kernel takes them, 32 queries a wave:
    about 0% of the tiles qualify at 512 keys, 5% at 2,048 and a third at
    8,192. The bound needs the tile's integer maximum (the MFMAs still run),
    so a skipped tile saves the conversion, scaling and maximum (about 40
    VALU instructions a lane a tile) while the bound and its wave-wide test
    cost about 12 on every tile: it breaks even near 30%."""
    rng = np.random.default_rng(7)
    D, Q = 64, 32
    share = {}
    for n in (512, 2048, 8192):
        q = np.clip(np.rint(rng.standard_normal((Q, D)) * 40), -127, 127).astype(np.int64)
        k = np.clip(np.rint(rng.standard_normal((n, D)) * 40), -127, 127).astype(np.int64)
        ks = (rng.uniform(0.8, 1.2, n) * 1e-3).astype(np.float32)
        acc = q @ k.T  # [Q][n]
        s = acc.astype(np.float32) * ks[None, :]
        run = np.full(Q, -np.inf, np.float32)
        skip = 0
        for t0 in range(0, n, 32):
            a = acc[:, t0:t0 + 32].max(axis=1).astype(np.float32)
            kmax, kmin = ks[t0:t0 + 32].max(), ks[t0:t0 + 32].min()
            bound = np.where(a >= 0, a * kmax, a * kmin)
            skip += bool((bound < run).all())
            run = np.maximum(run, s[:, t0:t0 + 32].max(axis=1))
        share[n] = skip / (n // 32)
    print(share)
    assert share[512] < 0.02 and share[2048] < 0.1 and share[8192] < 0.5
