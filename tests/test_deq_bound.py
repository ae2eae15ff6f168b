"""The dequantisation shortcut of the 64-row MLP kernel (mlp_block.hip):
for a weight row with 127 * sum|w| + |128 * colsum| < 2^24, the
reference's f32(acc + 128*colsum) - zc (kernel_vnni_amd64.s:144-200,
int8.go:72-75: zc = 128 * f32(colsum)) equals f32(acc) for every int8
activation row, because the tile is then exact in float32 and so is its
difference with zc. Past the bound it does not hold, which is why the host
checks the bound on upload (Mat::small) and runs the exact kernels for
such weights."""
import numpy as np


def ref_minus_zc(acc, colsum):
    tile = acc + 128 * colsum
    zc = np.float32(128) * colsum.astype(np.float32)
    return tile.astype(np.float32) - zc


def bound(w):
    return 127 * np.abs(w.astype(np.int64)).sum(axis=1) + 128 * np.abs(w.astype(np.int64).sum(axis=1))


def test_shortcut_exact_within_bound():
    rng = np.random.default_rng(5)
    for k in (256, 768, 1152):
        w = rng.integers(-127, 128, size=(64, k), dtype=np.int8)
        assert (bound(w) < 1 << 24).all()
        colsum = w.astype(np.int64).sum(axis=1)
        for a in (rng.integers(-127, 128, size=(256, k)), np.full((1, k), 127), np.full((1, k), -127),
                  np.sign(w[:1]).astype(np.int64) * 127, -np.sign(w[:1]).astype(np.int64) * 127):
            acc = a.astype(np.int64) @ w.astype(np.int64).T
            got = acc.astype(np.float32)
            want = ref_minus_zc(acc, colsum[None, :])
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_shortcut_fails_past_bound():
    """A row of equal weights near 127 breaks the bound, and an activation
    row aligned with it gives a tile past 2^24 that float32 rounds: the
    shortcut would then change the result (a planted use of it is caught)."""
    k = 768
    w = np.full((1, k), 127, np.int8)
    w[0, 0] = 126
    assert bound(w)[0] >= 1 << 24
    colsum = w.astype(np.int64).sum(axis=1)
    a = np.full((1, k), 127, np.int64)
    a[0, :5] = 126
    acc = a @ w.astype(np.int64).T
    assert (acc + 128 * colsum)[0, 0] > 1 << 24
    assert (acc + 128 * colsum)[0, 0] % 2 == 1  # odd past 2^24: not exact in float32
    got = acc.astype(np.float32)
    want = ref_minus_zc(acc, colsum[None, :])
    assert not np.array_equal(got, want)
