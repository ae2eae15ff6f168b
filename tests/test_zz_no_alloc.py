"""ixh_matmul8_noalloc (MatMul8N on device buffers, no allocation: the
quantised activations go to the library's fixed per-GPU scratch) against
ixh_matmul8 (MatMul8N, int8.go:89-155, on host buffers) bit for bit,
through the C ABI: two calls in a row, the second with fewer rows (the
scratch keeps the first call's contents), stored and accumulated, with row
strides wider than the rows; calls issued on two streams without waiting in
between (the library orders them on the device); sizes over the scratch
are refused."""
import ctypes as C

import numpy as np
import pytest

from helpers import f32_bits_equal, mismatch_report
from indecis_amd import _lib, linalg

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _call(b, dc, ldc, da, lda, m, acc, stream):
    _lib.check(_lib.lib().ixh_matmul8_noalloc(b._h, C.c_void_p(dc.data_ptr()), ldc, C.c_void_p(da.data_ptr()),
                                              lda, m, 1 if acc else 0, C.c_void_p(stream)))


@pytest.mark.parametrize("k,n", [(768, 2304), (1152, 768), (68, 40)])
def test_matmul8_noalloc_equals_matmul8(k, n):
    rng = np.random.default_rng(k + n)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    b = linalg.PackedB8(q, s)
    lda, ldc = k + 4, n + 8
    stream = torch.cuda.current_stream().cuda_stream
    for m in (3001, 517):  # the second call is smaller
        a = (rng.standard_normal((m, k)) * 2).astype(np.float32)
        c0 = rng.standard_normal((m, n)).astype(np.float32)
        for acc in (False, True):
            want = linalg.matmul8(c0.copy(), a, b, m, accumulate=acc)
            ap = np.zeros((m, lda), np.float32)
            ap[:, :k] = a
            cp = np.full((m, ldc), 3.5, np.float32)
            cp[:, :n] = c0
            da = torch.from_numpy(ap).cuda()
            dc = torch.from_numpy(cp).cuda()
            torch.cuda.synchronize()
            _call(b, dc, ldc, da, lda, m, acc, stream)
            torch.cuda.synchronize()
            got = dc.cpu().numpy()
            assert f32_bits_equal(got[:, :n], want), mismatch_report(got[:, :n], want)
            assert np.all(got[:, n:] == 3.5)  # past n: untouched
    b.close()


def test_matmul8_noalloc_two_streams():
    """Calls on two streams, issued back to back, each bit-exact: the second
    call's quantisation into the shared scratch waits for the first call's
    GEMM."""
    rng = np.random.default_rng(17)
    k, n = 1152, 768
    b = linalg.PackedB8(rng.integers(-127, 128, size=(n, k), dtype=np.int8),
                        rng.uniform(1e-3, 1e-2, size=n).astype(np.float32))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    sizes = [4096, 2500, 4096, 1]
    cases = []
    for i, m in enumerate(sizes):
        a = (rng.standard_normal((m, k)) * 2).astype(np.float32)
        want = linalg.matmul8(np.zeros((m, n), np.float32), a, b, m)
        cases.append((m, torch.from_numpy(a).cuda(), torch.zeros((m, n), dtype=torch.float32, device="cuda"),
                      want))
    torch.cuda.synchronize()
    for rep in range(3):
        for _, _, dc, _ in cases:
            dc.fill_(7.0)  # fill kernels on the current stream, finished before the calls
        torch.cuda.synchronize()
        for i, (m, da, dc, _) in enumerate(cases):
            _call(b, dc, n, da, k, m, False, streams[i % 2].cuda_stream)
        torch.cuda.synchronize()
        for i, (m, da, dc, want) in enumerate(cases):
            got = dc.cpu().numpy()
            assert f32_bits_equal(got, want), f"rep {rep} call {i}: " + mismatch_report(got, want)
    b.close()


def test_matmul8_noalloc_limits():
    rng = np.random.default_rng(5)
    k, n = 1152, 256
    b = linalg.PackedB8(rng.integers(-127, 128, size=(n, k), dtype=np.int8),
                        rng.uniform(1e-3, 1e-2, size=n).astype(np.float32))
    m = (32 << 20) // (k + 4) + 1  # one row more than the scratch holds
    da = torch.zeros((m, k), dtype=torch.float32, device="cuda")
    dc = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    with pytest.raises(_lib.IxhError, match="need .* bytes of scratch, over its 33554432"):
        _call(b, dc, n, da, k, m, False, 0)
    with pytest.raises(_lib.IxhError, match="lda >= k"):
        _call(b, dc, n, da, k - 4, 10, False, 0)
    _call(b, dc, n, da, k, 0, False, 0)  # nothing to do
    b.close()
