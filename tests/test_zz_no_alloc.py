"""qmatmul_device_noalloc (the allocation-free qmatmul for callers that cannot
allocate) through the C ABI, against the existing qmatmul entry point: equal
bit for bit on two calls in a row, the second smaller, across the one-row GEMV,
the skinny MFMA and the GEMM paths; sizes past the static scratch are refused
with an error."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
import qlib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def Q():
    q = qlib.load()
    assert q.lib().qllama_device_count() > 0, "no GPU visible to the HIP library"
    q.lib().qmatmul_device_noalloc.argtypes = [C.c_void_p, C.c_int, C.POINTER(q.QTensor), C.c_void_p]
    return q


class DevBuf:
    """A device buffer the caller owns (qllama_dev_alloc), filled from host memory."""

    def __init__(self, Q, host):
        self.L = Q.lib()
        self.host = np.ascontiguousarray(host)
        self.p = self.L.qllama_dev_alloc(self.host.nbytes)
        assert self.p
        assert self.L.qllama_h2d(self.p, self.host.ctypes.data, self.host.nbytes) == 0

    def read(self):
        out = np.empty_like(self.host)
        assert self.L.qllama_d2h(out.ctypes.data, self.p, out.nbytes) == 0
        return out

    def free(self):
        self.L.qllama_dev_free(self.p)


def _noalloc(Q, A, W):
    """A (host) -> a caller's device buffer, qmatmul_device_noalloc, C back."""
    dA = DevBuf(Q, A)
    dC = DevBuf(Q, np.full((A.shape[0], W.cols), np.nan, np.float32))
    try:
        assert Q.lib().qmatmul_device_noalloc(dA.p, A.shape[0], C.byref(W.t), dC.p) == 0
        assert Q.lib().qllama_sync() == 0
        return dC.read()
    finally:
        dA.free()
        dC.free()


# (M, K, N) pairs: each second call is smaller than the first
CALLS = [((8, 4096, 1024), (3, 1000, 517)),       # skinny MFMA path, K not a multiple of 64 on the second
         ((40, 2048, 300), (1, 2048, 300)),       # MFMA GEMM, then the one-row decode GEMV
         ((16, 14336, 4096), (2, 4096, 4096))]    # BASELINE's down-projection and Wo shapes


@pytest.mark.parametrize("calls", CALLS, ids=lambda c: f"{c[0][0]}x{c[0][1]}x{c[0][2]}_then_{c[1][0]}x{c[1][1]}x{c[1][2]}")
def test_noalloc_matches_qmatmul(Q, calls):
    rng = np.random.default_rng(sum(sum(c) for c in calls))
    for (M, K, N) in calls:
        A = rng.standard_normal((M, K)).astype(np.float32)
        A[0, :7] = 0.0
        w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
        W = Q.QWeight(w)
        try:
            ref = Q.qmatmul(A, W)
            got = _noalloc(Q, A, W)
        finally:
            W.close()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (M, K, N)
        q, s = O.quantize(w)
        assert np.array_equal(ref.view(np.uint32), O.qmatmul(A, q, s).view(np.uint32)), (M, K, N)


def test_noalloc_refuses_sizes_past_its_scratch(Q):
    w = np.zeros((8192, 16), np.float32)
    W = Q.QWeight(w)
    dA = DevBuf(Q, np.zeros((2049, 8192), np.float32))    # 2049 rows of 8 KiB: past the 16 MiB scratch
    dC = DevBuf(Q, np.zeros((2049, 16), np.float32))
    try:
        assert Q.lib().qmatmul_device_noalloc(dA.p, 2049, C.byref(W.t), dC.p) != 0
        # the refusal touched nothing: the library stays usable
        A = np.ones((2, 8192), np.float32)
        assert np.array_equal(_noalloc(Q, A, W), Q.qmatmul(A, W))
    finally:
        dA.free()
        dC.free()
        W.close()
