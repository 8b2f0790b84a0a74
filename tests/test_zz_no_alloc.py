"""qtts_gemm_q4_noalloc: qtts_gemm_q4 on device rows with nothing allocated
(split-K partial sums in the library's per-GPU scratch array).

Checked through the C ABI against qtts_gemm_q4 on the same weight and rows:
two calls in a row on the same device buffers, the second with fewer rows
(the scratch keeps the first call's contents), on both paths (GEMV passes
and the matrix-core GEMM) and on a ragged n; bit-identical, since both run
the same kernels in the same order, and within 1e-3 of the oracle; rows far
outside the f16 range on the matrix cores (their largest |x| staged in the
same array).  A weight whose passes need more scratch than the array holds
is refused.
The device buffers are the caller's, allocated here with hipMalloc.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


def hip():
    lib = ctypes.CDLL("libamdhip64.so")
    lib.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    lib.hipFree.argtypes = [ctypes.c_void_p]
    lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    lib.hipSetDevice.argtypes = [ctypes.c_int]
    return lib


class DevBuf:
    def __init__(self, h, nbytes):
        self.h, self.ptr = h, ctypes.c_void_p()
        assert h.hipMalloc(ctypes.byref(self.ptr), nbytes) == 0
        self.nbytes = nbytes

    def put(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        assert self.h.hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D) == 0

    def get(self, shape):
        out = np.empty(shape, np.float32)
        assert out.nbytes <= self.nbytes
        assert self.h.hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H) == 0
        return out

    def free(self):
        self.h.hipFree(self.ptr)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("k,n,rows,path", [(2048, 6144, (5, 3), "rowwise"), (3072, 1000, (7, 2), None),
                                           (2048, 4096, (40, 17), "mfma"), (6144, 2048, (20, 16), None)])
def test_gemm_noalloc_matches_gemm(ctx_factory, k, n, rows, path):
    print(f"gemm_noalloc k={k} n={n} rows={rows} path={path}", flush=True)
    c = ctx_factory(256)
    h = hip()
    assert h.hipSetDevice(0) == 0
    rng = np.random.Generator(np.random.PCG64(k + n + rows[0]))
    w = synth.q4_random(rng, k, n)
    dw = c.upload(w)
    X = rng.standard_normal((rows[0], k)).astype(np.float32)
    dx, dy = DevBuf(h, X.nbytes), DevBuf(h, rows[0] * n * 4)
    try:
        for r in rows:
            Xr = X[:r] * (1.0 + r)          # the second call's rows differ from the first's
            ref = c.gemm(dw, Xr, path=path)
            dx.put(Xr)
            dy.put(np.full((rows[0], n), np.nan, np.float32))
            c.gemm_noalloc(dw, dx.ptr.value, r, dy.ptr.value, path=path)
            c.sync()
            Y = dy.get((rows[0], n))
            assert np.array_equal(bits(Y[:r]), bits(ref)), f"rows {r}: differs from qtts_gemm_q4"
            assert np.all(np.isnan(Y[r:])), f"rows {r}: wrote past its rows"
            R = O.gemm(Xr[:2], w)
            for i in range(2):
                scale = max(np.abs(R[i]).max(), np.sqrt((R[i].astype(np.float64) ** 2).mean()))
                assert np.abs(Y[i] - R[i]).max() <= 1e-3 * scale
    finally:
        dx.free()
        dy.free()
        dw.free()


def test_gemm_noalloc_extreme_rows(ctx_factory):
    """Rows far outside the f16 range on the matrix cores: the rows' largest
    |x| (the staging range) go to the scratch array too; bit-identical to
    qtts_gemm_q4 on two calls in a row, the second with fewer rows."""
    c = ctx_factory(256)
    h = hip()
    assert h.hipSetDevice(0) == 0
    rng = np.random.Generator(np.random.PCG64(1234))
    k, n = 2048, 4096
    w = synth.q4_random(rng, k, n)
    dw = c.upload(w)
    X = rng.standard_normal((24, k)).astype(np.float32)
    X[0] *= 1e5
    X[1] *= 1e-6
    X[2, 5] = 1e5
    X[20] *= 3e4
    dx, dy = DevBuf(h, X.nbytes), DevBuf(h, X.shape[0] * n * 4)
    try:
        for r in (24, 18):
            Xr = X[:r]
            ref = c.gemm(dw, Xr, path="mfma")
            dx.put(Xr)
            c.gemm_noalloc(dw, dx.ptr.value, r, dy.ptr.value, path="mfma")
            c.sync()
            Y = dy.get((r, n))
            assert np.array_equal(bits(Y), bits(ref)), f"rows {r}: differs from qtts_gemm_q4"
        R = O.gemm(X[:3], w)
        for i in range(3):
            assert np.abs(Y[i].astype(np.float64) - R[i]).max() <= 1e-3 * np.abs(R[i]).max()
    finally:
        dx.free()
        dy.free()
        dw.free()


def test_gemm_noalloc_refuses_oversized_scratch(ctx_factory, monkeypatch):
    """16 slices of 128 rows (tile G8_T128) x 33,792 columns need 1,081,344
    floats of partial sums, beyond the 1,048,576 the array holds."""
    monkeypatch.setenv("QTTS_TILE_GEMV", "1")
    c = ctx_factory(256)
    h = hip()
    rng = np.random.Generator(np.random.PCG64(77))
    dw = c.upload(synth.q4_random(rng, 2048, 33792))
    dx, dy = DevBuf(h, 2 * 2048 * 4), DevBuf(h, 2 * 33792 * 4)
    try:
        with pytest.raises(qtts.QttsError) as e:
            c.gemm_noalloc(dw, dx.ptr.value, 2, dy.ptr.value, path="rowwise")
        assert e.value.code == qtts.ERR_CAPACITY
    finally:
        dx.free()
        dy.free()
        dw.free()
