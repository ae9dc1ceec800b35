"""The allocation-free reduction entry (dpuf_amd_reduce_check_noalloc) against
the allocating one (dpuf_amd_reduce_check), through the C ABI.

Device buffers for its inputs and outputs come from the HIP runtime the
library itself links (libamdhip64.so.7, loaded through ctypes: the same
instance, so the pointers are valid for the library).  Two calls in a row on
the same device, the second with a smaller input, for the argmax and the
top-2 margin check: the second call must not see the first call's partials.
"""
import ctypes as C

import numpy as np
import pytest

from dpuf_amd import model as M

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


@pytest.fixture(scope="module")
def hip(eng):
    lib = C.CDLL("libamdhip64.so.7")
    lib.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    lib.hipFree.argtypes = [C.c_void_p]
    lib.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    lib.hipDeviceSynchronize.argtypes = []
    return lib


class Dev:
    """A device buffer holding a copy of a host array."""

    def __init__(self, hip, host):
        self.hip, self.n = hip, host.nbytes
        self.p = C.c_void_p()
        assert hip.hipMalloc(C.byref(self.p), max(self.n, 4)) == 0
        if self.n:
            assert hip.hipMemcpy(self.p, M.ptr(host), self.n, H2D) == 0

    def get(self, like):
        out = np.empty_like(like)
        assert self.hip.hipMemcpy(M.ptr(out), self.p, out.nbytes, D2H) == 0
        return out

    def free(self):
        self.hip.hipFree(self.p)


def _noalloc(eng, hip, x, mode, thr):
    dx = Dev(hip, x)
    do = Dev(hip, np.full(1, -7, np.int32))
    try:
        rc = eng.dpuf_amd_reduce_check_noalloc(dx.p, x.size, mode, thr, do.p, None)
        assert rc == 0, (rc, eng.dpuf_amd_last_error())
        assert hip.hipDeviceSynchronize() == 0
        return int(do.get(np.zeros(1, np.int32))[0])
    finally:
        dx.free()
        do.free()


@pytest.mark.parametrize("mode", [1, 0])
def test_noalloc_matches_allocating_entry(eng, hip, mode):
    rng = np.random.default_rng(7 + mode)
    big = rng.standard_normal(151936).astype(np.float32)
    big[[1234, 90000]] = 9.5  # a repeated maximum: first one wins
    small = rng.standard_normal(1001).astype(np.float32)
    small[17] = 4.0
    for thr in ((0.0,) if mode == 1 else (0.05, 3.0)):
        for x in (big, small):  # the second call is the smaller one
            want = eng.dpuf_amd_reduce_check(M.ptr(x), x.size, 0, mode, thr)
            got = _noalloc(eng, hip, x, mode, thr)
            print(f"noalloc mode={mode} n={x.size} thr={thr}: {got} (allocating entry {want})", flush=True)
            assert want >= 0 and got == want


def test_noalloc_rejects_bad_arguments(eng, hip):
    x = np.ones(8, np.float32)
    dx = Dev(hip, x)
    do = Dev(hip, np.zeros(1, np.int32))
    try:
        assert eng.dpuf_amd_reduce_check_noalloc(dx.p, 0, 1, 0.0, do.p, None) == -2
        assert eng.dpuf_amd_reduce_check_noalloc(dx.p, (1 << 30) + 1, 1, 0.0, do.p, None) == -2
        assert eng.dpuf_amd_reduce_check_noalloc(None, 8, 1, 0.0, do.p, None) == -1
        assert eng.dpuf_amd_reduce_check_noalloc(dx.p, 8, 2, 0.0, do.p, None) == -1
    finally:
        dx.free()
        do.free()
