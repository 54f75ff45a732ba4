"""The allocation-free ConvEval (sh_conv_eval_noalloc): device buffers the caller owns, the
operand planes and split-product partials in the library's static per-GPU scratch, no
allocation in the call. Its output must equal sh_conv_eval's bit for bit (the same kernels),
on two calls in a row, the second with a smaller input (the scratch keeps the first call's
contents, which the second must not read), and a size beyond the scratch must be refused
with a message."""
import ctypes as C

import numpy as np
import pytest

import stories_hip as sh

pytestmark = pytest.mark.gpu


class Hip:
    """The few HIP runtime calls the test needs to own device buffers (the caller's side),
    looked up through the library's handle: dlsym on it searches the library's own
    dependencies, so these are the calls of the HIP runtime the library itself runs on
    (a process may already hold another copy, e.g. one loaded with torch)."""

    def __init__(self):
        self.h = sh.load()
        self.h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.h.hipFree.argtypes = [C.c_void_p]
        self.h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.h.hipDeviceSynchronize.argtypes = []

    def malloc(self, n):
        p = C.c_void_p()
        assert self.h.hipMalloc(C.byref(p), n) == 0
        return p

    def h2d(self, dst, a):
        assert self.h.hipMemcpy(dst, a.ctypes.data_as(C.c_void_p), a.nbytes, 1) == 0

    def d2h(self, a, src):
        assert self.h.hipMemcpy(a.ctypes.data_as(C.c_void_p), src, a.nbytes, 2) == 0

    def sync(self):
        assert self.h.hipDeviceSynchronize() == 0

    def free(self, p):
        self.h.hipFree(p)


@pytest.mark.parametrize("out_dim,in_dim", [(192, 256), (768, 768)])
def test_conv_eval_noalloc_matches_conv_eval(gpu, out_dim, in_dim):
    lib = sh.load()
    hip = Hip()
    rng = np.random.default_rng(181 + out_dim)
    w = (rng.standard_normal((out_dim, in_dim)) * 0.05).astype(np.float32)
    conv = sh.Conv(w)
    s_max = 96
    dx = hip.malloc(4 * s_max * in_dim)
    dy = hip.malloc(4 * s_max * out_dim)
    try:
        for s in (s_max, 5):   # a long input, then a shorter one over the same scratch
            x = rng.standard_normal((s, in_dim)).astype(np.float32)
            want = conv.eval(x)
            hip.h2d(dx, x)
            rc = lib.sh_conv_eval_noalloc(conv.h, dx, s, dy, None)
            assert rc == 0, sh.last_error()
            hip.sync()
            got = np.empty((s, out_dim), np.float32)
            hip.d2h(got, dy)
            np.testing.assert_array_equal(got, want)
        # beyond the 16 MiB scratch: refused, with the size it would need
        big = (16 << 20) // (4 * in_dim) + 1
        assert lib.sh_conv_eval_noalloc(conv.h, dx, big, dy, None) != 0
        assert "scratch" in sh.last_error()
    finally:
        hip.free(dx)
        hip.free(dy)
        conv.close()
