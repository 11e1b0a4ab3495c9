"""cora_tool_assign_noalloc, the allocation-free variant of cora_tool_assign, through the
C-ABI: the same assignment as cora_tool_assign on the same inputs for two calls in a row,
the second with a smaller input (the scratch array keeps the first call's contents), and
sizes beyond its maximum rejected with an error. Device buffers come from the HIP runtime
the library itself links (hipMalloc through ctypes, outside the entry point under test)."""
import ctypes as C
import sys

import numpy as np
import pytest

import coraanns_amd as ca

pytestmark = pytest.mark.gpu
H2D, D2H = 1, 2  # hipMemcpyHostToDevice, hipMemcpyDeviceToHost


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def hip_runtime():
    ca.libs()  # loads libcora_gpu.so and, with it, the HIP runtime it links
    rt = C.CDLL("libamdhip64.so.7")
    rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    rt.hipFree.argtypes = [C.c_void_p]
    rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    rt.hipSetDevice.argtypes = [C.c_int]
    for f in (rt.hipMalloc, rt.hipFree, rt.hipMemcpy, rt.hipSetDevice):
        f.restype = C.c_int
    return rt


class DeviceArray:
    def __init__(self, rt, host):
        self.rt, self.host = rt, np.ascontiguousarray(host)
        self.ptr = C.c_void_p()
        assert rt.hipMalloc(C.byref(self.ptr), max(1, self.host.nbytes)) == 0
        assert rt.hipMemcpy(self.ptr, self.host.ctypes.data, self.host.nbytes, H2D) == 0

    def read(self):
        out = np.empty_like(self.host)
        assert self.rt.hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H) == 0
        return out

    def free(self):
        if self.ptr:
            self.rt.hipFree(self.ptr)
            self.ptr = C.c_void_p()


def test_assign_noalloc_matches_assign():
    rt = hip_runtime()
    assert rt.hipSetDevice(0) == 0
    gpu = ca._load()[0]
    rng = np.random.default_rng(5)
    # the first call fills the scratch with 8 blocks of distances; the second, smaller one
    # (fewer rows, centroids and dimensions) reuses it
    for n, dim, k in [(30000, 128, 1024), (7000, 96, 300)]:
        say(f"[gpu] assign_noalloc n={n} dim={dim} k={k}")
        centers = rng.normal(0, 1, (k, dim)).astype(np.float32)
        x = (centers[rng.integers(0, k, n)] + rng.normal(0, 0.5, (n, dim))).astype(np.float32)
        want = ca.gpu_assign(x, centers)
        dx, dc = DeviceArray(rt, x), DeviceArray(rt, centers)
        da = DeviceArray(rt, np.full(n, 0xFFFFFFFF, np.uint32))
        try:
            ca._tool_check(gpu.cora_tool_assign_noalloc(dx.ptr, n, dim, dc.ptr, k, da.ptr, 0))
            got = da.read()
        finally:
            for a in (dx, dc, da):
                a.free()
        assert np.array_equal(got, want), (n, dim, k, int((got != want).sum()))


def test_assign_noalloc_rejects_sizes_beyond_its_scratch():
    rt = hip_runtime()
    assert rt.hipSetDevice(0) == 0
    gpu = ca._load()[0]
    x = np.zeros((4, 8), np.float32)
    dx, da = DeviceArray(rt, x), DeviceArray(rt, np.zeros(4, np.uint32))
    try:
        for k, dim in [(1048577, 8), (4, 4097)]:
            rc = gpu.cora_tool_assign_noalloc(dx.ptr, 4, dim, dx.ptr, k, da.ptr, 0)
            assert rc == ca.ERR_INVALID_ARGUMENT
            assert b"at most" in gpu.cora_tool_last_error()
        assert gpu.cora_tool_assign_noalloc(None, 4, 8, dx.ptr, 4, da.ptr, 0) == ca.ERR_INVALID_ARGUMENT
    finally:
        dx.free()
        da.free()
