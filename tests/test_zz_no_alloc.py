"""draco_gemv_q8k_f32_noalloc (no reference counterpart: the allocation-free
variant of draco_gemv_q8k_f32 for callers that cannot allocate) through the C
ABI, against draco_gemv_q8k_f32 on the same inputs: bit-identical outputs
(the same kernels on the same bytes), on two calls in a row, the second with
a smaller input, and a size past the static staging array rejected.

Device buffers come from the HIP runtime the library itself links
(/opt/rocm libamdhip64, through ctypes), not from torch: torch bundles a HIP
runtime of its own, and two runtimes in one process are not relied on."""
import ctypes as ct
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class Hip:
    """hipMalloc / hipMemcpy / hipFree of the library's own HIP runtime."""

    def __init__(self):
        path = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so")
        self.rt = ct.CDLL(path)
        self.rt.hipMalloc.argtypes = [ct.POINTER(ct.c_void_p), ct.c_size_t]
        self.rt.hipFree.argtypes = [ct.c_void_p]
        self.rt.hipMemcpy.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_size_t, ct.c_int]
        self.rt.hipDeviceSynchronize.argtypes = []
        self.live = []

    def upload(self, a):
        p = ct.c_void_p()
        assert self.rt.hipMalloc(ct.byref(p), a.nbytes) == 0
        self.live.append(p.value)
        assert self.rt.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) == 0  # host -> device
        return p.value

    def download(self, p, a):
        assert self.rt.hipDeviceSynchronize() == 0
        assert self.rt.hipMemcpy(a.ctypes.data, p, a.nbytes, 2) == 0  # device -> host
        return a

    def free(self):
        self.rt.hipDeviceSynchronize()
        for p in self.live:
            self.rt.hipFree(p)
        self.live = []


def _packed(lib, code, W, n_out, n_in):
    off = (ct.c_size_t * 4)()
    nbytes = lib.load().draco_layout_query(code, n_out, n_in, off)
    packed = np.zeros(nbytes, np.uint8)
    lib.check(lib.load().draco_repack(code, lib.pu8(W), n_out, n_in, lib.pu8(packed)), "draco_repack")
    return packed


@pytest.mark.parametrize("code", [5, 4])
def test_noalloc_matches_allocating_entry(code):
    from dracohip import lib
    L = lib.load()
    hip = Hip()
    try:
        for k, (n_out, n_in, nvec) in enumerate([(4096, 14336, 8), (520, 2048, 1)]):
            rng = np.random.default_rng(300 + k)
            W = lib.quantize(code, rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02))
            x = rng.standard_normal((nvec, n_in)).astype(np.float32)
            want = np.zeros(nvec * n_out, np.float32)
            lib.check(L.draco_gemv_q8k_f32(code, lib.pf(x), nvec, lib.pu8(W), n_out, n_in, lib.pf(want)),
                      "draco_gemv_q8k_f32")
            dW = hip.upload(_packed(lib, code, W, n_out, n_in))
            dx = hip.upload(x)
            dy = hip.upload(np.full(nvec * n_out, np.nan, np.float32))
            print(f"[noalloc] code {code} call {k}: {n_out}x{n_in} nvec {nvec}", flush=True)
            rc = L.draco_gemv_q8k_f32_noalloc(code, dx, nvec, dW, n_out, n_in, dy, None)
            assert rc == 0, lib.last_error()
            got = hip.download(dy, np.zeros(nvec * n_out, np.float32))
            assert np.array_equal(got, want), float(np.nanmax(np.abs(got - want)))
    finally:
        hip.free()


def test_noalloc_rejects_oversize():
    from dracohip import lib
    L = lib.load()
    cap = L.draco_noalloc_capacity()
    n_in = 256 * (cap // (8 * 292) + 1)  # one block past the array at nvec 8
    # rejected before any pointer is used or any kernel enqueued
    rc = L.draco_gemv_q8k_f32_noalloc(5, 16, 8, 16, 16, n_in, 16, None)
    assert rc == -1 and "static array" in lib.last_error()
