"""gorch_hip_linear_bf16_noalloc — the Linear for callers that cannot
allocate device memory — against gorch_hip_linear_bf16 on the same inputs,
through the C-ABI. Both run the same kernels, so the outputs must be
bit-identical. Two calls in a row (the second smaller) show that the fixed
scratch array carries nothing from one call into the next; a fresh stream
shows that the call allocates nothing (the allocating entry point would
create that stream's partials buffer on first use)."""
import ctypes as C

import numpy as np
import pytest

from gorch_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _mem_free():
    hip_rt = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip_rt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


class Dev:
    def __init__(self, lib, a=None, nbytes=None):
        self.lib = lib
        if a is not None:
            a = np.ascontiguousarray(a)
            nbytes = a.nbytes
        self.p = lib.gorch_hip_alloc(nbytes)
        assert self.p, lib.gorch_hip_last_error()
        if a is not None:
            assert lib.gorch_hip_upload(None, self.p, a.ctypes.data, a.nbytes) == 0

    def get(self, shape):
        out = np.empty(shape, np.float32)
        assert self.lib.gorch_hip_download(None, out.ctypes.data, self.p, out.nbytes) == 0
        return out

    def free(self):
        self.lib.gorch_hip_release(self.p)


@pytest.fixture(scope="module")
def lib(gpu):
    return gpu.lib()


def _pair(lib, M, N, K, epi, seed, residual=False, stream=None, check_mem=True):
    x, W, b = syn.gemv_inputs(M, K, N, seed=seed)
    b = (b + np.random.default_rng(seed).standard_normal(N).astype(np.float32)).astype(np.float32)
    dx, dW, db = Dev(lib, x), Dev(lib, W), Dev(lib, b)
    r = np.random.default_rng(seed + 1).standard_normal((M, N)).astype(np.float32) if residual else None
    dr = Dev(lib, r) if residual else None
    y0, y1 = Dev(lib, nbytes=M * N * 4), Dev(lib, nbytes=M * N * 4)
    rp = dr.p if residual else None
    # the allocating entry point first, on the null stream: the runtime
    # loads a kernel's code object (device memory) at its first launch
    assert lib.gorch_hip_linear_bf16(None, dx.p, dW.p, db.p, rp, y0.p, M, N, K, epi) == 0
    want = y0.get((M, N))
    assert lib.gorch_hip_sync(None) == 0
    free0 = _mem_free()
    held0, live0 = lib.gorch_hip_scratch_bytes(), lib.gorch_hip_live_bytes()
    assert lib.gorch_hip_linear_bf16_noalloc(stream, dx.p, dW.p, db.p, rp, y1.p, M, N, K, epi) == 0, \
        lib.gorch_hip_last_error()
    assert lib.gorch_hip_sync(stream) == 0
    # a fresh stream has no partials buffer: an allocating call would take
    # one, which the library's own counters show (the device-wide free bytes
    # are a second signal, exposed to other tenants of the GPU)
    assert lib.gorch_hip_scratch_bytes() == held0
    assert lib.gorch_hip_live_bytes() == live0
    if check_mem:
        assert _mem_free() == free0
    got = y1.get((M, N))
    for t in (dx, dW, db, y0, y1) + ((dr,) if residual else ()):
        t.free()
    return got, want


def test_noalloc_two_calls_second_smaller(lib):
    import torch

    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    # the runtime sets up a stream's launch resources (device memory too) at
    # its first launch: one unsplit call first, then every call is measured
    _pair(lib, 1, 64, 64, 0, seed=0, stream=s.cuda_stream, check_mem=False)
    # a narrow weight over a long K: the K split through the scratch array
    # (8 slices x 16 rows x 768 columns of partials)
    got, want = _pair(lib, 16, 768, 3072, 0, seed=1, stream=s.cuda_stream)
    assert np.array_equal(got, want)
    # smaller, with GELU and a residual: fewer slices and rows, so stale
    # partials of the first call sit beyond what this one reads
    got, want = _pair(lib, 4, 512, 2048, 1, seed=2, residual=True, stream=s.cuda_stream)
    assert np.array_equal(got, want)
    # the largest split the routing takes (127 tiles, 16 rows)
    got, want = _pair(lib, 16, 2032, 1024, 0, seed=3, stream=s.cuda_stream)
    assert np.array_equal(got, want)
    # no split: one row, and the GEMM path above 16 rows
    got, want = _pair(lib, 1, 768, 3072, 0, seed=4, stream=s.cuda_stream)
    assert np.array_equal(got, want)
    got, want = _pair(lib, 40, 256, 512, 0, seed=5, stream=s.cuda_stream)
    assert np.array_equal(got, want)
    # the counter the checks above rely on does see an allocation: the
    # allocating entry point takes a partials buffer for a new stream's
    # first K split (a stream made here: torch hands out streams from a
    # pool, which earlier calls may have used)
    hip_rt = C.CDLL("libamdhip64.so")
    s2 = C.c_void_p()
    assert hip_rt.hipStreamCreate(C.byref(s2)) == 0
    x, W, b = syn.gemv_inputs(16, 3072, 768, seed=6)
    dx, dW, db, dy = Dev(lib, x), Dev(lib, W), Dev(lib, b), Dev(lib, nbytes=16 * 768 * 4)
    held = lib.gorch_hip_scratch_bytes()
    assert lib.gorch_hip_linear_bf16(s2, dx.p, dW.p, db.p, None, dy.p, 16, 768, 3072, 0) == 0
    assert lib.gorch_hip_sync(s2) == 0
    assert lib.gorch_hip_scratch_bytes() > held
    for t in (dx, dW, db, dy):
        t.free()
    # (the stream stays: the library keeps its partials buffer for it)


def test_noalloc_rejects_bad_arguments(lib):
    assert lib.gorch_hip_linear_bf16_noalloc(None, None, None, None, None, None, 2, 8, 8, 0) == 2
    assert lib.gorch_hip_linear_bf16_noalloc(None, None, None, None, None, None, 2, 8, 8, 7) == 2
    assert lib.gorch_hip_linear_bf16_noalloc(None, None, None, None, None, None, 0, 8, 8, 0) == 0
