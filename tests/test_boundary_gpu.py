"""The C-ABI the way gorch's Go binding would drive it (metal/metal.go:251-309,
:405-422; tensor.go:318-323, :388-406): device memory from gorch_hip_alloc,
host data moved with gorch_hip_upload / gorch_hip_download, compute on raw
device pointers, gorch_hip_sync as the read barrier, gorch_hip_release to
free. No torch allocation or stream is involved: the stream argument is
NULL (the device's null stream), as a cgo caller without a stream of its
own would pass.

Results are checked against the CPU oracle at the reference's bars:
matmul within 1e-3 of RMS (bf16_matmul_metal_test.go:100-117), codec
bit-exact (tensor.go:85-121).
"""
import ctypes as C

import numpy as np
import pytest

import oracle as orc
from gorch_amd import synthetic as syn
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


class Dev:
    """A device buffer owned through the C-ABI (alloc / release)."""

    def __init__(self, lib, nbytes):
        self.lib = lib
        self.n = nbytes
        self.p = lib.gorch_hip_alloc(nbytes)
        assert self.p, lib.gorch_hip_last_error()

    def put(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.n
        assert self.lib.gorch_hip_upload(None, self.p, a.ctypes.data, a.nbytes) == 0
        return self

    def get(self, dtype, shape):
        out = np.empty(shape, dtype)
        assert self.lib.gorch_hip_download(None, out.ctypes.data, self.p, out.nbytes) == 0
        return out

    def free(self):
        self.lib.gorch_hip_release(self.p)
        self.p = None


@pytest.fixture(scope="module")
def lib(gpu):
    return gpu.lib()


def up(lib, a):
    a = np.ascontiguousarray(a)
    return Dev(lib, a.nbytes).put(a)


def test_memory_round_trip_and_errors(lib):
    rng = np.random.default_rng(1)
    a = rng.standard_normal(12345).astype(np.float32)
    d = up(lib, a)
    assert np.array_equal(d.get(np.float32, a.shape), a)
    # partial download of a prefix
    assert np.array_equal(d.get(np.float32, (100,)), a[:100])
    d.free()
    lib.gorch_hip_release(None)                       # release(NULL) is a no-op
    z = lib.gorch_hip_alloc(0)                        # zero bytes: a valid, releasable handle
    assert z
    lib.gorch_hip_release(z)
    host = np.zeros(4, np.float32)
    assert lib.gorch_hip_upload(None, None, host.ctypes.data, 16) == 2      # EINVAL
    assert lib.gorch_hip_download(None, host.ctypes.data, None, 16) == 2
    assert lib.gorch_hip_last_error()


@pytest.mark.parametrize("M,N,K", [(1, 3072, 768), (16, 768, 3072), (64, 300, 200)])
def test_linear_on_raw_pointers(lib, M, N, K):
    x, W, b = syn.gemv_inputs(M, K, N, seed=M + N)
    dx, dW, db = up(lib, x), up(lib, W), up(lib, b)
    dy = Dev(lib, M * N * 4)
    assert lib.gorch_hip_linear_bf16(None, dx.p, dW.p, db.p, None, dy.p, M, N, K, 0) == 0
    assert lib.gorch_hip_sync(None) == 0
    got = dy.get(np.float32, (M, N))
    assert rel_err(got, orc.linear(x, W, b)) <= 1e-3
    if M <= 16:
        # the resident tile-packed format and the GEMV over it
        dWp = Dev(lib, lib.gorch_hip_packed_bf16_bytes(N, K))
        assert lib.gorch_hip_pack_bf16(None, dW.p, dWp.p, N, K) == 0
        dy2 = Dev(lib, M * N * 4)
        assert lib.gorch_hip_linear_bf16_packed(None, dx.p, dWp.p, db.p, None, dy2.p, M, N, K, 0) == 0
        assert lib.gorch_hip_sync(None) == 0
        assert rel_err(dy2.get(np.float32, (M, N)), orc.linear(x, W, b)) <= 1e-3
        dWp.free()
        dy2.free()
    for t in (dx, dW, db, dy):
        t.free()


@pytest.mark.parametrize("transA,transB,aBF16,bBF16", [(0, 1, 0, 1), (0, 0, 1, 1), (1, 0, 0, 1), (0, 0, 1, 0)])
def test_matmul_dt_on_raw_pointers(lib, transA, transB, aBF16, bBF16):
    M, N, K = 24, 40, 56
    rng = np.random.default_rng(7)
    A = rng.standard_normal((K, M) if transA else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if transB else (K, N)).astype(np.float32)
    A = orc.f32_to_bf16(A) if aBF16 else A
    B = orc.f32_to_bf16(B) if bBF16 else B
    dA, dB, dC = up(lib, A), up(lib, B), Dev(lib, M * N * 4)
    assert lib.gorch_hip_matmul_dt(None, dA.p, dB.p, dC.p, M, N, K, transA, transB, aBF16, bBF16) == 0
    got = dC.get(np.float32, (M, N))          # download is the read barrier
    assert rel_err(got, orc.matmul_dt(A, B, M, N, K, bool(transA), bool(transB))) <= 1e-3
    for t in (dA, dB, dC):
        t.free()


def test_codec_on_raw_pointers(lib):
    bits = np.arange(1 << 16, dtype=np.uint16)
    dh, df = up(lib, bits), Dev(lib, bits.size * 4)
    assert lib.gorch_hip_bf16_to_f32(None, dh.p, df.p, bits.size) == 0
    wide = df.get(np.float32, bits.shape)
    assert np.array_equal(wide.view(np.uint32), bits.astype(np.uint32) << 16)
    rng = np.random.default_rng(3)
    f = (rng.standard_normal(1 << 18) * 1e3).astype(np.float32)
    dff, dn = up(lib, f), Dev(lib, f.size * 2)
    assert lib.gorch_hip_f32_to_bf16(None, dff.p, dn.p, f.size) == 0
    assert np.array_equal(dn.get(np.uint16, f.shape), orc.f32_to_bf16(f))
    for t in (dh, df, dff, dn):
        t.free()


def test_bf16_probe_gates_the_matmul_path(gpu, lib, monkeypatch):
    """MetalBF16MatMulSupported / bf16MatMulEligible (bf16_matmul.go:52-119):
    the probe passes on a healthy device; when its host-side check rejects
    the result (the comparison tolerance forced negative), every bf16 matmul
    entry point returns GORCH_HIP_EUNSUPPORTED, the caller's cue to take its
    CPU path, while f32 x f32 still runs; a passing probe re-enables them."""
    assert gpu.bf16_matmul_supported()
    M, N, K = 4, 64, 64
    x, W, b = syn.gemv_inputs(M, K, N, seed=5)
    dx, dW, dy = up(lib, x), up(lib, W), Dev(lib, M * N * 4)
    Wf = up(lib, orc.bf16_to_f32(W))
    try:
        monkeypatch.setenv("GORCH_HIP_BF16_PROBE_TOL", "-1")
        assert not gpu.bf16_probe()
        assert not gpu.bf16_matmul_supported()
        assert lib.gorch_hip_linear_bf16(None, dx.p, dW.p, None, None, dy.p, M, N, K, 0) == 1
        assert lib.gorch_hip_matmul_dt(None, dx.p, dW.p, dy.p, M, N, K, 0, 1, 0, 1) == 1
        assert "probe" in lib.gorch_hip_last_error().decode()
        # no bf16 operand: not gated
        assert lib.gorch_hip_matmul_dt(None, dx.p, Wf.p, dy.p, M, N, K, 0, 1, 0, 0) == 0
    finally:
        monkeypatch.delenv("GORCH_HIP_BF16_PROBE_TOL")
        assert gpu.bf16_probe()
    assert lib.gorch_hip_linear_bf16(None, dx.p, dW.p, None, None, dy.p, M, N, K, 0) == 0
    assert rel_err(dy.get(np.float32, (M, N)), orc.linear(x, W)) <= 1e-3
    for t in (dx, dW, dy, Wf):
        t.free()


def test_buffer_handles_host_mirror(gpu, lib):
    """Buffer handles as gorch's Tensor would hold them (ToMetal, Data(),
    Release; tensor.go:318-406, metal/metal.go:405-422): zero-filled on
    creation, host writes reach the device before its next use, kernel
    writes reach the host at the Data() barrier, release is exactly-once."""
    M, N, K = 3, 96, 128
    x, W, b = syn.gemv_inputs(M, K, N, seed=9)
    live0 = lib.gorch_hip_live_bytes()
    bx = gpu.Buffer(x.nbytes, host_mirror=True)
    bw = gpu.Buffer(W.nbytes, host_mirror=True)
    by = gpu.Buffer(M * N * 4, host_mirror=True)
    assert len(bx) == x.nbytes
    assert lib.gorch_hip_live_bytes() - live0 == x.nbytes + W.nbytes + M * N * 4
    # fresh buffers read back as zeros
    z = np.ctypeslib.as_array(C.cast(by.host(), C.POINTER(C.c_float)), shape=(M * N,))
    assert not z.any()
    # the caller fills the mirrors (Data() with intent to write) ...
    C.memmove(bx.host(will_write=True), x.ctypes.data, x.nbytes)
    C.memmove(bw.host(will_write=True), W.ctypes.data, W.nbytes)
    # ... and the kernel reads the device copies, which are brought up to date
    rc = lib.gorch_hip_linear_bf16(None, bx.device(), bw.device(), None, None, by.device(will_write=True),
                                   M, N, K, 0)
    assert rc == 0
    got = np.ctypeslib.as_array(C.cast(by.host(), C.POINTER(C.c_float)), shape=(M, N)).copy()
    assert rel_err(got, orc.linear(x, W)) <= 1e-3
    # a buffer without a mirror has no host view
    plain = gpu.Buffer(64)
    with pytest.raises(gpu.HipError):
        plain.host()
    for buf in (bx, bw, by, plain):
        buf.release()
        buf.release()                      # exactly-once: the second is a no-op
    assert lib.gorch_hip_live_bytes() == live0
    with pytest.raises(gpu.HipError):
        bx.device()                        # released handles are unknown
    lib.gorch_hip_buf_release(None)


def test_sync_dispatch_mode(gpu, lib):
    """SetMetalAsync(false) (metal_async.go:30-38): every compute call waits
    for its stream before returning; results are the same in both modes."""
    M, N, K = 2, 512, 256
    x, W, b = syn.gemv_inputs(M, K, N, seed=11)
    dx, dW, db, dy = up(lib, x), up(lib, W), up(lib, b), Dev(lib, M * N * 4)
    assert gpu.async_enabled()
    try:
        gpu.set_async(False)
        assert not gpu.async_enabled()
        assert lib.gorch_hip_linear_bf16(None, dx.p, dW.p, db.p, None, dy.p, M, N, K, 0) == 0
        # no gorch_hip_sync: the call itself waited
        host = np.empty((M, N), np.float32)
        assert lib.gorch_hip_download(None, host.ctypes.data, dy.p, host.nbytes) == 0
        assert rel_err(host, orc.linear(x, W, b)) <= 1e-3
    finally:
        gpu.set_async(True)
    assert gpu.async_enabled()
    for t in (dx, dW, db, dy):
        t.free()


def test_release_stream_scratch(gpu, lib):
    """gorch_hip_release_stream_scratch: the narrow long-K GEMV's split takes
    scratch for the stream it runs on; releasing that stream's scratch gives
    the bytes back, and the next split launch on the stream allocates again
    and still matches the oracle."""
    import torch

    s = torch.cuda.Stream()
    M, K, N = 4, 3072, 768
    x, W, b = syn.gemv_inputs(M, K, N, seed=5)
    ref = orc.linear(x, W, b)
    Wp = gpu.pack_bf16(torch.from_numpy(W.view(np.int16)).cuda())
    xd, bd = torch.from_numpy(x).cuda(), torch.from_numpy(b).cuda()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    held0 = lib.gorch_hip_scratch_bytes()
    for _ in range(2):
        y.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            gpu.linear_bf16_packed(xd, Wp, N, bd, y)
        s.synchronize()
        assert lib.gorch_hip_scratch_bytes() > held0
        assert rel_err(y.cpu().numpy(), ref) <= 1e-3
        lib.gorch_hip_release_stream_scratch(C.c_void_p(s.cuda_stream))
        assert lib.gorch_hip_scratch_bytes() == held0
