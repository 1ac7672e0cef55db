"""GPU tests of the tile-packed weight format and the Linear over it.

The format is checked element by element against its definition (fragment
(t, j) of 64 lanes x 8 bf16: lane l holds row 16t + l%16, columns 32j +
8(l//16) .. +8, zero outside the weight), restated here with numpy index
arithmetic; the packed Linear is held to the same bars as the row-major one:
1e-3 of RMS against the oracle (gorch's widen + f32 sgemm) and 1e-4 of RMS
against an f64 product of the same bf16 weights.
"""
import numpy as np
import pytest
import torch

import oracle as orc
from gorch_amd import synthetic as syn
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def dev(a):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def packed_reference(W):
    N, K = W.shape
    nt, nks = -(-N // 16), -(-K // 32)
    Wz = np.zeros((nt * 16, nks * 32), dtype=np.uint16)
    Wz[:N, :K] = W
    t, j, l, e = np.meshgrid(np.arange(nt), np.arange(nks), np.arange(64), np.arange(8), indexing="ij")
    return Wz[16 * t + l % 16, 32 * j + 8 * (l // 16) + e].reshape(-1)


@pytest.mark.parametrize("N,K", [(1, 8), (16, 32), (17, 40), (100, 768), (4800, 1600), (50257, 768)])
def test_pack_layout(gpu, N, K):
    rng = np.random.default_rng(N + K)
    W = rng.integers(0, 1 << 16, size=(N, K), dtype=np.uint32).astype(np.uint16)
    Wp = gpu.pack_bf16(dev(W))
    assert Wp.numel() * 2 == gpu.lib().gorch_hip_packed_bf16_bytes(N, K)
    assert np.array_equal(host(Wp).view(np.uint16), packed_reference(W))


def run_packed(hip, x, W, b=None, residual=None, epilogue=0):
    M, N = x.shape[0], W.shape[0]
    Wp = hip.pack_bf16(dev(W))
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    res = None if residual is None else dev(residual)
    if res is not None:
        y = res
    hip.linear_bf16_packed(dev(x), Wp, N, None if b is None else dev(b), y, residual=res, epilogue=epilogue)
    return host(y)


@pytest.mark.parametrize("K,N", [(768, 3072), (768, 50257), (1600, 4800), (1600, 6400), (768, 2304),
                                 (3072, 768), (6400, 1600), (1600, 1600)])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_packed_decode_shapes(gpu, M, K, N):
    x, W, b = syn.gemv_inputs(M, K, N, seed=M * 11 + K + N)
    got = run_packed(gpu, x, W, b)
    assert rel_err(got, orc.linear(x, W, b)) <= 1e-3
    f64 = x.astype(np.float64) @ orc.bf16_to_f32(W).astype(np.float64).T
    assert rel_err(got, f64) <= 1e-4


@pytest.mark.parametrize("M,N,K", [(1, 1, 8), (3, 7, 40), (16, 65, 128), (2, 33, 2048), (13, 4801, 1600),
                                   (7, 200, 1032), (16, 1000, 1032), (5, 17, 2040), (16, 768, 3072),
                                   (4, 770, 3064), (1, 100, 2056)])
def test_packed_ragged_shapes(gpu, M, N, K):
    rng = np.random.default_rng(M * 1000 + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = syn.bf16_normal(rng, (N, K))
    b = rng.standard_normal(N).astype(np.float32)
    got = run_packed(gpu, x, W, b)
    assert rel_err(got, orc.linear(x, W, b)) <= 1e-3


def test_packed_epilogues_and_determinism(gpu):
    rng = np.random.default_rng(5)
    M, K, N = 4, 768, 3072
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = syn.bf16_normal(rng, (N, K), std=0.05)
    b = rng.standard_normal(N).astype(np.float32) * 0.1
    res = rng.standard_normal((M, N)).astype(np.float32)
    ref_lin = orc.linear(x, W, b)
    assert rel_err(run_packed(gpu, x, W, b, epilogue=gpu.EPI_GELU), orc.gelu(ref_lin)) <= 1e-3
    assert rel_err(run_packed(gpu, x, W, b, residual=res), orc.add(res, ref_lin)) <= 1e-3
    a = run_packed(gpu, x, W, b)
    for _ in range(3):
        assert np.array_equal(a, run_packed(gpu, x, W, b))


@pytest.mark.parametrize("M,N,K", [(2, 16, 4096), (16, 100, 12288), (1, 40, 1024), (5, 2020, 3080)])
def test_packed_k_split(gpu, M, N, K):
    # narrow weights over a long K: K split across blocks, ordered epilogue
    rng = np.random.default_rng(N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = syn.bf16_normal(rng, (N, K))
    b = rng.standard_normal(N).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    got = run_packed(gpu, x, W, b, residual=res)
    assert rel_err(got, orc.add(res, orc.linear(x, W, b))) <= 1e-3


def test_packed_k_split_repeats_and_graph(gpu):
    """The narrow K-split Linear (partials per K slice in the stream's
    scratch, then the ordered epilogue with bias, GELU or the residual):
    repeated calls and graph replays on a stream whose scratch exists before
    capture give identical bits, within 1e-3 of the oracle."""
    rng = np.random.default_rng(21)
    M, K, N = 16, 3072, 768
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = syn.bf16_normal(rng, (N, K), std=0.05)
    b = rng.standard_normal(N).astype(np.float32) * 0.1
    res = rng.standard_normal((M, N)).astype(np.float32)
    ref = orc.gelu(orc.linear(x, W, b))
    first = run_packed(gpu, x, W, b, epilogue=gpu.EPI_GELU)
    assert rel_err(first, ref) <= 1e-3
    for _ in range(4):
        assert np.array_equal(first, run_packed(gpu, x, W, b, epilogue=gpu.EPI_GELU))
    from gorch_amd import hip
    Wp = hip.pack_bf16(torch.from_numpy(W.view(np.int16)).cuda())
    xd, bd, rd = dev(x), dev(b), dev(res)
    y = torch.empty((M, N), device="cuda")
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):   # the stream's scratch and counters exist before capture
        hip.linear_bf16_packed(xd, Wp, N, bd, y, epilogue=gpu.EPI_GELU)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        hip.linear_bf16_packed(xd, Wp, N, bd, y, epilogue=gpu.EPI_GELU)
    for _ in range(3):
        y.zero_()
        g.replay()
        assert np.array_equal(host(y), first)
    y2 = rd.clone()
    hip.linear_bf16_packed(xd, Wp, N, bd, y2, residual=y2)
    assert rel_err(host(y2), orc.add(res, orc.linear(x, W, b))) <= 1e-3


def test_packed_rejects(gpu):
    W = torch.zeros((2048, 4096), dtype=torch.int16, device="cuda")
    Wp = gpu.pack_bf16(W)
    x = torch.zeros((2, 4096), device="cuda")
    y = torch.zeros((2, 2048), device="cuda")
    with pytest.raises(gpu.HipError):   # K above 3072 over a wide weight
        gpu.linear_bf16_packed(x, Wp, 2048, None, y)
    x17 = torch.zeros((17, 32), device="cuda")
    Wp2 = gpu.pack_bf16(torch.zeros((16, 32), dtype=torch.int16, device="cuda"))
    with pytest.raises(gpu.HipError):   # M above 16
        gpu.linear_bf16_packed(x17, Wp2, 16, None, torch.zeros((17, 16), device="cuda"))
