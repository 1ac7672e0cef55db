"""GPU parity of the bf16 codec, the fused bf16 Linear (GEMV/GEMM) and the
matmul_dt family against the CPU oracle, through the C-ABI.

Bars: bf16<->f32 bit-exact; matmul outputs within
1e-3 of RMS(reference) (the reference's |delta| <= tol*RMS metric,
bf16_matmul_metal_test.go:20-48). The kernel is also held to 1e-4 of RMS
against an f64 product of the same bf16 weights, which its hi/lo activation
split keeps with margin.
"""
import numpy as np
import pytest
import torch

import oracle as orc
from gorch_amd import synthetic as syn
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

GEMV_SHAPES = [(768, 3072), (3072, 768), (768, 50257)]


def dev(a):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def run_linear(hip, x, W, b=None, residual=None, epilogue=0):
    M, N = x.shape[0], W.shape[0]
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    res = None if residual is None else dev(residual)
    if res is not None:
        y = res  # in-place residual, as the decode step uses it
    hip.linear_bf16(dev(x), dev(W), None if b is None else dev(b), y, residual=res, epilogue=epilogue)
    return host(y)


def test_codec_widen_exhaustive(gpu):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    out = torch.empty(1 << 16, dtype=torch.float32, device="cuda")
    gpu.bf16_to_f32(dev(h), out)
    assert np.array_equal(host(out).view(np.uint32), orc.bf16_to_f32(h).view(np.uint32))


@pytest.mark.parametrize("n", [1, 7, 8, 1 << 20, (1 << 20) + 3])
def test_codec_narrow_bitexact(gpu, n):
    rng = np.random.default_rng(n)
    bits = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    out = torch.empty(n, dtype=torch.int16, device="cuda")
    gpu.f32_to_bf16(dev(x), out)
    assert np.array_equal(host(out).view(np.uint16), orc.f32_to_bf16(x))


@pytest.mark.parametrize("K,N", GEMV_SHAPES)
@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_microbench_shapes(gpu, M, K, N):
    x, W, b = syn.gemv_inputs(M, K, N, seed=M * 7 + K)
    gpu.reset_dispatch_counts()
    got = run_linear(gpu, x, W, b)
    # the HIP GEMV ran: one launch, or two when K is split across blocks
    # (narrow N, M >= 2: partials, then the epilogue kernel)
    assert gpu.dispatch_counts()["gemv"] in (1, 2)
    ref = orc.linear(x, W, b)
    assert rel_err(got, ref) <= 1e-3
    f64 = x.astype(np.float64) @ orc.bf16_to_f32(W).astype(np.float64).T
    assert rel_err(got, f64) <= 1e-4


@pytest.mark.parametrize("M,N,K", [(1, 1, 8), (3, 7, 40), (16, 65, 128), (5, 16, 3072), (2, 33, 6400),
                                   (16, 6400, 1600), (16, 1600, 6400), (13, 4800, 1600), (17, 100, 96),
                                   (33, 65, 128), (64, 300, 256), (7, 200, 4104), (16, 1000, 1032),
                                   (1, 300, 776), (1, 100, 1280), (1, 50, 4096), (1, 2304, 768), (1, 768, 3072)])
def test_linear_ragged_shapes(gpu, M, N, K):
    rng = np.random.default_rng(M * 1000 + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = syn.bf16_normal(rng, (N, K))
    b = rng.standard_normal(N).astype(np.float32)
    got = run_linear(gpu, x, W, b)
    assert rel_err(got, orc.linear(x, W, b)) <= 1e-3


def test_linear_fused_epilogues(gpu):
    rng = np.random.default_rng(21)
    M, K, N = 4, 768, 3072
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = syn.bf16_normal(rng, (N, K), std=0.05)
    b = rng.standard_normal(N).astype(np.float32) * 0.1
    res = rng.standard_normal((M, N)).astype(np.float32)
    ref_lin = orc.linear(x, W, b)
    got = run_linear(gpu, x, W, b, epilogue=gpu.EPI_GELU)
    assert rel_err(got, orc.gelu(ref_lin)) <= 1e-3
    got = run_linear(gpu, x, W, b, residual=res)
    assert rel_err(got, orc.add(res, ref_lin)) <= 1e-3
    got = run_linear(gpu, x, W, b, residual=res, epilogue=gpu.EPI_GELU)
    assert rel_err(got, orc.add(res, orc.gelu(ref_lin))) <= 1e-3


def test_linear_deterministic(gpu):
    # the cross-wave reduction runs in a fixed order: repeated calls agree bitwise
    x, W, b = syn.gemv_inputs(16, 3072, 768, seed=22)
    a = run_linear(gpu, x, W, b)
    for _ in range(3):
        assert np.array_equal(a, run_linear(gpu, x, W, b))


def test_linear_rejects_bad_arguments(gpu):
    x = torch.zeros((2, 12), device="cuda")
    W = torch.zeros((4, 12), dtype=torch.int16, device="cuda")
    y = torch.zeros((2, 4), device="cuda")
    with pytest.raises(gpu.HipError):          # K % 8 != 0 -> unsupported (CPU path)
        gpu.linear_bf16(x, W, None, y)
    xs = torch.zeros((2, 16), device="cuda")
    Ws = torch.zeros((16, 16), dtype=torch.int16, device="cuda")
    with pytest.raises(gpu.HipError) as e:     # x aliasing y
        gpu.linear_bf16(xs, Ws, None, xs)
    assert e.value.rc == 2


@pytest.mark.parametrize("transA,transB", [(False, True), (False, False), (True, False)])
@pytest.mark.parametrize("aBF16,bBF16", [(False, True), (True, True), (False, False), (True, False)])
def test_matmul_dt_all_layouts(gpu, transA, transB, aBF16, bBF16):
    rng = np.random.default_rng(23)
    M, N, K = 33, 65, 128
    a = rng.standard_normal((K, M) if transA else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if transB else (K, N)).astype(np.float32)
    A = orc.f32_to_bf16(a) if aBF16 else a
    B = orc.f32_to_bf16(b) if bBF16 else b
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    gpu.matmul_dt(dev(A), dev(B), C, M, N, K, transA, transB, aBF16, bBF16)
    assert rel_err(host(C), orc.matmul_dt(A, B, M, N, K, transA, transB)) <= 1e-3
    # against float64 over the operands' stored values: the Linear layout
    # (f32 A, bf16 B stored [N, K]) takes the weight-streaming kernels, whose
    # activations are two bf16 terms (x = hi + lo to ~2^-16: <= 1e-4); every
    # other route splits an f32 operand into three (x = hi + mid + lo to
    # ~2^-25), f32-level error (a two-term split measures ~1e-5 here)
    a64 = (orc.bf16_to_f32(A) if aBF16 else a).astype(np.float64)
    b64 = (orc.bf16_to_f32(B) if bBF16 else b).astype(np.float64)
    ref64 = (a64.T if transA else a64) @ (b64.T if transB else b64)
    linear_route = not transA and transB and not aBF16 and bBF16
    assert rel_err(host(C), ref64) <= (1e-4 if linear_route else 2e-6)


@pytest.mark.parametrize("transA,transB", [(0, 0), (1, 0), (0, 1)])
@pytest.mark.parametrize("aBF16,bBF16", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_batched_matmul_dt_all_layouts(gpu, transA, transB, aBF16, bBF16):
    """Every layout and dtype pair of batchedMatMulDTGrad / batchedMatMulBF16
    (bf16_matmul.go:185-212, :257-304) in one launch, with edges in every
    dimension (M, N not multiples of the 64-wide tile, K not of the 32-wide
    step), against the oracle's per-batch f32 sgemm."""
    rng = np.random.default_rng(25 + 4 * transA + 2 * transB + aBF16)
    B_, M, N, K = 3, 70, 130, 100
    a = rng.standard_normal((B_,) + ((K, M) if transA else (M, K))).astype(np.float32)
    b = rng.standard_normal((B_,) + ((N, K) if transB else (K, N))).astype(np.float32)
    A = orc.f32_to_bf16(a) if aBF16 else a
    Bm = orc.f32_to_bf16(b) if bBF16 else b
    C = torch.empty((B_, M, N), dtype=torch.float32, device="cuda")
    gpu.reset_dispatch_counts()
    gpu.batched_matmul_dt(dev(A), dev(Bm), C, M, N, K, B_, transA, transB, aBF16, bBF16)
    assert gpu.dispatch_counts()["generic_matmul"] == 1
    ref = orc.batched_matmul_dt(A, Bm, B_, M, N, K, bool(transA), bool(transB))
    assert rel_err(host(C), ref) <= 1e-3
    # f32 operands as two bf16 terms each: ~2^-15 per product, far inside
    # what one bf16 rounding of an operand would give (~2^-9)
    if not (aBF16 or bBF16):
        assert rel_err(host(C), ref) <= 2e-4


def test_matmul_dt_double_transpose_unsupported(gpu):
    A = torch.zeros((4, 4), device="cuda")
    with pytest.raises(gpu.HipError) as e:
        gpu.matmul_dt(A, A, torch.zeros((4, 4), device="cuda"), 4, 4, 4, True, True)
    assert e.value.rc == 1


def test_batched_matmul_dt(gpu):
    rng = np.random.default_rng(24)
    B_, M, N, K = 4, 17, 23, 64
    a = rng.standard_normal((B_, M, K)).astype(np.float32)
    for transB in (True, False):
        b = orc.f32_to_bf16(rng.standard_normal((B_, N, K) if transB else (B_, K, N)).astype(np.float32))
        C = torch.empty((B_, M, N), dtype=torch.float32, device="cuda")
        gpu.batched_matmul_dt(dev(a), dev(b), C, M, N, K, B_, False, transB, False, True)
        ref = orc.batched_matmul_dt(a, b, B_, M, N, K, False, transB)
        assert rel_err(host(C), ref) <= 1e-3


def test_matmul_probe(gpu, known_answers):
    # the reference's once-per-process numeric probe (bf16_matmul.go:63-112)
    n = 16
    i = np.arange(n * n)
    af = ((i % 7) * 0.25 - 0.75).astype(np.float32).reshape(n, n)
    bff = (((i * 5) % 11) * 0.125 - 0.625).astype(np.float32).reshape(n, n)
    ref = orc.matmul_dt(af, bff, n, n, n)
    for B, bb in ((orc.f32_to_bf16(bff), True), (bff, False)):
        C = torch.empty((n, n), dtype=torch.float32, device="cuda")
        gpu.matmul_dt(dev(orc.f32_to_bf16(af)), dev(B), C, n, n, n, False, False, True, bb)
        assert np.max(np.abs(host(C) - ref)) <= known_answers["bf16_matmul_probe"]["tol_abs"]


@pytest.mark.parametrize("N", [2304, 3072])
def test_prefill_gemm_config(gpu, N):
    """M=512 x K=768 x N (fused QKV 2304 / MLP-up 3072),
    f32 N(0,1) activations, bf16 N(0,0.02) weights, f32 out."""
    M, K = 512, 768
    x, W, b = syn.gemv_inputs(M, K, N, seed=N)
    gpu.reset_dispatch_counts()
    got = run_linear(gpu, x, W, b)                         # f32-accurate activations
    assert gpu.dispatch_counts()["gemm"] == 1
    ref = orc.linear(x, W, b)
    assert rel_err(got, ref) <= 1e-3
    # bf16-rounded activations on the matrix cores (the dtyped MPSGraph path):
    # 1e-3 against the oracle on bf16-rounded A, 5e-2 against f32 A
    # (bf16_ops_test.go:22-26).
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    gpu.linear_bf16(dev(x), dev(W), dev(b), y, act_bf16=True)
    got16 = host(y)
    xr = orc.bf16_to_f32(orc.f32_to_bf16(x))
    assert rel_err(got16, orc.linear(xr, W, b)) <= 1e-3
    assert rel_err(got16, ref) <= 5e-2


@pytest.mark.parametrize("M,N,K", [(17, 50257, 768), (100, 1600, 6400), (256, 4800, 1600), (8192, 64, 64),
                                   (33, 8, 8)])
def test_gemm_shapes(gpu, M, N, K):
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = syn.bf16_normal(rng, (N, K))
    b = rng.standard_normal(N).astype(np.float32) * 0.1
    res = rng.standard_normal((M, N)).astype(np.float32)
    got = run_linear(gpu, x, W, b, residual=res, epilogue=gpu.EPI_GELU)
    assert rel_err(got, orc.add(res, orc.gelu(orc.linear(x, W, b)))) <= 1e-3
