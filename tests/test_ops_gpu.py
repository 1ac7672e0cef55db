"""GPU parity of the decode-step ops against the CPU oracle (C-ABI calls).

Tolerances: exact f32 adds and row copies are bit-exact; LayerNorm/RMSNorm
(f64 statistics on both sides) within 1e-5; transcendental ops (GELU,
SiLU, SwiGLU, softmax) within 1e-6 relative-to-scale (libm vs device
expf/tanhf); attention within 1e-5 (summation order). The reference's own
GPU-vs-CPU gates are 1e-4 for elementwise and 1e-3 for reductions and
softmax (silu_metal_test.go:19-21, softmax_metal_test.go:11-19).
"""
import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("M,N", [(1, 768), (5, 1600), (3, 7)])
def test_layernorm(gpu, M, N):
    rng = np.random.default_rng(M + N)
    x = (rng.standard_normal((M, N)) * 2 + 0.5).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(N)).astype(np.float32)
    b = (0.1 * rng.standard_normal(N)).astype(np.float32)
    y = torch.empty((M, N), device="cuda")
    gpu.layernorm(dev(x), dev(g), dev(b), y)
    assert np.max(np.abs(host(y) - orc.layernorm(x, g, b))) < 1e-5


def test_rmsnorm(gpu, known_answers):
    ka = known_answers["rmsnorm_spec"]
    x = np.array(ka["x"], np.float32)
    y = torch.empty(x.shape, device="cuda")
    gpu.rmsnorm(dev(x), dev(np.ones(4, np.float32)), y, eps=0.0)
    assert np.max(np.abs(host(y) - np.array(ka["want"]))) <= ka["tol"]
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 1024)).astype(np.float32)
    g = rng.standard_normal(1024).astype(np.float32)
    y = torch.empty(x.shape, device="cuda")
    gpu.rmsnorm(dev(x), dev(g), y)
    assert np.max(np.abs(host(y) - orc.rmsnorm(x, g))) < 1e-5


def test_exact_elementwise(gpu):
    rng = np.random.default_rng(4)
    a = rng.standard_normal(100003).astype(np.float32)
    b = rng.standard_normal(100003).astype(np.float32)
    c = torch.empty_like(dev(a))
    gpu.add(dev(a), dev(b), c)
    assert np.array_equal(host(c), orc.add(a, b))
    x = rng.standard_normal((7, 300)).astype(np.float32)
    bias = rng.standard_normal(300).astype(np.float32)
    xd = dev(x)
    gpu.bias_add(xd, dev(bias))
    assert np.array_equal(host(xd), x + bias)
    w = rng.standard_normal((50, 64)).astype(np.float32)
    ids = np.array([3, 0, 49, 3, 17], np.int32)
    out = torch.empty((5, 64), device="cuda")
    gpu.embedding(dev(w), dev(ids), out)
    assert np.array_equal(host(out), orc.embedding_lookup(w, ids))


def test_activations(gpu):
    x = np.linspace(-15, 15, 200001, dtype=np.float32)
    v = np.cos(x).astype(np.float32)
    y = torch.empty_like(dev(x))
    gpu.gelu(dev(x), y)
    assert np.max(np.abs(host(y) - orc.gelu(x))) < 2e-6 * 15
    gpu.silu(dev(x), y)
    assert np.max(np.abs(host(y) - orc.silu(x))) < 2e-6 * 15
    gpu.swiglu(dev(x), dev(v), y)
    assert np.max(np.abs(host(y) - orc.swiglu(x, v))) < 2e-6 * 15


@pytest.mark.parametrize("M,N", [(1, 1024), (3, 128), (5, 2048)])
def test_add_rmsnorm(gpu, M, N):
    # a decoder block's residual add then RMSNorm (model/qwen/block.go:74-76)
    rng = np.random.default_rng(M + N)
    x = rng.standard_normal((M, N)).astype(np.float32)
    b = rng.standard_normal((M, N)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(N)).astype(np.float32)
    s = torch.empty((M, N), device="cuda")
    y = torch.empty((M, N), device="cuda")
    gpu.add_rmsnorm(dev(x), dev(b), dev(g), s, y)
    ref_s = orc.add(x, b)
    assert np.array_equal(host(s), ref_s)
    assert np.max(np.abs(host(y) - orc.rmsnorm(ref_s, g))) < 1e-5


@pytest.mark.parametrize("batch,new_seq,pos,heads,hd", [(1, 1, 0, 12, 64), (1, 1, 95, 12, 64),
                                                        (2, 5, 40, 12, 64), (3, 1, 767, 25, 64),
                                                        (1, 32, 0, 12, 64), (2, 3, 9, 4, 80),
                                                        (2, 5, 300, 4, 128), (1, 3, 700, 2, 128),
                                                        (64, 1, 400, 20, 64), (2, 1, 1300, 3, 64),
                                                        (2, 3, 150, 4, 128), (1, 1, 250, 16, 128),
                                                        # 128..1023 (head, row) blocks over caches longer
                                                        # than 256 rows: the 16-wave two-pass kernel that
                                                        # the GPT-2 XL batch-16 step runs (25 heads x 16)
                                                        (16, 1, 511, 25, 64), (16, 1, 767, 25, 64),
                                                        (8, 1, 600, 16, 128), (4, 1, 300, 8, 80),
                                                        # a short cache in a longer capacity, causal new
                                                        # rows, 900 rows
                                                        (12, 1, 255, 25, 64), (2, 5, 600, 25, 64),
                                                        (16, 1, 900, 25, 64),
                                                        # past 16384 visible rows (no LDS score row):
                                                        # the online-softmax long-cache kernel
                                                        (1, 1, 16400, 2, 64), (2, 1, 17000, 4, 128)])
def test_attention_cached(gpu, batch, new_seq, pos, heads, hd):
    rng = np.random.default_rng(pos + heads)
    d = heads * hd
    max_seq = pos + new_seq + 3
    q = rng.standard_normal((batch * new_seq, d)).astype(np.float32)
    kc = rng.standard_normal((batch, max_seq, d)).astype(np.float32)
    vc = rng.standard_normal((batch, max_seq, d)).astype(np.float32)
    out = torch.empty((batch * new_seq, d), device="cuda")
    gpu.attention_cached(dev(q), dev(kc), dev(vc), out, batch, new_seq, pos, heads, hd, max_seq)
    got = host(out)
    for b in range(batch):
        T = pos + new_seq
        ref = orc.attention_cached(q[b * new_seq:(b + 1) * new_seq], kc[b, :T], vc[b, :T], pos, heads)
        assert np.max(np.abs(got[b * new_seq:(b + 1) * new_seq] - ref)) < 1e-5


@pytest.mark.parametrize("batch,new_seq,pos,heads,hd,causal", [
    (1, 32, 0, 12, 64, True), (2, 100, 0, 4, 64, True), (1, 257, 37, 3, 64, True), (3, 64, 5, 2, 128, True),
    (1, 130, 0, 2, 64, False), (2, 48, 20, 2, 128, False), (16, 64, 0, 2, 64, True)])
def test_attention_prefill_rows(gpu, batch, new_seq, pos, heads, hd, causal):
    # many new rows per sequence: the matrix-core (flash) kernel; held to
    # 1e-4 absolute (the reference bounds cached vs one-shot logits at 1e-3)
    rng = np.random.default_rng(new_seq * 7 + pos + hd)
    d = heads * hd
    max_seq = pos + new_seq + 5
    q = rng.standard_normal((batch * new_seq, d)).astype(np.float32)
    kc = rng.standard_normal((batch, max_seq, d)).astype(np.float32)
    vc = rng.standard_normal((batch, max_seq, d)).astype(np.float32)
    out = torch.empty((batch * new_seq, d), device="cuda")
    gpu.reset_dispatch_counts()
    gpu.attention_cached(dev(q), dev(kc), dev(vc), out, batch, new_seq, pos, heads, hd, max_seq, causal=causal)
    assert gpu.dispatch_counts()["attention"] == 1
    got = host(out)
    for b in range(batch):
        T = pos + new_seq
        ref = orc.attention_cached(q[b * new_seq:(b + 1) * new_seq], kc[b, :T], vc[b, :T], pos, heads,
                                   causal=causal)
        assert np.max(np.abs(got[b * new_seq:(b + 1) * new_seq] - ref)) < 1e-4


def test_attention_noncausal(gpu):
    rng = np.random.default_rng(5)
    heads, hd, pos, n = 4, 64, 6, 3
    d = heads * hd
    q = rng.standard_normal((n, d)).astype(np.float32)
    kc = rng.standard_normal((1, pos + n, d)).astype(np.float32)
    vc = rng.standard_normal((1, pos + n, d)).astype(np.float32)
    out = torch.empty((n, d), device="cuda")
    gpu.attention_cached(dev(q), dev(kc), dev(vc), out, 1, n, pos, heads, hd, pos + n, causal=False)
    ref = orc.attention_cached(q, kc[0], vc[0], pos, heads, causal=False)
    assert np.max(np.abs(host(out) - ref)) < 1e-5


def test_attention_noncausal_long(gpu):
    # a long cache (the online-softmax kernel) without the causal mask: every
    # new row sees all pos + n keys
    rng = np.random.default_rng(11)
    heads, hd, pos, n = 3, 64, 500, 4
    d = heads * hd
    q = rng.standard_normal((n, d)).astype(np.float32)
    kc = rng.standard_normal((1, pos + n + 2, d)).astype(np.float32)
    vc = rng.standard_normal((1, pos + n + 2, d)).astype(np.float32)
    out = torch.empty((n, d), device="cuda")
    gpu.attention_cached(dev(q), dev(kc), dev(vc), out, 1, n, pos, heads, hd, pos + n + 2, causal=False)
    ref = orc.attention_cached(q, kc[0, :pos + n], vc[0, :pos + n], pos, heads, causal=False)
    assert np.max(np.abs(host(out) - ref)) < 1e-5


def test_attention_rejects_overflow(gpu):
    z = torch.zeros((1, 64), device="cuda")
    with pytest.raises(gpu.HipError):
        gpu.attention_cached(z, z, z, z, 1, 1, 1, 1, 64, 1)


@pytest.mark.parametrize("rows,cols,q_seq", [(12, 33, 1), (36, 40, 3), (5, 1000, 5)])
def test_causal_softmax(gpu, rows, cols, q_seq):
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 3
    y = torch.empty((rows, cols), device="cuda")
    gpu.causal_softmax(dev(x), y, q_seq, 0.125)
    ref = orc.causal_softmax(x, q_seq, 0.125)
    got = host(y)
    assert np.max(np.abs(got - ref)) < 1e-6
    assert np.array_equal(got == 0, ref == 0)     # masked entries exactly 0


def test_softmax_rows(gpu):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((9, 513)).astype(np.float32) * 5
    xd = dev(x)
    gpu.softmax_rows(xd)
    assert np.max(np.abs(host(xd) - orc.softmax_inplace(x))) < 1e-6


def test_argmax(gpu):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 50257)).astype(np.float32)
    x[1, 100] = x[1, 40000] = 9.0             # tie: the first index wins
    x[2, 0] = np.nan                          # NaN first -> 0 (reference loop)
    x[3, 7] = np.nan                          # NaN elsewhere is never chosen
    x[4, :] = -np.inf                         # all -inf -> 0
    x[5, 50256] = 12.0                        # last element
    out = torch.empty(6, dtype=torch.int32, device="cuda")
    gpu.argmax(dev(x), out)
    assert list(host(out)) == [orc.argmax(r) for r in x]
