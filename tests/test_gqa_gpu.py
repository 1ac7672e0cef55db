"""GPU parity of RoPE (nn/rope.go), grouped-query attention and the GQA
cached-decode module (nn/gqa.go:213-363) against the CPU oracle.

Bars: RoPE rotation bit-exact given the same tables (no FMA contraction on
either side); device-computed tables within 2 f32 ulps of the oracle's
(libm vs device cos/sin of the same f64 angle); GQA outputs within 1e-3 of
RMS, cache rows within 1e-4.
"""
import numpy as np
import pytest
import torch

import oracle as orc
from gorch_amd import synthetic as syn
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("hd,max_seq,base", [(64, 256, 10000.0), (128, 4096, 1000000.0)])
def test_rope_tables(gpu, hd, max_seq, base):
    c, s = gpu.rope_tables(hd, max_seq, base)
    rc, rs = orc.rope_tables(hd, max_seq, base)
    for got, ref in ((host(c), rc), (host(s), rs)):
        ulps = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        assert ulps.max() <= 2


@pytest.mark.parametrize("neox", [False, True])
def test_rope_apply_bitexact(gpu, neox):
    rc, rs = orc.rope_tables(64, 64, 10000.0)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 10, 64)).astype(np.float32)
    for sign in (1.0, -1.0):
        y = torch.empty((3, 10, 64), device="cuda")
        gpu.rope_apply(dev(x), y, dev(rc), dev(rs), start_pos=7, neox=neox, sign=sign)
        assert np.array_equal(host(y), orc.rope_apply(x, rc, rs, 7, neox, sign))
    xd = dev(x)
    gpu.rope_apply(xd, xd, dev(rc), dev(rs), start_pos=0, neox=neox)      # in place, pos 0 = identity
    assert np.array_equal(host(xd)[:, :1], x[:, :1])


def test_rope_rejects_overflow(gpu):
    c, s = gpu.rope_tables(64, 8, 10000.0)
    x = torch.zeros((1, 4, 64), device="cuda")
    with pytest.raises(gpu.HipError):
        gpu.rope_apply(x, x, c, s, start_pos=6)


@pytest.mark.parametrize("batch,nq,nkv,S,pos,hd", [
    (1, 8, 2, 1, 30, 32), (1, 8, 8, 4, 12, 32), (1, 16, 8, 3, 0, 32),
    # Qwen3-0.6B heads (16 query / 8 KV heads of 128): the 8-wave one-pass
    # kernel (cache 129..256 rows), the online-softmax long-cache kernel
    # (fewer than 128 (head, row) blocks), and the 16-wave two-pass kernel
    # (128..1023 blocks over a cache longer than 256 rows)
    (1, 16, 8, 1, 200, 128), (1, 16, 8, 1, 500, 128), (1, 16, 8, 1, 1300, 128),
    (2, 16, 8, 3, 300, 128), (8, 16, 8, 1, 400, 128), (8, 8, 2, 2, 290, 64)])
def test_gqa_attention_vs_f64(gpu, batch, nq, nkv, S, pos, hd):
    import math
    import scipy.special
    rng = np.random.default_rng(nq + S + pos + batch)
    T = pos + S
    cap = T + 2
    q = rng.standard_normal((batch * S, nq * hd)).astype(np.float32)
    kc = rng.standard_normal((batch, cap, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((batch, cap, nkv * hd)).astype(np.float32)
    out = torch.empty((batch * S, nq * hd), device="cuda")
    gpu.gqa_attention_cached(dev(q), dev(kc), dev(vc), out, batch, S, pos, nq, nkv, hd, cap)
    got = host(out)
    g = nq // nkv
    for b in range(batch):
        qb, gb = q[b * S:(b + 1) * S], got[b * S:(b + 1) * S]
        for h in range(nq):
            kk = kc[b, :T, (h // g) * hd:(h // g + 1) * hd].astype(np.float64)
            vv = vc[b, :T, (h // g) * hd:(h // g + 1) * hd].astype(np.float64)
            s = qb[:, h * hd:(h + 1) * hd].astype(np.float64) @ kk.T / math.sqrt(hd)
            for i in range(S):
                s[i, pos + i + 1:] = -np.inf
            ref = scipy.special.softmax(s, axis=1) @ vv
            assert np.max(np.abs(gb[:, h * hd:(h + 1) * hd] - ref)) < 1e-5, (b, h)


def _run(gpu, w, chunks, cap=24):
    kvdim = w["num_kv"] * w["head_dim"]
    ow = dict(w)
    m = gpu.GQA(w)
    if w.get("rope"):  # the oracle uses the GPU's tables so the check isolates the module
        ow["rope_cos"], ow["rope_sin"] = host(m.t["rope_cos"]), host(m.t["rope_sin"])
    kc_d = torch.zeros((cap, kvdim), device="cuda")
    vc_d = torch.zeros((cap, kvdim), device="cuda")
    kc = np.zeros((cap, kvdim), np.float32)
    vc = np.zeros((cap, kvdim), np.float32)
    pos = 0
    for x in chunks:
        got = host(m.forward_cached(dev(x), kc_d, vc_d, pos))
        ref = orc.gqa_forward_cached(ow, kc, vc, pos, x)
        assert rel_err(got, ref) <= 1e-3
        pos += x.shape[0]
    assert rel_err(host(kc_d)[:pos], kc[:pos]) <= 1e-4
    assert rel_err(host(vc_d)[:pos], vc[:pos]) <= 1e-4


@pytest.mark.parametrize("qk_norm,rope,bias", [(True, True, True), (False, False, False), (False, True, False)])
def test_gqa_module_vs_oracle(gpu, qk_norm, rope, bias):
    w = syn.gqa_weights(seed=5, qk_norm=qk_norm, rope=rope, bias=bias)
    rng = np.random.default_rng(6)
    chunks = [rng.standard_normal((n, w["dim"])).astype(np.float32) for n in (5, 1, 1, 3)]
    _run(gpu, w, chunks)


@pytest.mark.parametrize("hd,qk_norm", [(16, True), (32, False), (40, True)])
def test_gqa_module_neox_rope(gpu, hd, qk_norm):
    # interleaved (GPT-NeoX) pairs through the fused per-head norm + RoPE
    # kernel (head dims that are multiples of 8); RoPE tables from the GPU
    w = syn.gqa_weights(head_dim=hd, seed=9, qk_norm=qk_norm, rope=True, bias=False)
    w["rope_neox"] = 1
    rng = np.random.default_rng(10)
    chunks = [rng.standard_normal((n, w["dim"])).astype(np.float32) for n in (4, 1, 2)]
    _run(gpu, w, chunks)


def test_gqa_module_unfused_head(gpu):
    # head dim 20 (not a multiple of 8): per-head norm and RoPE as separate
    # kernels
    w = syn.gqa_weights(dim=40, num_q=4, num_kv=2, head_dim=20, seed=12, qk_norm=True, rope=True, bias=False)
    rng = np.random.default_rng(13)
    chunks = [rng.standard_normal((n, w["dim"])).astype(np.float32) for n in (3, 1)]
    _run(gpu, w, chunks)


def test_gqa_qwen3_shaped_decode(gpu):
    """Qwen3-0.6B attention shape: d 1024, 16 query
    heads x 128, 8 KV heads, qk-norm, RoPE base 1e6; 32-token prefill then
    two decode steps."""
    w = syn.gqa_weights(dim=1024, num_q=16, num_kv=8, head_dim=128, max_seq=128, seed=7, bias=False,
                        qk_norm=True, rope=True, base=1000000.0)
    rng = np.random.default_rng(8)
    chunks = [rng.standard_normal((n, 1024)).astype(np.float32) for n in (32, 1, 1)]
    _run(gpu, w, chunks, cap=40)


@pytest.mark.parametrize("kw,prefill,qk_norm,neox", [
    # Qwen3-0.6B attention (16 query / 8 KV heads of 128) over a 290-row
    # prefill, then one-row steps: 10 key chunks of 32 per head
    (dict(dim=1024, num_q=16, num_kv=8, head_dim=128, base=1000000.0), 290, True, 0),
    # heads of 64 over 600 rows: 10 chunks of 64 keys per head
    (dict(dim=256, num_q=4, num_kv=2, head_dim=64, base=10000.0), 600, True, 0),
    # interleaved (NeoX) pairs, and RoPE without the per-head norm
    (dict(dim=512, num_q=4, num_kv=2, head_dim=128, base=10000.0), 70, True, 1),
    (dict(dim=256, num_q=4, num_kv=4, head_dim=64, base=10000.0), 130, False, 0),
    # q/k/v and output biases, and query width (8 x 64) above the model width
    (dict(dim=256, num_q=8, num_kv=2, head_dim=64, base=10000.0, bias=True), 100, True, 0)])
def test_gqa_module_key_split_steps(gpu, kw, prefill, qk_norm, neox):
    """One-row steps over few heads and a cache longer than one key chunk:
    the key-split attention (per-chunk max, weight sum and weighted values,
    merged per head by the kernel that also adds the output projection and
    its bias) with the q/k RMSNorm and RoPE
    applied inside it (the new K row written to the cache by the kernel);
    outputs within 1e-3 of the oracle, cache rows within 1e-4."""
    kw = dict(kw)
    bias = kw.pop("bias", False)
    w = syn.gqa_weights(max_seq=prefill + 8, seed=14, bias=bias, qk_norm=qk_norm, rope=True, **kw)
    w["rope_neox"] = neox
    rng = np.random.default_rng(15)
    chunks = [rng.standard_normal((n, w["dim"])).astype(np.float32) for n in (prefill, 1, 1, 1)]
    _run(gpu, w, chunks, cap=prefill + 4)
