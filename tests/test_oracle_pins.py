"""Pins the CPU oracle (oracle/liborc.so) independently of its own formulas.

Each function of the oracle is checked against at least one of: the
reference's own known answers (tests/golden/reference_known_answers.json,
transcribed from gorch's *_test.go files), an independent library routine
(torch's bf16 rounding and activations, scipy's softmax, numpy f64 linear
algebra), exhaustive enumeration, or an invariant the reference's tests
state (cached == uncached, causality, routing weights summing to 1).
"""
import math

import numpy as np
import pytest
import scipy.special
import torch

import oracle as orc
from gorch_amd import bf16 as hb
from gorch_amd import synthetic as syn


# ------------------------------------------------------------------ A1 codec

def test_bf16_widen_narrow_exhaustive():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = orc.bf16_to_f32(h)
    # widening is the top half of an f32 (tensor.go:97-99)
    assert np.array_equal(f.view(np.uint32), h.astype(np.uint32) << 16)
    back = orc.f32_to_bf16(f)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], h[~nan])           # exact for every finite/inf bf16
    assert np.array_equal(back[nan], h[nan] | 0x40)       # NaN: quiet bit forced


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    # add exact halfway cases (low half 0x8000) at both parities
    half = (rng.integers(0, 1 << 16, size=4096, dtype=np.uint32) << 16) | 0x8000
    bits = np.concatenate([bits, half])
    x = bits.view(np.float32)
    ok = ~np.isnan(x)
    ours = orc.f32_to_bf16(x)[ok]
    ref = torch.from_numpy(x[ok].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_bf16_known_answers(known_answers):
    ka = known_answers
    for v in ka["bf16_roundtrip_exact"]["inputs"]:
        exact = np.array([v], np.float32).view(np.uint32) & np.uint32(0xFFFF0000)
        exact = exact.view(np.float32)
        assert orc.bf16_to_f32(orc.f32_to_bf16(exact))[0] == exact[0]
    for v in ka["bf16_roundtrip_approx"]["inputs"]:
        got = orc.bf16_to_f32(orc.f32_to_bf16(np.array([v], np.float32)))[0]
        assert abs(float(got) - float(np.float32(v))) / abs(float(np.float32(v))) <= ka["bf16_roundtrip_approx"]["max_rel"]
    for s in ka["bf16_special"]["inputs"]:
        v = np.array([float(s)], np.float32)
        assert orc.bf16_to_f32(orc.f32_to_bf16(v))[0] == v[0]
    ints = np.array(ka["bf16_integers"]["inputs"], np.float32)
    assert np.array_equal(orc.bf16_to_f32(orc.f32_to_bf16(ints)), ints)
    sv = np.array(ka["bf16_safetensors_values"]["inputs"], np.float32)
    rt = orc.bf16_to_f32(orc.f32_to_bf16(sv))
    assert list(rt == sv) == ka["bf16_safetensors_values"]["representable"]


def test_product_host_codec_matches_oracle():
    rng = np.random.default_rng(2)
    x = rng.integers(0, 1 << 32, size=1 << 18, dtype=np.uint64).astype(np.uint32).view(np.float32)
    assert np.array_equal(hb.f32_to_bf16(x), orc.f32_to_bf16(x))
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(hb.bf16_to_f32(h).view(np.uint32), orc.bf16_to_f32(h).view(np.uint32))


# ------------------------------------------------------------------ matmul

@pytest.mark.parametrize("transA,transB", [(False, True), (False, False), (True, False)])
@pytest.mark.parametrize("aBF16,bBF16", [(False, True), (True, True), (False, False)])
def test_matmul_dt_vs_f64(transA, transB, aBF16, bBF16):
    rng = np.random.default_rng(3)
    M, N, K = 33, 65, 128   # bf16_matmul_metal_test.go parity shape
    a = rng.standard_normal((K, M) if transA else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if transB else (K, N)).astype(np.float32)
    A = orc.f32_to_bf16(a) if aBF16 else a
    B = orc.f32_to_bf16(b) if bBF16 else b
    got = orc.matmul_dt(A, B, M, N, K, transA, transB)
    af = (orc.bf16_to_f32(A) if aBF16 else a).astype(np.float64)
    bf = (orc.bf16_to_f32(B) if bBF16 else b).astype(np.float64)
    ref = (af.T if transA else af) @ (bf.T if transB else bf)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.sqrt(K) * np.max(np.abs(ref))


def test_matmul_rejects_double_transpose():
    with pytest.raises(ValueError):
        orc.matmul_dt(np.zeros((4, 4), np.float32), np.zeros((4, 4), np.float32), 4, 4, 4, True, True)


def test_matmul_probe_inputs(known_answers):
    n = known_answers["bf16_matmul_probe"]["n"]
    i = np.arange(n * n)
    af = ((i % 7) * 0.25 - 0.75).astype(np.float32).reshape(n, n)
    bff = (((i * 5) % 11) * 0.125 - 0.625).astype(np.float32).reshape(n, n)
    ref = af.astype(np.float64) @ bff.astype(np.float64)  # exact in bf16 (multiples of 1/8)
    got = orc.matmul_dt(orc.f32_to_bf16(af), orc.f32_to_bf16(bff), n, n, n)
    assert np.max(np.abs(got - ref)) <= known_answers["bf16_matmul_probe"]["tol_abs"]
    got2 = orc.matmul_dt(orc.f32_to_bf16(af), bff, n, n, n)
    assert np.max(np.abs(got2 - ref)) <= known_answers["bf16_matmul_probe"]["tol_abs"]


def test_batched_matmul_vs_f64():
    rng = np.random.default_rng(4)
    B_, M, N, K = 4, 17, 23, 64    # bf16_matmul_metal_test.go batched shape
    a = rng.standard_normal((B_, M, K)).astype(np.float32)
    b = orc.f32_to_bf16(rng.standard_normal((B_, N, K)).astype(np.float32))
    got = orc.batched_matmul_dt(a, b, B_, M, N, K, False, True)
    ref = np.einsum("bmk,bnk->bmn", a.astype(np.float64), orc.bf16_to_f32(b).astype(np.float64))
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_linear_bias_and_widen_modes():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((5, 16)).astype(np.float32)
    W = orc.f32_to_bf16(rng.standard_normal((7, 16)).astype(np.float32))
    b = rng.standard_normal(7).astype(np.float32)
    ref = x.astype(np.float64) @ orc.bf16_to_f32(W).astype(np.float64).T + b
    y1 = orc.linear(x, W, b)
    orc.set_widen_per_call(False)
    try:
        y2 = orc.linear(x, W, b)
    finally:
        orc.set_widen_per_call(True)
    assert np.array_equal(y1, y2)
    assert np.max(np.abs(y1 - ref)) < 1e-5


# ------------------------------------------------------------------ row ops

def test_layernorm_closed_form():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((9, 768)) * 3 + 1.5).astype(np.float32)
    g = rng.standard_normal(768).astype(np.float32)
    b = rng.standard_normal(768).astype(np.float32)
    y = orc.layernorm(x, g, b)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * g + b
    assert np.max(np.abs(y - ref)) < 2e-5
    y1 = orc.layernorm(x, np.ones(768, np.float32), np.zeros(768, np.float32))
    assert np.allclose(y1.mean(1), 0, atol=1e-5) and np.allclose(y1.var(1), 1, atol=1e-3)


def test_activations_vs_torch():
    x = np.linspace(-12, 12, 100001, dtype=np.float32)
    t = torch.from_numpy(x).double()
    assert np.max(np.abs(orc.gelu(x) - torch.nn.functional.gelu(t, approximate="tanh").numpy())) < 2e-6 * 12
    assert np.max(np.abs(orc.sigmoid(x) - torch.sigmoid(t).numpy())) < 1e-6
    assert np.max(np.abs(orc.silu(x) - torch.nn.functional.silu(t).numpy())) < 1e-5
    v = np.cos(x).astype(np.float32)
    ref = (torch.nn.functional.silu(t) * torch.from_numpy(v).double()).numpy()
    assert np.max(np.abs(orc.swiglu(x, v) - ref)) < 1e-5
    assert orc.gelu(np.zeros(1, np.float32))[0] == 0.0


def test_softmax_vs_scipy():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((6, 97)) * 4).astype(np.float32)
    y = orc.softmax_inplace(x)
    assert np.max(np.abs(y - scipy.special.softmax(x.astype(np.float64), axis=1))) < 1e-6
    assert np.allclose(y.sum(1), 1, atol=1e-6)


def test_causal_softmax_vs_composed_chain():
    rng = np.random.default_rng(8)
    q_seq, cols, heads = 5, 12, 3
    x = rng.standard_normal((heads * q_seq, cols)).astype(np.float32)
    scale = 0.37
    y = orc.causal_softmax(x, q_seq, scale)
    ref = np.zeros_like(y, dtype=np.float64)
    for r in range(heads * q_seq):
        limit = r % q_seq + cols - q_seq
        s = x[r].astype(np.float64) * scale
        s[limit + 1:] = -np.inf
        ref[r] = scipy.special.softmax(s)
        assert np.all(y[r, limit + 1:] == 0.0)          # masked entries exactly 0
    assert np.max(np.abs(y - ref)) < 1e-6


def test_rmsnorm_known_answers(known_answers):
    ka = known_answers["rmsnorm_spec"]
    x = np.array(ka["x"], np.float32)
    y = orc.rmsnorm(x, np.ones(4, np.float32), eps=0.0)
    assert np.max(np.abs(y - np.array(ka["want"]))) <= ka["tol"]
    y2 = orc.rmsnorm(x, np.full(4, 2.0, np.float32), eps=0.0)     # nn/rmsnorm_test.go:36-58
    assert np.array_equal(y2, 2 * y)


def test_rope_invariants():
    hd, S = 64, 40
    c, s = orc.rope_tables(hd, S, 10000.0)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 7, hd)).astype(np.float32)
    for neox in (False, True):
        # independent formulation: complex rotation by pos * base^(-2i/hd)
        y = orc.rope_apply(x, c, s, start_pos=5, neox=neox)
        half = hd // 2
        ia = np.arange(half) * 2 if neox else np.arange(half)
        ib = ia + 1 if neox else ia + half
        inv = np.float32(10000.0) ** (-(2 * np.arange(half)) / hd)
        for si in range(7):
            theta = (5 + si) * inv.astype(np.float64)
            z = (x[:, si, ia] + 1j * x[:, si, ib]) * np.exp(1j * theta)
            assert np.max(np.abs(y[:, si, ia] - z.real)) < 1e-4
            assert np.max(np.abs(y[:, si, ib] - z.imag)) < 1e-4
        # pos-0 identity (nn/rope_test.go:14-40)
        y0 = orc.rope_apply(x[:, :1], c, s, start_pos=0, neox=neox)
        assert np.array_equal(y0, x[:, :1])
        # norm preservation per pair
        assert np.allclose(y[..., ia] ** 2 + y[..., ib] ** 2, x[..., ia] ** 2 + x[..., ib] ** 2, rtol=1e-5)
        # startPos equivalence: rows 2.. of a start-0 apply == start-2 apply of those rows
        full = orc.rope_apply(x, c, s, start_pos=0, neox=neox)
        part = orc.rope_apply(x[:, 2:], c, s, start_pos=2, neox=neox)
        assert np.array_equal(full[:, 2:], part)
        # inverse rotation undoes the forward one
        back = orc.rope_apply(y, c, s, start_pos=5, neox=neox, sign=-1.0)
        assert np.max(np.abs(back - x)) < 1e-5
    assert not np.allclose(orc.rope_apply(x, c, s, 5, False), orc.rope_apply(x, c, s, 5, True))


def test_topk_vs_argsort():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((50, 8)).astype(np.float32)
    vals, idx = orc.topk(x, 2)
    ref = np.argsort(-x, axis=1, kind="stable")[:, :2]
    assert np.array_equal(idx, ref)
    assert np.array_equal(vals, np.take_along_axis(x, ref, 1))


# ------------------------------------------------------------------ GPT

TINY = dict(vocab=64, dim=32, heads=4, layers=2, max_seq=40)


def _np_gpt_forward(w, ids):
    """Independent f64 numpy GPT-2 forward (pre-norm, tanh GELU, causal MHA)."""
    cfg = w["cfg"]
    d, H = cfg["dim"], cfg["heads"]
    hd = d // H
    f = lambda a: hb.bf16_to_f32(a).astype(np.float64) if a.dtype == np.uint16 else a.astype(np.float64)
    n = len(ids)
    x = f(w["wte"])[ids] + f(w["wpe"])[np.arange(n)]

    def ln(v, g, b):
        return (v - v.mean(1, keepdims=True)) / np.sqrt(v.var(1, keepdims=True) + 1e-5) * f(g) + f(b)

    for L in w["layers"]:
        h = ln(x, L["ln1_g"], L["ln1_b"])
        q, k, v = (h @ f(L[a]).T + f(L[b]) for a, b in (("wq", "bq"), ("wk", "bk"), ("wv", "bv")))
        att = np.zeros_like(q)
        for hh in range(H):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = q[:, sl] @ k[:, sl].T / math.sqrt(hd)
            s[np.triu_indices(n, 1)] = -np.inf
            att[:, sl] = scipy.special.softmax(s, axis=1) @ v[:, sl]
        x = x + att @ f(L["wo"]).T + f(L["bo"])
        h = ln(x, L["ln2_g"], L["ln2_b"])
        u = h @ f(L["w1"]).T + f(L["b1"])
        u = 0.5 * u * (1 + np.tanh(0.7978845608 * (u + 0.044715 * u ** 3)))
        x = x + u @ f(L["w2"]).T + f(L["b2"])
    x = ln(x, w["lnf_g"], w["lnf_b"])
    return x @ f(w["wlm"]).T + f(w["blm"])


@pytest.fixture(scope="module")
def tiny():
    w = syn.gpt2_weights(TINY, seed=11, random_affine=True)
    # larger weights so attention is far from uniform and mistakes show
    for L in w["layers"]:
        for key in ("wq", "wk"):
            L[key] = hb.f32_to_bf16(hb.bf16_to_f32(L[key]) * 20)
    return w, orc.GPT(w)


def test_gpt_forward_vs_numpy_f64(tiny):
    w, g = tiny
    ids = syn.prompt_ids(13, TINY["vocab"], seed=12)
    got = g.forward(ids)
    ref = _np_gpt_forward(w, ids)
    assert np.max(np.abs(got - ref)) < 1e-4 * np.max(np.abs(ref)) + 1e-6


def test_gpt_cached_equals_uncached(tiny):
    # nn/kvcache_test.go:53-114: prefill then two steps; logits within 1e-3
    w, g = tiny
    ids = syn.prompt_ids(10, TINY["vocab"], seed=13)
    cache = g.new_cache()
    pre = g.forward_cached(ids[:8], cache)
    assert len(cache) == 8                                       # position advances
    s1 = g.forward_cached(ids[8:9], cache)
    s2 = g.forward_cached(ids[9:10], cache)
    assert len(cache) == 10
    full = g.forward(ids)
    assert np.max(np.abs(pre - full[:8])) < 1e-3
    assert np.max(np.abs(s1[0] - full[8])) < 1e-3
    assert np.max(np.abs(s2[0] - full[9])) < 1e-3


def test_gpt_causality(tiny):
    # nn/kvcache_test.go:147-172: a later token never changes earlier logits
    w, g = tiny
    ids = syn.prompt_ids(9, TINY["vocab"], seed=14)
    a = g.forward(ids)
    ids2 = ids.copy()
    ids2[-1] = (ids2[-1] + 1) % TINY["vocab"]
    b = g.forward(ids2)
    assert np.array_equal(a[:-1], b[:-1])
    assert not np.array_equal(a[-1], b[-1])


def test_gpt_greedy_cached_equals_uncached(tiny):
    # model/generate_test.go:107-126: greedy cached tokens == uncached tokens
    w, g = tiny
    prompt = syn.prompt_ids(5, TINY["vocab"], seed=15)
    toks, _, _ = g.generate_cached(prompt, 12)
    seq = list(prompt)
    for _ in range(12):
        seq.append(int(np.argmax(g.forward(np.array(seq, np.int32))[-1])))
    assert list(toks) == seq


def test_gpt_generate_stops_at_max_seq(tiny):
    # model/generate.go:119-124: no step forward once the cache is full
    w, g = tiny
    prompt = syn.prompt_ids(TINY["max_seq"] - 2, TINY["vocab"], seed=16)
    toks, _, _ = g.generate_cached(prompt, 10)
    assert len(toks) == TINY["max_seq"] + 1


def test_gpt_generate_stop_token(tiny):
    # model/generate.go:116-118 against the uncached greedy sequence built by
    # argmax over full forwards: generation ends at the first occurrence of
    # the stop token, which is not kept; a token never chosen changes nothing
    w, g = tiny
    prompt = syn.prompt_ids(5, TINY["vocab"], seed=17)
    seq = list(prompt)
    for _ in range(12):
        seq.append(int(np.argmax(g.forward(np.array(seq, np.int32))[-1])))
    new = seq[len(prompt):]
    stop = new[4]
    first = new.index(stop)
    toks, _, _ = g.generate_cached(prompt, 12, stop_token=stop)
    assert list(toks) == seq[:len(prompt) + first]
    unused = next(t for t in range(TINY["vocab"]) if t not in new)
    toks, _, _ = g.generate_cached(prompt, 12, stop_token=unused)
    assert list(toks) == seq
    toks, _, _ = g.generate_cached(prompt, 12, stop_token=new[0])
    assert list(toks) == list(prompt)


def test_gpt_max_seq_error(tiny):
    w, g = tiny
    with pytest.raises(ValueError):
        g.forward_cached(np.zeros(TINY["max_seq"] + 1, np.int32), g.new_cache())


# ------------------------------------------------------------------ MoE

def _np_expert(w, e, x):
    f = lambda a: hb.bf16_to_f32(a).astype(np.float64)
    gt = x @ f(w["wgate"][e]).T + w["bgate"][e]
    up = x @ f(w["wup"][e]).T + w["bup"][e]
    h = gt / (1 + np.exp(-gt)) * up
    return h @ f(w["wdown"][e]).T + w["bdown"][e]


def test_moe_vs_numpy_f64():
    x, logits, w = syn.moe_inputs(M=40, dim=32, ffn=64, experts=4, top_k=2, seed=17)
    rng = np.random.default_rng(18)
    for key in ("bgate", "bup", "bdown"):
        w[key] = [rng.standard_normal(b.shape).astype(np.float32) * 0.1 for b in w[key]]
    out, idx, wts = orc.moe_forward(w, x, logits)
    xd = x.astype(np.float64)
    ref = np.zeros_like(xd)
    for t in range(40):
        top = np.argsort(-logits[t], kind="stable")[:2]
        p = scipy.special.softmax(logits[t, top].astype(np.float64))
        assert np.array_equal(idx[t], top)
        for e, pe in zip(top, p):
            ref[t] += pe * _np_expert(w, e, xd[t:t + 1])[0]
    assert np.allclose(wts.sum(1), 1, atol=1e-6)                  # nn/moe_test.go:100-126
    assert np.max(np.abs(out - ref)) < 1e-5 * np.max(np.abs(ref))


def test_moe_single_expert_is_expert():
    # nn/moe_test.go:30-45: E=1, K=1 reduces to the expert itself
    x, logits, w = syn.moe_inputs(M=9, dim=16, ffn=32, experts=1, top_k=1, seed=19, with_router=True)
    out, idx, wts = orc.moe_forward(w, x)
    assert np.all(idx == 0) and np.all(wts == 1.0)
    ref = _np_expert(w, 0, x.astype(np.float64))
    assert np.max(np.abs(out - ref)) < 1e-5 * np.max(np.abs(ref))


def test_moe_rejects_bad_top_k():
    x, logits, w = syn.moe_inputs(M=4, dim=16, ffn=32, experts=2, top_k=3, seed=20)
    with pytest.raises(ValueError):
        orc.moe_forward(w, x, logits)


def test_attention_cached_vs_f64():
    rng = np.random.default_rng(25)
    heads, hd, pos, n = 3, 16, 7, 4
    d = heads * hd
    q = rng.standard_normal((n, d)).astype(np.float32)
    K = rng.standard_normal((pos + n, d)).astype(np.float32)
    V = rng.standard_normal((pos + n, d)).astype(np.float32)
    for causal in (True, False):
        got = orc.attention_cached(q, K, V, pos, heads, causal)
        ref = np.zeros((n, d))
        for h in range(heads):
            sl = slice(h * hd, (h + 1) * hd)
            s = q[:, sl].astype(np.float64) @ K[:, sl].T.astype(np.float64) / math.sqrt(hd)
            if causal:
                for i in range(n):
                    s[i, pos + i + 1:] = -np.inf
            ref[:, sl] = scipy.special.softmax(s, axis=1) @ V[:, sl]
        assert np.max(np.abs(got - ref)) < 1e-5
    # one visible key: the output is that key's value row (closed form)
    one = orc.attention_cached(q[:1], K[:1], V[:1], 0, heads, True)
    assert np.allclose(one, V[:1], atol=1e-7)


def _np_gqa(w, kc, vc, pos, x, cos_t, sin_t):
    """Independent float64 GQA.ForwardCached."""
    f = lambda a: hb.bf16_to_f32(a).astype(np.float64) if a.dtype == np.uint16 else a.astype(np.float64)
    S, nq, nkv, hd = x.shape[0], w["num_q"], w["num_kv"], w["head_dim"]
    g = nq // nkv
    xd = x.astype(np.float64)
    q = xd @ f(w["wq"]).T + w.get("bq", 0)
    k = xd @ f(w["wk"]).T + w.get("bk", 0)
    v = xd @ f(w["wv"]).T + w.get("bv", 0)
    q = q.reshape(S, nq, hd)
    k = k.reshape(S, nkv, hd)
    if "q_norm" in w:
        q = q / np.sqrt((q ** 2).mean(-1, keepdims=True) + w["norm_eps"]) * w["q_norm"]
        k = k / np.sqrt((k ** 2).mean(-1, keepdims=True) + w["norm_eps"]) * w["k_norm"]
    if cos_t is not None:
        half = hd // 2
        inv = np.float32(w["rope_base"]) ** (-(2 * np.arange(half)) / hd)
        theta = ((pos + np.arange(S))[:, None] * inv[None, :].astype(np.float64))[:, None, :]

        def rot(t):
            z = (t[..., :half] + 1j * t[..., half:]) * np.exp(1j * theta)
            return np.concatenate([z.real, z.imag], -1)
        q, k = rot(q), rot(k)
    K = np.concatenate([kc[:pos].reshape(pos, nkv, hd).astype(np.float64), k])
    V = np.concatenate([vc[:pos].reshape(pos, nkv, hd).astype(np.float64), v.reshape(S, nkv, hd)])
    att = np.zeros((S, nq, hd))
    for h in range(nq):
        s = q[:, h] @ K[:, h // g].T / math.sqrt(hd)
        for i in range(S):
            s[i, pos + i + 1:] = -np.inf
        att[:, h] = scipy.special.softmax(s, axis=1) @ V[:, h // g]
    return att.reshape(S, nq * hd) @ f(w["wo"]).T + w.get("bo", 0), K, V


@pytest.mark.parametrize("qk_norm,rope,bias", [(True, True, True), (False, False, False), (False, True, True)])
def test_gqa_forward_cached_vs_f64(qk_norm, rope, bias):
    w = syn.gqa_weights(seed=26, qk_norm=qk_norm, rope=rope, bias=bias)
    cos_t, sin_t = orc.rope_tables(w["head_dim"], w["rope_max_seq"], w["rope_base"]) if rope else (None, None)
    if rope:
        w["rope_cos"], w["rope_sin"] = cos_t, sin_t
    rng = np.random.default_rng(27)
    kvdim = w["num_kv"] * w["head_dim"]
    kc = np.zeros((20, kvdim), np.float32)
    vc = np.zeros((20, kvdim), np.float32)
    x0 = rng.standard_normal((5, w["dim"])).astype(np.float32)
    orc.gqa_forward_cached(w, kc, vc, 0, x0)            # prefill 5 tokens
    x1 = rng.standard_normal((3, w["dim"])).astype(np.float32)
    got = orc.gqa_forward_cached(w, kc, vc, 5, x1)      # 3 more (staircase mask)
    ref, K, V = _np_gqa(w, kc, vc, 5, x1, cos_t, sin_t)
    assert np.max(np.abs(got - ref)) < 1e-4 * np.max(np.abs(ref))
    assert np.max(np.abs(kc[:8] - K.reshape(8, kvdim))) < 1e-4
    assert np.max(np.abs(vc[:8] - V.reshape(8, kvdim))) < 1e-4
