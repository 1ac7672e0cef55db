"""Seeded synthetic inputs at the benchmark shapes (there are no checkpoints
or datasets offline). One numpy PCG64 generator per call, seed recorded by
the caller; bf16 tensors are gorch-rounded (RNE) N(0, 0.02^2) samples, the
init gorch's NewEmbedding/NewLinear use (nn/embedding.go:16-24).

Weight dicts use the layout the host engine and the test oracle share:
``cfg`` (vocab, dim, heads, layers, max_seq), ``wte``/``wpe`` f32,
``layers`` = list of dicts with ln1_g, ln1_b, wq, bq, wk, bk, wv, bv, wo, bo,
ln2_g, ln2_b, w1, b1, w2, b2 (Linear weights [out, in] bf16 as uint16),
and lnf_g, lnf_b, wlm (untied LM head, bf16), blm.
"""
from __future__ import annotations

import numpy as np

from .bf16 import f32_to_bf16, round_f32

GPT2_SMALL = dict(vocab=50257, dim=768, heads=12, layers=12, max_seq=1024)
GPT2_XL = dict(vocab=50257, dim=1600, heads=25, layers=48, max_seq=1024)


def normal(rng, shape, std=1.0):
    a = rng.standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        a *= np.float32(std)
    return a


def bf16_normal(rng, shape, std=0.02):
    return f32_to_bf16(normal(rng, shape, std))


def gemv_inputs(M, K, N, seed=0):
    """x ~ N(0,1) f32 [M,K]; W bf16 [N,K] from N(0,0.02); bias zeros [N]."""
    rng = np.random.default_rng(seed)
    x = normal(rng, (M, K))
    W = bf16_normal(rng, (N, K))
    b = np.zeros(N, np.float32)
    return x, W, b


def gpt2_weights(cfg: dict, seed: int = 0, random_affine: bool = False) -> dict:
    """GPT-2-shaped weights. With ``random_affine`` the biases and LayerNorm
    parameters are random too (tests), else biases 0, gamma 1, beta 0."""
    rng = np.random.default_rng(seed)
    V, d, L, S = cfg["vocab"], cfg["dim"], cfg["layers"], cfg["max_seq"]
    f = 4 * d

    def vec(n, base=0.0, std=0.02):
        if random_affine:
            return (np.float32(base) + normal(rng, (n,), std)).astype(np.float32)
        return np.full(n, base, np.float32)

    w = {"cfg": dict(cfg)}
    w["wte"] = round_f32(normal(rng, (V, d), 0.02))
    w["wpe"] = round_f32(normal(rng, (S, d), 0.02))
    layers = []
    for _ in range(L):
        layers.append({
            "ln1_g": vec(d, 1.0, 0.1), "ln1_b": vec(d),
            "wq": bf16_normal(rng, (d, d)), "bq": vec(d),
            "wk": bf16_normal(rng, (d, d)), "bk": vec(d),
            "wv": bf16_normal(rng, (d, d)), "bv": vec(d),
            "wo": bf16_normal(rng, (d, d)), "bo": vec(d),
            "ln2_g": vec(d, 1.0, 0.1), "ln2_b": vec(d),
            "w1": bf16_normal(rng, (f, d)), "b1": vec(f),
            "w2": bf16_normal(rng, (d, f)), "b2": vec(d),
        })
    w["layers"] = layers
    w["lnf_g"] = vec(d, 1.0, 0.1)
    w["lnf_b"] = vec(d)
    w["wlm"] = bf16_normal(rng, (V, d))
    w["blm"] = vec(V)
    return w


def prompt_ids(n, vocab, seed=0):
    rng = np.random.default_rng(seed)
    return rng.integers(0, vocab, size=n, dtype=np.int64).astype(np.int32)


def moe_inputs(M=2048, dim=1024, ffn=4096, experts=8, top_k=2, seed=0, with_router=False):
    """x ~ N(0,1) [M,dim]; gate logits ~ N(0,1) [M,E] (injected, as the
    benchmark config states); expert weights bf16 N(0,0.02); biases zero."""
    rng = np.random.default_rng(seed)
    x = normal(rng, (M, dim))
    logits = normal(rng, (M, experts))
    w = {"dim": dim, "ffn": ffn, "experts": experts, "top_k": top_k,
         "wgate": [], "wup": [], "wdown": [], "bgate": [], "bup": [], "bdown": []}
    for _ in range(experts):
        w["wgate"].append(bf16_normal(rng, (ffn, dim)))
        w["wup"].append(bf16_normal(rng, (ffn, dim)))
        w["wdown"].append(bf16_normal(rng, (dim, ffn)))
        w["bgate"].append(np.zeros(ffn, np.float32))
        w["bup"].append(np.zeros(ffn, np.float32))
        w["bdown"].append(np.zeros(dim, np.float32))
    if with_router:
        w["wr"] = bf16_normal(rng, (experts, dim))
        w["br"] = np.zeros(experts, np.float32)
    return x, logits, w


def gqa_weights(dim=64, num_q=8, num_kv=2, head_dim=16, max_seq=64, seed=0, bias=True, qk_norm=True,
                rope=True, base=10000.0):
    """A GQAConfig-shaped module (nn/gqa.go:64-98) with bf16 Linear weights;
    RoPE tables are left to the caller (``rope_base``/``rope_max_seq``)."""
    rng = np.random.default_rng(seed)
    qdim, kvdim = num_q * head_dim, num_kv * head_dim
    w = {"dim": dim, "num_q": num_q, "num_kv": num_kv, "head_dim": head_dim, "causal": True,
         "norm_eps": 1e-6,
         "wq": bf16_normal(rng, (qdim, dim), 0.1), "wk": bf16_normal(rng, (kvdim, dim), 0.1),
         "wv": bf16_normal(rng, (kvdim, dim), 0.1), "wo": bf16_normal(rng, (dim, qdim), 0.1)}
    if bias:
        for n, size in (("bq", qdim), ("bk", kvdim), ("bv", kvdim), ("bo", dim)):
            w[n] = normal(rng, (size,), 0.05)
    if qk_norm:
        w["q_norm"] = (1 + normal(rng, (head_dim,), 0.1)).astype(np.float32)
        w["k_norm"] = (1 + normal(rng, (head_dim,), 0.1)).astype(np.float32)
    w["rope"] = bool(rope)
    w["rope_base"] = base
    w["rope_max_seq"] = max_seq
    return w


def qwen_weights(cfg, seed: int = 0) -> dict:
    """Random weights for gorch_amd.qwen.Qwen (model/qwen/qwen.go:28-48,
    block.go:27-55): bf16 Linear weights N(0, 0.02) [out, in], a bf16
    embedding table, RMSNorm and q/k-norm gains 1 + N(0, 0.1)."""
    rng = np.random.default_rng(seed)
    q, kv, d = cfg.num_q * cfg.head_dim, cfg.kv_dim, cfg.hidden

    def gain(n):
        return (1 + normal(rng, (n,), 0.1)).astype(np.float32)

    layers = []
    for _ in range(cfg.layers):
        L = {"wq": bf16_normal(rng, (q, d)), "wk": bf16_normal(rng, (kv, d)),
             "wv": bf16_normal(rng, (kv, d)), "wo": bf16_normal(rng, (d, q)),
             "norm_attn": gain(d), "norm_ffn": gain(d),
             "wgate": bf16_normal(rng, (cfg.inter, d)), "wup": bf16_normal(rng, (cfg.inter, d)),
             "wdown": bf16_normal(rng, (d, cfg.inter))}
        if getattr(cfg, "use_qk_norm", True):
            L["q_norm"], L["k_norm"] = gain(cfg.head_dim), gain(cfg.head_dim)
        if getattr(cfg, "attn_bias", False):
            L["bq"], L["bk"], L["bv"] = normal(rng, (q,), 0.05), normal(rng, (kv,), 0.05), normal(rng, (kv,), 0.05)
        layers.append(L)
    return {"embed": bf16_normal(rng, (cfg.vocab, d)), "norm": gain(d), "layers": layers}
