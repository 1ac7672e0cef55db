"""Qwen3-style decoder on the GPU: gorch's model/qwen (qwen.go:12-98,
block.go:27-79) — tokens -> embedding -> L x [x1 = x + GQA(RMSNorm(x)); x =
x1 + SwiGLU-MLP(RMSNorm(x1))] -> RMSNorm -> tied LM head — composed from the
library's kernels through its C-ABI (gorch_amd.hip): the embedding gather,
one gorch_hip_qwen_block_forward_cached call per block (RMSNorm, Q/K/V as one
weight stream, per-head q/k RMSNorm + RoPE into the cache, grouped-query
cached attention, Wo + residual, RMSNorm, gate/up as one weight, SwiGLU, down
+ residual: five launches for a one-token step), the final RMSNorm and the tied
head. Every launch goes on torch's current stream, so a decode step can be
captured in a CUDA graph and replayed.

Weights are host arrays as gorch_amd.synthetic.qwen_weights builds them, or
device tensors of the same layout (bf16 as int16): bf16 Linear weights [out,
in], f32 RMSNorm gains, a bf16 embedding table (looked up widened to f32; the tied LM head reads the bf16 table, as
MatMulTransB(last, Embed.Weight) does for a bf16 checkpoint, qwen.go:84).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import hip


@dataclass(frozen=True)
class QwenConfig:
    """model/qwen/config.go:13-28. attn_bias: q/k/v projection biases
    (Qwen2.5); use_qk_norm: per-head q/k RMSNorm (Qwen3); tied_embeddings:
    the LM head is the embedding table (the reference's Model always ties it,
    qwen.go:84); eos_tokens: generation stop ids."""
    hidden: int
    layers: int
    num_q: int
    num_kv: int
    head_dim: int
    inter: int
    vocab: int
    rope_theta: float = 1_000_000.0
    eps: float = 1e-6
    max_seq: int = 4096
    attn_bias: bool = False
    use_qk_norm: bool = True
    tied_embeddings: bool = True
    eos_tokens: tuple = ()

    @property
    def kv_dim(self) -> int:
        return self.num_kv * self.head_dim


# model/qwen/config.go:40-56 (Qwen3-0.6B) and :61-78 (Qwen2.5-0.5B-Instruct)
QWEN3_0_6B = QwenConfig(hidden=1024, layers=28, num_q=16, num_kv=8, head_dim=128, inter=3072, vocab=151936,
                        max_seq=40960, attn_bias=False, use_qk_norm=True, tied_embeddings=True,
                        eos_tokens=(151645, 151643))
QWEN2_5_0_5B = QwenConfig(hidden=896, layers=24, num_q=14, num_kv=2, head_dim=64, inter=4864, vocab=151936,
                          max_seq=32768, attn_bias=True, use_qk_norm=False, tied_embeddings=True,
                          eos_tokens=(151645, 151643))


class Qwen:
    """model/qwen Model.ForwardCached (qwen.go:69-89) on the GPU."""

    def __init__(self, cfg: QwenConfig, w: dict):
        import torch

        def up(a):
            a = np.ascontiguousarray(a)
            return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()

        if not cfg.tied_embeddings:
            raise ValueError("qwen: only the tied LM head is supported (the reference Model ties it)")
        self.cfg = cfg
        self._engine = None
        self.embed_bf16 = w["embed"] if isinstance(w["embed"], torch.Tensor) else up(w["embed"])
        self.embed = torch.empty((cfg.vocab, cfg.hidden), dtype=torch.float32, device="cuda")
        hip.bf16_to_f32(self.embed_bf16, self.embed)
        self.norm = w["norm"] if isinstance(w["norm"], torch.Tensor) else up(w["norm"])
        # one RoPE table shared by every layer (New, qwen.go:31-36)
        self.rope_cos, self.rope_sin = hip.rope_tables(cfg.head_dim, cfg.max_seq, cfg.rope_theta)
        self.layers = []
        for lw in w["layers"]:
            has_bias = all(lw.get(n) is not None for n in ("bq", "bk", "bv"))
            if cfg.attn_bias != has_bias:
                raise ValueError("qwen: attn_bias says %s but the layer weights %s q/k/v biases"
                                 % (cfg.attn_bias, "carry" if has_bias else "lack"))
            has_norm = lw.get("q_norm") is not None and lw.get("k_norm") is not None
            if cfg.use_qk_norm != has_norm:
                raise ValueError("qwen: use_qk_norm says %s but the layer weights %s q/k norm gains"
                                 % (cfg.use_qk_norm, "carry" if has_norm else "lack"))
            # Q, K, V rows as consecutive ranges of one weight (and one bias)
            # so that a step streams them as one projection
            q, kv = cfg.num_q * cfg.head_dim, cfg.kv_dim
            wqkv = torch.cat([lw[n] if isinstance(lw[n], torch.Tensor) else up(lw[n]) for n in ("wq", "wk", "wv")])
            gw = {"dim": cfg.hidden, "num_q": cfg.num_q, "num_kv": cfg.num_kv, "head_dim": cfg.head_dim,
                  "causal": True, "norm_eps": cfg.eps, "wq": wqkv[:q], "wk": wqkv[q:q + kv], "wv": wqkv[q + kv:],
                  "wo": lw["wo"], "rope": True, "rope_base": cfg.rope_theta, "rope_max_seq": cfg.max_seq,
                  "rope_cos": self.rope_cos, "rope_sin": self.rope_sin}
            if cfg.use_qk_norm:
                gw["q_norm"], gw["k_norm"] = lw["q_norm"], lw["k_norm"]
            if cfg.attn_bias:
                bqkv = torch.cat([lw[n] if isinstance(lw[n], torch.Tensor) else up(lw[n]) for n in ("bq", "bk", "bv")])
                gw["bq"], gw["bk"], gw["bv"] = bqkv[:q], bqkv[q:q + kv], bqkv[q + kv:]
            layer = {"attn": hip.GQA(gw)}
            for n in ("norm_attn", "norm_ffn", "wgate", "wup", "wdown"):
                layer[n] = lw[n] if isinstance(lw[n], torch.Tensor) else up(lw[n])
            # gate and up rows in one [2 * inter, d] weight: one GEMV (or one
            # GEMM with two output segments) produces [gate | up]
            layer["wgu"] = torch.cat([layer.pop("wgate"), layer.pop("wup")], 0)
            layer["block"] = hip.QwenBlock(layer["attn"], layer["norm_attn"], layer["norm_ffn"], layer["wgu"],
                                           layer["wdown"], cfg.inter, cfg.eps)
            self.layers.append(layer)

    def generate(self, prompt, max_new: int, stop_tokens=None, want_logits=False, use_graph=True,
                 temperature=0.0, top_k=0, top_p=0.0, seed=0):
        """Generate (model/qwen/generate.go:35-66) on the device: prefill,
        then one token per step, each step replayed from a HIP graph that
        reads the position on the device. temperature 0 (the Greedy config):
        the argmax fused into the tied head; temperature > 0: sampleLogits
        (:94-181) on the device with top_k / top_p, new token i drawn from
        Philox(seed, i, 0). stop_tokens (default cfg.eos_tokens, the
        reference's Greedy list) end generation and are not kept. Returns
        (ids: prompt + new tokens, step logits [n_new, vocab] or None,
        timing dict)."""
        import ctypes as C

        cfg = self.cfg
        if self._engine is None:
            blocks = (hip._QwenBlockW * len(self.layers))(*[layer["block"].s for layer in self.layers])
            h = hip.lib().gorch_hip_qwen_create(blocks, len(self.layers), self.embed_bf16.data_ptr(),
                                                self.embed.data_ptr(), self.norm.data_ptr(), cfg.eps, cfg.vocab,
                                                cfg.max_seq)
            if not h:
                raise hip.HipError(2, hip.last_error())
            self._engine = h
        prompt = np.ascontiguousarray(np.asarray(prompt, np.int32).reshape(-1))
        stops = np.ascontiguousarray(np.asarray(cfg.eos_tokens if stop_tokens is None else stop_tokens, np.int32))
        out = np.zeros(prompt.size + max(max_new, 0), np.int32)
        n = C.c_int(0)
        logits = np.zeros((max(max_new, 1), cfg.vocab), np.float32) if want_logits else None
        timing = (C.c_float * 4)()
        hip._ok(hip.lib().gorch_hip_qwen_generate_sampled(
            hip._stream(), self._engine, prompt.ctypes.data, prompt.size, max_new,
            stops.ctypes.data if stops.size else None, stops.size, float(temperature), int(top_k), float(top_p),
            int(seed), out.ctypes.data, C.byref(n), None if logits is None else logits.ctypes.data, timing,
            int(use_graph)))
        ids = out[: n.value].copy()
        if logits is not None:
            logits = logits[: n.value - prompt.size]
        return ids, logits, {"prefill_ms": timing[0], "decode_ms": timing[1], "decode_forwards": int(timing[2]),
                             "graph": bool(timing[3])}

    def close(self):
        """Releases the generation engine (its cache and buffers)."""
        if getattr(self, "_engine", None):
            hip.lib().gorch_hip_qwen_destroy(self._engine)
            self._engine = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def new_cache(self, capacity: int):
        """Per-layer K and V rows [capacity, kv_dim] f32 (nn/kvcache.go:14-60)."""
        import torch

        if capacity > self.cfg.max_seq:
            raise ValueError("qwen: cache capacity above the RoPE table length")
        return [(torch.zeros((capacity, self.cfg.kv_dim), device="cuda"),
                 torch.zeros((capacity, self.cfg.kv_dim), device="cuda")) for _ in self.layers]

    def forward_cached(self, ids, cache, pos: int):
        """Logits [1, vocab] of the last of ``ids`` (int32 device tensor),
        whose rows take cache positions pos .. pos + len(ids) - 1."""
        import torch

        cfg = self.cfg
        S = ids.numel()
        if S == 0:
            raise ValueError("qwen: empty token slice")
        if pos + S > cache[0][0].shape[0]:
            raise ValueError("qwen: cache capacity exceeded")
        d = cfg.hidden
        x = torch.empty((S, d), device="cuda")
        hip.embedding(self.embed, ids, x)
        for layer, (kc, vc) in zip(self.layers, cache):
            layer["block"].forward_cached(x, kc, vc, pos)
        last = torch.empty((1, d), device="cuda")
        hip.rmsnorm(x[S - 1:S], self.norm, last, cfg.eps)
        logits = torch.empty((1, cfg.vocab), device="cuda")
        hip.linear_bf16(last, self.embed_bf16, None, logits)
        return logits
