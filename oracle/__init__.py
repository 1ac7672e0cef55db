"""ctypes view of the CPU oracle (oracle/liborc.so).

TEST INFRASTRUCTURE ONLY. Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py may import this package, and only as the
checker or the timed CPU baseline. The product package (gorch_amd) never
imports it.

The C library restates gorch's CPU semantics function by function; see the
citations in oracle/gorch_oracle.c.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liborc.so")

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load() -> C.CDLL:
    if not os.path.exists(_SO):
        build()
    lib = C.CDLL(_SO)
    vp = C.c_void_p
    sig = {
        "orc_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_f32_to_bf16_slice": (None, [f32p, u16p, C.c_int64]),
        "orc_bf16_to_f32_slice": (None, [u16p, f32p, C.c_int64]),
        "orc_sgemm": (None, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, f32p, f32p, f32p]),
        "orc_matmul_dt": (C.c_int, [vp, vp, f32p] + [C.c_int] * 7),
        "orc_batched_matmul_dt": (C.c_int, [vp, vp, f32p] + [C.c_int] * 8),
        "orc_linear": (None, [f32p, C.c_int, C.c_int, vp, C.c_int, vp, C.c_int, f32p]),
        "orc_set_widen_per_call": (None, [C.c_int]),
        "orc_set_threads": (C.c_int, [C.c_int]),
        "orc_clear_widen_cache": (None, []),
        "orc_add": (None, [f32p, f32p, f32p, C.c_int64]),
        "orc_gelu": (None, [f32p, f32p, C.c_int64]),
        "orc_sigmoid": (None, [f32p, f32p, C.c_int64]),
        "orc_silu": (None, [f32p, f32p, C.c_int64]),
        "orc_swiglu": (None, [f32p, f32p, f32p, C.c_int64]),
        "orc_layernorm": (None, [f32p, C.c_int, C.c_int, f32p, f32p, C.c_float, f32p]),
        "orc_rmsnorm": (None, [f32p, C.c_int, C.c_int, f32p, C.c_float, f32p]),
        "orc_softmax_inplace": (None, [f32p, C.c_int, C.c_int]),
        "orc_causal_softmax": (None, [f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_float]),
        "orc_embedding_lookup": (None, [f32p, C.c_int, i32p, C.c_int, f32p]),
        "orc_rope_tables": (None, [C.c_int, C.c_int, C.c_float, f32p, f32p]),
        "orc_rope_apply": (None, [f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int, f32p, f32p,
                                  C.c_int, C.c_float]),
        "orc_topk": (None, [f32p, C.c_int, C.c_int, C.c_int, f32p, i32p]),
        "orc_argmax": (C.c_int, [f32p, C.c_int]),
        "orc_kth_largest": (C.c_float, [f32p, C.c_int, C.c_int]),
        "orc_sample": (C.c_int, [f32p, C.c_int, C.c_float, C.c_int, C.c_float, C.c_double, vp]),
        "orc_sample_nucleus": (C.c_int, [f32p, C.c_int, C.c_float, C.c_int, C.c_float, C.c_double, vp]),
        "orc_philox_uniform": (C.c_double, [C.c_uint64, C.c_uint32, C.c_uint32]),
        "orc_philox4x32_10": (None, [vp, vp, vp]),
        "orc_generate_sampled": (C.c_int, [vp, i32p, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, C.c_float,
                                           C.c_uint64, C.c_int, i32p]),
        "orc_attention_cached": (None, [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.c_int]),
        "orc_kvcache_new": (vp, [C.c_int, C.c_int, C.c_int]),
        "orc_kvcache_free": (None, [vp]),
        "orc_kvcache_len": (C.c_int, [vp]),
        "orc_kvcache_reset": (None, [vp]),
        "orc_kvcache_keys": (C.POINTER(C.c_float), [vp, C.c_int]),
        "orc_kvcache_values": (C.POINTER(C.c_float), [vp, C.c_int]),
        "orc_gpt_forward_cached": (C.c_int, [vp, vp, i32p, C.c_int, f32p]),
        "orc_gpt_forward": (C.c_int, [vp, i32p, C.c_int, f32p]),
        "orc_generate_cached": (C.c_int, [vp, i32p, C.c_int, C.c_int, C.c_int, i32p, vp, vp]),
        "orc_moe_forward": (C.c_int, [vp, f32p, C.c_int, vp, f32p, vp, vp]),
        "orc_gqa_forward_cached": (C.c_int, [vp, f32p, f32p, C.c_int, f32p, C.c_int, f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- codec

def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib.orc_f32_to_bf16_slice(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib.orc_bf16_to_f32_slice(h.reshape(-1), out.reshape(-1), h.size)
    return out


# ---------------------------------------------------------------- matmul

def matmul_dt(A, B, M, N, K, transA=False, transB=False):
    """bf16_matmul.go:159-180. A/B are float32 or uint16 (bf16) arrays."""
    A = np.ascontiguousarray(A)
    B = np.ascontiguousarray(B)
    C_ = np.empty((M, N), np.float32)
    rc = lib.orc_matmul_dt(_ptr(A), _ptr(B), C_, M, N, K, int(transA), int(transB),
                           int(A.dtype == np.uint16), int(B.dtype == np.uint16))
    if rc != 0:
        raise ValueError("orc_matmul_dt: transA && transB is not supported")
    return C_


def batched_matmul_dt(A, B, batch, M, N, K, transA=False, transB=False):
    A = np.ascontiguousarray(A)
    B = np.ascontiguousarray(B)
    C_ = np.empty((batch, M, N), np.float32)
    rc = lib.orc_batched_matmul_dt(_ptr(A), _ptr(B), C_, M, N, K, batch, int(transA), int(transB),
                                   int(A.dtype == np.uint16), int(B.dtype == np.uint16))
    if rc != 0:
        raise ValueError("orc_batched_matmul_dt: transA && transB is not supported")
    return C_


def linear(x, W, bias=None):
    """nn/module.go:61-88: x [M,K] f32, W [N,K] bf16 (uint16) or f32."""
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W)
    M, K = x.shape
    N = W.shape[0]
    y = np.empty((M, N), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib.orc_linear(x, M, K, _ptr(W), int(W.dtype == np.uint16), _ptr(b), N, y)
    return y


def set_threads(n: int) -> int:
    """OpenMP threads of the oracle (n <= 0 keeps the current count); returns
    the count in effect."""
    return int(lib.orc_set_threads(n))


def set_widen_per_call(on: bool) -> None:
    lib.orc_set_widen_per_call(int(on))
    if on:
        lib.orc_clear_widen_cache()


# ---------------------------------------------------------------- row ops

def _unary(fn, x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    fn(x.reshape(-1), y.reshape(-1), x.size)
    return y


def gelu(x):
    return _unary(lib.orc_gelu, x)


def sigmoid(x):
    return _unary(lib.orc_sigmoid, x)


def silu(x):
    return _unary(lib.orc_silu, x)


def swiglu(gate, val):
    gate = np.ascontiguousarray(gate, np.float32)
    val = np.ascontiguousarray(val, np.float32)
    y = np.empty_like(gate)
    lib.orc_swiglu(gate.reshape(-1), val.reshape(-1), y.reshape(-1), gate.size)
    return y


def add(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    c = np.empty_like(a)
    lib.orc_add(a.reshape(-1), b.reshape(-1), c.reshape(-1), a.size)
    return c


def layernorm(x, gamma, beta, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    M, N = x.shape
    y = np.empty_like(x)
    lib.orc_layernorm(x, M, N, np.ascontiguousarray(gamma, np.float32),
                      np.ascontiguousarray(beta, np.float32), eps, y)
    return y


def rmsnorm(x, gamma, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    M, N = x.shape
    y = np.empty_like(x)
    lib.orc_rmsnorm(x, M, N, np.ascontiguousarray(gamma, np.float32), eps, y)
    return y


def softmax_inplace(x):
    x = np.array(x, np.float32, copy=True, order="C")
    rows, cols = x.shape
    lib.orc_softmax_inplace(x, rows, cols)
    return x


def causal_softmax(x, q_seq, scale):
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    y = np.empty_like(x)
    lib.orc_causal_softmax(x, y, rows, cols, q_seq, scale)
    return y


def embedding_lookup(weight, ids):
    weight = np.ascontiguousarray(weight, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.empty((ids.size, weight.shape[1]), np.float32)
    lib.orc_embedding_lookup(weight, weight.shape[1], ids, ids.size, out)
    return out


def rope_tables(head_dim, max_seq, base):
    half = head_dim // 2
    c = np.empty((max_seq, half), np.float32)
    s = np.empty((max_seq, half), np.float32)
    lib.orc_rope_tables(head_dim, max_seq, base, c, s)
    return c, s


def rope_apply(x, cos_t, sin_t, start_pos=0, neox=False, sign=1.0):
    """x: (..., seq, head_dim)."""
    x = np.ascontiguousarray(x, np.float32)
    seq, hd = x.shape[-2], x.shape[-1]
    outer = int(np.prod(x.shape[:-2])) if x.ndim > 2 else 1
    y = np.empty_like(x)
    lib.orc_rope_apply(x.reshape(-1), y.reshape(-1), outer, seq, hd, start_pos,
                       np.ascontiguousarray(cos_t, np.float32).reshape(-1),
                       np.ascontiguousarray(sin_t, np.float32).reshape(-1), int(neox), sign)
    return y


def attention_cached(q, K, V, pos_offset, heads, causal=True):
    """q [new_seq, dim]; K, V [pos_offset + new_seq, dim] -> [new_seq, dim]."""
    q = np.ascontiguousarray(q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    new_seq, dim = q.shape
    out = np.empty_like(q)
    lib.orc_attention_cached(q, K, V, out, new_seq, pos_offset, heads, dim // heads, int(causal))
    return out


def topk(x, k):
    x = np.ascontiguousarray(x, np.float32)
    B, V = x.shape
    vals = np.empty((B, k), np.float32)
    idx = np.empty((B, k), np.int32)
    lib.orc_topk(x, B, V, k, vals, idx)
    return vals, idx


def argmax(logits):
    logits = np.ascontiguousarray(logits, np.float32)
    return int(lib.orc_argmax(logits, logits.size))


def kth_largest(data, k):
    """model/generate.go:247-262."""
    data = np.ascontiguousarray(data, np.float32)
    return float(lib.orc_kth_largest(data, data.size, k))


def sample(logits, temperature, top_k, top_p, r):
    """model/generate.go:147-243 with the uniform draw r given. Returns
    (token, final distribution as float64)."""
    logits = np.ascontiguousarray(logits, np.float32)
    probs = np.empty(logits.size, np.float64)
    tok = lib.orc_sample(logits, logits.size, temperature, top_k, top_p, r, _ptr(probs))
    return int(tok), probs


def sample_nucleus(logits, temperature, top_k, top_p, r):
    """model/qwen/generate.go:94-163 (sampleLogits) with the uniform draw r
    given; equal probabilities in the nucleus sort by ascending index.
    Returns (token, final distribution as float64)."""
    logits = np.ascontiguousarray(logits, np.float32)
    probs = np.empty(logits.size, np.float64)
    tok = lib.orc_sample_nucleus(logits, logits.size, temperature, top_k, top_p, r, _ptr(probs))
    return int(tok), probs


def philox4x32_10(ctr, key):
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.empty(4, np.uint32)
    lib.orc_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return [int(v) for v in out]


def philox_uniform(seed, step, row):
    """The device sampler's draw for (seed, step, row)."""
    return float(lib.orc_philox_uniform(seed, step, row))


# ---------------------------------------------------------------- GPT

class _GPTWeights(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab", "dim", "heads", "layers", "max_seq", "linear_bf16")] + [
        ("wte", C.c_void_p), ("wpe", C.c_void_p),
    ] + [(n, C.POINTER(C.c_void_p)) for n in (
        "ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
        "ln2_g", "ln2_b", "w1", "b1", "w2", "b2")] + [
        ("lnf_g", C.c_void_p), ("lnf_b", C.c_void_p), ("wlm", C.c_void_p), ("blm", C.c_void_p),
    ]


_LAYER_KEYS = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
               "ln2_g", "ln2_b", "w1", "b1", "w2", "b2")


class GPT:
    """Oracle GPT over a weight dict (see gorch_amd.synthetic.gpt2_weights):
    ``cfg`` keys vocab/dim/heads/layers/max_seq; ``layers`` a list of dicts."""

    def __init__(self, w: dict):
        self._keep = []
        cfg = w["cfg"]
        s = _GPTWeights()
        s.vocab, s.dim, s.heads = cfg["vocab"], cfg["dim"], cfg["heads"]
        s.layers, s.max_seq = cfg["layers"], cfg["max_seq"]
        s.linear_bf16 = int(w["layers"][0]["wq"].dtype == np.uint16)
        for key in ("wte", "wpe", "lnf_g", "lnf_b", "wlm", "blm"):
            arr = np.ascontiguousarray(w[key])
            self._keep.append(arr)
            setattr(s, key, _ptr(arr))
        for key in _LAYER_KEYS:
            arrs = [np.ascontiguousarray(L[key]) for L in w["layers"]]
            self._keep.extend(arrs)
            ptrs = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
            self._keep.append(ptrs)
            setattr(s, key, C.cast(ptrs, C.POINTER(C.c_void_p)))
        self.s = s
        self.cfg = cfg

    @property
    def ref(self):
        return C.byref(self.s)

    def new_cache(self):
        return KVCache(self.cfg["layers"], self.cfg["dim"], self.cfg["max_seq"])

    def forward_cached(self, ids, cache: "KVCache"):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((ids.size, self.cfg["vocab"]), np.float32)
        rc = lib.orc_gpt_forward_cached(self.ref, cache.h, ids, ids.size, out)
        if rc != 0:
            raise ValueError("gorch: cached sequence length exceeds MaxSeq")
        return out

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((ids.size, self.cfg["vocab"]), np.float32)
        rc = lib.orc_gpt_forward(self.ref, ids, ids.size, out)
        if rc != 0:
            raise ValueError("gorch: sequence length exceeds MaxSeq")
        return out

    def generate_cached(self, prompt, max_new, want_logits=False, stop_token=-1):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(prompt.size + max_new, np.int32)
        V = self.cfg["vocab"]
        logits = np.empty((max_new, V), np.float32) if want_logits else None
        gaps = np.empty(max_new, np.float32)
        n = lib.orc_generate_cached(self.ref, prompt, prompt.size, max_new, stop_token, out,
                                    _ptr(logits), _ptr(gaps))
        return out[:n].copy(), logits, gaps

    def generate_sampled(self, prompt, max_new, temperature, top_k, top_p, seed, row=0, stop_token=-1):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(prompt.size + max_new, np.int32)
        n = lib.orc_generate_sampled(self.ref, prompt, prompt.size, max_new, stop_token, temperature, top_k,
                                     top_p, seed, row, out)
        return out[:n].copy()


class KVCache:
    def __init__(self, layers, dim, max_seq):
        self.h = lib.orc_kvcache_new(layers, dim, max_seq)
        self.dim = dim

    def __len__(self):
        return lib.orc_kvcache_len(self.h)

    def reset(self):
        lib.orc_kvcache_reset(self.h)

    def keys(self, layer):
        n = len(self) * self.dim
        return np.ctypeslib.as_array(lib.orc_kvcache_keys(self.h, layer), shape=(n,)).copy()

    def values(self, layer):
        n = len(self) * self.dim
        return np.ctypeslib.as_array(lib.orc_kvcache_values(self.h, layer), shape=(n,)).copy()

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_kvcache_free(self.h)
            self.h = None


# ---------------------------------------------------------------- MoE

class _MoEWeights(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("dim", "ffn", "experts", "top_k", "experts_bf16")] + [
        ("wr", C.c_void_p), ("br", C.c_void_p),
    ] + [(n, C.POINTER(C.c_void_p)) for n in ("wgate", "bgate", "wup", "bup", "wdown", "bdown")]


def moe_forward(w: dict, x, logits=None):
    """nn/moe.go:130-182. ``w``: dim, ffn, experts, top_k, wr, br (router,
    optional when logits are injected), wgate/bgate/wup/bup/wdown/bdown lists."""
    keep = []
    s = _MoEWeights()
    s.dim, s.ffn, s.experts, s.top_k = w["dim"], w["ffn"], w["experts"], w["top_k"]
    s.experts_bf16 = int(w["wgate"][0].dtype == np.uint16)
    for key in ("wr", "br"):
        arr = w.get(key)
        if arr is not None:
            arr = np.ascontiguousarray(arr)
            keep.append(arr)
        setattr(s, key, _ptr(arr))
    for key in ("wgate", "bgate", "wup", "bup", "wdown", "bdown"):
        arrs = w.get(key)
        if arrs is None:
            setattr(s, key, None)
            continue
        arrs = [np.ascontiguousarray(a) for a in arrs]
        keep.extend(arrs)
        ptrs = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
        keep.append(ptrs)
        setattr(s, key, C.cast(ptrs, C.POINTER(C.c_void_p)))
    x = np.ascontiguousarray(x, np.float32)
    M = x.shape[0]
    out = np.empty((M, w["dim"]), np.float32)
    idx = np.empty((M, w["top_k"]), np.int32)
    wts = np.empty((M, w["top_k"]), np.float32)
    lg = None if logits is None else np.ascontiguousarray(logits, np.float32)
    rc = lib.orc_moe_forward(C.byref(s), x, M, _ptr(lg), out, _ptr(idx), _ptr(wts))
    if rc != 0:
        raise ValueError("gorch/nn: MoE numExpertsPerToken out of range")
    return out, idx, wts


# ---------------------------------------------------------------- GQA

class _GQAWeights(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("dim", "num_q", "num_kv", "head_dim", "causal", "linear_bf16")] + [
        ("norm_eps", C.c_float)] + [(n, C.c_void_p) for n in (
            "wq", "wk", "wv", "wo", "bq", "bk", "bv", "bo", "q_norm", "k_norm", "rope_cos", "rope_sin")] + [
        ("rope_max_seq", C.c_int), ("rope_neox", C.c_int)]


def gqa_forward_cached(w: dict, k_cache, v_cache, pos_offset, x):
    """nn/gqa.go:259-363. ``w``: dim, num_q, num_kv, head_dim, causal,
    norm_eps, wq/wk/wv/wo (uint16 bf16 or f32), optional bq.. bo, q_norm,
    k_norm, rope_cos/rope_sin (+ rope_neox). k_cache/v_cache are float32
    [capacity, num_kv*head_dim] arrays updated in place."""
    keep = []
    s = _GQAWeights()
    for n in ("dim", "num_q", "num_kv", "head_dim"):
        setattr(s, n, w[n])
    s.causal = int(w.get("causal", True))
    s.linear_bf16 = int(w["wq"].dtype == np.uint16)
    s.norm_eps = w.get("norm_eps", 1e-6)
    for n in ("wq", "wk", "wv", "wo", "bq", "bk", "bv", "bo", "q_norm", "k_norm", "rope_cos", "rope_sin"):
        a = w.get(n)
        if a is not None:
            a = np.ascontiguousarray(a)
            keep.append(a)
        setattr(s, n, _ptr(a))
    s.rope_max_seq = 0 if w.get("rope_cos") is None else w["rope_cos"].shape[0]
    s.rope_neox = int(w.get("rope_neox", 0))
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty((x.shape[0], w["dim"]), np.float32)
    rc = lib.orc_gqa_forward_cached(C.byref(s), k_cache, v_cache, pos_offset, x, x.shape[0], out)
    if rc != 0:
        raise ValueError("gorch/nn: GQA numQueryHeads must be divisible by numKVHeads")
    return out
