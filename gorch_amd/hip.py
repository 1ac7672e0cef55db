"""ctypes binding of include/gorch_hip.h — the Python-side sibling of gorch's
metal/metal.go (the Go binding over metal/shim.h).

Device memory and streams come from PyTorch-ROCm tensors (plumbing only):
every call takes ``torch.Tensor`` arguments that already live on the GPU and
passes their device pointers and the current HIP stream to the C-ABI.

There is no CPU fallback here: if libgorch_hip.so is missing or the GPU is
absent, calls raise. A nonzero return code from the C-ABI raises
``HipError`` carrying gorch_hip_last_error().
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgorch_hip.so")

EPI_NONE = 0
EPI_GELU = 1
LINEAR_ACT_BF16 = 1

COUNTER_NAMES = ("gemv", "gemm", "generic_matmul", "attention", "norm", "elementwise", "moe",
                 "argmax", "codec")


class HipError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"gorch_hip rc={rc}: {msg}")
        self.rc = rc


_lib = None

vp, i32, i64, u32, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_uint32, C.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "gorch_hip_init": (i32, [i32]),
    "gorch_hip_device_count": (i32, []),
    "gorch_hip_last_error": (C.c_char_p, []),
    "gorch_hip_alloc": (vp, [C.c_size_t]),
    "gorch_hip_release": (None, [vp]),
    "gorch_hip_upload": (i32, [vp, vp, vp, C.c_size_t]),
    "gorch_hip_download": (i32, [vp, vp, vp, C.c_size_t]),
    "gorch_hip_sync": (i32, [vp]),
    "gorch_hip_live_bytes": (C.c_longlong, []),
    "gorch_hip_scratch_bytes": (C.c_longlong, []),
    "gorch_hip_release_stream_scratch": (None, [vp]),
    "gorch_hip_qwen_create": (C.c_void_p, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_float,
                                           C.c_int, C.c_int]),
    "gorch_hip_qwen_destroy": (None, [C.c_void_p]),
    "gorch_hip_qwen_generate": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int,
                                          C.c_void_p, C.POINTER(C.c_int), C.c_void_p, C.c_void_p, C.c_int]),
    "gorch_hip_qwen_generate_sampled": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                                  C.c_int, C.c_float, C.c_int, C.c_float, C.c_uint64, C.c_void_p,
                                                  C.POINTER(C.c_int), C.c_void_p, C.c_void_p, C.c_int]),
    "gorch_hip_set_deterministic": (C.c_int, [C.c_int]),
    "gorch_hip_deterministic_enabled": (C.c_int, []),
    "gorch_hip_buf_new": (vp, [C.c_size_t, i32]),
    "gorch_hip_buf_release": (None, [vp]),
    "gorch_hip_buf_len": (C.c_size_t, [vp]),
    "gorch_hip_buf_device": (vp, [vp, vp, i32]),
    "gorch_hip_buf_host": (vp, [vp, vp, i32]),
    "gorch_hip_set_async": (i32, [i32]),
    "gorch_hip_async_enabled": (i32, []),
    "gorch_hip_bf16_matmul_supported": (i32, []),
    "gorch_hip_bf16_probe": (i32, []),
    "gorch_hip_read_dispatch_counts": (i32, [C.POINTER(C.c_uint64), i32]),
    "gorch_hip_reset_dispatch_counts": (None, []),
    "gorch_hip_bf16_to_f32": (i32, [vp, vp, vp, i64]),
    "gorch_hip_f32_to_bf16": (i32, [vp, vp, vp, i64]),
    "gorch_hip_matmul_dt": (i32, [vp, vp, vp, vp, u32, u32, u32, i32, i32, i32, i32]),
    "gorch_hip_batched_matmul_dt": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, i32, i32, i32, i32]),
    "gorch_hip_linear_bf16": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "gorch_hip_linear_bf16_ex": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32]),
    "gorch_hip_packed_bf16_bytes": (C.c_size_t, [i32, i32]),
    "gorch_hip_pack_bf16": (i32, [vp, vp, vp, i32, i32]),
    "gorch_hip_linear_bf16_packed": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "gorch_hip_linear_bf16_noalloc": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "gorch_hip_layernorm": (i32, [vp, vp, vp, vp, vp, i32, i32, f32]),
    "gorch_hip_rmsnorm": (i32, [vp, vp, vp, vp, i32, i32, f32]),
    "gorch_hip_add_rmsnorm": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, f32]),
    "gorch_hip_add": (i32, [vp, vp, vp, vp, i64]),
    "gorch_hip_bias_add": (i32, [vp, vp, vp, i32, i32]),
    "gorch_hip_gelu": (i32, [vp, vp, vp, i64]),
    "gorch_hip_silu": (i32, [vp, vp, vp, i64]),
    "gorch_hip_swiglu": (i32, [vp, vp, vp, vp, i64]),
    "gorch_hip_embedding": (i32, [vp, vp, i32, vp, i32, vp]),
    "gorch_hip_attention_cached": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32]),
    "gorch_hip_causal_softmax": (i32, [vp, vp, vp, i32, i32, i32, f32]),
    "gorch_hip_softmax_rows": (i32, [vp, vp, i32, i32]),
    "gorch_hip_argmax": (i32, [vp, vp, i32, i32, vp]),
    "gorch_hip_sample": (i32, [vp, vp, i32, i32, C.c_float, i32, C.c_float, vp, vp, vp]),
    "gorch_hip_sample_nucleus": (i32, [vp, vp, i32, i32, C.c_float, i32, C.c_float, vp, vp, vp]),
    "gorch_hip_sample_workspace_size": (C.c_size_t, [i32]),
    "gorch_hip_sample_with_workspace": (i32, [vp, vp, i32, i32, C.c_float, i32, C.c_float, vp, vp, vp, i32, vp]),
    "gorch_hip_rope_tables": (i32, [vp, i32, i32, f32, vp, vp]),
    "gorch_hip_rope_apply": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, i32, i32, f32]),
    "gorch_hip_gqa_attention_cached": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32]),
    "gorch_hip_gqa_workspace_size": (C.c_size_t, [vp, i32]),
    "gorch_hip_gqa_forward_cached": (i32, [vp, vp, vp, i32, vp, vp, i32, i32, vp, vp, C.c_size_t]),
    "gorch_hip_qwen_block_workspace_size": (C.c_size_t, [vp, i32]),
    "gorch_hip_qwen_block_forward_cached": (i32, [vp, vp, vp, i32, vp, vp, i32, i32, vp, C.c_size_t]),
    "gorch_hip_moe_workspace_size": (C.c_size_t, [i32, i32, i32, i32, i32]),
    "gorch_hip_moe_forward": (i32, [vp, vp, vp, i32, vp, vp, vp, vp, vp, C.c_size_t]),
    "gorch_hip_gpt_create": (vp, [vp]),
    "gorch_hip_gpt_load_gpt2": (vp, [C.c_char_p, i32, i32, i32, i32, i32]),
    "gorch_hip_st_open": (vp, [C.c_char_p]),
    "gorch_hip_st_close": (None, [vp]),
    "gorch_hip_st_count": (i32, [vp]),
    "gorch_hip_st_name": (C.c_char_p, [vp, i32]),
    "gorch_hip_st_info": (i32, [vp, C.c_char_p, C.POINTER(i32), C.POINTER(i32), C.POINTER(i64),
                                C.POINTER(i64)]),
    "gorch_hip_st_load": (i32, [vp, vp, C.c_char_p, vp, i32, i32]),
    "gorch_hip_gpt_free": (None, [vp]),
    "gorch_hip_gpt_drop_packed": (C.c_size_t, [vp]),
    "gorch_hip_kvcache_create": (vp, [vp, i32, i32]),
    "gorch_hip_kvcache_free": (None, [vp]),
    "gorch_hip_kvcache_len": (i32, [vp]),
    "gorch_hip_kvcache_reset": (i32, [vp]),
    "gorch_hip_kvcache_read": (i32, [vp, i32, i32, vp, vp]),
    "gorch_hip_gpt_forward_cached": (i32, [vp, vp, vp, vp, i32, vp]),
    "gorch_hip_generate_cached": (i32, [vp, vp, vp, i32, i32, i32, vp, vp, vp, vp, i32]),
    "gorch_hip_generate": (i32, [vp, vp, vp, i32, i32, vp, vp, vp, vp, vp]),
}


def lib() -> C.CDLL:
    """Loads libgorch_hip.so (once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m gorch_amd.build` "
                "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().gorch_hip_last_error().decode()


def _ok(rc: int) -> None:
    if rc != 0:
        raise HipError(rc, last_error())


def _p(t):
    """Device pointer of a tensor (or None)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("gorch_amd.hip: tensor is not on the GPU")
    if not t.is_contiguous():
        raise ValueError("gorch_amd.hip: tensor must be contiguous")
    return t.data_ptr()


def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def init(device: int = 0) -> None:
    _ok(lib().gorch_hip_init(device))


def device_count() -> int:
    return lib().gorch_hip_device_count()


def dispatch_counts() -> dict:
    arr = (C.c_uint64 * len(COUNTER_NAMES))()
    n = lib().gorch_hip_read_dispatch_counts(arr, len(COUNTER_NAMES))
    return {COUNTER_NAMES[i]: int(arr[i]) for i in range(n)}


def reset_dispatch_counts() -> None:
    lib().gorch_hip_reset_dispatch_counts()


def set_async(on: bool) -> None:
    """SetMetalAsync (metal_async.go:30-34): off makes every compute call wait."""
    _ok(lib().gorch_hip_set_async(int(on)))


def async_enabled() -> bool:
    return bool(lib().gorch_hip_async_enabled())


def set_deterministic(on: bool) -> bool:
    """Fixed-order sums only (no float atomics in the one-row decode steps);
    returns the previous setting."""
    return bool(lib().gorch_hip_set_deterministic(int(on)))


def deterministic_enabled() -> bool:
    return bool(lib().gorch_hip_deterministic_enabled())


def bf16_matmul_supported() -> bool:
    """MetalBF16MatMulSupported (bf16_matmul.go:52-59) for the current device."""
    return bool(lib().gorch_hip_bf16_matmul_supported())


def bf16_probe() -> bool:
    """Runs the bf16 matmul probe again; returns its verdict."""
    return bool(lib().gorch_hip_bf16_probe())


BUF_HOST_MIRROR = 1


class Buffer:
    """A device buffer handle (metal.Buffer, metal/metal.go:240-422):
    ``bytes`` of zero-filled HBM, optionally with a pinned host mirror.
    ``release()`` is idempotent; the handle is also released when collected
    (the reference's finaliser)."""

    def __init__(self, nbytes: int, host_mirror: bool = False):
        self.h = lib().gorch_hip_buf_new(nbytes, BUF_HOST_MIRROR if host_mirror else 0)
        if not self.h:
            raise HipError(4, last_error())

    def __len__(self):
        return lib().gorch_hip_buf_len(self.h)

    def device(self, will_write: bool = False, stream=None) -> int:
        p = lib().gorch_hip_buf_device(stream, self.h, int(will_write))
        if not p:
            raise HipError(2, last_error())
        return p

    def host(self, will_write: bool = False, stream=None) -> int:
        """Data(): waits for ``stream`` and returns the current host mirror."""
        p = lib().gorch_hip_buf_host(stream, self.h, int(will_write))
        if not p:
            raise HipError(2, last_error())
        return p

    def release(self) -> None:
        lib().gorch_hip_buf_release(self.h)

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


# ------------------------------------------------------------------ codec

def bf16_to_f32(inp, out) -> None:
    """inp: uint16-storage tensor (torch.int16/uint16/bfloat16), out: float32."""
    _ok(lib().gorch_hip_bf16_to_f32(_stream(), _p(inp), _p(out), inp.numel()))


def f32_to_bf16(inp, out) -> None:
    _ok(lib().gorch_hip_f32_to_bf16(_stream(), _p(inp), _p(out), inp.numel()))


# ------------------------------------------------------------------ matmul

def matmul_dt(A, B, C_, M, N, K, transA=False, transB=False, aBF16=False, bBF16=False) -> None:
    _ok(lib().gorch_hip_matmul_dt(_stream(), _p(A), _p(B), _p(C_), M, N, K, int(transA), int(transB),
                                  int(aBF16), int(bBF16)))


def batched_matmul_dt(A, B, C_, M, N, K, batch, transA=False, transB=False, aBF16=False,
                      bBF16=False) -> None:
    _ok(lib().gorch_hip_batched_matmul_dt(_stream(), _p(A), _p(B), _p(C_), M, N, K, batch, int(transA),
                                          int(transB), int(aBF16), int(bBF16)))


def _n(t):
    return t.numel()


def layernorm(x, gamma, beta, y, eps=1e-5) -> None:
    M, N = x.shape
    _ok(lib().gorch_hip_layernorm(_stream(), _p(x), _p(gamma), _p(beta), _p(y), M, N, eps))


def rmsnorm(x, gamma, y, eps=1e-6) -> None:
    M, N = x.shape
    _ok(lib().gorch_hip_rmsnorm(_stream(), _p(x), _p(gamma), _p(y), M, N, eps))


def add_rmsnorm(x, b, gamma, s, y, eps=1e-6) -> None:
    """s = x + b; y = RMSNorm(s) (a decoder block's residual add + next norm)."""
    M, N = x.shape
    _ok(lib().gorch_hip_add_rmsnorm(_stream(), _p(x), _p(b), _p(gamma), _p(s), _p(y), M, N, eps))


def add(a, b, c) -> None:
    _ok(lib().gorch_hip_add(_stream(), _p(a), _p(b), _p(c), _n(a)))


def bias_add(x, bias) -> None:
    M, N = x.shape
    _ok(lib().gorch_hip_bias_add(_stream(), _p(x), _p(bias), M, N))


def gelu(x, y) -> None:
    _ok(lib().gorch_hip_gelu(_stream(), _p(x), _p(y), _n(x)))


def silu(x, y) -> None:
    _ok(lib().gorch_hip_silu(_stream(), _p(x), _p(y), _n(x)))


def swiglu(gate, value, y) -> None:
    _ok(lib().gorch_hip_swiglu(_stream(), _p(gate), _p(value), _p(y), _n(gate)))


def embedding(weight, ids, out) -> None:
    """ids: int32 device tensor."""
    _ok(lib().gorch_hip_embedding(_stream(), _p(weight), weight.shape[1], _p(ids), _n(ids), _p(out)))


def attention_cached(q, k_cache, v_cache, out, batch, new_seq, pos_offset, heads, head_dim, max_seq,
                     causal=True) -> None:
    _ok(lib().gorch_hip_attention_cached(_stream(), _p(q), _p(k_cache), _p(v_cache), _p(out), batch, new_seq,
                                         pos_offset, heads, head_dim, max_seq, int(causal)))


def causal_softmax(x, y, q_seq, scale) -> None:
    rows, cols = x.shape
    _ok(lib().gorch_hip_causal_softmax(_stream(), _p(x), _p(y), rows, cols, q_seq, scale))


def softmax_rows(x) -> None:
    rows, cols = x.shape
    _ok(lib().gorch_hip_softmax_rows(_stream(), _p(x), rows, cols))


def argmax(logits, out) -> None:
    """out: int32 device tensor [rows]."""
    rows, n = logits.shape
    _ok(lib().gorch_hip_argmax(_stream(), _p(logits), rows, n, _p(out)))


def sample(logits, temperature, top_k, top_p, u, out, probs=None) -> None:
    """sample() (model/generate.go:147-243) per row: logits f32 [rows, n],
    u f64 draws [rows], out int32 [rows], probs f64 [rows, n] or None (all
    device tensors)."""
    rows, n = logits.shape
    _ok(lib().gorch_hip_sample(_stream(), _p(logits), rows, n, float(temperature), int(top_k), float(top_p), _p(u),
                               _p(out), _p(probs)))


def sample_nucleus(logits, temperature, top_k, top_p, u, out, probs=None) -> None:
    """sampleLogits (model/qwen/generate.go:94-181) per row: the arguments of
    sample(), top-p as the Qwen loop's nucleus cut."""
    rows, n = logits.shape
    _ok(lib().gorch_hip_sample_nucleus(_stream(), _p(logits), rows, n, float(temperature), int(top_k), float(top_p),
                                       _p(u), _p(out), _p(probs)))


def sample_workspace(rows):
    """A zeroed device workspace for sample_with_workspace over `rows` rows."""
    import torch

    n = lib().gorch_hip_sample_workspace_size(rows)
    return torch.zeros(n, dtype=torch.uint8, device="cuda")


def sample_with_workspace(logits, temperature, top_k, top_p, u, out, ws, probs=None, nucleus=False) -> None:
    """sample() (or with nucleus the Qwen loop's sampleLogits) per row, the
    top-k candidate search spread over many blocks per row; ws from
    sample_workspace (left zero by every call)."""
    rows, n = logits.shape
    _ok(lib().gorch_hip_sample_with_workspace(_stream(), _p(logits), rows, n, float(temperature), int(top_k),
                                              float(top_p), _p(u), _p(out), _p(probs), int(bool(nucleus)), _p(ws)))


def linear_bf16(x, W, bias, y, residual=None, epilogue=EPI_NONE, act_bf16=False) -> None:
    """y = residual + epi(x @ W^T + bias); x [M,K] f32, W [N,K] bf16 storage.
    act_bf16: round activations to bf16 on the MFMA GEMM (one MFMA per step)."""
    M, K = x.shape
    N = W.shape[0]
    _ok(lib().gorch_hip_linear_bf16_ex(_stream(), _p(x), _p(W), _p(bias), _p(residual), _p(y), M, N, K,
                                       epilogue, LINEAR_ACT_BF16 if act_bf16 else 0))


def pack_bf16(W):
    """Tile-packed device copy of a row-major bf16 weight W [N,K] (int16
    storage): a flat int16 tensor in the decode GEMV's resident format."""
    import torch

    N, K = W.shape
    n = lib().gorch_hip_packed_bf16_bytes(N, K) // 2
    Wp = torch.empty(n, dtype=torch.int16, device=W.device)
    _ok(lib().gorch_hip_pack_bf16(_stream(), _p(W), _p(Wp), N, K))
    return Wp


def linear_bf16_packed(x, Wp, N, bias, y, residual=None, epilogue=EPI_NONE) -> None:
    """linear_bf16 over a pack_bf16 weight of N rows; M = x.shape[0] <= 16."""
    M, K = x.shape
    _ok(lib().gorch_hip_linear_bf16_packed(_stream(), _p(x), _p(Wp), _p(bias), _p(residual), _p(y), M, N, K,
                                           epilogue))


# ------------------------------------------------------------------ GPT engine

class _GPTWeights(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab", "dim", "heads", "layers", "max_seq")] + [
        ("wte", vp), ("wpe", vp),
    ] + [(n, C.POINTER(vp)) for n in (
        "ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
        "ln2_g", "ln2_b", "w1", "b1", "w2", "b2")] + [
        ("lnf_g", vp), ("lnf_b", vp), ("wlm", vp), ("blm", vp),
    ]


_LAYER_KEYS = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
               "ln2_g", "ln2_b", "w1", "b1", "w2", "b2")


ST_F32, ST_F16, ST_BF16 = 0, 1, 2
_ST_NAMES = {ST_F32: "F32", ST_F16: "F16", ST_BF16: "BF16"}


class SafeTensors:
    """A safetensors checkpoint opened through the C-ABI
    (model/safetensors.go:52-130): the header is parsed and validated on
    open (host only); tensors load on demand into device tensors."""

    def __init__(self, path: str):
        self.h = lib().gorch_hip_st_open(os.fsencode(path))
        if not self.h:
            raise HipError(2, last_error())

    def names(self) -> list:
        n = lib().gorch_hip_st_count(self.h)
        return [lib().gorch_hip_st_name(self.h, i).decode() for i in range(n)]

    def info(self, name: str):
        """(dtype name, shape tuple, stored bytes)."""
        dt, nd = C.c_int(), C.c_int()
        shape = (C.c_int64 * 8)()
        nb = C.c_int64()
        _ok(lib().gorch_hip_st_info(self.h, name.encode(), C.byref(dt), C.byref(nd), shape, C.byref(nb)))
        return _ST_NAMES[dt.value], tuple(shape[i] for i in range(nd.value)), nb.value

    def load(self, name: str, dst, dtype: int, transpose: bool = False) -> None:
        """Reads tensor ``name`` into the device tensor ``dst`` as F32 or BF16."""
        _ok(lib().gorch_hip_st_load(_stream(), self.h, name.encode(), _p(dst), dtype, 1 if transpose else 0))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().gorch_hip_st_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GenerateConfig(C.Structure):
    """gorch_hip_generate_config: GenerateConfig (model/generate.go:13-20)."""
    _fields_ = [("max_new_tokens", C.c_int), ("temperature", C.c_float), ("top_k", C.c_int),
                ("top_p", C.c_float), ("stop_token", C.c_int), ("use_kv_cache", C.c_int), ("flags", C.c_int),
                ("seed", C.c_uint64)]


class GPT:
    """gorch's nn.GPT on the GPU (nn/gpt.go:12-121). ``weights`` is a dict
    of numpy arrays in the layout gorch_amd.synthetic produces (Linear
    weights bf16 as uint16 [out, in])."""

    @classmethod
    def from_gpt2_safetensors(cls, path: str, cfg: dict) -> "GPT":
        """LoadGPT2 (model/gpt2_loader.go:56-133) from a Hugging Face GPT-2
        model.safetensors, straight into device memory."""
        h = lib().gorch_hip_gpt_load_gpt2(os.fsencode(path), cfg["vocab"], cfg["dim"], cfg["heads"],
                                          cfg["layers"], cfg["max_seq"])
        if not h:
            raise HipError(2, last_error())
        g = cls.__new__(cls)
        g.cfg = dict(cfg)
        g.h = h
        return g

    def __init__(self, weights: dict):
        import numpy as np

        cfg = weights["cfg"]
        self.cfg = dict(cfg)
        keep = []
        s = _GPTWeights()
        s.vocab, s.dim, s.heads = cfg["vocab"], cfg["dim"], cfg["heads"]
        s.layers, s.max_seq = cfg["layers"], cfg["max_seq"]
        for key in ("wte", "wpe", "lnf_g", "lnf_b", "wlm", "blm"):
            a = np.ascontiguousarray(weights[key])
            keep.append(a)
            setattr(s, key, a.ctypes.data)
        for key in _LAYER_KEYS:
            arrs = [np.ascontiguousarray(L[key]) for L in weights["layers"]]
            if key.startswith("w") and any(a.dtype != np.uint16 for a in arrs):
                raise ValueError(f"{key}: Linear weights must be bf16 (uint16 storage)")
            keep.extend(arrs)
            ptrs = (vp * len(arrs))(*[a.ctypes.data for a in arrs])
            keep.append(ptrs)
            setattr(s, key, C.cast(ptrs, C.POINTER(vp)))
        h = lib().gorch_hip_gpt_create(C.byref(s))
        if not h:
            raise HipError(4, last_error())
        self.h = h

    def new_cache(self, batch: int = 1, capacity: int | None = None) -> "KVCache":
        return KVCache(self, batch, capacity or self.cfg["max_seq"])

    def forward_cached(self, ids, cache: "KVCache"):
        """ids: [batch, n] (or [n] for batch 1) -> logits [batch*n, vocab]."""
        import numpy as np

        ids = np.ascontiguousarray(ids, np.int32)
        n = ids.shape[-1]
        out = np.empty((cache.batch * n, self.cfg["vocab"]), np.float32)
        _ok(lib().gorch_hip_gpt_forward_cached(None, self.h, cache.h, ids.ctypes.data, n, out.ctypes.data))
        return out

    def generate_cached(self, prompts, max_new: int, want_logits=False, use_graph=True):
        """Greedy generateCached for a [batch, n_prompt] array of prompts.
        Returns (ids [batch, len], step_logits or None, timing dict)."""
        import numpy as np

        prompts = np.ascontiguousarray(np.atleast_2d(prompts), np.int32)
        B, n = prompts.shape
        out = np.empty((B, n + max_new), np.int32)
        out_len = C.c_int(0)
        V = self.cfg["vocab"]
        logits = np.empty((max_new, B, V), np.float32) if want_logits else None
        timing = (C.c_float * 3)()
        _ok(lib().gorch_hip_generate_cached(None, self.h, prompts.ctypes.data, B, n, max_new, out.ctypes.data,
                                            C.byref(out_len), None if logits is None else logits.ctypes.data,
                                            timing, int(use_graph)))
        L = out_len.value
        ids = out.reshape(-1)[: B * L].reshape(B, L).copy()
        return ids, logits, {"prefill_ms": timing[0], "decode_ms": timing[1], "decode_forwards": int(timing[2])}

    def generate(self, prompts, max_new: int, stop_token: int = -1, want_logits=False, use_graph=True,
                 temperature: float = 0.0, top_k: int = 0, top_p: float = 0.0, seed: int = 0):
        """GenerateWithConfig(cfg, UseKVCache) (model/generate.go:52-131)
        for [batch, n_prompt] prompts: greedy with temperature 0, else
        sample() with top_k / top_p and Philox draws from ``seed``. Returns
        (a list of per-sequence id arrays, step logits or None, timing
        dict)."""
        import numpy as np

        prompts = np.ascontiguousarray(np.atleast_2d(prompts), np.int32)
        B, n = prompts.shape
        width = min(n, self.cfg["max_seq"]) + max_new
        out = np.zeros((B, width), np.int32)
        lens = np.zeros(B, np.int32)
        cfg = GenerateConfig(max_new, float(temperature), int(top_k), float(top_p), stop_token, 1, int(use_graph),
                             int(seed))
        V = self.cfg["vocab"]
        logits = np.empty((max_new, B, V), np.float32) if want_logits else None
        timing = (C.c_float * 3)()
        _ok(lib().gorch_hip_generate(None, self.h, prompts.ctypes.data, B, n, C.byref(cfg), out.ctypes.data,
                                     lens.ctypes.data, None if logits is None else logits.ctypes.data, timing))
        ids = [out[b, :lens[b]].copy() for b in range(B)]
        return ids, logits, {"prefill_ms": timing[0], "decode_ms": timing[1], "decode_forwards": int(timing[2])}

    def drop_packed(self) -> int:
        """Frees the engine's tile-packed weight copies (2..16-row steps then
        run the row-major GEMVs); returns the bytes freed."""
        return int(lib().gorch_hip_gpt_drop_packed(self.h))

    def close(self):
        if getattr(self, "h", None):
            lib().gorch_hip_gpt_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


class KVCache:
    """nn.KVCache (nn/kvcache.go:14-60) for ``batch`` independent sequences."""

    def __init__(self, gpt: GPT, batch: int, capacity: int):
        self.gpt = gpt
        self.batch = batch
        self.h = lib().gorch_hip_kvcache_create(gpt.h, batch, capacity)
        if not self.h:
            raise HipError(2, last_error())

    def __len__(self):
        return lib().gorch_hip_kvcache_len(self.h)

    def reset(self):
        _ok(lib().gorch_hip_kvcache_reset(self.h))

    def read(self, layer: int, seq: int = 0):
        import numpy as np

        n, d = len(self), self.gpt.cfg["dim"]
        k = np.empty((n, d), np.float32)
        v = np.empty((n, d), np.float32)
        _ok(lib().gorch_hip_kvcache_read(self.h, layer, seq, k.ctypes.data, v.ctypes.data))
        return k, v

    def close(self):
        if getattr(self, "h", None):
            lib().gorch_hip_kvcache_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


# ------------------------------------------------------------------ MoE

class _MoEWeights(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("dim", "ffn", "experts", "top_k")] + [
        (n, vp) for n in ("wr", "br", "wgate", "bgate", "wup", "bup", "wdown", "bdown")]


class MoE:
    """gorch's nn.MoE (nn/moe.go:28-182) on the GPU. ``w`` holds numpy
    arrays as gorch_amd.synthetic.moe_inputs builds them (per-expert lists);
    they are stacked and uploaded once."""

    def __init__(self, w: dict):
        import numpy as np
        import torch

        def stack(key, dtype):
            arrs = w.get(key)
            if arrs is None:
                return None
            a = np.ascontiguousarray(np.stack(arrs))
            t = torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()
            return t

        self.dim, self.ffn, self.experts, self.top_k = w["dim"], w["ffn"], w["experts"], w["top_k"]
        self.t = {k: stack(k, None) for k in ("wgate", "bgate", "wup", "bup", "wdown", "bdown")}
        self.t["wr"] = None if w.get("wr") is None else torch.from_numpy(
            np.ascontiguousarray(w["wr"]).view(np.int16)).cuda()
        self.t["br"] = None if w.get("br") is None else torch.from_numpy(np.ascontiguousarray(w["br"])).cuda()
        s = _MoEWeights()
        s.dim, s.ffn, s.experts, s.top_k = self.dim, self.ffn, self.experts, self.top_k
        for k, v in self.t.items():
            setattr(s, k, None if v is None else v.data_ptr())
        self.s = s
        self.ws = None

    def workspace(self, M):
        import torch

        n = lib().gorch_hip_moe_workspace_size(M, self.dim, self.ffn, self.experts, self.top_k)
        if self.ws is None or self.ws.numel() < n:
            self.ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        return self.ws

    def forward(self, x, logits=None, out=None):
        """x [M, dim] device f32; logits [M, experts] device f32 or None.
        Returns (out, topk_idx, topk_w) device tensors."""
        import torch

        M = x.shape[0]
        ws = self.workspace(M)
        out = torch.empty((M, self.dim), dtype=torch.float32, device="cuda") if out is None else out
        idx = torch.empty((M, self.top_k), dtype=torch.int32, device="cuda")
        wts = torch.empty((M, self.top_k), dtype=torch.float32, device="cuda")
        _ok(lib().gorch_hip_moe_forward(_stream(), C.byref(self.s), _p(x), M, _p(logits), _p(out), _p(idx),
                                        _p(wts), ws.data_ptr(), ws.numel()))
        return out, idx, wts


# ------------------------------------------------------------------ RoPE / GQA

def rope_tables(head_dim: int, max_seq: int, base: float):
    """NewRoPE's tables on the GPU: (cos, sin) [max_seq, head_dim/2]."""
    import torch

    c = torch.empty((max_seq, head_dim // 2), dtype=torch.float32, device="cuda")
    s_ = torch.empty_like(c)
    _ok(lib().gorch_hip_rope_tables(_stream(), head_dim, max_seq, base, _p(c), _p(s_)))
    return c, s_


def rope_apply(x, y, cos_t, sin_t, start_pos=0, neox=False, sign=1.0) -> None:
    """RoPE.Apply over x [..., seq, head_dim] (y may be x)."""
    seq, hd = x.shape[-2], x.shape[-1]
    outer = x.numel() // (seq * hd)
    _ok(lib().gorch_hip_rope_apply(_stream(), _p(x), _p(y), outer, seq, hd, start_pos, _p(cos_t), _p(sin_t),
                                   cos_t.shape[0], int(neox), sign))


def gqa_attention_cached(q, k_cache, v_cache, out, batch, new_seq, pos_offset, num_q, num_kv, head_dim, max_seq,
                         causal=True) -> None:
    _ok(lib().gorch_hip_gqa_attention_cached(_stream(), _p(q), _p(k_cache), _p(v_cache), _p(out), batch, new_seq,
                                             pos_offset, num_q, num_kv, head_dim, max_seq, int(causal)))


class _GQAW(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("dim", "num_q", "num_kv", "head_dim", "causal")] + [
        ("norm_eps", C.c_float)] + [(n, vp) for n in (
            "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "q_norm", "k_norm", "rope_cos", "rope_sin")] + [
        ("rope_max_seq", C.c_int), ("rope_neox", C.c_int)]


class GQA:
    """gorch's nn.GQA (nn/gqa.go) with bf16 projections on the GPU. ``w`` is a
    dict as gorch_amd.synthetic.gqa_weights builds it; the RoPE tables are
    computed on the GPU (rope_base, rope_max_seq) when w['rope'] is set."""

    def __init__(self, w: dict):
        import numpy as np
        import torch

        def up(a):
            if a is None or isinstance(a, torch.Tensor):
                return a
            a = np.ascontiguousarray(a)
            return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()

        self.w = w
        self.t = {n: up(w.get(n)) for n in ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "q_norm", "k_norm")}
        if w.get("rope"):
            if isinstance(w.get("rope_cos"), torch.Tensor):  # tables shared with other layers
                self.t["rope_cos"], self.t["rope_sin"] = w["rope_cos"], w["rope_sin"]
            else:
                self.t["rope_cos"], self.t["rope_sin"] = rope_tables(w["head_dim"], w["rope_max_seq"],
                                                                     w["rope_base"])
        s = _GQAW()
        for n in ("dim", "num_q", "num_kv", "head_dim"):
            setattr(s, n, w[n])
        s.causal = int(w.get("causal", True))
        s.norm_eps = w.get("norm_eps", 1e-6)
        for n, t in self.t.items():
            setattr(s, n, None if t is None else t.data_ptr())
        s.rope_max_seq = w["rope_max_seq"] if w.get("rope") else 0
        s.rope_neox = int(w.get("rope_neox", 0))
        self.s = s
        self.ws = None

    def forward_cached(self, x, k_cache, v_cache, pos_offset):
        """x [new_seq, dim] device; caches [capacity, num_kv*head_dim] device."""
        import torch

        S = x.shape[0]
        n = lib().gorch_hip_gqa_workspace_size(C.byref(self.s), S)
        if self.ws is None or self.ws.numel() < n:
            self.ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        out = torch.empty((S, self.w["dim"]), dtype=torch.float32, device="cuda")
        _ok(lib().gorch_hip_gqa_forward_cached(_stream(), C.byref(self.s), _p(x), S, _p(k_cache), _p(v_cache),
                                               pos_offset, k_cache.shape[0], _p(out), self.ws.data_ptr(),
                                               self.ws.numel()))
        return out


class _QwenBlockW(C.Structure):
    _fields_ = [("attn", _GQAW), ("norm_attn", vp), ("norm_ffn", vp), ("wgate_up", vp), ("wdown", vp),
                ("inter", C.c_int), ("eps", C.c_float)]


class QwenBlock:
    """model/qwen Block.ForwardCached (block.go:71-79) as one C-ABI call.
    ``attn`` is the block's GQA (its weights and RoPE tables stay owned by
    it); norm gains, the [2 * inter, dim] gate/up weight and the down weight
    are device tensors."""

    def __init__(self, attn: GQA, norm_attn, norm_ffn, wgate_up, wdown, inter: int, eps: float):
        self.attn = attn
        self.t = {"norm_attn": norm_attn, "norm_ffn": norm_ffn, "wgate_up": wgate_up, "wdown": wdown}
        s = _QwenBlockW()
        s.attn = attn.s
        for n, t in self.t.items():
            setattr(s, n, t.data_ptr())
        s.inter, s.eps = inter, eps
        self.s = s
        self.ws = None

    def forward_cached(self, x, k_cache, v_cache, pos_offset):
        """x [new_seq, dim] device f32, updated in place."""
        import torch

        S = x.shape[0]
        n = lib().gorch_hip_qwen_block_workspace_size(C.byref(self.s), S)
        if self.ws is None or self.ws.numel() < n:
            self.ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        _ok(lib().gorch_hip_qwen_block_forward_cached(_stream(), C.byref(self.s), _p(x), S, _p(k_cache),
                                                      _p(v_cache), pos_offset, k_cache.shape[0],
                                                      self.ws.data_ptr(), self.ws.numel()))
