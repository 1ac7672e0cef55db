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
    "gorch_hip_read_dispatch_counts": (i32, [C.POINTER(C.c_uint64), i32]),
    "gorch_hip_reset_dispatch_counts": (None, []),
    "gorch_hip_bf16_to_f32": (i32, [vp, vp, vp, i64]),
    "gorch_hip_f32_to_bf16": (i32, [vp, vp, vp, i64]),
    "gorch_hip_matmul_dt": (i32, [vp, vp, vp, vp, u32, u32, u32, i32, i32, i32, i32]),
    "gorch_hip_batched_matmul_dt": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, i32, i32, i32, i32]),
    "gorch_hip_linear_bf16": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
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


def linear_bf16(x, W, bias, y, residual=None, epilogue=EPI_NONE) -> None:
    """y = residual + epi(x @ W^T + bias); x [M,K] f32, W [N,K] bf16 storage."""
    M, K = x.shape
    N = W.shape[0]
    _ok(lib().gorch_hip_linear_bf16(_stream(), _p(x), _p(W), _p(bias), _p(residual), _p(y), M, N, K,
                                    epilogue))
