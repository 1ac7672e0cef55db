"""CPU-only checks of the C-ABI boundary: the library loads without a GPU and
exports every entry point include/gorch_hip.h declares, and the Python
binding covers each of them. No compute call is made here."""
import ctypes
import os
import re

from gorch_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names |= set(re.findall(r"\b(gorch_hip_\w+)\s*\(", src))
    return names


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "gorch_hip_matmul_dt" in names and "gorch_hip_linear_bf16" in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(hip.LIB_PATH)
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_covers_every_declared_symbol():
    missing = sorted(declared_symbols() - set(hip.SIGNATURES))
    assert not missing, f"no ctypes signature for: {missing}"
    hip.lib()  # loads and binds every signature


def test_error_string_without_gpu():
    # Init on a machine without gfx950 must fail cleanly with a message.
    if hip.device_count() == 0:
        rc = hip.lib().gorch_hip_init(0)
        assert rc != 0
        assert hip.last_error()


def test_moe_rejects_bad_shapes_without_gpu():
    # Argument checks come before any device work (nn/moe.go:130-140's
    # panics become rc 2): top-k above 8, dim not a multiple of 8, and the
    # 32-bit buffer-offset bound M * top_k * dim < 2^29.
    import ctypes as C

    ws = hip._MoEWeights()
    fake = C.c_void_p(0x1000)
    ws.wgate = ws.wup = ws.wdown = fake
    ws.wr = fake
    x = out = C.c_void_p(0x2000)
    L = hip.lib()

    def call(dim, ffn, experts, top_k, M):
        ws.dim, ws.ffn, ws.experts, ws.top_k = dim, ffn, experts, top_k
        return L.gorch_hip_moe_forward(None, C.byref(ws), x, M, None, out, None, None, fake, 1 << 40)

    assert call(64, 64, 16, 9, 8) == 2
    assert call(60, 64, 8, 2, 8) == 2
    assert call(1024, 64, 8, 2, 1 << 18) == 2
    assert "2^29" in hip.last_error()
    assert hip.lib().gorch_hip_moe_workspace_size(8, 64, 64, 8, 0) == 0
