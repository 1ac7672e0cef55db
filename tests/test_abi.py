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


def test_attention_rejects_cache_span_of_2gib_without_gpu():
    # The attention kernels address one sequence's K/V rows with 32-bit
    # buffer offsets: a span of max_seq * kv_dim * 4 bytes at or above
    # 0x7fff0000 is refused with rc 1 (use the CPU path) before any device
    # work, for MHA and GQA alike. Just below the bound the same call gets
    # past the check (and then fails for want of a GPU, not for the span).
    import ctypes as C

    L = hip.lib()
    q = kc = vc = out = C.c_void_p(0x10000)
    # 64 heads x 128 dims = 8192 floats per row: 65,535 rows is under 2 GiB,
    # 65,536 rows is 2 GiB
    rc = L.gorch_hip_attention_cached(None, q, kc, vc, out, 1, 1, 0, 64, 128, 65536, 1)
    assert rc == 1 and "2 GiB" in hip.last_error()
    rc = L.gorch_hip_gqa_attention_cached(None, q, kc, vc, out, 1, 1, 0, 64, 64, 128, 65536, 1)
    assert rc == 1 and "2 GiB" in hip.last_error()
    # GQA: the span counts KV heads only; 8 KV heads x 128 fit at 65,536 rows
    if hip.device_count() == 0:
        rc = L.gorch_hip_gqa_attention_cached(None, q, kc, vc, out, 1, 1, 0, 64, 8, 128, 65536, 1)
        assert rc != 1 or "2 GiB" not in hip.last_error()
    rc = L.gorch_hip_attention_cached(None, q, kc, vc, out, 1, 1, 0, 64, 128, 1 << 22, 1)
    assert rc == 1


def test_sample_workspace_arguments_without_gpu():
    # gorch_hip_sample_with_workspace: its size is linear in the rows (0 for
    # none), and its argument checks come before any device work: a null
    # workspace, a temperature of 0 and a top_p without 1 <= top_k <= 4096
    # are refused like gorch_hip_sample's.
    import ctypes as C

    L = hip.lib()
    one = L.gorch_hip_sample_workspace_size(1)
    assert one > 0 and L.gorch_hip_sample_workspace_size(3) == 3 * one
    assert L.gorch_hip_sample_workspace_size(0) == 0
    fake = C.c_void_p(0x1000)

    def call(T, K, P, ws):
        return L.gorch_hip_sample_with_workspace(None, fake, 2, 50257, C.c_float(T), K, C.c_float(P), fake, fake,
                                                 None, 0, ws)

    assert call(0.8, 40, 0.9, None) == 2
    assert "workspace" in hip.last_error()
    assert call(0.0, 40, 0.9, fake) == 2
    assert call(0.8, 0, 0.9, fake) == 1
    assert call(0.8, 5000, 0.9, fake) == 1
