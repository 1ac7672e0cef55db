"""GPU tests of safetensors loading into device memory and of the GPT-2
checkpoint loader (model/safetensors.go:52-184, model/gpt2_loader.go:56-244).

Decoding is held bit-exact against its definitions: BF16 kept as stored
(LoadSafetensorsNative), BF16/F16 widened exactly, F32 rounded to BF16 with
gorch's f32ToBF16 (the oracle's codec, itself pinned exhaustively); the
2-D transpose against numpy. The GPT-2 loader is checked by writing a
checkpoint in Hugging Face's layout (Conv1D (in, out) weights, fused c_attn)
with the official `safetensors` writer and comparing the loaded engine with
one built from the same weights directly: logits bitwise equal.
"""
import numpy as np
import pytest
import torch

import oracle as orc
from gorch_amd import synthetic as syn
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def save_np(path, tensors, metadata=None):
    import safetensors.numpy
    safetensors.numpy.save_file(tensors, str(path), metadata=metadata)


def save_mixed(path, tensors):
    """numpy arrays; uint16 arrays are written as BF16."""
    import safetensors.torch
    t = {}
    for k, v in tensors.items():
        if v.dtype == np.uint16:
            t[k] = torch.from_numpy(v.view(np.int16).copy()).view(torch.bfloat16)
        else:
            t[k] = torch.from_numpy(np.ascontiguousarray(v))
    safetensors.torch.save_file(t, str(path))


def test_bf16_native_round_trip(gpu, tmp_path):
    # TestBF16SafetensorsNativeRoundTrip (model/safetensors_bf16_test.go:18-80)
    vals = np.array([0.1, 1.5, -2, 1e-3, 3.14159, -0.4567], np.float32)
    bits = orc.f32_to_bf16(vals)
    assert bits[0] == 0x3DCD and bits[1] == 0x3FC0 and bits[2] == 0xC000   # 0.1 rounds up; 1.5, -2 exact
    fvals = np.array([1, -2.5, 0.125, 9], np.float32)
    p = tmp_path / "bf16_roundtrip.safetensors"
    save_mixed(p, {"w_bf16": bits.reshape(2, 3), "w_f32": fvals})
    st = gpu.SafeTensors(str(p))
    assert st.info("w_bf16") == ("BF16", (2, 3), 12)
    out16 = torch.empty(6, dtype=torch.int16, device="cuda")
    st.load("w_bf16", out16, gpu.ST_BF16)
    assert np.array_equal(host(out16).view(np.uint16), bits)
    out32 = torch.empty(6, dtype=torch.float32, device="cuda")
    st.load("w_bf16", out32, gpu.ST_F32)
    assert np.array_equal(host(out32).view(np.uint32), orc.bf16_to_f32(bits).view(np.uint32))
    f = torch.empty(4, dtype=torch.float32, device="cuda")
    st.load("w_f32", f, gpu.ST_F32)
    assert np.array_equal(host(f), fvals)


def test_f16_exhaustive(gpu, tmp_path):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    p = tmp_path / "f16.safetensors"
    save_np(p, {"h": h.view(np.float16)})
    st = gpu.SafeTensors(str(p))
    out = torch.empty(1 << 16, dtype=torch.float32, device="cuda")
    st.load("h", out, gpu.ST_F32)
    got = host(out)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    out16 = torch.empty(1 << 16, dtype=torch.int16, device="cuda")
    st.load("h", out16, gpu.ST_BF16)
    ref16 = orc.f32_to_bf16(ref)
    g16 = host(out16).view(np.uint16)
    assert np.array_equal(g16[~nan], ref16[~nan])


def test_f32_to_bf16_rounding(gpu, tmp_path):
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    bits[:6] = [0x3F808000, 0x3F818000, 0x7F800000, 0xFF800000, 0x7FC00001, 0x00008000]  # ties, infs, NaN
    p = tmp_path / "f32.safetensors"
    save_np(p, {"x": bits.view(np.float32)})
    st = gpu.SafeTensors(str(p))
    out = torch.empty(bits.size, dtype=torch.int16, device="cuda")
    st.load("x", out, gpu.ST_BF16)
    assert np.array_equal(host(out).view(np.uint16), orc.f32_to_bf16(bits.view(np.float32)))


@pytest.mark.parametrize("R,C", [(1, 7), (33, 65), (64, 32), (300, 200), (768, 2304)])
def test_transpose_all_modes(gpu, tmp_path, R, C):
    rng = np.random.default_rng(R * C)
    f32 = rng.standard_normal((R, C)).astype(np.float32)
    b16 = orc.f32_to_bf16(rng.standard_normal((R, C)).astype(np.float32))
    f16 = rng.standard_normal((R, C)).astype(np.float16)
    p = tmp_path / "tr.safetensors"
    save_mixed(p, {"f32": f32, "b16": b16, "f16": f16})
    st = gpu.SafeTensors(str(p))
    cases = [("f32", gpu.ST_F32, f32.T), ("f32", gpu.ST_BF16, orc.f32_to_bf16(f32).T),
             ("b16", gpu.ST_BF16, b16.T), ("b16", gpu.ST_F32, orc.bf16_to_f32(b16).T),
             ("f16", gpu.ST_F32, f16.astype(np.float32).T),
             ("f16", gpu.ST_BF16, orc.f32_to_bf16(f16.astype(np.float32)).T)]
    for name, dt, ref in cases:
        out = torch.empty(R * C, dtype=torch.float32 if dt == gpu.ST_F32 else torch.int16, device="cuda")
        st.load(name, out, dt, transpose=True)
        got = host(out).reshape(C, R)
        if dt == gpu.ST_BF16:
            got = got.view(np.uint16)
        assert np.array_equal(got.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8)), (name, dt)
    with pytest.raises(gpu.HipError):   # transpose needs 2-D
        save_np(tmp_path / "v.safetensors", {"v": np.zeros(4, np.float32)})
        gpu.SafeTensors(str(tmp_path / "v.safetensors")).load(
            "v", torch.empty(4, device="cuda"), gpu.ST_F32, transpose=True)


TINY2 = dict(vocab=96, dim=64, heads=4, layers=2, max_seq=24)


def tied_weights(seed=7):
    w = syn.gpt2_weights(TINY2, seed=seed, random_affine=True)
    w["wlm"] = orc.f32_to_bf16(w["wte"])           # TieLMHeadToEmbedding, as bf16
    w["blm"] = np.zeros(TINY2["vocab"], np.float32)
    return w


def hf_checkpoint(w, linear_dtype="F32", prefix=""):
    """The weights in Hugging Face GPT-2 naming and Conv1D (in, out) layout."""
    def lin(a):  # a bf16 [out, in] weight -> Conv1D (in, out)
        t = np.ascontiguousarray(a.T)
        return t if linear_dtype == "BF16" else orc.bf16_to_f32(t)
    t = {prefix + "wte.weight": w["wte"], prefix + "wpe.weight": w["wpe"],
         prefix + "ln_f.weight": w["lnf_g"], prefix + "ln_f.bias": w["lnf_b"]}
    for i, L in enumerate(w["layers"]):
        p = f"{prefix}h.{i}."
        t[p + "ln_1.weight"], t[p + "ln_1.bias"] = L["ln1_g"], L["ln1_b"]
        t[p + "ln_2.weight"], t[p + "ln_2.bias"] = L["ln2_g"], L["ln2_b"]
        t[p + "attn.c_attn.weight"] = lin(np.concatenate([L["wq"], L["wk"], L["wv"]], axis=0))
        t[p + "attn.c_attn.bias"] = np.concatenate([L["bq"], L["bk"], L["bv"]])
        t[p + "attn.c_proj.weight"], t[p + "attn.c_proj.bias"] = lin(L["wo"]), L["bo"]
        t[p + "mlp.c_fc.weight"], t[p + "mlp.c_fc.bias"] = lin(L["w1"]), L["b1"]
        t[p + "mlp.c_proj.weight"], t[p + "mlp.c_proj.bias"] = lin(L["w2"]), L["b2"]
    return t


@pytest.mark.parametrize("linear_dtype,prefix", [("F32", ""), ("BF16", "transformer.")])
def test_gpt2_loader_matches_direct_engine(gpu, tmp_path, linear_dtype, prefix):
    w = tied_weights()
    p = tmp_path / "model.safetensors"
    save_mixed(p, hf_checkpoint(w, linear_dtype, prefix))
    loaded = gpu.GPT.from_gpt2_safetensors(str(p), TINY2)
    direct = gpu.GPT(w)
    ids = syn.prompt_ids(9, TINY2["vocab"], seed=4)
    # bit-identical engines: compared with fixed-order sums (by default the
    # batched rows' residual Linears add their K slices with float atomics)
    prev = gpu.set_deterministic(True)
    try:
        for batch in (1, 3):
            pr = np.stack([syn.prompt_ids(9, TINY2["vocab"], seed=4 + b) for b in range(batch)])
            a = loaded.forward_cached(pr, loaded.new_cache(batch, TINY2["max_seq"]))
            b = direct.forward_cached(pr, direct.new_cache(batch, TINY2["max_seq"]))
            assert np.array_equal(a, b)
    finally:
        gpu.set_deterministic(prev)
    ta, _, _ = loaded.generate_cached(ids[None, :], 10)
    tb, _, _ = direct.generate_cached(ids[None, :], 10)
    assert np.array_equal(ta, tb)
    o = orc.GPT(w)
    ref = o.forward_cached(ids, o.new_cache())
    got = loaded.forward_cached(ids[None, :], loaded.new_cache(1, TINY2["max_seq"]))
    assert rel_err(got, ref) <= 1e-3
    loaded.close()
    direct.close()


def test_gpt2_loader_errors(gpu, tmp_path):
    w = tied_weights()
    t = hf_checkpoint(w)
    del t["h.1.mlp.c_fc.bias"]
    p = tmp_path / "missing.safetensors"
    save_mixed(p, t)
    with pytest.raises(gpu.HipError) as e:
        gpu.GPT.from_gpt2_safetensors(str(p), TINY2)
    assert 'h.1.mlp.c_fc.bias" not found' in str(e.value)
    p2 = tmp_path / "ok.safetensors"
    save_mixed(p2, hf_checkpoint(w))
    with pytest.raises(gpu.HipError) as e:   # copyTensor's size check
        gpu.GPT.from_gpt2_safetensors(str(p2), dict(TINY2, max_seq=32))
    assert "size mismatch" in str(e.value)
