"""GPU parity of the GPT decode engine (fused QKV GEMV -> KV cache ->
attention -> fused residual GEMVs -> LM head -> argmax) against the CPU
oracle's GPT.ForwardCached / generateCached, through the C-ABI.

Bars: logits within 1e-3 of RMS for a forward;
greedy tokens identical; full-run logits within 2e-2 of RMS. The reference
invariants are re-checked on the GPU path: cached prefill + steps equals a
one-shot forward over the whole sequence (nn/kvcache_test.go:53-114), the
cache length advances (:116-141), and generation stops at MaxSeq
(model/generate.go:119-124).
"""
import numpy as np
import pytest

import oracle as orc
from gorch_amd import synthetic as syn
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

TINY = dict(vocab=64, dim=32, heads=4, layers=2, max_seq=40)


def tiny_weights(seed=31):
    w = syn.gpt2_weights(TINY, seed=seed, random_affine=True)
    from gorch_amd import bf16 as hb
    for L in w["layers"]:   # sharper attention so mistakes in it show
        for key in ("wq", "wk"):
            L[key] = hb.f32_to_bf16(hb.bf16_to_f32(L[key]) * 20)
    return w


@pytest.fixture(scope="module")
def tiny(gpu):
    w = tiny_weights()
    return w, gpu.GPT(w), orc.GPT(w)


def test_forward_cached_prefill_and_steps(tiny):
    w, g, o = tiny
    ids = syn.prompt_ids(11, TINY["vocab"], seed=1)
    gc, oc = g.new_cache(1, TINY["max_seq"]), o.new_cache()
    for chunk in (ids[:8], ids[8:9], ids[9:11]):
        got = g.forward_cached(chunk[None, :], gc)
        ref = o.forward_cached(chunk, oc)
        assert rel_err(got, ref) <= 1e-3
        assert len(gc) == len(oc)
    for layer in range(TINY["layers"]):
        k, v = gc.read(layer)
        assert rel_err(k, oc.keys(layer).reshape(k.shape)) <= 1e-4
        assert rel_err(v, oc.values(layer).reshape(v.shape)) <= 1e-4


def test_cached_steps_equal_one_shot(tiny):
    w, g, o = tiny
    ids = syn.prompt_ids(12, TINY["vocab"], seed=2)
    c1 = g.new_cache(1, 20)
    full = g.forward_cached(ids[None, :], c1)
    c2 = g.new_cache(1, 20)
    rows = [g.forward_cached(ids[None, :5], c2)]
    for t in range(5, 12):
        rows.append(g.forward_cached(ids[None, t:t + 1], c2))
    assert np.max(np.abs(np.concatenate(rows) - full)) < 1e-3


def test_forward_cached_capacity_error(tiny, gpu):
    w, g, o = tiny
    c = g.new_cache(1, 4)
    g.forward_cached(np.zeros((1, 3), np.int32), c)
    with pytest.raises(gpu.HipError):
        g.forward_cached(np.zeros((1, 2), np.int32), c)
    c.reset()
    assert len(c) == 0
    g.forward_cached(np.zeros((1, 4), np.int32), c)


def test_generate_tokens_identical(tiny):
    w, g, o = tiny
    prompt = syn.prompt_ids(6, TINY["vocab"], seed=3)
    ref_ids, ref_logits, gaps = o.generate_cached(prompt, 30, want_logits=True)
    ids, logits, _ = g.generate_cached(prompt[None, :], 30, want_logits=True)
    assert list(ids[0]) == list(ref_ids)
    for i in range(30):
        assert rel_err(logits[i, 0], ref_logits[i]) <= 1e-3
    ids_graph, _, t = g.generate_cached(prompt[None, :], 30, use_graph=True)
    assert np.array_equal(ids_graph, ids)
    assert t["decode_forwards"] == 30


def test_generate_batch_matches_per_sequence(tiny):
    w, g, o = tiny
    prompts = np.stack([syn.prompt_ids(7, TINY["vocab"], seed=10 + b) for b in range(3)])
    ids, _, _ = g.generate_cached(prompts, 12)
    for b in range(3):
        ref, _, _ = o.generate_cached(prompts[b], 12)
        assert list(ids[b]) == list(ref)


def test_generate_stops_at_max_seq(tiny):
    w, g, o = tiny
    prompt = syn.prompt_ids(TINY["max_seq"] - 2, TINY["vocab"], seed=4)
    ids, _, t = g.generate_cached(prompt[None, :], 10)
    ref, _, _ = o.generate_cached(prompt, 10)
    assert ids.shape[1] == TINY["max_seq"] + 1 == len(ref)
    assert list(ids[0]) == list(ref)
    assert t["decode_forwards"] == 2


def test_generate_truncates_long_prompt(tiny):
    w, g, o = tiny
    prompt = syn.prompt_ids(TINY["max_seq"] + 5, TINY["vocab"], seed=5)
    ids, _, _ = g.generate_cached(prompt[None, :], 3)
    ref, _, _ = o.generate_cached(prompt, 3)
    assert list(ids[0]) == list(ref)


@pytest.fixture(scope="module")
def gpt2_small(gpu):
    w = syn.gpt2_weights(syn.GPT2_SMALL, seed=0)
    return w, gpu.GPT(w), orc.GPT(w)


def test_gpt2_small_greedy_decode(gpt2_small):
    """GPT-2 small, bf16 weights N(0,0.02), 32-token
    seeded prompt, 64 greedy tokens with the KV cache, batch 1."""
    w, g, o = gpt2_small
    prompt = syn.prompt_ids(32, syn.GPT2_SMALL["vocab"], seed=0)
    orc.set_widen_per_call(False)     # same numerics, widened once
    try:
        ref_ids, ref_logits, gaps = o.generate_cached(prompt, 64, want_logits=True)
    finally:
        orc.set_widen_per_call(True)
    ids, logits, _ = g.generate_cached(prompt[None, :], 64, want_logits=True)
    print(f"min top-1/top-2 logit gap over 64 steps: {float(np.min(gaps)):.3e}")
    assert list(ids[0]) == list(ref_ids)
    assert rel_err(logits[0, 0], ref_logits[0]) <= 1e-3          # prefill logits
    assert rel_err(logits[:, 0], ref_logits) <= 2e-2             # full run
    ids_graph, _, _ = g.generate_cached(prompt[None, :], 64, use_graph=True)
    assert np.array_equal(ids_graph, ids)


def test_generate_batch_above_16(tiny):
    # batches over 16 take the standalone argmax path instead of the fused one
    w, g, o = tiny
    prompts = np.stack([syn.prompt_ids(3, TINY["vocab"], seed=40 + b) for b in range(17)])
    ids, _, _ = g.generate_cached(prompts, 5)
    for b in (0, 9, 16):
        ref, _, _ = o.generate_cached(prompts[b], 5)
        assert list(ids[b]) == list(ref)


WIDE = dict(vocab=16400, dim=1600, heads=25, layers=1, max_seq=24)


@pytest.fixture(scope="module")
def wide(gpu):
    w = syn.gpt2_weights(WIDE, seed=41, random_affine=True)
    return w, gpu.GPT(w), orc.GPT(w)


@pytest.mark.parametrize("batch", [4, 16])
def test_generate_batch_wide_lm_head(wide, batch):
    """Batched decode whose LM head has >= 1024 16-row weight tiles and
    K = 1600 (the GPT-2 XL width): the multi-row GEMV with the final
    LayerNorm and the argmax fused, activations staged in LDS. Tokens
    identical to the oracle run per sequence, eager and graph-replayed."""
    w, g, o = wide
    prompts = np.stack([syn.prompt_ids(6, WIDE["vocab"], seed=60 + b) for b in range(batch)])
    ids, logits, _ = g.generate_cached(prompts, 8, want_logits=True)
    for b in range(batch):
        ref, ref_logits, _ = o.generate_cached(prompts[b], 8, want_logits=True)
        assert list(ids[b]) == list(ref)
        assert rel_err(logits[0, b], ref_logits[0]) <= 1e-3
    ids_graph, _, _ = g.generate_cached(prompts, 8, use_graph=True)
    assert np.array_equal(ids_graph, ids)


def test_generate_batch_wide_model(gpu):
    """Batched decode of a model wider than the per-row reducer (d = 2176 >
    2048): the engine keeps the unsplit fused GEMVs; tokens identical to the
    oracle per sequence."""
    cfg = dict(vocab=64, dim=2176, heads=17, layers=1, max_seq=16)
    w = syn.gpt2_weights(cfg, seed=43, random_affine=True)
    g, o = gpu.GPT(w), orc.GPT(w)
    prompts = np.stack([syn.prompt_ids(4, cfg["vocab"], seed=70 + b) for b in range(2)])
    ids, _, _ = g.generate_cached(prompts, 5)
    for b in range(2):
        ref, _, _ = o.generate_cached(prompts[b], 5)
        assert list(ids[b]) == list(ref)
    g.close()


def test_generate_long_cache(gpu):
    """Batched decode with a cache of 300 positions (the long-cache attention
    kernel); greedy tokens identical to the oracle, logits of the first step
    within 1e-3."""
    cfg = dict(vocab=64, dim=64, heads=4, layers=2, max_seq=300)
    w = syn.gpt2_weights(cfg, seed=44, random_affine=True)
    g, o = gpu.GPT(w), orc.GPT(w)
    prompts = np.stack([syn.prompt_ids(270, cfg["vocab"], seed=80 + b) for b in range(3)])
    ids, logits, _ = g.generate_cached(prompts, 12, want_logits=True)
    for b in range(3):
        ref, ref_logits, _ = o.generate_cached(prompts[b], 12, want_logits=True)
        assert list(ids[b]) == list(ref)
        assert rel_err(logits[0][b], ref_logits[0]) <= 1e-3
    g.close()


@pytest.mark.parametrize("prompt", [270, 40])
def test_generate_long_cache_batch1(gpu, prompt):
    """One sequence over a cache of 300 positions: the key-split long-cache
    attention (each head's keys over several blocks, their records merged by
    the combine kernel). A 40-token prompt leaves most key chunks empty.
    Greedy tokens identical to the oracle, first-step logits within 1e-3."""
    cfg = dict(vocab=64, dim=128, heads=2, layers=2, max_seq=300)
    w = syn.gpt2_weights(cfg, seed=45, random_affine=True)
    g, o = gpu.GPT(w), orc.GPT(w)
    prompts = syn.prompt_ids(prompt, cfg["vocab"], seed=81)[None, :]
    ids, logits, _ = g.generate_cached(prompts, 12, want_logits=True)
    ref, ref_logits, _ = o.generate_cached(prompts[0], 12, want_logits=True)
    assert list(ids[0]) == list(ref)
    assert rel_err(logits[0][0], ref_logits[0]) <= 1e-3
    g.close()


XL2 = dict(vocab=50257, dim=1600, heads=25, layers=2, max_seq=768)


def test_generate_gpt2_xl_width_batch16(gpu):
    """BASELINE configs[4] at its full per-step shape with 2 of its 48 layers:
    d 1600, 25 heads of 64, vocab 50257, batch 16, 512-token prompts (the
    matrix-core prefill GEMMs, flash attention over 512 rows, K/V rows
    written into the cache segments by the fused QKV GEMM), then 256 greedy
    steps through the batched decode path (tile-packed GEMVs reading their
    activations in the MFMA fragment layout, the fused QKV split over K with
    the attention adding its slices, Wo/FFN2 K slices added into the
    residual with float atomics and the LayerNorm row passes, the 16-wave
    two-pass attention kernel at 400 (head, row) blocks, the LM head with
    the argmax fused) out to a 768-row cache.
    Every sequence against the oracle's generateCached: tokens identical
    over all 256 steps, first-step logits within 1e-3 and the run's within
    2e-2; the graph-replayed run gives the same tokens."""
    w = syn.gpt2_weights(XL2, seed=90, random_affine=True)
    g, o = gpu.GPT(w), orc.GPT(w)
    B, P, steps = 16, 512, 256
    prompts = np.stack([syn.prompt_ids(P, XL2["vocab"], seed=200 + b) for b in range(B)])
    ids, logits, _ = g.generate_cached(prompts, steps, want_logits=True)
    assert ids.shape == (B, P + steps)
    orc.set_widen_per_call(False)
    try:
        gaps = []
        for b in range(B):
            ref, ref_logits, gap = o.generate_cached(prompts[b], steps, want_logits=True)
            gaps.append(float(np.min(gap)))
            assert list(ids[b]) == list(ref), b
            assert rel_err(logits[0, b], ref_logits[0]) <= 1e-3, b
            assert rel_err(logits[:, b], ref_logits) <= 2e-2, b
    finally:
        orc.set_widen_per_call(True)
    print(f"min top-1/top-2 logit gap: {min(gaps):.3e}")
    del logits
    ids_graph, _, t = g.generate_cached(prompts, steps, use_graph=True)
    assert np.array_equal(ids_graph, ids)
    assert t["decode_forwards"] == steps
    g.close()


@pytest.mark.parametrize("use_graph", [False, True])
def test_generate_stop_token(tiny, use_graph):
    """GenerateConfig.StopToken (model/generate.go:116-118) per sequence: each
    sequence ends before the first occurrence of the stop token, which it
    does not keep; sequences that never produce it run to max_new. The
    token is chosen from the oracle's own unstopped runs so that it occurs
    in some sequences and not in others."""
    w, g, o = tiny
    prompts = np.stack([syn.prompt_ids(5, TINY["vocab"], seed=90 + b) for b in range(4)])
    runs = [o.generate_cached(prompts[b], 20)[0][5:] for b in range(4)]
    counts = np.zeros(TINY["vocab"], int)
    for r in runs:
        counts[np.unique(r)] += 1
    cand = [t for t in range(TINY["vocab"]) if 0 < counts[t] < 4]
    stop = cand[0] if cand else int(runs[0][3])
    ids, _, t = g.generate(prompts, 20, stop_token=stop, use_graph=use_graph)
    for b in range(4):
        ref, _, _ = o.generate_cached(prompts[b], 20, stop_token=stop)
        assert list(ids[b]) == list(ref), b
    if all(stop in r for r in runs):
        assert t["decode_forwards"] < 20
    # no stop token: the same as generate_cached
    ids2, _, _ = g.generate(prompts, 20, use_graph=use_graph)
    full, _, _ = g.generate_cached(prompts, 20, use_graph=use_graph)
    assert all(np.array_equal(ids2[b], full[b]) for b in range(4))


@pytest.mark.parametrize("cfg,prompt,batch", [
    # one sequence, short cache: the one-pass attention kernel with Wo fused
    # by float atomics in the default mode
    (dict(vocab=64, dim=64, heads=4, layers=2, max_seq=64), 20, 1),
    # one sequence, 300-row cache: the key-split attention with Wo in its
    # chunk merge in the default mode
    (dict(vocab=64, dim=128, heads=2, layers=2, max_seq=300), 270, 1),
    # four sequences: the batched step, whose Wo and FFN2 K slices add
    # themselves into the residual stream with float atomics in the default
    # mode (K 1024 / 4096: four and seven slices)
    (dict(vocab=96, dim=1024, heads=8, layers=2, max_seq=64), 24, 4),
])
def test_deterministic_mode_bit_identical(gpu, cfg, prompt, batch):
    """gorch_hip_set_deterministic(1): the decode step takes the output
    projection as a GEMV of its own and the batched residual Linears' K
    slices are summed in slice order (no float atomics), so two runs give
    bit-identical logits, tokens identical to the oracle and first-step
    logits within 1e-3 (model/generate.go:134-144 is a fixed-order loop).
    The default (atomic) mode matches the oracle to the same bar."""
    w = syn.gpt2_weights(cfg, seed=46, random_affine=True)
    g, o = gpu.GPT(w), orc.GPT(w)
    prompts = np.stack([syn.prompt_ids(prompt, cfg["vocab"], seed=82 + b) for b in range(batch)])
    refs = [o.generate_cached(prompts[b], 10, want_logits=True) for b in range(batch)]
    prev = gpu.set_deterministic(True)
    try:
        assert gpu.deterministic_enabled()
        runs = []
        for use_graph in (False, True, True):
            ids, logits, _ = g.generate_cached(prompts, 10, want_logits=True, use_graph=use_graph)
            for b, (ref, ref_logits, _) in enumerate(refs):
                assert list(ids[b]) == list(ref)
                assert rel_err(logits[0][b], ref_logits[0]) <= 1e-3
                assert rel_err(logits[:, b], ref_logits) <= 2e-2
            runs.append(logits)
        assert np.array_equal(runs[0], runs[1]) and np.array_equal(runs[1], runs[2])
    finally:
        gpu.set_deterministic(prev)
    assert not gpu.deterministic_enabled()
    ids, logits, _ = g.generate_cached(prompts, 10, want_logits=True)
    for b, (ref, ref_logits, _) in enumerate(refs):
        assert list(ids[b]) == list(ref)
        assert rel_err(logits[0][b], ref_logits[0]) <= 1e-3
    g.close()


@pytest.mark.parametrize("use_graph", [False, True])
@pytest.mark.parametrize("T,K,P", [(1.0, 0, 0.0), (0.8, 10, 0.9), (1.5, 5, 0.4)])
def test_generate_sampled_matches_oracle(tiny, use_graph, T, K, P):
    """GenerateWithConfig with Temperature > 0 and the KV cache
    (model/generate.go:94-131, sample() at :147-243): every new token drawn
    from the step's logits with the Philox draw (seed, token index,
    sequence); token-identical to the oracle's generateCached + sample()
    given the same draws, for 4 sequences and 20 tokens."""
    w, g, o = tiny
    prompts = np.stack([syn.prompt_ids(6, TINY["vocab"], seed=120 + b) for b in range(4)])
    ids, _, _ = g.generate(prompts, 20, use_graph=use_graph, temperature=T, top_k=K, top_p=P, seed=2024)
    for b in range(4):
        ref = o.generate_sampled(prompts[b], 20, T, K, P, 2024, row=b)
        assert list(ids[b]) == list(ref), b


def test_generate_sampled_seed_and_stop(tiny):
    w, g, o = tiny
    prompts = np.stack([syn.prompt_ids(6, TINY["vocab"], seed=130 + b) for b in range(2)])
    a, _, _ = g.generate(prompts, 16, temperature=1.0, seed=5)
    b_, _, _ = g.generate(prompts, 16, temperature=1.0, seed=5)
    c, _, _ = g.generate(prompts, 16, temperature=1.0, seed=6)
    assert all(np.array_equal(a[i], b_[i]) for i in range(2))
    assert any(not np.array_equal(a[i], c[i]) for i in range(2))
    # top_k = 1 keeps only the maximum: the greedy tokens
    s1, _, _ = g.generate(prompts, 16, temperature=0.7, top_k=1, seed=9)
    gr, _, _ = g.generate(prompts, 16)
    assert all(np.array_equal(s1[i], gr[i]) for i in range(2))
    # a stop token drawn in the sampled run ends that sequence without it
    stop = int(a[0][8])
    st, _, _ = g.generate(prompts, 16, stop_token=stop, temperature=1.0, seed=5)
    for i in range(2):
        ref = o.generate_sampled(prompts[i], 16, 1.0, 0, 0.0, 5, row=i, stop_token=stop)
        assert list(st[i]) == list(ref), i


def test_generate_sampled_gpt2_vocab(gpu):
    """The sampler at GPT-2's vocabulary (50,257 logits per row, top-k 40,
    temperature 0.8: the reference's DefaultGenerateConfig) over a small
    model, 2 sequences, graph-replayed steps."""
    cfg = dict(vocab=50257, dim=64, heads=4, layers=2, max_seq=48)
    w = syn.gpt2_weights(cfg, seed=47, random_affine=True)
    g, o = gpu.GPT(w), orc.GPT(w)
    prompts = np.stack([syn.prompt_ids(8, cfg["vocab"], seed=140 + b) for b in range(2)])
    ids, _, _ = g.generate(prompts, 12, temperature=0.8, top_k=40, seed=77)
    for b in range(2):
        ref = o.generate_sampled(prompts[b], 12, 0.8, 40, 0.0, 77, row=b)
        assert list(ids[b]) == list(ref), b
    g.close()


def test_generate_sampled_argument_errors(tiny, gpu):
    w, g, o = tiny
    prompts = np.stack([syn.prompt_ids(4, TINY["vocab"], seed=150 + b) for b in range(17)])
    with pytest.raises(gpu.HipError) as e:   # sampled generation: up to 16 sequences
        g.generate(prompts, 4, temperature=1.0)
    assert e.value.rc == 1
    with pytest.raises(gpu.HipError) as e:   # top-p needs 1 <= top_k <= 4096
        g.generate(prompts[:2], 4, temperature=1.0, top_p=0.5)
    assert e.value.rc == 1


def test_drop_packed_weights(gpu):
    """gorch_hip_gpt_drop_packed: the engine frees its tile-packed weight
    copies (the bytes of its bf16 Linear and LM-head weights again) and its
    captured step; batched decode then runs the row-major GEMVs with the
    same greedy tokens as the oracle, eager and graph-replayed."""
    cfg = dict(vocab=4096, dim=1024, heads=16, layers=2, max_seq=48)
    w = syn.gpt2_weights(cfg, seed=47, random_affine=True)
    g, o = gpu.GPT(w), orc.GPT(w)
    prompts = np.stack([syn.prompt_ids(12, cfg["vocab"], seed=120 + b) for b in range(4)])
    refs = [o.generate_cached(prompts[b], 10, want_logits=True) for b in range(4)]
    before, _, _ = g.generate_cached(prompts, 10, use_graph=True)
    d, V, L = cfg["dim"], cfg["vocab"], cfg["layers"]
    freed = g.drop_packed()
    assert freed >= 2 * (L * 12 * d * d + V * d)
    assert g.drop_packed() == 0
    for use_graph in (False, True):
        ids, logits, _ = g.generate_cached(prompts, 10, want_logits=True, use_graph=use_graph)
        assert np.array_equal(ids, before)
        for b, (ref, ref_logits, _) in enumerate(refs):
            assert list(ids[b]) == list(ref)
            assert rel_err(logits[0, b], ref_logits[0]) <= 1e-3
    g.close()
