"""GPU parity of the Qwen3-style decoder (gorch_amd.qwen; model/qwen/qwen.go:
69-89, block.go:71-79) against the same model composed from the CPU oracle's
functions: greedy tokens identical, last-row logits within 1e-3 relative
(the reference's own bar for cached vs one-shot logits), prefill then
one-token steps, and the cache rows the layers wrote.
"""
import numpy as np
import pytest
import torch

import oracle as orc
from gorch_amd import synthetic as syn
from gorch_amd.qwen import Qwen, QwenConfig
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

TINY = QwenConfig(hidden=64, layers=2, num_q=4, num_kv=2, head_dim=32, inter=96, vocab=300, max_seq=64)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


class OracleQwen:
    """The same model on the oracle (the GQA layers take the GPU's RoPE
    tables, so the check isolates the composition)."""

    def __init__(self, cfg, w, model):
        self.cfg, self.w = cfg, w
        self.embed = orc.bf16_to_f32(w["embed"]).reshape(cfg.vocab, cfg.hidden)
        self.gqa = []
        for lw, layer in zip(w["layers"], model.layers):
            t = layer["attn"].t
            gw = {"dim": cfg.hidden, "num_q": cfg.num_q, "num_kv": cfg.num_kv,
                  "head_dim": cfg.head_dim, "causal": True, "norm_eps": cfg.eps,
                  "wq": lw["wq"], "wk": lw["wk"], "wv": lw["wv"], "wo": lw["wo"],
                  "rope_cos": host(t["rope_cos"]), "rope_sin": host(t["rope_sin"])}
            for n in ("q_norm", "k_norm", "bq", "bk", "bv"):
                if lw.get(n) is not None:
                    gw[n] = lw[n]
            self.gqa.append(gw)
        cap = cfg.max_seq
        self.cache = [(np.zeros((cap, cfg.kv_dim), np.float32), np.zeros((cap, cfg.kv_dim), np.float32))
                      for _ in w["layers"]]

    def forward_cached(self, ids, pos):
        cfg = self.cfg
        x = orc.embedding_lookup(self.embed, np.asarray(ids, np.int32))
        for lw, gw, (kc, vc) in zip(self.w["layers"], self.gqa, self.cache):
            h = orc.rmsnorm(x, lw["norm_attn"], cfg.eps)
            x1 = orc.add(x, orc.gqa_forward_cached(gw, kc, vc, pos, h))
            h2 = orc.rmsnorm(x1, lw["norm_ffn"], cfg.eps)
            hid = orc.swiglu(orc.linear(h2, lw["wgate"]), orc.linear(h2, lw["wup"]))
            x = orc.add(x1, orc.linear(hid, lw["wdown"]))
        last = orc.rmsnorm(x[-1:], self.w["norm"], cfg.eps)
        return orc.linear(last, self.w["embed"])


@pytest.mark.parametrize("n_prompt", [6, 40])
def test_qwen_greedy_matches_oracle(gpu, n_prompt):
    # 40 prompt rows: the Linears take the MFMA GEMM and the attention the
    # prefill kernel; 6 rows: the decode kernels throughout
    w = syn.qwen_weights(TINY, seed=3)
    m = Qwen(TINY, w)
    ref = OracleQwen(TINY, w, m)
    cache = m.new_cache(TINY.max_seq)
    rng = np.random.default_rng(n_prompt)
    ids = rng.integers(0, TINY.vocab, n_prompt).astype(np.int32)
    pos = 0
    toks, ref_toks = [], []
    for step in range(6):
        got = host(m.forward_cached(torch.from_numpy(ids).cuda(), cache, pos))
        want = ref.forward_cached(ids, pos)
        assert rel_err(got, want) <= 1e-3, step
        nxt, ref_nxt = int(np.argmax(got[0])), orc.argmax(want)
        toks.append(nxt)
        ref_toks.append(ref_nxt)
        assert nxt == ref_nxt, (step, toks, ref_toks)
        pos += ids.size
        ids = np.array([nxt], np.int32)
    for (kd, vd), (kc, vc) in zip(cache, ref.cache):
        assert rel_err(host(kd)[:pos], kc[:pos]) <= 1e-4
        assert rel_err(host(vd)[:pos], vc[:pos]) <= 1e-4


def test_qwen_rejects_overflow(gpu):
    w = syn.qwen_weights(TINY, seed=4)
    m = Qwen(TINY, w)
    cache = m.new_cache(8)
    with pytest.raises(ValueError):
        m.forward_cached(torch.zeros(9, dtype=torch.int32, device="cuda"), cache, 0)
    with pytest.raises(ValueError):
        m.new_cache(TINY.max_seq + 1)


def test_qwen_greedy_long_cache(gpu):
    """A cache longer than 256 rows: 270-row prefill (matrix-core GEMMs and
    flash attention), then one-token steps through the online-softmax
    long-cache attention kernel (4 query heads over 2 KV heads)."""
    cfg = QwenConfig(hidden=64, layers=2, num_q=4, num_kv=2, head_dim=32, inter=96, vocab=300, max_seq=320)
    w = syn.qwen_weights(cfg, seed=5)
    m = Qwen(cfg, w)
    ref = OracleQwen(cfg, w, m)
    cache = m.new_cache(cfg.max_seq)
    ids = np.random.default_rng(11).integers(0, cfg.vocab, 270).astype(np.int32)
    pos = 0
    for step in range(5):
        got = host(m.forward_cached(torch.from_numpy(ids).cuda(), cache, pos))
        want = ref.forward_cached(ids, pos)
        assert rel_err(got, want) <= 1e-3, step
        nxt = int(np.argmax(got[0]))
        assert nxt == orc.argmax(want), step
        pos += ids.size
        ids = np.array([nxt], np.int32)
    for (kd, vd), (kc, vc) in zip(cache, ref.cache):
        assert rel_err(host(kd)[:pos], kc[:pos]) <= 1e-4
        assert rel_err(host(vd)[:pos], vc[:pos]) <= 1e-4


def test_qwen25_style_bias_no_qk_norm(gpu):
    """The Qwen2.5 configuration switches (config.go:61-78): q/k/v projection
    biases on, per-head q/k RMSNorm off; greedy tokens and logits against the
    oracle composition, and a config that disagrees with the weights is
    refused rather than silently ignoring them."""
    import dataclasses
    cfg = dataclasses.replace(TINY, attn_bias=True, use_qk_norm=False)
    w = syn.qwen_weights(cfg, seed=7)
    m = Qwen(cfg, w)
    ref = OracleQwen(cfg, w, m)
    cache = m.new_cache(cfg.max_seq)
    ids = np.random.default_rng(12).integers(0, cfg.vocab, 9).astype(np.int32)
    pos = 0
    for step in range(4):
        got = host(m.forward_cached(torch.from_numpy(ids).cuda(), cache, pos))
        want = ref.forward_cached(ids, pos)
        assert rel_err(got, want) <= 1e-3, step
        nxt = int(np.argmax(got[0]))
        assert nxt == orc.argmax(want), step
        pos += ids.size
        ids = np.array([nxt], np.int32)
    with pytest.raises(ValueError):
        Qwen(TINY, w)                      # weights carry biases, config says none
    with pytest.raises(ValueError):
        Qwen(dataclasses.replace(cfg, tied_embeddings=False), w)


@pytest.mark.parametrize("cfg_kw", [
    # inter 256: the one-row MLP path (RMSNorm in the gate/up GEMV's loads,
    # SwiGLU in the down GEMV's loads)
    dict(hidden=128, layers=2, num_q=4, num_kv=2, head_dim=32, inter=256, vocab=500, max_seq=48),
    # Qwen3-0.6B width (d 1024, 16 / 8 heads of 128, SwiGLU 3072), two of its
    # 28 layers and a small vocabulary: the shapes the decode bench times
    dict(hidden=1024, layers=2, num_q=16, num_kv=8, head_dim=128, inter=3072, vocab=1000, max_seq=48),
    # the same width past one 32-key chunk: one-token steps through the
    # key-split attention with q/k norm and RoPE inside it
    dict(hidden=1024, layers=2, num_q=16, num_kv=8, head_dim=128, inter=3072, vocab=1000, max_seq=80,
         prefill=40)])
def test_qwen_fused_block_steps(gpu, cfg_kw):
    """The one-token block (gorch_hip_qwen_block_forward_cached) against the
    oracle composition of model/qwen's block: a 7-token (or longer) prefill
    (the separate-kernel path), then one-token steps (the fused path); greedy
    tokens identical, logits within 1e-3, cache rows within 1e-4."""
    cfg_kw = dict(cfg_kw)
    prefill = cfg_kw.pop("prefill", 7)
    cfg = QwenConfig(**cfg_kw)
    w = syn.qwen_weights(cfg, seed=21)
    m = Qwen(cfg, w)
    ref = OracleQwen(cfg, w, m)
    cache = m.new_cache(cfg.max_seq)
    ids = np.random.default_rng(22).integers(0, cfg.vocab, prefill).astype(np.int32)
    pos = 0
    for step in range(6):
        got = host(m.forward_cached(torch.from_numpy(ids).cuda(), cache, pos))
        want = ref.forward_cached(ids, pos)
        assert rel_err(got, want) <= 1e-3, step
        nxt = int(np.argmax(got[0]))
        assert nxt == orc.argmax(want), step
        pos += ids.size
        ids = np.array([nxt], np.int32)
    for (kd, vd), (kc, vc) in zip(cache, ref.cache):
        assert rel_err(host(kd)[:pos], kc[:pos]) <= 1e-4
        assert rel_err(host(vd)[:pos], vc[:pos]) <= 1e-4


@pytest.mark.parametrize("preset", ["qwen3_0_6b", "qwen2_5_0_5b"])
def test_qwen_full_size_greedy(gpu, preset):
    """The presets at full size (Qwen3-0.6B: 28 layers, d 1024, 16 / 8 heads
    of 128, SwiGLU 3072, vocab 151936, tied head, q/k norm; Qwen2.5-0.5B: 24
    layers, d 896, 14 / 2 heads of 64, SwiGLU 4864, q/k/v biases) with random
    weights, a 70-token prefill (matrix-core GEMMs, flash attention) and 4
    one-token steps through the serving path the decode bench times (past one
    key chunk: the key-split attention), against the oracle composition:
    greedy tokens identical, logits within 1e-3, cache rows within 1e-4."""
    import dataclasses

    from gorch_amd.qwen import QWEN2_5_0_5B, QWEN3_0_6B
    base = QWEN3_0_6B if preset == "qwen3_0_6b" else QWEN2_5_0_5B
    cfg = dataclasses.replace(base, max_seq=96)
    w = syn.qwen_weights(cfg, seed=31)
    m = Qwen(cfg, w)
    ref = OracleQwen(cfg, w, m)
    cache = m.new_cache(cfg.max_seq)
    ids = np.random.default_rng(32).integers(0, cfg.vocab, 70).astype(np.int32)
    pos = 0
    for step in range(5):
        got = host(m.forward_cached(torch.from_numpy(ids).cuda(), cache, pos))
        want = ref.forward_cached(ids, pos)
        assert rel_err(got, want) <= 1e-3, step
        nxt = int(np.argmax(got[0]))
        assert nxt == orc.argmax(want), step
        pos += ids.size
        ids = np.array([nxt], np.int32)
    for (kd, vd), (kc, vc) in zip(cache, ref.cache):
        assert rel_err(host(kd)[:pos], kc[:pos]) <= 1e-4
        assert rel_err(host(vd)[:pos], vc[:pos]) <= 1e-4


def test_qwen_deterministic_steps(gpu):
    """gorch_hip_set_deterministic(1) on the Qwen block's one-row steps (the
    key-split attention without Wo in its merge; Wo as a GEMV with the
    residual): the same logits bit for bit on a second run, and the oracle
    composition's tokens and 1e-3 logits."""
    from gorch_amd import hip

    cfg = QwenConfig(hidden=64, layers=2, num_q=4, num_kv=2, head_dim=64, inter=96, vocab=300, max_seq=320)
    w = syn.qwen_weights(cfg, seed=6)
    m = Qwen(cfg, w)
    ref = OracleQwen(cfg, w, m)
    prompt = np.random.default_rng(12).integers(0, cfg.vocab, 200).astype(np.int32)
    prev = hip.set_deterministic(True)
    try:
        runs = []
        for run in range(2):
            cache = m.new_cache(cfg.max_seq)
            ids, pos, out = prompt, 0, []
            for step in range(5):
                got = host(m.forward_cached(torch.from_numpy(ids).cuda(), cache, pos))
                if run == 0:
                    want = ref.forward_cached(ids, pos)
                    assert rel_err(got, want) <= 1e-3, step
                    assert int(np.argmax(got[0])) == orc.argmax(want), step
                out.append(got)
                pos += ids.size
                ids = np.array([int(np.argmax(got[0]))], np.int32)
            runs.append(np.concatenate(out))
        assert np.array_equal(runs[0], runs[1])
    finally:
        hip.set_deterministic(prev)


def oracle_generate(ref, prompt, max_new, stops, max_seq):
    """model/qwen/generate.go:35-66 with a greedy config over the oracle
    composition: token i from the latest logits; a stop token ends the loop
    and is not kept; the loop also ends once the cache holds MaxSeq rows
    (after keeping that token)."""
    result = [int(t) for t in prompt]
    logits = ref.forward_cached(np.asarray(prompt, np.int32), 0)
    pos, steps = len(prompt), []
    for _ in range(max_new):
        nxt = orc.argmax(logits)
        steps.append(logits[0])
        if nxt in stops:
            break
        result.append(nxt)
        if pos >= max_seq:
            break
        logits = ref.forward_cached(np.array([nxt], np.int32), pos)
        pos += 1
    return result, np.stack(steps)


GEN = QwenConfig(hidden=128, layers=2, num_q=4, num_kv=2, head_dim=64, inter=192, vocab=500, max_seq=96)


@pytest.mark.parametrize("cfg", [GEN, TINY], ids=["hd64", "hd32"])
def test_qwen_generate_matches_oracle(gpu, cfg):
    """The device generation loop (gorch_hip_qwen_generate): tokens identical
    to the oracle loop, each step's logits within 1e-3 and the run within
    2e-2; the graph-replayed steps (position read on the device) give the
    same tokens as the directly launched ones (head_dim 64 and 32: the
    one-pass short-cache attention after a q/k norm + RoPE launch, both at
    the device position)."""
    w = syn.qwen_weights(cfg, seed=21)
    m = Qwen(cfg, w)
    ref = OracleQwen(cfg, w, m)
    prompt = np.random.default_rng(22).integers(0, cfg.vocab, 10).astype(np.int32)
    want, want_logits = oracle_generate(ref, prompt, 20, (), cfg.max_seq)
    ids, logits, t = m.generate(prompt, 20, stop_tokens=(), want_logits=True)
    assert list(ids) == want
    assert rel_err(logits[0], want_logits[0]) <= 1e-3
    assert rel_err(logits, want_logits) <= 2e-2
    ids_g, _, t = m.generate(prompt, 20, stop_tokens=())
    assert list(ids_g) == want
    assert t["decode_forwards"] == 19
    assert t["graph"]
    # a second run reuses the engine (cache, captured step)
    ids_g2, _, _ = m.generate(prompt, 20, stop_tokens=())
    assert np.array_equal(ids_g2, ids_g)
    m.close()


@pytest.mark.parametrize("use_graph", [False, True])
def test_qwen_generate_stops_on_stop_token(gpu, use_graph):
    """A stop token ends generation and is not kept (generate.go:50-53):
    the oracle's 6th new token as the stop id (one of two, as Greedy's
    ChatML pair) cuts the output before its first occurrence; the steps run
    stop within the 8-step read-back window."""
    w = syn.qwen_weights(GEN, seed=23)
    m = Qwen(GEN, w)
    ref = OracleQwen(GEN, w, m)
    prompt = np.random.default_rng(24).integers(0, GEN.vocab, 12).astype(np.int32)
    full, _ = oracle_generate(ref, prompt, 40, (), GEN.max_seq)
    stop = full[len(prompt) + 5]
    stops = (GEN.vocab - 1 if stop != GEN.vocab - 1 else 0, stop)
    ref2 = OracleQwen(GEN, w, m)
    want, _ = oracle_generate(ref2, prompt, 40, stops, GEN.max_seq)
    assert len(want) <= len(prompt) + 5
    ids, _, t = m.generate(prompt, 40, stop_tokens=stops, use_graph=use_graph)
    assert list(ids) == want
    assert t["decode_forwards"] < 39
    m.close()


def test_qwen_generate_max_seq_and_errors(gpu):
    """Generation ends once the cache holds MaxSeq rows, keeping the token
    chosen then (generate.go:55-57): a 90-row prompt at MaxSeq 96 yields 7
    new tokens, not 20. An empty prompt is an error ("qwen: empty prompt"),
    as is one longer than MaxSeq; max_new 0 returns the prompt."""
    w = syn.qwen_weights(GEN, seed=25)
    m = Qwen(GEN, w)
    ref = OracleQwen(GEN, w, m)
    prompt = np.random.default_rng(26).integers(0, GEN.vocab, 90).astype(np.int32)
    want, _ = oracle_generate(ref, prompt, 20, (), GEN.max_seq)
    assert len(want) == GEN.max_seq + 1
    ids, _, _ = m.generate(prompt, 20, stop_tokens=())
    assert list(ids) == want
    ids0, _, _ = m.generate(prompt, 0, stop_tokens=())
    assert list(ids0) == list(prompt)
    from gorch_amd import hip
    with pytest.raises(hip.HipError, match="empty prompt"):
        m.generate(np.zeros(0, np.int32), 4)
    with pytest.raises(hip.HipError):
        m.generate(np.zeros(GEN.max_seq + 1, np.int32), 4)
    m.close()


def oracle_generate_sampled(ref, prompt, max_new, stops, max_seq, T, K, P, seed):
    """model/qwen/generate.go:35-66 with a sampling config over the oracle
    composition: token i = sampleLogits (the oracle's restatement) of the
    latest logits with the draw Philox(seed, i, 0), the device loop's draw."""
    result = [int(t) for t in prompt]
    logits = ref.forward_cached(np.asarray(prompt, np.int32), 0)
    pos = len(prompt)
    for i in range(max_new):
        nxt, _ = orc.sample_nucleus(logits[0], T, K, P, orc.philox_uniform(seed, i, 0))
        if nxt in stops:
            break
        result.append(nxt)
        if pos >= max_seq:
            break
        logits = ref.forward_cached(np.array([nxt], np.int32), pos)
        pos += 1
    return result


@pytest.mark.parametrize("T,K,P", [(1.0, 0, 0.0), (0.7, 20, 0.8), (1.5, 50, 0.95), (0.9, 5, 0.0)])
def test_qwen_generate_sampled_matches_oracle(gpu, T, K, P):
    """Sampled generation (gorch_hip_qwen_generate_sampled): every token the
    oracle loop's, given the same Philox draws, with the steps launched
    directly and replayed from the graph; a second seed gives another
    sequence."""
    w = syn.qwen_weights(GEN, seed=31)
    m = Qwen(GEN, w)
    ref = OracleQwen(GEN, w, m)
    prompt = np.random.default_rng(32).integers(0, GEN.vocab, 10).astype(np.int32)
    want = oracle_generate_sampled(ref, prompt, 24, (), GEN.max_seq, T, K, P, seed=77)
    for use_graph in (False, True):
        ids, _, t = m.generate(prompt, 24, stop_tokens=(), use_graph=use_graph, temperature=T, top_k=K, top_p=P,
                               seed=77)
        assert list(ids) == want
        assert t["graph"] == use_graph
    ids2, _, _ = m.generate(prompt, 24, stop_tokens=(), temperature=T, top_k=K, top_p=P, seed=78)
    assert list(ids2) == oracle_generate_sampled(OracleQwen(GEN, w, m), prompt, 24, (), GEN.max_seq, T, K, P, 78)
    assert list(ids2) != want
    # greedy again on the same engine (the sampled graph is not reused)
    ids_g, _, _ = m.generate(prompt, 24, stop_tokens=())
    assert list(ids_g) == oracle_generate(OracleQwen(GEN, w, m), prompt, 24, (), GEN.max_seq)[0]
    m.close()


def test_qwen_generate_sampled_stop_and_errors(gpu):
    """A sampled stop token ends generation and is not kept; a negative
    temperature or top_k is EINVAL, top-p without 1 <= top_k <= 4096
    EUNSUPPORTED."""
    from gorch_amd import hip
    w = syn.qwen_weights(GEN, seed=33)
    m = Qwen(GEN, w)
    ref = OracleQwen(GEN, w, m)
    prompt = np.random.default_rng(34).integers(0, GEN.vocab, 12).astype(np.int32)
    full = oracle_generate_sampled(ref, prompt, 30, (), GEN.max_seq, 1.2, 30, 0.9, 5)
    stop = full[len(prompt) + 4]
    want = oracle_generate_sampled(OracleQwen(GEN, w, m), prompt, 30, (stop,), GEN.max_seq, 1.2, 30, 0.9, 5)
    assert len(want) <= len(prompt) + 4
    ids, _, _ = m.generate(prompt, 30, stop_tokens=(stop,), temperature=1.2, top_k=30, top_p=0.9, seed=5)
    assert list(ids) == want
    with pytest.raises(hip.HipError) as e:
        m.generate(prompt, 4, temperature=-1.0)
    assert e.value.rc == 2
    with pytest.raises(hip.HipError) as e:
        m.generate(prompt, 4, temperature=1.0, top_k=-1)
    assert e.value.rc == 2
    with pytest.raises(hip.HipError) as e:
        m.generate(prompt, 4, temperature=1.0, top_k=0, top_p=0.5)
    assert e.value.rc == 1
    m.close()


def test_qwen_full_size_sampled(gpu):
    """Sampled generation at the full Qwen3-0.6B shape (vocab 151,936):
    tokens identical to the oracle loop for 8 new tokens with Qwen's
    recommended sampling (temperature 0.7, top-k 20, top-p 0.8)."""
    import dataclasses

    from gorch_amd.qwen import QWEN3_0_6B
    cfg = dataclasses.replace(QWEN3_0_6B, max_seq=96)
    w = syn.qwen_weights(cfg, seed=41)
    m = Qwen(cfg, w)
    ref = OracleQwen(cfg, w, m)
    prompt = np.random.default_rng(42).integers(0, cfg.vocab, 16).astype(np.int32)
    want = oracle_generate_sampled(ref, prompt, 8, (), cfg.max_seq, 0.7, 20, 0.8, 11)
    ids, _, _ = m.generate(prompt, 8, stop_tokens=(), temperature=0.7, top_k=20, top_p=0.8, seed=11)
    assert list(ids) == want
    m.close()
