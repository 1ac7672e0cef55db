#!/usr/bin/env python3
"""Benchmark of the BF16-weight inference hot path on one MI355X.

Workload: the BF16-weight Linear GEMV microbench,
y[M,N] = x[M,K] @ W[N,K]^T + b with x f32 N(0,1), W bf16 N(0,0.02), b = 0,
f32 accumulate and output, for M in {1,4,16} x (K,N) in {(768,3072),
(3072,768), (768,50257)}. One step = one launch of each of the 9 shapes.
Each shape cycles through enough distinct weight copies that its working set
exceeds 512 MB, so weights stream from HBM rather than the 256 MB MALL.
Launches are replayed from HIP graphs (one graph per step) so the host does
not pace the GPU.

value = algorithmic bytes of one step (sum over shapes of 2KN + 4MK + 4MN)
x steps / wall time of the timed steps. roofline = the shape with the
largest kernel time, its algorithmic bytes / its average launch duration
(HIP events on the stream the kernels run on). cpu_baseline = the CPU oracle
(gorch's widen-per-call + f32 sgemm semantics) on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "BF16 GEMV GB/s (% HBM peak); GPT-2 decode tokens/sec at batch 1 and 16"
HBM_PEAK_GBS = 8000.0
MS = (1, 4, 16)
KN = ((768, 3072), (3072, 768), (768, 50257))
ROTATE_BYTES = 512 << 20


def algo_bytes(M, K, N):
    return 2 * K * N + 4 * M * K + 4 * M * N


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--steps-per-graph", type=int, default=32,
                    help="timed GEMV steps captured per graph replay (1 = one replay per step)")
    ap.add_argument("--shape", default=None,
                    help="restrict to one shape 'M,K,N' (for profiling one kernel)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the GPT decode legs")
    ap.add_argument("--only", choices=("decode", "gemm", "decode-xl", "moe", "decode-qwen", "cpu-decode", "cpu-configs",
                                       "attn-xl"),
                    default=None,
                    help="run only one secondary leg and print its JSON (for profiling)")
    ap.add_argument("--decode-steps", type=int, default=0, metavar="N",
                    help="with --only decode-xl: N new tokens instead of 256 (short runs for PMC counters)")
    ap.add_argument("--cpu-seconds", type=float, default=9.0)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES (PMC byte-counter calibration)")
    return ap.parse_args()


def copy_calibration(nbytes, reps=20):
    """A plain device-to-device copy of known size, the reference point that
    scales rocprofv3's FETCH_SIZE / WRITE_SIZE readings."""
    import torch

    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "reps": reps}))


def gpu_leg(args, shapes):
    import torch

    from gorch_amd import hip
    from gorch_amd import synthetic as syn

    hip.init(0)
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()  # default priority
    torch.cuda.set_stream(stream)

    bufs = []
    for (M, K, N) in shapes:
        x, W, b = syn.gemv_inputs(M, K, N, seed=M * 131 + K + N)
        wbytes = 2 * K * N
        copies = max(2, -(-ROTATE_BYTES // wbytes))
        Wd = torch.from_numpy(W.view(np.int16)).cuda()
        layout = resident_layout(M, K, N)
        if layout == "packed":
            # the resident decode format, converted once outside the timing
            Wp = hip.pack_bf16(Wd)
            del Wd
            Ws = [Wp] + [Wp.clone() for _ in range(copies - 1)]
        else:
            Ws = [Wd] + [Wd.clone() for _ in range(copies - 1)]
        bufs.append(dict(M=M, K=K, N=N, x=torch.from_numpy(x).cuda(), W=Ws, layout=layout,
                         b=torch.from_numpy(b).cuda(),
                         y=torch.empty((M, N), dtype=torch.float32, device="cuda")))
    torch.cuda.synchronize()

    def launch(buf, i):
        Wi = buf["W"][i % len(buf["W"])]
        if buf["layout"] == "packed":
            hip.linear_bf16_packed(buf["x"], Wi, buf["N"], buf["b"], buf["y"])
        else:
            hip.linear_bf16(buf["x"], Wi, buf["b"], buf["y"])

    # eager warm-up reserves any split-K workspace before graph capture
    for buf in bufs:
        launch(buf, 0)
    torch.cuda.synchronize()

    # per-shape kernel timing: one graph of L launches cycling the copies
    per_shape = []
    for buf in bufs:
        L = 4 * len(buf["W"]) if len(buf["W"]) < 64 else 2 * len(buf["W"])
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(L):
                launch(buf, i)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 5
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * L)
        nbytes = algo_bytes(buf["M"], buf["K"], buf["N"])
        per_shape.append(dict(M=buf["M"], K=buf["K"], N=buf["N"], layout=buf["layout"], us=round(us, 3),
                              GBs=round(nbytes / us / 1e3, 1), copies=len(buf["W"]),
                              frac=round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)))
        del g

    # step graphs: step s launches every shape once, on copy s. The timed
    # steps replay G of them per graph (a serving loop's capture), so the
    # per-replay submission cost is paid once per G steps; a remainder of
    # fewer than G steps replays one-step graphs.
    n_graphs = max(len(buf["W"]) for buf in bufs)
    G = max(1, min(args.steps_per_graph, args.steps))

    def capture(first, count):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for s in range(first, first + count):
                for buf in bufs:
                    launch(buf, s % n_graphs)
        return g

    graphs = [capture(s, 1) for s in range(n_graphs)]
    groups = {}
    for j in range(args.steps // G):
        c = (args.warmup + j * G) % n_graphs
        if c not in groups:
            groups[c] = capture(c, G)

    def run(nsteps, start, grouped):
        s = 0
        while grouped and nsteps - s >= G and G > 1:
            groups[(start + s) % n_graphs].replay()
            s += G
        for s in range(s, nsteps):
            graphs[(start + s) % n_graphs].replay()

    run(args.warmup, 0, False)
    for g in groups.values():  # first replay of each grouped graph, untimed
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(args.steps, args.warmup, True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_bytes = sum(algo_bytes(b_["M"], b_["K"], b_["N"]) for b_ in bufs)
    value = step_bytes * args.steps / wall / 1e9
    # the same steps with one graph replay each (the submission cost paid
    # per step), reported beside the grouped figure
    value_one = None
    if G > 1:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run(args.steps, args.warmup, False)
        torch.cuda.synchronize()
        value_one = step_bytes * args.steps / (time.perf_counter() - t0) / 1e9
    dom = max(per_shape, key=lambda r: r["us"])
    return value, wall, per_shape, dom, value_one


MFMA_PEAK_TFLOPS = 2516.6  # dense bf16: 256 CU x 2.4 GHz x 4096 FLOP/clk


def resident_layout(M, K, N):
    """Weight layout the decode path keeps resident for a GEMV of this
    shape, as the GPT engine does (gorch_amd/csrc/gpt.hip): the tile-packed
    format for 2..16 rows (wide weights with K <= 3072 streamed whole,
    narrow ones with K split across blocks); row-major for one row (the
    register GEMV, LayerNorm fusable)."""
    wide = (N + 15) // 16 >= 128
    if 2 <= M <= 16 and ((wide and K <= 3072) or (not wide and K >= 1024)):
        return "packed"
    return "row-major"


def gemv_kernel(M, K, N):
    """Which kernel libgorch_hip.so runs for a GEMV of this shape (the
    routing of launch_linear_bf16_od in gorch_amd/csrc/gemv.hip)."""
    if resident_layout(M, K, N) == "packed":
        return "k_gemv_tiles"
    if M == 1:
        chunks = K // 8
        if any(chunks % t == 0 and chunks // t <= 8 for t in (64, 32, 16, 8)):
            return "k_gemv_m1"
        return "k_gemv_valu"
    mr = 4 if M <= 4 else (8 if M <= 8 else 16)
    if (N + 15) // 16 >= 1024 and ((K + 127) // 128) * 16 * mr * 32 <= 128 * 1024:
        return "k_gemv_mt"
    return "k_linear_bf16_mfma"


def measured_traffic(kernel, M, K, N):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 PMC summary (FETCH_SIZE / WRITE_SIZE, copy-calibrated), when
    one exists for this kernel and shape; else None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            rows = json.load(f)
    except (OSError, ValueError):
        return None
    for r in rows:
        if r.get("kernel") == kernel and tuple(r.get("shape", ())) == (M, K, N):
            return r.get("traffic_bytes")
    return None


def gemm_leg(M=512, K=768, Ns=(2304, 3072)):
    """Prefill GEMM: operands resident (re-used across
    launches), timed over a graph of back-to-back launches."""
    import torch

    from gorch_amd import hip
    from gorch_amd import synthetic as syn

    out = []
    stream = torch.cuda.current_stream()
    for N in Ns:
        x, W, b = syn.gemv_inputs(M, K, N, seed=N)
        xd, Wd = torch.from_numpy(x).cuda(), torch.from_numpy(W.view(np.int16)).cuda()
        bd = torch.from_numpy(b).cuda()
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        for act_bf16 in (True, False):
            hip.linear_bf16(xd, Wd, bd, y, act_bf16=act_bf16)
            torch.cuda.synchronize()
            L = 200
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for _ in range(L):
                    hip.linear_bf16(xd, Wd, bd, y, act_bf16=act_bf16)
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(3):
                g.replay()
            e1.record(stream)
            e1.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (3 * L)
            flops = 2.0 * M * K * N
            # algorithmic bytes: f32 A, bf16 W, f32 C once each; the roofline
            # ceiling min(MFMA peak, AI x HBM peak) is the HBM side here
            # (AI 184 / 192 FLOP/B: 58-61% of the MFMA peak)
            nbytes = 4 * M * K + 2 * K * N + 4 * M * N
            ceiling = min(MFMA_PEAK_TFLOPS, flops / nbytes * HBM_PEAK_GBS / 1e3)
            # the f32-accurate mode issues two MFMAs per fragment: report the
            # algorithmic rate (2MKN / time) for both
            out.append({"M": M, "K": K, "N": N, "activations": "bf16" if act_bf16 else "f32 (hi+lo split)",
                        "us": round(us, 3), "TFLOPs": round(flops / us / 1e6, 1),
                        "frac_mfma_peak": round(flops / us / 1e6 / MFMA_PEAK_TFLOPS, 4),
                        "algorithmic_bytes": nbytes, "roofline_ceiling_TFLOPs": round(ceiling, 1),
                        "frac_roofline_ceiling": round(flops / us / 1e6 / ceiling, 4),
                        "frac_hbm_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)})
            del g
    return out


def moe_leg():
    """MoE layer: 2048 tokens, d 1024, 8 experts of ffn
    4096, top-2, injected logits. Algorithmic FLOPs 6*d*ffn per assignment."""
    import torch

    from gorch_amd import hip
    from gorch_amd import synthetic as syn

    x, logits, w = syn.moe_inputs(seed=0)
    m = hip.MoE(w)
    xd, ld = torch.from_numpy(x).cuda(), torch.from_numpy(logits).cuda()
    out = torch.empty_like(xd)
    m.forward(xd, ld, out)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    L = 20
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(L):
            m.forward(xd, ld, out)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(3):
        g.replay()
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (3 * L)
    flops = 2048 * 2 * 6.0 * 1024 * 4096
    return {"tokens": 2048, "dim": 1024, "ffn": 4096, "experts": 8, "top_k": 2, "us": round(us, 2),
            "TFLOPs": round(flops / us / 1e6, 1), "frac_mfma_peak": round(flops / us / 1e6 / MFMA_PEAK_TFLOPS, 4)}


def qwen_leg(ctxs=(128, 512), steps=100, gen_tokens=65):
    """Qwen3-0.6B-shaped cached decode (the reference's BenchmarkQwenDecode,
    model/qwen/bench_test.go:21-43): 28 layers, d 1024, 16 query / 8 KV heads
    of 128, SwiGLU 3072, vocab 151936 tied head; random bf16 weights N(0,0.02)
    generated on the device. The cache is prefilled to ctx tokens, then one
    graph-captured single-token step at position ctx is replayed (it rewrites
    the same cache row, as the reference trims the cache back each step).
    "generate" times the device generation loop from the same prompt."""
    import dataclasses

    import torch

    from gorch_amd import hip
    from gorch_amd.qwen import QWEN3_0_6B, Qwen

    cfg = dataclasses.replace(QWEN3_0_6B, max_seq=max(ctxs) + gen_tokens + 8)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)

    def bf16(shape):
        f = torch.randn(shape, device="cuda", generator=gen) * 0.02
        out = torch.empty(shape, dtype=torch.int16, device="cuda")
        hip.f32_to_bf16(f, out)
        return out

    def gain(n):
        return 1 + 0.1 * torch.randn(n, device="cuda", generator=gen)

    q, kv, d = cfg.num_q * cfg.head_dim, cfg.kv_dim, cfg.hidden
    w = {"embed": bf16((cfg.vocab, d)), "norm": gain(d), "layers": [
        {"wq": bf16((q, d)), "wk": bf16((kv, d)), "wv": bf16((kv, d)), "wo": bf16((d, q)),
         "q_norm": gain(cfg.head_dim), "k_norm": gain(cfg.head_dim), "norm_attn": gain(d), "norm_ffn": gain(d),
         "wgate": bf16((cfg.inter, d)), "wup": bf16((cfg.inter, d)), "wdown": bf16((d, cfg.inter))}
        for _ in range(cfg.layers)]}
    m = Qwen(cfg, w)
    stream = torch.cuda.current_stream()
    out = []
    for ctx in ctxs:
        cache = m.new_cache(ctx + 1)
        ids = torch.randint(0, cfg.vocab, (ctx,), dtype=torch.int32, device="cuda", generator=gen)
        m.forward_cached(ids, cache, 0)
        tok = ids[:1].clone()
        m.forward_cached(tok, cache, ctx)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            m.forward_cached(tok, cache, ctx)
        for _ in range(5):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            g.replay()
        e1.record(stream)
        e1.synchronize()
        ms = e0.elapsed_time(e1) / steps
        del g, cache
        # the greedy generation loop on the device (model/qwen/generate.go:
        # 35-66): prefill of the ctx prompt, then new_tokens - 1 graph-replayed
        # steps with the argmax fused into the tied head; decode time only
        prompt = ids.cpu().numpy()
        m.generate(prompt, gen_tokens, stop_tokens=())
        _, _, t = m.generate(prompt, gen_tokens, stop_tokens=())
        gen_ms = t["decode_ms"] / max(t["decode_forwards"], 1)
        # the same loop with Qwen's recommended sampling config (sampleLogits,
        # :94-181, on the device after the tied head)
        smp = dict(temperature=0.7, top_k=20, top_p=0.8, seed=1)
        m.generate(prompt, gen_tokens, stop_tokens=(), **smp)
        _, _, ts = m.generate(prompt, gen_tokens, stop_tokens=(), **smp)
        smp_ms = ts["decode_ms"] / max(ts["decode_forwards"], 1)
        out.append({"model": "qwen3-0.6b-shaped", "batch": 1, "ctx": ctx, "tok_s": round(1e3 / ms, 1),
                    "ms_per_token": round(ms, 4), "weights": "bf16 N(0,0.02) random init on the device",
                    "roofline": roofline_block(qwen_step_bytes(cfg, ctx), ms / 1e3,
                                               "bf16 weights + tied head + gains once, K/V rows read "
                                               "and written, logits; per token"),
                    "generate": {"new_tokens": gen_tokens, "decode_forwards": t["decode_forwards"],
                                 "graph": t["graph"], "tok_s": round(1e3 / gen_ms, 1),
                                 "ms_per_token": round(gen_ms, 4), "prefill_ms": round(t["prefill_ms"], 3)},
                    "generate_sampled": {**smp, "decode_forwards": ts["decode_forwards"], "graph": ts["graph"],
                                         "tok_s": round(1e3 / smp_ms, 1), "ms_per_token": round(smp_ms, 4)}})
    m.close()
    return out


def gpt_step_bytes(cfg, batch, ctx_mean):
    """Algorithmic HBM bytes of one GPT decode step (every sequence forwards
    one token): the bf16 Linear weights (fused QKV, Wo, FFN1, FFN2 per layer
    and the LM head) and the f32 biases / LayerNorm parameters once each,
    the embedding rows, the K and V cache rows read by attention (ctx_mean
    keys per sequence and layer) and written for the new token, and the
    logits written. Activations between kernels (a few KB per row) are left
    out."""
    d, V, L = cfg["dim"], cfg["vocab"], cfg["layers"]
    weights = L * 2 * 12 * d * d + 2 * V * d
    params = L * 4 * (3 * d + d + 4 * d + d + 4 * d) + 4 * 2 * d + 4 * V
    emb = batch * 2 * d * 4
    kv = batch * L * 2 * d * 4 * (ctx_mean + 1)
    logits = batch * V * 4
    return weights + params + emb + kv + logits


def qwen_step_bytes(cfg, ctx):
    """Algorithmic HBM bytes of one Qwen3-shaped decode token: the bf16
    projection weights of every layer (Q, K, V, O, gate, up, down) and the
    tied bf16 head once each, the f32 norm gains, the K/V cache rows read
    (ctx + 1 keys per layer) and written, and the logits written."""
    d, q, kv, inter, V, L = cfg.hidden, cfg.num_q * cfg.head_dim, cfg.kv_dim, cfg.inter, cfg.vocab, cfg.layers
    weights = L * 2 * (q * d + 2 * kv * d + d * q + 3 * inter * d) + 2 * V * d
    params = L * 4 * (2 * d + 2 * cfg.head_dim) + 4 * d
    kvb = L * 2 * kv * 4 * (ctx + 2)
    return weights + params + kvb + 4 * V


def roofline_block(nbytes, seconds, what):
    gbs = nbytes / seconds / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_step": int(nbytes), "bytes": what}


def attn_leg(batch=16, heads=25, hd=64, ctx=640, capacity=768, reps=200):
    """The GPT-2 XL batch-16 step's cached attention alone (MHA.ForwardCached's
    core, nn/attention.go:355-397): one new row per sequence at position
    ctx - 1 over a [batch][capacity][heads*hd] f32 cache (the engine's
    layout), the mean context of configs[4]'s 256 steps. Algorithmic bytes =
    the K and V rows read (2 * batch * ctx * heads * hd * 4) plus q and out."""
    import torch

    from gorch_amd import hip

    d = heads * hd
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    q = torch.randn((batch, d), device="cuda", generator=gen)
    kc = torch.randn((batch, capacity, d), device="cuda", generator=gen)
    vc = torch.randn((batch, capacity, d), device="cuda", generator=gen)
    out = torch.empty((batch, d), device="cuda")
    stream = torch.cuda.current_stream()
    hip.attention_cached(q, kc, vc, out, batch, 1, ctx - 1, heads, hd, capacity)
    torch.cuda.synchronize()
    L = 20
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(L):
            hip.attention_cached(q, kc, vc, out, batch, 1, ctx - 1, heads, hd, capacity)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps // L):
        g.replay()
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps // L * L)
    nbytes = 2 * batch * ctx * d * 4 + 2 * batch * d * 4
    return {"batch": batch, "heads": heads, "head_dim": hd, "ctx": ctx, "capacity": capacity, "us": round(us, 2),
            "algorithmic_bytes": nbytes, "GBs": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


def decode_leg(cfg_name, batch, n_prompt, max_new, reps=3, w=None):
    """Greedy KV-cache decode through the engine (graph-replayed step).
    tok/s = batch * decode forwards / decode wall time (prefill timed apart).
    w: the host weights when the caller made them already."""
    from gorch_amd import hip
    from gorch_amd import synthetic as syn

    cfg = dict(syn.GPT2_SMALL if cfg_name == "gpt2-small" else syn.GPT2_XL)
    g = hip.GPT(w if w is not None else syn.gpt2_weights(cfg, seed=0))
    prompts = np.stack([syn.prompt_ids(n_prompt, cfg["vocab"], seed=b) for b in range(batch)])
    g.generate_cached(prompts, max_new, use_graph=True)   # warm-up (graph build, caches)
    runs = []
    for _ in range(reps):
        _, _, t = g.generate_cached(prompts, max_new, use_graph=True)
        runs.append(t)
    # the same steps with sampled choices (GenerateConfig Temperature 0.8,
    # TopK 40, TopP 0.95: sample() on the device after the LM head)
    smp = dict(temperature=0.8, top_k=40, top_p=0.95, seed=1)
    g.generate(prompts, max_new, **smp)
    sruns = sorted((g.generate(prompts, max_new, **smp)[2] for _ in range(reps)), key=lambda t: t["decode_ms"])
    ts = sruns[len(sruns) // 2]
    g.close()
    runs.sort(key=lambda t: t["decode_ms"])
    t = runs[len(runs) // 2]
    fwd = t["decode_forwards"]
    step_s = t["decode_ms"] / 1e3 / fwd
    # step i forwards the token at position n_prompt + i over n_prompt + i + 1 keys
    nbytes = gpt_step_bytes(cfg, batch, n_prompt + (fwd - 1) / 2.0)
    return {"model": cfg_name, "batch": batch, "prompt": n_prompt, "new_tokens": max_new,
            "tok_s": round(batch * fwd / (t["decode_ms"] / 1e3), 1),
            "ms_per_step": round(t["decode_ms"] / fwd, 4), "prefill_ms": round(t["prefill_ms"], 3),
            "weights": "bf16 N(0,0.02) random init, synthetic prompts",
            "roofline": roofline_block(nbytes, step_s, "bf16 weights + f32 params once, K/V rows read at the "
                                                        "mean context and written, embeddings, logits; per step"),
            "sampled": {**smp, "decode_forwards": ts["decode_forwards"],
                        "tok_s": round(batch * ts["decode_forwards"] / (ts["decode_ms"] / 1e3), 1),
                        "ms_per_step": round(ts["decode_ms"] / max(ts["decode_forwards"], 1), 4)}}


def host_info():
    """The CPU the baseline ran on: model name, logical CPUs, the CPUs this
    process may use, and the thread count the box grants (OMP_NUM_THREADS)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or avail
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity": avail, "threads_granted": share}


def cpu_leg(shapes, seconds, host):
    """The oracle (gorch CPU semantics: widen the bf16 weight per call, f32
    sgemm, bias add) over the same 9 shapes, repeated for ~`seconds` on the
    threads the box grants this job, then for a third of that on one thread."""
    import oracle as orc
    from gorch_amd import synthetic as syn

    threads = host["threads_granted"]
    inputs = [syn.gemv_inputs(M, K, N, seed=M * 131 + K + N) for (M, K, N) in shapes]
    step_bytes = sum(algo_bytes(M, K, N) for (M, K, N) in shapes)
    orc.set_widen_per_call(True)

    def sweep(nthreads, budget):
        orc.set_threads(nthreads)
        for (x, W, b) in inputs:  # warm
            orc.linear(x, W, b)
        n = 0
        t0 = time.perf_counter()
        while True:
            for (x, W, b) in inputs:
                orc.linear(x, W, b)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return n, el

    n, el = sweep(threads, seconds)
    n1, el1 = sweep(1, seconds / 3)
    orc.set_threads(threads)
    return dict(value=round(step_bytes * n / el / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                sample=f"{n} steps of the {len(shapes)}-shape sweep in {el:.1f} s on {threads} threads; oracle "
                       f"widens the bf16 weight on every call (bf16_matmul.go:166) then runs an f32 sgemm",
                single_thread=dict(value=round(step_bytes * n1 / el1 / 1e9, 3), unit="GB/s",
                                   sample=f"{n1} steps in {el1:.1f} s"),
                **host)


def cpu_decode_leg(seconds, host, n_prompt=32):
    """gorch's CPU greedy decode of GPT-2 small at batch 1 (generateCached,
    model/generate.go:94-131: ForwardCached of one token, then argmax) on the
    oracle, after a 32-token prefill. Faithful: the bf16 weights are widened
    on every Linear call (bf16_matmul.go:147-166); pre-widened: widened once.
    Each mode on the granted threads and on one thread, ~`seconds` each.
    tok/s = decode steps / their wall time (prefill not timed)."""
    import oracle as orc
    from gorch_amd import synthetic as syn

    cfg = syn.GPT2_SMALL
    w = syn.gpt2_weights(cfg, seed=0)
    o = orc.GPT(w)
    prompt = syn.prompt_ids(n_prompt, cfg["vocab"], seed=0)
    out = []
    for widen in (True, False):
        for threads in (host["threads_granted"], 1):
            orc.set_threads(threads)
            orc.set_widen_per_call(widen)
            cache = o.new_cache()
            tok = orc.argmax(o.forward_cached(prompt, cache)[-1])
            n = 0
            t0 = time.perf_counter()
            while True:
                tok = orc.argmax(o.forward_cached(np.array([tok], np.int32), cache)[-1])
                n += 1
                el = time.perf_counter() - t0
                if el >= seconds or len(cache) >= cfg["max_seq"]:
                    break
            out.append({"mode": "faithful (widen per call)" if widen else "pre-widened",
                        "threads": threads, "tok_s": round(n / el, 2), "steps": n, "seconds": round(el, 2)})
    orc.set_widen_per_call(True)
    orc.set_threads(host["threads_granted"])
    return {"model": "gpt2-small", "batch": 1, "prompt": n_prompt, "kind": "port", "unit": "tok/s",
            "runs": out, **host}


def cpu_configs_leg(host, gemm, moe, xl, xl_w, seconds=2.0):
    """The oracle beside the GPU for the other configs, on the granted
    threads and on one thread (bounded samples):
    P: the prefill GEMM 512 x 768 x N (bf16-rounded activations, the weight
       widened per call as bf16_matmul.go:166), repeated ~seconds;
    E: the MoE layer (configs[3], 2048 tokens): one forward on the granted
       threads, a 256-token slice of the same input on one thread;
    X: the GPT-2 XL-shaped model (configs[4] weights): an 8-token prompt
       (not timed), then decode steps of one sequence, faithful (widen per
       call) and pre-widened; the per-token cost is the weights' (at context
       9 rather than 512-767: attention is ~6% of a step's FLOPs there).
    GPU/CPU speed-ups against the GPU legs of the same run."""
    import oracle as orc
    from gorch_amd import synthetic as syn

    threads = host["threads_granted"]

    def timed(fn, budget, min_n=1):
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget and n >= min_n:
                return el / n, n

    out = {"kind": "port", "cores": threads, **host}
    orc.set_widen_per_call(True)
    p = []
    for N in (2304, 3072):
        x, W, b = syn.gemv_inputs(512, 768, N, seed=N)
        xb = orc.bf16_to_f32(orc.f32_to_bf16(x))
        gpu_us = next((g["us"] for g in gemm if g["N"] == N and g["activations"] == "bf16"), None)
        for th in (threads, 1):
            orc.set_threads(th)
            sec, n = timed(lambda: orc.linear(xb, W, b), seconds if th == threads else seconds / 2)
            p.append({"N": N, "threads": th, "us": round(sec * 1e6, 1), "calls": n,
                      "TFLOPs": round(2.0 * 512 * 768 * N / sec / 1e12, 4),
                      "gpu_speedup": round(sec * 1e6 / gpu_us, 1) if gpu_us else None})
    out["prefill_gemm"] = p
    x, logits, w = syn.moe_inputs(seed=0)
    e = []
    for th, rows in ((threads, x.shape[0]), (1, 256)):
        orc.set_threads(th)
        t0 = time.perf_counter()
        orc.moe_forward(w, x[:rows], logits[:rows])
        sec = (time.perf_counter() - t0) * x.shape[0] / rows
        e.append({"threads": th, "tokens_timed": rows, "us_per_layer": round(sec * 1e6, 1),
                  "gpu_speedup": round(sec * 1e6 / moe["us"], 1) if moe else None})
    out["moe_layer"] = e
    del x, logits, w
    if xl_w is not None:
        o = orc.GPT(xl_w)
        prompt = syn.prompt_ids(8, syn.GPT2_XL["vocab"], seed=0)
        runs = []
        gpu_tok_s = xl["tok_s"] if xl else None
        for widen in (True, False):
            orc.set_widen_per_call(widen)
            for th in (threads, 1):
                orc.set_threads(th)
                cache = o.new_cache()
                tok = orc.argmax(o.forward_cached(prompt, cache)[-1])
                if not widen:   # the one-time widening happens on the first call
                    tok = orc.argmax(o.forward_cached(np.array([tok], np.int32), cache)[-1])
                steps = 2 if th == threads else 1
                t0 = time.perf_counter()
                for _ in range(steps):
                    tok = orc.argmax(o.forward_cached(np.array([tok], np.int32), cache)[-1])
                el = time.perf_counter() - t0
                runs.append({"mode": "faithful (widen per call)" if widen else "pre-widened", "threads": th,
                             "steps": steps, "tok_s": round(steps / el, 3),
                             "gpu_speedup": round(gpu_tok_s / (steps / el), 1) if gpu_tok_s else None})
        out["decode_xl"] = {"model": "gpt2-xl", "prompt": 8, "runs": runs,
                            "gpu": "batch 16 tok/s of the decode leg (16 sequences at once)"}
        del o
    orc.set_widen_per_call(True)
    orc.set_threads(threads)
    return out


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.only == "cpu-configs":
        # the oracle legs alone (no GPU); the XL model's weights are made here
        from gorch_amd import synthetic as syn
        print(json.dumps(cpu_configs_leg(host_info(), [], None, None,
                                         syn.gpt2_weights(dict(syn.GPT2_XL), seed=0))))
        return
    if args.only:
        import torch

        from gorch_amd import hip
        hip.init(0)
        torch.cuda.set_device(0)
        torch.cuda.set_stream(torch.cuda.Stream())  # graphs capture on a non-default stream
        if args.only == "decode":
            print(json.dumps(decode_leg("gpt2-small", 1, 32, 64)))
        elif args.only == "decode-xl":
            print(json.dumps(decode_leg("gpt2-xl", 16, 512, args.decode_steps or 256, reps=1)))
        elif args.only == "moe":
            print(json.dumps(moe_leg()))
        elif args.only == "decode-qwen":
            print(json.dumps(qwen_leg()))
        elif args.only == "attn-xl":
            print(json.dumps(attn_leg()))
        elif args.only == "cpu-decode":
            print(json.dumps(cpu_decode_leg(3.0, host_info())))
        else:
            print(json.dumps(gemm_leg()))
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is described, not run)", file=sys.stderr)
        sys.exit(2)
    if args.shape:
        M, K, N = (int(v) for v in args.shape.split(","))
        shapes = [(M, K, N)]
    else:
        shapes = [(M, K, N) for (K, N) in KN for M in MS]

    value, wall, per_shape, dom, value_one = gpu_leg(args, shapes)
    # the metric's two decode rates: GPT-2 small at batch 1 (configs[0]'s
    # workload) and the GPT-2 XL shape at batch 16
    from gorch_amd import synthetic as syn
    xl_w = None if (args.shape or args.no_decode) else syn.gpt2_weights(dict(syn.GPT2_XL), seed=0)
    decode = [] if (args.shape or args.no_decode) else [decode_leg("gpt2-small", 1, 32, 64),
                                                         decode_leg("gpt2-xl", 16, 512, 256, reps=1, w=xl_w)]
    gemm = [] if args.shape else gemm_leg()
    moe = None if args.shape else moe_leg()
    qwen = [] if (args.shape or args.no_decode) else qwen_leg()
    host = host_info()
    cpu = None if args.no_cpu else cpu_leg(shapes, args.cpu_seconds, host)
    cpu_decode = None if (args.no_cpu or args.shape or args.no_decode) else cpu_decode_leg(3.0, host)
    cpu_configs = None if (args.no_cpu or args.shape) else cpu_configs_leg(
        host, gemm, moe, decode[1] if len(decode) > 1 else None, xl_w if not args.no_cpu else None)
    del xl_w
    dom_bytes = algo_bytes(dom["M"], dom["K"], dom["N"])
    dom_kernel = gemv_kernel(dom["M"], dom["K"], dom["N"])
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "bf16-weight Linear GEMV microbench (BASELINE configs[1]): x f32 N(0,1) [M,K], "
                        "W bf16 N(0,0.02) [N,K], f32 out; one step = one launch per shape",
            "steps_per_graph_replay": max(1, min(args.steps_per_graph, args.steps)),
            "value_one_replay_per_step": None if value_one is None else round(value_one, 1),
            "shapes": [f"M={s[0]},K={s[1]},N={s[2]}" for s in shapes],
            "weights_rotated_over_bytes": ROTATE_BYTES,
            "weight_layout": "each shape on the decode path's resident format (per_shape.layout): "
                             "tile-packed 1 KB matrix-core fragments for 2..16 rows (packed once before "
                             "timing; narrow weights with K split across blocks); row-major for one row",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{dom_kernel} M={dom['M']} K={dom['K']} N={dom['N']}",
            "achieved": round(dom_bytes / dom["us"] / 1e3, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom_bytes / dom["us"] / 1e3 / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(dom_kernel, dom["M"], dom["K"], dom["N"]),
            "algorithmic_bytes_per_launch": dom_bytes,
            "avg_launch_us": dom["us"],
        },
        "cpu_baseline": cpu,
        "per_shape": per_shape,
        "decode": decode,
        "cpu_decode": cpu_decode,
        "cpu_configs": cpu_configs,
        "prefill_gemm": gemm,
        "moe_layer": moe,
        "decode_qwen": qwen,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
