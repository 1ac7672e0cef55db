// qwen.hip — one Qwen3/Qwen2.5 decoder block with a KV cache (model/qwen
// Block.ForwardCached, block.go:71-79) as one C-ABI call:
//   x1 = x + GQA(RMSNorm_attn(x));  x = x1 + down(SwiGLU(gate(h), up(h))), h = RMSNorm_ffn(x1)
//
// One-row decode (the serving step) runs in five launches, each fusing what
// the reference does as separate ops:
//   1. RMSNorm_attn applied as the QKV GEMV loads x, Q/K/V as one weight
//      stream (V written straight into its cache row);
//   2-3. grouped-query attention over the cache and Wo: with few heads the
//      key-split kernel, which applies the per-head q/k RMSNorm + RoPE
//      itself, writes the K row and sets x1 = x, then the kernel that
//      merges its key chunks and adds each head's Wo . o_h (+ bias) into
//      x1; else a q/k norm + RoPE launch, the attention and a Wo GEMV with
//      the residual add (x1 = x + ...);
//   4. RMSNorm_ffn applied as the gate/up GEMV loads x1 (one [2F, d] weight),
//      gate row j and up row F + j in one wave so it writes silu(gate) * up;
//   5. down GEMV with the residual add.
// Longer inputs (prefill) take the same steps with the norms and SwiGLU as
// launches of their own and the matrix-core GEMM for the Linears.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <vector>

#include "common.h"

namespace gh {

int launch_embedding(hipStream_t s, const float* w, const int* ids, float* out, int dim, int rows);

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

static size_t qwen_ws(const gorch_hip_qwen_block* b, int S) {
    const gorch_hip_gqa_weights& w = b->attn;
    // GQA scratch, x1 [S, d], h [S, d], gate/up [S, 2F]
    return al256(gqa_ws(S, w.num_q, w.num_kv, w.head_dim, w.dim)) + 2 * al256((size_t)S * w.dim * 4) +
           al256((size_t)S * 2 * b->inter * 4);
}

}  // namespace gh

using namespace gh;

extern "C" size_t gorch_hip_qwen_block_workspace_size(const gorch_hip_qwen_block* b, int new_seq) {
    if (!b || new_seq <= 0) return 0;
    return qwen_ws(b, new_seq);
}

namespace gh {

// The block on stream s (arguments checked by the caller). pos_dev: the
// position read on the device (one-row steps of a captured decode step).
static int qwen_block_core(hipStream_t s, const gorch_hip_qwen_block* b, float* x, int new_seq, float* k_cache,
                           float* v_cache, int pos_offset, int max_seq, void* workspace,
                           const int* pos_dev = nullptr) {
    const gorch_hip_gqa_weights* w = &b->attn;
    const int S = new_seq, d = w->dim, F = b->inter;
    char* base = static_cast<char*>(workspace);
    char* gws = base;
    float* x1 = reinterpret_cast<float*>(base + al256(gqa_ws(S, w->num_q, w->num_kv, w->head_dim, d)));
    float* h = reinterpret_cast<float*>(reinterpret_cast<char*>(x1) + al256((size_t)S * d * 4));
    float* gu = reinterpret_cast<float*>(reinterpret_cast<char*>(h) + al256((size_t)S * d * 4));

    // x1 = x + Wo(attention(RMSNorm_attn(x)))
    GH_TRY(gqa_core(s, w, x, S, k_cache, v_cache, pos_offset, max_seq, x1, gws, b->norm_attn, b->eps, x, pos_dev));
    if (S == 1 && gemv_m1_prologue_ok(d) && gemv_m1_prologue_ok(F)) {
        // [gate | up] = W_gu . RMSNorm_ffn(x1), then x = x1 + W_down . (silu(gate) * up)
        LinearExtras pre;
        pre.ln_g = b->norm_ffn;
        pre.ln_rms = true;
        pre.ln_eps = b->eps;
        if (gemv_pair_swiglu_ok(F, d)) {
            // gate row j and up row F + j in one wave: h = silu(gate) * up
            // straight from the GEMV, then x = x1 + W_down . h
            pre.pair_swiglu = F;
            GH_TRY(launch_linear_bf16_od(s, x1, b->wgate_up, nullptr, nullptr, OutDesc::plain(gu, F), 1, 2 * F, d,
                                         GORCH_HIP_EPI_NONE, pre));
            return launch_linear_bf16_od(s, gu, b->wdown, nullptr, x1, OutDesc::plain(x, d), 1, d, F,
                                         GORCH_HIP_EPI_NONE, LinearExtras{});
        }
        GH_TRY(launch_linear_bf16_od(s, x1, b->wgate_up, nullptr, nullptr, OutDesc::plain(gu, 2 * F), 1, 2 * F, d,
                                     GORCH_HIP_EPI_NONE, pre));
        LinearExtras sw;
        sw.swiglu = true;
        return launch_linear_bf16_od(s, gu, b->wdown, nullptr, x1, OutDesc::plain(x, d), 1, d, F,
                                     GORCH_HIP_EPI_NONE, sw);
    }
    // longer inputs: h = RMSNorm_ffn(x1), gate and up as two column
    // segments of one GEMM, SwiGLU, down
    GH_TRY(launch_rmsnorm(s, x1, b->norm_ffn, h, S, d, b->eps));
    float* gate = gu;
    float* up = gu + (size_t)S * F;
    OutDesc od{};
    od.nseg = 2;
    od.rows_per_seq = 1 << 30;
    od.pos_dev = nullptr;
    od.ptr[0] = gate;
    od.ptr[1] = od.ptr[2] = up;
    od.n_end[0] = F;
    od.n_end[1] = od.n_end[2] = 2 * F;
    od.row_stride[0] = od.row_stride[1] = od.row_stride[2] = F;
    GH_TRY(launch_linear_bf16_od(s, h, b->wgate_up, nullptr, nullptr, od, S, 2 * F, d, GORCH_HIP_EPI_NONE,
                                 LinearExtras{}));
    GH_TRY(launch_swiglu(s, gate, up, gate, (int64_t)S * F));
    return launch_linear_bf16(s, gate, b->wdown, nullptr, x1, x, S, d, F, GORCH_HIP_EPI_NONE);
}

}  // namespace gh

extern "C" int gorch_hip_qwen_block_forward_cached(void* stream, const gorch_hip_qwen_block* b, float* x,
                                                   int new_seq, float* k_cache, float* v_cache, int pos_offset,
                                                   int max_seq, void* workspace, size_t workspace_bytes) {
    GH_REQUIRE(b && x && k_cache && v_cache && new_seq > 0, "gorch_hip_qwen_block_forward_cached: bad arguments");
    GH_REQUIRE(b->norm_attn && b->norm_ffn && b->wgate_up && b->wdown && b->inter > 0,
               "gorch_hip_qwen_block_forward_cached: null block weight");
    GH_TRY(bf16_gate(stream_of(stream)));
    GH_TRY(gqa_check(&b->attn, new_seq, pos_offset, max_seq));
    GH_REQUIRE(workspace && workspace_bytes >= qwen_ws(b, new_seq),
               "gorch_hip_qwen_block_forward_cached: workspace too small");
    return finish(stream, qwen_block_core(stream_of(stream), b, x, new_seq, k_cache, v_cache, pos_offset, max_seq,
                                          workspace));
}

// ---------------------------------------------------------------- the model

// model/qwen Model (qwen.go:12-98) over caller-owned weights, with its own KV
// cache, activations and decode state, for generation (Generate,
// generate.go:35-66). Per token, one captured HIP graph: the blocks' one-row
// steps reading the position from device memory, the final RMSNorm, the tied
// head with the argmax fused into it (greedy) or followed by the sampler
// (sampleLogits, generate.go:94-181, which leaves its token in the argmax
// key), and a kernel that turns the key into the next token, appends it to
// the history, advances the position and writes the next input row (the
// token's embedding).
struct gorch_hip_qwen {
    std::vector<gorch_hip_qwen_block> blocks;
    const uint16_t* embed_bf16 = nullptr;
    const float* embed_f32 = nullptr;
    const float* norm = nullptr;
    float eps = 1e-6f;
    int vocab = 0, dim = 0, kv_dim = 0, max_seq = 0;
    int cap = 0;             // cache rows allocated per layer
    float* kv = nullptr;     // [layer][K | V][cap][kv_dim]
    char* ws = nullptr;      // block workspace
    size_t ws_bytes = 0;
    float* x = nullptr;      // [x_rows, dim]
    int x_rows = 0;
    float* h = nullptr;      // the final-norm row [dim]
    float* logits = nullptr; // [vocab]
    int* ids = nullptr;      // prompt ids [ids_cap]
    int ids_cap = 0;
    int* state = nullptr;    // [0] = cache length, [1] = step
    int* hist = nullptr;     // chosen tokens [hist_cap]
    int hist_cap = 0;
    unsigned long long* key = nullptr;  // fused-argmax key, zero between steps
    int* sample_err = nullptr;          // set by the sampler: top-p candidates past its sort
    int* sample_ws = nullptr;           // the sampler's multi-block candidate search (zero when idle)
    // the running generation's sampling config (temperature 0: greedy)
    float smp_t = 0.f, smp_p = 0.f;
    int smp_k = 0;
    unsigned long long smp_seed = 0;
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<const void*> sig;
};

namespace gh {

// The token the fused argmax chose (first maximum wins, generate.go's
// argmaxF32), appended to the history; the cache length advances by inc and
// the next input row is that token's embedding (qwen.go:71-72).
__global__ __launch_bounds__(256) void k_qwen_finalize(unsigned long long* key, int* hist, int* state, int inc,
                                                       const float* __restrict__ embed, float* __restrict__ x,
                                                       int dim) {
    __shared__ int tok;
    if (threadIdx.x == 0) {
        const int t = argmax_unpack(argmax_take(key, 0));
        const int step = state[1];
        tok = t;
        hist[step] = t;
        state[0] += inc;
        state[1] = step + 1;
    }
    __syncthreads();
    const float* e = embed + (size_t)tok * dim;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) x[i] = e[i];
}

static void qwen_drop_graph(gorch_hip_qwen* m) {
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
    m->sig.clear();
}

// Buffers for a prompt of n rows and a cache of cap rows (kept while large
// enough; growing moves them, and the captured step with them).
static int qwen_ensure(gorch_hip_qwen* m, int n, int cap, int hist) {
    const int L = (int)m->blocks.size();
    auto grow = [&](auto** p, size_t bytes) -> int {
        (void)hipFree(*p);
        *p = nullptr;
        return check(hipMalloc(reinterpret_cast<void**>(p), bytes), "qwen hipMalloc");
    };
    if (cap > m->cap) {
        qwen_drop_graph(m);
        m->cap = 0;
        GH_TRY(grow(&m->kv, (size_t)L * 2 * cap * m->kv_dim * sizeof(float)));
        m->cap = cap;
    }
    size_t ws = 0;
    for (const auto& b : m->blocks) ws = std::max({ws, qwen_ws(&b, n), qwen_ws(&b, 1)});
    if (ws > m->ws_bytes) {
        qwen_drop_graph(m);
        m->ws_bytes = 0;
        GH_TRY(grow(&m->ws, ws));
        m->ws_bytes = ws;
    }
    if (n > m->x_rows) {
        qwen_drop_graph(m);
        m->x_rows = 0;
        GH_TRY(grow(&m->x, (size_t)n * m->dim * sizeof(float)));
        m->x_rows = n;
    }
    if (n > m->ids_cap) {
        m->ids_cap = 0;
        GH_TRY(grow(&m->ids, (size_t)n * sizeof(int)));
        m->ids_cap = n;
    }
    if (hist > m->hist_cap) {
        qwen_drop_graph(m);
        m->hist_cap = 0;
        GH_TRY(grow(&m->hist, (size_t)hist * sizeof(int)));
        m->hist_cap = hist;
    }
    if (!m->h) {
        GH_TRY(check(hipMalloc(&m->h, (size_t)m->dim * sizeof(float)), "qwen hipMalloc"));
        GH_TRY(check(hipMalloc(&m->logits, (size_t)m->vocab * sizeof(float)), "qwen hipMalloc"));
        GH_TRY(check(hipMalloc(&m->state, 2 * sizeof(int)), "qwen hipMalloc"));
        GH_TRY(check(hipMalloc(&m->key, kArgmaxKeys * sizeof(unsigned long long)), "qwen hipMalloc"));
        GH_TRY(check(hipMalloc(&m->sample_err, sizeof(int)), "qwen hipMalloc"));
        GH_TRY(check(hipMalloc(&m->sample_ws, sample_ws_bytes(1)), "qwen hipMalloc"));
        GH_TRY(check(hipMemsetAsync(m->sample_ws, 0, sample_ws_bytes(1), m->stream), "qwen clear sample workspace"));
        GH_TRY(check(hipStreamSynchronize(m->stream), "qwen clear sample workspace"));
    }
    return GORCH_HIP_OK;
}

// Model.ForwardCached (qwen.go:69-89) for n rows at the cache length, then
// the next token. The prefill embeds the prompt ids in m->ids; a step (n =
// 1) finds its row's embedding in x (the previous choice wrote it) and
// takes its position from the host (pos) or, in the captured step, from
// the device (pos_dev = m->state).
static int qwen_forward(gorch_hip_qwen* m, hipStream_t s, int n, bool prefill, int pos, const int* pos_dev) {
    const int d = m->dim;
    if (prefill) GH_TRY(launch_embedding(s, m->embed_f32, m->ids, m->x, d, n));
    for (size_t l = 0; l < m->blocks.size(); l++) {
        float* kc = m->kv + (size_t)l * 2 * m->cap * m->kv_dim;
        float* vc = kc + (size_t)m->cap * m->kv_dim;
        GH_TRY(qwen_block_core(s, &m->blocks[l], m->x, n, kc, vc, pos, m->cap, m->ws, pos_dev));
    }
    // final RMSNorm of the last row, then the tied head (MatMulTransB with
    // the bf16 embedding, qwen.go:84) with the greedy choice fused in, or
    // the logits sampled (the draw of token i is Philox(seed, i, 0), the
    // step read from state[1])
    // (RMSNorm in the one-row GEMV's prologue where its shape table takes d)
    LinearExtras ex;
    if (m->smp_t <= 0.f) ex.argmax_key = m->key;
    const float* head_in = m->h;
    if (gemv_m1_prologue_ok(d)) {
        ex.ln_g = m->norm;
        ex.ln_rms = true;
        ex.ln_eps = m->eps;
        head_in = m->x + (size_t)(n - 1) * d;
    } else {
        GH_TRY(launch_rmsnorm(s, m->x + (size_t)(n - 1) * d, m->norm, m->h, 1, d, m->eps));
    }
    GH_TRY(launch_linear_bf16_od(s, head_in, m->embed_bf16, nullptr, nullptr, OutDesc::plain(m->logits, m->vocab), 1,
                                 m->vocab, d, GORCH_HIP_EPI_NONE, ex));
    if (m->smp_t > 0.f)
        GH_TRY(launch_sample(s, m->logits, 1, m->vocab, m->smp_t, m->smp_k, m->smp_p, nullptr, m->smp_seed,
                             m->state + 1, nullptr, nullptr, m->key, m->sample_err, true, m->sample_ws));
    hipLaunchKernelGGL(k_qwen_finalize, dim3(1), dim3(256), 0, s, m->key, m->hist, m->state, n, m->embed_f32, m->x,
                       d);
    count(CNT_ARGMAX);
    return check_launch("qwen_finalize");
}

}  // namespace gh

extern "C" {

gorch_hip_qwen* gorch_hip_qwen_create(const gorch_hip_qwen_block* blocks, int layers, const uint16_t* embed_bf16,
                                      const float* embed_f32, const float* norm, float eps, int vocab, int max_seq) {
    if (!blocks || layers <= 0 || !embed_bf16 || !embed_f32 || !norm || vocab <= 0 || max_seq <= 0) {
        set_error("gorch_hip_qwen_create: bad arguments");
        return nullptr;
    }
    const int d = blocks[0].attn.dim, kvd = blocks[0].attn.num_kv * blocks[0].attn.head_dim;
    for (int l = 0; l < layers; l++) {
        const gorch_hip_qwen_block& b = blocks[l];
        if (b.attn.dim != d || b.attn.num_kv * b.attn.head_dim != kvd || !b.norm_attn || !b.norm_ffn ||
            !b.wgate_up || !b.wdown || b.inter <= 0 || !b.attn.rope_cos) {
            set_error("gorch_hip_qwen_create: every block needs the same dim and KV width, its weights and RoPE tables");
            return nullptr;
        }
        if (b.attn.rope_max_seq < max_seq || !kv_span_ok(max_seq, kvd)) {
            set_error("gorch_hip_qwen_create: max_seq beyond the RoPE tables or a 2 GiB cache span");
            return nullptr;
        }
    }
    auto* m = new gorch_hip_qwen();
    m->blocks.assign(blocks, blocks + layers);
    m->embed_bf16 = embed_bf16;
    m->embed_f32 = embed_f32;
    m->norm = norm;
    m->eps = eps;
    m->vocab = vocab;
    m->dim = d;
    m->kv_dim = kvd;
    m->max_seq = max_seq;
    if (check(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "qwen stream")) {
        delete m;
        return nullptr;
    }
    return m;
}

void gorch_hip_qwen_destroy(gorch_hip_qwen* m) {
    if (!m) return;
    (void)hipStreamSynchronize(m->stream);
    qwen_drop_graph(m);
    for (void* p : {(void*)m->kv, (void*)m->ws, (void*)m->x, (void*)m->h, (void*)m->logits, (void*)m->ids,
                    (void*)m->state, (void*)m->hist, (void*)m->key, (void*)m->sample_err, (void*)m->sample_ws})
        (void)hipFree(p);
    release_stream_scratch(m->stream);
    (void)hipStreamDestroy(m->stream);
    delete m;
}

}  // extern "C"

namespace gh {

// Generate (model/qwen/generate.go:35-66) with temperature t (0: greedy) and
// the sampling config of sampleLogits otherwise.
static int qwen_generate(void* stream, gorch_hip_qwen* m, const int* prompt, int n_prompt, int max_new,
                         const int* stop_tokens, int n_stop, int* out_ids, int* out_len, float* step_logits,
                         float* timing_ms, int flags, float t, int top_k, float top_p, unsigned long long seed) {
    GH_REQUIRE(m && prompt && out_ids && out_len && max_new >= 0 && n_stop >= 0 && (n_stop == 0 || stop_tokens),
               "gorch_hip_qwen_generate: bad arguments");
    GH_REQUIRE(n_prompt > 0, "qwen: empty prompt");
    GH_REQUIRE(n_prompt <= m->max_seq, "qwen: prompt longer than MaxSeq");
    for (int i = 0; i < n_prompt; i++)
        GH_REQUIRE(prompt[i] >= 0 && prompt[i] < m->vocab, "gorch_hip_qwen_generate: token id out of range");
    GH_TRY(bf16_gate(stream_of(stream)));
    for (int i = 0; i < n_prompt; i++) out_ids[i] = prompt[i];
    *out_len = n_prompt;
    if (timing_ms) timing_ms[0] = timing_ms[1] = timing_ms[2] = timing_ms[3] = 0.f;
    if (max_new == 0) return GORCH_HIP_OK;
    // tokens t_0 .. t_k: t_0 from the prefill, t_i from the forward of
    // t_{i-1}; the loop ends after max_new tokens or once the cache holds
    // MaxSeq rows (the token chosen then is kept, not forwarded)
    const int k = std::min(max_new - 1, m->max_seq - n_prompt);
    const int cap = ((n_prompt + k + 63) / 64) * 64;
    GH_TRY(qwen_ensure(m, n_prompt, std::min(cap, m->max_seq), k + 1));
    GH_TRY(check(hipStreamSynchronize(stream_of(stream)), "caller stream sync"));
    hipStream_t s = m->stream;
    GH_TRY(check(hipMemsetAsync(m->state, 0, 2 * sizeof(int), s), "reset state"));
    GH_TRY(check(hipMemsetAsync(m->key, 0, kArgmaxKeys * sizeof(unsigned long long), s), "reset key"));
    GH_TRY(check(hipMemsetAsync(m->sample_err, 0, sizeof(int), s), "reset sample flag"));
    m->smp_t = t;
    m->smp_k = top_k;
    m->smp_p = top_p;
    m->smp_seed = seed;
    GH_TRY(check(hipMemcpyAsync(m->ids, prompt, (size_t)n_prompt * sizeof(int), hipMemcpyHostToDevice, s), "ids"));
    const auto t0 = std::chrono::steady_clock::now();
    GH_TRY(qwen_forward(m, s, n_prompt, true, 0, nullptr));
    auto copy_logits = [&](int i) -> int {
        if (!step_logits) return GORCH_HIP_OK;
        return check(hipMemcpyAsync(step_logits + (size_t)i * m->vocab, m->logits, (size_t)m->vocab * 4,
                                    hipMemcpyDeviceToHost, s),
                     "logits");
    };
    GH_TRY(copy_logits(0));
    GH_TRY(check(hipStreamSynchronize(s), "prefill sync"));
    const auto t1 = std::chrono::steady_clock::now();
    // the step graph needs the key-split attention for every block (the
    // position is read on the device); otherwise, or with per-step logits,
    // each step is launched directly with the host's position
    bool graph = (flags & 1) && !step_logits && k > 0;
    if (graph) {
        uint32_t tb, pb;
        memcpy(&tb, &t, 4);
        memcpy(&pb, &top_p, 4);
        const std::vector<const void*> sig = {m->kv, m->ws, m->x, m->hist,
                                              reinterpret_cast<const void*>(deterministic() ? 1 : 0),
                                              reinterpret_cast<const void*>((uintptr_t)tb),
                                              reinterpret_cast<const void*>((uintptr_t)pb),
                                              reinterpret_cast<const void*>((uintptr_t)(unsigned)top_k),
                                              reinterpret_cast<const void*>((uintptr_t)seed)};
        if (!m->exec || m->sig != sig) {
            qwen_drop_graph(m);
            GH_TRY(check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture"));
            const int r = qwen_forward(m, s, 1, false, 0, m->state);
            const hipError_t e = hipStreamEndCapture(s, &m->graph);
            if (r == GORCH_HIP_EUNSUPPORTED && e == hipSuccess) {
                // this shape's step needs its position on the host
                qwen_drop_graph(m);
                (void)hipGetLastError();
                clear_error();
                graph = false;
            } else {
                GH_TRY(r);
                GH_TRY(check(e, "end capture"));
                GH_TRY(check(hipGraphInstantiate(&m->exec, m->graph, nullptr, nullptr, 0), "instantiate"));
                m->sig = sig;
            }
        }
    }
    // stop tokens are read back every kStopCheck steps (generation ends at
    // the first; tokens chosen past it are discarded)
    constexpr int kStopCheck = 8;
    std::vector<int> hist((size_t)k + 1);
    auto stopped_at = [&](int chosen) -> int {
        GH_TRY(check(hipMemcpyAsync(hist.data(), m->hist, (size_t)chosen * sizeof(int), hipMemcpyDeviceToHost, s),
                     "hist"));
        GH_TRY(check(hipStreamSynchronize(s), "stop check sync"));
        return 0;
    };
    auto first_stop = [&](int chosen) {
        for (int i = 0; i < chosen; i++)
            for (int j = 0; j < n_stop; j++)
                if (hist[i] == stop_tokens[j]) return i;
        return -1;
    };
    int chosen = 1, done = 0;
    bool stop = false;
    if (n_stop > 0) {
        GH_TRY(stopped_at(chosen));
        stop = first_stop(chosen) >= 0;
    }
    for (int i = 0; i < k && !stop; i++) {
        if (graph) GH_TRY(check(hipGraphLaunch(m->exec, s), "graph launch"));
        else GH_TRY(qwen_forward(m, s, 1, false, n_prompt + i, nullptr));
        done++;
        chosen++;
        GH_TRY(copy_logits(chosen - 1));
        if (n_stop > 0 && (chosen % kStopCheck == 0 || i + 1 == k)) {
            GH_TRY(stopped_at(chosen));
            stop = first_stop(chosen) >= 0;
        }
    }
    GH_TRY(stopped_at(chosen));
    const auto t2 = std::chrono::steady_clock::now();
    int keep = chosen;
    const int cut = first_stop(chosen);
    if (cut >= 0) keep = cut;
    if (t > 0.f) {
        int err = 0;
        GH_TRY(check(hipMemcpy(&err, m->sample_err, sizeof(int), hipMemcpyDeviceToHost), "sample flag"));
        if (err) {
            set_error("qwen generate: more than 4096 top-p candidates (values tied at the top-k threshold)");
            return GORCH_HIP_EUNSUPPORTED;
        }
    }
    for (int i = 0; i < keep; i++) out_ids[n_prompt + i] = hist[i];
    *out_len = n_prompt + keep;
    if (timing_ms) {
        timing_ms[0] = std::chrono::duration<float, std::milli>(t1 - t0).count();
        timing_ms[1] = std::chrono::duration<float, std::milli>(t2 - t1).count();
        timing_ms[2] = (float)done;
        timing_ms[3] = graph ? 1.f : 0.f;
    }
    return GORCH_HIP_OK;
}

}  // namespace gh

extern "C" {

int gorch_hip_qwen_generate(void* stream, gorch_hip_qwen* m, const int* prompt, int n_prompt, int max_new,
                            const int* stop_tokens, int n_stop, int* out_ids, int* out_len, float* step_logits,
                            float* timing_ms, int flags) {
    return qwen_generate(stream, m, prompt, n_prompt, max_new, stop_tokens, n_stop, out_ids, out_len, step_logits,
                         timing_ms, flags, 0.f, 0, 0.f, 0ull);
}

int gorch_hip_qwen_generate_sampled(void* stream, gorch_hip_qwen* m, const int* prompt, int n_prompt, int max_new,
                                    const int* stop_tokens, int n_stop, float temperature, int top_k, float top_p,
                                    unsigned long long seed, int* out_ids, int* out_len, float* step_logits,
                                    float* timing_ms, int flags) {
    GH_REQUIRE(m, "gorch_hip_qwen_generate_sampled: null model");
    GH_REQUIRE(temperature >= 0.f && std::isfinite(temperature),
               "gorch_hip_qwen_generate_sampled: temperature must be finite and >= 0");
    if (temperature > 0.f) GH_TRY(sample_check(1, m->vocab, temperature, top_k, top_p));
    return qwen_generate(stream, m, prompt, n_prompt, max_new, stop_tokens, n_stop, out_ids, out_len, step_logits,
                         timing_ms, flags, temperature, top_k, top_p, seed);
}

}  // extern "C"
