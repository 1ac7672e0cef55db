// gpt.hip — host-side GPT decode engine over the HIP kernels: the C++
// counterpart of gorch's nn.GPT / nn.KVCache / model.generateCached
// (nn/gpt.go:12-121, nn/transformer.go:53-63, nn/attention.go:313-400,
// nn/kvcache.go:14-60, model/generate.go:94-131), with weights resident in
// HBM (gpt.ToMetal, nn/gpt.go:241-257).
//
// Layout in HBM:
//   - one weight blob; per layer a fused QKV weight [3d, d] bf16 (the rows of
//     Wq, Wk, Wv back to back — what gorch's Q/K/V Linears compute, in one
//     weight stream), Wo [d, d], FFN1 [4d, d], FFN2 [d, 4d] bf16, f32 biases
//     and LayerNorm parameters; f32 wte/wpe; LM head [V, d] bf16;
//   - KV cache f32 [layer][batch][capacity][d] for K and for V;
//   - the cache length (`pos`) and the generation step live in device memory,
//     so a decode step is position-independent and is captured once as a HIP
//     graph and replayed for every token without host synchronisation.
//
// Per layer and forward: LayerNorm -> fused QKV GEMV writing Q to a buffer
// and K/V rows straight into the cache at pos -> cached attention -> Wo GEMV
// with bias and residual fused -> LayerNorm -> FFN1 GEMV with bias+GELU ->
// FFN2 GEMV with bias and residual fused. Then the final LayerNorm (on the
// last row of each sequence when generating), LM head GEMV, and argmax.
#include <cstring>
#include <vector>

#include <algorithm>

#include "common.h"

namespace gh {

int launch_layernorm(hipStream_t s, const float* x, const float* g, const float* b, float* y, int M, int N,
                     float eps, long long in_stride);
int launch_embed_pos(hipStream_t s, const float* wte, const float* wpe, const int* ids, const int* pos_dev,
                     float* out, int dim, int n_per_seq, int rows);
int launch_argmax(hipStream_t s, const float* logits, int rows, int n, int* out, int* hist, const int* step_dev,
                  int hist_stride, int* pos_dev, int pos_inc);
int launch_advance_step(hipStream_t s, int* step_dev);

__global__ void k_pos_add(int* pos_dev, int n) { *pos_dev += n; }

struct LayerW {
    uint16_t *wqkv, *wo, *w1, *w2;
    float *bqkv, *bo, *b1, *b2, *ln1_g, *ln1_b, *ln2_g, *ln2_b;
    // tile-packed copies for the 2..16-row decode GEMVs (null when not packed)
    uint16_t *wqkv_p = nullptr, *w1_p = nullptr, *wo_p = nullptr, *w2_p = nullptr;
};

}  // namespace gh

using namespace gh;

struct gorch_hip_gpt {
    int vocab = 0, dim = 0, heads = 0, layers = 0, max_seq = 0;
    char* blob = nullptr;
    char* pblob = nullptr;  // tile-packed weights
    size_t pblob_bytes = 0;
    float *wte = nullptr, *wpe = nullptr, *lnf_g = nullptr, *lnf_b = nullptr, *blm = nullptr;
    uint16_t* wlm = nullptr;
    uint16_t* wlm_p = nullptr;
    std::vector<LayerW> L;
    // activations, grown on demand
    size_t rows_cap = 0, logit_rows_cap = 0;
    float *x = nullptr, *h = nullptr, *q = nullptr, *att = nullptr, *ff = nullptr, *logits = nullptr;
    // batched decode (2..16 rows): K-split partials of the residual Linears
    // and the LayerNorm row statistics they leave for the next GEMV
    float* part = nullptr;
    float2* stats = nullptr;
    // batched one-token steps: K-split partials of the fused QKV Linear,
    // summed by the cached attention kernel
    float* wpart = nullptr;
    // batched decode over tile-packed weights: the GEMVs' activations
    // pre-split in the fragment layout (LayerNorm outputs; FFN1's GELU
    // output), zeroed at allocation
    uint16_t *hfrag = nullptr, *ffrag = nullptr, *afrag = nullptr;
    int* ids = nullptr;
    size_t ids_cap = 0;
    hipStream_t stream = nullptr;  // engine stream (default priority), used for graph capture
    // generate_cached keeps its KV cache and the captured decode-step graph
    // between calls with the same (batch, capacity) while the buffers the
    // graph points at are unchanged, so repeated generation does not pay the
    // capture and instantiation again
    gorch_hip_kvcache* gen_cache = nullptr;
    hipGraph_t gen_graph = nullptr;
    hipGraphExec_t gen_exec = nullptr;
    std::vector<const void*> gen_sig;
    int* sample_err = nullptr;  // sampled generation: top-p support overflow flag
    // sampled generation: the sampler's multi-block candidate search for up
    // to sample_ws_rows rows (zero when idle)
    int* sample_ws = nullptr;
    int sample_ws_rows = 0;
};

struct gorch_hip_kvcache {
    gorch_hip_gpt* gpt = nullptr;
    int batch = 0, capacity = 0, len = 0;
    float *k = nullptr, *v = nullptr;
    int* state = nullptr;  // [0] = pos (cache length), [1] = generation step
    int* hist = nullptr;   // generated tokens [capacity][batch]
    unsigned long long* key = nullptr;  // fused-argmax keys [batch], zero between steps
};

namespace gh {

static float* kc_layer(gorch_hip_kvcache* c, int l) {
    return c->k + (size_t)l * c->batch * c->capacity * c->gpt->dim;
}
static float* vc_layer(gorch_hip_kvcache* c, int l) {
    return c->v + (size_t)l * c->batch * c->capacity * c->gpt->dim;
}

constexpr int kMaxSplit = 8;  // K slices of the batched-decode residual Linears

static int ensure_acts(gorch_hip_gpt* g, size_t rows, size_t logit_rows) {
    if (rows > g->rows_cap) {
        (void)hipFree(g->x);
        (void)hipFree(g->h);
        (void)hipFree(g->q);
        (void)hipFree(g->att);
        (void)hipFree(g->ff);
        g->x = g->h = g->q = g->att = g->ff = nullptr;
        g->rows_cap = 0;
        const size_t d = g->dim;
        GH_TRY(check(hipMalloc(&g->x, rows * d * 4), "hipMalloc x"));
        GH_TRY(check(hipMalloc(&g->h, rows * d * 4), "hipMalloc h"));
        GH_TRY(check(hipMalloc(&g->q, rows * d * 4), "hipMalloc q"));
        GH_TRY(check(hipMalloc(&g->att, rows * d * 4), "hipMalloc att"));
        GH_TRY(check(hipMalloc(&g->ff, rows * 4 * d * 4), "hipMalloc ff"));
        g->rows_cap = rows;
        if (!g->part) {
            GH_TRY(check(hipMalloc(&g->part, (size_t)kMaxSplit * 16 * d * 4), "hipMalloc part"));
            GH_TRY(check(hipMalloc(&g->stats, 16 * sizeof(float2)), "hipMalloc stats"));
            GH_TRY(check(hipMalloc(&g->wpart, (size_t)kMaxPartSlices * 16 * 3 * d * 4), "hipMalloc wpart"));
            GH_TRY(check(hipMalloc(&g->hfrag, xfrag_bytes((int)d)), "hipMalloc hfrag"));
            GH_TRY(check(hipMalloc(&g->ffrag, xfrag_bytes(4 * (int)d)), "hipMalloc ffrag"));
            // (cleared on the engine's stream, which does not wait for the
            // null stream)
            GH_TRY(check(hipMemsetAsync(g->hfrag, 0, xfrag_bytes((int)d), g->stream), "clear hfrag"));
            GH_TRY(check(hipMemsetAsync(g->ffrag, 0, xfrag_bytes(4 * (int)d), g->stream), "clear ffrag"));
            GH_TRY(check(hipMalloc(&g->afrag, xfrag_bytes((int)d)), "hipMalloc afrag"));
            GH_TRY(check(hipMemsetAsync(g->afrag, 0, xfrag_bytes((int)d), g->stream), "clear afrag"));
            // (forwards may run on a caller's stream: finish the clears here)
            GH_TRY(check(hipStreamSynchronize(g->stream), "clear fragment buffers"));
        }
    }
    if (logit_rows > g->logit_rows_cap) {
        (void)hipFree(g->logits);
        g->logits = nullptr;
        g->logit_rows_cap = 0;
        GH_TRY(check(hipMalloc(&g->logits, logit_rows * g->vocab * 4), "hipMalloc logits"));
        g->logit_rows_cap = logit_rows;
    }
    if (rows > g->ids_cap) {
        (void)hipFree(g->ids);
        g->ids = nullptr;
        g->ids_cap = 0;
        GH_TRY(check(hipMalloc(&g->ids, rows * sizeof(int)), "hipMalloc ids"));
        g->ids_cap = rows;
    }
    return GORCH_HIP_OK;
}

// One GPT forward over n new tokens per sequence (ids already in g->ids,
// row-major [batch, n]). all_rows: LM head on every row (logits
// [batch*n, V]); otherwise only on the last row of each sequence
// (logits [batch, V]). With at most 16 rows the LayerNorms run inside the
// following GEMV; argmax_key (last-row mode, batch <= 16) receives the
// packed greedy choice per sequence. x_ready: x already holds the input
// rows (k_finalize_embed wrote them). Does not advance pos.
static int forward(gorch_hip_gpt* g, gorch_hip_kvcache* c, int n, bool all_rows, hipStream_t s,
                   unsigned long long* argmax_key, bool x_ready = false) {
    const int d = g->dim, B = c->batch, rows = B * n, hd = d / g->heads;
    const float eps = 1e-5f;
    const int* pos = c->state;
    const bool fused = rows <= 16;
    // 2..16 rows: the residual Linears (Wo, FFN2) are split over K across
    // blocks (their N = d alone gives too few blocks to pull HBM at full
    // rate); the slices add themselves into x with float atomics (in
    // deterministic mode one small per-row kernel adds them, the bias and the
    // residual in slice order), and a per-row kernel writes the next
    // LayerNorm's output h, which the following GEMV reads as a plain
    // operand (a LayerNorm fused into the GEMV's loads costs ~3.5 us per
    // call at 16 rows, d 1600, for its gamma/beta loads).
    const bool batched = fused && rows >= 2 && d <= kReduceRowsMaxCols;
    // batched steps over tile-packed weights: the LayerNorm row passes and
    // FFN1 write their outputs in the fragment layout the following tile
    // GEMVs read as their MFMA operand (one contiguous 1 KB per wave and
    // k-step instead of 16 rows of 32-byte pieces, and no split in the
    // GEMV); the LM head reads it when it takes every row
    const bool xfrag = batched && g->wlm_p && g->hfrag;
    const bool head_frag = xfrag && (n == 1 || all_rows);
    LinearExtras xin;
    xin.x_frag = xfrag ? g->hfrag : nullptr;
    // the LayerNorm output of a row pass: fragment layout, or row-major h
    // (and the final one for a head that picks rows)
    auto ln_h = [&](bool last) { return (xfrag && (!last || head_frag)) ? nullptr : g->h; };
    auto ln_hf = [&](bool last) { return ln_h(last) ? nullptr : g->hfrag; };
    // row-major weights (no packed copy, dim above 3072): the K split aims
    // at ~300 blocks of 4 tiles
    constexpr int split_blocks = 300, split_nt = 4;
    // Batched steps over tile-packed weights split the Linears over K: every
    // block of a K slice loads that slice of the activations, so activation
    // traffic is (blocks per slice) x (activation bytes): at 16 rows, d 1600,
    // 1.7x the weight bytes for an unsplit fused QKV and 2.6x for Wo in 2
    // slices. More slices cut it;
    // the partials of the fused QKV are added by the two-pass attention
    // kernel, those of Wo and FFN2 into x (above). The fused QKV takes 3
    // slices by default (XL batch 16, exact-k-step tiles, CU-capped grid:
    // 1 / 2 / 3 / 4 slices 5,249 / 5,330 / 5,335 / 5,240 tok/s).
    constexpr int qkv_split_req = 3;
    // deterministic mode keeps the one-row output projection a GEMV of its
    // own (the fused forms add per-head products with float atomics)
    const bool wo_fuse = !deterministic();
    // Wo's slices, measured at XL batch 16 (with the 3-slice QKV): 2 / 3 / 4
    // / 5 / 6 / 8 slices 5,335 / 5,336 / 5,359 / 5,332 / 5,258 / 5,254 tok/s
    constexpr int wo_split_req = 4;
    // FFN2's slices: packed_split_slices' rule (7 at XL's 6400 x 1600)
    auto res_split = [&](int K) { return packed_split_slices(K, d); };
    auto split_for = [&](int K) {
        const int tiles = ((d + 15) / 16 + split_nt - 1) / split_nt;
        int S = std::min(kMaxSplit, std::max(1, split_blocks / tiles));
        return ksplit_slices(K, S);
    };
    if (!x_ready) GH_TRY(launch_embed_pos(s, g->wte, g->wpe, g->ids, pos, g->x, d, n, rows));
    if (batched)
        GH_TRY(launch_reduce_rows(s, nullptr, 0, nullptr, g->x, rows, d, eps, g->stats, g->L[0].ln1_g,
                                  g->L[0].ln1_b, ln_h(false), ln_hf(false)));
    for (int l = 0; l < g->layers; l++) {
        const LayerW& w = g->L[l];
        OutDesc od{};
        od.nseg = 3;
        od.rows_per_seq = n;
        od.pos_dev = pos;
        od.ptr[0] = g->q;
        od.n_end[0] = d;
        od.seq_stride[0] = (long long)n * d;
        od.row_stride[0] = d;
        od.use_pos[0] = 0;
        od.ptr[1] = kc_layer(c, l);
        od.ptr[2] = vc_layer(c, l);
        od.n_end[1] = 2 * d;
        od.n_end[2] = 3 * d;
        for (int sgi = 1; sgi < 3; sgi++) {
            od.seq_stride[sgi] = (long long)c->capacity * d;
            od.row_stride[sgi] = d;
            od.use_pos[sgi] = 1;
        }
        AttnArgs a{g->q, kc_layer(c, l), vc_layer(c, l), g->att, pos, 0, n, d, hd, c->capacity, d, 1,
                   1.0f / (float)sqrt((double)hd)};
        // chunk records of the key-split long-cache attention (one-row
        // steps): the residual Linears' partial buffer, idle until Wo
        a.split_ws = g->part;
        a.split_ws_floats = (long long)kMaxSplit * 16 * d;
        // one token per sequence over tile-packed weights: the fused QKV
        // Linear split over K into raw partials; the attention kernel adds
        // the slices and the bias and writes the K/V cache rows
        const bool qkv_split = batched && w.wqkv_p && n == 1 &&
                               attn_takes_qkv_part(a, g->heads, rows);
        LinearExtras ln1, ln2;
        if (qkv_split) {
            LinearExtras sp = xin;
            sp.part = g->wpart;
            sp.ksplit = qkv_split_req;
            GH_TRY(launch_linear_packed_od(s, g->h, w.wqkv_p, nullptr, nullptr, OutDesc::plain(nullptr, 3 * d), rows,
                                           3 * d, d, GORCH_HIP_EPI_NONE, sp));
            a.qkv_part = g->wpart;
            a.qkv_bias = w.bqkv;
            a.qkv_slices = ksplit_slices(d, qkv_split_req);
            a.qkv_slice_stride = (long long)rows * 3 * d;
        } else if (batched && w.wqkv_p) {
            GH_TRY(launch_linear_packed_od(s, g->h, w.wqkv_p, w.bqkv, nullptr, od, rows, 3 * d, d,
                                           GORCH_HIP_EPI_NONE, xin));
        } else if (batched) {
            GH_TRY(launch_linear_bf16_od(s, g->h, w.wqkv, w.bqkv, nullptr, od, rows, 3 * d, d, GORCH_HIP_EPI_NONE,
                                         LinearExtras{}));
        } else if (fused) {
            ln1.ln_g = w.ln1_g;
            ln1.ln_b = w.ln1_b;
            ln2.ln_g = w.ln2_g;
            ln2.ln_b = w.ln2_b;
            ln1.ln_eps = ln2.ln_eps = eps;
            GH_TRY(launch_linear_bf16_od(s, g->x, w.wqkv, w.bqkv, nullptr, od, rows, 3 * d, d, GORCH_HIP_EPI_NONE,
                                         ln1));
        } else {
            GH_TRY(launch_layernorm(s, g->x, w.ln1_g, w.ln1_b, g->h, rows, d, eps, d));
            GH_TRY(launch_linear_bf16_od(s, g->h, w.wqkv, w.bqkv, nullptr, od, rows, 3 * d, d, GORCH_HIP_EPI_NONE,
                                         LinearExtras{}));
        }
        // one row (batch 1, one token): the output projection runs inside
        // the attention kernel, which adds Wo . attention + bias into x
        const bool wo_fused = !batched && rows == 1 && wo_fuse && attn_rows_wo_ok(a, g->heads, rows);
        // a longer cache on the key-split path: Wo in its chunk merge, added
        // into x in place
        const bool wo_split = !batched && rows == 1 && wo_fuse && !wo_fused && d % 8 == 0 &&
                              (reinterpret_cast<uintptr_t>(w.wo) % 16) == 0 && attn_split_takes_qk(a, g->heads, rows);
        if (wo_fused) {
            a.wo = w.wo;
            a.wo_bias = w.bo;
            a.wo_out = g->x;
            GH_TRY(launch_attn_rows_wo(s, a, g->heads));
        } else if (wo_split) {
            a.wo = w.wo;
            a.wo_bias = w.bo;
            a.wo_out = g->x;
            a.wo_rows = d;
            a.wo_resid = g->x;
            GH_TRY(launch_attn_cached(s, a, g->heads, rows));
        } else {
            // batched: the attention output in the fragment layout for Wo
            if (xfrag) a.out_frag = g->afrag;
            GH_TRY(launch_attn_cached(s, a, g->heads, rows));
        }
        if (!wo_fused && batched && w.wo_p && wo_fuse) {
            // K slices add themselves (slice 0 with the bias) into x, which
            // holds the residual; the reducer then only normalises
            LinearExtras sp;
            sp.accumulate = true;
            sp.ksplit = ksplit_slices(d, wo_split_req);
            sp.x_frag = xfrag ? g->afrag : nullptr;
            GH_TRY(launch_linear_packed_od(s, g->att, w.wo_p, w.bo, nullptr, OutDesc::plain(g->x, d), rows, d, d,
                                           GORCH_HIP_EPI_NONE, sp));
            GH_TRY(launch_reduce_rows(s, nullptr, 0, nullptr, g->x, rows, d, eps, g->stats, w.ln2_g, w.ln2_b,
                                      ln_h(false), ln_hf(false)));
        } else if (!wo_fused && batched) {
            LinearExtras sp;
            sp.part = g->part;
            sp.ksplit = w.wo_p ? ksplit_slices(d, wo_split_req) : split_for(d);
            sp.x_frag = xfrag ? g->afrag : nullptr;
            if (w.wo_p)
                GH_TRY(launch_linear_packed_od(s, g->att, w.wo_p, nullptr, nullptr, OutDesc::plain(g->x, d), rows, d,
                                               d, GORCH_HIP_EPI_NONE, sp));
            else
                GH_TRY(launch_linear_bf16_od(s, g->att, w.wo, nullptr, nullptr, OutDesc::plain(g->x, d), rows, d, d,
                                             GORCH_HIP_EPI_NONE, sp));
            GH_TRY(launch_reduce_rows(s, g->part, sp.ksplit, w.bo, g->x, rows, d, eps, g->stats, w.ln2_g, w.ln2_b,
                                      ln_h(false), ln_hf(false)));
        } else if (!wo_fused && !wo_split) {
            GH_TRY(launch_linear_bf16(s, g->att, w.wo, w.bo, g->x, g->x, rows, d, d, GORCH_HIP_EPI_NONE));
        }
        if (batched && w.w1_p) {
            LinearExtras f1 = xin;
            f1.out_frag = xfrag ? g->ffrag : nullptr;
            GH_TRY(launch_linear_packed_od(s, g->h, w.w1_p, w.b1, nullptr, OutDesc::plain(g->ff, 4 * d), rows, 4 * d,
                                           d, GORCH_HIP_EPI_GELU, f1));
        } else if (batched) {
            GH_TRY(launch_linear_bf16(s, g->h, w.w1, w.b1, nullptr, g->ff, rows, 4 * d, d, GORCH_HIP_EPI_GELU));
        } else if (fused) {
            GH_TRY(launch_linear_bf16_od(s, g->x, w.w1, w.b1, nullptr, OutDesc::plain(g->ff, 4 * d), rows, 4 * d,
                                         d, GORCH_HIP_EPI_GELU, ln2));
        } else {
            GH_TRY(launch_layernorm(s, g->x, w.ln2_g, w.ln2_b, g->h, rows, d, eps, d));
            GH_TRY(launch_linear_bf16(s, g->h, w.w1, w.b1, nullptr, g->ff, rows, 4 * d, d, GORCH_HIP_EPI_GELU));
        }
        if (batched && w.w2_p && wo_fuse) {
            LinearExtras sp;
            sp.accumulate = true;
            sp.ksplit = res_split(4 * d);
            sp.x_frag = xfrag ? g->ffrag : nullptr;
            GH_TRY(launch_linear_packed_od(s, g->ff, w.w2_p, w.b2, nullptr, OutDesc::plain(g->x, d), rows, d, 4 * d,
                                           GORCH_HIP_EPI_NONE, sp));
            const bool last = l + 1 == g->layers;
            GH_TRY(launch_reduce_rows(s, nullptr, 0, nullptr, g->x, rows, d, eps, g->stats,
                                      last ? g->lnf_g : g->L[l + 1].ln1_g, last ? g->lnf_b : g->L[l + 1].ln1_b,
                                      ln_h(last), ln_hf(last)));
        } else if (batched) {
            LinearExtras sp;
            sp.part = g->part;
            sp.ksplit = w.w2_p ? res_split(4 * d) : split_for(4 * d);
            sp.x_frag = xfrag ? g->ffrag : nullptr;
            if (w.w2_p)
                GH_TRY(launch_linear_packed_od(s, g->ff, w.w2_p, nullptr, nullptr, OutDesc::plain(g->x, d), rows, d,
                                               4 * d, GORCH_HIP_EPI_NONE, sp));
            else
                GH_TRY(launch_linear_bf16_od(s, g->ff, w.w2, nullptr, nullptr, OutDesc::plain(g->x, d), rows, d,
                                             4 * d, GORCH_HIP_EPI_NONE, sp));
            // the next LayerNorm: the next layer's first, or the final one
            const bool last = l + 1 == g->layers;
            GH_TRY(launch_reduce_rows(s, g->part, sp.ksplit, w.b2, g->x, rows, d, eps, g->stats,
                                      last ? g->lnf_g : g->L[l + 1].ln1_g, last ? g->lnf_b : g->L[l + 1].ln1_b,
                                      ln_h(last), ln_hf(last)));
        } else {
            GH_TRY(launch_linear_bf16(s, g->ff, w.w2, w.b2, g->x, g->x, rows, d, 4 * d, GORCH_HIP_EPI_NONE));
        }
    }
    const int head_rows = all_rows ? rows : B;
    const float* head_in = all_rows ? g->x : g->x + (size_t)(n - 1) * d;
    const long long head_stride = all_rows ? d : (long long)n * d;
    if (batched) {
        // h holds LayerNorm_f of every row of x, laid out like x
        LinearExtras lf;
        lf.x_stride = head_stride;
        lf.argmax_key = all_rows ? nullptr : argmax_key;
        if (head_frag) lf.x_frag = g->hfrag;
        const float* head_h = g->h + (head_in - g->x);
        if (g->wlm_p)
            GH_TRY(launch_linear_packed_od(s, head_h, g->wlm_p, g->blm, nullptr, OutDesc::plain(g->logits, g->vocab),
                                           head_rows, g->vocab, d, GORCH_HIP_EPI_NONE, lf));
        else
            GH_TRY(launch_linear_bf16_od(s, head_h, g->wlm, g->blm, nullptr, OutDesc::plain(g->logits, g->vocab),
                                         head_rows, g->vocab, d, GORCH_HIP_EPI_NONE, lf));
    } else if (head_rows <= 16) {
        LinearExtras lf;
        lf.ln_g = g->lnf_g;
        lf.ln_b = g->lnf_b;
        lf.ln_eps = eps;
        lf.x_stride = head_stride;
        lf.argmax_key = all_rows ? nullptr : argmax_key;
        if (head_rows == 1 && gemv_m1_prologue_ok(d)) {
            // one row: the register GEMV over the row-major head, LayerNorm_f
            // staged once per block in its prologue (GPT-2 small batch 1:
            // 17.1 us on the tile-packed head)
            GH_TRY(launch_linear_bf16_od(s, head_in, g->wlm, g->blm, nullptr, OutDesc::plain(g->logits, g->vocab), 1,
                                         g->vocab, d, GORCH_HIP_EPI_NONE, lf));
        } else if (g->wlm_p && d <= 1024) {
            // tile-packed head with LayerNorm_f fused: each block normalises
            // the rows it holds in registers, so no separate LayerNorm launch
            GH_TRY(launch_linear_packed_od(s, head_in, g->wlm_p, g->blm, nullptr,
                                           OutDesc::plain(g->logits, g->vocab), head_rows, g->vocab, d,
                                           GORCH_HIP_EPI_NONE, lf));
        } else if (head_rows == 1 && g->vocab >= 16384) {
            // one row, many weight rows: one small kernel writes the
            // normalised row and the register GEMV streams the head over it
            // plainly (fused into the GEMV, the LayerNorm's registers halve
            // its occupancy: 58 vs 17 us at vocab 50257, d 768)
            GH_TRY(launch_reduce_rows(s, nullptr, 0, nullptr, const_cast<float*>(head_in), 1, d, eps, nullptr,
                                      g->lnf_g, g->lnf_b, g->h));
            LinearExtras hf;
            hf.argmax_key = lf.argmax_key;
            GH_TRY(launch_linear_bf16_od(s, g->h, g->wlm, g->blm, nullptr, OutDesc::plain(g->logits, g->vocab), 1,
                                         g->vocab, d, GORCH_HIP_EPI_NONE, hf));
        } else {
            GH_TRY(launch_linear_bf16_od(s, head_in, g->wlm, g->blm, nullptr, OutDesc::plain(g->logits, g->vocab),
                                         head_rows, g->vocab, d, GORCH_HIP_EPI_NONE, lf));
        }
    } else {
        GH_TRY(launch_layernorm(s, head_in, g->lnf_g, g->lnf_b, g->h, head_rows, d, eps, head_stride));
        GH_TRY(launch_linear_bf16(s, g->h, g->wlm, g->blm, nullptr, g->logits, head_rows, g->vocab, d,
                                  GORCH_HIP_EPI_NONE));
    }
    return GORCH_HIP_OK;
}

// Turns the last forward's logits into each sequence's next token: writes
// it as the next input id and into the history, advances pos by `inc` and
// the step by one. Batches of up to 16 use the argmax fused into the LM
// head (one tiny kernel decodes and clears the keys); larger batches run
// the standalone argmax kernel.
__global__ void k_finalize_step(unsigned long long* key, int B, int* ids, int* hist, int* state, int inc) {
    const int step = state[1];
    for (int b = threadIdx.x; b < B; b += blockDim.x) {
        const int tok = argmax_unpack(argmax_take(key, b));
        ids[b] = tok;
        hist[(size_t)step * B + b] = tok;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        state[0] += inc;
        state[1] = step + 1;
    }
}

// k_finalize_step and the next step's embedding in one launch (up to 16
// sequences): the chosen tokens' wte rows plus the wpe row of the advanced
// position become the next step's input x (k_embed_pos's sum). After the
// last step the position can reach max_seq; that x is never used and reads
// wpe's last row.
__global__ __launch_bounds__(1024) void k_finalize_embed(unsigned long long* key, int B, int* ids, int* hist,
                                                         int* state, int inc, const float* __restrict__ wte,
                                                         const float* __restrict__ wpe, float* __restrict__ x,
                                                         int dim, int max_seq) {
    __shared__ int tok[16];
    const int step = state[1];
    const int pos = state[0] + inc;
    if ((int)threadIdx.x < B) {
        const int t = argmax_unpack(argmax_take(key, threadIdx.x));
        tok[threadIdx.x] = t;
        ids[threadIdx.x] = t;
        hist[(size_t)step * B + threadIdx.x] = t;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        state[0] = pos;
        state[1] = step + 1;
    }
    const float* pe = wpe + (size_t)min(pos, max_seq - 1) * dim;
    constexpr int kV = 8;
    if (dim % 4 == 0 && B * (dim / 4) <= kV * (int)blockDim.x) {
        // at most 8 float4 per thread (16 rows of 2048 floats with 1024
        // threads), all loads issued before the adds and stores
        const int d4 = dim / 4, n4 = B * d4;
        float4 e[kV], p[kV];
#pragma unroll
        for (int u = 0; u < kV; u++) {
            const int i = min((int)threadIdx.x + u * (int)blockDim.x, n4 - 1);
            const int b = i / d4, c4 = i - b * d4;
            e[u] = reinterpret_cast<const float4*>(wte + (size_t)tok[b] * dim)[c4];
            p[u] = reinterpret_cast<const float4*>(pe)[c4];
        }
#pragma unroll
        for (int u = 0; u < kV; u++) {
            const int i = (int)threadIdx.x + u * (int)blockDim.x;
            if (i < n4)
                reinterpret_cast<float4*>(x)[i] =
                    make_float4(e[u].x + p[u].x, e[u].y + p[u].y, e[u].z + p[u].z, e[u].w + p[u].w);
        }
        return;
    }
    for (int i = threadIdx.x; i < B * dim; i += blockDim.x) {
        const int b = i / dim, col = i - b * dim;
        x[i] = wte[(size_t)tok[b] * dim + col] + pe[col];
    }
}

// Decodes the chosen tokens (see k_finalize_step); with embed_next (batches
// of up to 16) it also writes the next step's input rows, and the next
// forward then skips its embedding.
static int choose_tokens(gorch_hip_gpt* g, gorch_hip_kvcache* c, int inc, hipStream_t s, bool embed_next = false) {
    if (c->batch <= 16 && embed_next) {
        // 1024 threads cover 16 rows of 2048 floats with 8 float4 each
        hipLaunchKernelGGL(k_finalize_embed, dim3(1), dim3(c->batch * g->dim > 8 * 4 * 256 ? 1024 : 256), 0, s, c->key,
                           c->batch, g->ids, c->hist, c->state, inc, g->wte, g->wpe, g->x, g->dim, g->max_seq);
        count(CNT_ARGMAX);
        return check_launch("finalize_embed");
    }
    if (c->batch <= 16) {
        hipLaunchKernelGGL(k_finalize_step, dim3(1), dim3(64), 0, s, c->key, c->batch, g->ids, c->hist, c->state,
                           inc);
        count(CNT_ARGMAX);
        return check_launch("finalize_step");
    }
    GH_TRY(launch_argmax(s, g->logits, c->batch, g->vocab, g->ids, c->hist, c->state + 1, c->batch, c->state, inc));
    return launch_advance_step(s, c->state + 1);
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace gh

extern "C" {

namespace gh {

static bool gpt_config_ok(int vocab, int dim, int heads, int layers, int max_seq, const char* who) {
    if (vocab <= 0 || dim <= 0 || heads <= 0 || layers <= 0 || max_seq <= 0 || dim % heads != 0) {
        set_error(std::string(who) + ": bad configuration");
        return false;
    }
    const int hd = dim / heads;
    if (hd % 4 != 0 || hd > 256 || dim % 8 != 0) {
        set_error(std::string(who) + ": needs dim % 8 == 0 and head_dim a multiple of 4, <= 256");
        return false;
    }
    if (!kv_span_ok(max_seq, dim)) {
        set_error(std::string(who) + ": a sequence's cache span (max_seq x dim x 4 bytes) must be below 2 GiB");
        return false;
    }
    if (max_seq > (int)(kAttnMaxLdsBytes / sizeof(float)) && hd != 64 && hd != 128) {
        set_error(std::string(who) + ": max_seq above 16384 needs head_dim 64 or 128");
        return false;
    }
    return true;
}

// Allocates the engine and its weight blob (256-byte aligned slices) and
// points every weight at its slice; the contents are filled by the caller.
static gorch_hip_gpt* gpt_alloc(int vocab, int dim, int heads, int layers, int max_seq) {
    auto* g = new gorch_hip_gpt();
    g->vocab = vocab;
    g->dim = dim;
    g->heads = heads;
    g->layers = layers;
    g->max_seq = max_seq;
    const size_t d = dim, V = vocab, S = max_seq;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off += align256(bytes);
        return o;
    };
    const size_t o_wte = take(V * d * 4), o_wpe = take(S * d * 4), o_lnf_g = take(d * 4), o_lnf_b = take(d * 4);
    const size_t o_wlm = take(V * d * 2), o_blm = take(V * 4);
    struct LOff {
        size_t wqkv, bqkv, wo, bo, w1, b1, w2, b2, ln1_g, ln1_b, ln2_g, ln2_b;
    };
    std::vector<LOff> lo(layers);
    for (int l = 0; l < layers; l++) {
        lo[l].wqkv = take(3 * d * d * 2);
        lo[l].bqkv = take(3 * d * 4);
        lo[l].wo = take(d * d * 2);
        lo[l].bo = take(d * 4);
        lo[l].w1 = take(4 * d * d * 2);
        lo[l].b1 = take(4 * d * 4);
        lo[l].w2 = take(4 * d * d * 2);
        lo[l].b2 = take(d * 4);
        lo[l].ln1_g = take(d * 4);
        lo[l].ln1_b = take(d * 4);
        lo[l].ln2_g = take(d * 4);
        lo[l].ln2_b = take(d * 4);
    }
    if (check(hipMalloc(&g->blob, off), "hipMalloc weights")) {
        delete g;
        return nullptr;
    }
    auto F = [&](size_t o) { return reinterpret_cast<float*>(g->blob + o); };
    auto H = [&](size_t o) { return reinterpret_cast<uint16_t*>(g->blob + o); };
    g->wte = F(o_wte);
    g->wpe = F(o_wpe);
    g->lnf_g = F(o_lnf_g);
    g->lnf_b = F(o_lnf_b);
    g->wlm = H(o_wlm);
    g->blm = F(o_blm);
    g->L.resize(layers);
    for (int l = 0; l < layers; l++) {
        LayerW& L = g->L[l];
        L.wqkv = H(lo[l].wqkv);
        L.bqkv = F(lo[l].bqkv);
        L.wo = H(lo[l].wo);
        L.bo = F(lo[l].bo);
        L.w1 = H(lo[l].w1);
        L.b1 = F(lo[l].b1);
        L.w2 = H(lo[l].w2);
        L.b2 = F(lo[l].b2);
        L.ln1_g = F(lo[l].ln1_g);
        L.ln1_b = F(lo[l].ln1_b);
        L.ln2_g = F(lo[l].ln2_g);
        L.ln2_b = F(lo[l].ln2_b);
    }
    return g;
}

// Creates the engine stream and tile-packed copies of the Linear weights
// (fused QKV, Wo, FFN1, FFN2, LM head), the layout the 2..16-row decode
// GEMVs stream with contiguous 1 KB fragment loads (Wo and FFN2 with K split
// across blocks); the row-major originals serve the single-row decode
// (LayerNorm fused) and prefill. Frees g on failure.
static gorch_hip_gpt* gpt_finish(gorch_hip_gpt* g) {
    if (check(hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking), "hipStreamCreate")) {
        gorch_hip_gpt_free(g);
        return nullptr;
    }
    if (g->dim <= 3072) {
        const int D = g->dim;
        const size_t pq = align256(packed_bf16_elems(3 * D, D) * 2), p1 = align256(packed_bf16_elems(4 * D, D) * 2);
        const size_t po = align256(packed_bf16_elems(D, D) * 2), p2 = align256(packed_bf16_elems(D, 4 * D) * 2);
        const size_t plm = align256(packed_bf16_elems(g->vocab, D) * 2);
        const size_t per_layer = pq + p1 + po + p2;
        g->pblob_bytes = plm + (size_t)g->layers * per_layer;
        if (check(hipMalloc(&g->pblob, g->pblob_bytes), "hipMalloc packed weights")) {
            gorch_hip_gpt_free(g);
            return nullptr;
        }
        g->wlm_p = reinterpret_cast<uint16_t*>(g->pblob);
        int rc = launch_pack_bf16(g->stream, g->wlm, g->wlm_p, g->vocab, D);
        for (int l = 0; l < g->layers && rc == 0; l++) {
            LayerW& L = g->L[l];
            char* base = g->pblob + plm + (size_t)l * per_layer;
            L.wqkv_p = reinterpret_cast<uint16_t*>(base);
            L.w1_p = reinterpret_cast<uint16_t*>(base + pq);
            L.wo_p = reinterpret_cast<uint16_t*>(base + pq + p1);
            L.w2_p = reinterpret_cast<uint16_t*>(base + pq + p1 + po);
            rc = launch_pack_bf16(g->stream, L.wqkv, L.wqkv_p, 3 * D, D);
            if (rc == 0) rc = launch_pack_bf16(g->stream, L.w1, L.w1_p, 4 * D, D);
            if (rc == 0) rc = launch_pack_bf16(g->stream, L.wo, L.wo_p, D, D);
            if (rc == 0) rc = launch_pack_bf16(g->stream, L.w2, L.w2_p, D, 4 * D);
        }
        if (rc != 0 || check(hipStreamSynchronize(g->stream), "pack weights")) {
            gorch_hip_gpt_free(g);
            return nullptr;
        }
    }
    return g;
}

}  // namespace gh

gorch_hip_gpt* gorch_hip_gpt_create(const gorch_hip_gpt_weights* w) {
    if (!w) {
        set_error("gorch_hip_gpt_create: null weights");
        return nullptr;
    }
    if (!gpt_config_ok(w->vocab, w->dim, w->heads, w->layers, w->max_seq, "gorch_hip_gpt_create")) return nullptr;
    gorch_hip_gpt* g = gpt_alloc(w->vocab, w->dim, w->heads, w->layers, w->max_seq);
    if (!g) return nullptr;
    const size_t d = w->dim, V = w->vocab, S = w->max_seq;
    bool ok = true;
    auto put = [&](void* dst, const void* src, size_t bytes) {
        if (!ok) return;
        if (!src) {
            set_error("gorch_hip_gpt_create: null weight pointer");
            ok = false;
            return;
        }
        ok = check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "upload weights") == 0;
    };
    put(g->wte, w->wte, V * d * 4);
    put(g->wpe, w->wpe, S * d * 4);
    put(g->lnf_g, w->lnf_g, d * 4);
    put(g->lnf_b, w->lnf_b, d * 4);
    put(g->wlm, w->wlm, V * d * 2);
    put(g->blm, w->blm, V * 4);
    for (int l = 0; l < w->layers && ok; l++) {
        LayerW& L = g->L[l];
        // the rows of Wq, Wk, Wv back to back: one fused [3d, d] weight
        put(L.wqkv, w->wq[l], d * d * 2);
        put(L.wqkv + d * d, w->wk[l], d * d * 2);
        put(L.wqkv + 2 * d * d, w->wv[l], d * d * 2);
        put(L.bqkv, w->bq[l], d * 4);
        put(L.bqkv + d, w->bk[l], d * 4);
        put(L.bqkv + 2 * d, w->bv[l], d * 4);
        put(L.wo, w->wo[l], d * d * 2);
        put(L.bo, w->bo[l], d * 4);
        put(L.w1, w->w1[l], 4 * d * d * 2);
        put(L.b1, w->b1[l], 4 * d * 4);
        put(L.w2, w->w2[l], 4 * d * d * 2);
        put(L.b2, w->b2[l], d * 4);
        put(L.ln1_g, w->ln1_g[l], d * 4);
        put(L.ln1_b, w->ln1_b[l], d * 4);
        put(L.ln2_g, w->ln2_g[l], d * 4);
        put(L.ln2_b, w->ln2_b[l], d * 4);
    }
    if (!ok) {
        gorch_hip_gpt_free(g);
        return nullptr;
    }
    return gpt_finish(g);
}

gorch_hip_gpt* gorch_hip_gpt_load_gpt2(const char* path, int vocab, int dim, int heads, int layers, int max_seq) {
    if (!gpt_config_ok(vocab, dim, heads, layers, max_seq, "gorch_hip_gpt_load_gpt2")) return nullptr;
    gorch_hip_st* f = gorch_hip_st_open(path);
    if (!f) return nullptr;
    gorch_hip_gpt* g = gpt_alloc(vocab, dim, heads, layers, max_seq);
    if (!g) {
        gorch_hip_st_close(f);
        return nullptr;
    }
    const long long d = dim, V = vocab, S = max_seq;
    bool ok = true;
    // name with or without the GPT2LMHeadModel "transformer." prefix
    auto resolve = [&](const std::string& n) -> std::string {
        if (st_tensor(f, n.c_str())) return n;
        const std::string p = "transformer." + n;
        if (st_tensor(f, p.c_str())) return p;
        return n;
    };
    // copyTensor's checks (model/gpt2_loader.go:139-150): present, same size
    auto load = [&](const std::string& n0, void* dst, long long want_elems, std::vector<long long> want_shape,
                    int dst_dtype, int transpose) {
        if (!ok) return;
        const std::string n = resolve(n0);
        const StTensor* t = st_tensor(f, n.c_str());
        if (!t) {
            set_error("tensor \"" + n0 + "\" not found in safetensors");
            ok = false;
            return;
        }
        long long elems = 1;
        for (long long x : t->shape) elems *= x;
        if (elems != want_elems || (!want_shape.empty() && t->shape != want_shape)) {
            set_error("size mismatch for \"" + n + "\": file=" + std::to_string(elems) +
                      " model=" + std::to_string(want_elems));
            ok = false;
            return;
        }
        ok = st_load_tensor(nullptr, f, n.c_str(), dst, dst_dtype, transpose) == 0;
    };
    constexpr int F32 = GORCH_HIP_ST_F32, B16 = GORCH_HIP_ST_BF16;
    load("wte.weight", g->wte, V * d, {V, d}, F32, 0);
    load("wpe.weight", g->wpe, S * d, {S, d}, F32, 0);
    for (int l = 0; l < layers && ok; l++) {
        const std::string p = "h." + std::to_string(l) + ".";
        LayerW& L = g->L[l];
        load(p + "ln_1.weight", L.ln1_g, d, {}, F32, 0);
        load(p + "ln_1.bias", L.ln1_b, d, {}, F32, 0);
        // Conv1D (d, 3d) -> its transpose [3d, d]: rows 0..d-1 are Q's
        // output features, then K's, then V's (loadFusedQKV, :190-244)
        load(p + "attn.c_attn.weight", L.wqkv, 3 * d * d, {d, 3 * d}, B16, 1);
        load(p + "attn.c_attn.bias", L.bqkv, 3 * d, {}, F32, 0);
        load(p + "attn.c_proj.weight", L.wo, d * d, {d, d}, B16, 1);
        load(p + "attn.c_proj.bias", L.bo, d, {}, F32, 0);
        load(p + "ln_2.weight", L.ln2_g, d, {}, F32, 0);
        load(p + "ln_2.bias", L.ln2_b, d, {}, F32, 0);
        load(p + "mlp.c_fc.weight", L.w1, 4 * d * d, {d, 4 * d}, B16, 1);
        load(p + "mlp.c_fc.bias", L.b1, 4 * d, {}, F32, 0);
        load(p + "mlp.c_proj.weight", L.w2, 4 * d * d, {4 * d, d}, B16, 1);
        load(p + "mlp.c_proj.bias", L.b2, d, {}, F32, 0);
    }
    load("ln_f.weight", g->lnf_g, d, {}, F32, 0);
    load("ln_f.bias", g->lnf_b, d, {}, F32, 0);
    // tied LM head (TieLMHeadToEmbedding): the bf16 rounding of wte, no bias
    load("wte.weight", g->wlm, V * d, {V, d}, B16, 0);
    if (ok) ok = check(hipMemset(g->blm, 0, (size_t)V * 4), "zero LM-head bias") == 0;
    gorch_hip_st_close(f);
    if (!ok) {
        gorch_hip_gpt_free(g);
        return nullptr;
    }
    return gpt_finish(g);
}

size_t gorch_hip_gpt_drop_packed(gorch_hip_gpt* g) {
    if (!g || !g->pblob) return 0;
    (void)hipStreamSynchronize(g->stream);
    // the captured generate step points at the packed weights
    if (g->gen_exec) (void)hipGraphExecDestroy(g->gen_exec);
    if (g->gen_graph) (void)hipGraphDestroy(g->gen_graph);
    g->gen_exec = nullptr;
    g->gen_graph = nullptr;
    g->gen_sig.clear();
    (void)hipFree(g->pblob);
    g->pblob = nullptr;
    g->wlm_p = nullptr;
    for (LayerW& L : g->L) L.wqkv_p = L.w1_p = L.wo_p = L.w2_p = nullptr;
    const size_t freed = g->pblob_bytes;
    g->pblob_bytes = 0;
    return freed;
}

void gorch_hip_gpt_free(gorch_hip_gpt* g) {
    if (!g) return;
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    if (g->gen_exec) (void)hipGraphExecDestroy(g->gen_exec);
    if (g->gen_graph) (void)hipGraphDestroy(g->gen_graph);
    if (g->stream) {
        release_stream_scratch(g->stream);
        (void)hipStreamDestroy(g->stream);
    }
    gorch_hip_kvcache_free(g->gen_cache);
    (void)hipFree(g->blob);
    (void)hipFree(g->pblob);
    (void)hipFree(g->x);
    (void)hipFree(g->h);
    (void)hipFree(g->q);
    (void)hipFree(g->att);
    (void)hipFree(g->ff);
    (void)hipFree(g->logits);
    (void)hipFree(g->part);
    (void)hipFree(g->stats);
    (void)hipFree(g->wpart);
    (void)hipFree(g->hfrag);
    (void)hipFree(g->ffrag);
    (void)hipFree(g->afrag);
    (void)hipFree(g->ids);
    (void)hipFree(g->sample_err);
    (void)hipFree(g->sample_ws);
    delete g;
}

gorch_hip_kvcache* gorch_hip_kvcache_create(gorch_hip_gpt* g, int batch, int capacity) {
    if (!g || batch <= 0 || capacity <= 0 || capacity > g->max_seq) {
        set_error("gorch_hip_kvcache_create: bad batch or capacity (1..max_seq)");
        return nullptr;
    }
    auto* c = new gorch_hip_kvcache();
    c->gpt = g;
    c->batch = batch;
    c->capacity = capacity;
    const size_t elems = (size_t)g->layers * batch * capacity * g->dim;
    if (check(hipMalloc(&c->k, elems * 4), "hipMalloc kv") || check(hipMalloc(&c->v, elems * 4), "hipMalloc kv") ||
        check(hipMalloc(&c->state, 2 * sizeof(int)), "hipMalloc state") ||
        check(hipMalloc(&c->hist, ((size_t)capacity + 1) * batch * sizeof(int)), "hipMalloc hist") ||
        check(hipMalloc(&c->key, (size_t)kArgmaxKeys * sizeof(unsigned long long)), "hipMalloc key") ||
        check(hipMemset(c->key, 0, (size_t)kArgmaxKeys * sizeof(unsigned long long)), "hipMemset key") ||
        check(hipMemset(c->state, 0, 2 * sizeof(int)), "hipMemset state")) {
        gorch_hip_kvcache_free(c);
        return nullptr;
    }
    return c;
}

void gorch_hip_kvcache_free(gorch_hip_kvcache* c) {
    if (!c) return;
    (void)hipFree(c->k);
    (void)hipFree(c->v);
    (void)hipFree(c->state);
    (void)hipFree(c->hist);
    (void)hipFree(c->key);
    delete c;
}

int gorch_hip_kvcache_len(const gorch_hip_kvcache* c) { return c ? c->len : 0; }

int gorch_hip_kvcache_reset(gorch_hip_kvcache* c) {
    GH_REQUIRE(c, "gorch_hip_kvcache_reset: null cache");
    c->len = 0;
    return check(hipMemset(c->state, 0, 2 * sizeof(int)), "kvcache reset");
}

int gorch_hip_kvcache_read(const gorch_hip_kvcache* c, int layer, int seq, float* keys, float* values) {
    GH_REQUIRE(c && layer >= 0 && layer < c->gpt->layers && seq >= 0 && seq < c->batch,
               "gorch_hip_kvcache_read: bad layer or sequence");
    const size_t d = c->gpt->dim, off = ((size_t)layer * c->batch + seq) * c->capacity * d;
    if (keys) GH_TRY(check(hipMemcpy(keys, c->k + off, (size_t)c->len * d * 4, hipMemcpyDeviceToHost), "read k"));
    if (values)
        GH_TRY(check(hipMemcpy(values, c->v + off, (size_t)c->len * d * 4, hipMemcpyDeviceToHost), "read v"));
    return GORCH_HIP_OK;
}

int gorch_hip_gpt_forward_cached(void* stream, gorch_hip_gpt* g, gorch_hip_kvcache* c, const int* ids, int n,
                                 float* logits) {
    GH_REQUIRE(g && c && c->gpt == g && ids && n > 0, "gorch_hip_gpt_forward_cached: bad arguments");
    GH_TRY(bf16_gate(stream_of(stream)));
    if (c->len + n > c->capacity) {
        set_error("gorch_hip_gpt_forward_cached: cached sequence length exceeds MaxSeq");
        return GORCH_HIP_EINVAL;
    }
    const int rows = c->batch * n;
    for (int i = 0; i < rows; i++)
        GH_REQUIRE(ids[i] >= 0 && ids[i] < g->vocab, "gorch_hip_gpt_forward_cached: token id out of range");
    hipStream_t s = stream_of(stream);
    GH_TRY(ensure_acts(g, rows, rows));
    GH_TRY(check(hipMemcpyAsync(g->ids, ids, rows * sizeof(int), hipMemcpyHostToDevice, s), "upload ids"));
    GH_TRY(forward(g, c, n, true, s, nullptr));
    hipLaunchKernelGGL(k_pos_add, dim3(1), dim3(1), 0, s, c->state, n);
    GH_TRY(check_launch("pos_add"));
    c->len += n;
    if (logits)
        GH_TRY(check(hipMemcpyAsync(logits, g->logits, (size_t)rows * g->vocab * 4, hipMemcpyDeviceToHost, s),
                     "download logits"));
    return check(hipStreamSynchronize(s), "forward sync");
}

}  // extern "C"

namespace gh {

// generateCached (model/generate.go:94-131) for `batch` independent prompts:
// greedy choice, stop at StopToken (stop_token >= 0; the token is not kept)
// or once the cache holds MaxSeq tokens. Every sequence's row of out_ids is
// np + max_new wide; its length goes to out_lens[b] (nullable) and the
// longest to *out_len (nullable).
// Sampled choice (generateCached with Temperature > 0, model/generate.go:
// 105-110): the step's LM head writes logits instead of argmax keys and
// k_sample draws each sequence's token into its key slot, which the
// finalize kernel decodes as it does the argmax's.
struct GenSample {
    float temperature;
    int top_k;
    float top_p;
    unsigned long long seed;
};

static int generate_impl(void* stream, gorch_hip_gpt* g, const int* prompts, int batch, int n_prompt, int max_new,
                         int stop_token, int* out_ids, int* out_lens, int* out_len, float* step_logits,
                         float* timing_ms, int flags, const GenSample* smp = nullptr) {
    GH_REQUIRE(g && prompts && out_ids && batch > 0 && n_prompt > 0 && max_new >= 0,
               "gorch_hip_generate_cached: bad arguments");
    GH_TRY(bf16_gate(stream_of(stream)));
    // Prompt truncation to the last MaxSeq tokens (model/generate.go:101-103).
    const int np = n_prompt > g->max_seq ? g->max_seq : n_prompt;
    const int skip = n_prompt - np;
    std::vector<int> ids((size_t)batch * np);
    for (int b = 0; b < batch; b++)
        for (int i = 0; i < np; i++) {
            int t = prompts[(size_t)b * n_prompt + skip + i];
            GH_REQUIRE(t >= 0 && t < g->vocab, "gorch_hip_generate_cached: token id out of range");
            ids[(size_t)b * np + i] = t;
        }
    // The reference loop: token i comes from the latest logits; stop before
    // a forward once the cache holds MaxSeq tokens (model/generate.go:107-129).
    int tokens = 0, forwards = 0, len = np;
    for (int i = 0; i < max_new; i++) {
        tokens++;
        if (len >= g->max_seq) break;
        forwards++;
        len++;
    }
    const int capacity = len;
    GH_TRY(check(hipStreamSynchronize(stream_of(stream)), "caller stream sync"));
    hipStream_t s = g->stream;
    gorch_hip_kvcache* c = g->gen_cache;
    if (c && c->batch == batch && c->capacity == capacity) {
        // reuse: empty cache, zero keys (the graph reads both from device memory)
        c->len = 0;
        GH_TRY(check(hipMemsetAsync(c->state, 0, 2 * sizeof(int), s), "reset state"));
        GH_TRY(check(hipMemsetAsync(c->key, 0, (size_t)kArgmaxKeys * sizeof(unsigned long long), s), "reset keys"));
    } else {
        if (g->gen_exec) (void)hipGraphExecDestroy(g->gen_exec);
        if (g->gen_graph) (void)hipGraphDestroy(g->gen_graph);
        g->gen_exec = nullptr;
        g->gen_graph = nullptr;
        g->gen_sig.clear();
        gorch_hip_kvcache_free(g->gen_cache);
        g->gen_cache = nullptr;
        c = gorch_hip_kvcache_create(g, batch, capacity);
        if (!c) return GORCH_HIP_ENOMEM;
        g->gen_cache = c;
    }
    if (smp) {
        if (!g->sample_err && check(hipMalloc(&g->sample_err, sizeof(int)), "hipMalloc sample flag"))
            return GORCH_HIP_ENOMEM;
        GH_TRY(check(hipMemsetAsync(g->sample_err, 0, sizeof(int), s), "reset sample flag"));
        if (batch > g->sample_ws_rows) {
            GH_TRY(check(hipStreamSynchronize(s), "sample workspace"));
            (void)hipFree(g->sample_ws);
            g->sample_ws = nullptr;
            g->sample_ws_rows = 0;
            if (check(hipMalloc(&g->sample_ws, sample_ws_bytes(batch)), "hipMalloc sample workspace"))
                return GORCH_HIP_ENOMEM;
            GH_TRY(check(hipMemsetAsync(g->sample_ws, 0, sample_ws_bytes(batch), s), "clear sample workspace"));
            g->sample_ws_rows = batch;
        }
    }
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    int rc = GORCH_HIP_OK;
    const bool use_graph = (flags & 1) && !step_logits;
    // the step's choice: the fused argmax, or the sampler over the logits
    unsigned long long* head_key = smp ? nullptr : c->key;
    auto sample_tokens = [&]() -> int {
        if (!smp) return GORCH_HIP_OK;
        return launch_sample(s, g->logits, batch, g->vocab, smp->temperature, smp->top_k, smp->top_p, nullptr,
                             smp->seed, c->state + 1, nullptr, nullptr, c->key, g->sample_err, false,
                             g->sample_ws);
    };
    auto fail = [&](int r) {
        rc = r;
        return r;
    };
    do {
        if (ensure_acts(g, (size_t)batch * np, batch)) { fail(GORCH_HIP_ENOMEM); break; }
        for (auto& e : ev)
            if (check(hipEventCreate(&e), "hipEventCreate")) { fail(GORCH_HIP_ERUNTIME); break; }
        if (rc) break;
        if (check(hipMemcpyAsync(g->ids, ids.data(), ids.size() * sizeof(int), hipMemcpyHostToDevice, s), "ids")) {
            fail(GORCH_HIP_ERUNTIME);
            break;
        }
        (void)hipEventRecord(ev[0], s);
        // prefill: logits of the last prompt row per sequence -> token 0
        // batches of up to 16: each choice also embeds the next step's input
        const bool fin_embed = batch <= 16;
        if (forward(g, c, np, false, s, head_key) || sample_tokens() || choose_tokens(g, c, np, s, fin_embed)) {
            fail(GORCH_HIP_ERUNTIME);
            break;
        }
        (void)hipEventRecord(ev[1], s);
        if (step_logits) {
            if (check(hipMemcpyAsync(step_logits, g->logits, (size_t)batch * g->vocab * 4, hipMemcpyDeviceToHost, s),
                      "logits")) { fail(GORCH_HIP_ERUNTIME); break; }
        }
        // one decode step: forward the latest token of each sequence, choose the next
        auto step = [&]() -> int {
            GH_TRY(forward(g, c, 1, false, s, head_key, fin_embed));
            GH_TRY(sample_tokens());
            return choose_tokens(g, c, 1, s, fin_embed);
        };
        if (use_graph && forwards > 0) {
            // capture the step once (or again when a buffer it points at moved)
            const std::vector<const void*> sig = {g->x,    g->h,    g->q,    g->att,      g->ff,
                                                  g->logits, g->ids, g->part, g->stats, c->k,
                                                  c->v,    c->state, c->hist, c->key,
                                                  // the kernels differ by the deterministic setting
                                                  reinterpret_cast<const void*>(deterministic() ? 1 : 0),
                                                  // and by the sampling parameters (kernel arguments)
                                                  reinterpret_cast<const void*>(smp ? 1 : 0), g->sample_err,
                                                  g->sample_ws,
                                                  reinterpret_cast<const void*>(
                                                      smp ? (uintptr_t)__builtin_bit_cast(uint32_t, smp->temperature) : 0),
                                                  reinterpret_cast<const void*>(smp ? (uintptr_t)smp->top_k : 0),
                                                  reinterpret_cast<const void*>(
                                                      smp ? (uintptr_t)__builtin_bit_cast(uint32_t, smp->top_p) : 0),
                                                  reinterpret_cast<const void*>(smp ? (uintptr_t)smp->seed : 0)};
            if (!g->gen_exec || g->gen_sig != sig) {
                if (g->gen_exec) (void)hipGraphExecDestroy(g->gen_exec);
                if (g->gen_graph) (void)hipGraphDestroy(g->gen_graph);
                g->gen_exec = nullptr;
                g->gen_graph = nullptr;
                g->gen_sig.clear();
                // the step's K-split Linears take their partials from the
                // stream's scratch, which cannot grow under capture: size
                // it for the widest of them (the FFN-up, 4d) first
                (void)stream_scratch(s, (size_t)kMaxSplit * std::min(batch, 16) * 4 * g->dim * sizeof(float));
                if (check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture")) {
                    fail(GORCH_HIP_ERUNTIME);
                    break;
                }
                int r = step();
                hipError_t e = hipStreamEndCapture(s, &g->gen_graph);
                if (r || check(e, "end capture") ||
                    check(hipGraphInstantiate(&g->gen_exec, g->gen_graph, nullptr, nullptr, 0), "instantiate")) {
                    fail(GORCH_HIP_ERUNTIME);
                    break;
                }
                g->gen_sig = sig;
            }
        }
        // With a stop token, the tokens chosen so far are read back every
        // kStopCheck steps and generation ends once every sequence has
        // produced it (the reference's loop breaks there; a sequence that
        // stopped early keeps decoding into ignored positions meanwhile).
        constexpr int kStopCheck = 8;
        std::vector<int> seen;
        int chosen = 1;  // tokens chosen so far (the prefill chose token 0)
        int done_forwards = 0;
        auto all_stopped = [&]() -> int {
            seen.resize((size_t)chosen * batch);
            GH_TRY(check(hipMemcpyAsync(seen.data(), c->hist, seen.size() * sizeof(int), hipMemcpyDeviceToHost, s),
                         "hist"));
            GH_TRY(check(hipStreamSynchronize(s), "stop check sync"));
            for (int b = 0; b < batch; b++) {
                bool hit = false;
                for (int i = 0; i < chosen && !hit; i++) hit = seen[(size_t)i * batch + b] == stop_token;
                if (!hit) return 0;
            }
            return 1;
        };
        bool stopped = false;
        if (stop_token >= 0) {
            const int r = all_stopped();
            if (r < 0 || r > 1) { fail(r); break; }
            stopped = r == 1;
        }
        for (int i = 0; i < forwards && !rc && !stopped; i++) {
            if (use_graph) {
                if (check(hipGraphLaunch(g->gen_exec, s), "graph launch")) { fail(GORCH_HIP_ERUNTIME); break; }
            } else {
                if (step()) { fail(GORCH_HIP_ERUNTIME); break; }
                if (step_logits && i + 1 < tokens) {
                    if (check(hipMemcpyAsync(step_logits + (size_t)(i + 1) * batch * g->vocab, g->logits,
                                             (size_t)batch * g->vocab * 4, hipMemcpyDeviceToHost, s), "logits"))
                        fail(GORCH_HIP_ERUNTIME);
                }
            }
            chosen++;
            done_forwards++;
            if (stop_token >= 0 && (chosen % kStopCheck == 0 || i + 1 == forwards)) {
                const int r = all_stopped();
                if (r < 0 || r > 1) { fail(r); break; }
                stopped = r == 1;
            }
        }
        if (rc) break;
        (void)hipEventRecord(ev[2], s);
        const int have = std::min(tokens, chosen);  // tokens chosen on the device
        std::vector<int> hist((size_t)have * batch);
        if (have > 0 &&
            check(hipMemcpyAsync(hist.data(), c->hist, hist.size() * sizeof(int), hipMemcpyDeviceToHost, s), "hist")) {
            fail(GORCH_HIP_ERUNTIME);
            break;
        }
        if (check(hipStreamSynchronize(s), "generate sync")) { fail(GORCH_HIP_ERUNTIME); break; }
        if (smp) {
            int flag = 0;
            if (check(hipMemcpy(&flag, g->sample_err, sizeof(int), hipMemcpyDeviceToHost), "sample flag")) {
                fail(GORCH_HIP_ERUNTIME);
                break;
            }
            if (flag) {
                set_error("gorch_hip_generate: more than 4096 top-p candidates (ties at the top-k threshold)");
                fail(GORCH_HIP_EUNSUPPORTED);
                break;
            }
        }
        // result = (truncated) prompt followed by the generated tokens, each
        // sequence cut before its first stop token
        const int width = np + max_new;
        int longest = np;
        for (int b = 0; b < batch; b++) {
            int* row = out_ids + (size_t)b * width;
            for (int i = 0; i < np; i++) row[i] = ids[(size_t)b * np + i];
            int n = 0;
            while (n < have && !(stop_token >= 0 && hist[(size_t)n * batch + b] == stop_token)) {
                row[np + n] = hist[(size_t)n * batch + b];
                n++;
            }
            if (out_lens) out_lens[b] = np + n;
            longest = std::max(longest, np + n);
        }
        if (out_len) *out_len = longest;
        if (timing_ms) {
            float a = 0.f, bb = 0.f;
            (void)hipEventElapsedTime(&a, ev[0], ev[1]);
            (void)hipEventElapsedTime(&bb, ev[1], ev[2]);
            timing_ms[0] = a;
            timing_ms[1] = bb;
            timing_ms[2] = (float)done_forwards;
        }
    } while (false);
    for (auto& e : ev)
        if (e) (void)hipEventDestroy(e);
    (void)hipStreamSynchronize(s);
    return rc;
}

}  // namespace gh

extern "C" {

int gorch_hip_generate_cached(void* stream, gorch_hip_gpt* g, const int* prompts, int batch, int n_prompt,
                              int max_new, int* out_ids, int* out_len, float* step_logits, float* timing_ms,
                              int flags) {
    GH_REQUIRE(out_len, "gorch_hip_generate_cached: null out_len");
    // rows are n_prompt + max_new wide before truncation; this entry point
    // has no stop token, so every row has the same length: repack densely
    const int rc = generate_impl(stream, g, prompts, batch, n_prompt, max_new, -1, out_ids, nullptr, out_len,
                                 step_logits, timing_ms, flags);
    if (rc) return rc;
    const int np = n_prompt > g->max_seq ? g->max_seq : n_prompt, width = np + max_new, len = *out_len;
    for (int b = 1; b < batch; b++)
        std::memmove(out_ids + (size_t)b * len, out_ids + (size_t)b * width, (size_t)len * sizeof(int));
    return GORCH_HIP_OK;
}

int gorch_hip_generate(void* stream, gorch_hip_gpt* g, const int* prompts, int batch, int n_prompt,
                       const gorch_hip_generate_config* cfg, int* out_ids, int* out_lens, float* step_logits,
                       float* timing_ms) {
    GH_REQUIRE(cfg && out_lens, "gorch_hip_generate: null config or out_lens");
    if (!cfg->use_kv_cache) {
        set_error("gorch_hip_generate: only decoding with the KV cache runs here (UseKVCache)");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if (cfg->temperature == 0.0f)
        return generate_impl(stream, g, prompts, batch, n_prompt, cfg->max_new_tokens, cfg->stop_token, out_ids,
                             out_lens, nullptr, step_logits, timing_ms, cfg->flags);
    // sampled: up to 16 sequences (the finalize kernel's key path)
    GH_REQUIRE(g && batch >= 1, "gorch_hip_generate: bad arguments");
    if (batch > 16) {
        set_error("gorch_hip_generate: sampled generation runs for up to 16 sequences");
        return GORCH_HIP_EUNSUPPORTED;
    }
    GH_TRY(sample_check(batch, g->vocab, cfg->temperature, cfg->top_k, cfg->top_p));
    const GenSample smp{cfg->temperature, cfg->top_k, cfg->top_p, cfg->seed};
    return generate_impl(stream, g, prompts, batch, n_prompt, cfg->max_new_tokens, cfg->stop_token, out_ids,
                         out_lens, nullptr, step_logits, timing_ms, cfg->flags, &smp);
}

}  // extern "C"
