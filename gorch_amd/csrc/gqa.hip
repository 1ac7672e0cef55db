// gqa.hip — grouped-query attention with a KV cache (GQA.forwardCached,
// nn/gqa.go:259-363, with ProjectQKV :213-256) as a host-side composite of
// the library's kernels, on one stream, no allocation (caller workspace):
//   Q, K, V projections (bf16 Linears) -> optional per-head QK RMSNorm
//   (Qwen3 qk-norm, applied before RoPE) -> RoPE on Q and on K at absolute
//   positions (K rotated straight into the cache rows, V projected straight
//   into them) -> grouped-query attention over the cache -> Wo Linear.
// Activations stay token-major [seq, heads*hd]; the reference's permutes to
// (heads, seq, hd) only change layout, not values.
#include "common.h"

namespace gh {
int launch_rope_rows(hipStream_t s, const float* x, float* y, int rows, int heads, int hd, int start_pos,
                     const float* cosT, const float* sinT, int neox);
int launch_rmsnorm(hipStream_t s, const float* x, const float* g, float* y, int M, int N, float eps);
int launch_norm_rope_rows(hipStream_t s, const float* x, float* y, int rows, int heads, int hd, const float* g,
                          float eps, int start_pos, const float* cosT, const float* sinT, int neox);
// pos_dev (nullable): start position read on the device; yk then starts at
// yk + *pos_dev * yk_pos_stride
int launch_norm_rope_rows2(hipStream_t s, const float* xq, float* yq, int rows_q, int heads_q, const float* gq,
                           const float* xk, float* yk, int rows_k, int heads_k, const float* gk, int hd, float eps,
                           int start_pos, const float* cosT, const float* sinT, int neox,
                           const int* pos_dev = nullptr, long long yk_pos_stride = 0);
}  // namespace gh

using namespace gh;

namespace gh {
// q, the attention output (both [S, q heads * hd]), k before RoPE [S, kv
// heads * hd], room for a normalised input [S, dim] (the block path), and
// for one-row steps the key-split attention's chunk records.
size_t gqa_ws(int new_seq, int num_q, int num_kv, int hd, int dim) {
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    return al((size_t)new_seq * num_q * hd * 4) * 2 + al((size_t)new_seq * num_kv * hd * 4) +
           al((size_t)new_seq * dim * 4) + (new_seq == 1 ? al((size_t)num_q * kAttnSplitMax * (hd + 2) * 4) : 0);
}
}  // namespace gh

extern "C" size_t gorch_hip_gqa_workspace_size(const gorch_hip_gqa_weights* w, int new_seq) {
    if (!w || new_seq <= 0) return 0;
    return gqa_ws(new_seq, w->num_q, w->num_kv, w->head_dim, w->dim);
}

namespace gh {

// GQA.forwardCached for one sequence. pre_gain (nullable): an RMSNorm of x
// (gain, pre_eps) applied first — the decoder block's norm before attention
// — fused into the one-row QKV GEMV, else a separate launch into h. resid
// (nullable): added to the Wo output (the block's residual add).
int gqa_core(hipStream_t s, const gorch_hip_gqa_weights* w, const float* x, int S, float* k_cache, float* v_cache,
             int pos_offset, int max_seq, float* out, char* ws, const float* pre_gain, float pre_eps,
             const float* resid, const int* pos_dev) {
    const int nq = w->num_q, nkv = w->num_kv, hd = w->head_dim, d = w->dim;
    const int qdim = nq * hd, kvdim = nkv * hd;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    float* q = (float*)ws;
    float* att = (float*)(ws + al((size_t)S * qdim * 4));
    float* kt = (float*)(ws + 2 * al((size_t)S * qdim * 4));
    float* h = (float*)(ws + 2 * al((size_t)S * qdim * 4) + al((size_t)S * kvdim * 4));
    float* split = S == 1 ? (float*)((char*)h + al((size_t)S * d * 4)) : nullptr;
    if (pos_dev && S != 1) {
        set_error("gqa: a device-side position needs one new row");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if (pos_dev) pos_offset = 0;
    float* krow = k_cache + (size_t)pos_offset * kvdim;
    float* vrow = v_cache + (size_t)pos_offset * kvdim;

    // Q, K, V in one GEMV/GEMM when the three weights (and biases) are one
    // contiguous [q + 2 kv, d] block: Q and K to the workspace, V straight
    // into its cache rows
    const bool wfused = w->wk == w->wq + (size_t)qdim * d && w->wv == w->wk + (size_t)kvdim * d;
    const bool bnone = !w->bq && !w->bk && !w->bv;
    const bool bfused = w->bq && w->bk == w->bq + qdim && w->bv == w->bk + kvdim;
    const bool one_row_norm = pre_gain && S == 1 && gemv_m1_prologue_ok(d);
    if (pre_gain && !(one_row_norm && wfused && (bnone || bfused))) {
        GH_TRY(launch_rmsnorm(s, x, pre_gain, h, S, d, pre_eps));
        x = h;
        pre_gain = nullptr;
    }
    if (wfused && (bnone || bfused)) {
        OutDesc od{};
        od.nseg = 3;
        od.rows_per_seq = 1 << 30;
        od.pos_dev = pos_dev;
        float* dst[3] = {q, kt, vrow};
        const int ends[3] = {qdim, qdim + kvdim, qdim + 2 * kvdim};
        const int widths[3] = {qdim, kvdim, kvdim};
        for (int i = 0; i < 3; i++) {
            od.ptr[i] = dst[i];
            od.n_end[i] = ends[i];
            od.seq_stride[i] = 0;
            od.row_stride[i] = widths[i];
            // the V row at the device position (vrow is the cache base then)
            od.use_pos[i] = pos_dev && i == 2 ? 1 : 0;
        }
        LinearExtras ex;
        if (pre_gain) {
            ex.ln_g = pre_gain;
            ex.ln_rms = true;
            ex.ln_eps = pre_eps;
        }
        GH_TRY(launch_linear_bf16_od(s, x, w->wq, w->bq, nullptr, od, S, qdim + 2 * kvdim, d, GORCH_HIP_EPI_NONE,
                                     ex));
    } else {
        if (pos_dev) {
            set_error("gqa: a device-side position needs Q, K and V rows of one weight");
            return GORCH_HIP_EUNSUPPORTED;
        }
        GH_TRY(launch_linear_bf16(s, x, w->wq, w->bq, nullptr, q, S, qdim, d, GORCH_HIP_EPI_NONE));
        GH_TRY(launch_linear_bf16(s, x, w->wk, w->bk, nullptr, kt, S, kvdim, d, GORCH_HIP_EPI_NONE));
        GH_TRY(launch_linear_bf16(s, x, w->wv, w->bv, nullptr, vrow, S, kvdim, d, GORCH_HIP_EPI_NONE));
    }
    AttnArgs a{q, k_cache, v_cache, att, pos_dev, pos_offset, S, qdim, hd, max_seq, qdim, w->causal ? 1 : 0,
               (float)(1.0 / sqrt((double)hd)), nkv, kvdim, 1};
    a.split_ws = split;
    a.split_ws_floats = split ? (long long)nq * kAttnSplitMax * (hd + 2) : 0;
    // per-head RMSNorm and RoPE of q and k: inside the key-split attention
    // kernel for one-row steps that take it; else in one launch when the
    // head fits one wave (hd % 8 == 0, hd <= 256, 16-byte rows)
    const bool aligned16 = ((reinterpret_cast<uintptr_t>(krow) | reinterpret_cast<uintptr_t>(q) |
                             reinterpret_cast<uintptr_t>(kt) | reinterpret_cast<uintptr_t>(w->q_norm) |
                             reinterpret_cast<uintptr_t>(w->k_norm)) % 16) == 0;
    const bool fused = w->rope_cos && hd % 8 == 0 && hd <= 256 &&
                       ((reinterpret_cast<uintptr_t>(krow) | reinterpret_cast<uintptr_t>(q) |
                         reinterpret_cast<uintptr_t>(kt)) % 16) == 0;
    if (aligned16 && attn_split_takes_qk(a, nq, S)) {
        a.k_raw = kt;
        a.q_gain = w->q_norm;
        a.k_gain = w->k_norm;
        a.qk_eps = w->norm_eps;
        a.rope_cos = w->rope_cos;
        a.rope_sin = w->rope_sin;
        a.rope_neox = w->rope_neox;
    } else if (fused) {
        // (with pos_dev krow is the cache base and the kernel offsets it)
        GH_TRY(launch_norm_rope_rows2(s, q, q, S * nq, nq, w->q_norm, kt, krow, S * nkv, nkv, w->k_norm, hd,
                                      w->norm_eps, pos_offset, w->rope_cos, w->rope_sin, w->rope_neox, pos_dev,
                                      kvdim));
    } else if (pos_dev) {
        set_error("gqa: a device-side position needs RoPE and head_dim % 8 == 0, <= 256");
        return GORCH_HIP_EUNSUPPORTED;
    } else {
        if (w->q_norm) GH_TRY(launch_rmsnorm(s, q, w->q_norm, q, S * nq, hd, w->norm_eps));
        if (w->k_norm) GH_TRY(launch_rmsnorm(s, kt, w->k_norm, kt, S * nkv, hd, w->norm_eps));
        if (w->rope_cos) {
            GH_TRY(launch_rope_rows(s, q, q, S * nq, nq, hd, pos_offset, w->rope_cos, w->rope_sin, w->rope_neox));
            GH_TRY(launch_rope_rows(s, kt, krow, S * nkv, nkv, hd, pos_offset, w->rope_cos, w->rope_sin,
                                    w->rope_neox));
        } else {
            GH_TRY(check(hipMemcpyAsync(krow, kt, (size_t)S * kvdim * 4, hipMemcpyDeviceToDevice, s),
                         "gqa k copy"));
        }
    }
    // one-row steps on the key-split path: Wo (+ bias and the residual) in
    // the kernel that merges the key chunks, added into out with float
    // atomics per head (not in deterministic mode)
    const bool wo_in_attn = !deterministic();
    if (wo_in_attn && S == 1 && qdim % 8 == 0 && (reinterpret_cast<uintptr_t>(w->wo) % 16) == 0 &&
        attn_split_takes_qk(a, nq, S)) {
        a.wo = w->wo;
        a.wo_bias = w->bo;
        a.wo_out = out;
        a.wo_rows = d;
        a.wo_resid = resid;
        return launch_attn_cached(s, a, nq, S);
    }
    GH_TRY(launch_attn_cached(s, a, nq, S));
    return launch_linear_bf16(s, att, w->wo, w->bo, resid, out, S, d, qdim, GORCH_HIP_EPI_NONE);
}

int gqa_check(const gorch_hip_gqa_weights* w, int S, int pos_offset, int max_seq) {
    const int nq = w->num_q, nkv = w->num_kv, hd = w->head_dim, d = w->dim;
    GH_REQUIRE(nq > 0 && nkv > 0 && hd > 0 && d > 0, "gorch/nn: GQAConfig fields must be positive");
    GH_REQUIRE(nq % nkv == 0, "gorch/nn: GQA NumQ must be divisible by NumKV");
    GH_REQUIRE(pos_offset >= 0 && pos_offset + S <= max_seq, "gorch_hip_gqa_forward_cached: cache overflow");
    GH_SUPPORTED(kv_span_ok(max_seq, (long long)nkv * hd),
               "gorch_hip_gqa_forward_cached: a sequence's cache span (max_seq x kv_dim x 4 bytes) must be below 2 GiB");
    GH_REQUIRE(w->wq && w->wk && w->wv && w->wo, "gorch_hip_gqa_forward_cached: null projection weight");
    GH_REQUIRE(!w->rope_cos == !w->rope_sin, "gorch_hip_gqa_forward_cached: need both RoPE tables");
    GH_REQUIRE(!w->rope_cos || pos_offset + S <= w->rope_max_seq, "gorch/nn: RoPE startPos+seqLen exceeds MaxSeq");
    return GORCH_HIP_OK;
}

}  // namespace gh

extern "C" int gorch_hip_gqa_forward_cached(void* stream, const gorch_hip_gqa_weights* w, const float* x,
                                            int new_seq, float* k_cache, float* v_cache, int pos_offset,
                                            int max_seq, float* out, void* workspace, size_t workspace_bytes) {
    GH_REQUIRE(w && x && k_cache && v_cache && out && new_seq > 0, "gorch_hip_gqa_forward_cached: bad arguments");
    GH_TRY(bf16_gate(stream_of(stream)));
    GH_TRY(gqa_check(w, new_seq, pos_offset, max_seq));
    const size_t need = gqa_ws(new_seq, w->num_q, w->num_kv, w->head_dim, w->dim);
    GH_REQUIRE(workspace && workspace_bytes >= need, "gorch_hip_gqa_forward_cached: workspace too small");
    return finish(stream, gqa_core(stream_of(stream), w, x, new_seq, k_cache, v_cache, pos_offset, max_seq, out,
                                   static_cast<char*>(workspace), nullptr, 0.f, nullptr));
}
