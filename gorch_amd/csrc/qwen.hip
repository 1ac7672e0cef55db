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
#include "common.h"

namespace gh {

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

extern "C" int gorch_hip_qwen_block_forward_cached(void* stream, const gorch_hip_qwen_block* b, float* x,
                                                   int new_seq, float* k_cache, float* v_cache, int pos_offset,
                                                   int max_seq, void* workspace, size_t workspace_bytes) {
    GH_REQUIRE(b && x && k_cache && v_cache && new_seq > 0, "gorch_hip_qwen_block_forward_cached: bad arguments");
    GH_REQUIRE(b->norm_attn && b->norm_ffn && b->wgate_up && b->wdown && b->inter > 0,
               "gorch_hip_qwen_block_forward_cached: null block weight");
    GH_TRY(bf16_gate(stream_of(stream)));
    const gorch_hip_gqa_weights* w = &b->attn;
    GH_TRY(gqa_check(w, new_seq, pos_offset, max_seq));
    GH_REQUIRE(workspace && workspace_bytes >= qwen_ws(b, new_seq),
               "gorch_hip_qwen_block_forward_cached: workspace too small");
    hipStream_t s = stream_of(stream);
    const int S = new_seq, d = w->dim, F = b->inter;
    char* base = static_cast<char*>(workspace);
    char* gws = base;
    float* x1 = reinterpret_cast<float*>(base + al256(gqa_ws(S, w->num_q, w->num_kv, w->head_dim, d)));
    float* h = reinterpret_cast<float*>(reinterpret_cast<char*>(x1) + al256((size_t)S * d * 4));
    float* gu = reinterpret_cast<float*>(reinterpret_cast<char*>(h) + al256((size_t)S * d * 4));

    // x1 = x + Wo(attention(RMSNorm_attn(x)))
    GH_TRY(gqa_core(s, w, x, S, k_cache, v_cache, pos_offset, max_seq, x1, gws, b->norm_attn, b->eps, x));
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
            return finish(stream, launch_linear_bf16_od(s, gu, b->wdown, nullptr, x1, OutDesc::plain(x, d), 1, d, F,
                                                        GORCH_HIP_EPI_NONE, LinearExtras{}));
        }
        GH_TRY(launch_linear_bf16_od(s, x1, b->wgate_up, nullptr, nullptr, OutDesc::plain(gu, 2 * F), 1, 2 * F, d,
                                     GORCH_HIP_EPI_NONE, pre));
        LinearExtras sw;
        sw.swiglu = true;
        return finish(stream, launch_linear_bf16_od(s, gu, b->wdown, nullptr, x1, OutDesc::plain(x, d), 1, d, F,
                                                    GORCH_HIP_EPI_NONE, sw));
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
    return finish(stream, launch_linear_bf16(s, gate, b->wdown, nullptr, x1, x, S, d, F, GORCH_HIP_EPI_NONE));
}
