// rope.hip — rotary position embedding (nn/rope.go:71-223; RoPEApplyMetal,
// rope_metal.go:35-62; MSL rope_apply, metal/kernels.go:470-500).
//
// Tables: invFreq = f32(base^(-2i/hd)) (computed in f64), theta =
// f64(f32(pos) * invFreq) — the product is rounded to f32 first, as the
// reference does to match HF's float32 rotary tables — cos/sin in f64
// rounded to f32. Rotation of each pair (a, b) by (c, s*sign):
// (a*c - b*s, a*s + b*c), the Llama half-split pairing (x[i], x[i+hd/2]) or
// the NeoX interleaved one (x[2i], x[2i+1]). Products and sums are rounded
// separately (no fused multiply-add), exactly as the reference's statements
// read (contraction is switched off in rotate_pair), so with equal tables the
// GPU result is bit-identical to that unfused order.
#include "common.h"

namespace gh {

__global__ void k_rope_tables(int hd, int max_seq, float base, float* cosT, float* sinT) {
    const int half = hd / 2;
    for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < (int64_t)max_seq * half;
         id += (int64_t)gridDim.x * blockDim.x) {
        const int pos = (int)(id / half), i = (int)(id - (int64_t)pos * half);
        const float inv_freq = (float)pow((double)base, -(double)(2 * i) / (double)hd);
        const float prod = __fmul_rn((float)pos, inv_freq);
        const double theta = (double)prod;
        cosT[id] = (float)cos(theta);
        sinT[id] = (float)sin(theta);
    }
}

__device__ __forceinline__ void rotate_pair(const float* x, float* y, int64_t row_off, int i, int half, int neox,
                                            float c, float si) {
#pragma clang fp contract(off)
    const int ia = neox ? 2 * i : i;
    const int ib = neox ? 2 * i + 1 : half + i;
    const float a = x[row_off + ia], b = x[row_off + ib];
    y[row_off + ia] = a * c - b * si;
    y[row_off + ib] = a * si + b * c;
}

// Reference layout (outer, seq, hd): row t = (o, s) is at position
// start_pos + (t mod seq).
__global__ void k_rope_apply(const float* x, float* y, int64_t outer_seq, int seq, int half, int start_pos,
                             const float* __restrict__ cosT, const float* __restrict__ sinT, int neox, float sign) {
    for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < outer_seq * half;
         id += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = id / half;
        const int i = (int)(id - t * half);
        const int s = (int)(t % seq);
        const int64_t cs = (int64_t)(start_pos + s) * half + i;
        rotate_pair(x, y, t * 2 * half, i, half, neox, cosT[cs], sinT[cs] * sign);
    }
}

// Token-major layout [rows = seq*heads, hd]: row r is token r / heads (the
// same rotation as the reference applies to its (heads, seq, hd) view).
__global__ void k_rope_rows(const float* x, float* y, int64_t rows, int heads, int half, int start_pos,
                            const float* __restrict__ cosT, const float* __restrict__ sinT, int neox) {
    for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < rows * half;
         id += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = id / half;
        const int i = (int)(id - r * half);
        const int64_t cs = (int64_t)(start_pos + (int)(r / heads)) * half + i;
        rotate_pair(x, y, r * 2 * half, i, half, neox, cosT[cs], sinT[cs]);
    }
}

static int grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    return (int)(g < 1 ? 1 : (g > 16384 ? 16384 : g));
}

int launch_rope_rows(hipStream_t s, const float* x, float* y, int rows, int heads, int hd, int start_pos,
                     const float* cosT, const float* sinT, int neox) {
    const int64_t n = (int64_t)rows * (hd / 2);
    if (n == 0) return GORCH_HIP_OK;
    hipLaunchKernelGGL(k_rope_rows, dim3(grid_for(n)), dim3(256), 0, s, x, y, (int64_t)rows, heads, hd / 2, start_pos,
                       cosT, sinT, neox);
    count(CNT_ELEMENTWISE);
    return check_launch("rope_rows");
}

}  // namespace gh

using namespace gh;

extern "C" int gorch_hip_rope_tables(void* stream, int head_dim, int max_seq, float base, float* cos_t, float* sin_t) {
    GH_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "gorch/nn: RoPE requires even headDim");
    GH_REQUIRE(max_seq > 0 && cos_t && sin_t, "gorch_hip_rope_tables: bad arguments");
    const int64_t n = (int64_t)max_seq * (head_dim / 2);
    hipLaunchKernelGGL(k_rope_tables, dim3(grid_for(n)), dim3(256), 0, stream_of(stream), head_dim, max_seq, base,
                       cos_t, sin_t);
    count(CNT_ELEMENTWISE);
    return check_launch("rope_tables");
}

extern "C" int gorch_hip_rope_apply(void* stream, const float* x, float* y, int outer, int seq_len, int head_dim,
                                    int start_pos, const float* cos_t, const float* sin_t, int max_seq, int neox,
                                    float sign) {
    GH_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "gorch/nn: RoPE requires even headDim");
    GH_REQUIRE(outer >= 0 && seq_len >= 0 && start_pos >= 0, "gorch_hip_rope_apply: bad shape");
    GH_REQUIRE(start_pos + seq_len <= max_seq, "gorch/nn: RoPE startPos+seqLen exceeds MaxSeq");
    const int64_t n = (int64_t)outer * seq_len * (head_dim / 2);
    if (n == 0) return GORCH_HIP_OK;
    GH_REQUIRE(x && y && cos_t && sin_t, "gorch_hip_rope_apply: null pointer");
    hipLaunchKernelGGL(k_rope_apply, dim3(grid_for(n)), dim3(256), 0, stream_of(stream), x, y,
                       (int64_t)outer * seq_len, seq_len, head_dim / 2, start_pos, cos_t, sin_t, neox, sign);
    count(CNT_ELEMENTWISE);
    return check_launch("rope_apply");
}
