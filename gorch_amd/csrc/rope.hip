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

// The GQA q/k epilogue in one launch (nn/gqa.go:300-330 order: per-head
// RMSNorm, then RoPE at the row's absolute position): one wave per row of hd
// floats (hd % 4 == 0, hd <= 256; lane l holds elements 4l .. 4l + 3), every
// load first; with gains, y = x * inv * g (inv from the f64 sum of squares,
// as k_rmsnorm_rows), then each pair rotated with rotate_pair's unfused
// operations, the Llama partner element fetched from lane l +- hd / 8. Row r
// is token r / heads. In place is fine: a lane writes only its own elements,
// after every value it needs is in registers.
// A second segment of rows (x2, y2, heads2, g2) follows the first rows
// rows: the q and k heads of one projection in one launch.
__global__ __launch_bounds__(256) void k_norm_rope_rows(const float* x, float* y, int rows, int heads, int hd,
                                                        const float* __restrict__ g, float eps, int start_pos,
                                                        const float* __restrict__ cosT,
                                                        const float* __restrict__ sinT, int neox,
                                                        const float* x2 = nullptr, float* y2 = nullptr,
                                                        int rows2 = 0, int heads2 = 1,
                                                        const float* __restrict__ g2 = nullptr,
                                                        const int* __restrict__ pos_dev = nullptr,
                                                        long long y2_pos_stride = 0) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    int r = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (r >= rows + rows2) return;
    // pos_dev: the start position read on the device (a captured decode
    // step); the second segment's output (the K cache rows) then starts at
    // y2 + start_pos * y2_pos_stride
    if (pos_dev) start_pos = *pos_dev;
    if (r >= rows) {  // wave-uniform: a wave is one row
        r -= rows;
        x = x2;
        y = y2 + (pos_dev ? (long long)start_pos * y2_pos_stride : 0);
        heads = heads2;
        g = g2;
    }
    const int half = hd / 2, nl = hd / 4;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (size_t)r * hd, (long long)hd * 4);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(g, g ? (long long)hd * 4 : 0);
    float4 v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, 16 * lane, 0, 0));
    const float4 gv = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rg, 16 * lane, 0, 0));
    const int p = start_pos + r / heads;
    // this lane's cos / sin, requested with the row (before the norm's
    // reduction): raw buffer loads, so no load waits on another
    const bool lo = lane < nl / 2;
    float co[4], sn[4];
    {
        const long long tb = (long long)(p + 1) * half * 4;
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(cosT, tb), rs = make_rsrc(sinT, tb);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            int cs;
            if (neox) {
                cs = p * half + min(2 * lane + q / 2, half - 1);  // pair q / 2 of the lane
            } else {
                const int k = 4 * lane + q;
                const int i = lo ? k : k - half;
                cs = p * half + min(max(i, 0), half - 1);
            }
            co[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rc, cs * 4, 0, 0));
            sn[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, cs * 4, 0, 0));
        }
    }
    if (g) {
        double s = ((double)v.x * (double)v.x + (double)v.y * (double)v.y) +
                   ((double)v.z * (double)v.z + (double)v.w * (double)v.w);
        s = wave_sum_d(s);
        const float inv = (float)rsqrt_f64(div_rcp(s, (double)hd, 1.0 / hd) + (double)eps);
        v = make_float4(v.x * inv * gv.x, v.y * inv * gv.y, v.z * inv * gv.z, v.w * inv * gv.w);
    }
    float o[4];
    const float e[4] = {v.x, v.y, v.z, v.w};
    if (neox) {
        // pairs (2i, 2i + 1) inside the lane's four elements, i = 2l, 2l + 1
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const float c = co[2 * q], si = sn[2 * q];
            o[2 * q] = e[2 * q] * c - e[2 * q + 1] * si;
            o[2 * q + 1] = e[2 * q] * si + e[2 * q + 1] * c;
        }
    } else {
        // Llama pairs (i, i + half): the partner sits hd / 8 lanes away
        const int src = lo ? lane + nl / 2 : lane - nl / 2;
        float pe[4];
#pragma unroll
        for (int q = 0; q < 4; q++) pe[q] = __shfl(e[q], src);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float c = co[q], si = sn[q];
            o[q] = lo ? e[q] * c - pe[q] * si : pe[q] * si + e[q] * c;
        }
    }
    if (lane < nl) *reinterpret_cast<float4*>(y + (size_t)r * hd + 4 * lane) = make_float4(o[0], o[1], o[2], o[3]);
}

int launch_norm_rope_rows(hipStream_t s, const float* x, float* y, int rows, int heads, int hd, const float* g,
                          float eps, int start_pos, const float* cosT, const float* sinT, int neox) {
    if (rows == 0) return GORCH_HIP_OK;
    hipLaunchKernelGGL(k_norm_rope_rows, dim3((rows + 3) / 4), dim3(256), 0, s, x, y, rows, heads, hd, g, eps,
                       start_pos, cosT, sinT, neox);
    count(CNT_ELEMENTWISE);
    return check_launch("norm_rope_rows");
}

static int grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    return (int)(g < 1 ? 1 : (g > 16384 ? 16384 : g));
}

int launch_norm_rope_rows2(hipStream_t s, const float* xq, float* yq, int rows_q, int heads_q, const float* gq,
                           const float* xk, float* yk, int rows_k, int heads_k, const float* gk, int hd, float eps,
                           int start_pos, const float* cosT, const float* sinT, int neox, const int* pos_dev,
                           long long yk_pos_stride) {
    if (rows_q + rows_k == 0) return GORCH_HIP_OK;
    hipLaunchKernelGGL(k_norm_rope_rows, dim3((rows_q + rows_k + 3) / 4), dim3(256), 0, s, xq, yq, rows_q, heads_q,
                       hd, gq, eps, start_pos, cosT, sinT, neox, xk, yk, rows_k, heads_k, gk, pos_dev, yk_pos_stride);
    count(CNT_ELEMENTWISE);
    return check_launch("norm_rope_rows2");
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
    return finish(stream, check_launch("rope_tables"));
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
    return finish(stream, check_launch("rope_apply"));
}
