// norm.hip — LayerNorm (nn/layernorm.go:31-91) and RMSNorm
// (nn/rmsnorm.go:39-81; MSL rmsnorm_forward, metal/kernels.go:152-190).
//
// One 256-thread block per row. Statistics accumulate in f64 exactly as the
// reference's CPU loops do (mean and variance for LayerNorm, sum of squares
// for RMSNorm); the row stays in L1/L2 between the two passes. The inverse
// is rounded to f32 and the output computed in f32 in the reference's
// operand order.
#include "common.h"

namespace gh {

__device__ double block_sum_d(double v, double* sh) {
    v = wave_sum_d(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    double t = 0.0;
    const int nw = blockDim.x >> 6;
    for (int w = 0; w < nw; w++) t += sh[w];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(256) void k_layernorm(const float* __restrict__ x, const float* __restrict__ g,
                                                   const float* __restrict__ b, float* __restrict__ y, int N,
                                                   float eps, long long in_stride) {
    __shared__ double sh[4];
    const float* row = x + (size_t)blockIdx.x * in_stride;
    float* out = y + (size_t)blockIdx.x * N;
    double s = 0.0;
    for (int j = threadIdx.x; j < N; j += blockDim.x) s += (double)row[j];
    const double rn = 1.0 / N;
    const double mean = div_rcp(block_sum_d(s, sh), (double)N, rn);
    double v = 0.0;
    for (int j = threadIdx.x; j < N; j += blockDim.x) {
        double d = (double)row[j] - mean;
        v += d * d;
    }
    const double var = div_rcp(block_sum_d(v, sh), (double)N, rn);
    const float inv = (float)rsqrt_f64(var + (double)eps);
    const float fm = (float)mean;
    for (int j = threadIdx.x; j < N; j += blockDim.x) {
        float normalized = (row[j] - fm) * inv;
        out[j] = normalized * g[j] + b[j];
    }
}

// (also used in place by the GQA qk-norm: each thread rewrites only the
// elements it read after the row's sum is complete)
__global__ __launch_bounds__(256) void k_rmsnorm(const float* x, const float* __restrict__ g, float* y, int N,
                                                 float eps) {
    __shared__ double sh[4];
    const float* row = x + (size_t)blockIdx.x * N;
    float* out = y + (size_t)blockIdx.x * N;
    double s = 0.0;
    for (int j = threadIdx.x; j < N; j += blockDim.x) s += (double)row[j] * (double)row[j];
    const double ss = block_sum_d(s, sh);
    const float inv = (float)rsqrt_f64(div_rcp(ss, (double)N, 1.0 / N) + (double)eps);
    for (int j = threadIdx.x; j < N; j += blockDim.x) out[j] = row[j] * inv * g[j];
}

// One wave per row for rows of at most 256 * R floats (N % 4 == 0): every
// load of the row and the gains is issued first (raw buffer loads, columns
// past N read as zeros), the f64 sum of squares is reduced on DPP with no
// barrier, and the outputs are written after every load has been used (a
// load issued after a store would make its use wait for the store). In place
// is fine: a lane rewrites only the elements it read. Four rows per block.
// With b (the fused residual add of a decoder block): the row is x + b,
// written to sum before the normalised row goes to y.
template <int R>
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float* x, const float* __restrict__ g, float* y, int M,
                                                      int N, float eps, const float* b = nullptr,
                                                      float* sum = nullptr) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (size_t)m * N, (long long)N * 4);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(g, (long long)N * 4);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(b ? b + (size_t)m * N : nullptr, b ? (long long)N * 4 : 0);
    float4 v[R], gv[R], bv[R];
#pragma unroll
    for (int c = 0; c < R; c++) {
        const int off = (4 * (lane + 64 * c)) * 4;
        v[c] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
        gv[c] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0));
        bv[c] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
    }
    if (b) {
#pragma unroll
        for (int c = 0; c < R; c++)
            v[c] = make_float4(v[c].x + bv[c].x, v[c].y + bv[c].y, v[c].z + bv[c].z, v[c].w + bv[c].w);
    }
    double s = 0.0;
#pragma unroll
    for (int c = 0; c < R; c++)
        s += ((double)v[c].x * (double)v[c].x + (double)v[c].y * (double)v[c].y) +
             ((double)v[c].z * (double)v[c].z + (double)v[c].w * (double)v[c].w);
    s = wave_sum_d(s);
    const float inv = (float)rsqrt_f64(div_rcp(s, (double)N, 1.0 / N) + (double)eps);
    float* out = y + (size_t)m * N;
#pragma unroll
    for (int c = 0; c < R; c++) {
        const int j = 4 * (lane + 64 * c);
        if (b && j < N) *reinterpret_cast<float4*>(sum + (size_t)m * N + j) = v[c];
        if (j < N)
            *reinterpret_cast<float4*>(out + j) =
                make_float4(v[c].x * inv * gv[c].x, v[c].y * inv * gv[c].y, v[c].z * inv * gv[c].z,
                            v[c].w * inv * gv[c].w);
    }
}

// One block per row: x[m] += bias + sum_s part[s][m] (slices in order, the
// residual add of a K-split Linear), then the row's LayerNorm statistics in
// f64 (nn/layernorm.go:61-91) and, given gamma/beta, the normalised row h.
// Each thread owns up to kRedVec groups of 4 consecutive columns and issues
// all of their 16-byte loads (row, S <= kRedSlices slices, bias, gamma,
// beta) before adding, so the row costs one memory round trip. N % 4 == 0.
constexpr int kRedVec = kReduceRowsMaxCols / 4 / 256, kRedSlices = 8;

template <int RS>
__global__ __launch_bounds__(256) void k_reduce_rows(const float* __restrict__ part, int S,
                                                     const float* __restrict__ bias, float* __restrict__ x, int M,
                                                     int N, float eps, float2* __restrict__ stats,
                                                     const float* __restrict__ ln_g, const float* __restrict__ ln_b,
                                                     float* __restrict__ h, uint16_t* __restrict__ hf) {
    __shared__ double2 sh2[4];
    const int m = blockIdx.x;
    float* row = x + (size_t)m * N;
    // raw buffer loads, all issued before any add and with no branch around
    // them: columns past N, slices past S and a missing bias read as zeros
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(row, (long long)N * 4);
    // slice q of row m sits at part + (q * M + m) * N; the resource spans
    // slice 0's row through slice S - 1's row (empty when S == 0)
    const long long pspan = S > 0 ? ((long long)(S - 1) * M + 1) * N * 4 : 0;
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part + (S > 0 ? (size_t)m * N : 0), pspan);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bias, bias ? (long long)N * 4 : 0);
    const bool norm = h || hf;
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(ln_g, norm ? (long long)N * 4 : 0);
    const __amdgpu_buffer_rsrc_t rbe = make_rsrc(ln_b, norm ? (long long)N * 4 : 0);
    float4 v[kRedVec], bv[kRedVec], gv[kRedVec], be[kRedVec];
    float4 p[kRedVec][RS];
    auto ld = [](__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    };
    // the moments' shift: column 0 of the updated row (its old value plus
    // bias and slices), the same for every thread
    const float x0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, 0, 0, 0));
    const float b0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, 0, 0, 0));
    float p0[RS];
#pragma unroll
    for (int q = 0; q < RS; q++)
        p0[q] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rp, q < S ? (int)((size_t)q * M * N * 4) : kOutOfRange, 0, 0));
#pragma unroll
    for (int c = 0; c < kRedVec; c++) {
        const int j = 4 * (threadIdx.x + 256 * c);
        const int off = j < N ? j * 4 : kOutOfRange;
        v[c] = ld(rx, off);
        bv[c] = ld(rb, off);
        gv[c] = ld(rg, off);
        be[c] = ld(rbe, off);
#pragma unroll
        for (int q = 0; q < RS; q++)
            p[c][q] = ld(rp, (j < N && q < S) ? (int)(((size_t)q * M * N + j) * 4) : kOutOfRange);
    }
    float shift = x0;
    if (S > 0) {
        float acc = p0[0];
#pragma unroll
        for (int q = 1; q < RS; q++)
            if (q < S) acc += p0[q];
        if (bias) acc = acc + b0;
        shift = x0 + acc;
    }
    // shifted one-pass moments in f64 (one block reduction): mean = shift +
    // s1 / N, var = s2 / N - (s1 / N)^2, the two-pass values to f64
    // rounding for rows whose mean is not many orders above their spread
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int c = 0; c < kRedVec; c++) {
        const int j = 4 * (threadIdx.x + 256 * c);
        if (j >= N) continue;
        float* vc = reinterpret_cast<float*>(&v[c]);
        if (S > 0) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float acc = reinterpret_cast<const float*>(&p[c][0])[e];
#pragma unroll
                for (int q = 1; q < RS; q++)
                    if (q < S) acc += reinterpret_cast<const float*>(&p[c][q])[e];
                if (bias) acc = acc + reinterpret_cast<const float*>(&bv[c])[e];
                vc[e] = vc[e] + acc;
            }
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const double d = (double)vc[e] - (double)shift;
            s1 += d;
            s2 += d * d;
        }
    }
    if (stats || norm) {
        wave_sum2_d(s1, s2);
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        if (lane == 0) sh2[wave] = make_double2(s1, s2);
        __syncthreads();
        s1 = (sh2[0].x + sh2[1].x) + (sh2[2].x + sh2[3].x);
        s2 = (sh2[0].y + sh2[1].y) + (sh2[2].y + sh2[3].y);
    }
    // the updated row's stores after every load has been used
    if (S > 0) {
#pragma unroll
        for (int c = 0; c < kRedVec; c++) {
            const int j = 4 * (threadIdx.x + 256 * c);
            if (j < N) *reinterpret_cast<float4*>(row + j) = v[c];
        }
    }
    if (!stats && !norm) return;
    const double rn = 1.0 / N;
    const double d1 = div_rcp(s1, (double)N, rn);
    const double mean = (double)shift + d1;
    const double var = fmax(div_rcp(s2, (double)N, rn) - d1 * d1, 0.0);
    const float fm = (float)mean, inv = (float)rsqrt_f64(var + (double)eps);
    if (stats && threadIdx.x == 0) stats[m] = make_float2(fm, inv);
    if (!norm) return;
    // the same f32 operations as a LayerNorm fused into a GEMV's operand load
#pragma unroll
    for (int c = 0; c < kRedVec; c++) {
        const int j = 4 * (threadIdx.x + 256 * c);
        if (j >= N) continue;
        const float* vc = reinterpret_cast<const float*>(&v[c]);
        const float* gc = reinterpret_cast<const float*>(&gv[c]);
        const float* bc = reinterpret_cast<const float*>(&be[c]);
        float4 o;
        float* oc = reinterpret_cast<float*>(&o);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float normalized = (vc[e] - fm) * inv;
            oc[e] = normalized * gc[e] + bc[e];
        }
        if (hf) {
            // columns j .. j + 3 share one lane's 8-element group: 8-byte
            // hi and lo stores
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; e++) split_hi_lo1(oc[e], hi[e], lo[e]);
            const size_t i = xfrag_index(m, j);
            *reinterpret_cast<uint2*>(hf + i) =
                make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
            *reinterpret_cast<uint2*>(hf + i + 512) =
                make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
        } else {
            *reinterpret_cast<float4*>(h + (size_t)m * N + j) = o;
        }
    }
}

int launch_reduce_rows(hipStream_t s, const float* part, int S, const float* bias, float* x, int M, int N,
                       float eps, float2* stats, const float* ln_g, const float* ln_b, float* h, uint16_t* hf) {
    if (M == 0) return GORCH_HIP_OK;
    if (hf && (h || M > 16)) {
        set_error("reduce_rows: a fragment-layout output takes at most 16 rows and no row-major h");
        return GORCH_HIP_EINVAL;
    }
    if (N > 1024 * kRedVec || S > kRedSlices || N % 4) {
        set_error("reduce_rows: at most 2048 columns (a multiple of 4) and 8 slices");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if ((h || hf) && (!ln_g || !ln_b)) {
        set_error("reduce_rows: the normalised output needs gamma and beta");
        return GORCH_HIP_EINVAL;
    }
    // slice registers sized to S (loads of absent slices still cost their
    // instructions)
    if (S <= 2)
        hipLaunchKernelGGL(k_reduce_rows<2>, dim3(M), dim3(256), 0, s, part, S, bias, x, M, N, eps, stats, ln_g, ln_b, h, hf);
    else if (S <= 4)
        hipLaunchKernelGGL(k_reduce_rows<4>, dim3(M), dim3(256), 0, s, part, S, bias, x, M, N, eps, stats, ln_g, ln_b, h, hf);
    else
        hipLaunchKernelGGL(k_reduce_rows<kRedSlices>, dim3(M), dim3(256), 0, s, part, S, bias, x, M, N, eps, stats,
                           ln_g, ln_b, h, hf);
    count(CNT_NORM);
    return check_launch("reduce_rows");
}

// Row i of the input starts at x + i * in_stride (in_stride = N for a dense
// matrix); the output is dense [M, N].
int launch_layernorm(hipStream_t s, const float* x, const float* g, const float* b, float* y, int M, int N,
                     float eps, long long in_stride) {
    if (M == 0) return GORCH_HIP_OK;
    hipLaunchKernelGGL(k_layernorm, dim3(M), dim3(256), 0, s, x, g, b, y, N, eps, in_stride);
    count(CNT_NORM);
    return check_launch("layernorm");
}

int launch_rmsnorm(hipStream_t s, const float* x, const float* g, float* y, int M, int N, float eps) {
    if (M == 0) return GORCH_HIP_OK;
    const bool aligned = N % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16) == 0;
    if (aligned && N <= 2048) {
        const dim3 grid((M + 3) / 4);
        if (N <= 256) hipLaunchKernelGGL(k_rmsnorm_rows<1>, grid, dim3(256), 0, s, x, g, y, M, N, eps);
        else if (N <= 512) hipLaunchKernelGGL(k_rmsnorm_rows<2>, grid, dim3(256), 0, s, x, g, y, M, N, eps);
        else if (N <= 1024) hipLaunchKernelGGL(k_rmsnorm_rows<4>, grid, dim3(256), 0, s, x, g, y, M, N, eps);
        else hipLaunchKernelGGL(k_rmsnorm_rows<8>, grid, dim3(256), 0, s, x, g, y, M, N, eps);
        count(CNT_NORM);
        return check_launch("rmsnorm");
    }
    hipLaunchKernelGGL(k_rmsnorm, dim3(M), dim3(256), 0, s, x, g, y, N, eps);
    count(CNT_NORM);
    return check_launch("rmsnorm");
}

}  // namespace gh

using namespace gh;

extern "C" int gorch_hip_layernorm(void* stream, const float* x, const float* gamma, const float* beta,
                                   float* y, int M, int N, float eps) {
    GH_REQUIRE(M >= 0 && N > 0, "gorch_hip_layernorm: bad shape");
    if (M == 0) return GORCH_HIP_OK;
    GH_REQUIRE(x && gamma && beta && y, "gorch_hip_layernorm: null pointer");
    return finish(stream, launch_layernorm(stream_of(stream), x, gamma, beta, y, M, N, eps, N));
}

extern "C" int gorch_hip_add_rmsnorm(void* stream, const float* x, const float* b, const float* gamma, float* sum,
                                     float* y, int M, int N, float eps) {
    GH_REQUIRE(M >= 0 && N > 0, "gorch_hip_add_rmsnorm: bad shape");
    if (M == 0) return GORCH_HIP_OK;
    GH_REQUIRE(x && b && gamma && sum && y, "gorch_hip_add_rmsnorm: null pointer");
    GH_REQUIRE(N % 4 == 0 && N <= 2048 &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(b) |
                     reinterpret_cast<uintptr_t>(sum) | reinterpret_cast<uintptr_t>(y)) % 16) == 0,
               "gorch_hip_add_rmsnorm: needs N % 4 == 0, N <= 2048 and 16-byte aligned rows");
    hipStream_t s = stream_of(stream);
    const dim3 grid((M + 3) / 4);
    if (N <= 256) hipLaunchKernelGGL(k_rmsnorm_rows<1>, grid, dim3(256), 0, s, x, gamma, y, M, N, eps, b, sum);
    else if (N <= 512) hipLaunchKernelGGL(k_rmsnorm_rows<2>, grid, dim3(256), 0, s, x, gamma, y, M, N, eps, b, sum);
    else if (N <= 1024) hipLaunchKernelGGL(k_rmsnorm_rows<4>, grid, dim3(256), 0, s, x, gamma, y, M, N, eps, b, sum);
    else hipLaunchKernelGGL(k_rmsnorm_rows<8>, grid, dim3(256), 0, s, x, gamma, y, M, N, eps, b, sum);
    count(CNT_NORM);
    return finish(stream, check_launch("add_rmsnorm"));
}

extern "C" int gorch_hip_rmsnorm(void* stream, const float* x, const float* gamma, float* y, int M, int N,
                                 float eps) {
    GH_REQUIRE(M >= 0 && N > 0, "gorch_hip_rmsnorm: bad shape");
    if (M == 0) return GORCH_HIP_OK;
    GH_REQUIRE(x && gamma && y, "gorch_hip_rmsnorm: null pointer");
    return finish(stream, launch_rmsnorm(stream_of(stream), x, gamma, y, M, N, eps));
}
