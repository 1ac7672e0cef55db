// gemv.hip — BF16-weight Linear for decode-sized M (the kernel behind
// nn.Linear.Forward's bf16 branch, nn/module.go:61-88, and the GPT LM head).
//
//   y[m,n] = residual[m,n] + epi( sum_k x[m,k] * W[n,k] + bias[n] )
//
// Design (gfx950): the weight W [N,K] bf16 is streamed from HBM exactly
// once with 16-byte loads; this is the whole cost of the op for M <= 16.
// The reduction over K runs on the matrix cores: one
// v_mfma_f32_16x16x32_bf16 consumes a 16(n) x 32(k) weight tile whose
// B-operand layout (lane l: row n = l%16, k-chunk 8*(l/16)..+8) is exactly
// a 16-byte load from row-major W. The f32 activations become the A operand
// through an exact-enough split x = hi + lo (two bf16 MFMAs), so products
// keep ~2^-16 relative accuracy with f32 accumulation — the reference widens
// the bf16 weight and runs an f32 sgemm (bf16_matmul.go:166-173).
//
// Grid: blockIdx.x = group of NT 16-row weight tiles, blockIdx.y = K split,
// blockIdx.z = group of 16 activation rows (M > 16 re-reads W per group).
// A block is 4 waves, each owning a contiguous K slice; the 4 partial
// 16x16 tiles are summed in LDS in wave order. With more than one K split,
// blocks write partials to the library workspace and the last block to
// arrive (per output tile) sums them in split order — deterministic, one
// launch, counters left at zero for the next call.
#include "common.h"

namespace gh {

constexpr int kWaves = 4;

template <int NT>
__global__ __launch_bounds__(256) void k_linear_bf16_mfma(
    const float* __restrict__ x, const uint16_t* __restrict__ W, const float* __restrict__ bias,
    const float* residual, float* y, int M, int N, int K, int kw, int ksplit, int epilogue,
    float* __restrict__ partial, unsigned* __restrict__ counters) {
    __shared__ floatx4 red[kWaves][NT][64];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;  // A: activation row; B: weight row within tile
    const int g = lane >> 4;  // k-chunk group within a 32-wide k-step
    const int n0 = blockIdx.x * (16 * NT);
    const int m0 = blockIdx.z * 16;
    const int mrow = m0 + r;
    const int ks = blockIdx.y;
    const int kb = ks * kWaves * kw + wave * kw;
    const int ke = min(kb + kw, K);

    const bool arow_ok = mrow < M;
    const float* xrow = x + (size_t)(arow_ok ? mrow : 0) * K;

    const uint16_t* wrow[NT];
    bool wrow_ok[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        int n = n0 + 16 * t + r;
        wrow_ok[t] = n < N;
        wrow[t] = W + (size_t)(wrow_ok[t] ? n : 0) * K;
    }

    floatx4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

    // U k-steps per iteration: all weight loads of the group are issued
    // before any MFMA so several 16-byte loads per lane are in flight.
    constexpr int U = (NT >= 4) ? 2 : 4;
    for (int k0 = kb; k0 < ke; k0 += 32 * U) {
        uint4 wv[U][NT];
        float f[U][8];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int kc = k0 + 32 * u + 8 * g;
            const bool k_ok = kc < ke;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (k_ok && wrow_ok[t])
                    wv[u][t] = *reinterpret_cast<const uint4*>(wrow[t] + kc);
                else
                    wv[u][t] = make_uint4(0, 0, 0, 0);
            }
            if (k_ok && arow_ok) {
                float4 a0 = *reinterpret_cast<const float4*>(xrow + kc);
                float4 a1 = *reinterpret_cast<const float4*>(xrow + kc + 4);
                f[u][0] = a0.x; f[u][1] = a0.y; f[u][2] = a0.z; f[u][3] = a0.w;
                f[u][4] = a1.x; f[u][5] = a1.y; f[u][6] = a1.z; f[u][7] = a1.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) f[u][i] = 0.f;
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            bf16x8 hi, lo;
            split_hi_lo(f[u], hi, lo);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                bf16x8 b = __builtin_bit_cast(bf16x8, wv[u][t]);
                acc[t] = mfma16x16x32(hi, b, acc[t]);
                acc[t] = mfma16x16x32(lo, b, acc[t]);
            }
        }
    }

#pragma unroll
    for (int t = 0; t < NT; t++) red[wave][t][lane] = acc[t];
    __syncthreads();

    // Thread tid owns (tile t, lane e, slot v) for v = tid / 64: output row
    // m = m0 + 4*(e/16) + v, column n = n0 + 16*t + e%16.
    const int e = threadIdx.x & 63;
    const int v = threadIdx.x >> 6;
    const int om = m0 + 4 * (e >> 4) + v;
    float val[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        float s = red[0][t][e][v];
#pragma unroll
        for (int w = 1; w < kWaves; w++) s += red[w][t][e][v];
        val[t] = s;
    }

    if (ksplit > 1) {
        // Publish this split's partial tile, then elect the last arrival.
#pragma unroll
        for (int t = 0; t < NT; t++) {
            int on = n0 + 16 * t + (e & 15);
            if (om < M && on < N) partial[((size_t)ks * M + om) * N + on] = val[t];
        }
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned slot = blockIdx.z * gridDim.x + blockIdx.x;
            unsigned prev = atomicAdd(&counters[slot], 1u);
            s_last = (prev == (unsigned)(ksplit - 1));
            if (s_last) __hip_atomic_store(&counters[slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!s_last) return;
        __threadfence();
#pragma unroll
        for (int t = 0; t < NT; t++) {
            int on = n0 + 16 * t + (e & 15);
            float s = 0.f;
            if (om < M && on < N) {
                for (int q = 0; q < ksplit; q++)
                    s += __hip_atomic_load(&partial[((size_t)q * M + om) * N + on], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            }
            val[t] = s;
        }
    }

#pragma unroll
    for (int t = 0; t < NT; t++) {
        int on = n0 + 16 * t + (e & 15);
        if (om < M && on < N) {
            float o = val[t];
            if (bias) o = o + bias[on];
            if (epilogue == GORCH_HIP_EPI_GELU) o = gelu_tanh(o);
            size_t idx = (size_t)om * N + on;
            if (residual) o = residual[idx] + o;
            y[idx] = o;
        }
    }
}

// Launch plan for one call. Tunable from the environment for sweeps:
// GORCH_HIP_GEMV_NT (1|2|4), GORCH_HIP_GEMV_WAVES_TARGET.
struct GemvPlan {
    int nt, kw, ksplit, nblk, mblk;
};

static int env_int(const char* name, int dflt) {
    const char* s = getenv(name);
    return s ? atoi(s) : dflt;
}

static GemvPlan plan_gemv(int M, int N, int K) {
    static const int nt_env = env_int("GORCH_HIP_GEMV_NT", 0);
    static const int target = env_int("GORCH_HIP_GEMV_WAVES_TARGET", 2048);
    GemvPlan p;
    int ntiles = (N + 15) / 16;
    p.nt = nt_env ? nt_env : (ntiles >= 2048 ? 2 : 1);
    p.mblk = (M + 15) / 16;
    p.nblk = (ntiles + p.nt - 1) / p.nt;
    int waves = p.nblk * kWaves * p.mblk;
    int ksplit = 1;
    if (waves < target) ksplit = (target + waves - 1) / waves;
    // Each wave keeps at least two 32-wide k-steps.
    int max_split = K / (kWaves * 64);
    if (max_split < 1) max_split = 1;
    if (ksplit > max_split) ksplit = max_split;
    int per = (K + ksplit * kWaves - 1) / (ksplit * kWaves);
    p.kw = (per + 31) / 32 * 32;
    p.ksplit = (K + kWaves * p.kw - 1) / (kWaves * p.kw);
    return p;
}

int launch_linear_bf16(hipStream_t s, const float* x, const uint16_t* W, const float* bias,
                       const float* residual, float* y, int M, int N, int K, int epilogue) {
    GemvPlan p = plan_gemv(M, N, K);
    float* partial = nullptr;
    unsigned* counters = nullptr;
    if (p.ksplit > 1) {
        Workspace* ws;
        size_t need = (size_t)p.ksplit * M * N * sizeof(float);
        if (!workspace_reserve(need, (size_t)p.nblk * p.mblk, &ws)) return GORCH_HIP_ENOMEM;
        partial = ws->partial;
        counters = ws->counters;
    }
    dim3 grid(p.nblk, p.ksplit, p.mblk);
    switch (p.nt) {
        case 1:
            hipLaunchKernelGGL(k_linear_bf16_mfma<1>, grid, dim3(256), 0, s, x, W, bias, residual, y, M,
                               N, K, p.kw, p.ksplit, epilogue, partial, counters);
            break;
        case 2:
            hipLaunchKernelGGL(k_linear_bf16_mfma<2>, grid, dim3(256), 0, s, x, W, bias, residual, y, M,
                               N, K, p.kw, p.ksplit, epilogue, partial, counters);
            break;
        default:
            hipLaunchKernelGGL(k_linear_bf16_mfma<4>, grid, dim3(256), 0, s, x, W, bias, residual, y, M,
                               N, K, p.kw, p.ksplit, epilogue, partial, counters);
            break;
    }
    count(M <= 16 ? CNT_GEMV : CNT_GEMM);
    return check_launch("linear_bf16");
}

}  // namespace gh
