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
// Grid: blockIdx.x = group of NT 16-row weight tiles,
// blockIdx.y = group of 16 activation rows (M > 16 re-reads W per group).
// A block is NW waves, each owning a contiguous K slice; the NW partial
// 16x16 tiles are summed in LDS in wave order (deterministic). K is never
// split across blocks: on gfx950 the agent-scope fence a cross-block
// reduction needs writes back the L2 and costs tens of microseconds, while
// a 16-wave block over a narrow N still keeps enough loads in flight.
#include "common.h"

namespace gh {

// NW waves per block split K; NT 16-row weight tiles per block; U k-steps
// of loads issued per wave before their MFMAs.
template <int NT, int NW, int U>
__global__ __launch_bounds__(NW * 64) void k_linear_bf16_mfma(
    const float* __restrict__ x, const uint16_t* __restrict__ W, const float* __restrict__ bias,
    const float* residual, OutDesc od, int M, int N, int K, int kw, int epilogue, LinearExtras ex) {
    __shared__ floatx4 red[NW][NT][64];
    __shared__ float s_mean[16], s_inv[16];
    __shared__ unsigned long long s_key[16];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;  // A: activation row; B: weight row within tile
    const int g = lane >> 4;  // k-chunk group within a 32-wide k-step
    const int n0 = blockIdx.x * (16 * NT);
    const int m0 = blockIdx.y * 16;
    const int mrow = m0 + r;
    const int kb = wave * kw;
    const int ke = min(kb + kw, K);

    const long long xs = ex.x_stride ? ex.x_stride : K;
    const bool arow_ok = mrow < M;
    const float* xrow = x + (size_t)(arow_ok ? mrow : 0) * xs;

    const uint16_t* wrow[NT];
    bool wrow_ok[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        int n = n0 + 16 * t + r;
        wrow_ok[t] = n < N;
        wrow[t] = W + (size_t)(wrow_ok[t] ? n : 0) * K;
    }

    if (ex.ln_g) {
        // LayerNorm prologue (nn/layernorm.go:61-91): per-row mean and
        // variance in f64 over the whole K, computed by each block for its
        // (at most 16) rows; the A operand is normalised as it is loaded.
        for (int rr = wave; rr < 16; rr += NW) {
            const int m = m0 + rr;
            if (m >= M) break;
            const float* row = x + (size_t)m * xs;
            double s1 = 0.0;
            for (int k = 4 * lane; k < K; k += 256) {
                float4 v = *reinterpret_cast<const float4*>(row + k);
                s1 += (double)v.x + (double)v.y + (double)v.z + (double)v.w;
            }
            const double mean = wave_sum_d(s1) / (double)K;
            double s2 = 0.0;
            for (int k = 4 * lane; k < K; k += 256) {
                float4 v = *reinterpret_cast<const float4*>(row + k);
                double d0 = (double)v.x - mean, d1 = (double)v.y - mean, d2 = (double)v.z - mean,
                       d3 = (double)v.w - mean;
                s2 += d0 * d0 + d1 * d1 + d2 * d2 + d3 * d3;
            }
            const double var = wave_sum_d(s2) / (double)K;
            if (lane == 0) {
                s_mean[rr] = (float)mean;
                s_inv[rr] = (float)(1.0 / sqrt(var + (double)ex.ln_eps));
            }
        }
        __syncthreads();
    }
    const float ln_mean = ex.ln_g ? s_mean[r] : 0.f;
    const float ln_inv = ex.ln_g ? s_inv[r] : 1.f;

    floatx4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

    // U k-steps per iteration: all weight loads of the group are issued
    // before any MFMA so several 16-byte loads per lane are in flight.
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
                if (ex.ln_g) {
                    float4 g0 = *reinterpret_cast<const float4*>(ex.ln_g + kc);
                    float4 g1 = *reinterpret_cast<const float4*>(ex.ln_g + kc + 4);
                    float4 b0 = *reinterpret_cast<const float4*>(ex.ln_b + kc);
                    float4 b1 = *reinterpret_cast<const float4*>(ex.ln_b + kc + 4);
                    const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
                    const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        float normalized = (f[u][i] - ln_mean) * ln_inv;
                        f[u][i] = normalized * gg[i] + bb[i];
                    }
                }
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

    if (ex.argmax_key && threadIdx.x < 16) s_key[threadIdx.x] = 0ull;
    if (ex.argmax_key) __syncthreads();

    // Output element o = (tile t, lane e, slot v): row m0 + 4*(e/16) + v,
    // column n0 + 16*t + e%16. Partials are summed in wave order.
    for (int o = threadIdx.x; o < NT * 256; o += NW * 64) {
        const int t = o >> 8, e = o & 63, v = (o >> 6) & 3;
        const int om = m0 + 4 * (e >> 4) + v;
        const int on = n0 + 16 * t + (e & 15);
        if (om < M && on < N) {
            float s = red[0][t][e][v];
#pragma unroll
            for (int w = 1; w < NW; w++) s += red[w][t][e][v];
            if (bias) s = s + bias[on];
            if (epilogue == GORCH_HIP_EPI_GELU) s = gelu_tanh(s);
            if (residual) s = residual[(size_t)om * N + on] + s;
            *od.at(om, on) = s;
            if (ex.argmax_key) atomicMax(&s_key[om - m0], argmax_pack(s, on));
        }
    }
    if (ex.argmax_key) {
        __syncthreads();
        if (threadIdx.x < 16 && m0 + (int)threadIdx.x < M)
            atomicMax(&ex.argmax_key[m0 + threadIdx.x], s_key[threadIdx.x]);
    }
}

static int env_int(const char* name, int dflt) {
    const char* s = getenv(name);
    return s ? atoi(s) : dflt;
}

// Launch plan: NT weight tiles and NW K-splitting waves per block, chosen
// from a sweep of the decode shapes (GPT-2 small and XL, M = 1..16) on
// MI355X. GORCH_HIP_GEMV_NT / GORCH_HIP_GEMV_NW override them.
struct GemvPlan {
    int nt, nw, u;
};

static GemvPlan plan_gemv(int M, int N, int K) {
    static const int nt_env = env_int("GORCH_HIP_GEMV_NT", 0);
    static const int nw_env = env_int("GORCH_HIP_GEMV_NW", 0);
    static const int u_env = env_int("GORCH_HIP_GEMV_U", 0);
    const int ntiles = (N + 15) / 16;
    GemvPlan p;
    if (ntiles >= 2048) {          // LM-head class: many tiles
        p.nt = 2;
        if (M == 1 && K < 1024) {
            p.nw = 4;
            p.u = 8;
        } else {
            p.nw = 1;
            p.u = 2;
        }
    } else if (ntiles >= 256) {    // FFN-up / fused-QKV class
        p.nt = N >= 4096 ? 2 : 1;
        p.nw = 8;
        p.u = 2;
    } else {                       // narrow N: deep K split inside the block
        p.nt = 1;
        p.nw = 8;
        p.u = M == 1 ? 4 : 2;
    }
    // keep at least one 32-wide k-step per wave
    while (p.nw > 1 && (K + p.nw - 1) / p.nw < 32) p.nw /= 2;
    if (nt_env) p.nt = nt_env;
    if (nw_env) p.nw = nw_env;
    if (u_env) p.u = u_env;
    return p;
}

template <int NT, int NW, int U>
static void launch_t(hipStream_t s, dim3 grid, const float* x, const uint16_t* W, const float* bias,
                     const float* residual, const OutDesc& od, int M, int N, int K, int kw, int epilogue,
                     const LinearExtras& ex) {
    hipLaunchKernelGGL((k_linear_bf16_mfma<NT, NW, U>), grid, dim3(NW * 64), 0, s, x, W, bias, residual, od,
                       M, N, K, kw, epilogue, ex);
}

int launch_linear_bf16(hipStream_t s, const float* x, const uint16_t* W, const float* bias,
                       const float* residual, float* y, int M, int N, int K, int epilogue) {
    return launch_linear_bf16_od(s, x, W, bias, residual, OutDesc::plain(y, N), M, N, K, epilogue,
                                 LinearExtras{});
}

int launch_gemm_bf16w(hipStream_t s, const float* A, const uint16_t* W, const float* bias,
                      const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                      bool act_bf16);

// M <= 16: the weight-streaming GEMV below; larger M: the tiled MFMA GEMM
// (gemm.hip), which re-reads each weight tile only once per BM rows.
int launch_linear_bf16_od(hipStream_t s, const float* x, const uint16_t* W, const float* bias,
                          const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                          const LinearExtras& ex) {
    if (M > 16) {
        if (ex.ln_g || ex.argmax_key) {
            set_error("linear_bf16: fused LayerNorm / argmax need M <= 16");
            return GORCH_HIP_EUNSUPPORTED;
        }
        return launch_gemm_bf16w(s, x, W, bias, residual, od, M, N, K, epilogue, false);
    }
    GemvPlan p = plan_gemv(M, N, K);
    int per = (K + p.nw - 1) / p.nw;
    int kw = (per + 31) / 32 * 32;
    dim3 grid((N + 16 * p.nt - 1) / (16 * p.nt), (M + 15) / 16);
#define GH_CASE(T, WV, UV)                                                                   \
    if (p.nt == T && p.nw == WV && p.u == UV) {                                              \
        launch_t<T, WV, UV>(s, grid, x, W, bias, residual, od, M, N, K, kw, epilogue, ex);   \
        count(M <= 16 ? CNT_GEMV : CNT_GEMM);                                                \
        return check_launch("linear_bf16");                                                  \
    }
#define GH_CASES_U(T, WV) GH_CASE(T, WV, 2) GH_CASE(T, WV, 4) GH_CASE(T, WV, 8)
#define GH_CASES_W(T) GH_CASES_U(T, 1) GH_CASES_U(T, 2) GH_CASES_U(T, 4) GH_CASES_U(T, 8) GH_CASES_U(T, 16)
    GH_CASES_W(1) GH_CASES_W(2) GH_CASES_W(4)
#undef GH_CASES_W
#undef GH_CASES_U
#undef GH_CASE
    set_error("linear_bf16: unsupported tile plan");
    return GORCH_HIP_EUNSUPPORTED;
}

}  // namespace gh
