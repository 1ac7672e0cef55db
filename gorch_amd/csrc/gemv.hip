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
#include <algorithm>

#include "common.h"

namespace gh {

// NW waves per block split K; NT 16-row weight tiles per block; U k-steps
// per load group. Each wave walks its K range in groups of U k-steps with
// two register sets: group i + 1's loads (weights, activation rows and, with
// LN, gamma/beta) are in flight while group i feeds the matrix cores. All
// loads are raw buffer loads without branches: rows past M or N and k past
// the wave's range read as zeros (a load under a branch would make the
// compiler wait for every outstanding load before each use).
template <int NT, int NW, int U, bool LN>
__global__ __launch_bounds__(NW * 64) void k_linear_bf16_mfma(
    const float* __restrict__ x, const uint16_t* __restrict__ W, const float* __restrict__ bias,
    const float* residual, OutDesc od, int M, int N, int K, int kw, int epilogue, LinearExtras ex) {
    __shared__ floatx4 red[NW][NT][64];
    __shared__ float s_mean[16], s_inv[16];
    __shared__ unsigned long long s_key[16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;  // A: activation row; B: weight row within tile
    const int g = lane >> 4;  // k-chunk group within a 32-wide k-step
    const int n0 = blockIdx.x * (16 * NT);
    // partial mode: blockIdx.y is the K slice (M <= 16), else the row group
    const int m0 = ex.part ? 0 : blockIdx.y * 16;
    const int kbase = ex.part ? blockIdx.y * ex.kslice : 0;
    const int kend = ex.part ? min(K, kbase + ex.kslice) : K;
    const int kb = kbase + wave * kw;
    const int ke = min(kb + kw, kend);

    const long long xs = ex.x_stride ? ex.x_stride : K;
    const int mrows = max(0, min(16, M - m0));
    const __amdgpu_buffer_rsrc_t rsx = make_rsrc(x + (size_t)m0 * xs, (long long)mrows * xs * 4);
    __amdgpu_buffer_rsrc_t rsw[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int rows = max(0, min(16, N - n0 - 16 * t));
        rsw[t] = make_rsrc(W + (size_t)(n0 + 16 * t) * K, (long long)rows * K * 2);
    }
    const __amdgpu_buffer_rsrc_t rsg = make_rsrc(ex.ln_g, LN ? (long long)K * 4 : 0);
    const __amdgpu_buffer_rsrc_t rsb = make_rsrc(ex.ln_b, LN ? (long long)K * 4 : 0);

    if (LN && ex.ln_stats) {
        if (threadIdx.x < 16 && m0 + (int)threadIdx.x < M) {
            const float2 st = ex.ln_stats[m0 + threadIdx.x];
            s_mean[threadIdx.x] = st.x;
            s_inv[threadIdx.x] = st.y;
        }
        __syncthreads();
    } else if (LN) {
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
            const double mean = div_rcp(wave_sum_d(s1), (double)K, 1.0 / K);
            double s2 = 0.0;
            for (int k = 4 * lane; k < K; k += 256) {
                float4 v = *reinterpret_cast<const float4*>(row + k);
                double d0 = (double)v.x - mean, d1 = (double)v.y - mean, d2 = (double)v.z - mean,
                       d3 = (double)v.w - mean;
                s2 += d0 * d0 + d1 * d1 + d2 * d2 + d3 * d3;
            }
            const double var = div_rcp(wave_sum_d(s2), (double)K, 1.0 / K);
            if (lane == 0) {
                s_mean[rr] = (float)mean;
                s_inv[rr] = (float)rsqrt_f64(var + (double)ex.ln_eps);
            }
        }
        __syncthreads();
    }
    const float ln_mean = LN ? s_mean[r] : 0.f;
    const float ln_inv = LN ? s_inv[r] : 1.f;

    floatx4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

    struct Group {
        u32x4 w[U][NT];
        u32x4 xa[U][2];
        u32x4 lg[LN ? U : 1][2], lb[LN ? U : 1][2];
    };
    auto load = [&](int k0, Group& gr) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int kc = k0 + 32 * u + 8 * g;
            const bool ok = kc < ke;
#pragma unroll
            for (int t = 0; t < NT; t++)
                gr.w[u][t] = __builtin_amdgcn_raw_buffer_load_b128(rsw[t], ok ? (r * K + kc) * 2 : kOutOfRange, 0, 0);
            const int xo = ok ? (int)((r * xs + kc) * 4) : kOutOfRange;
            gr.xa[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rsx, xo, 0, 0);
            gr.xa[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rsx, xo + 16, 0, 0);
            if constexpr (LN) {
                const int go = ok ? kc * 4 : kOutOfRange;
                gr.lg[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rsg, go, 0, 0);
                gr.lg[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rsg, go + 16, 0, 0);
                gr.lb[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rsb, go, 0, 0);
                gr.lb[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rsb, go + 16, 0, 0);
            }
        }
    };
    auto compute = [&](int k0, const Group& gr) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            float f[8];
#pragma unroll
            // element by value: __builtin_bit_cast on a vector-element
            // lvalue reads element 0 with this compiler
            for (int i = 0; i < 8; i++) f[i] = __uint_as_float(gr.xa[u][i >> 2][i & 3]);
            if constexpr (LN) {
                // k past the range: the normalised zero is masked so it can
                // never meet an infinite inverse deviation
                const bool ok = k0 + 32 * u + 8 * g < ke;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float gg = __uint_as_float(gr.lg[u][i >> 2][i & 3]);
                    const float bb = __uint_as_float(gr.lb[u][i >> 2][i & 3]);
                    const float normalized = (f[i] - ln_mean) * ln_inv;
                    f[i] = ok ? normalized * gg + bb : 0.f;
                }
            }
            bf16x8 hi, lo;
            split_hi_lo(f, hi, lo);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const bf16x8 b = __builtin_bit_cast(bf16x8, gr.w[u][t]);
                acc[t] = mfma16x16x32(hi, b, acc[t]);
                acc[t] = mfma16x16x32(lo, b, acc[t]);
            }
        }
    };
    const int nit = ke > kb ? (ke - kb + 32 * U - 1) / (32 * U) : 0;
    Group ga, gb;
    load(kb, ga);
    for (int i = 0; i < nit; i += 2) {
        load(kb + 32 * U * (i + 1), gb);
        compute(kb + 32 * U * i, ga);
        load(kb + 32 * U * (i + 2), ga);
        if (i + 1 < nit) compute(kb + 32 * U * (i + 1), gb);
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
            if (ex.part) {
                ex.part[((size_t)blockIdx.y * M + om) * N + on] = s;
                continue;
            }
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
            atomicMax(argmax_slot(ex.argmax_key) + m0 + threadIdx.x, s_key[threadIdx.x]);
    }
}


// ---------------------------------------------------------------------------
// VALU GEMV for M <= 4 (decode batch 1..4): the weight stream uses the
// access pattern that reaches the highest HBM bandwidth on MI355X — T lanes
// (8..32) read one row's contiguous 16*T bytes per instruction, 64/T rows
// per wavefront instruction — instead of the 16-row x 64-byte footprint an
// MFMA B operand imposes. bf16 weights are widened in registers (a shift)
// and multiplied in f32 against the activations, which the block first
// stages in LDS (normalised there when a LayerNorm is fused). Each row's T
// partial sums are combined with lane shuffles. Wavefronts walk row groups
// with a grid stride, so the staging cost is shared by several row groups.
template <int MT, int T>
__global__ __launch_bounds__(256) void k_gemv_valu(const float* __restrict__ x, const uint16_t* __restrict__ W,
                                                   const float* __restrict__ bias, const float* residual,
                                                   OutDesc od, int M, int N, int K, int epilogue,
                                                   LinearExtras ex) {
    extern __shared__ __align__(16) float xs[];  // [MT][K]
    __shared__ double red[8];
    __shared__ unsigned long long s_key[MT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const long long xstr = ex.x_stride ? ex.x_stride : K;

    // stage the activation rows (LayerNorm applied here when fused)
    for (int m = 0; m < MT; m++) {
        float* dst = xs + (size_t)m * K;
        if (m >= M) {
            for (int k = tid; k < K; k += 256) dst[k] = 0.f;
            continue;
        }
        const float* row = x + (size_t)m * xstr;
        if (!ex.ln_g) {
            for (int k = 4 * tid; k < K; k += 1024)
                *reinterpret_cast<float4*>(dst + k) = *reinterpret_cast<const float4*>(row + k);
            continue;
        }
        double s1 = 0.0;
        for (int k = tid; k < K; k += 256) s1 += (double)row[k];
        s1 = wave_sum_d(s1);
        if (lane == 0) red[wave] = s1;
        __syncthreads();
        const double mean = div_rcp(red[0] + red[1] + red[2] + red[3], (double)K, 1.0 / K);
        __syncthreads();
        double s2 = 0.0;
        for (int k = tid; k < K; k += 256) {
            double dd = (double)row[k] - mean;
            s2 += dd * dd;
        }
        s2 = wave_sum_d(s2);
        if (lane == 0) red[wave] = s2;
        __syncthreads();
        const double var = div_rcp(red[0] + red[1] + red[2] + red[3], (double)K, 1.0 / K);
        __syncthreads();
        const float inv = (float)rsqrt_f64(var + (double)ex.ln_eps);
        const float fm = (float)mean;
        for (int k = tid; k < K; k += 256) {
            float normalized = (row[k] - fm) * inv;
            dst[k] = normalized * ex.ln_g[k] + ex.ln_b[k];
        }
    }
    if (ex.argmax_key && tid < MT) s_key[tid] = 0ull;
    __syncthreads();

    constexpr int RPI = 64 / T;         // rows per wavefront instruction
    constexpr int CU = 8;               // 16-byte chunks per lane in flight
    const int sub = lane % T, rloc = lane / T;
    const int C = K / (8 * T);          // chunks per lane per row
    const int ngroups = (N + RPI - 1) / RPI;
    for (int rg = blockIdx.x * 4 + wave; rg < ngroups; rg += gridDim.x * 4) {
        const int row = rg * RPI + rloc;
        const bool row_ok = row < N;
        const uint4* wr = reinterpret_cast<const uint4*>(W + (size_t)(row_ok ? row : 0) * K) + sub;
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; m++) acc[m] = 0.f;
        for (int c0 = 0; c0 < C; c0 += CU) {
            uint4 wv[CU];
#pragma unroll
            for (int u = 0; u < CU; u++)
                wv[u] = (row_ok && c0 + u < C) ? wr[(size_t)T * (c0 + u)] : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int u = 0; u < CU; u++) {
                if (c0 + u >= C) break;
                const int k = 8 * (sub + T * (c0 + u));
                const float w8[8] = {bf16_lo(wv[u].x), bf16_hi(wv[u].x), bf16_lo(wv[u].y), bf16_hi(wv[u].y),
                                     bf16_lo(wv[u].z), bf16_hi(wv[u].z), bf16_lo(wv[u].w), bf16_hi(wv[u].w)};
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    const float4 a0 = *reinterpret_cast<const float4*>(xs + (size_t)m * K + k);
                    const float4 a1 = *reinterpret_cast<const float4*>(xs + (size_t)m * K + k + 4);
                    acc[m] += a0.x * w8[0] + a0.y * w8[1] + a0.z * w8[2] + a0.w * w8[3] +
                              a1.x * w8[4] + a1.y * w8[5] + a1.z * w8[6] + a1.w * w8[7];
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; m++) acc[m] = seg_sum<T>(acc[m]);
        if (sub == 0 && row_ok) {
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if (m >= M) break;
                float s = acc[m];
                if (bias) s = s + bias[row];
                if (epilogue == GORCH_HIP_EPI_GELU) s = gelu_tanh(s);
                if (residual) s = residual[(size_t)m * N + row] + s;
                *od.at(m, row) = s;
                if (ex.argmax_key) atomicMax(&s_key[m], argmax_pack(s, row));
            }
        }
    }
    if (ex.argmax_key) {
        __syncthreads();
        if (tid < MT && tid < M) atomicMax(argmax_slot(ex.argmax_key) + tid, s_key[tid]);
    }
}

// M = 1 variant with the activation row held in registers: lane `sub`
// always needs the same C chunks of x (k = 8*(sub + T*c)). The block stages
// the row once in LDS (with a fused norm, its moments too) behind one
// barrier, while the first two row groups' weight loads are already in
// flight; each lane then keeps its chunks (normalised) in registers. The
// next row group's weight loads are issued before the current group is
// reduced.
// PRO selects what is applied to the activation row as it is loaded: 0
// nothing, 1 LayerNorm (gamma, beta), 2 RMSNorm (gamma), 3 SwiGLU of a
// [gate | up] row of 2K values (silu(gate) * up, silu.go:121-136).
template <int T, int C, int PRO>
__global__ __launch_bounds__(256) void k_gemv_m1(const float* __restrict__ x, const uint16_t* __restrict__ W,
                                                 const float* __restrict__ bias, const float* residual, OutDesc od,
                                                 int N, int K, int epilogue, LinearExtras ex) {
    constexpr bool LN = PRO == 1 || PRO == 2;
    __shared__ unsigned long long s_key;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane % T, rloc = lane / T;
    constexpr int RPI = 64 / T;
    // paired SwiGLU rows (RPI == 2): group g is gate row g and up row F + g
    const int F = ex.pair_swiglu;
    const int ngroups = F ? F : (N + RPI - 1) / RPI;
    const int stride = gridDim.x * 4;
    int rg = blockIdx.x * 4 + wave;

    // Group g = rows g*RPI .. of W with their bias and residual values, as
    // raw buffer loads over the group's rows: rows past N (and groups past
    // the wave's last) read zeros, with no branch around the loads, so the
    // next group stays in flight while this one is reduced and written.
    struct Group {
        uint4 w[C];
        float b, r;
    };
    auto load = [&](int g, Group& gr) {
        const int rows = max(0, min(RPI, N - g * RPI));
        // paired rows: one resource from gate row g through up row F + g
        const __amdgpu_buffer_rsrc_t rs =
            F ? make_rsrc(W + (size_t)g * K, g < F ? ((long long)F * K + K) * 2 : 0)
              : make_rsrc(W + (size_t)g * RPI * K, (long long)rows * K * 2);
        const int roff = F ? (rloc ? F * K : 0) : rloc * K;
#pragma unroll
        for (int c = 0; c < C; c++)
            gr.w[c] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (roff + 8 * (sub + T * c)) * 2, 0, kStreamPolicy));
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(bias + (size_t)g * RPI, bias ? (long long)rows * 4 : 0);
        const __amdgpu_buffer_rsrc_t rr = make_rsrc(residual + (size_t)g * RPI, residual ? (long long)rows * 4 : 0);
        gr.b = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, rloc * 4, 0, 0));
        gr.r = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, rloc * 4, 0, 0));
    };
    // The activation row (K = 8*T*C exactly) is loaded once per block, not
    // once per wave: thread t takes float4 t, t + 256, ... of x (and of
    // gamma/beta, or of the up half), computes its share of the row moments
    // and parks the values in LDS; after one barrier every lane reads the
    // chunks it needs (k = 8*(sub + T*c)). A CU's vector-memory requests are
    // what bounds this kernel, so four waves each fetching the whole row (and
    // gamma/beta) cost as much as a large part of the weight slice.
    constexpr int KX = 8 * T * C, NV = KX / 4, PER = (NV + 255) / 256;
    __shared__ float4 s_x[NV];
    __shared__ float4 s_g[LN ? NV : 1];
    __shared__ float4 s_b[PRO == 1 ? NV : 1];
    __shared__ double2 s_mom[4];
    auto ld4 = [](__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    };
    // raw buffer loads with no branch around them: float4s past the row read
    // zeros and are neither counted nor stored
    const __amdgpu_buffer_rsrc_t rxs = make_rsrc(x, (long long)(PRO == 3 ? 2 : 1) * KX * 4);
    const __amdgpu_buffer_rsrc_t rgs = make_rsrc(ex.ln_g, LN ? (long long)KX * 4 : 0);
    const __amdgpu_buffer_rsrc_t rbs = make_rsrc(ex.ln_b, PRO == 1 ? (long long)KX * 4 : 0);
    float4 vx[PER], vg[LN ? PER : 1], vb[PRO == 1 ? PER : 1], vu[PRO == 3 ? PER : 1];
#pragma unroll
    for (int p = 0; p < PER; p++) {
        const int i = tid + 256 * p;
        const int off = i < NV ? 16 * i : kOutOfRange;
        vx[p] = ld4(rxs, off);
        if constexpr (LN) vg[p] = ld4(rgs, off);
        if constexpr (PRO == 1) vb[p] = ld4(rbs, off);
        if constexpr (PRO == 3) vu[p] = ld4(rxs, i < NV ? 16 * (NV + i) : kOutOfRange);
    }
    // LayerNorm's moment shift: the row's first value, the same for every thread
    const float x0 = PRO == 1 ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rxs, 0, 0, 0)) : 0.f;
    // then two row groups of the weight stream: the activation loads above
    // come from L2 and were issued first, so using them waits for them
    // alone, not for the weights (a wave's loads complete in issue order)
    Group ga, gb;
    load(rg, ga);
    load(rg + stride, gb);
    const int posv = od.pos_dev ? *od.pos_dev : 0;
    const bool own_stats = LN && !(PRO == 1 && ex.ln_stats);
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int p = 0; p < PER; p++) {
        const int i = tid + 256 * p;
        if constexpr (PRO == 3) {
            // silu(gate) * up (silu.go:121-136), the up half K values later
            const float gv[4] = {vx[p].x, vx[p].y, vx[p].z, vx[p].w};
            const float up[4] = {vu[p].x, vu[p].y, vu[p].z, vu[p].w};
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = gv[e] * sigmoidf_ref(gv[e]) * up[e];
            vx[p] = make_float4(o[0], o[1], o[2], o[3]);
        }
        if (i < NV) {
            if (own_stats) {
                const float e4[4] = {vx[p].x, vx[p].y, vx[p].z, vx[p].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    // RMSNorm: sum(x^2); LayerNorm: shifted moments
                    const double dd = (double)e4[e] - (double)x0;
                    if constexpr (PRO == 1) s1 += dd;
                    s2 += dd * dd;
                }
            }
            s_x[i] = vx[p];
            if constexpr (LN) s_g[i] = vg[p];
            if constexpr (PRO == 1) s_b[i] = vb[p];
        }
    }
    if (own_stats) {
        wave_sum2_d(s1, s2);
        if (lane == 0) s_mom[wave] = make_double2(s1, s2);
    }
    if (ex.argmax_key && tid == 0) s_key = 0ull;
    __syncthreads();
    float fm = 0.f, inv = 1.f;
    if constexpr (PRO == 2) {
        // RMSNorm (nn/rmsnorm.go:39-81): y = x * f32(1/sqrt(sum(x^2)/K + eps))
        // * gamma, the sum in f64
        const double t2 = (s_mom[0].y + s_mom[1].y) + (s_mom[2].y + s_mom[3].y);
        inv = (float)rsqrt_f64(div_rcp(t2, (double)KX, 1.0 / KX) + (double)ex.ln_eps);
    }
    if constexpr (PRO == 1) {
        if (ex.ln_stats) {
            fm = ex.ln_stats[0].x;
            inv = ex.ln_stats[0].y;
        } else {
            // The row's mean and variance in f64 (nn/layernorm.go:61-75) as
            // shifted moments in one pass: with c = x[0], s1 = sum(x - c)
            // and s2 = sum((x - c)^2), mean = c + s1/K and var = s2/K -
            // (s1/K)^2 — the reference's two-pass values to f64 rounding
            // (the shift keeps the subtraction well conditioned)
            const double t1 = (s_mom[0].x + s_mom[1].x) + (s_mom[2].x + s_mom[3].x);
            const double t2 = (s_mom[0].y + s_mom[1].y) + (s_mom[2].y + s_mom[3].y);
            const double ms = div_rcp(t1, (double)KX, 1.0 / KX);
            const double var = fmax(div_rcp(t2, (double)KX, 1.0 / KX) - ms * ms, 0.0);
            inv = (float)rsqrt_f64(var + (double)ex.ln_eps);
            fm = (float)((double)x0 + ms);
        }
    }
    // this lane's chunks of the (normalised) row
    float xr[C][8];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int v4 = 2 * (sub + T * c);
        const float4 a0 = s_x[v4], a1 = s_x[v4 + 1];
        xr[c][0] = a0.x; xr[c][1] = a0.y; xr[c][2] = a0.z; xr[c][3] = a0.w;
        xr[c][4] = a1.x; xr[c][5] = a1.y; xr[c][6] = a1.z; xr[c][7] = a1.w;
        if constexpr (LN) {
            const float4 g0 = s_g[v4], g1 = s_g[v4 + 1];
            const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
            float bb[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if constexpr (PRO == 1) {
                const float4 b0 = s_b[v4], b1 = s_b[v4 + 1];
                bb[0] = b0.x; bb[1] = b0.y; bb[2] = b0.z; bb[3] = b0.w;
                bb[4] = b1.x; bb[5] = b1.y; bb[6] = b1.z; bb[7] = b1.w;
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if constexpr (PRO == 2) {
                    xr[c][i] = xr[c][i] * inv * gg[i];
                } else {
                    const float normalized = (xr[c][i] - fm) * inv;
                    xr[c][i] = normalized * gg[i] + bb[i];
                }
            }
        }
    }

    unsigned long long best = 0ull;
    auto compute = [&](int g, const Group& gr) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < C; c++) {
            const uint4 cw = gr.w[c];
            acc += xr[c][0] * bf16_lo(cw.x) + xr[c][1] * bf16_hi(cw.x) + xr[c][2] * bf16_lo(cw.y) +
                   xr[c][3] * bf16_hi(cw.y) + xr[c][4] * bf16_lo(cw.z) + xr[c][5] * bf16_hi(cw.z) +
                   xr[c][6] * bf16_lo(cw.w) + xr[c][7] * bf16_hi(cw.w);
        }
        acc = seg_sum<T>(acc);
        if (F) {
            // lane 0 holds gate_g, lane 32 up_g (silu.go:121-136 order)
            const float up = readlane_f(acc, 32);
            if (lane == 0 && g < F) *od.at_p(0, g, posv) = acc * sigmoidf_ref(acc) * up;
            return;
        }
        const int row = g * RPI + rloc;
        if (sub == 0 && row < N) {
            float v = acc;
            if (bias) v = v + gr.b;
            if (epilogue == GORCH_HIP_EPI_GELU) v = gelu_tanh(v);
            if (residual) v = gr.r + v;
            *od.at_p(0, row, posv) = v;
            if (ex.argmax_key) {
                const unsigned long long key = argmax_pack(v, row);
                best = key > best ? key : best;
            }
        }
    };
    // two register sets: the next group's stream is in flight while this
    // one is reduced and written
    for (; rg < ngroups; rg += 2 * stride) {
        compute(rg, ga);
        load(rg + 2 * stride, ga);
        if (rg + stride < ngroups) compute(rg + stride, gb);
        load(rg + 3 * stride, gb);
    }
    if (ex.argmax_key) {
        // the wave's maximum, then one LDS atomic per wave
        best = wave_max_u64(best);
        if (lane == 0) atomicMax(&s_key, best);
        __syncthreads();
        if (tid == 0) atomicMax(argmax_slot(ex.argmax_key), s_key);
    }
}

// ---------------------------------------------------------------------------
// Multi-row GEMV for 2 <= M <= 16 over wide N (LM-head class, >= 1024
// 16-row weight tiles).
//
// bps ~ 256 blocks of NW waves (every CU streams about the same number of
// tiles); wave w of block b takes the 16-row weight tiles t = b + bps * (w
// + NW * i) over the whole K. The block first stages all of the
// activations in LDS, already split into bf16 hi/lo in the MFMA A layout
// ([k-step][k-chunk g][row r], 16 bytes each; one conflict-free LDS read per
// k-step): loading A from global memory per k-step instead spends the
// vector-memory slots the weight stream needs and halves its bandwidth on
// MI355X. B fragments are read straight from HBM with 16-byte loads, ST
// 128-wide stages per batch; the first batch is issued before the staging.
// K is never split across blocks (that would need a cross-block reduction):
// shapes whose activations exceed the LDS budget use the in-block-split
// kernel above.

// LayerNorm statistics (nn/layernorm.go:61-91) in f64 over full rows.
template <int NW>
__device__ void mt_ln_stats(const float* x, long long xs, int M, int K, float eps, float* s_mean, float* s_inv) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int rr = wave; rr < M; rr += NW) {
        const float* row = x + (size_t)rr * xs;
        double s1 = 0.0;
        for (int k = 4 * lane; k < K; k += 256) {
            float4 a = *reinterpret_cast<const float4*>(row + k);
            s1 += (double)a.x + (double)a.y + (double)a.z + (double)a.w;
        }
        const double mean = div_rcp(wave_sum_d(s1), (double)K, 1.0 / K);
        double s2 = 0.0;
        for (int k = 4 * lane; k < K; k += 256) {
            float4 a = *reinterpret_cast<const float4*>(row + k);
            double d0 = (double)a.x - mean, d1 = (double)a.y - mean, d2 = (double)a.z - mean, d3 = (double)a.w - mean;
            s2 += d0 * d0 + d1 * d1 + d2 * d2 + d3 * d3;
        }
        const double var = div_rcp(wave_sum_d(s2), (double)K, 1.0 / K);
        if (lane == 0) {
            s_mean[rr] = (float)mean;
            s_inv[rr] = (float)rsqrt_f64(var + (double)eps);
        }
    }
}

// Stage x[0..M)[kb..ke) into LDS as bf16 hi/lo A fragments (LayerNorm
// applied first when fused): entry ((k-step * 4 + g) * mr + r) holds
// x[r][kb + 32*kstep + 8*g .. +8] for r < mr (M rounded up to 4, 8 or 16);
// rows >= M and k >= ke are zero. Thread t owns entries t + NW*64*p. The
// first PX of them are fetched into registers by mt_fetch_x before the
// weight stream is issued (a wave's loads complete in issue order, so
// activations loaded after the weights would wait for them); mt_stage_x
// converts those and loads any further entries itself.
struct MtX {
    __amdgpu_buffer_rsrc_t rs;
    long long xs;
    int M, mr, kb, ke, n;  // n = number of entries
};
__device__ __forceinline__ int mt_x_off(const MtX& X, int i) {
    const int rr = i % X.mr, gg = (i / X.mr) & 3, kst = i / (4 * X.mr);
    const int k = X.kb + 32 * kst + 8 * gg;
    return (i < X.n && rr < X.M && k < X.ke) ? (int)((rr * X.xs + k) * 4) : kOutOfRange;
}
template <int NW, int PX>
__device__ __forceinline__ void mt_fetch_x(const MtX& X, u32x4 (&xv)[PX][2]) {
#pragma unroll
    for (int p = 0; p < PX; p++) {
        const int off = mt_x_off(X, threadIdx.x + NW * 64 * p);
        xv[p][0] = __builtin_amdgcn_raw_buffer_load_b128(X.rs, off, 0, 0);
        xv[p][1] = __builtin_amdgcn_raw_buffer_load_b128(X.rs, off + 16, 0, 0);
    }
}
__device__ __forceinline__ void mt_put_x(const MtX& X, int i, float (&f)[8], const LinearExtras& ex,
                                         const float* s_mean, const float* s_inv, uint4* xh, uint4* xl) {
    const int rr = i % X.mr, gg = (i / X.mr) & 3, kst = i / (4 * X.mr);
    const int k = X.kb + 32 * kst + 8 * gg;
    if (ex.ln_g) {
        if (rr < X.M && k < X.ke) {
            const float mu = s_mean[rr], inv = s_inv[rr];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float normalized = (f[e] - mu) * inv;
                f[e] = normalized * ex.ln_g[k + e] + ex.ln_b[k + e];
            }
        }
    }
    bf16x8 hi, lo;
    split_hi_lo(f, hi, lo);
    xh[i] = __builtin_bit_cast(uint4, hi);
    xl[i] = __builtin_bit_cast(uint4, lo);
}
template <int NW, int PX>
__device__ void mt_stage_x(const MtX& X, const u32x4 (&xv)[PX][2], const LinearExtras& ex, const float* s_mean,
                           const float* s_inv, uint4* xh, uint4* xl) {
#pragma unroll
    for (int p = 0; p < PX; p++) {
        const int i = threadIdx.x + NW * 64 * p;
        if (i >= X.n) break;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; e++) f[e] = __uint_as_float(xv[p][e >> 2][e & 3]);
        mt_put_x(X, i, f, ex, s_mean, s_inv, xh, xl);
    }
    for (int i = threadIdx.x + NW * 64 * PX; i < X.n; i += NW * 64) {
        const int off = mt_x_off(X, i);
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(X.rs, off, 0, 0);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(X.rs, off + 16, 0, 0);
        float f[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            f[e] = __uint_as_float(a[e]);
            f[4 + e] = __uint_as_float(b[e]);
        }
        mt_put_x(X, i, f, ex, s_mean, s_inv, xh, xl);
    }
}

// A fragments of k-step ks for lane (r, g); zero for r >= MR.
template <int MR>
__device__ __forceinline__ void mt_a(const uint4* xh, const uint4* xl, int ks, int g, int r, bf16x8& hi,
                                     bf16x8& lo) {
    if constexpr (MR == 16) {
        const int ai = (ks * 4 + g) * 16 + r;
        hi = __builtin_bit_cast(bf16x8, xh[ai]);
        lo = __builtin_bit_cast(bf16x8, xl[ai]);
    } else {
        const bool ok = r < MR;
        const int ai = (ks * 4 + g) * MR + (ok ? r : 0);
        const uint4 h = xh[ai], l = xl[ai];
        const uint4 z = make_uint4(0, 0, 0, 0);
        hi = __builtin_bit_cast(bf16x8, ok ? h : z);
        lo = __builtin_bit_cast(bf16x8, ok ? l : z);
    }
}

// Finish tile ct: bias, GELU, output and the block's argmax key (no
// residual: a residual load here would wait for the prefetched weights).
// acc: rows 4g..4g+3 of column 16*ct + r; bv = bias[16*ct + r], loaded with
// the tile's weights.
__device__ __forceinline__ void mt_finish(const floatx4& acc, int ct, int M, int N, const float* bias, float bv,
                                          const OutDesc& od, int epilogue, const LinearExtras& ex,
                                          unsigned long long* s_key) {
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int on = ct * 16 + r;
    if (on >= N) return;
#pragma unroll
    for (int v4 = 0; v4 < 4; v4++) {
        const int om = 4 * g + v4;
        if (om >= M) break;
        float sum = acc[v4];
        if (bias) sum = sum + bv;  // bias[on], loaded with the tile's weights
        if (epilogue == GORCH_HIP_EPI_GELU) sum = gelu_tanh(sum);
        *od.at(om, on) = sum;
        if (ex.argmax_key) atomicMax(&s_key[om], argmax_pack(sum, on));
    }
}

template <int NW, int ST, int MR>
__global__ __launch_bounds__(NW * 64) void k_gemv_mt(
    const float* __restrict__ x, const uint16_t* __restrict__ W, const float* __restrict__ bias,
    const float* residual, OutDesc od, int M, int N, int K, int bps, int epilogue, LinearExtras ex) {
    constexpr int mr = MR;
    extern __shared__ uint4 smem[];
    __shared__ float s_mean[16], s_inv[16];
    __shared__ unsigned long long s_key[16];
    // wave index read as a scalar: the tile (and so each buffer resource) is
    // wave-uniform, so the resources live in SGPRs
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int bidx = blockIdx.x;
    const int kb = 0, ke = K;
    const int nst = (K + 127) >> 7;  // 128-wide stages
    uint4* xh = smem;
    uint4* xl = smem + nst * 16 * mr;
    const long long xs = ex.x_stride ? ex.x_stride : K;
    const int ntiles = (N + 15) >> 4;

    const int nbat = (nst + ST - 1) / ST;  // load batches per tile
    const int tstride = bps * NW;
    const int t0 = bidx + bps * wave;
    const int my_tiles = t0 < ntiles ? (ntiles - 1 - t0) / tstride + 1 : 0;
    const int total = my_tiles * nbat;  // this wave's batches, tile-major

    // Batch j: stages (j % nbat) * ST .. of tile t0 + tstride * (j / nbat),
    // with the tile's bias value. Raw buffer resources over the tile's rows
    // make rows past N, stages past K and batches past the wave's last read
    // as zeros with no branch around the loads, so the compiler can keep the
    // next batch in flight while this one feeds the matrix cores.
    uint4 va[ST][4], vb[ST][4];
    float ba, bb;
    auto load = [&](int j, uint4 (&v)[ST][4], float& bv) {
        // (the division runs on the vector unit; readfirstlane hands the
        // uniform results back as scalars for the resources)
        const int ti = __builtin_amdgcn_readfirstlane(j / nbat), bat = j - ti * nbat;
        const int t = t0 + tstride * ti;
        const int rows = max(0, min(16, N - 16 * t));
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(W + (size_t)t * 16 * K, (long long)rows * K * 2);
#pragma unroll
        for (int q = 0; q < ST; q++) {
            const int st = bat * ST + q;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int k = 128 * st + 32 * jj + 8 * g;
                const int off = k < K ? (r * K + k) * 2 : kOutOfRange;
                v[q][jj] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kStreamPolicy));
            }
        }
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(bias + (size_t)t * 16, bias ? (long long)rows * 4 : 0);
        bv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, r * 4, 0, 0));
    };
    // activations first (from L2), then two weight batches: staging waits
    // for the activation loads only
    MtX X;
    X.xs = xs;
    X.M = M;
    X.mr = mr;
    X.kb = kb;
    X.ke = ke;
    X.n = nst * 16 * mr;
    X.rs = make_rsrc(x, M > 0 ? ((long long)(M - 1) * xs + K) * 4 : 0);
    constexpr int PX = NW >= 16 ? 2 : (NW == 8 ? 3 : 2);
    u32x4 xv[PX][2];
    mt_fetch_x<NW, PX>(X, xv);
    load(0, va, ba);
    load(1, vb, bb);

    if (ex.ln_g && ex.ln_stats) {
        if (threadIdx.x < 16 && (int)threadIdx.x < M) {
            const float2 st = ex.ln_stats[threadIdx.x];
            s_mean[threadIdx.x] = st.x;
            s_inv[threadIdx.x] = st.y;
        }
        __syncthreads();
    } else if (ex.ln_g) {
        mt_ln_stats<NW>(x, xs, M, K, ex.ln_eps, s_mean, s_inv);
        __syncthreads();
    }
    if (ex.argmax_key && threadIdx.x < 16) s_key[threadIdx.x] = 0ull;
    mt_stage_x<NW, PX>(X, xv, ex, s_mean, s_inv, xh, xl);
    __syncthreads();

    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int j, const uint4 (&v)[ST][4], float bv) {
        const int ti = j / nbat, bat = j - ti * nbat;
#pragma unroll
        for (int q = 0; q < ST; q++) {
            const int st = bat * ST + q;
            if (st >= nst) break;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                bf16x8 ah, al;
                mt_a<MR>(xh, xl, 4 * st + u, g, r, ah, al);
                const bf16x8 wb = __builtin_bit_cast(bf16x8, v[q][u]);
                acc = mfma16x16x32(ah, wb, acc);
                acc = mfma16x16x32(al, wb, acc);
            }
        }
        if (bat == nbat - 1) {
            mt_finish(acc, t0 + tstride * ti, M, N, bias, bv, od, epilogue, ex, s_key);
            acc = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    };
    for (int j = 0; j < total; j += 2) {
        compute(j, va, ba);
        load(j + 2, va, ba);
        if (j + 1 < total) compute(j + 1, vb, bb);
        load(j + 3, vb, bb);
    }
    if (ex.argmax_key) {
        __syncthreads();
        if (threadIdx.x < 16 && (int)threadIdx.x < M) atomicMax(argmax_slot(ex.argmax_key) + threadIdx.x, s_key[threadIdx.x]);
    }
}

// ---------------------------------------------------------------------------
// Persistent multi-row GEMV for 1 <= M <= 16 over tile-packed weights.
//
// A block is NW waves; wave w owns k-steps [w*ks, (w+1)*ks) of every 16-row
// weight tile. It loads the activation A fragments of that K range once, as
// bf16 hi/lo in registers (x = hi + lo, two MFMAs per fragment), and keeps
// them for the whole kernel; then the block walks the tiles t = blockIdx.x
// + gridDim.x * i with two register sets of B fragments, so the next tile's
// weights are in flight while this one feeds the matrix cores. Per tile the
// NW partial 16x16 results go through LDS (two buffers by tile parity) and
// wave 0 sums them in wave order and finishes the tile (bias, GELU,
// residual, output, argmax keys). Every load is a raw buffer load with no
// branch around it: k past the wave's range, rows past M or N and tiles
// past the last read as zeros.
// Activation input of k_gemv_tiles: f32 rows, f32 rows with LayerNorm
// fused, or the fragment layout (a template argument, so the f32 kernels
// compile as if the other forms did not exist)
constexpr int kXmRows = 0, kXmLn = 1, kXmFrag = 2;
template <int NW, int KS, bool EARLY, int XM>
__global__ __launch_bounds__(NW * 64) void k_gemv_tiles(const float* __restrict__ x, const uint16_t* __restrict__ W,
                                                        const float* __restrict__ bias, const float* residual,
                                                        OutDesc od, int M, int N, int K, int ks, int epilogue,
                                                        LinearExtras ex) {
    __shared__ floatx4 red[2][NW][64];
    __shared__ unsigned long long s_key[16];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    // K-split mode (ex.part or ex.accumulate): blockIdx.y is the K slice
    // [ex.kslice * y, ..) and the block writes raw partial sums for a
    // following reduction, or adds them into the output
    const bool ksplit = ex.part || ex.accumulate;
    const int k_off = ksplit ? (int)blockIdx.y * ex.kslice : 0;
    const int k_end = ksplit ? min(K, k_off + ex.kslice) : K;
    const int kb = k_off + wave * ks * 32, ke = min(k_end, kb + ks * 32);
    const long long xs = ex.x_stride ? ex.x_stride : K;
    const int ntiles = (N + 15) >> 4;
    const int G = gridDim.x;

    // activations first (they come from L2): converting them waits for
    // them alone, not for the weights issued after them
    // (pre-split activations: k-step j's hi and lo fragments, one
    // contiguous 1 KB each per wave)
    constexpr bool LN = XM == kXmLn, XF = XM == kXmFrag;
    u32x4 xa[KS][2];
    if constexpr (XF) {
        const __amdgpu_buffer_rsrc_t rsf = make_rsrc(ex.x_frag, (long long)xfrag_bytes(K));
#pragma unroll
        for (int u = 0; u < KS; u++) {
            const int k0 = kb + 32 * u;
            const int off = k0 < ke ? (k0 >> 5) * 2048 + 16 * lane : kOutOfRange;
            xa[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rsf, off, 0, 0);
            xa[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rsf, off + 1024, 0, 0);
        }
    } else {
        const __amdgpu_buffer_rsrc_t rsx = make_rsrc(x, ((long long)(M - 1) * xs + K) * 4);
#pragma unroll
        for (int u = 0; u < KS; u++) {
            const int kc = kb + 32 * u + 8 * g;
            const int off = (r < M && kc < ke) ? (int)((r * xs + kc) * 4) : kOutOfRange;
            xa[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rsx, off, 0, 0);
            xa[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rsx, off + 16, 0, 0);
        }
    }
    // LayerNorm gamma/beta fragments (nn/layernorm.go:31-91), loaded with the
    // activations
    u32x4 ga[LN ? KS : 1][2], be[LN ? KS : 1][2];
    if constexpr (LN) {
        const __amdgpu_buffer_rsrc_t rg = make_rsrc(ex.ln_g, (long long)K * 4);
        const __amdgpu_buffer_rsrc_t rbe = make_rsrc(ex.ln_b, (long long)K * 4);
#pragma unroll
        for (int u = 0; u < KS; u++) {
            const int kc = kb + 32 * u + 8 * g;
            const int off = kc < ke ? kc * 4 : kOutOfRange;
            ga[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0);
            ga[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rg, off + 16, 0, 0);
            be[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rbe, off, 0, 0);
            be[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rbe, off + 16, 0, 0);
        }
    }
    const __amdgpu_buffer_rsrc_t rsr = make_rsrc(residual, residual ? (long long)M * N * 4 : 0);
    // Tile epilogue split over the waves: wave w finishes outputs o = w *
    // OPW + lane (lane < OPW, OPW = 256 / NW), o = 16 * m + c for row m and
    // column c of the tile; the partial 16x16 results hold (m, c) in lane
    // 16 * (m / 4) + c, component m % 4.
    constexpr int OPW = 256 / NW;
    const bool out_lane = lane < OPW;
    const int o = wave * OPW + (out_lane ? lane : 0);
    const int om = o >> 4, oc = o & 15;
    struct Tile {
        u32x4 w[KS];
        float b, res;
    };
    // tile t is 16 * K32 bf16 from W + t * 16 * K32 (K32 = K rounded up to
    // 32), fragment (t, k-step j) the 1 KB at byte 1024 * j, lane l's 16
    // bytes at 16 * l
    const int K32 = (K + 31) & ~31;
    auto load = [&](int t, Tile& tl) {
        const int rows = max(0, min(16, N - 16 * t));
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc(W + (size_t)t * 16 * K32, t < ntiles ? (long long)16 * K32 * 2 : 0);
#pragma unroll
        for (int u = 0; u < KS; u++) {
            const int kc = kb + 32 * u + 8 * g;
            const int off = (kb + 32 * u) * 32 + 16 * lane;
            tl.w[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, kc < ke ? off : kOutOfRange, 0, kStreamPolicy);
        }
        // this lane's output column's bias and residual
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(bias + (size_t)t * 16, bias ? (long long)rows * 4 : 0);
        tl.b = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, oc * 4, 0, 0));
        const int on = 16 * t + oc;
        const int roff = (om < M && on < N) ? (om * N + on) * 4 : kOutOfRange;
        tl.res = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsr, roff, 0, 0));
    };
    Tile ta, tb;
    int t = blockIdx.x;
    load(t, ta);
    load(t + G, tb);

    // Fused LayerNorm: the block holds each activation row exactly once (row
    // r in the lanes r, r+16, r+32, r+48 of every wave, each over its K
    // slice), so the row's f64 sums come from registers: per-lane sums, then
    // LDS across lane groups and waves; mean = s1/K, var = s2/K - mean^2
    // (the reference's two-pass values to f64 rounding for activations whose
    // mean is not many orders above their spread).
    float ln_mean = 0.f, ln_inv = 1.f;
    if constexpr (LN) {
        __shared__ double2 s_mom[NW][64];
        __shared__ float s_stat[16][2];
        double s1 = 0.0, s2 = 0.0;
#pragma unroll
        for (int u = 0; u < KS; u++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const double v = (double)__uint_as_float(xa[u][e >> 2][e & 3]);
                s1 += v;
                s2 += v * v;
            }
        s_mom[wave][lane] = make_double2(s1, s2);
        __syncthreads();
        if (threadIdx.x < 16 && (int)threadIdx.x < M) {
            double t1 = 0.0, t2 = 0.0;
            for (int w = 0; w < NW; w++)
                for (int gg = 0; gg < 4; gg++) {
                    const double2 q = s_mom[w][16 * gg + threadIdx.x];
                    t1 += q.x;
                    t2 += q.y;
                }
            const double rk = 1.0 / K;
            const double mean = div_rcp(t1, (double)K, rk);
            const double var = fmax(div_rcp(t2, (double)K, rk) - mean * mean, 0.0);
            s_stat[threadIdx.x][0] = (float)mean;
            s_stat[threadIdx.x][1] = (float)rsqrt_f64(var + (double)ex.ln_eps);
        }
        __syncthreads();
        ln_mean = s_stat[r][0];
        ln_inv = s_stat[r][1];
    }
    bf16x8 ah[KS], al[KS];
#pragma unroll
    for (int u = 0; u < KS; u++) {
        if constexpr (XF) {
            ah[u] = __builtin_bit_cast(bf16x8, xa[u][0]);
            al[u] = __builtin_bit_cast(bf16x8, xa[u][1]);
            continue;
        }
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; e++) f[e] = __uint_as_float(xa[u][e >> 2][e & 3]);
        if constexpr (LN) {
            // k past the range: the normalised zero is masked
            const bool ok = kb + 32 * u + 8 * g < ke && r < M;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float normalized = (f[e] - ln_mean) * ln_inv;
                f[e] = ok ? normalized * __uint_as_float(ga[u][e >> 2][e & 3]) + __uint_as_float(be[u][e >> 2][e & 3])
                          : 0.f;
            }
        }
        split_hi_lo(f, ah[u], al[u]);
    }
    const int posv = od.pos_dev ? *od.pos_dev : 0;
    if (ex.argmax_key) {
        if (threadIdx.x < 16) s_key[threadIdx.x] = 0ull;
        __syncthreads();
    }
    unsigned long long best = 0ull;
    const float* redf = reinterpret_cast<const float*>(&red[0][0][0]);

    // Tile tt from register set tl, whose registers are then refilled with
    // tile next: with EARLY as soon as the matrix cores have read them
    // (before the barrier and the epilogue: measured faster with one or two
    // tiles per block), else after the epilogue (faster with many)
    auto step = [&](int tt, Tile& tl, int buf, int next) {
        // hi and lo products in two accumulators: two independent MFMA chains
        floatx4 acc_h = {0.f, 0.f, 0.f, 0.f}, acc_l = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < KS; u++) {
            const bf16x8 b = __builtin_bit_cast(bf16x8, tl.w[u]);
            acc_h = mfma16x16x32(ah[u], b, acc_h);
            acc_l = mfma16x16x32(al[u], b, acc_l);
        }
        float bv = 0.f, rv = 0.f;
        if constexpr (EARLY) {
            bv = tl.b;
            rv = tl.res;
            load(next, tl);
        }
        red[buf][wave][lane] = acc_h + acc_l;
        __syncthreads();
        const int on = 16 * tt + oc;
        if (out_lane && om < M && on < N) {
            const int src = 16 * (om >> 2) + oc, comp = om & 3;
            float val = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) val += redf[((buf * NW + w) * 64 + src) * 4 + comp];
            if (ex.accumulate) {
                if (bias && blockIdx.y == 0) val = val + (EARLY ? bv : tl.b);
                __hip_atomic_fetch_add(od.at_p(om, on, posv), val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return;
            }
            if (ex.part) {
                ex.part[((size_t)blockIdx.y * M + om) * N + on] = val;
                return;
            }
            if (bias) val = val + (EARLY ? bv : tl.b);
            if (epilogue == GORCH_HIP_EPI_GELU) val = gelu_tanh(val);
            if (residual) val = (EARLY ? rv : tl.res) + val;
            if constexpr (XF) {
                if (ex.out_frag) {
                    uint16_t hi, lo;
                    split_hi_lo1(val, hi, lo);
                    const size_t i = xfrag_index(om, on);
                    ex.out_frag[i] = hi;
                    ex.out_frag[i + 512] = lo;
                    return;
                }
            }
            *od.at_p(om, on, posv) = val;
            if (ex.argmax_key) {
                const unsigned long long key = argmax_pack(val, on);
                best = key > best ? key : best;
            }
        }
    };
    for (; t < ntiles; t += 2 * G) {
        if constexpr (EARLY) {
            step(t, ta, 0, t + 2 * G);
            if (t + G < ntiles) step(t + G, tb, 1, t + 3 * G);
        } else {
            step(t, ta, 0, 0);
            load(t + 2 * G, ta);
            if (t + G < ntiles) step(t + G, tb, 1, 0);
            load(t + 3 * G, tb);
        }
    }
    if (ex.argmax_key) {
        // row om's maximum over the 16 columns (the 16 lanes of one DPP row
        // share om), then one LDS atomic per row and block
        best = row16_max_u64(best);
        if (out_lane && oc == 0 && om < M) atomicMax(&s_key[om], best);
        __syncthreads();
        if (threadIdx.x < 16 && (int)threadIdx.x < M) atomicMax(argmax_slot(ex.argmax_key) + threadIdx.x, s_key[threadIdx.x]);
    }
}

// Epilogue of a K-split Linear: y[m, n] = epi(sum_s part[s][m][n] + bias[n])
// (+ residual), slices added in order, written through the output
// descriptor. All slice loads of an element are issued before the adds.
constexpr int kEpiSlices = kMaxPartSlices;
template <int ES>
__global__ __launch_bounds__(256) void k_splitk_epilogue(const float* __restrict__ part, int S, int M, int N,
                                                         const float* __restrict__ bias, const float* residual,
                                                         OutDesc od, int epilogue) {
    const int64_t total = (int64_t)M * N;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int m = (int)(i / N), n = (int)(i - (int64_t)m * N);
    // raw buffer loads with no branch around them (slices past S, a missing
    // bias or residual read as zeros), all in flight before the adds
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, (long long)S * total * 4);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bias, bias ? (long long)N * 4 : 0);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(residual, residual ? total * 4 : 0);
    float p[ES];
#pragma unroll
    for (int q = 0; q < ES; q++) {
        const int off = q < S ? (int)(((int64_t)q * total + i) * 4) : kOutOfRange;
        p[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, off, 0, 0));
    }
    const float bv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, n * 4, 0, 0));
    const float rv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, (int)(i * 4), 0, 0));
    float sum = p[0];
#pragma unroll
    for (int q = 1; q < ES; q++)
        if (q < S) sum += p[q];
    if (bias) sum = sum + bv;
    if (epilogue == GORCH_HIP_EPI_GELU) sum = gelu_tanh(sum);
    if (residual) sum = rv + sum;
    *od.at(m, n) = sum;
}

int launch_splitk_epilogue(hipStream_t s, const float* part, int S, int M, int N, const float* bias,
                           const float* residual, const OutDesc& od, int epilogue) {
    if (S < 1 || S > kEpiSlices) {
        set_error("splitk_epilogue: 1..8 slices");
        return GORCH_HIP_EUNSUPPORTED;
    }
    const int64_t total = (int64_t)M * N;
    if (total == 0) return GORCH_HIP_OK;
    // slice registers sized to S (loads of absent slices still cost their
    // instructions)
    const dim3 grid((unsigned)((total + 255) / 256));
    if (S <= 4)
        hipLaunchKernelGGL(k_splitk_epilogue<4>, grid, dim3(256), 0, s, part, S, M, N, bias, residual, od, epilogue);
    else
        hipLaunchKernelGGL(k_splitk_epilogue<kEpiSlices>, grid, dim3(256), 0, s, part, S, M, N, bias, residual, od,
                           epilogue);
    count(CNT_GEMV);
    return check_launch("splitk_epilogue");
}

// (T, C) for the register-x M = 1 kernel: T lanes per row, C 16-byte chunks
// per lane, C <= 8; {0, 0} when K does not fit.
static void m1_shape(int K, int* T, int* C) {
    *T = *C = 0;
    if (K % 8 != 0) return;  // the kernel reads K = 8*T*C values exactly
    const int chunks = K / 8;
    for (int t = 64; t >= 8; t >>= 1)
        if (chunks % t == 0 && chunks / t <= 8) {
            *T = t;
            *C = chunks / t;
            return;
        }
}

bool gemv_pair_swiglu_ok(int F, int K) {
    return F > 0 && K % 256 == 0 && K / 256 >= 1 && K / 256 <= 8 && (long long)2 * F * K * 2 < (1ll << 31);
}

bool gemv_m1_prologue_ok(int K) {
    int T1, C1;
    m1_shape(K, &T1, &C1);
    return T1 != 0 && K % 8 == 0;
}

static int launch_m1(hipStream_t s, const float* x, const uint16_t* W, const float* bias, const float* residual,
                     const OutDesc& od, int N, int K, int epilogue, const LinearExtras& ex, int T, int C) {
    const int rpi = 64 / T;
    const int ngroups = (N + rpi - 1) / rpi;
    constexpr int max_blocks = 768;
    // with the argmax fusion every block ends in one 64-bit atomicMax on the
    // same global word, and those serialise at one L2 channel (4096 of them
    // cost ~40 us): fewer, longer-running blocks
    constexpr int max_blocks_argmax = 512;
    // one row group per wave; two with a fused LayerNorm, whose activation,
    // gamma and beta rows every wave loads whole (GPT-2 small batch-1 decode
    // with 1, 3 or 4 groups per wave: 4,135 / 4,168 / 4,023 tok/s, 2: 4,450)
    int blocks = ex.ln_g ? (ngroups + 7) / 8 : (ngroups + 3) / 4;
    if (blocks > max_blocks) blocks = max_blocks;
    if (ex.argmax_key && blocks > max_blocks_argmax) blocks = max_blocks_argmax;
    // between one and two blocks per CU: one per CU, each taking more row
    // groups (a second block on a CU doubles that CU's time when each
    // streams several rounds)
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            n = 256;
        return n;
    }();
    // (rounded up to two per CU when that leaves at most two groups per
    // wave, all in flight from the start: Qwen3-shaped gate/up, 3,072 paired
    // groups on 512 blocks, 1,377 -> 1,391 tok/s at context 128)
    if (blocks > cus && blocks < 2 * cus) blocks = ngroups <= 16 * cus ? 2 * cus : cus;
    const int pro = ex.swiglu ? 3 : (ex.ln_g ? (ex.ln_rms ? 2 : 1) : 0);
#define GH_M1_L(TT, CC, PV)                                                                                 \
    hipLaunchKernelGGL((k_gemv_m1<TT, CC, PV>), dim3(blocks), dim3(256), 0, s, x, W, bias, residual, od, N, K, \
                       epilogue, ex)
#define GH_M1(TT, CC)                                                                                        \
    if (T == TT && C == CC) {                                                                                \
        if (pro == 1) GH_M1_L(TT, CC, 1);                                                                    \
        else if (pro == 2) GH_M1_L(TT, CC, 2);                                                               \
        else if (pro == 3) GH_M1_L(TT, CC, 3);                                                               \
        else GH_M1_L(TT, CC, 0);                                                                             \
        count(CNT_GEMV);                                                                                     \
        return check_launch("gemv_m1");                                                                      \
    }
    GH_M1(64, 1) GH_M1(64, 2) GH_M1(64, 3) GH_M1(64, 4) GH_M1(64, 5) GH_M1(64, 6) GH_M1(64, 7) GH_M1(64, 8)
    GH_M1(32, 1) GH_M1(32, 3) GH_M1(32, 5) GH_M1(32, 7)
    if (ex.pair_swiglu) {
        GH_M1(32, 2) GH_M1(32, 4) GH_M1(32, 6) GH_M1(32, 8)
    }
    GH_M1(16, 1) GH_M1(16, 3) GH_M1(16, 5) GH_M1(16, 7)
    GH_M1(8, 1) GH_M1(8, 3) GH_M1(8, 5) GH_M1(8, 7)
#undef GH_M1
#undef GH_M1_L
    return -1;  // not instantiated: caller falls through
}

template <int NW, int ST, int MR>
static int launch_mt_t(hipStream_t s, int grid, size_t lds, const float* x, const uint16_t* W, const float* bias,
                       const float* residual, const OutDesc& od, int M, int N, int K, int bps, int epilogue,
                       const LinearExtras& ex) {
    static bool attr_set = false;
    if (!attr_set) {
        GH_TRY(check(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_mt<NW, ST, MR>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, 136 * 1024),
                     "gemv_mt attribute"));
        attr_set = true;
    }
    hipLaunchKernelGGL((k_gemv_mt<NW, ST, MR>), dim3(grid), dim3(NW * 64), lds, s, x, W, bias, residual, od, M, N, K,
                       bps, epilogue, ex);
    return GORCH_HIP_OK;
}

// LDS for the staged activations: up to 128 KB (all of K).
constexpr size_t kMtLds = 128 * 1024;

// Multi-row GEMV launch; returns -1 when the activations do not fit LDS
// (the caller then uses the in-block-split MFMA kernel).
static int launch_mt(hipStream_t s, const float* x, const uint16_t* W, const float* bias, const float* residual,
                     const OutDesc& od, int M, int N, int K, int epilogue, const LinearExtras& ex) {
    const int ntiles = (N + 15) / 16;
    const int mr = M <= 4 ? 4 : (M <= 8 ? 8 : 16);
    const size_t lds = (size_t)((K + 127) / 128) * 16 * mr * 16 * 2;
    if (lds > kMtLds || residual) return -1;  // the kernel has no residual add
    const int nw = 16, st = 2;
    const int bps = std::min(256, ntiles);
    int rc = -1;
#define GH_MT(NWV, STV, MRV)                                                                                 \
    if (nw == NWV && st == STV && mr == MRV)                                                                 \
        rc = launch_mt_t<NWV, STV, MRV>(s, bps, lds, x, W, bias, residual, od, M, N, K, bps, epilogue, ex);
#define GH_MT_R(NWV, STV) GH_MT(NWV, STV, 4) GH_MT(NWV, STV, 8) GH_MT(NWV, STV, 16)
    GH_MT_R(4, 2) GH_MT_R(4, 3) GH_MT_R(4, 6) GH_MT_R(8, 1) GH_MT_R(8, 2) GH_MT_R(8, 3) GH_MT_R(16, 1) GH_MT_R(16, 2)
#undef GH_MT_R
#undef GH_MT
    if (rc < 0) return -1;
    if (rc != GORCH_HIP_OK) return rc;
    count(CNT_GEMV);
    return check_launch("gemv_mt");
}

// Persistent multi-row GEMV launch; -1 when K exceeds 8 x 12 k-steps.
static int launch_tiles(hipStream_t s, const float* x, const uint16_t* W, const float* bias, const float* residual,
                        const OutDesc& od, int M, int N, int K, int epilogue, const LinearExtras& ex) {

    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            n = 256;
        return n;
    }();
    const int ntiles = (N + 15) / 16;
    // with ex.part or ex.accumulate the grid's y dimension is ex.ksplit K
    // slices of ex.kslice
    const bool ksplit = ex.part || ex.accumulate;
    const int S = ksplit ? ex.ksplit : 1;
    const int ksteps = ksplit ? ex.kslice / 32 : (K + 31) / 32;
    // 8 waves per block; 4 when the blocks hold one or two tiles each (the
    // weight is short in tiles for the grid) and a 4-wave instantiation
    // takes the k-steps (measured: 9-shape GEMV sweep, 768x3072 at M = 4 /
    // 16 3.43 / 3.95 -> 3.21 / 3.74 us; the LM head keeps 8)
    int nw = 8;
    if (!ex.ln_g) {
        const int ks4 = (ksteps + 3) / 4;
        const bool fits4 = ks4 <= 8 && ks4 != 5 && ks4 != 7;
        if (fits4 && ntiles * S <= 2 * cus) nw = 4;
    }
    const int ks = (ksteps + nw - 1) / nw;
    // one round of resident blocks: a block beyond what the CUs hold at once
    // would run as a second, mostly idle round (measured 10 vs 7 us)
    auto blocks_for = [&](const void* kern, int threads) {
        int per_cu = 0, cus = 0, dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, 0) != hipSuccess || per_cu < 1)
            per_cu = 1, cus = cus > 0 ? cus : 256;
        return per_cu * cus;
    };
#define GH_TILES_L(NWV, KSV, EA)                                                                        \
    if (ex.x_frag)                                                                                      \
        hipLaunchKernelGGL((k_gemv_tiles<NWV, KSV, EA, kXmFrag>), dim3(blocks, S), dim3(NWV * 64), 0, s, x, W, \
                           bias, residual, od, M, N, K, ks, epilogue, ex);                              \
    else                                                                                                \
        hipLaunchKernelGGL((k_gemv_tiles<NWV, KSV, EA, kXmRows>), dim3(blocks, S), dim3(NWV * 64), 0, s, x, W, \
                           bias, residual, od, M, N, K, ks, epilogue, ex)
    // fused LayerNorm: packed weights, 8 waves, K <= 1024 (the LM head of a
    // one-row decode step)
    if (ex.ln_g) {
        if (nw != 8 || ks > 4 || S != 1) return -1;
        static const int blocks_ln =
            blocks_for(reinterpret_cast<const void*>(&k_gemv_tiles<8, 4, false, kXmLn>), 512);
        const int blocks = std::min(blocks_ln, ntiles);
#define GH_TILES_LN(KSV)                                                                                    \
    if (ntiles <= 2 * blocks)                                                                               \
        hipLaunchKernelGGL((k_gemv_tiles<8, KSV, true, kXmLn>), dim3(blocks), dim3(512), 0, s, x, W, bias, \
                           residual, od, M, N, K, ks, epilogue, ex);                                        \
    else                                                                                                    \
        hipLaunchKernelGGL((k_gemv_tiles<8, KSV, false, kXmLn>), dim3(blocks), dim3(512), 0, s, x, W, bias, \
                           residual, od, M, N, K, ks, epilogue, ex);
        if (ks <= 3) {
            GH_TILES_LN(3)
        } else {
            GH_TILES_LN(4)
        }
#undef GH_TILES_LN
        count(CNT_GEMV);
        return check_launch("gemv_tiles_ln");
    }
    // one or two tiles per block: no more blocks (over all K slices) than
    // CUs, since a second block on a CU streams beside the first and
    // doubles that CU's time (XL batch 16: FFN2's 7 K slices on 36 instead
    // of 73 blocks each, 5,059 -> 5,146 tok/s)
#define GH_TILES(NWV, KSV)                                                                                \
    if (nw == NWV && ks <= KSV) {                                                                         \
        static const int blocks_p = blocks_for(reinterpret_cast<const void*>(&k_gemv_tiles<NWV, KSV, false, kXmRows>), NWV * 64); \
        int blocks = std::min(std::max(1, blocks_p / S), ntiles);                                         \
        if (ntiles <= 2 * blocks) blocks = std::min(blocks, std::max(1, cus / S));                        \
        if (ntiles <= 2 * blocks) GH_TILES_L(NWV, KSV, true);                                             \
        else GH_TILES_L(NWV, KSV, false);                                                                 \
        count(CNT_GEMV);                                                                                  \
        return check_launch("gemv_tiles");                                                                \
    }
    // exact k-step counts where they occur (K = 768: 3 per wave, K = 1600: 7):
    // a padding slot still costs its instructions and registers (measured:
    // 8 waves x 3 against x 4 at K = 768, 9-shape GEMV sweep 3,362 -> 3,435
    // GB/s)
    GH_TILES(4, 3) GH_TILES(4, 4) GH_TILES(4, 6) GH_TILES(4, 8) GH_TILES(8, 2) GH_TILES(8, 3) GH_TILES(8, 4) GH_TILES(8, 7)
    GH_TILES(8, 8) GH_TILES(8, 12)
    GH_TILES(16, 4)
#undef GH_TILES
#undef GH_TILES_L
    return -1;
}

template <int MT>
static int launch_valu_mt(hipStream_t s, const float* x, const uint16_t* W, const float* bias, const float* residual,
                          const OutDesc& od, int M, int N, int K, int epilogue, const LinearExtras& ex, int T) {
    const int rpi = 64 / T;
    const int ngroups = (N + rpi - 1) / rpi;
    constexpr int max_blocks = 2048;
    int blocks = (ngroups + 3) / 4;
    if (blocks > max_blocks) blocks = max_blocks;
    const size_t lds = (size_t)MT * K * sizeof(float);
    switch (T) {
        case 32:
            hipLaunchKernelGGL((k_gemv_valu<MT, 32>), dim3(blocks), dim3(256), lds, s, x, W, bias, residual, od, M,
                               N, K, epilogue, ex);
            break;
        case 16:
            hipLaunchKernelGGL((k_gemv_valu<MT, 16>), dim3(blocks), dim3(256), lds, s, x, W, bias, residual, od, M,
                               N, K, epilogue, ex);
            break;
        default:
            hipLaunchKernelGGL((k_gemv_valu<MT, 8>), dim3(blocks), dim3(256), lds, s, x, W, bias, residual, od, M,
                               N, K, epilogue, ex);
            break;
    }
    count(CNT_GEMV);
    return check_launch("gemv_valu");
}

// Lanes per row for the VALU GEMV: the largest of 32/16/8 dividing K/8;
// 0 when K fits none (then the MFMA kernel runs).
static int valu_lanes_per_row(int K) {
    const int chunks = K / 8;
    for (int t = 32; t >= 8; t >>= 1)
        if (chunks % t == 0) return t;
    return 0;
}

// Launch plan: NT weight tiles and NW K-splitting waves per block, chosen
// from a sweep of the decode shapes (GPT-2 small and XL, M = 1..16) on
// MI355X.
struct GemvPlan {
    int nt, nw, u;
};

static GemvPlan plan_gemv(int M, int N, int K) {
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
    } else if (ntiles >= 128 && K <= 1024) {  // 2048..4095 rows over a short K
        p.nt = 1;
        p.nw = 4;
        p.u = M <= 4 ? 4 : 2;
    } else {                       // narrow N: deep K split inside the block
        p.nt = 1;
        p.nw = 8;
        p.u = M == 1 ? 4 : 2;
    }
    // keep at least one 32-wide k-step per wave
    while (p.nw > 1 && (K + p.nw - 1) / p.nw < 32) p.nw /= 2;
    return p;
}

template <int NT, int NW, int U>
static void launch_t(hipStream_t s, dim3 grid, const float* x, const uint16_t* W, const float* bias,
                     const float* residual, const OutDesc& od, int M, int N, int K, int kw, int epilogue,
                     const LinearExtras& ex) {
    if (ex.ln_g)
        hipLaunchKernelGGL((k_linear_bf16_mfma<NT, NW, U, true>), grid, dim3(NW * 64), 0, s, x, W, bias, residual,
                           od, M, N, K, kw, epilogue, ex);
    else
        hipLaunchKernelGGL((k_linear_bf16_mfma<NT, NW, U, false>), grid, dim3(NW * 64), 0, s, x, W, bias, residual,
                           od, M, N, K, kw, epilogue, ex);
}

int launch_linear_bf16(hipStream_t s, const float* x, const uint16_t* W, const float* bias,
                       const float* residual, float* y, int M, int N, int K, int epilogue) {
    return launch_linear_bf16_od(s, x, W, bias, residual, OutDesc::plain(y, N), M, N, K, epilogue,
                                 LinearExtras{});
}

int launch_gemm_bf16w(hipStream_t s, const float* A, const uint16_t* W, const float* bias,
                      const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                      bool act_bf16);

// The in-block-split MFMA GEMV; with ex.part the grid's y dimension is the
// K slice and the kernel writes raw partial sums.
static int launch_mfma_gemv(hipStream_t s, const float* x, const uint16_t* W, const float* bias,
                            const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                            const LinearExtras& ex_in) {
    LinearExtras ex = ex_in;
    GemvPlan p = plan_gemv(M, N, K);
    int span = K, gy = (M + 15) / 16;
    if (ex.part) {
        // more tiles per block: each block's activation slice then feeds
        // more weight rows
        const int split_nt = ex.split_nt ? ex.split_nt : 4;
        if ((N + 15) / 16 >= 4 * split_nt) p.nt = split_nt;
        ex.kslice = ((K + ex.ksplit - 1) / ex.ksplit + 31) / 32 * 32;
        span = ex.kslice;
        gy = (K + ex.kslice - 1) / ex.kslice;
        ex.ksplit = gy;
        // about one 64-wide load group (U = 2) per wave and slice
        while (p.nw > 1 && (span + p.nw - 1) / p.nw < 64) p.nw /= 2;
        p.u = 2;
    }
    // the double-buffered load groups spill beyond these (NW * U) sizes
    if (p.nw >= 8 && p.u > 4) p.u = 4;
    if (p.nw >= 16 && p.u > 2) p.u = 2;
    int per = (span + p.nw - 1) / p.nw;
    int kw = (per + 31) / 32 * 32;
    dim3 grid((N + 16 * p.nt - 1) / (16 * p.nt), gy);
#define GH_CASE(T, WV, UV)                                                                   \
    if (p.nt == T && p.nw == WV && p.u == UV) {                                              \
        launch_t<T, WV, UV>(s, grid, x, W, bias, residual, od, M, N, K, kw, epilogue, ex);   \
        count(M <= 16 ? CNT_GEMV : CNT_GEMM);                                                \
        return check_launch("linear_bf16");                                                  \
    }
#define GH_CASES_U(T, WV) GH_CASE(T, WV, 2) GH_CASE(T, WV, 4) GH_CASE(T, WV, 8)
#define GH_CASES_W(T) \
    GH_CASES_U(T, 1) GH_CASES_U(T, 2) GH_CASES_U(T, 4) GH_CASE(T, 8, 2) GH_CASE(T, 8, 4) GH_CASE(T, 16, 2)
    GH_CASES_W(1) GH_CASES_W(2) GH_CASES_W(4) GH_CASE(8, 1, 2) GH_CASE(8, 2, 2) GH_CASE(8, 4, 2)
#undef GH_CASES_W
#undef GH_CASES_U
#undef GH_CASE
    set_error("linear_bf16: unsupported tile plan");
    return GORCH_HIP_EUNSUPPORTED;
}


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
    if (ex.part) {
        if (M > 16 || ex.ksplit < 1) {
            set_error("linear_bf16: K-split partials need 1 <= M <= 16");
            return GORCH_HIP_EUNSUPPORTED;
        }
        return launch_mfma_gemv(s, x, W, bias, residual, od, M, N, K, epilogue, ex);
    }
    // 2..16 rows over a narrow weight (few 16-row tiles) and a long K: split
    // K across blocks into partials in the stream's scratch, then one small
    // epilogue kernel (a CU streams only ~20 GB/s, so 48..128 tiles alone
    // cannot pull the weight at full rate). Wider weights stay unsplit:
    // 8-tile K-slice blocks measured slower at 16 rows (12.5 vs 9.4 us at
    // K 1600, N 4800) once the epilogue kernel is counted.
    constexpr int split_blocks = 300;
    constexpr int split_max_tiles = 128;
    constexpr int split_nt_wide = 2;
    const int ntiles_all = (N + 15) / 16;
    if (M >= 2 && !ex.argmax_key && ntiles_all < split_max_tiles && K >= 1024) {
        const int nt = ntiles_all >= 128 ? split_nt_wide : 2;
        const int blocks_per_slice = (ntiles_all + nt - 1) / nt;
        const int S = ksplit_slices(K, std::min(kEpiSlices, std::max(2, split_blocks / blocks_per_slice)));
        void* part = nullptr;
        if (S >= 2) {
            const size_t need = (size_t)S * M * N * sizeof(float);
            if (ex.scratch && need > ex.scratch_bytes) {
                set_error("linear_bf16: the K split needs " + std::to_string(need) + " bytes of scratch, above the " +
                          std::to_string(ex.scratch_bytes) + "-byte maximum");
                return GORCH_HIP_EINVAL;
            }
            part = ex.scratch ? ex.scratch : stream_scratch(s, need);
        }
        if (part) {
            LinearExtras sx = ex;
            sx.part = static_cast<float*>(part);
            sx.ksplit = S;
            sx.split_nt = nt;
            GH_TRY(launch_mfma_gemv(s, x, W, nullptr, nullptr, OutDesc::plain(nullptr, N), M, N, K,
                                    GORCH_HIP_EPI_NONE, sx));
            return launch_splitk_epilogue(s, sx.part, S, M, N, bias, residual, od, epilogue);
        }
    }
    // M = 1: the register-activation kernel whenever K fits its shape table
    // (K/8 = T*C with C <= 8), else the LDS-staged VALU kernel.
    if (ex.pair_swiglu) {
        // paired [gate | up] rows: two rows per wave (32 lanes each)
        if (M != 1 || !gemv_pair_swiglu_ok(ex.pair_swiglu, K) || N != 2 * ex.pair_swiglu || bias || residual ||
            epilogue != GORCH_HIP_EPI_NONE || ex.argmax_key || ex.swiglu) {
            set_error("linear_bf16: paired SwiGLU rows need one row, K a multiple of 256 up to 2048, no epilogue");
            return GORCH_HIP_EUNSUPPORTED;
        }
        return launch_m1(s, x, W, nullptr, nullptr, od, N, K, GORCH_HIP_EPI_NONE, ex, 32, K / 256);
    }
    if (M == 1) {
        int T1, C1;
        m1_shape(K, &T1, &C1);
        if (T1) {
            int rc = launch_m1(s, x, W, bias, residual, od, N, K, epilogue, ex, T1, C1);
            if (rc >= 0) return rc;
        }
    }
    if (ex.ln_rms || ex.swiglu) {
        set_error("linear_bf16: the RMSNorm / SwiGLU prologues need one row with K/8 = T*C (T in 8..64, C <= 8)");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if (M >= 2 && (N + 15) / 16 >= 1024) {
        int rc = launch_mt(s, x, W, bias, residual, od, M, N, K, epilogue, ex);
        if (rc >= 0) return rc;
    }
    const int T = valu_lanes_per_row(K);
    // one row whose K the register kernel's shape table does not take: the
    // LDS-staged VALU kernel (2..16 rows run on the matrix cores)
    if (M == 1 && T && (size_t)4 * K * sizeof(float) <= 64 * 1024)
        return launch_valu_mt<1>(s, x, W, bias, residual, od, M, N, K, epilogue, ex, T);
    return launch_mfma_gemv(s, x, W, bias, residual, od, M, N, K, epilogue, ex);
}

// Tile-packed weights: W [N, K] bf16 row-major -> ceil(N/16) tiles of
// ceil(K/32) 1 KB fragments, each in v_mfma_f32_16x16x32_bf16 B-operand
// lane order (lane l: row l % 16, k 8*(l/16) .. +8 of the 32-wide step),
// zero beyond N and K. A wave then reads every fragment as one contiguous
// 1 KB; row-major B fragments touch 16 rows K*2 bytes apart per load, which
// on MI355X streams at ~60-70% of the rate (measured 7.6 vs 5.3 us for a
// 15.4 MB weight at K = 1600).
size_t packed_bf16_elems(int N, int K) { return (size_t)((N + 15) / 16) * 16 * (size_t)((K + 31) & ~31); }

__global__ __launch_bounds__(256) void k_pack_bf16_tiles(const uint16_t* __restrict__ W, uint16_t* __restrict__ Wp,
                                                         int N, int K, long long chunks) {
    const long long c = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= chunks) return;
    const int nks = (K + 31) / 32;
    const int l = (int)(c & 63);
    const long long f = c >> 6;  // fragment index = tile * nks + k-step
    const int t = (int)(f / nks), j = (int)(f - (long long)t * nks);
    const int row = 16 * t + (l & 15), k0 = 32 * j + 8 * (l >> 4);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < N && k0 < K) v = *reinterpret_cast<const uint4*>(W + (size_t)row * K + k0);
    *reinterpret_cast<uint4*>(Wp + (size_t)c * 8) = v;
}

int launch_pack_bf16(hipStream_t s, const uint16_t* W, uint16_t* Wp, int N, int K) {
    const long long chunks = (long long)packed_bf16_elems(N, K) / 8;
    if (chunks == 0) return GORCH_HIP_OK;
    hipLaunchKernelGGL(k_pack_bf16_tiles, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, s, W, Wp, N, K,
                       chunks);
    return check_launch("pack_bf16");
}

// K slices of a K-split packed GEMV: about 32 k-steps (1024 of K) per slice
// and at least ~192 blocks in all, at most 8 slices (measured best at
// K = 1600 / 3072 / 6400 over 1600 / 768 / 1600 rows: 7.2 / 7.1 / 10.9 us at
// 16 rows against 7.7 / 7.2 / 15.6 us for the row-major split).
int packed_split_slices(int K, int N) {
    // blocks a K split aims at (3072x768 at M = 4 / 16 with 4-wave blocks:
    // 192 -> 384 took 5.16 / 5.77 to 5.05 / 5.50 us)
    constexpr int split_target = 384;
    const int ksteps = (K + 31) / 32, ntiles = (N + 15) / 16;
    int S = std::max((ksteps + 31) / 32, (split_target + ntiles - 1) / ntiles);
    S = std::min(std::min(S, kEpiSlices), std::max(1, ksteps / 3));
    return ksplit_slices(K, S);
}

// Linear over tile-packed weights, 1 <= M <= 16 (the decode GEMV).
int launch_linear_packed_od(hipStream_t s, const float* x, const uint16_t* Wp, const float* bias,
                            const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                            const LinearExtras& ex) {
    if (M < 1 || M > 16 || ((ex.part || ex.accumulate) && (ex.argmax_key || ex.ln_g)) || (ex.ln_g && ex.ln_stats) ||
        (ex.accumulate && (ex.part || residual || epilogue != GORCH_HIP_EPI_NONE))) {
        set_error("linear_bf16_packed: needs 1 <= M <= 16, no argmax or LayerNorm with a K split");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if ((ex.x_frag && ex.ln_g) || (ex.out_frag && (!ex.x_frag || ex.part || ex.accumulate || ex.argmax_key))) {
        set_error("linear_bf16_packed: fragment-layout activations take no fused LayerNorm, and a fragment-layout "
                  "output needs fragment-layout activations, no K split and no argmax");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if (ex.part || ex.accumulate) {
        // caller-owned partials (the engine's row reducer sums them), or
        // slices added into the output
        LinearExtras sx = ex;
        sx.kslice = ((K + ex.ksplit - 1) / ex.ksplit + 31) / 32 * 32;
        sx.ksplit = (K + sx.kslice - 1) / sx.kslice;
        const int rc = ex.accumulate
                           ? launch_tiles(s, x, Wp, bias, nullptr, od, M, N, K, GORCH_HIP_EPI_NONE, sx)
                           : launch_tiles(s, x, Wp, nullptr, nullptr, OutDesc::plain(nullptr, N), M, N, K,
                                          GORCH_HIP_EPI_NONE, sx);
        if (rc < 0) set_error("linear_bf16_packed: K slice above 3072 is not supported");
        return rc < 0 ? GORCH_HIP_EUNSUPPORTED : rc;
    }
    // a narrow weight (few 16-row tiles) over a long K: split K across blocks
    // into the stream's scratch, then the ordered epilogue kernel (a CU
    // streams ~25 GB/s, so 48..127 tiles alone leave most of the chip idle)
    const int ntiles = (N + 15) / 16;
    if (!ex.argmax_key && !ex.ln_g && !ex.out_frag && ntiles < 128 && K >= 1024) {
        const int S = packed_split_slices(K, N);
        void* part = S >= 2 ? stream_scratch(s, (size_t)S * M * N * sizeof(float)) : nullptr;
        if (part) {
            LinearExtras sx = ex;
            sx.part = static_cast<float*>(part);
            sx.kslice = ((K + S - 1) / S + 31) / 32 * 32;
            sx.ksplit = (K + sx.kslice - 1) / sx.kslice;
            const int rc = launch_tiles(s, x, Wp, nullptr, nullptr, OutDesc::plain(nullptr, N), M, N, K,
                                        GORCH_HIP_EPI_NONE, sx);
            if (rc >= 0) {
                GH_TRY(rc);
                return launch_splitk_epilogue(s, sx.part, sx.ksplit, M, N, bias, residual, od, epilogue);
            }
        }
    }
    const int rc = launch_tiles(s, x, Wp, bias, residual, od, M, N, K, epilogue, ex);
    if (rc < 0) {
        set_error(ex.ln_g ? "linear_bf16_packed: a fused LayerNorm needs K <= 1024"
                          : "linear_bf16_packed: K above 3072 is not supported");
        return GORCH_HIP_EUNSUPPORTED;
    }
    return rc;
}

}  // namespace gh
