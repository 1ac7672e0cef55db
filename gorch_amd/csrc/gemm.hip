// gemm.hip — BF16-weight Linear for prefill- and MoE-sized M (M > 16):
//   C[m,n] = residual[m,n] + epi( sum_k A[m,k] * W[n,k] + bias[n] )
// with A f32 [M,K], W bf16 [N,K] (the nn.Linear layout, nn/module.go:61-88).
//
// Block tile BM x BN, K stepped by 64. 256 threads = 4 waves in a 2x2 grid,
// each wave owning a (BM/2) x (BN/2) sub-tile of 16x16 MFMA accumulators
// (v_mfma_f32_16x16x32_bf16). Each K step stages the A tile (converted from
// f32 as it is written to LDS) and the W tile in LDS; later steps' global
// loads (raw buffer loads, no branches) are issued into registers before the
// current step's MFMAs so memory latency overlaps the math. LDS rows are
// padded to 160 bytes, which makes the 16-byte fragment reads conflict-free
// on gfx950 (a 144-byte row measured 2-way conflicted).
//
// Activation modes:
//   split (default): A = hi + lo in bf16 (two MFMAs per fragment pair),
//     ~2^-16 relative, i.e. f32-activation accuracy like the reference's
//     widen + f32 sgemm (bf16_matmul.go:166-173);
//   bf16 (GORCH_HIP_LINEAR_ACT_BF16): A rounded to bf16 (RNE), one MFMA —
//     the bf16 x bf16 -> f32 MPSGraph path (metal/shim.m:808-857).
#include "common.h"

namespace gh {

constexpr int kBK = 64;
constexpr int kLDA = kBK + 16;  // bf16 elements per LDS row (160 bytes: conflict-free 16-byte fragment reads)

template <int BM, int BN, bool SPLIT, int PF, bool KT>
__global__ __launch_bounds__(256) void k_gemm_bf16w(const float* __restrict__ A, const uint16_t* __restrict__ W,
                                                    const float* __restrict__ bias, const float* residual,
                                                    OutDesc od, int M, int N, int K, int epilogue) {
    constexpr int NA = SPLIT ? 2 : 1;
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 16, TN = WN / 16;
    constexpr int A_F4 = BM * kBK / 4 / 256;  // float4 loads of A per thread
    constexpr int W_U4 = BN * kBK / 8 / 256;  // uint4 loads of W per thread
    __shared__ __align__(16) uint16_t As[NA][BM][kLDA];
    __shared__ __align__(16) uint16_t Ws[BN][kLDA];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    // PF register stages: the loads of K-step i + PF are issued as soon as
    // step i has been written to LDS, so PF steps of latency are in flight.
    // Raw buffer loads over the block's rows, branch-free: rows past M or N
    // are clamped into the tile (computed, never stored) and a K-tail chunk
    // gets an out-of-range offset, which reads as zeros. (A load under a
    // branch makes the compiler drain every outstanding load before each
    // LDS store, so no prefetch would survive a step.)
    const int mrows = min(BM, M - m0), ncols = min(BN, N - n0);
    const __amdgpu_buffer_rsrc_t rsa = make_rsrc(A + (size_t)m0 * K, (long long)mrows * K * 4);
    const __amdgpu_buffer_rsrc_t rsw = make_rsrc(W + (size_t)n0 * K, (long long)ncols * K * 2);
    float4 ra[PF][A_F4];
    uint4 rw[PF][W_U4];
    auto gload = [&](int k0, float4 (&a)[A_F4], uint4 (&wv)[W_U4]) {
#pragma unroll
        for (int i = 0; i < A_F4; i++) {
            const int idx = tid + 256 * i, row = idx >> 4, c4 = idx & 15;
            const int k = k0 + 4 * c4;
            const int off = (!KT || k < K) ? (min(row, mrows - 1) * K + k) * 4 : kOutOfRange;
            a[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsa, off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < W_U4; i++) {
            const int idx = tid + 256 * i, row = idx >> 3, c8 = idx & 7;
            const int k = k0 + 8 * c8;
            const int off = (!KT || k < K) ? (min(row, ncols - 1) * K + k) * 2 : kOutOfRange;
            wv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsw, off, 0, 0));
        }
    };
    auto sstore = [&](const float4 (&a)[A_F4], const uint4 (&wv)[W_U4]) {
#pragma unroll
        for (int i = 0; i < A_F4; i++) {
            const int idx = tid + 256 * i, row = idx >> 4, c4 = idx & 15;
            const float f[4] = {a[i].x, a[i].y, a[i].z, a[i].w};
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (SPLIT) {
                    uint32_t u = __float_as_uint(f[e]) & 0xffff0000u;
                    hi[e] = (uint16_t)(u >> 16);
                    lo[e] = __builtin_bit_cast(uint16_t, (__bf16)(f[e] - __uint_as_float(u)));
                } else {
                    hi[e] = __builtin_bit_cast(uint16_t, (__bf16)f[e]);
                }
            }
            uint2 h2 = make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
            *reinterpret_cast<uint2*>(&As[0][row][4 * c4]) = h2;
            if (SPLIT) {
                uint2 l2 = make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
                *reinterpret_cast<uint2*>(&As[NA - 1][row][4 * c4]) = l2;
            }
        }
#pragma unroll
        for (int i = 0; i < W_U4; i++) {
            const int idx = tid + 256 * i, row = idx >> 3, c8 = idx & 7;
            *reinterpret_cast<uint4*>(&Ws[row][8 * c8]) = wv[i];
        }
    };

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int r = lane & 15, g = lane >> 4;
    // the epilogue's bias values, loaded while the main loop runs
    float bn[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + wn * WN + j * 16 + r;
        bn[j] = (bias && n < N) ? bias[n] : 0.f;
    }
    // the step count is padded to a multiple of PF (padding steps read
    // zeros) so the loop body has no branch around its loads
    const int nk = (K + kBK - 1) / kBK;
    const int nkp = (nk + PF - 1) / PF * PF;
    // issue the stages in order: the loop waits for stage s while later
    // stages stay in flight (memory counters complete in issue order), and
    // the scheduler would otherwise interleave the prologue's loads
#pragma unroll
    for (int s = 0; s < PF; s++) {
        gload(s * kBK, ra[s], rw[s]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int it0 = 0; it0 < nkp; it0 += PF) {
#pragma unroll
        for (int s = 0; s < PF; s++) {
            const int it = it0 + s;
            __syncthreads();  // previous step's fragment reads are done
            sstore(ra[s], rw[s]);
            __syncthreads();
            gload((it + PF) * kBK, ra[s], rw[s]);
#pragma unroll
            for (int kk = 0; kk < kBK; kk += 32) {
                bf16x8 bfr[TN];
#pragma unroll
                for (int j = 0; j < TN; j++)
                    bfr[j] = *reinterpret_cast<const bf16x8*>(&Ws[wn * WN + j * 16 + r][kk + 8 * g]);
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const bf16x8 ahi = *reinterpret_cast<const bf16x8*>(&As[0][wm * WM + i * 16 + r][kk + 8 * g]);
#pragma unroll
                    for (int j = 0; j < TN; j++) acc[i][j] = mfma16x16x32(ahi, bfr[j], acc[i][j]);
                    if (SPLIT) {
                        const bf16x8 alo =
                            *reinterpret_cast<const bf16x8*>(&As[NA - 1][wm * WM + i * 16 + r][kk + 8 * g]);
#pragma unroll
                        for (int j = 0; j < TN; j++) acc[i][j] = mfma16x16x32(alo, bfr[j], acc[i][j]);
                    }
                }
            }
        }
    }

    // Epilogue. Stores and loads share one memory counter, so a loaded value
    // first used after a store makes that use wait for the store's write
    // too (and, past a branch, for every store before it): the position and
    // the residual are loaded and every output value computed before the
    // first store.
    const int pos = __builtin_amdgcn_readfirstlane(od.pos_dev ? *od.pos_dev : 0);
    float res[TM][TN][4];
    if (residual) {
        const __amdgpu_buffer_rsrc_t rsr = make_rsrc(residual + (size_t)m0 * N, (long long)mrows * N * 4);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = n0 + wn * WN + j * 16 + r;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int ml = wm * WM + i * 16 + 4 * g + v;
                    const int off = (n < N && ml < mrows) ? (ml * N + n) * 4 : kOutOfRange;
                    res[i][j][v] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsr, off, 0, 0));
                }
            }
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float s = acc[i][j][v];
                if (bias) s = s + bn[j];
                if (epilogue == GORCH_HIP_EPI_GELU) s = gelu_tanh(s);
                if (residual) s = res[i][j][v] + s;
                acc[i][j][v] = s;
            }
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + wn * WN + j * 16 + r;
        const OutDesc::Col c = od.col(min(n, N - 1), pos);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = m0 + wm * WM + i * 16 + 4 * g + v;
                if (m < M && n < N) *od.row(c, m) = acc[i][j][v];
            }
    }
}

template <int BM, int BN, bool SPLIT>
static void launch_gemm_t(hipStream_t s, const float* A, const uint16_t* W, const float* bias,
                          const float* residual, const OutDesc& od, int M, int N, int K, int epilogue) {
    static const int pf_env = [] {
        const char* e = getenv("GORCH_HIP_GEMM_PF");
        return e ? atoi(e) : 0;
    }();
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    // measured: one register stage for 128 x 128 tiles (more stages cost
    // occupancy: 4096^3 247 vs 301 us), two for the smaller tiles
    const int pf = pf_env ? pf_env : (BM * BN >= 128 * 128 ? 1 : 2);
    // no K tail and a step count the stages divide: loads with no bound on k
    // (a select on every offset compiles to branches around the loads)
    const int nk = (K + kBK - 1) / kBK;
    const bool kt = K % kBK != 0 || nk % pf != 0;
#define GH_GEMM_L(PFV, KTV)                                                                                    \
    hipLaunchKernelGGL((k_gemm_bf16w<BM, BN, SPLIT, PFV, KTV>), grid, dim3(256), 0, s, A, W, bias, residual, od, M, \
                       N, K, epilogue)
    if (pf == 1) {
        if (kt) GH_GEMM_L(1, true);
        else GH_GEMM_L(1, false);
    } else if (pf == 2) {
        if (kt) GH_GEMM_L(2, true);
        else GH_GEMM_L(2, false);
    } else {
        if (kt) GH_GEMM_L(3, true);
        else GH_GEMM_L(3, false);
    }
#undef GH_GEMM_L
}

// Tile choice: the largest tile that still gives every CU a block.
int launch_gemm_bf16w(hipStream_t s, const float* A, const uint16_t* W, const float* bias,
                      const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                      bool act_bf16) {
    const long long big = (long long)((M + 127) / 128) * ((N + 127) / 128);
    const long long mid = (long long)((M + 63) / 64) * ((N + 127) / 128);
    int tile = big >= 256 ? 2 : (mid >= 256 ? 1 : 0);
    static const int tile_env = [] {
        const char* e = getenv("GORCH_HIP_GEMM_TILE");
        return e ? atoi(e) : -1;
    }();
    if (tile_env >= 0) tile = tile_env;
    if (act_bf16) {
        if (tile == 2) launch_gemm_t<128, 128, false>(s, A, W, bias, residual, od, M, N, K, epilogue);
        else if (tile == 1) launch_gemm_t<64, 128, false>(s, A, W, bias, residual, od, M, N, K, epilogue);
        else launch_gemm_t<64, 64, false>(s, A, W, bias, residual, od, M, N, K, epilogue);
    } else {
        if (tile == 2) launch_gemm_t<128, 128, true>(s, A, W, bias, residual, od, M, N, K, epilogue);
        else if (tile == 1) launch_gemm_t<64, 128, true>(s, A, W, bias, residual, od, M, N, K, epilogue);
        else launch_gemm_t<64, 64, true>(s, A, W, bias, residual, od, M, N, K, epilogue);
    }
    count(CNT_GEMM);
    return check_launch("gemm_bf16w");
}

}  // namespace gh
