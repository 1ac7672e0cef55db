// gemm.hip — BF16-weight Linear for prefill- and MoE-sized M (M > 16):
//   C[m,n] = residual[m,n] + epi( sum_k A[m,k] * W[n,k] + bias[n] )
// with A f32 [M,K], W bf16 [N,K] (the nn.Linear layout, nn/module.go:61-88).
//
// Two kernels, both staging 64-wide K steps of A (converted from f32 as it
// is written to LDS) and W through LDS into v_mfma_f32_16x16x32_bf16:
//   k_gemm_bf16w: 128 x 128 tiles of 4 waves (2 x 2 waves of 64 x 64), for
//     problems with at least 256 such tiles (long prefills);
//   k_gemm_db: 64-row tiles of 64, 96 or 128 columns on 2 x (2..4) waves of
//     32 x 32, double-buffered LDS, for the few-tile shapes of a short
//     prefill (512 x 768 x 2304: 72 tiles of 128 x 128).
// Later steps' global loads (raw buffer loads, no branches) are issued into
// registers before the current step's MFMAs so memory latency overlaps the
// math. LDS rows are padded to 160 bytes, which makes the 16-byte fragment
// reads conflict-free on gfx950 (a 144-byte row measured 2-way conflicted).
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

// Bias of the wave's TN output columns (column nb + 16 j + r), loaded
// before the main loop; zeros without a bias or past N (a buffer resource
// of size 0 or an out-of-range offset, no branch).
template <int TN>
__device__ __forceinline__ void gemm_bias(const float* bias, int N, int nb, int r, float (&bn)[TN]) {
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bias, bias ? (long long)N * 4 : 0);
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = nb + j * 16 + r;
        bn[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, n < N ? n * 4 : kOutOfRange, 0, 0));
    }
}

// Epilogue kinds (template argument EPI of the GEMM kernels): bit 0 the
// tanh GELU, bit 1 a residual input. A residual decided at run time costs
// ~0.4 us at 512 x 768 x 2304 even when absent, so it is compiled in or out.
constexpr int kEpiGelu = 1, kEpiResidual = 2;
inline int epi_kind(int epilogue, const float* residual) {
    return (epilogue == GORCH_HIP_EPI_GELU ? kEpiGelu : 0) | (residual ? kEpiResidual : 0);
}

// Epilogue of a wave's TM x TN accumulators (16 x 16 MFMA tiles; lane
// (r, g) holds rows 4g .. 4g+3 of column r of each): out = residual +
// epi(acc + bias), written through the output descriptor. mb / nb: the
// wave's first row relative to the block's m0 and its first column. The
// residual is loaded and every value finished before the first store (a
// load after a store waits for the store's write: both count on vmcnt),
// and the bias is added unconditionally (bn reads zeros without one).
template <int TM, int TN, int EPI>
__device__ __forceinline__ void gemm_epilogue(floatx4 (&acc)[TM][TN], const float (&bn)[TN], const float* residual, const OutDesc& od, int pos, int M, int N,
                                              int m0, int mrows, int mb, int nb, int r, int g) {
    constexpr bool GELU = (EPI & kEpiGelu) != 0, RES = (EPI & kEpiResidual) != 0;
    float res[TM][TN][4];
    if constexpr (RES) {
        const __amdgpu_buffer_rsrc_t rsr = make_rsrc(residual + (size_t)m0 * N, (long long)mrows * N * 4);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = nb + j * 16 + r;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int ml = mb + i * 16 + 4 * g + v;
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
                // bn is zero without a bias (a select here costs ~0.2 us)
                float s = acc[i][j][v] + bn[j];
                if constexpr (GELU) s = gelu_tanh(s);
                if constexpr (RES) s = res[i][j][v] + s;
                acc[i][j][v] = s;
            }
    // One output segment without per-sequence rows (every Linear but the
    // fused QKV projection): row m at ptr + (m + pos?) * row_stride. The
    // descriptor's general addressing costs ~1.4 us at 512 x 768 x 2304.
    if (od.nseg == 1 && od.rows_per_seq >= (1 << 30) && od.row_stride[0] < (1ll << 31)) {
        const int rs = __builtin_amdgcn_readfirstlane((int)od.row_stride[0]);
        float* base = od.ptr[0] + (long long)(m0 + (od.use_pos[0] ? pos : 0)) * rs;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = nb + j * 16 + r;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int ml = mb + i * 16 + 4 * g + v;
                    if (ml < mrows && n < N) base[(size_t)ml * rs + n] = acc[i][j][v];
                }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = nb + j * 16 + r;
        const OutDesc::Col c = od.col(min(n, N - 1), pos);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = m0 + mb + i * 16 + 4 * g + v;
                if (m < M && n < N) *od.row(c, m) = acc[i][j][v];
            }
    }
}

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

// Linear for M > 16 when 128 x 128 tiles would not fill the chip (prefill of
// a few hundred rows: 512 x 768 x {2304, 3072} gives 72..96 such tiles):
// 64 x BN tiles (BN = 32 * WGN) on 2 x WGN waves, each wave a 32 x 32
// sub-tile of 2 x 2 MFMA accumulators. The block's A and W K-steps (64
// wide) go global -> registers -> one of two LDS stage buffers, so each
// step has a single barrier: step i computes from buffer i & 1 while the
// registers of step i + 1 are written into the other buffer. The loads of
// step i + 2 go out at the top of step i (its register set was emptied
// into LDS during step i - 1), so they have two steps to arrive, and the
// LDS writes of step i + 1 are kept after step i's MFMAs (a wait for their
// loads placed between the MFMAs stalls them). The last two steps issue no
// loads; with KT the K tail and the padding step read zeros.
template <int WGN, bool SPLIT, bool KT, int EPI>
__global__ __launch_bounds__(128 * WGN) void k_gemm_db(const float* __restrict__ A, const uint16_t* __restrict__ W,
                                                       const float* __restrict__ bias, const float* residual,
                                                       OutDesc od, int M, int N, int K) {
    constexpr int BM = 64, BN = 32 * WGN, NT = 128 * WGN;
    constexpr int NA = SPLIT ? 2 : 1;
    constexpr int TM = 2, TN = 2;
    constexpr int A_TOT = BM * kBK / 4, W_TOT = BN * kBK / 8;  // float4 / uint4 chunks per step
    constexpr int A_F4 = (A_TOT + NT - 1) / NT, W_U4 = (W_TOT + NT - 1) / NT;
    constexpr int STAGE = (NA * BM + BN) * kLDA;  // bf16 elements per stage buffer
    __shared__ __align__(16) uint16_t lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int mrows = min(BM, M - m0), ncols = min(BN, N - n0);
    const __amdgpu_buffer_rsrc_t rsa = make_rsrc(A + (size_t)m0 * K, (long long)mrows * K * 4);
    const __amdgpu_buffer_rsrc_t rsw = make_rsrc(W + (size_t)n0 * K, (long long)ncols * K * 2);
    // Chunk q of a step: A row q / 16, float4 column q % 16; W row q / 8,
    // uint4 column q % 8. Threads past the chunk count (WGN = 3) repeat the
    // last chunk: the same value to the same LDS slot. Rows past M or N are
    // clamped into the tile (computed, never stored).
    float4 ra[2][A_F4];
    uint4 rw[2][W_U4];
    auto gload = [&](int k0, float4 (&a)[A_F4], uint4 (&wv)[W_U4]) {
#pragma unroll
        for (int i = 0; i < A_F4; i++) {
            const int q = min(tid + NT * i, A_TOT - 1), row = q >> 4, k = k0 + 4 * (q & 15);
            const int off = (!KT || k < K) ? (min(row, mrows - 1) * K + k) * 4 : kOutOfRange;
            a[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsa, off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < W_U4; i++) {
            const int q = min(tid + NT * i, W_TOT - 1), row = q >> 3, k = k0 + 8 * (q & 7);
            const int off = (!KT || k < K) ? (min(row, ncols - 1) * K + k) * 2 : kOutOfRange;
            wv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsw, off, 0, 0));
        }
    };
    auto sstore = [&](int b, const float4 (&a)[A_F4], const uint4 (&wv)[W_U4]) {
        uint16_t* As = lds + b * STAGE;
        uint16_t* Ws = As + NA * BM * kLDA;
#pragma unroll
        for (int i = 0; i < A_F4; i++) {
            const int q = min(tid + NT * i, A_TOT - 1), row = q >> 4, c4 = q & 15;
            const float f[4] = {a[i].x, a[i].y, a[i].z, a[i].w};
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (SPLIT) {
                    const uint32_t u = __float_as_uint(f[e]) & 0xffff0000u;
                    hi[e] = (uint16_t)(u >> 16);
                    lo[e] = __builtin_bit_cast(uint16_t, (__bf16)(f[e] - __uint_as_float(u)));
                } else {
                    hi[e] = __builtin_bit_cast(uint16_t, (__bf16)f[e]);
                }
            }
            *reinterpret_cast<uint2*>(&As[row * kLDA + 4 * c4]) =
                make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
            if (SPLIT)
                *reinterpret_cast<uint2*>(&As[(BM + row) * kLDA + 4 * c4]) =
                    make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
        }
#pragma unroll
        for (int i = 0; i < W_U4; i++) {
            const int q = min(tid + NT * i, W_TOT - 1), row = q >> 3, c8 = q & 7;
            *reinterpret_cast<uint4*>(&Ws[row * kLDA + 8 * c8]) = wv[i];
        }
    };
    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, g = lane >> 4;
    auto compute = [&](int b) {
        const uint16_t* As = lds + b * STAGE;
        const uint16_t* Ws = As + NA * BM * kLDA;
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 32) {
            bf16x8 bfr[TN];
#pragma unroll
            for (int j = 0; j < TN; j++)
                bfr[j] = *reinterpret_cast<const bf16x8*>(&Ws[(wn * 32 + j * 16 + r) * kLDA + kk + 8 * g]);
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const bf16x8 ahi = *reinterpret_cast<const bf16x8*>(&As[(wm * 32 + i * 16 + r) * kLDA + kk + 8 * g]);
#pragma unroll
                for (int j = 0; j < TN; j++) acc[i][j] = mfma16x16x32(ahi, bfr[j], acc[i][j]);
                if (SPLIT) {
                    const bf16x8 alo =
                        *reinterpret_cast<const bf16x8*>(&As[(BM + wm * 32 + i * 16 + r) * kLDA + kk + 8 * g]);
#pragma unroll
                    for (int j = 0; j < TN; j++) acc[i][j] = mfma16x16x32(alo, bfr[j], acc[i][j]);
                }
            }
        }
    };
    float bn[TN];
    gemm_bias<TN>(bias, N, n0 + wn * 32, r, bn);
    const int pos = __builtin_amdgcn_readfirstlane(od.pos_dev ? *od.pos_dev : 0);
    // steps padded to an even count (a padding step reads zeros, KT)
    const int nk = (K + kBK - 1) / kBK;
    const int nkp = (nk + 1) & ~1;
    gload(0, ra[0], rw[0]);
    __builtin_amdgcn_sched_barrier(0);
    gload(kBK, ra[1], rw[1]);
    __builtin_amdgcn_sched_barrier(0);
    sstore(0, ra[0], rw[0]);
    __syncthreads();
    auto step = [&](int s, int it, bool st, bool ld) {
        if (ld) gload((it + 2) * kBK, ra[s], rw[s]);
        compute(it & 1);
        __builtin_amdgcn_sched_barrier(0);
        if (st) sstore((it + 1) & 1, ra[s ^ 1], rw[s ^ 1]);
        __syncthreads();
    };
    int it0 = 0;
    for (; it0 < nkp - 2; it0 += 2) {
        step(0, it0, true, true);
        step(1, it0 + 1, true, true);
    }
    step(0, it0, true, false);
    step(1, it0 + 1, false, false);

    gemm_epilogue<TM, TN, EPI>(acc, bn, residual, od, pos, M, N, m0, mrows, wm * 32, n0 + wn * 32, r, g);
}

// Tile width for k_gemm_db: the most 64-row blocks that still fit one
// round on the chip (measured at 512 x 768: N = 2304 on 64 x 96, 192
// blocks, 7.1 us; N = 3072 on 64 x 96, 256 blocks, 7.4 us, against 7.5 /
// 7.6 us on 64 x 128), the widest when every width exceeds it.
static int db_waves(int M, int N) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            n = 256;
        return n;
    }();
    const long long mb = (M + 63) / 64;
    int best = 4;
    long long best_blocks = 0;
    for (int w = 4; w >= 2; w--) {
        const long long blocks = mb * ((N + 32 * w - 1) / (32 * w));
        if (blocks <= cus && blocks > best_blocks) {
            best = w;
            best_blocks = blocks;
        }
    }
    return best;
}

template <int WGN, bool SPLIT>
static void launch_db_t(hipStream_t s, const float* A, const uint16_t* W, const float* bias, const float* residual,
                        const OutDesc& od, int M, int N, int K, int epilogue) {
    dim3 grid((N + 32 * WGN - 1) / (32 * WGN), (M + 63) / 64);
    const int nk = (K + kBK - 1) / kBK;
    const bool kt = K % kBK != 0 || nk % 2 != 0;
#define GH_DB_L(KTV, EV) \
    hipLaunchKernelGGL((k_gemm_db<WGN, SPLIT, KTV, EV>), grid, dim3(128 * WGN), 0, s, A, W, bias, residual, od, M, N, K)
#define GH_DB_E(KTV)                               \
    switch (epi_kind(epilogue, residual)) {        \
        case 0: GH_DB_L(KTV, 0); break;            \
        case kEpiGelu: GH_DB_L(KTV, kEpiGelu); break; \
        case kEpiResidual: GH_DB_L(KTV, kEpiResidual); break; \
        default: GH_DB_L(KTV, kEpiGelu | kEpiResidual); break; \
    }
    if (kt) GH_DB_E(true)
    else GH_DB_E(false)
#undef GH_DB_E
#undef GH_DB_L
}

template <bool SPLIT>
static void launch_db(hipStream_t s, const float* A, const uint16_t* W, const float* bias, const float* residual,
                      const OutDesc& od, int M, int N, int K, int epilogue) {
    switch (db_waves(M, N)) {
        case 2: launch_db_t<2, SPLIT>(s, A, W, bias, residual, od, M, N, K, epilogue); break;
        case 3: launch_db_t<3, SPLIT>(s, A, W, bias, residual, od, M, N, K, epilogue); break;
        default: launch_db_t<4, SPLIT>(s, A, W, bias, residual, od, M, N, K, epilogue); break;
    }
}

template <int BM, int BN, bool SPLIT>
static void launch_gemm_t(hipStream_t s, const float* A, const uint16_t* W, const float* bias,
                          const float* residual, const OutDesc& od, int M, int N, int K, int epilogue) {
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    // one register stage for 128 x 128 tiles (more stages cost occupancy:
    // 4096^3 247 vs 301 us); no K tail: loads with no bound on k (a select
    // on every offset compiles to branches around the loads)
    constexpr int pf = 1;
    if (K % kBK != 0)
        hipLaunchKernelGGL((k_gemm_bf16w<BM, BN, SPLIT, pf, true>), grid, dim3(256), 0, s, A, W, bias, residual, od, M,
                           N, K, epilogue);
    else
        hipLaunchKernelGGL((k_gemm_bf16w<BM, BN, SPLIT, pf, false>), grid, dim3(256), 0, s, A, W, bias, residual, od,
                           M, N, K, epilogue);
}

// Tile choice: 128 x 128 tiles (k_gemm_bf16w) when they give every CU a
// block, else the double-buffered 64-row kernel (k_gemm_db).
int launch_gemm_bf16w(hipStream_t s, const float* A, const uint16_t* W, const float* bias,
                      const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                      bool act_bf16) {
    const long long big = (long long)((M + 127) / 128) * ((N + 127) / 128);
    if (big < 256) {
        if (act_bf16) launch_db<false>(s, A, W, bias, residual, od, M, N, K, epilogue);
        else launch_db<true>(s, A, W, bias, residual, od, M, N, K, epilogue);
    } else if (act_bf16) {
        launch_gemm_t<128, 128, false>(s, A, W, bias, residual, od, M, N, K, epilogue);
    } else {
        launch_gemm_t<128, 128, true>(s, A, W, bias, residual, od, M, N, K, epilogue);
    }
    count(CNT_GEMM);
    return check_launch("gemm_bf16w");
}

}  // namespace gh
