// gemm_wide.h — a wide-tile MFMA main loop for the MoE expert GEMMs.
//
//   acc[b] = A[rows, K] x W_b[cols, K]^T   (b < NB weights, BNW columns each)
//
// A arrives as bf16 planes (hi, and lo when SPLIT: x = hi + lo, ~2^-16
// relative), written once by the producer kernel, so the main loop only
// moves bytes: every global load and LDS store is 16 bytes. W is bf16 in the
// nn.Linear [out, in] layout.
//
// Measured on MI355X (MoE gate/up GEMM, 2048 tokens x top-2, d 1024, ffn
// 4096): the matrix cores and LDS together take most of the time — with the
// global loads switched off 163 of 180 us, with the MFMAs switched off 127
// us (global -> LDS alone, ~16 B/clock per CU, 73% L2 hits) — and the MFMAs
// run at ~42% of their measured 2.05 PFLOP/s peak. Wide tiles (128 rows x up
// to 256 weight columns on WGM x WGN waves, each a region of 16x16
// v_mfma_f32_16x16x32_bf16 accumulators) bound the L2 traffic (A re-read
// once per column tile, W once per row tile) and the LDS fragment reads per
// MFMA; 16 waves (4 x 4) measured faster than 8 (2 x 4): four waves per SIMD
// cover one another's LDS round trips. 64-wide K stages read whole 128-byte
// cache lines (a 32-wide stage reads half a line per row and fetches every
// line twice).
//
// Pipeline: LDS is double-buffered and registers hold two stages, so stage
// i+3's loads are issued while stage i runs on the matrix cores; one barrier
// per stage. The loads are raw buffer loads, branch-free: rows and columns
// past the tile's edge are clamped into it (computed, never stored) and a
// K-tail chunk gets an out-of-range offset, which the buffer unit returns as
// zeros. A load under a branch (or a flat load) would make the compiler wait
// for every outstanding load (vmcnt(0)) before the next LDS store, draining
// the prefetch each stage. K % 8 == 0. LDS rows are unpadded with
// XOR-swizzled 16-byte chunks (no bank conflicts).
#pragma once
#include <type_traits>
#include "common.h"

namespace gh {

template <int BM, int BNW, int NB, bool SPLIT, int BK = 64, bool IL = false, int WGM = 2, int WGN = 4, int PD = 2>
struct WideGemm {
    static constexpr int kThreads = 64 * WGM * WGN;  // WGM (rows) x WGN (columns) waves
    static constexpr int CH = BK / 8;                // 16-byte chunks per row and stage
    static constexpr int NA = SPLIT ? 2 : 1;
    static constexpr int WM = BM / WGM, WNW = BNW / WGN;
    static constexpr int TM = WM / 16, TN = WNW / 16;
    static constexpr int A_U4 = NA * BM * CH / kThreads;  // 16-byte loads per thread per stage
    static constexpr int W_U4 = NB * BNW * CH / kThreads;
    static_assert(BK == 32 || BK == 64, "stage width");
    static_assert(A_U4 >= 1 && W_U4 >= 1 && TM >= 1 && TN >= 1, "tile too small");
    static_assert(NA * BM * CH % kThreads == 0 && NB * BNW * CH % kThreads == 0, "uneven loads");
    // each load instruction stays inside one plane / weight (uniform resource)
    static_assert((BM * CH) % kThreads == 0 && (BNW * CH) % kThreads == 0, "plane split across a load");

    // Chunk c of LDS row `row` sits at c ^ (row & 7) (64-wide rows) or
    // c ^ ((row >> 1) & 3) (32-wide rows): conflict-free for both the row
    // stores and the 16-row fragment reads (measured on gfx950).
    __device__ static __forceinline__ int swz(int row, int c) {
        return BK == 64 ? (c ^ (row & 7)) : (c ^ ((row >> 1) & 3));
    }

    struct Smem {
        uint16_t a[2][NA][BM][BK];
        uint16_t w[2][NB][BNW][BK];
    };

    // a[p] + row * lda: row of plane p (nrows valid); w[b] + n * K: column n
    // of weight b (ncols valid). Sums k in [kb, ke) (a K slice; kb % 8 ==
    // 0). Per valid output, xform(row, col, vals[NB]) finishes the values in
    // place (it may load), then store(row, col, vals) writes them: every
    // xform runs before the first store, since stores and loads share one
    // memory counter and a load's use after a store would wait for the
    // store's write.
    template <class Xform, class Store>
    __device__ static void run(Smem& sm, const uint16_t* const* a, long long lda, int nrows,
                               const uint16_t* const* w, int ncols, int K, int kb, int ke, Xform& xform,
                               Store& store) {
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int wm = wave / WGN, wn = wave % WGN;
        const int r = lane & 15, g = lane >> 4;
        const int nk = (ke - kb + BK - 1) / BK;

        // one buffer resource per plane / weight, covering the tile's rows
        __amdgpu_buffer_rsrc_t rsa[NA], rsw[NB];
#pragma unroll
        for (int p = 0; p < NA; p++) rsa[p] = make_rsrc(a[p], (long long)nrows * lda * 2);
#pragma unroll
        for (int b = 0; b < NB; b++) rsw[b] = make_rsrc(w[b], (long long)ncols * K * 2);

        u32x4 ra[PD][A_U4], rw[PD][W_U4];
        auto gload = [&](int st, u32x4 (&ar)[A_U4], u32x4 (&wr)[W_U4]) {
            const int k0 = kb + st * BK;
#pragma unroll
            for (int i = 0; i < A_U4; i++) {
                const int idx = tid + kThreads * i;
                const int p = kThreads * i / (BM * CH), rem = idx % (BM * CH), row = rem / CH, c = rem % CH;
                const int k = k0 + 8 * c;
                const int off = k < ke ? (min(row, nrows - 1) * (int)lda + k) * 2 : kOutOfRange;
                ar[i] = __builtin_amdgcn_raw_buffer_load_b128(rsa[p], off, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < W_U4; i++) {
                const int idx = tid + kThreads * i;
                const int b = kThreads * i / (BNW * CH), rem = idx % (BNW * CH), row = rem / CH, c = rem % CH;
                const int k = k0 + 8 * c;
                const int off = k < ke ? (min(row, ncols - 1) * K + k) * 2 : kOutOfRange;
                wr[i] = __builtin_amdgcn_raw_buffer_load_b128(rsw[b], off, 0, 0);
            }
        };
        auto sstore = [&](int buf, const u32x4 (&ar)[A_U4], const u32x4 (&wr)[W_U4]) {
#pragma unroll
            for (int i = 0; i < A_U4; i++) {
                const int idx = tid + kThreads * i;
                const int p = kThreads * i / (BM * CH), rem = idx % (BM * CH), row = rem / CH, c = rem % CH;
                *reinterpret_cast<u32x4*>(&sm.a[buf][p][row][8 * swz(row, c)]) = ar[i];
            }
#pragma unroll
            for (int i = 0; i < W_U4; i++) {
                const int idx = tid + kThreads * i;
                const int b = kThreads * i / (BNW * CH), rem = idx % (BNW * CH), row = rem / CH, c = rem % CH;
                *reinterpret_cast<u32x4*>(&sm.w[buf][b][row][8 * swz(row, c)]) = wr[i];
            }
        };

        floatx4 acc[NB][TM][TN];
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) acc[b][i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

        auto compute = [&](int buf) {
#pragma unroll
            for (int kk = 0; kk < BK / 32; kk++) {
                bf16x8 bfr[NB][TN];
#pragma unroll
                for (int b = 0; b < NB; b++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        bfr[b][j] = *reinterpret_cast<const bf16x8*>(
                            &sm.w[buf][b][wn * WNW + j * 16 + r][8 * swz(r, 4 * kk + g)]);
#pragma unroll
                for (int i = 0; i < TM; i++) {
#pragma unroll
                    for (int p = 0; p < NA; p++) {
                        const bf16x8 af = *reinterpret_cast<const bf16x8*>(
                            &sm.a[buf][p][wm * WM + i * 16 + r][8 * swz(r, 4 * kk + g)]);
#pragma unroll
                        for (int b = 0; b < NB; b++)
#pragma unroll
                            for (int j = 0; j < TN; j++) acc[b][i][j] = mfma16x16x32(af, bfr[b][j], acc[b][i][j]);
                    }
                }
            }
        };

        // IL: one stage as an interleaved schedule. The fragments of both
        // 32-wide halves of the stage are read up front; the second half's
        // reads are spread between the first half's MFMAs, and the next
        // stage's LDS writes and global loads between the second half's, so
        // the matrix cores wait less on LDS round trips (measured: the MoE
        // gate/up GEMM 191 -> 183 us, down 119 -> 110 us).
        struct Frag {
            bf16x8 b[NB][TN];
            bf16x8 a[TM][NA];
        };
        auto read_frags = [&](int buf, int kk, Frag& f) {
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    f.b[b][j] = *reinterpret_cast<const bf16x8*>(
                        &sm.w[buf][b][wn * WNW + j * 16 + r][8 * swz(r, 4 * kk + g)]);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int p = 0; p < NA; p++)
                    f.a[i][p] = *reinterpret_cast<const bf16x8*>(
                        &sm.a[buf][p][wm * WM + i * 16 + r][8 * swz(r, 4 * kk + g)]);
        };
        auto mfmas = [&](const Frag& f) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int p = 0; p < NA; p++)
#pragma unroll
                    for (int b = 0; b < NB; b++)
#pragma unroll
                        for (int j = 0; j < TN; j++) acc[b][i][j] = mfma16x16x32(f.a[i][p], f.b[b][j], acc[b][i][j]);
        };
        constexpr int NFR = NB * TN + TM * NA;   // fragment reads per half
        constexpr int NMF = TM * NA * NB * TN;   // MFMAs per half
        constexpr int NLD = A_U4 + W_U4;         // LDS writes (and global loads) per stage
        static_assert(!IL || (BK == 64 && NMF >= NFR && NMF >= 2 * NLD), "interleave shape");
        auto stage_il = [&](int buf, u32x4 (&ar)[A_U4], u32x4 (&wr)[W_U4], int next) {
            Frag f0, f1;
            read_frags(buf, 0, f0);
            read_frags(buf, 1, f1);
            mfmas(f0);
            sstore(buf ^ 1, ar, wr);
            gload(next, ar, wr);
            mfmas(f1);
            // scheduling groups (mask 0x100 LDS reads, 0x008 MFMAs, 0x200
            // LDS writes, 0x020 global loads): f0's reads; f1's reads spread
            // between f0's MFMAs; the next stage's writes and loads between
            // f1's MFMAs
            __builtin_amdgcn_sched_group_barrier(0x100, NFR, 0);
#pragma unroll
            for (int q = 0; q < NFR; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, NMF / NFR, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NMF - NFR * (NMF / NFR), 0);
#pragma unroll
            for (int q = 0; q < NLD; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
            }
#pragma unroll
            for (int q = 0; q < NLD; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NMF - 2 * NLD, 0);
            __syncthreads();
        };

        // A wave whose rows all lie past nrows (the tail tile of an expert)
        // computes nothing that is stored: it still moves its share of the
        // stage's loads and meets every barrier, but reads no fragments and
        // issues no MFMAs, leaving its SIMD's matrix core to the live waves.
        auto stage_idle = [&](int buf, u32x4 (&ar)[A_U4], u32x4 (&wr)[W_U4], int next) {
            sstore(buf ^ 1, ar, wr);
            gload(next, ar, wr);
            __syncthreads();
        };
        // wave-uniform by construction (scalar registers), so the choice is
        // a scalar branch and each wave meets the same barriers in either arm
        const int wave_s = __builtin_amdgcn_readfirstlane(tid >> 6);
        const bool live = (wave_s / WGN) * WM < __builtin_amdgcn_readfirstlane(nrows);

        // stage s lives in register set s % 2 until it is stored to LDS
        // buffer s % 2; stage s + 3 is requested once stage s + 1 has left
        // its registers. The body is unconditional (stages past K load
        // zeros; an odd stage count runs one all-zero stage) so the compiler
        // can keep the newer stage's loads in flight across the wait.
        const int nk2 = (nk + 1) & ~1;
        auto main_loop = [&](auto live_tag) {
            constexpr bool LIVE = decltype(live_tag)::value;
            auto stage = [&](int buf, u32x4 (&ar)[A_U4], u32x4 (&wr)[W_U4], int next) {
                if constexpr (!LIVE) {
                    stage_idle(buf, ar, wr, next);
                } else if constexpr (IL) {
                    stage_il(buf, ar, wr, next);
                } else {
                    compute(buf);
                    sstore(buf ^ 1, ar, wr);
                    gload(next, ar, wr);
                    __syncthreads();
                }
            };
            if constexpr (PD == 1) {
                // one register set: stage s + 2 is requested as stage s + 1
                // leaves it (one stage of load latency covered)
                gload(0, ra[0], rw[0]);
                sstore(0, ra[0], rw[0]);
                gload(1, ra[0], rw[0]);
                __syncthreads();
                for (int it = 0; it < nk2; it += 2) {
                    stage(0, ra[0], rw[0], it + 2);
                    stage(1, ra[0], rw[0], it + 3);
                }
            } else {
                gload(0, ra[0], rw[0]);
                gload(1, ra[1], rw[1]);
                sstore(0, ra[0], rw[0]);
                gload(2, ra[0], rw[0]);
                __syncthreads();
                for (int it = 0; it < nk2; it += 2) {
                    stage(0, ra[1], rw[1], it + 3);
                    stage(1, ra[0], rw[0], it + 4);
                }
            }
        };
        if (live)
            main_loop(std::true_type{});
        else
            main_loop(std::false_type{});

        // lane holds rows 4g..4g+3 of column r in each 16x16 fragment
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int col = wn * WNW + j * 16 + r;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int row = wm * WM + i * 16 + 4 * g + v;
                    float vals[NB];
#pragma unroll
                    for (int b = 0; b < NB; b++) vals[b] = acc[b][i][j][v];
                    if (row < nrows && col < ncols) xform(row, col, vals);
#pragma unroll
                    for (int b = 0; b < NB; b++) acc[b][i][j][v] = vals[b];
                }
            }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int col = wn * WNW + j * 16 + r;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int row = wm * WM + i * 16 + 4 * g + v;
                    float vals[NB];
#pragma unroll
                    for (int b = 0; b < NB; b++) vals[b] = acc[b][i][j][v];
                    if (row < nrows && col < ncols) store(row, col, vals);
                }
            }
    }
};

}  // namespace gh
