// moe.hip — the MoE FFN layer of nn.MoE.Forward (nn/moe.go:130-182):
// router logits -> top-K (index_ops.go:153-186) -> softmax over the K
// values with exp in f64 (softmaxRows, nn/moe.go:247-268) -> tokens grouped
// per expert in token order (:143-149) -> per expert Gather -> Wgate, Wup
// Linears -> SwiGLU -> Wdown Linear -> x routing weight -> ScatterAdd,
// experts accumulated in ascending index (:155-180).
//
// On the GPU (one stream, no host round trip, no allocation):
//   k_moe_topk       one thread per token: top-K and the routing weights;
//   k_moe_route      one block: stable counting sort of the (token, slot)
//                    assignments by expert, the inverse map, and the tile
//                    table of the grouped GEMMs;
//   k_moe_gather_split packs each expert's rows contiguously (Xg), as bf16
//                    hi/lo planes for the wide-tile GEMMs (gemm_wide.h);
//   grouped GEMM 1   H = SwiGLU(Xg We_gate^T + bg, Xg We_up^T + bu): gate and
//                    up tiles accumulate side by side, SwiGLU in the epilogue;
//   grouped GEMM 2   Yg = (H We_down^T + bd) * w(row), the routing weight
//                    applied in the epilogue (the reference's Mul);
//   k_moe_combine    out[t] = sum of the token's rows in ascending expert order.
// Expert weights are stacked [E][out][in] bf16 in one device array each.
#include <algorithm>

#include "common.h"
#include "gemm_wide.h"

namespace gh {

// The tile table's row unit for sizing: at most M*K / kMoeBM + E + 1 row
// tiles (the grouped GEMMs take 128-row tiles, kWideBM, so fewer are used).
constexpr int kMoeBM = 64;
constexpr int kMaxExperts = 64;
constexpr int kDownSlices = 2;  // K slices of the wide down GEMM at most
constexpr int kMaxTopK = 8;

struct MoeWs {
    float* logits;   // [M, E] router output (injected logits are read in place)
    int* topi;       // [M, K]
    float* topw;     // [M, K]
    int* perm_tok;   // [M*K] token of packed row p
    float* perm_w;   // [M*K] routing weight of packed row p
    int* inv;        // [M, K] packed row of (token, slot)
    int* tile_e;     // [max_tiles] expert of m-tile i
    int* tile_r0;    // [max_tiles] first packed row
    int* tile_n;     // [max_tiles] rows in the tile
    int* ntiles;     // [1]
    float* xg;       // [M*K, dim]
    float* h;        // [M*K, ffn]
    float* yg;       // [kDownSlices][M*K, dim] (slice 0 only when unsplit)
};

static size_t al(size_t b) { return (b + 255) & ~(size_t)255; }

static size_t moe_layout(int M, int dim, int ffn, int E, int K, char* base, MoeWs* ws) {
    const size_t MK = (size_t)M * K;
    const size_t max_tiles = MK / kMoeBM + E + 1;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off += al(bytes);
        return base ? base + o : nullptr;
    };
    MoeWs w;
    w.logits = (float*)take((size_t)M * E * 4);
    w.topi = (int*)take(MK * 4);
    w.topw = (float*)take(MK * 4);
    w.perm_tok = (int*)take(MK * 4);
    w.perm_w = (float*)take(MK * 4);
    w.inv = (int*)take(MK * 4);
    w.tile_e = (int*)take(max_tiles * 4);
    w.tile_r0 = (int*)take(max_tiles * 4);
    w.tile_n = (int*)take(max_tiles * 4);
    w.ntiles = (int*)take(4);
    w.xg = (float*)take(MK * dim * 4);
    w.h = (float*)take(MK * ffn * 4);
    w.yg = (float*)take(kDownSlices * MK * dim * 4);
    if (ws) *ws = w;
    return off;
}

// One thread per token: top-K of the router logits (descending; ties keep
// the lower index first, and a NaN never replaces the running best, as in
// the reference's > compare) and the routing weights, softmaxRows over the
// K values: max, exp in f64 rounded to f32, f32 sum, divide. Written to the
// workspace and, when given, to the caller's arrays.
// The top-K of one token (EV >= E logits, KT >= K slots): the logits come
// through raw buffer loads over the whole [M, E] table, all in flight at
// once (slots past E read the next row or, past the table, zeros, and are
// never selected; a load under a branch would be waited on before the
// next one, one round trip per expert). M * E < 2^29 (host check).
template <int EV, int KT>
__device__ __forceinline__ void moe_topk_token(__amdgpu_buffer_rsrc_t rl, int tok, int E, int K, int (&idx)[KT],
                                               float (&wgt)[KT]) {
    float lv[EV];
#pragma unroll
    for (int j = 0; j < EV; j++)
        lv[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rl, (tok * E + j) * 4, 0, 0));
    float val[KT];
    unsigned long long taken = 0ull;
#pragma unroll
    for (int s = 0; s < KT; s++) {
        idx[s] = -1;
        val[s] = 0.f;
        if (s >= K) continue;
        int best = -1;
        float bv = 0.f;
#pragma unroll
        for (int j = 0; j < EV; j++) {
            if (j >= E || ((taken >> j) & 1ull)) continue;
            if (best < 0 || lv[j] > bv) {
                best = j;
                bv = lv[j];
            }
        }
        idx[s] = best;
        val[s] = bv;
        taken |= 1ull << best;
    }
    float mx = val[0];
#pragma unroll
    for (int s = 1; s < KT; s++)
        if (s < K) mx = val[s] > mx ? val[s] : mx;
    float e_[KT];
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < KT; s++) {
        e_[s] = 0.f;
        if (s < K) {
            e_[s] = (float)exp((double)(val[s] - mx));
            sum += e_[s];
        }
    }
#pragma unroll
    for (int s = 0; s < KT; s++) wgt[s] = s < K ? e_[s] / sum : 0.f;
}

template <int EV>
__global__ __launch_bounds__(256) void k_moe_topk(const float* __restrict__ logits, int M, int E, int K,
                                                  int* __restrict__ topi, float* __restrict__ topw,
                                                  int* __restrict__ topi_out, float* __restrict__ topw_out) {
    const int tok = blockIdx.x * blockDim.x + threadIdx.x;
    if (tok >= M) return;
    int idx[kMaxTopK];
    float wgt[kMaxTopK];
    moe_topk_token<EV, kMaxTopK>(make_rsrc(logits, (long long)M * E * 4), tok, E, K, idx, wgt);
#pragma unroll
    for (int s = 0; s < kMaxTopK; s++)
        if (s < K) {
            const size_t a = (size_t)tok * K + s;
            topi[a] = idx[s];
            topw[a] = wgt[s];
            if (topi_out) topi_out[a] = idx[s];
            if (topw_out) topw_out[a] = wgt[s];
        }
}

// One 1024-thread block over the top-K table; thread t takes tokens t,
// t + 1024, ... (rounds). Per round: the token's rank inside each chosen
// expert's group — earlier rounds' counts, then the counts of lower waves
// and lower lanes of this round from wavefront ballots — so the grouping is
// stable in token order like the reference's per-expert token lists. Ranks
// are parked in inv; once every expert's size is known the bases, the GEMM
// tile table (one thread per expert) and the packed-row maps follow.
constexpr int kRouteThreads = 1024, kRouteWaves = kRouteThreads / 64;
// EV > 0: the block takes each token's top-K itself (moe_topk_token, E <=
// EV) and writes the tables and the caller's arrays as k_moe_topk does.
template <int KT, int EV = 0>
__global__ __launch_bounds__(kRouteThreads) void k_moe_route(int M, int E, int K, int tile_rows, MoeWs ws,
                                                             const float* __restrict__ logits, int* topi_out,
                                                             float* topw_out) {
    __shared__ int wtot[kRouteWaves][kMaxExperts];
    __shared__ int wpre[kRouteWaves][kMaxExperts];
    __shared__ int run[kMaxExperts];
    __shared__ int base[kMaxExperts + 1];
    __shared__ int tbase[kMaxExperts + 1];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const unsigned long long lt_mask = (1ull << lane) - 1ull;
    if (t < E) run[t] = 0;
    __syncthreads();
    // up to RR rounds keep their slots' experts, ranks and weights in
    // registers for the final scatter (no second read of the tables); fewer
    // rounds with more slots, within the 128 registers of a 1024-thread block
    constexpr int RR = KT <= 2 ? 4 : 1;
    const bool regs = M <= RR * kRouteThreads;
    int ridx[RR][KT], rrank[RR][KT];
    float rw[RR][KT];
    int round = 0;
    for (int r0 = 0; r0 < M; r0 += kRouteThreads, round++) {
        const int tok = r0 + t;
        const bool live = tok < M;
        int idx[KT];
        float wv[KT];
        if constexpr (EV > 0) {
            moe_topk_token<EV, KT>(make_rsrc(logits, (long long)M * E * 4), live ? tok : 0, E, K, idx, wv);
#pragma unroll
            for (int s = 0; s < KT; s++) {
                if (!live) idx[s] = -1;
                if (live && s < K) {
                    const size_t a = (size_t)tok * K + s;
                    ws.topi[a] = idx[s];
                    ws.topw[a] = wv[s];
                    if (topi_out) topi_out[a] = idx[s];
                    if (topw_out) topw_out[a] = wv[s];
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < KT; s++) idx[s] = (live && s < K) ? ws.topi[(size_t)tok * K + s] : -1;
#pragma unroll
            for (int s = 0; s < KT; s++) wv[s] = (regs && live && s < K) ? ws.topw[(size_t)tok * K + s] : 0.f;
        }
        // this round's per-wave counts and lane prefixes, expert by expert
        int pre[KT];
#pragma unroll
        for (int s = 0; s < KT; s++) pre[s] = 0;
        for (int e = 0; e < E; e++) {
            bool mine = false;
#pragma unroll
            for (int s = 0; s < KT; s++) mine |= (idx[s] == e);
            const unsigned long long bits = __ballot(mine);
            if (lane == 0) wtot[wave][e] = __popcll(bits);
            const int lp = __popcll(bits & lt_mask);
#pragma unroll
            for (int s = 0; s < KT; s++)
                if (idx[s] == e) pre[s] = lp;
        }
        __syncthreads();
        // per expert: the ranks lower waves of this round take (after the
        // earlier rounds' run), and the run advanced past this round
        if (t < E) {
            int acc = run[t];
            for (int w = 0; w < kRouteWaves; w++) {
                wpre[w][t] = acc;
                acc += wtot[w][t];
            }
            run[t] = acc;
        }
        __syncthreads();
        if (live)
#pragma unroll
            for (int s = 0; s < KT; s++) {
                if (s >= K) break;
                const int e = idx[s];
                const int rank = wpre[wave][e] + pre[s];
                if (regs) {
#pragma unroll
                    for (int q = 0; q < RR; q++)
                        if (q == round) {
                            ridx[q][s] = e;
                            rrank[q][s] = rank;
                            rw[q][s] = wv[s];
                        }
                } else {
                    ws.inv[(size_t)tok * K + s] = rank;  // rank inside expert e for now
                }
            }
    }
    __syncthreads();
    if (t == 0) {
        int b = 0, nt = 0;
        for (int e = 0; e < E; e++) {
            base[e] = b;
            tbase[e] = nt;
            b += run[e];
            nt += (run[e] + tile_rows - 1) / tile_rows;
        }
        base[E] = b;
        tbase[E] = nt;
        *ws.ntiles = nt;
    }
    __syncthreads();
    if (t < E) {
        const int n = run[t];
        for (int r = 0, i = tbase[t]; r < n; r += tile_rows, i++) {
            ws.tile_e[i] = t;
            ws.tile_r0[i] = base[t] + r;
            ws.tile_n[i] = min(tile_rows, n - r);
        }
    }
    if (regs) {
#pragma unroll
        for (int q = 0; q < RR; q++) {
            const int tok = t + q * kRouteThreads;
            if (tok >= M) break;
#pragma unroll
            for (int s = 0; s < KT; s++) {
                if (s >= K) break;
                const size_t a = (size_t)tok * K + s;
                const int p = base[ridx[q][s]] + rrank[q][s];
                ws.perm_tok[p] = tok;
                ws.perm_w[p] = rw[q][s];
                ws.inv[a] = p;
            }
        }
        return;
    }
    for (int tok = t; tok < M; tok += kRouteThreads)
        for (int s = 0; s < K; s++) {
            const size_t a = (size_t)tok * K + s;
            const int p = base[ws.topi[a]] + ws.inv[a];
            ws.perm_tok[p] = tok;
            ws.perm_w[p] = ws.topw[a];
            ws.inv[a] = p;
        }
}

// out[t] = sum over the token's K packed rows in ascending expert order
// (the reference adds each expert's ScatterAdd contribution in order). One
// thread per (token, 4 columns); dim % 4 == 0. nsl > 1: the down GEMM left
// raw K-slice partials, and a row's value is ((sum of slices) + bias) * w.
// out[t] = the token's K expert rows summed in ascending expert order
// (nn/moe.go:155-180). KT >= K slots: the token's expert indices and packed
// rows are loaded together, sorted in registers, then every row's chunk is
// loaded at once (raw buffer loads, unused slots out of range), so a chunk
// costs two dependent round trips. With nsl > 1 K slices of the down GEMM
// the slices, bias and routing weight are added here.
template <int KT>
__global__ void k_moe_combine(const float* __restrict__ yg, const int* __restrict__ inv,
                              const int* __restrict__ topi, float* out, int M, int K, int dim, int nsl,
                              long long cslice, const float* __restrict__ bdown,
                              const float* __restrict__ perm_w) {
    const int d4 = dim / 4;
    const long long MK = (long long)M * K;
    const __amdgpu_buffer_rsrc_t rt = make_rsrc(topi, MK * 4);
    const __amdgpu_buffer_rsrc_t ri = make_rsrc(inv, MK * 4);
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(yg, MK * dim * 4);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (int64_t)M * d4;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(i / d4), c = (int)(i - (int64_t)t * d4);
        int e[KT], p[KT], order[KT];
#pragma unroll
        for (int s = 0; s < KT; s++) {
            const int off = s < K ? (t * K + s) * 4 : kOutOfRange;
            e[s] = (int)__builtin_amdgcn_raw_buffer_load_b32(rt, off, 0, 0);
            p[s] = (int)__builtin_amdgcn_raw_buffer_load_b32(ri, off, 0, 0);
            order[s] = s;
        }
#pragma unroll
        for (int a = 1; a < KT; a++)  // insertion sort of the slots by expert index
#pragma unroll
            for (int b = a; b > 0; b--) {
                const bool sw = b < K && e[order[b]] < e[order[b - 1]];
                const int lo = sw ? order[b] : order[b - 1], hi = sw ? order[b - 1] : order[b];
                order[b - 1] = lo;
                order[b] = hi;
            }
        float4 v[KT];
#pragma unroll
        for (int s = 0; s < KT; s++) {
            const int q = order[s];
            int pq = p[0];
#pragma unroll
            for (int u = 1; u < KT; u++) pq = q == u ? p[u] : pq;
            const int off = s < K ? (pq * dim + 4 * c) * 4 : kOutOfRange;
            v[s] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ry, off, 0, 0));
            if (nsl > 1 && s < K) {
                int eq = e[0];
#pragma unroll
                for (int u = 1; u < KT; u++) eq = q == u ? e[u] : eq;
                for (int z = 1; z < nsl; z++) {
                    const float4 w = reinterpret_cast<const float4*>(yg + z * cslice + (size_t)pq * dim)[c];
                    v[s].x = v[s].x + w.x;
                    v[s].y = v[s].y + w.y;
                    v[s].z = v[s].z + w.z;
                    v[s].w = v[s].w + w.w;
                }
                if (bdown) {
                    const float4 b = reinterpret_cast<const float4*>(bdown + (size_t)eq * dim)[c];
                    v[s].x = v[s].x + b.x;
                    v[s].y = v[s].y + b.y;
                    v[s].z = v[s].z + b.z;
                    v[s].w = v[s].w + b.w;
                }
                const float wgt = perm_w[pq];  // weighted = exOut * w
                v[s].x = v[s].x * wgt;
                v[s].y = v[s].y * wgt;
                v[s].z = v[s].z * wgt;
                v[s].w = v[s].w * wgt;
            }
        }
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int s = 0; s < KT; s++)
            if (s < K) {
                acc.x = acc.x + v[s].x;
                acc.y = acc.y + v[s].y;
                acc.z = acc.z + v[s].z;
                acc.w = acc.w + v[s].w;
            }
        reinterpret_cast<float4*>(out)[i] = acc;
    }
}

// Wide-tile path. The gather writes Xg as two bf16 planes (hi, lo: x = hi +
// lo to ~2^-16 relative, the split the MFMA kernels use) in the space of the
// f32 Xg, and GEMM 1's epilogue writes H the same way, so both GEMMs load
// 16-byte bf16 words only. Rows are grouped in 128-row tiles. The down GEMM
// keeps 256-wide tiles although at d = 1024 that leaves half the CUs idle:
// 128-wide tiles on every CU measured slower (148 vs 121 us, 2048 tokens).
// Splitting the down GEMM's K over twice the blocks (raw partials, summed
// with bias and routing weight by the combine) measured within noise of the
// unsplit kernel (118 vs 121 us): these GEMMs are bound by the traffic from
// beyond L2, not by the number of busy CUs. (64 x 64 tiles over f32
// activations were slower than these 128-row bf16 hi/lo tiles.)
constexpr int kWideBM = 128, kWideBNDual = 128, kWideBNDown = 256;

// Token-major: item (t, chunk c) loads x's chunk and the token's K packed
// rows (inv) together — no load waits on another — splits once and stores
// the planes at each of the K rows.
template <int KT>
__global__ void k_moe_gather_split(const float* __restrict__ x, const int* __restrict__ inv, uint16_t* hi,
                                   uint16_t* lo, int M, int K, int dim) {
    const int d8 = dim / 8;
    const __amdgpu_buffer_rsrc_t ri = make_rsrc(inv, (long long)M * K * 4);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (int64_t)M * d8;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(i / d8), c = (int)(i - (int64_t)t * d8);
        int p[KT];
#pragma unroll
        for (int s = 0; s < KT; s++)
            p[s] = (int)__builtin_amdgcn_raw_buffer_load_b32(ri, s < K ? (t * K + s) * 4 : kOutOfRange, 0, 0);
        const float4* src = reinterpret_cast<const float4*>(x + (size_t)t * dim + 8 * c);
        const float4 u = src[0], v = src[1];
        const float f[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
        bf16x8 h, l;
        split_hi_lo(f, h, l);
#pragma unroll
        for (int s = 0; s < KT; s++)
            if (s < K) {
                *reinterpret_cast<bf16x8*>(hi + (size_t)p[s] * dim + 8 * c) = h;
                *reinterpret_cast<bf16x8*>(lo + (size_t)p[s] * dim + 8 * c) = l;
            }
    }
}

// blockIdx.y = 128-row tile of the table, blockIdx.x = BNW output columns.
// A: planes (hi, lo) of [rows, Kd]. DUAL: gate and up side by side, H =
// SwiGLU(gate, up) written as planes (Chi, Clo); else C = (acc + b) * w(row)
// in f32.
// Staged epilogue (STG): the finished tile goes to LDS first (the stage
// buffers are free once the main loop's last barrier has passed), then out
// in 16-byte row chunks, instead of one 2- or 4-byte store per element
// straight from the accumulators.
template <bool DUAL, int BNW>
struct MoeStage {
    // padded rows: conflict-free element writes. DUAL: one u32 per element,
    // hi in the high half and lo in the low half
    static constexpr int LDH = BNW + 4, LDC = BNW + 4;
    static constexpr size_t kBytes = DUAL ? (size_t)kWideBM * LDH * 4 : (size_t)kWideBM * LDC * 4;
};

template <bool DUAL, int BNW, bool IL = false, int WGM = 2, int PD = 2, bool STG = false>
__global__ __launch_bounds__(WGM * 256) void k_moe_wide(const uint16_t* __restrict__ Ahi, const uint16_t* __restrict__ Alo,
                                                  const uint16_t* __restrict__ W1, const uint16_t* __restrict__ W2,
                                                  const float* __restrict__ b1, const float* __restrict__ b2,
                                                  float* __restrict__ C, uint16_t* __restrict__ Chi,
                                                  uint16_t* __restrict__ Clo, int N, int Kd, long long cslice,
                                                  int xcd_map, MoeWs ws) {
    using G = WideGemm<kWideBM, BNW, DUAL ? 2 : 1, true, 64, IL, WGM, 4, PD>;
    extern __shared__ __align__(16) uint4 moe_smem[];
    int tx = blockIdx.x, ty = blockIdx.y;
    if (xcd_map) {
        // Blocks are dealt to the 8 XCDs round-robin by linear index; here
        // XCD k takes the k-th contiguous run of the live (row tile, column
        // tile) items, row-tile major, so the column tiles of one row tile
        // share that XCD's L2 for their A reads. The host pads the grid to
        // at least 8 * ceil(items / 8) blocks per K slice.
        const int L = blockIdx.y * gridDim.x + blockIdx.x;
        const int items = *ws.ntiles * (int)gridDim.x;
        const int per = (items + 7) >> 3;
        const int item = (L & 7) * per + (L >> 3);
        if ((L >> 3) >= per || item >= items) return;
        tx = item % gridDim.x;
        ty = item / gridDim.x;
    } else if (ty >= *ws.ntiles) {
        return;
    }
    const int e = ws.tile_e[ty], r0 = ws.tile_r0[ty], nrows = ws.tile_n[ty];
    const int n0 = tx * BNW;
    const uint16_t* a[2] = {Ahi + (size_t)r0 * Kd, Alo + (size_t)r0 * Kd};
    const uint16_t* w[2] = {W1 + ((size_t)e * N + n0) * Kd, DUAL ? W2 + ((size_t)e * N + n0) * Kd : nullptr};
    const float* bg = b1 ? b1 + (size_t)e * N + n0 : nullptr;
    const float* bu = (DUAL && b2) ? b2 + (size_t)e * N + n0 : nullptr;
    // gridDim.z > 1 (down GEMM only): K slice blockIdx.z, raw partial sums
    // to C + blockIdx.z * cslice; the combine adds the slices, bias and
    // routing weight
    // (the grid's default order already keeps each weight column tile on one
    // XCD, blocks being dealt round-robin; an XCD-contiguous order of whole
    // row tiles measured slower: 238 vs 194 us for the gate/up GEMM)
    const int nsl = gridDim.z;
    const int kslice = (Kd + nsl * 64 - 1) / (nsl * 64) * 64;
    const int kb = blockIdx.z * kslice, ke = min(Kd, kb + kslice);
    // xform: bias, SwiGLU or routing weight (the loads); store: the writes
    auto xform = [&](int row, int col, float* v) {
        if (!DUAL && nsl > 1) return;
        float s = v[0];
        if (bg) s = s + bg[col];
        if constexpr (DUAL) {
            float u = v[1];
            if (bu) u = u + bu[col];
            v[0] = s * sigmoidf_ref(s) * u;  // SwiGLU: gate * sigma(gate) * up
        } else {
            v[0] = s * ws.perm_w[r0 + row];  // weighted = exOut * w
        }
    };
    using ST = MoeStage<DUAL, BNW>;
    uint32_t* hs = reinterpret_cast<uint32_t*>(moe_smem);  // STG, DUAL: [kWideBM][LDH] (hi << 16 | lo)
    float* cs = reinterpret_cast<float*>(moe_smem);        // STG, else: [kWideBM][LDC]
    auto store = [&](int row, int col, const float* v) {
        if constexpr (STG) {
            if constexpr (DUAL) {
                const uint32_t hb = __float_as_uint(v[0]) & 0xffff0000u;
                hs[row * ST::LDH + col] =
                    hb | __builtin_bit_cast(uint16_t, (__bf16)(v[0] - __uint_as_float(hb)));
            } else {
                cs[row * ST::LDC + col] = v[0];
            }
            return;
        }
        const size_t o = (size_t)(r0 + row) * N + n0 + col;
        if constexpr (DUAL) {
            const uint32_t hb = __float_as_uint(v[0]) & 0xffff0000u;
            Chi[o] = (uint16_t)(hb >> 16);
            Clo[o] = __builtin_bit_cast(uint16_t, (__bf16)(v[0] - __uint_as_float(hb)));
        } else {
            C[(nsl > 1 ? (size_t)blockIdx.z * cslice : 0) + o] = v[0];
        }
    };
    const int ncols = min(BNW, N - n0);
    G::run(*reinterpret_cast<typename G::Smem*>(moe_smem), a, Kd, nrows, w, ncols, Kd, kb, ke, xform, store);
    if constexpr (STG) {
        __syncthreads();
        // N % 8 == 0 and n0 % BNW == 0: every chunk is whole and 16-byte aligned
        if constexpr (DUAL) {
            // 8 columns per chunk: 32 bytes of (hi, lo) pairs -> 16 bytes of each plane
            constexpr int CPR = BNW / 8, CHUNKS = kWideBM * CPR;
            for (int c = threadIdx.x; c < CHUNKS; c += G::kThreads) {
                const int row = c / CPR, ch = c % CPR;
                if (row < nrows && 8 * ch < ncols) {
                    const uint4 u0 = *reinterpret_cast<const uint4*>(hs + row * ST::LDH + 8 * ch);
                    const uint4 u1 = *reinterpret_cast<const uint4*>(hs + row * ST::LDH + 8 * ch + 4);
                    const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
                    uint4 hv, lv;
                    uint32_t* hp = reinterpret_cast<uint32_t*>(&hv);
                    uint32_t* lp = reinterpret_cast<uint32_t*>(&lv);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        hp[q] = (w[2 * q] >> 16) | (w[2 * q + 1] & 0xffff0000u);
                        lp[q] = (w[2 * q] & 0xffffu) | (w[2 * q + 1] << 16);
                    }
                    const size_t o = (size_t)(r0 + row) * N + n0 + 8 * ch;
                    *reinterpret_cast<uint4*>(Chi + o) = hv;
                    *reinterpret_cast<uint4*>(Clo + o) = lv;
                }
            }
        } else {
            constexpr int CPR = BNW / 4, CHUNKS = kWideBM * CPR;
            float* Cz = C + (nsl > 1 ? (size_t)blockIdx.z * cslice : 0);
            for (int c = threadIdx.x; c < CHUNKS; c += G::kThreads) {
                const int row = c / CPR, ch = c % CPR;
                if (row < nrows && 4 * ch < ncols)
                    *reinterpret_cast<float4*>(Cz + (size_t)(r0 + row) * N + n0 + 4 * ch) =
                        *reinterpret_cast<const float4*>(cs + row * ST::LDC + 4 * ch);
            }
        }
    }
}

template <bool DUAL, int BNW, bool IL, int WGM, int PD = 2, bool STG = false>
static int launch_moe_wide_t(hipStream_t s, dim3 grid, const uint16_t* Ahi, const uint16_t* Alo, const uint16_t* W1,
                             const uint16_t* W2, const float* b1, const float* b2, float* C, uint16_t* Chi,
                             uint16_t* Clo, int N, int Kd, long long cslice, int xcd_map, const MoeWs& ws) {
    using G = WideGemm<kWideBM, BNW, DUAL ? 2 : 1, true, 64, IL, WGM, 4, PD>;
    constexpr size_t smem = STG ? std::max(sizeof(typename G::Smem), MoeStage<DUAL, BNW>::kBytes)
                                : sizeof(typename G::Smem);
    static bool attr_set = false;
    if (!attr_set) {
        GH_TRY(check(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_moe_wide<DUAL, BNW, IL, WGM, PD, STG>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem),
                     "moe_wide attribute"));
        attr_set = true;
    }
    hipLaunchKernelGGL((k_moe_wide<DUAL, BNW, IL, WGM, PD, STG>), grid, dim3(G::kThreads), smem, s, Ahi, Alo,
                       W1, W2, b1, b2, C, Chi, Clo, N, Kd, cslice, xcd_map, ws);
    return check_launch(DUAL ? "moe_wide_gate_up" : "moe_wide_down");
}

// The expert GEMMs run 16 waves (4 x 4) per block, with the interleaved
// stage schedule and one register set for the global loads (measured,
// against 8-wave blocks and the compiler's own schedule: gate/up 180 -> 159
// us, down 108 -> 96 us at the MoE layer config). The down GEMM stages its
// finished tile in LDS for 16-byte stores (100.6 -> 97.3 us; gate/up 164.7 ->
// 165.9, so only down) and takes the XCD-contiguous block order.
template <bool DUAL, int BNW>
static int launch_moe_wide(hipStream_t s, dim3 grid, const uint16_t* Ahi, const uint16_t* Alo, const uint16_t* W1,
                           const uint16_t* W2, const float* b1, const float* b2, float* C, uint16_t* Chi,
                           uint16_t* Clo, int N, int Kd, long long cslice, const MoeWs& ws) {
    constexpr int xcd_map = DUAL ? 0 : 1;
    if (xcd_map) {
        // at least 8 * ceil(items / 8) blocks per slice, a multiple of 8
        const long long need = ((long long)grid.x * grid.y + 7) / 8 * 8;
        grid.y = (unsigned)((need + grid.x - 1) / grid.x);
        while (((long long)grid.x * grid.y) % 8) grid.y++;
    }
    return launch_moe_wide_t<DUAL, BNW, true, 4, 1, !DUAL>(s, grid, Ahi, Alo, W1, W2, b1, b2, C, Chi, Clo, N, Kd,
                                                           cslice, xcd_map, ws);
}

}  // namespace gh

using namespace gh;

extern "C" size_t gorch_hip_moe_workspace_size(int M, int dim, int ffn, int experts, int top_k) {
    if (M <= 0 || dim <= 0 || ffn <= 0 || experts <= 0 || top_k <= 0) return 0;
    return moe_layout(M, dim, ffn, experts, top_k, nullptr, nullptr);
}

extern "C" int gorch_hip_moe_forward(void* stream, const gorch_hip_moe_weights* w, const float* x, int M,
                                     const float* logits, float* out, int* topk_idx, float* topk_w,
                                     void* workspace, size_t workspace_bytes) {
    GH_REQUIRE(w && x && out && M > 0, "gorch_hip_moe_forward: bad arguments");
    const int E = w->experts, K = w->top_k, d = w->dim, F = w->ffn;
    GH_REQUIRE(K >= 1 && K <= E, "gorch/nn: MoE numExpertsPerToken out of range");
    GH_REQUIRE(E <= kMaxExperts && K <= kMaxTopK, "gorch_hip_moe_forward: at most 64 experts and top-8");
    GH_REQUIRE((long long)M * E < (1ll << 29) && (long long)M * K * d < (1ll << 29),
               "gorch_hip_moe_forward: M * experts and M * top_k * dim must be below 2^29");
    GH_REQUIRE(d % 8 == 0 && F % 8 == 0, "gorch_hip_moe_forward: dim and ffn must be multiples of 8");
    GH_REQUIRE(w->wgate && w->wup && w->wdown, "gorch_hip_moe_forward: null expert weights");
    GH_REQUIRE(logits || w->wr, "gorch_hip_moe_forward: need router weights or injected logits");
    GH_TRY(bf16_gate(stream_of(stream)));
    const size_t need = moe_layout(M, d, F, E, K, nullptr, nullptr);
    GH_REQUIRE(workspace && workspace_bytes >= need, "gorch_hip_moe_forward: workspace too small");
    MoeWs ws;
    moe_layout(M, d, F, E, K, (char*)workspace, &ws);
    hipStream_t s = stream_of(stream);
    const float* lg = logits;
    if (!lg) {
        GH_TRY(launch_linear_bf16(s, x, w->wr, w->br, nullptr, ws.logits, M, E, d, GORCH_HIP_EPI_NONE));
        lg = ws.logits;
    }
    const int tile_rows = kWideBM;
    // top-K slots sized to K (every absent slot still costs its compares).
    // Up to two slots, 8 experts and 4096 tokens: the routing block takes
    // the top-K itself (one launch fewer)
    if (K <= 2 && E <= 8 && M <= 4 * kRouteThreads) {
        hipLaunchKernelGGL((k_moe_route<2, 8>), dim3(1), dim3(kRouteThreads), 0, s, M, E, K, tile_rows, ws, lg,
                           topk_idx, topk_w);
    } else {
        const dim3 tgrid((M + 255) / 256);
        if (E <= 8)
            hipLaunchKernelGGL(k_moe_topk<8>, tgrid, dim3(256), 0, s, lg, M, E, K, ws.topi, ws.topw, topk_idx, topk_w);
        else if (E <= 16)
            hipLaunchKernelGGL(k_moe_topk<16>, tgrid, dim3(256), 0, s, lg, M, E, K, ws.topi, ws.topw, topk_idx,
                               topk_w);
        else
            hipLaunchKernelGGL(k_moe_topk<kMaxExperts>, tgrid, dim3(256), 0, s, lg, M, E, K, ws.topi, ws.topw,
                               topk_idx, topk_w);
        GH_TRY(check_launch("moe_topk"));
        if (K <= 2)
            hipLaunchKernelGGL((k_moe_route<2>), dim3(1), dim3(kRouteThreads), 0, s, M, E, K, tile_rows, ws, nullptr,
                               nullptr, nullptr);
        else
            hipLaunchKernelGGL((k_moe_route<kMaxTopK>), dim3(1), dim3(kRouteThreads), 0, s, M, E, K, tile_rows, ws,
                               nullptr, nullptr, nullptr);
    }
    GH_TRY(check_launch("moe_route"));
    const int MK = M * K;
    const int max_tiles = MK / tile_rows + E + 1;
    // Xg and H hold (hi, lo) bf16 planes in the space of their f32 form
    uint16_t* xhi = reinterpret_cast<uint16_t*>(ws.xg);
    uint16_t* xlo = xhi + (size_t)MK * d;
    uint16_t* hhi = reinterpret_cast<uint16_t*>(ws.h);
    uint16_t* hlo = hhi + (size_t)MK * F;
    const int gblocks = (int)std::min<int64_t>(8192, ((int64_t)M * d / 8 + 255) / 256);
    if (K <= 2)
        hipLaunchKernelGGL(k_moe_gather_split<2>, dim3(gblocks), dim3(256), 0, s, x, ws.inv, xhi, xlo, M, K, d);
    else
        hipLaunchKernelGGL(k_moe_gather_split<kMaxTopK>, dim3(gblocks), dim3(256), 0, s, x, ws.inv, xhi, xlo, M, K,
                           d);
    GH_TRY(check_launch("moe_gather"));
    GH_TRY((launch_moe_wide<true, kWideBNDual>(s, dim3((F + kWideBNDual - 1) / kWideBNDual, max_tiles), xhi, xlo,
                                              w->wgate, w->wup, w->bgate, w->bup, nullptr, hhi, hlo, F, d, 0, ws)));
    // the down GEMM unsplit over K (one slice of partials in yg)
    const int nsl = 1;
    const long long cslice = (long long)MK * d;
    GH_TRY((launch_moe_wide<false, kWideBNDown>(s, dim3((d + kWideBNDown - 1) / kWideBNDown, max_tiles, nsl), hhi,
                                                hlo, w->wdown, nullptr, w->bdown, nullptr, ws.yg, nullptr, nullptr, d,
                                                F, cslice, ws)));
    const int cblocks = (int)std::min<int64_t>(8192, ((int64_t)M * d / 4 + 255) / 256);
    if (K <= 2)
        hipLaunchKernelGGL(k_moe_combine<2>, dim3(cblocks), dim3(256), 0, s, ws.yg, ws.inv, ws.topi, out, M, K, d, nsl,
                           cslice, w->bdown, ws.perm_w);
    else
        hipLaunchKernelGGL(k_moe_combine<kMaxTopK>, dim3(cblocks), dim3(256), 0, s, ws.yg, ws.inv, ws.topi, out, M, K, d, nsl,
                           cslice, w->bdown, ws.perm_w);
    GH_TRY(check_launch("moe_combine"));
    count(CNT_MOE);
    return finish(stream, GORCH_HIP_OK);
}
