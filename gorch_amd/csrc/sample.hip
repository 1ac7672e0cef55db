// sample.hip — the sampled next-token choice of generateCached with
// Temperature > 0 (model/generate.go:105-110; sample() at :147-243,
// kthLargest at :247-262) and of the Qwen Generate loop (sampleLogits,
// model/qwen/generate.go:94-181), one 1024-thread block per row of logits.
//
//   scaled = logits / temperature (f32)
//   0 < top_k < n: values below the top_k-th largest scaled value -> -inf
//     (the value kthLargest returns, counting equal values). Up to
//     kSampleCap candidates: a 4096-bin histogram of the raw logits'
//     order-preserving 32-bit keys (division by T is monotone) locates the
//     bin of the top_k-th largest, one more pass collects every key at or
//     above it, and everything below runs on those candidates in index
//     order; otherwise a 4-pass radix select (256-bin histograms) over the
//     row and the passes below over the whole row.
//   p = exp(f64(scaled - max)) / sum (f64)
//   0 < top_p < 1: the reference zeroes the smallest positive probability
//     (lowest index first among equals) until the positive ones sum to at
//     most f64(top_p) * 1.5, then divides by their sum. That keeps the
//     longest prefix, in order of (p descending, index descending), whose
//     sum is at most that limit: the positive probabilities (at most
//     kSampleCap of them: top_p needs 1 <= top_k <= kSampleCap, and more
//     candidates through ties at the top-k threshold set the error flag) are
//     sorted in LDS by that order (bitonic), prefix-summed, and the prefix
//     kept.
//   nucleus (the Qwen loop's top-p, 0 < top_p < 1): the shortest prefix, in
//     order of (p descending, index ascending), whose running sum reaches
//     f64(top_p) is kept and divided by its sum, every other probability set
//     to 0 (sort.Slice leaves the order of equal probabilities open; this
//     one takes the lower index first). Same candidate limits and sort.
//   token = the first index whose running sum of the final probabilities
//     exceeds the uniform draw r (n - 1 if none), found over 16 contiguous
//     wave ranges read 64 entries at a time.
//
// The draw r is u[row] when u is given, else Philox4x32-10 (Salmon, Moraes,
// Dror and Shaw, SC 2011) of counter (row, step, 0, 0) under key (seed low,
// seed high), step read from the device (one graph serves every step),
// r = ((x0 >> 5) * 2^26 + (x1 >> 6)) / 2^53. The f64 sums are block
// reductions in a fixed order (the reference sums sequentially), so the
// probabilities agree with it to f64 rounding, and a choice can differ only
// where r or the top-p limit falls within that rounding of a boundary.
#include <climits>
#include <cmath>

#include "common.h"

namespace gh {

constexpr int kSampleThreads = 1024;
constexpr int kSampleCap = 4096;
constexpr int kSampleMaxN = 1 << 18;  // columns (the top-p bitmap's size)
constexpr int kRowUnroll = 8;         // row entries per thread in flight in a pass
// up to this many elements a sort places each one at its rank (one pass of
// comparisons, one barrier) instead of a bitonic network (a barrier per
// stage: 36 at 256 elements; across one wave's lanes 21 shuffle stages,
// ~2.5 us at 40 elements)
constexpr int kRankSortMax = 256;

__device__ __forceinline__ uint32_t f32_order_key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float f32_from_order_key(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ double philox_uniform(unsigned long long seed, uint32_t step, uint32_t row) {
    uint32_t c0 = row, c1 = step, c2 = 0u, c3 = 0u;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; r++) {
        const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return ((double)(c0 >> 5) * 67108864.0 + (double)(c1 >> 6)) / 9007199254740992.0;
}

// Sample workspace (launch_sample's ws), per row in ints: the 4096-bin
// histogram of the raw logits' order keys, the appended-candidate count,
// the maximum key, the NaN flag, the bin of the top_k-th largest key and the
// count of keys from that bin up, then kSampleCap candidate keys and
// kSampleCap indices. Zero while idle: k_sample clears all of it after
// reading it, so a captured step graph finds it zero again.
constexpr int kWsCnt = 4096, kWsMax = 4097, kWsNan = 4098, kWsBin = 4099, kWsC = 4100, kWsKey = 4104,
              kWsIdx = kWsKey + kSampleCap;
constexpr int kWsRowInts = kWsIdx + kSampleCap;
// below this row length the one-block passes are as fast
constexpr int kSampleWsMinN = 8192;
constexpr int kScanThreads = 256, kScanUnroll = 4;

// Pass one of the top-k candidate search spread over gridDim.x blocks per
// row (blockIdx.y): each block histograms the order keys of its chunk
// [chunk * blockIdx.x, ..) in LDS (zeros taken as +0, as in k_sample), then
// adds its non-empty bins into the row's histogram (one atomic per bin and
// block), its maximum key and its NaN flag.
__global__ __launch_bounds__(kScanThreads) void k_sample_scan(const float* __restrict__ logits, int n, int chunk,
                                                             int* __restrict__ ws) {
    __shared__ int h[4096];
    __shared__ uint32_t s_max[kScanThreads / 64];
    __shared__ int s_nan;
    const int row = blockIdx.y, tid = threadIdx.x;
    int* w = ws + (size_t)row * kWsRowInts;
    for (int b = tid; b < 4096; b += kScanThreads) h[b] = 0;
    if (tid == 0) s_nan = 0;
    __syncthreads();
    const int i0 = blockIdx.x * chunk, i1 = min(n, i0 + chunk);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(logits + (size_t)row * n, (long long)n * 4);
    uint32_t kmax = 0u;
    int nan = 0;
    for (int base = i0; base < i1; base += kScanUnroll * kScanThreads) {
        float v[kScanUnroll];
#pragma unroll
        for (int u = 0; u < kScanUnroll; u++) {
            const int i = base + u * kScanThreads + tid;
            v[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rr, i < i1 ? i * 4 : kOutOfRange, 0, 0));
        }
#pragma unroll
        for (int u = 0; u < kScanUnroll; u++) {
            if (base + u * kScanThreads + tid < i1) {
                const uint32_t key = f32_order_key(v[u] == 0.f ? 0.f : v[u]);
                kmax = max(kmax, key);
                nan |= v[u] != v[u];
                atomicAdd(&h[key >> 20], 1);
            }
        }
    }
    for (int o = 32; o > 0; o >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
    if ((tid & 63) == 0) s_max[tid >> 6] = kmax;
    if (nan) s_nan = 1;
    __syncthreads();
    for (int b = tid; b < 4096; b += kScanThreads)
        if (h[b]) atomicAdd(&w[b], h[b]);
    if (tid == 0) {
        for (int q = 0; q < kScanThreads / 64; q++) kmax = max(kmax, s_max[q]);
        atomicMax(reinterpret_cast<unsigned int*>(&w[kWsMax]), kmax);
        if (s_nan) atomicOr(&w[kWsNan], 1);
    }
}

// Pass two: every block locates the bin of the top_k-th largest key from the
// row's histogram (the same scan as k_sample's) and, when the candidates
// fit kSampleCap and no logit is NaN, appends its chunk's keys at or above
// that bin (one slot reservation per block).
__global__ __launch_bounds__(kScanThreads) void k_sample_gather(const float* __restrict__ logits, int n, int chunk,
                                                               int top_k, int* __restrict__ ws) {
    __shared__ int s_scan[kScanThreads / 64];
    __shared__ int s_bin, s_above, s_cnt, s_base;
    __shared__ uint32_t l_key[kSampleCap];
    __shared__ int l_idx[kSampleCap];
    const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int* w = ws + (size_t)row * kWsRowInts;
    // thread t sums bins 4095 - 16 t - q (q < 16): a scan of those sums in
    // thread order is the count above each group of bins
    constexpr int BPT = 4096 / kScanThreads;
    int hb[BPT];
    int gs = 0;
#pragma unroll
    for (int q = 0; q < BPT; q++) {
        hb[q] = w[4095 - BPT * tid - q];
        gs += hb[q];
    }
    int incl = gs;
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) s_scan[wave] = incl;
    if (tid == 0) s_cnt = 0;
    __syncthreads();
    int above = incl - gs;
    for (int q = 0; q < wave; q++) above += s_scan[q];
    if (above < top_k && above + gs >= top_k) {
        int cum = above;
#pragma unroll
        for (int q = 0; q < BPT; q++) {
            if (cum + hb[q] >= top_k) {
                s_bin = 4095 - BPT * tid - q;
                s_above = cum;
                break;
            }
            cum += hb[q];
        }
    }
    __syncthreads();
    const int dbin = s_bin;
    const int C = s_above + w[dbin];
    if (blockIdx.x == 0 && tid == 0) {
        w[kWsBin] = dbin;
        w[kWsC] = C;
    }
    if (C > kSampleCap || w[kWsNan] != 0) return;
    const int i0 = blockIdx.x * chunk, i1 = min(n, i0 + chunk);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(logits + (size_t)row * n, (long long)n * 4);
    for (int base = i0; base < i1; base += kScanUnroll * kScanThreads) {
        float v[kScanUnroll];
#pragma unroll
        for (int u = 0; u < kScanUnroll; u++) {
            const int i = base + u * kScanThreads + tid;
            v[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rr, i < i1 ? i * 4 : kOutOfRange, 0, 0));
        }
#pragma unroll
        for (int u = 0; u < kScanUnroll; u++) {
            const int i = base + u * kScanThreads + tid;
            const uint32_t key = f32_order_key(v[u] == 0.f ? 0.f : v[u]);
            if (i < i1 && (int)(key >> 20) >= dbin) {
                const int slot = atomicAdd(&s_cnt, 1);
                l_key[slot] = key;
                l_idx[slot] = i;
            }
        }
    }
    __syncthreads();
    const int cnt = s_cnt;
    if (cnt == 0) return;
    if (tid == 0) s_base = atomicAdd(&w[kWsCnt], cnt);
    __syncthreads();
    const int b0 = s_base;
    for (int j = tid; j < cnt; j += kScanThreads)
        if (b0 + j < kSampleCap) {
            w[kWsKey + b0 + j] = (int)l_key[j];
            w[kWsIdx + b0 + j] = l_idx[j];
        }
}

// Block reductions over 1024 threads in a fixed order (wave partials in
// LDS, summed by every thread in wave order).
__device__ double block_sum_f64(double v, double* sh) {
    v = wave_sum_d(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < kSampleThreads / 64; w++) t += sh[w];
    __syncthreads();
    return t;
}
__device__ float block_max_f32(float v, float* sh) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float t = sh[0];
    for (int w = 1; w < kSampleThreads / 64; w++) t = fmaxf(t, sh[w]);
    __syncthreads();
    return t;
}
__device__ int block_sum_i32(int v, int* sh) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    int t = 0;
    for (int w = 0; w < kSampleThreads / 64; w++) t += sh[w];
    __syncthreads();
    return t;
}
__device__ int block_min_i32(int v, int* sh) {
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    int t = sh[0];
    for (int w = 1; w < kSampleThreads / 64; w++) t = min(t, sh[w]);
    __syncthreads();
    return t;
}
// Exclusive prefix of one f64 per thread in thread order: an inclusive
// scan within each wave (lane shifts), then the waves' totals added in wave
// order; returns this thread's exclusive prefix, *total the block's sum.
__device__ double block_exclusive_scan_f64(double v, double* sc, double* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    double inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
    }
    if (lane == 63) sc[wave] = inc;
    __syncthreads();
    double before = 0.0, tot = 0.0;
    for (int w = 0; w < kSampleThreads / 64; w++) {
        const double x = sc[w];
        if (w < wave) before += x;
        tot += x;
    }
    *total = tot;
    __syncthreads();
    return before + (inc - v);
}

// Bitonic sort of one element per lane across the 64 lanes of a wave
// (before(a, b): a sorts first; elements must be distinct under it).
template <typename E, typename Before>
__device__ __forceinline__ E wave_bitonic_sort(E mine, Before before) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            E other;
            other.a = __shfl_xor(mine.a, stride);
            other.b = __shfl_xor(mine.b, stride);
            const bool lower = (lane & stride) == 0, asc = (lane & size) == 0;
            if (lower == asc ? before(other, mine) : before(mine, other)) mine = other;
        }
    }
    return mine;
}

struct SampleArgs {
    const float* logits;
    int n;
    float temperature;
    int top_k;
    float top_p;
    const double* u;           // draws per row, or null: Philox(seed, *step, row)
    unsigned long long seed;
    const int* step;
    int* out;                  // token per row (may be null)
    double* probs;             // final distribution [rows, n] (may be null)
    unsigned long long* key;   // fused-argmax key slot 0 of row b gets the token (may be null)
    int* err;                  // set to 1 when the top-p candidates exceed kSampleCap
    int nucleus;               // top-p as sampleLogits' nucleus cut, else as sample()
    int* ws = nullptr;         // workspace the two scan kernels filled (top-k rows), or null
};

__global__ __launch_bounds__(kSampleThreads) void k_sample(SampleArgs a) {
    __shared__ int hist[256];
    __shared__ double red_d[kSampleThreads / 64];
    __shared__ float red_f[kSampleThreads / 64];
    __shared__ int red_i[kSampleThreads / 64];
    __shared__ uint32_t red_u[kSampleThreads / 64];
    __shared__ uint32_t s_prefix;
    __shared__ int s_k, s_cnt, s_bin, s_above;
    __shared__ double s_p[kSampleCap];
    __shared__ int s_idx[kSampleCap];
    __shared__ double s_scan[kSampleThreads];
    // kept indices (top-p) as a bitmap over n; the top-k candidate pass's
    // 4096-bin key histogram before that
    __shared__ uint32_t s_keep[kSampleMaxN / 32];
    __shared__ uint32_t c_key[kSampleCap];  // top-k candidates: order keys
    __shared__ int c_idx[kSampleCap];       // and indices
    const int row = blockIdx.x, tid = threadIdx.x, n = a.n;
    const float* lg = a.logits + (size_t)row * n;
    const float T = a.temperature;
    const bool use_k = a.top_k > 0 && a.top_k < n;
    const bool use_p = a.top_p > 0.f && a.top_p < 1.f;
    const double r = a.u ? a.u[row] : philox_uniform(a.seed, (uint32_t)*a.step, (uint32_t)row);
    // the row's entries base + u * kSampleThreads + tid (u < kRowUnroll), all
    // loads in flight together; past n they read 0
    const __amdgpu_buffer_rsrc_t rrow = make_rsrc(lg, (long long)n * 4);
    auto load_row = [&](int base, float (&v)[kRowUnroll]) {
#pragma unroll
        for (int u = 0; u < kRowUnroll; u++)
            v[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rrow, (base + u * kSampleThreads + tid) * 4, 0, 0));
    };

    // The k-th largest of `count` order keys key_at(j), counting equal keys:
    // a 4-pass radix select, 256-bin LDS histograms.
    auto radix_kth = [&](auto key_at, int count, int k) -> uint32_t {
        uint32_t prefix = 0u, mask = 0u;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int b = tid; b < 256; b += kSampleThreads) hist[b] = 0;
            __syncthreads();
            for (int j = tid; j < count; j += kSampleThreads) {
                const uint32_t key = key_at(j);
                if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
            }
            __syncthreads();
            // the bin holding the k-th largest, from the top: wave 0, lane l
            // owning bins 255 - 4l - q (q < 4), an inclusive scan of the
            // lanes' sums
            if (tid < 64) {
                int gs = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) gs += hist[255 - 4 * tid - q];
                int inc = gs;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const int t = __shfl_up(inc, o);
                    if (tid >= o) inc += t;
                }
                const int above = inc - gs;
                if (above < k && inc >= k) {
                    int cum = above, d = 255 - 4 * tid;
#pragma unroll
                    for (int q = 0; q < 3; q++) {
                        if (cum + hist[d] >= k) break;
                        cum += hist[d];
                        d--;
                    }
                    s_prefix = prefix | ((uint32_t)d << shift);
                    s_k = k - cum;
                }
            }
            __syncthreads();
            prefix = s_prefix;
            k = s_k;
            mask |= 255u << shift;
        }
        return prefix;
    };

    // Top-p over the probabilities in s_p / s_idx[0, cnt) (cnt <= kSampleCap;
    // entries of probability 0 change nothing): sorted in LDS, the kept
    // prefix marked in the s_keep bitmap; returns the kept sum. sample()
    // keeps the longest prefix, in order of (p descending, index
    // descending), whose sum is at most 1.5 * top_p; the nucleus keeps, in
    // order of (p descending, index ascending), every entry whose preceding
    // sum is still below top_p.
    // rank_ok: every p is a number (the rank sort needs a strict order; the
    // bitonic network tolerates NaN)
    auto top_p_keep = [&](int cnt, bool rank_ok) -> double {
        int P = 1;
        while (P < cnt) P <<= 1;
        if (rank_ok && cnt <= kRankSortMax) {
            // (p descending, then index as below): distinct pairs, so the
            // ranks are a permutation
            double pm = 0.0;
            int im = 0, rank = 0;
            if (tid < cnt) {
                pm = s_p[tid];
                im = s_idx[tid];
                for (int i = 0; i < cnt; i++) {
                    const double pi = s_p[i];
                    const int ii = s_idx[i];
                    rank += pi > pm || (pi == pm && (a.nucleus ? ii < im : ii > im));
                }
            }
            __syncthreads();
            if (tid < cnt) {
                s_p[rank] = pm;
                s_idx[rank] = im;
            }
            P = 1;  // (the block sort below then does nothing)
        } else if (P <= 64) {
            // one wave sorts up to 64
            struct PI {
                double a;  // p
                int b;     // index
            };
            if (tid < 64) {
                PI e = tid < cnt ? PI{s_p[tid], s_idx[tid]} : PI{-1.0, -1};
                const bool nuc = a.nucleus != 0;
                e = wave_bitonic_sort(e, [nuc](const PI& x, const PI& y) {
                    return x.a > y.a || (x.a == y.a && (nuc ? x.b < y.b : x.b > y.b));
                });
                s_p[tid] = e.a;
                s_idx[tid] = e.b;
            }
            P = 1;  // (the block sort below then does nothing)
        }
        for (int i = cnt + tid; i < P; i += kSampleThreads) {
            s_p[i] = -1.0;
            s_idx[i] = -1;
        }
        __syncthreads();
        for (int size = 2; size <= P; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                for (int t = tid; t < P / 2; t += kSampleThreads) {
                    const int i = 2 * stride * (t / stride) + (t % stride), j = i + stride;
                    const bool desc = (i & size) == 0;
                    const double pi = s_p[i], pj = s_p[j];
                    const int ii = s_idx[i], ij = s_idx[j];
                    const bool j_first = pj > pi || (pj == pi && (a.nucleus ? ij < ii : ij > ii));
                    if (j_first == desc) {
                        s_p[i] = pj;
                        s_p[j] = pi;
                        s_idx[i] = ij;
                        s_idx[j] = ii;
                    }
                }
                __syncthreads();
            }
        }
        // (the prefix sums increase with the prefix's length)
        constexpr int PER = kSampleCap / kSampleThreads;
        const double limit = a.nucleus ? (double)a.top_p : (double)a.top_p * 1.5;
        double loc = 0.0;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int j = tid * PER + q;
            loc += j < cnt ? s_p[j] : 0.0;
        }
        double total;
        double run = block_exclusive_scan_f64(loc, s_scan, &total);
        int keep = 0;
        double kept_sum = 0.0;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int j = tid * PER + q;
            if (j < cnt) {
                const bool kept = a.nucleus ? run < limit : run + s_p[j] <= limit;
                run += s_p[j];
                if (kept) {
                    keep++;
                    kept_sum += s_p[j];
                }
            }
        }
        const int L = block_sum_i32(keep, red_i);
        const double rs = block_sum_f64(kept_sum, red_d);
        const int words = (n + 31) / 32;
        for (int w = tid; w < words; w += kSampleThreads) s_keep[w] = 0u;
        __syncthreads();
        for (int j = tid; j < L; j += kSampleThreads) atomicOr(&s_keep[s_idx[j] >> 5], 1u << (s_idx[j] & 31));
        __syncthreads();
        return rs;
    };
    auto is_kept = [&](int i) { return ((s_keep[i >> 5] >> (i & 31)) & 1u) != 0u; };
    // (with top-p every value is divided by the kept sum, as the reference
    // does: 0/0 = NaN everywhere when nothing was kept, and the draw then
    // falls through to n - 1)
    auto finish = [&](double p, bool kept, double resum) -> double {
        // (a NaN logit makes the sum and every p NaN; the nucleus cut then
        // never reaches top_p and keeps everything: NaN as well)
        if (!use_p || p != p) return p;
        if (a.nucleus) return kept ? p / resum : 0.0;
        return (kept ? p : 0.0) / resum;
    };
    auto emit = [&](int tok) {
        if (tid == 0) {
            if (a.out) a.out[row] = tok;
            // a key the fused-argmax consumers decode to tok (slot 0 of row)
            if (a.key) a.key[row] = (1ull << 32) | (unsigned long long)(0xffffffffu - (uint32_t)tok);
        }
    };

    // top-k on candidates. Division by T > 0 is monotone, so the scaled
    // values' top_k-th largest is the raw logits' top_k-th largest divided by
    // T: one pass builds a 4096-bin histogram of the raw logits' order keys
    // (zeros taken as +0, which compares equal), which locates the bin of the
    // top_k-th largest; a second pass collects every key at or above that
    // bin. When they fit kSampleCap and no logit is NaN, the threshold,
    // softmax, top-p and the inverse CDF run on them alone (scaled, in index
    // order); the rest of the row has probability 0. A logit below the bin
    // whose scaled value still equals the threshold (rounding) sends the
    // row to the full path.
    if (use_k && a.top_k <= kSampleCap) {
        int* hist12 = reinterpret_cast<int*>(s_keep);
        // with a workspace, k_sample_scan built the histogram, maximum and
        // NaN flag over many blocks; else the block's own pass
        int* w = a.ws ? a.ws + (size_t)row * kWsRowInts : nullptr;
        uint32_t kmax = 0u;
        bool any_nan = false;
        int dbin = 0, C = 0;
        if (w) {
            // (k_sample_gather located the bin and counted the candidates)
            kmax = (uint32_t)w[kWsMax];
            any_nan = w[kWsNan] != 0;
            dbin = w[kWsBin];
            C = w[kWsC];
        } else {
        for (int b = tid; b < 4096; b += kSampleThreads) hist12[b] = 0;
        __syncthreads();
        int nan = 0;
        for (int base = 0; base < n; base += kRowUnroll * kSampleThreads) {
            float v[kRowUnroll];
            load_row(base, v);
#pragma unroll
            for (int u = 0; u < kRowUnroll; u++) {
                if (base + u * kSampleThreads + tid < n) {
                    const uint32_t key = f32_order_key(v[u] == 0.f ? 0.f : v[u]);
                    kmax = max(kmax, key);
                    nan |= v[u] != v[u];
                    atomicAdd(&hist12[key >> 20], 1);
                }
            }
        }
        for (int o = 32; o > 0; o >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
        if ((tid & 63) == 0) red_u[tid >> 6] = kmax;
        // (its barriers also publish red_u and the histogram)
        any_nan = block_sum_i32(nan, red_i) > 0;
        for (int q = 0; q < kSampleThreads / 64; q++) kmax = max(kmax, red_u[q]);
        // thread t sums bins 4095 - 4t - q (q < 4): the scan of those sums in
        // thread order is the count above each group of bins
        int gs = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) gs += hist12[4095 - 4 * tid - q];
        double tot;
        const int above_g = (int)block_exclusive_scan_f64((double)gs, s_scan, &tot);
        if (above_g < a.top_k && above_g + gs >= a.top_k) {
            int cum = above_g;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int b = 4095 - 4 * tid - q;
                if (cum + hist12[b] >= a.top_k) {
                    s_bin = b;
                    s_above = cum;
                    break;
                }
                cum += hist12[b];
            }
        }
        __syncthreads();
        dbin = s_bin;
        C = s_above + hist12[dbin];
        }
        bool cand_ok = C <= kSampleCap && !any_nan;
        if (w) {
            // k_sample_gather appended exactly the C candidates (any order);
            // then the workspace is cleared for the next use
            const int wcnt = min(w[kWsCnt], kSampleCap);
            if (cand_ok) {
                cand_ok = wcnt == C;
                if (cand_ok)
                    for (int j = tid; j < C; j += kSampleThreads) {
                        c_key[j] = (uint32_t)w[kWsKey + j];
                        c_idx[j] = w[kWsIdx + j];
                    }
            }
            __syncthreads();
            for (int b = tid; b < 4096; b += kSampleThreads) w[b] = 0;
            for (int j = tid; j < wcnt; j += kSampleThreads) {
                w[kWsKey + j] = 0;
                w[kWsIdx + j] = 0;
            }
            if (tid < kWsKey - kWsCnt) w[kWsCnt + tid] = 0;
        }
        __syncthreads();
        if (cand_ok) {
            if (!w) {
            if (tid == 0) s_cnt = 0;
            __syncthreads();
            for (int base = 0; base < n; base += kRowUnroll * kSampleThreads) {
                float v[kRowUnroll];
                load_row(base, v);
#pragma unroll
                for (int u = 0; u < kRowUnroll; u++) {
                    const int i = base + u * kSampleThreads + tid;
                    const uint32_t key = f32_order_key(v[u] == 0.f ? 0.f : v[u]);
                    if (i < n && (int)(key >> 20) >= dbin) {
                        const int slot = atomicAdd(&s_cnt, 1);
                        c_key[slot] = key;
                        c_idx[slot] = i;
                    }
                }
            }
            __syncthreads();
            }
            // the top_k-th largest key (every key above dbin's floor is a
            // candidate, so it is the row's): with few candidates the largest
            // key that at least top_k keys reach, each thread counting for
            // its own candidates; else the radix select
            uint32_t tkey;
            if (C <= 512) {
                uint32_t best = 0u;
                for (int j = tid; j < C; j += kSampleThreads) {
                    const uint32_t kj = c_key[j];
                    int ge = 0;
                    for (int i = 0; i < C; i++) ge += c_key[i] >= kj;
                    if (ge >= a.top_k) best = max(best, kj);
                }
                for (int o = 32; o > 0; o >>= 1) best = max(best, (uint32_t)__shfl_xor((int)best, o));
                if ((tid & 63) == 0) red_u[tid >> 6] = best;
                __syncthreads();
                tkey = 0u;
                for (int w = 0; w < kSampleThreads / 64; w++) tkey = max(tkey, red_u[w]);
            } else {
                tkey = radix_kth([&](int j) { return c_key[j]; }, C, a.top_k);
            }
            const float thr = f32_from_order_key(tkey) / T;
            const float mx = f32_from_order_key(kmax) / T;
            const bool below = dbin > 0 && f32_from_order_key((uint32_t)dbin << 20) / T >= thr;
            if (!below) {
                // only the candidates at or above the threshold carry
                // probability: keep those (top_k plus ties) before the sorts,
                // the softmax, top-p and the inverse CDF
                int Ck;
                {
                    constexpr int PC = kSampleCap / kSampleThreads;
                    uint32_t kk[PC];
                    int ii[PC];
#pragma unroll
                    for (int q = 0; q < PC; q++) {
                        const int j = tid + q * kSampleThreads;
                        kk[q] = j < C ? c_key[j] : 0u;
                        ii[q] = j < C ? c_idx[j] : 0;
                    }
                    if (tid == 0) s_cnt = 0;
                    __syncthreads();
#pragma unroll
                    for (int q = 0; q < PC; q++) {
                        const int j = tid + q * kSampleThreads;
                        if (j < C && f32_from_order_key(kk[q]) / T >= thr) {
                            const int slot = atomicAdd(&s_cnt, 1);
                            c_key[slot] = kk[q];
                            c_idx[slot] = ii[q];
                        }
                    }
                    __syncthreads();
                    Ck = s_cnt;
                }
                // candidates into index order: by rank up to kRankSortMax,
                // else a bitonic network across the block (padding sorts last)
                int P = 1;
                while (P < Ck) P <<= 1;
                if (Ck <= kRankSortMax) {
                    // distinct indices: each candidate's rank is its slot
                    int im = INT_MAX, rank = 0;
                    uint32_t km = 0u;
                    if (tid < Ck) {
                        im = c_idx[tid];
                        km = c_key[tid];
                        for (int i = 0; i < Ck; i++) rank += c_idx[i] < im;
                    }
                    __syncthreads();
                    if (tid < Ck) {
                        c_idx[rank] = im;
                        c_key[rank] = km;
                    }
                    P = 1;  // (the block sort below then does nothing)
                }
                for (int j = Ck + tid; j < P; j += kSampleThreads) {
                    c_idx[j] = INT_MAX;
                    c_key[j] = 0u;
                }
                __syncthreads();
                for (int size = 2; size <= P; size <<= 1) {
                    for (int stride = size >> 1; stride > 0; stride >>= 1) {
                        for (int t = tid; t < P / 2; t += kSampleThreads) {
                            const int i = 2 * stride * (t / stride) + (t % stride), j = i + stride;
                            const bool up = (i & size) == 0;
                            const int ii = c_idx[i], ij = c_idx[j];
                            if ((ij < ii) == up) {
                                const uint32_t ki = c_key[i];
                                c_idx[i] = ij;
                                c_idx[j] = ii;
                                c_key[i] = c_key[j];
                                c_key[j] = ki;
                            }
                        }
                        __syncthreads();
                    }
                }
                if (Ck <= 64 && !a.probs) {
                    // up to 64 kept candidates and no distribution to write:
                    // wave 0 alone, candidate j in lane j (index order), the
                    // f64 sums across the wave, no barrier
                    if ((tid >> 6) != 0) return;
                    const int ln = tid & 63;
                    const bool on = ln < Ck;
                    const int ij = on ? c_idx[ln] : INT_MAX;
                    const float vj = on ? f32_from_order_key(c_key[ln]) / T : 0.f;
                    const double ej = on ? exp((double)(vj - mx)) : 0.0;
                    double sum = ej, zero = 0.0;
                    wave_sum2_d(sum, zero);
                    const double pj = ej / sum;
                    bool kept = false;
                    double resum = 1.0;
                    if (use_p) {
                        // the probabilities before this one in (p descending,
                        // then index: ascending for the nucleus cut,
                        // descending for sample()) order; kept as the block
                        // path's prefix rule
                        double before = 0.0;
                        for (int i = 0; i < Ck; i++) {
                            const double pi = __shfl(pj, i, 64);
                            const int ii = __shfl(ij, i, 64);
                            if (pi > pj || (pi == pj && (a.nucleus ? ii < ij : ii > ij))) before += pi;
                        }
                        const double limit = a.nucleus ? (double)a.top_p : (double)a.top_p * 1.5;
                        kept = on && (a.nucleus ? before < limit : before + pj <= limit);
                        double ks = kept ? pj : 0.0;
                        zero = 0.0;
                        wave_sum2_d(ks, zero);
                        resum = ks;
                    }
                    const double fj = on ? finish(pj, use_p && kept, resum) : 0.0;
                    // the inverse CDF in index order: the first candidate whose
                    // running sum exceeds the draw
                    double incl = fj;
                    for (int o = 1; o < 64; o <<= 1) {
                        const double y = __shfl_up(incl, o, 64);
                        if (ln >= o) incl += y;
                    }
                    const unsigned long long hit = __ballot(on && r < incl);
                    const int tok = hit ? __shfl(ij, __ffsll((long long)hit) - 1, 64) : n - 1;
                    emit(tok);
                    return;
                }
                // softmax over the kept (key >= tkey): the f64 exp of the f32
                // difference to the maximum, the sum in index order
                constexpr int PER = kSampleCap / kSampleThreads;
                double e[PER];
                double loc = 0.0;
#pragma unroll
                for (int q = 0; q < PER; q++) {
                    const int j = tid * PER + q;
                    e[q] = 0.0;
                    if (j < Ck) {
                        const float v = f32_from_order_key(c_key[j]) / T;
                        if (v >= thr) e[q] = exp((double)(v - mx));
                    }
                    loc += e[q];
                }
                const double sum = block_sum_f64(loc, red_d);
                double resum = 1.0;
                if (use_p) {
#pragma unroll
                    for (int q = 0; q < PER; q++) {
                        const int j = tid * PER + q;
                        if (j < Ck) {
                            s_p[j] = e[q] / sum;
                            s_idx[j] = c_idx[j];
                        }
                    }
                    __syncthreads();
                    resum = top_p_keep(Ck, std::isfinite(sum));
                }
                // the inverse CDF in index order over the candidates
                double f[PER];
                double seg = 0.0;
#pragma unroll
                for (int q = 0; q < PER; q++) {
                    const int j = tid * PER + q;
                    f[q] = j < Ck ? finish(e[q] / sum, use_p && is_kept(c_idx[j]), resum) : 0.0;
                    seg += f[q];
                }
                double total;
                double run = block_exclusive_scan_f64(seg, s_scan, &total);
                int cand = INT_MAX;
#pragma unroll
                for (int q = 0; q < PER; q++) {
                    const int j = tid * PER + q;
                    if (j < Ck) {
                        run += f[q];
                        if (cand == INT_MAX && r < run) cand = c_idx[j];
                    }
                }
                int tok = block_min_i32(cand, red_i);
                if (tok == INT_MAX) tok = n - 1;
                if (a.probs) {
                    // every other entry: 0, or 0 / resum as the reference divides
                    const double rest = finish(0.0, false, resum);
                    for (int i = tid; i < n; i += kSampleThreads) a.probs[(size_t)row * n + i] = rest;
                    __threadfence_block();
                    __syncthreads();
#pragma unroll
                    for (int q = 0; q < PER; q++) {
                        const int j = tid * PER + q;
                        if (j < Ck) a.probs[(size_t)row * n + c_idx[j]] = f[q];
                    }
                }
                emit(tok);
                return;
            }
        }
    }

    // top-k threshold (model/generate.go:155-163): the top_k-th largest
    // scaled value, counting equal values
    float thr = -INFINITY;
    if (use_k)
        thr = f32_from_order_key(radix_kth([&](int i) { return f32_order_key(lg[i] / T); }, n, a.top_k));
    // (top-k rows reach here with more than kSampleCap candidates, a NaN,
    // or a scaled tie below the candidates' bin)
    // the scaled value of a logit x, -inf below the top-k threshold
    auto value = [&](float x) {
        const float v = x / T;
        return (use_k && v < thr) ? -INFINITY : v;
    };

    // softmax in f64 of the f32 differences to the maximum (:165-180)
    float mx = -INFINITY;
    for (int base = 0; base < n; base += kRowUnroll * kSampleThreads) {
        float v[kRowUnroll];
        load_row(base, v);
#pragma unroll
        for (int u = 0; u < kRowUnroll; u++)
            if (base + u * kSampleThreads + tid < n) mx = fmaxf(mx, value(v[u]));
    }
    mx = block_max_f32(mx, red_f);
    // (exp of -inf is 0: entries below the top-k threshold skip the f64 exp)
    auto expo = [&](float x) {
        const float v = value(x);
        return v == -INFINITY ? 0.0 : exp((double)(v - mx));
    };
    // the f64 sum over 16 contiguous wave ranges of the row (seg entries,
    // a multiple of 64, read 64 at a time), added in wave order; the
    // inverse CDF below walks the same ranges
    const int lane = tid & 63, wave = tid >> 6;
    const int seg = ((n + kSampleThreads / 64 - 1) / (kSampleThreads / 64) + 63) & ~63;
    const int w0 = min(n, wave * seg), w1 = min(n, w0 + seg);
    // entries base + lane + 64 u (u < kRowUnroll), all loads in flight
    auto load_range = [&](int base, float (&v)[kRowUnroll]) {
#pragma unroll
        for (int u = 0; u < kRowUnroll; u++)
            v[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rrow, (base + lane + 64 * u) * 4, 0, 0));
    };
    double esum = 0.0;
    for (int base = w0; base < w1; base += 64 * kRowUnroll) {
        float v[kRowUnroll];
        load_range(base, v);
#pragma unroll
        for (int u = 0; u < kRowUnroll; u++)
            if (base + lane + 64 * u < w1) esum += expo(v[u]);
    }
    esum = wave_sum_d(esum);
    if (lane == 0) red_d[wave] = esum;
    __syncthreads();
    double sum = 0.0;
    for (int w = 0; w < kSampleThreads / 64; w++) sum += red_d[w];
    __syncthreads();

    // top-p (:182-229) over the positive probabilities
    double resum = 1.0;
    if (use_p) {
        if (tid == 0) s_cnt = 0;
        __syncthreads();
        for (int base = 0; base < n; base += kRowUnroll * kSampleThreads) {
            float v[kRowUnroll];
            load_row(base, v);
#pragma unroll
            for (int u = 0; u < kRowUnroll; u++) {
                const int i = base + u * kSampleThreads + tid;
                const double p = i < n ? expo(v[u]) / sum : 0.0;
                if (p > 0.0) {
                    const int slot = atomicAdd(&s_cnt, 1);
                    if (slot < kSampleCap) {
                        s_p[slot] = p;
                        s_idx[slot] = i;
                    }
                }
            }
        }
        __syncthreads();
        const int cnt = s_cnt;
        if (cnt > kSampleCap) {
            if (tid == 0) {
                if (a.err) atomicOr(a.err, 1);
                if (a.out) a.out[row] = -1;
            }
            return;
        }
        resum = top_p_keep(cnt, false);
    }
    auto final_p = [&](int i, float x) { return finish(expo(x) / sum, use_p && is_kept(i), resum); };

    // the draw and the inverse CDF in index order (:231-240) over the wave
    // ranges: each range's share of the final distribution (without top-p
    // its exp sum over the total; with it a pass of the final values), the
    // shares added in wave order, and only the wave whose range holds the
    // crossing (or every wave, when the distribution is written out) scans
    // its range again, 64 entries per step
    double rsum = 0.0;
    if (use_p) {
        for (int base = w0; base < w1; base += 64 * kRowUnroll) {
            float v[kRowUnroll];
            load_range(base, v);
#pragma unroll
            for (int u = 0; u < kRowUnroll; u++) {
                const int i = base + lane + 64 * u;
                if (i < w1) rsum += final_p(i, v[u]);
            }
        }
        rsum = wave_sum_d(rsum);
    } else {
        rsum = esum / sum;
    }
    if (lane == 0) s_scan[wave] = rsum;
    __syncthreads();
    double cum = 0.0;
    for (int w = 0; w < wave; w++) cum += s_scan[w];
    int cand = INT_MAX;
    if (a.probs || (r >= cum && r < cum + rsum)) {
        for (int base = w0; base < w1; base += 64) {
            const int i = base + lane;
            const double p = i < w1 ? final_p(i, lg[i]) : 0.0;
            if (a.probs && i < w1) a.probs[(size_t)row * n + i] = p;
            double inc = p;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const double t = __shfl_up(inc, o);
                if (lane >= o) inc += t;
            }
            const unsigned long long hit = __ballot(i < w1 && r < cum + inc);
            if (hit && cand == INT_MAX) cand = base + (int)__builtin_ctzll(hit);
            cum += readlane_d(inc, 63);
            if (cand != INT_MAX && !a.probs) break;
        }
        // within rounding of the range's end the rescan may not cross where
        // the range sums did: the range's last entry then
        if (cand == INT_MAX && w1 > w0 && r < cum) cand = w1 - 1;
    }
    int tok = block_min_i32(cand, red_i);
    if (tok == INT_MAX) tok = n - 1;
    emit(tok);
}

size_t sample_ws_bytes(int rows) { return (size_t)rows * kWsRowInts * sizeof(int); }

int launch_sample(hipStream_t s, const float* logits, int rows, int n, float temperature, int top_k, float top_p,
                  const double* u, unsigned long long seed, const int* step, int* out, double* probs,
                  unsigned long long* key, int* err, bool nucleus, int* ws) {
    SampleArgs a{logits, n, temperature, top_k, top_p, u, seed, step, out, probs, key, err, nucleus ? 1 : 0};
    if (ws && top_k > 0 && top_k < n && top_k <= kSampleCap && n >= kSampleWsMinN) {
        // the candidate search's two row passes over many blocks per row
        // (about 2048 entries each, at most ~512 blocks in all)
        const int G = std::max(1, std::min((n + 2047) / 2048, std::max(1, 512 / rows)));
        const int chunk = ((n + G - 1) / G + kScanThreads - 1) / kScanThreads * kScanThreads;
        const int g = (n + chunk - 1) / chunk;
        hipLaunchKernelGGL(k_sample_scan, dim3(g, rows), dim3(kScanThreads), 0, s, logits, n, chunk, ws);
        GH_TRY(check_launch("sample_scan"));
        hipLaunchKernelGGL(k_sample_gather, dim3(g, rows), dim3(kScanThreads), 0, s, logits, n, chunk, top_k, ws);
        GH_TRY(check_launch("sample_gather"));
        a.ws = ws;
    }
    hipLaunchKernelGGL(k_sample, dim3(rows), dim3(kSampleThreads), 0, s, a);
    count(CNT_ARGMAX);
    return check_launch("sample");
}

int sample_check(int rows, int n, float temperature, int top_k, float top_p) {
    if (rows < 1 || n < 1) {
        set_error("sample: needs rows >= 1 and n >= 1");
        return GORCH_HIP_EINVAL;
    }
    if (!(temperature > 0.f) || !std::isfinite(temperature)) {
        set_error("sample: temperature must be finite and > 0 (0 is the greedy argmax)");
        return GORCH_HIP_EINVAL;
    }
    if (top_k < 0) {
        set_error("sample: top_k must be >= 0");
        return GORCH_HIP_EINVAL;
    }
    if (n > kSampleMaxN) {
        set_error("sample: at most 262144 columns");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if (top_p > 0.f && top_p < 1.f && (top_k < 1 || top_k > kSampleCap)) {
        set_error("sample: top_p runs on the device with 1 <= top_k <= 4096");
        return GORCH_HIP_EUNSUPPORTED;
    }
    return GORCH_HIP_OK;
}

}  // namespace gh

using namespace gh;

extern "C" int gorch_hip_sample(void* stream, const float* logits, int rows, int n, float temperature, int top_k,
                                float top_p, const double* u, int* out, double* probs) {
    GH_REQUIRE(logits && u && out, "gorch_hip_sample: null logits, draws or output");
    GH_TRY(sample_check(rows, n, temperature, top_k, top_p));
    return launch_sample(stream_of(stream), logits, rows, n, temperature, top_k, top_p, u, 0ull, nullptr, out, probs,
                         nullptr, nullptr, false);
}

extern "C" int gorch_hip_sample_nucleus(void* stream, const float* logits, int rows, int n, float temperature,
                                        int top_k, float top_p, const double* u, int* out, double* probs) {
    GH_REQUIRE(logits && u && out, "gorch_hip_sample_nucleus: null logits, draws or output");
    GH_TRY(sample_check(rows, n, temperature, top_k, top_p));
    return launch_sample(stream_of(stream), logits, rows, n, temperature, top_k, top_p, u, 0ull, nullptr, out, probs,
                         nullptr, nullptr, true);
}

extern "C" size_t gorch_hip_sample_workspace_size(int rows) { return rows > 0 ? sample_ws_bytes(rows) : 0; }

extern "C" int gorch_hip_sample_with_workspace(void* stream, const float* logits, int rows, int n, float temperature,
                                               int top_k, float top_p, const double* u, int* out, double* probs,
                                               int nucleus, void* workspace) {
    GH_REQUIRE(logits && u && out && workspace, "gorch_hip_sample_with_workspace: null logits, draws, output or workspace");
    GH_TRY(sample_check(rows, n, temperature, top_k, top_p));
    return launch_sample(stream_of(stream), logits, rows, n, temperature, top_k, top_p, u, 0ull, nullptr, out, probs,
                         nullptr, nullptr, nucleus != 0, static_cast<int*>(workspace));
}
