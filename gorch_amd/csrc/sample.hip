// sample.hip — the sampled next-token choice of generateCached with
// Temperature > 0 (model/generate.go:105-110; sample() at :147-243,
// kthLargest at :247-262) and of the Qwen Generate loop (sampleLogits,
// model/qwen/generate.go:94-181), one 1024-thread block per row of logits.
//
//   scaled = logits / temperature (f32)
//   0 < top_k < n: values below the top_k-th largest scaled value -> -inf
//     (the threshold found by a 4-pass radix select over order-preserving
//     32-bit keys, 256-bin histograms in LDS: the value kthLargest returns)
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
// Exclusive prefix of one f64 per thread in thread order (Hillis-Steele in
// LDS); returns this thread's exclusive prefix, *total the block's sum.
__device__ double block_exclusive_scan_f64(double v, double* sc, double* total) {
    const int t = threadIdx.x;
    sc[t] = v;
    __syncthreads();
    for (int o = 1; o < kSampleThreads; o <<= 1) {
        const double add = t >= o ? sc[t - o] : 0.0;
        __syncthreads();
        sc[t] += add;
        __syncthreads();
    }
    const double incl = sc[t];
    *total = sc[kSampleThreads - 1];
    __syncthreads();
    return incl - v;
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
};

__global__ __launch_bounds__(kSampleThreads) void k_sample(SampleArgs a) {
    __shared__ int hist[256];
    __shared__ double red_d[kSampleThreads / 64];
    __shared__ float red_f[kSampleThreads / 64];
    __shared__ int red_i[kSampleThreads / 64];
    __shared__ uint32_t s_prefix;
    __shared__ int s_k, s_cnt;
    __shared__ double s_p[kSampleCap];
    __shared__ int s_idx[kSampleCap];
    __shared__ double s_scan[kSampleThreads];
    __shared__ uint32_t s_keep[kSampleMaxN / 32];  // kept indices (top-p)
    const int row = blockIdx.x, tid = threadIdx.x, n = a.n;
    const float* lg = a.logits + (size_t)row * n;
    const float T = a.temperature;

    // top-k threshold (model/generate.go:155-163): the top_k-th largest
    // scaled value, counting equal values
    const bool use_k = a.top_k > 0 && a.top_k < n;
    float thr = -INFINITY;
    if (use_k) {
        uint32_t prefix = 0u, mask = 0u;
        int k = a.top_k;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int b = tid; b < 256; b += kSampleThreads) hist[b] = 0;
            __syncthreads();
            for (int i = tid; i < n; i += kSampleThreads) {
                const uint32_t key = f32_order_key(lg[i] / T);
                if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
            }
            __syncthreads();
            if (tid == 0) {
                int cum = 0, d = 255;
                for (; d > 0; d--) {
                    if (cum + hist[d] >= k) break;
                    cum += hist[d];
                }
                s_prefix = prefix | ((uint32_t)d << shift);
                s_k = k - cum;
            }
            __syncthreads();
            prefix = s_prefix;
            k = s_k;
            mask |= 255u << shift;
        }
        thr = f32_from_order_key(prefix);
    }
    auto value = [&](int i) {
        const float v = lg[i] / T;
        return (use_k && v < thr) ? -INFINITY : v;
    };

    // softmax in f64 of the f32 differences to the maximum (:165-180)
    float mx = -INFINITY;
    for (int i = tid; i < n; i += kSampleThreads) mx = fmaxf(mx, value(i));
    mx = block_max_f32(mx, red_f);
    // (exp of -inf is 0: entries below the top-k threshold skip the f64 exp)
    auto expo = [&](int i) {
        const float v = value(i);
        return v == -INFINITY ? 0.0 : exp((double)(v - mx));
    };
    double part = 0.0;
    for (int i = tid; i < n; i += kSampleThreads) part += expo(i);
    const double sum = block_sum_f64(part, red_d);

    // top-p (:182-229)
    const bool use_p = a.top_p > 0.f && a.top_p < 1.f;
    double resum = 1.0;
    if (use_p) {
        if (tid == 0) s_cnt = 0;
        __syncthreads();
        for (int i = tid; i < n; i += kSampleThreads) {
            const double p = expo(i) / sum;
            if (p > 0.0) {
                const int slot = atomicAdd(&s_cnt, 1);
                if (slot < kSampleCap) {
                    s_p[slot] = p;
                    s_idx[slot] = i;
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
        int P = 1;
        while (P < cnt) P <<= 1;
        for (int i = cnt + tid; i < P; i += kSampleThreads) {
            s_p[i] = -1.0;
            s_idx[i] = -1;
        }
        __syncthreads();
        // bitonic sort into (p descending, index descending)
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
        // kept: the longest sorted prefix whose sum is at most the limit
        // (the prefix sums increase with its length); nucleus: every entry
        // whose preceding sum is still below top_p
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
        resum = block_sum_f64(kept_sum, red_d);
        // kept indices as a bitmap over n
        const int words = (n + 31) / 32;
        for (int w = tid; w < words; w += kSampleThreads) s_keep[w] = 0u;
        __syncthreads();
        for (int j = tid; j < L; j += kSampleThreads) atomicOr(&s_keep[s_idx[j] >> 5], 1u << (s_idx[j] & 31));
        __syncthreads();
    }
    // (with top-p every value is divided by the kept sum, as the reference
    // does: 0/0 = NaN everywhere when nothing was kept, and the draw then
    // falls through to n - 1)
    auto final_p = [&](int i) {
        const double p = expo(i) / sum;
        if (!use_p) return p;
        const bool kept = (s_keep[i >> 5] >> (i & 31)) & 1u;
        if (a.nucleus) return kept ? p / resum : 0.0;
        return (kept ? p : 0.0) / resum;
    };

    // the draw and the inverse CDF in index order (:231-240): wave w owns
    // the contiguous range [w * seg, (w + 1) * seg) of the row (seg a
    // multiple of 64) and reads it 64 consecutive entries at a time; the
    // range sums are added in wave order, and only the wave whose range
    // holds the crossing (or every wave, when the distribution is written
    // out) scans its range again, 64 entries per step
    const double r = a.u ? a.u[row] : philox_uniform(a.seed, (uint32_t)*a.step, (uint32_t)row);
    const int lane = tid & 63, wave = tid >> 6;
    const int seg = ((n + kSampleThreads / 64 - 1) / (kSampleThreads / 64) + 63) & ~63;
    const int w0 = min(n, wave * seg), w1 = min(n, w0 + seg);
    double rsum = 0.0;
    for (int i = w0 + lane; i < w1; i += 64) rsum += final_p(i);
    rsum = wave_sum_d(rsum);
    if (lane == 0) s_scan[wave] = rsum;
    __syncthreads();
    double cum = 0.0;
    for (int w = 0; w < wave; w++) cum += s_scan[w];
    int cand = INT_MAX;
    if (a.probs || (r >= cum && r < cum + rsum)) {
        for (int base = w0; base < w1; base += 64) {
            const int i = base + lane;
            const double p = i < w1 ? final_p(i) : 0.0;
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
    if (tid == 0) {
        if (a.out) a.out[row] = tok;
        // a key the fused-argmax consumers decode to tok (slot 0 of row)
        if (a.key) a.key[row] = (1ull << 32) | (unsigned long long)(0xffffffffu - (uint32_t)tok);
    }
}

int launch_sample(hipStream_t s, const float* logits, int rows, int n, float temperature, int top_k, float top_p,
                  const double* u, unsigned long long seed, const int* step, int* out, double* probs,
                  unsigned long long* key, int* err, bool nucleus) {
    SampleArgs a{logits, n, temperature, top_k, top_p, u, seed, step, out, probs, key, err, nucleus ? 1 : 0};
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
