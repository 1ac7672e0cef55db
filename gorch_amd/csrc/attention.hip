// attention.hip — attention over the KV cache for new query rows
// (MHA.ForwardCached's per-head loops, nn/attention.go:355-397), the fused
// staircase-causal softmax (causalSoftmaxForwardCPU, softmax_metal.go:111-141;
// MSL softmax_causal_forward, metal/kernels.go:260-332) and the plain row
// softmax (softmaxInPlace, nn/attention.go:274-296).
//
// Cache layout in HBM (f32, the reference's KVCache element type): per layer
// K and V are [batch][max_seq][dim] with heads interleaved along dim, i.e.
// one token's row is contiguous (nn/kvcache.go:14-19), so a head's 64-float
// slice is a 256-byte segment.
//
// k_attn_cached: one 256-thread block per (head, query row). Scores for all
// visible keys are staged in LDS (4 lanes per key, 64 keys per block
// iteration, 2-step shuffle reduce); block max / sum by LDS reduction; then
// P.V with lanes across the head's dims (coalesced 256-byte rows) and waves
// across keys, the 4 wave partials summed in wave order.
#include <algorithm>

#include "common.h"

namespace gh {

// Four consecutive output columns of row `row` (col % 4 == 0): f32 to
// a.out, or hi/lo halves to a.out_frag (8-byte stores: one lane's group of
// eight columns holds all four)
__device__ __forceinline__ void attn_out4(const AttnArgs& a, int row, int col, float4 t) {
    if (a.out_frag) {
        const float v[4] = {t.x, t.y, t.z, t.w};
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 4; e++) split_hi_lo1(v[e], hi[e], lo[e]);
        const size_t i = xfrag_index(row, col);
        *reinterpret_cast<uint2*>(a.out_frag + i) =
            make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
        *reinterpret_cast<uint2*>(a.out_frag + i + 512) =
            make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
    } else {
        *reinterpret_cast<float4*>(a.out + (size_t)row * a.dim + col) = t;
    }
}
// one output column: f32, or its hi/lo halves
__device__ __forceinline__ void attn_out1(const AttnArgs& a, int row, int col, float v) {
    if (a.out_frag) {
        uint16_t hi, lo;
        split_hi_lo1(v, hi, lo);
        const size_t i = xfrag_index(row, col);
        a.out_frag[i] = hi;
        a.out_frag[i + 512] = lo;
    } else {
        a.out[(size_t)row * a.dim + col] = v;
    }
}

__device__ float block_max(float v, float* sh) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float t = sh[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) t = fmaxf(t, sh[w]);
    __syncthreads();
    return t;
}

__device__ float block_sum(float v, float* sh) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) t += sh[w];
    __syncthreads();
    return t;
}


template <int NWV>
__global__ __launch_bounds__(NWV * 64) void k_attn_cached(AttnArgs a) {
    extern __shared__ float sc[];  // [max visible keys]
    __shared__ __align__(16) float qs[256];
    __shared__ float red[16];
    __shared__ float pv[NWV][256];

    const int h = blockIdx.x;
    const int row = blockIdx.y;
    const int b = row / a.new_seq;
    const int i = row - b * a.new_seq;
    const int pos = a.pos_dev ? *a.pos_dev : a.pos_host;
    const int T = a.causal ? pos + i + 1 : pos + a.new_seq;
    const int hd = a.hd;
    // grouped-query attention: query head h reads KV head h / (heads / kv_heads)
    const int kvh = a.kv_heads ? h / ((int)gridDim.x / a.kv_heads) : h;
    const int kvd = a.kv_dim ? a.kv_dim : a.dim;
    const size_t base = ((size_t)b * a.max_seq) * kvd + (size_t)kvh * hd;
    const float* K = a.kc + base;
    const float* V = a.vc + base;

    if (a.qkv_part) {
        // q, k, v of this head from the split QKV Linear's partials: slices
        // added in order, then the bias (k_splitk_epilogue's order); k and v
        // go to cache row pos (i = 0), which the score and P.V loops below
        // read back after the barrier. Buffer loads past the slice count
        // read zeros, so all of a lane's loads go out together.
        const int D = a.dim, S = a.qkv_slices;
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.qkv_part, (long long)S * a.qkv_slice_stride * 4);
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.qkv_bias, a.qkv_bias ? (long long)3 * D * 4 : 0);
        for (int d = threadIdx.x; d < hd; d += blockDim.x) {
            const int c = h * hd + d;
            float p[3][kMaxPartSlices];
#pragma unroll
            for (int s = 0; s < kMaxPartSlices; s++)
#pragma unroll
                for (int t = 0; t < 3; t++) {
                    const long long e = s * a.qkv_slice_stride + (long long)row * 3 * D + t * D + c;
                    p[t][s] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rp, s < S ? (int)(e * 4) : kOutOfRange, 0, 0));
                }
            float o[3];
#pragma unroll
            for (int t = 0; t < 3; t++) {
                float v = p[t][0];
#pragma unroll
                for (int s = 1; s < kMaxPartSlices; s++)
                    if (s < S) v = v + p[t][s];
                const float bv =
                    __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, (t * D + c) * 4, 0, 0));
                o[t] = a.qkv_bias ? v + bv : v;
            }
            qs[d] = o[0];
            const size_t at = (size_t)pos * kvd + d;
            const_cast<float*>(K)[at] = o[1];
            const_cast<float*>(V)[at] = o[2];
        }
    } else {
        for (int d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = a.q[(size_t)row * a.q_stride + h * hd + d];
    }
    __syncthreads();

    // scores: 4 lanes per key, each taking every 4th float4 of the head (so
    // the 4 lanes read 64 contiguous bytes per load); 16 keys per wavefront
    // and 64 per block per iteration, all loads of a lane issued together.
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane & 3, kslot = lane >> 2;
    const int hd4 = hd >> 2;
    const float4* q4 = reinterpret_cast<const float4*>(qs);
    float lmax = -INFINITY;
    for (int j0 = wave * 16; j0 < T; j0 += 16 * NWV) {
        const int j = j0 + kslot;
        float acc = 0.f;
        if (j < T) {
            const float4* kr = reinterpret_cast<const float4*>(K + (size_t)j * kvd);
#pragma unroll 4
            for (int d4 = sub; d4 < hd4; d4 += 4) {
                float4 kv = kr[d4];
                float4 qv = q4[d4];
                acc += qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
            }
        }
        acc = seg_sum<4>(acc);
        if (j < T && sub == 0) {
            float s = acc * a.scale;
            sc[j] = s;
            lmax = fmaxf(lmax, s);
        }
    }
    const float mx = block_max(lmax, red);

    float lsum = 0.f;
    for (int j = threadIdx.x; j < T; j += blockDim.x) {
        float e = expf(sc[j] - mx);
        sc[j] = e;
        lsum += e;
    }
    const float sum = block_sum(lsum, red);
    const float rs = 1.0f / sum;
    for (int j = threadIdx.x; j < T; j += blockDim.x) sc[j] = a.recip ? sc[j] * rs : sc[j] / sum;
    __syncthreads();

    // P.V: waves take keys j = wave, wave+NWV, ...; lanes take dims (one
    // coalesced 256-byte row per key); independent accumulators keep eight
    // (then four) rows in flight per lane.
    for (int d0 = 0; d0 < hd; d0 += 64) {
        const int d = d0 + lane;
        if (d < hd) {
            const float* Vd = V + d;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            int j = wave;
            // (measured at XL batch 16: 5,202 -> 5,227 tok/s against four)
            float a4 = 0.f, a5 = 0.f, a6 = 0.f, a7 = 0.f;
            for (; j + 7 * NWV < T; j += 8 * NWV) {
                a0 += sc[j] * Vd[(size_t)j * kvd];
                a1 += sc[j + NWV] * Vd[(size_t)(j + NWV) * kvd];
                a2 += sc[j + 2 * NWV] * Vd[(size_t)(j + 2 * NWV) * kvd];
                a3 += sc[j + 3 * NWV] * Vd[(size_t)(j + 3 * NWV) * kvd];
                a4 += sc[j + 4 * NWV] * Vd[(size_t)(j + 4 * NWV) * kvd];
                a5 += sc[j + 5 * NWV] * Vd[(size_t)(j + 5 * NWV) * kvd];
                a6 += sc[j + 6 * NWV] * Vd[(size_t)(j + 6 * NWV) * kvd];
                a7 += sc[j + 7 * NWV] * Vd[(size_t)(j + 7 * NWV) * kvd];
            }
            a0 += a4;
            a1 += a5;
            a2 += a6;
            a3 += a7;
            for (; j + 3 * NWV < T; j += 4 * NWV) {
                a0 += sc[j] * Vd[(size_t)j * kvd];
                a1 += sc[j + NWV] * Vd[(size_t)(j + NWV) * kvd];
                a2 += sc[j + 2 * NWV] * Vd[(size_t)(j + 2 * NWV) * kvd];
                a3 += sc[j + 3 * NWV] * Vd[(size_t)(j + 3 * NWV) * kvd];
            }
            for (; j < T; j += NWV) a0 += sc[j] * Vd[(size_t)j * kvd];
            pv[wave][d] = (a0 + a1) + (a2 + a3);
        }
    }
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = pv[0][d];
#pragma unroll
        for (int w = 1; w < NWV; w++) o = o + pv[w][d];
        attn_out1(a, row, h * hd + d, o);
    }
}

// k_attn_rows: the same computation with lanes over (key, 16-byte chunk of
// the head): HD4 = hd/4 lanes read one key's 64..512-byte head slice, so a
// wavefront instruction covers 64/HD4 keys and a lane issues the loads of
// UNR keys at once. Scores, softmax and P.V then take about one memory round
// trip each, instead of one per key-loop iteration (what limits the
// per-(head, row) block when the context is short and blocks are few).
//
// FULL: KB * UNR >= max_seq, so one chunk covers the whole cache. The K and
// V loads then span the cache's capacity rather than the visible length,
// and are issued before the cache length (written by the previous kernel)
// has arrived; keys at or past it are masked in the arithmetic (selects, so
// whatever the unused rows hold never reaches the result).
//
// WO (FULL, one row): the output projection in the same kernel. blockIdx.y
// is a group of WR rows of Wo; every block of head h computes that head's
// attention output o_h (the same values in each), then adds
// Wo[n][h*hd .. h*hd+hd) . o_h (+ the bias, from head 0) into a.wo_out[n]
// for its rows with float atomics. The Wo loads go out with the K/V loads.
constexpr int kWoRows = 48;  // Wo rows per block of the fused projection
template <int HD4, int UNR, bool FULL, int NW = 4, bool WO = false>
__global__ __launch_bounds__(NW * 64) void k_attn_rows(AttnArgs a) {
    extern __shared__ float sc[];  // [visible keys]
    __shared__ float red[16];
    __shared__ float4 po[NW][64];
    __shared__ float pl[NW][64];
    constexpr int KPI = 64 / HD4;  // keys per wavefront instruction
    constexpr int KB = NW * KPI;   // keys per block instruction
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane % HD4, slot = wave * KPI + lane / HD4;

    const int h = blockIdx.x;
    const int row = WO ? 0 : blockIdx.y;
    const int b = row / a.new_seq;
    const int i = row - b * a.new_seq;
    const int kvh = a.kv_heads ? h / ((int)gridDim.x / a.kv_heads) : h;
    const int kvd = a.kv_dim ? a.kv_dim : a.dim;
    const size_t base = ((size_t)b * a.max_seq) * kvd + (size_t)kvh * (4 * HD4);
    // the cache length as a vector load issued after the K/V loads when FULL
    // (a scalar load would share its wait counter with the kernel arguments
    // and hold back the K/V stream)
    auto load_pos = [&]() {
        if (!a.pos_dev) return a.pos_host;
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.pos_dev, 4);
        return __builtin_amdgcn_readfirstlane((int)__builtin_amdgcn_raw_buffer_load_b32(rp, 0, 0, 0));
    };
    int T = 0;
    if constexpr (!FULL) {
        const int pos = load_pos();
        T = a.causal ? pos + i + 1 : pos + a.new_seq;
    }
    // raw buffer resources over this head's slices of keys 0..T-1: keys at
    // or past T fall outside and read as zeros, with no branch around the
    // loads (a load under a branch makes the compiler wait for every
    // outstanding load before its first use)
    const int rows_read = FULL ? a.max_seq : T;
    const long long span = rows_read > 0 ? ((long long)(rows_read - 1) * kvd + 4 * HD4) * 4 : 0;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.kc + base, span);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.vc + base, span);
    auto kv_off = [&](int j) { return j * kvd * 4 + 16 * c; };
    auto ld4 = [](__amdgpu_buffer_rsrc_t rs, int off) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kStreamPolicy);
        return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                           __uint_as_float(v[3]));
    };
    const float4 q = *reinterpret_cast<const float4*>(a.q + (size_t)row * a.q_stride + h * (4 * HD4) + 4 * c);
    // the first chunk's keys and values in one round trip: V does not
    // depend on the scores
    float4 kv[UNR], vpre[UNR];
#pragma unroll
    for (int u = 0; u < UNR; u++) kv[u] = ld4(rk, kv_off(KB * u + slot));
#pragma unroll
    for (int u = 0; u < UNR; u++) vpre[u] = ld4(rv, kv_off(KB * u + slot));
    // fused projection: thread (row rr, 16-byte chunk cc) of the block's Wo
    // rows; rows past the block's group or past dim read zeros
    constexpr int WCH = HD4 / 2;                  // 16-byte chunks of a head's Wo row slice
    constexpr int WRP = NW * 64 / WCH;            // Wo rows per pass
    constexpr int WPASS = (kWoRows + WRP - 1) / WRP;
    const int cc = threadIdx.x % WCH, rr = threadIdx.x / WCH;
    u32x4 wov[WO ? WPASS : 1];
    float wob[WO ? WPASS : 1];  // head 0's bias values, loaded with Wo (no load in the epilogue)
    if constexpr (WO) {
        const int n0 = blockIdx.y * kWoRows;
        const int nrows = max(0, min(kWoRows, a.dim - n0));
        const __amdgpu_buffer_rsrc_t rw =
            make_rsrc(a.wo + (size_t)n0 * a.dim + h * (4 * HD4), nrows > 0 ? ((long long)(nrows - 1) * a.dim + 4 * HD4) * 2 : 0);
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.wo_bias + n0, (h == 0 && a.wo_bias) ? (long long)nrows * 4 : 0);
#pragma unroll
        for (int q = 0; q < WPASS; q++) {
            const int rl = rr + q * WRP;
            wov[q] = __builtin_amdgcn_raw_buffer_load_b128(rw, rl < nrows ? (rl * a.dim + 8 * cc) * 2 : kOutOfRange, 0,
                                                         kStreamPolicy);
            wob[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, rl * 4, 0, 0));
        }
    }
    if constexpr (FULL) {
        const int pos = load_pos();
        T = a.causal ? pos + i + 1 : pos + a.new_seq;
        // one chunk covers the cache (T <= max_seq <= KB * UNR): the scores
        // stay in registers, each key slot weights its values by p = exp(s -
        // max), and the slots' weighted sums and weight sums meet in LDS once
        // (sum_j p_j v_j / sum_j p_j: the softmax-weighted sum, divided last)
        float sj[UNR];
        float smax = -INFINITY;
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            float d = q.x * kv[u].x + q.y * kv[u].y + q.z * kv[u].z + q.w * kv[u].w;
            sj[u] = seg_sum<HD4>(d) * a.scale;
            if (KB * u + slot < T) smax = fmaxf(smax, sj[u]);
        }
        const float mx = block_max(smax, red);
        float l = 0.f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            // keys past T: cache rows not written yet, never multiplied
            if (KB * u + slot < T) {
                const float p = expf(sj[u] - mx);
                l += p;
                o.x += p * vpre[u].x;
                o.y += p * vpre[u].y;
                o.z += p * vpre[u].z;
                o.w += p * vpre[u].w;
            }
        }
        po[wave][lane] = o;
        pl[wave][lane] = l;
        __syncthreads();
        if (threadIdx.x < HD4) {
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
            float L = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++)
#pragma unroll
                for (int sl = 0; sl < KPI; sl++) {
                    const float4 pv = po[w][sl * HD4 + c];
                    t.x += pv.x;
                    t.y += pv.y;
                    t.z += pv.z;
                    t.w += pv.w;
                    L += pl[w][sl * HD4 + c];
                }
            if (a.recip) {
                const float rs = 1.0f / L;
                t = make_float4(t.x * rs, t.y * rs, t.z * rs, t.w * rs);
            } else {
                t = make_float4(t.x / L, t.y / L, t.z / L, t.w / L);
            }
            if constexpr (WO) po[0][c] = t;
            else attn_out4(a, row, h * (4 * HD4) + 4 * c, t);
        }
        if constexpr (WO) {
            __syncthreads();
            // this thread's 8 head dims (16-byte Wo chunk cc) of o_h
            const float4 t0 = po[0][2 * cc], t1 = po[0][2 * cc + 1];
            const float o8[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
            const int n0 = blockIdx.y * kWoRows;
#pragma unroll
            for (int q = 0; q < WPASS; q++) {
                float v = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) v += bf16_lo(e & 1 ? wov[q][e >> 1] >> 16 : wov[q][e >> 1] & 0xffffu) * o8[e];
                v = seg_sum<WCH>(v);
                const int rl = rr + q * WRP, n = n0 + rl;
                if (cc == 0 && rl < kWoRows && n < a.dim) {
                    if (h == 0 && a.wo_bias) v = v + wob[q];
                    __hip_atomic_fetch_add(a.wo_out + n, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        return;
    }

    float lmax = -INFINITY;
    for (int j0 = 0; j0 < T; j0 += KB * UNR) {
        if (j0 > 0) {
#pragma unroll
            for (int u = 0; u < UNR; u++) kv[u] = ld4(rk, kv_off(j0 + KB * u + slot));
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            float d = q.x * kv[u].x + q.y * kv[u].y + q.z * kv[u].z + q.w * kv[u].w;
            d = seg_sum<HD4>(d);
            const int j = j0 + KB * u + slot;
            if (c == 0 && j < T) {
                const float sj = d * a.scale;
                sc[j] = sj;
                lmax = fmaxf(lmax, sj);
            }
        }
    }
    const float mx = block_max(lmax, red);
    float lsum = 0.f;
    for (int j = threadIdx.x; j < T; j += blockDim.x) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        lsum += e;
    }
    const float sum = block_sum(lsum, red);
    const float rs = 1.0f / sum;
    for (int j = threadIdx.x; j < T; j += blockDim.x) sc[j] = a.recip ? sc[j] * rs : sc[j] / sum;
    __syncthreads();

    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j0 = 0; j0 < T; j0 += KB * UNR) {
        float4 vv[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++) vv[u] = j0 == 0 ? vpre[u] : ld4(rv, kv_off(j0 + KB * u + slot));
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int j = j0 + KB * u + slot;
            if (j < T) {
                const float p = sc[j];
                o.x += p * vv[u].x;
                o.y += p * vv[u].y;
                o.z += p * vv[u].z;
                o.w += p * vv[u].w;
            }
        }
    }
    // the NW waves' key slots, in order (wave, slot)
    po[wave][lane] = o;
    __syncthreads();
    if (threadIdx.x < HD4) {
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < NW; w++)
#pragma unroll
            for (int sl = 0; sl < KPI; sl++) {
                const float4 pv = po[w][sl * HD4 + c];
                t.x += pv.x;
                t.y += pv.y;
                t.z += pv.z;
                t.w += pv.w;
            }
        attn_out4(a, row, h * (4 * HD4) + 4 * c, t);
    }
}

// ---------------------------------------------------------------------------
// k_attn_flash: attention for many new rows at once (prefill; MHA.Forward's
// causal case, nn/attention.go:64-145, as the cached path's prompt pass) on
// the f32 matrix cores (v_mfma_f32_16x16x4_f32: products and sums in f32).
//
// A block of NW waves takes 16 * NW consecutive query rows of one (sequence,
// head); wave w owns 16 of them. Keys stream through LDS in stages of KT:
// K row-major [key][dim] and V transposed [dim][key], loaded once per block
// for all its waves. Per 16-key slice a wave computes S^T = K Q^T (lane
// (r, g) then holds keys 4g .. 4g+3 of query r), applies the scale
// ((q.k) * scale, as the reference), the causal mask and an online softmax
// per query (running max m and per-lane partial sums l rescaled by
// exp(m_old - m_new)), and accumulates O^T += V^T P^T: the probabilities are
// already in the B-operand position when the MFMA's k index runs over the
// keys a lane holds, so P never leaves registers. O = O^T / l at the end
// (the reference normalises P before P.V: same values up to rounding).
// The dims of the QK^T product are visited as 16u + 4g + c by (step, lane
// group), so both Q and K fragments are 16-byte reads.
__device__ __forceinline__ floatx4 mfma_f32x4(float a, float b, const floatx4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int HD, int NW>
__global__ __launch_bounds__(NW * 64) void k_attn_flash(AttnArgs a) {
    constexpr int KT = 32;   // keys per LDS stage
    constexpr int QU = HD / 16;
    __shared__ float4 Ks[KT][HD / 4 + 1];   // K[key][dims 4c..4c+3]
    __shared__ float4 Vt[HD][KT / 4 + 1];   // V^T[dim][keys 4c..4c+3]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int b = blockIdx.z, h = blockIdx.y;
    const int qbase = blockIdx.x * 16 * NW;
    const int qi = qbase + wave * 16 + r;  // this lane's query (column of S^T)
    const int pos = a.pos_dev ? *a.pos_dev : a.pos_host;
    const int kvh = a.kv_heads ? h / ((int)gridDim.y / a.kv_heads) : h;
    const int kvd = a.kv_dim ? a.kv_dim : a.dim;
    const size_t cbase = (size_t)b * a.max_seq * kvd + (size_t)kvh * HD;
    const float4* K4 = reinterpret_cast<const float4*>(a.kc + cbase);
    const float4* V4 = reinterpret_cast<const float4*>(a.vc + cbase);
    const int kvd4 = kvd >> 2;
    const int t_all = pos + a.new_seq;
    const int qlast = min(a.new_seq, qbase + 16 * NW) - 1;
    const int kend = a.causal ? pos + qlast + 1 : t_all;

    const bool qok = qi < a.new_seq;
    const float* qrow = a.q + (size_t)(b * a.new_seq + (qok ? qi : 0)) * a.q_stride + h * HD;
    float4 qf[QU];
#pragma unroll
    for (int u = 0; u < QU; u++)
        qf[u] = qok ? *reinterpret_cast<const float4*>(qrow + 16 * u + 4 * g) : make_float4(0.f, 0.f, 0.f, 0.f);
    const int P = pos + qi;  // absolute position of this lane's query

    floatx4 o[QU];
#pragma unroll
    for (int t = 0; t < QU; t++) o[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    for (int k0 = 0; k0 < kend; k0 += KT) {
        __syncthreads();  // the previous stage has been read
        for (int i = threadIdx.x; i < KT * HD / 4; i += NW * 64) {
            const int kr = i / (HD / 4), c4 = i - kr * (HD / 4);
            const int key = k0 + kr;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (key < t_all) {
                kv = K4[(size_t)key * kvd4 + c4];
                vv = V4[(size_t)key * kvd4 + c4];
            }
            Ks[kr][c4] = kv;
            float* vt = reinterpret_cast<float*>(&Vt[0][0]);
            constexpr int VS = 4 * (KT / 4 + 1);  // floats per V^T row
            vt[(4 * c4 + 0) * VS + kr] = vv.x;
            vt[(4 * c4 + 1) * VS + kr] = vv.y;
            vt[(4 * c4 + 2) * VS + kr] = vv.z;
            vt[(4 * c4 + 3) * VS + kr] = vv.w;
        }
        __syncthreads();
#pragma unroll
        for (int sub = 0; sub < KT / 16; sub++) {
            floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < QU; u++) {
                const float4 kf = Ks[sub * 16 + r][4 * u + g];
                s = mfma_f32x4(kf.x, qf[u].x, s);
                s = mfma_f32x4(kf.y, qf[u].y, s);
                s = mfma_f32x4(kf.z, qf[u].z, s);
                s = mfma_f32x4(kf.w, qf[u].w, s);
            }
            float sv[4];
            float tmax = -INFINITY;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int key = k0 + sub * 16 + 4 * g + v;
                const bool ok = qok && key < t_all && (!a.causal || key <= P);
                sv[v] = ok ? s[v] * a.scale : -INFINITY;
                tmax = fmaxf(tmax, sv[v]);
            }
            // the query's maximum over the 4 lane groups holding its keys
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float mnew = fmaxf(m, tmax);
            const float alpha = mnew == -INFINITY ? 1.f : expf(m - mnew);
            float p[4], psum = 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                p[v] = sv[v] == -INFINITY ? 0.f : expf(sv[v] - mnew);
                psum += p[v];
            }
            l = l * alpha + psum;
            m = mnew;
#pragma unroll
            for (int t = 0; t < QU; t++) {
                o[t] *= alpha;
                const float4 vf = Vt[16 * t + r][4 * sub + g];
                o[t] = mfma_f32x4(vf.x, p[0], o[t]);
                o[t] = mfma_f32x4(vf.y, p[1], o[t]);
                o[t] = mfma_f32x4(vf.z, p[2], o[t]);
                o[t] = mfma_f32x4(vf.w, p[3], o[t]);
            }
        }
    }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (qok) {
        const int orow = b * a.new_seq + qi;
        const float inv = 1.0f / l;
#pragma unroll
        for (int t = 0; t < QU; t++)
            attn_out4(a, orow, h * HD + 16 * t + 4 * g,
                      make_float4(o[t][0] * inv, o[t][1] * inv, o[t][2] * inv, o[t][3] * inv));
    }
}

// The q/k epilogue of a one-row projection (nn/gqa.go:300-330: per-head
// RMSNorm, then RoPE at the row's position) for one head held by segments
// of HD4 lanes, lane c of a segment holding elements 4c .. 4c + 3 (every
// segment of the wave holds the same row). k_norm_rope_rows' operations in
// its order: the f64 sum of squares over the head (the wave's 64 / HD4
// copies summed, then divided back out, which is exact), y = x * inv * g,
// then each pair rotated without contraction, the Llama partner element
// taken from lane c +- HD4 / 2 of the same segment.
// The values head_norm_rope reads besides the row: the gain's 4 elements
// and the RoPE cos / sin of this lane's pairs, loaded together through raw
// buffer resources (absent gain or tables read zeros, unused) so that no
// load waits on another — q and k share the tables.
template <int HD4>
struct HeadNormRopeIn {
    float4 gq, gk;
    float co[4], si[4];
};
template <int HD4>
__device__ __forceinline__ HeadNormRopeIn<HD4> head_norm_rope_load(int p, const AttnArgs& a, int c) {
    constexpr int hd = 4 * HD4, half = hd / 2;
    HeadNormRopeIn<HD4> in;
    auto ld4 = [](__amdgpu_buffer_rsrc_t r, int off) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                           __uint_as_float(v[3]));
    };
    in.gq = ld4(make_rsrc(a.q_gain, a.q_gain ? (long long)hd * 4 : 0), 16 * c);
    in.gk = ld4(make_rsrc(a.k_gain, a.k_gain ? (long long)hd * 4 : 0), 16 * c);
    const long long tb = a.rope_cos ? (long long)(p + 1) * half * 4 : 0;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.rope_cos, tb), rs = make_rsrc(a.rope_sin, tb);
    const bool lo = c < HD4 / 2;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        int cs;
        if (a.rope_neox) {
            cs = p * half + min(2 * c + q / 2, half - 1);  // pair q / 2 of the lane
        } else {
            const int k = 4 * c + q;
            const int i = lo ? k : k - half;
            cs = p * half + min(max(i, 0), half - 1);
        }
        in.co[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rc, cs * 4, 0, 0));
        in.si[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, cs * 4, 0, 0));
    }
    return in;
}

template <int HD4>
__device__ __forceinline__ float4 head_norm_rope(float4 v, bool norm, float4 gv, const HeadNormRopeIn<HD4>& in,
                                                 const AttnArgs& a, int c) {
#pragma clang fp contract(off)
    constexpr int hd = 4 * HD4;
    if (norm) {
        double s = ((double)v.x * (double)v.x + (double)v.y * (double)v.y) +
                   ((double)v.z * (double)v.z + (double)v.w * (double)v.w);
        s = wave_sum_d(s) / (double)(64 / HD4);
        const float inv = (float)rsqrt_f64(div_rcp(s, (double)hd, 1.0 / hd) + (double)a.qk_eps);
        v = make_float4(v.x * inv * gv.x, v.y * inv * gv.y, v.z * inv * gv.z, v.w * inv * gv.w);
    }
    if (!a.rope_cos) return v;
    const float e[4] = {v.x, v.y, v.z, v.w};
    float o[4];
    if (a.rope_neox) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const float co = in.co[2 * q], si = in.si[2 * q];
            o[2 * q] = e[2 * q] * co - e[2 * q + 1] * si;
            o[2 * q + 1] = e[2 * q] * si + e[2 * q + 1] * co;
        }
    } else {
        const int lane = threadIdx.x & 63;
        const bool lo = c < HD4 / 2;
        const int src = lo ? lane + HD4 / 2 : lane - HD4 / 2;
        float pe[4];
#pragma unroll
        for (int q = 0; q < 4; q++) pe[q] = __shfl(e[q], src);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float co = in.co[q], si = in.si[q];
            o[q] = lo ? e[q] * co - pe[q] * si : pe[q] * si + e[q] * co;
        }
    }
    return make_float4(o[0], o[1], o[2], o[3]);
}

// k_attn_long: caches longer than one chunk of keys when (head, row) blocks
// are few (a batch-1 step). Lanes over (key, 16-byte chunk of the head) as in
// k_attn_rows; NW waves take KB = NW * KPI keys per instruction and UNR
// instructions per chunk. Every key slot keeps an online softmax over its own
// keys (running max m, weight sum l, weighted value sum o, rescaled by
// exp(m_old - m_new) when the max grows), so the loop has no barrier and the
// next chunk's K and V rows (raw buffer loads over the visible rows,
// branch-free) are in flight while one is used. At the end every slot is
// rescaled to the block's max and the slots are summed through LDS: out =
// sum o / sum l.
// SPLIT (one new row per sequence): blockIdx.z is the row, blockIdx.y a
// chunk of its keys (gridDim.y chunks of a multiple of KC keys each); the
// block writes its chunk's max, weight sum and unnormalised weighted values
// to a.split_ws (record (row, head, chunk)) for k_attn_combine instead of
// the output. Each head's cache then streams through gridDim.y CUs instead
// of one.
// QK (with SPLIT): q and the new row's k finished here (AttnArgs::k_raw):
// head_norm_rope on both, the finished k written to its cache row by one
// block per KV head and used from registers for that key by every block
// whose chunk holds it.
template <int HD4, int NW, int UNR, bool SPLIT = false, bool QK = false>
__global__ __launch_bounds__(NW * 64) void k_attn_long(AttnArgs a) {
    constexpr int KPI = 64 / HD4;  // keys per wavefront instruction
    constexpr int KB = NW * KPI;   // keys per block instruction
    constexpr int KC = KB * UNR;   // keys per chunk
    __shared__ float4 po[NW][64];
    __shared__ float pl[NW][64];
    __shared__ float4 ps[NW][HD4];
    __shared__ float psl[NW];
    __shared__ float red[NW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane % HD4, slot = wave * KPI + lane / HD4;
    const int h = blockIdx.x;
    const int row = SPLIT ? blockIdx.z : blockIdx.y;
    const int b = row / a.new_seq;
    const int i = row - b * a.new_seq;
    const int kvh = a.kv_heads ? h / ((int)gridDim.x / a.kv_heads) : h;
    const int kvd = a.kv_dim ? a.kv_dim : a.dim;
    const size_t base = ((size_t)b * a.max_seq) * kvd + (size_t)kvh * (4 * HD4);
    const int pos = a.pos_dev ? *a.pos_dev : a.pos_host;
    const int T = a.causal ? pos + i + 1 : pos + a.new_seq;
    // keys [jb, je) of this block
    int jb = 0, je = T;
    if constexpr (SPLIT) {
        // with the fused output projection: the residual into the output
        // rows (chunk 0 of each head copies its share; nothing when they
        // are one buffer) before the combine kernel adds to them
        if (a.wo && blockIdx.y == 0 && a.wo_out != a.wo_resid) {
            const int rows_out = a.wo_rows ? a.wo_rows : a.dim;
            const int seg = (rows_out + (int)gridDim.x - 1) / (int)gridDim.x;
            for (int e = threadIdx.x; e < seg; e += blockDim.x) {
                const int n = h * seg + e;
                if (n < rows_out) a.wo_out[(size_t)row * rows_out + n] = a.wo_resid ? a.wo_resid[(size_t)row * rows_out + n] : 0.f;
            }
        }
        const int nc = gridDim.y;
        const int L = ((T + nc - 1) / nc + KC - 1) / KC * KC;
        jb = min(T, (int)blockIdx.y * L);
        je = min(T, jb + L);
    }
    const long long span = T > 0 ? ((long long)(T - 1) * kvd + 4 * HD4) * 4 : 0;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.kc + base, span);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.vc + base, span);
    auto ld4 = [](__amdgpu_buffer_rsrc_t rs, int off) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
        return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                           __uint_as_float(v[3]));
    };
    float4 q = *reinterpret_cast<const float4*>(a.q + (size_t)row * a.q_stride + h * (4 * HD4) + 4 * c);
    float4 knew = make_float4(0.f, 0.f, 0.f, 0.f);
    // keys past T lie outside the resources and read as zeros
    auto load = [&](int j0, float4 (&kk)[UNR], float4 (&vv)[UNR]) {
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int off = (j0 + KB * u + slot) * kvd * 4 + 16 * c;
            kk[u] = ld4(rk, off);
            vv[u] = ld4(rv, off);
        }
    };
    float4 ka[UNR], va[UNR], kb[UNR], vb[UNR];
    if constexpr (QK) {
        const float4 kr = *reinterpret_cast<const float4*>(a.k_raw + (size_t)kvh * (4 * HD4) + 4 * c);
        const HeadNormRopeIn<HD4> in = head_norm_rope_load<HD4>(pos + i, a, c);
        // the first two chunks' keys and values go out behind the epilogue's
        // loads and arrive while it computes (the new key's stale cache row
        // is replaced by knew in step; its value row is already written)
        load(jb, ka, va);
        __builtin_amdgcn_sched_barrier(0);
        load(jb + KC, kb, vb);
        __builtin_amdgcn_sched_barrier(0);
        q = head_norm_rope<HD4>(q, a.q_gain != nullptr, in.gq, in, a, c);
        knew = head_norm_rope<HD4>(kr, a.k_gain != nullptr, in.gk, in, a, c);
        const int group = a.kv_heads ? (int)gridDim.x / a.kv_heads : 1;
        if (h % group == 0 && jb <= T - 1 && T - 1 < je && threadIdx.x < HD4)
            *reinterpret_cast<float4*>(const_cast<float*>(a.kc) + base + (size_t)(T - 1) * kvd + 4 * c) = knew;
    }
    float m = -INFINITY, l = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    auto step = [&](int j0, const float4 (&kk)[UNR], const float4 (&vv)[UNR]) {
        float sj[UNR];
        float cm = -INFINITY;
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            float4 kx = kk[u];
            if constexpr (QK) {
                // the new key from registers (its cache row is being written)
                if (j0 + KB * u + slot == T - 1) kx = knew;
            }
            const float d = q.x * kx.x + q.y * kx.y + q.z * kx.z + q.w * kx.w;
            sj[u] = seg_sum<HD4>(d) * a.scale;
            if (j0 + KB * u + slot < je) cm = fmaxf(cm, sj[u]);
        }
        if (cm > -INFINITY) {
            const float mn = fmaxf(m, cm);
            const float al = expf(m - mn);
            l *= al;
            o = make_float4(o.x * al, o.y * al, o.z * al, o.w * al);
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                if (j0 + KB * u + slot < je) {
                    const float p = expf(sj[u] - mn);
                    l += p;
                    o.x += p * vv[u].x;
                    o.y += p * vv[u].y;
                    o.z += p * vv[u].z;
                    o.w += p * vv[u].w;
                }
            }
            m = mn;
        }
    };
    if constexpr (!QK) {
        load(jb, ka, va);
        __builtin_amdgcn_sched_barrier(0);
        load(jb + KC, kb, vb);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int j0 = jb; j0 < je; j0 += 2 * KC) {
        step(j0, ka, va);
        load(j0 + 2 * KC, ka, va);
        __builtin_amdgcn_sched_barrier(0);
        if (j0 + KC < je) step(j0 + KC, kb, vb);
        load(j0 + 3 * KC, kb, vb);
        __builtin_amdgcn_sched_barrier(0);
    }
    // the block's max, then every slot rescaled to it (empty slots weigh 0)
    const float wm = wave_max(m);
    if (lane == 0) red[wave] = wm;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) M = fmaxf(M, red[w]);
    const float f = m > -INFINITY ? expf(m - M) : 0.f;
    po[wave][lane] = make_float4(o.x * f, o.y * f, o.z * f, o.w * f);
    pl[wave][lane] = l * f;
    __syncthreads();
    // per wave, its KPI slots in order; then the waves in order
    if (threadIdx.x < NW * HD4) {
        const int w = threadIdx.x / HD4, cc = threadIdx.x % HD4;
        float4 t = po[w][cc];
        float tl = pl[w][cc];
#pragma unroll
        for (int sl = 1; sl < KPI; sl++) {
            const float4 pv = po[w][sl * HD4 + cc];
            t.x += pv.x;
            t.y += pv.y;
            t.z += pv.z;
            t.w += pv.w;
            tl += pl[w][sl * HD4 + cc];
        }
        ps[w][cc] = t;
        if (cc == 0) psl[w] = tl;
    }
    __syncthreads();
    if (threadIdx.x < HD4) {
        float4 t = ps[0][c];
        float L = psl[0];
#pragma unroll
        for (int w = 1; w < NW; w++) {
            const float4 pv = ps[w][c];
            t.x += pv.x;
            t.y += pv.y;
            t.z += pv.z;
            t.w += pv.w;
            L += psl[w];
        }
        if constexpr (SPLIT) {
            // record (h, chunk): [max, weight sum, 4 * HD4 weighted values]
            float* rec = a.split_ws + (((size_t)row * gridDim.x + h) * gridDim.y + blockIdx.y) * (4 * HD4 + 2);
            if (c == 0) {
                rec[0] = M;
                rec[1] = L;
            }
            rec[2 + 4 * c] = t.x;
            rec[3 + 4 * c] = t.y;
            rec[4 + 4 * c] = t.z;
            rec[5 + 4 * c] = t.w;
            return;
        }
        if (a.recip) {
            const float rs = 1.0f / L;
            t = make_float4(t.x * rs, t.y * rs, t.z * rs, t.w * rs);
        } else {
            t = make_float4(t.x / L, t.y / L, t.z / L, t.w / L);
        }
        attn_out4(a, row, h * (4 * HD4) + 4 * c, t);
    }
}

// The key-split long-cache attention's second half: per head, the chunks'
// records merged in chunk order, each weighted by exp(its max - the max of
// all), and the weighted values divided by the weighted sum (or multiplied
// by its reciprocal, a.recip). Grid (heads, rows). Thread (ch, c)
// loads chunk ch's max, sum and values c at once (one round trip for the
// whole record set), the weighted terms meet in LDS and threads c < HD4 add
// them in chunk order.
template <int HD4>
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a, int nc) {
    constexpr int CPP = 256 / HD4;  // chunks per pass
    __shared__ float4 st[kAttnSplitMax][HD4];
    __shared__ float sm[kAttnSplitMax], sl[kAttnSplitMax];
    const int h = blockIdx.x, row = blockIdx.y, c = threadIdx.x % HD4, ch0 = threadIdx.x / HD4;
    const float* rec = a.split_ws + ((size_t)row * gridDim.x + h) * nc * (4 * HD4 + 2);
    constexpr int NP = (kAttnSplitMax + CPP - 1) / CPP;
    float mc[NP], lc[NP];
    float4 tc[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int ch = ch0 + p * CPP;
        if (ch < nc) {
            const float* r = rec + (size_t)ch * (4 * HD4 + 2);
            mc[p] = r[0];
            lc[p] = r[1];
            tc[p] = make_float4(r[2 + 4 * c], r[3 + 4 * c], r[4 + 4 * c], r[5 + 4 * c]);
            if (c == 0) sm[ch] = mc[p];
        }
    }
    __syncthreads();
    float M = -INFINITY;
    for (int ch = 0; ch < nc; ch++) M = fmaxf(M, sm[ch]);
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int ch = ch0 + p * CPP;
        if (ch < nc) {
            const float w = mc[p] > -INFINITY ? expf(mc[p] - M) : 0.f;
            st[ch][c] = make_float4(w * tc[p].x, w * tc[p].y, w * tc[p].z, w * tc[p].w);
            if (c == 0) sl[ch] = w * lc[p];
        }
    }
    __syncthreads();
    if (threadIdx.x >= HD4) return;
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
    float L = 0.f;
    for (int ch = 0; ch < nc; ch++) {
        const float4 v = st[ch][c];
        L += sl[ch];
        t.x += v.x;
        t.y += v.y;
        t.z += v.z;
        t.w += v.w;
    }
    if (a.recip) {
        const float rs = 1.0f / L;
        t = make_float4(t.x * rs, t.y * rs, t.z * rs, t.w * rs);
    } else {
        t = make_float4(t.x / L, t.y / L, t.z / L, t.w / L);
    }
    attn_out4(a, row, h * (4 * HD4) + 4 * c, t);
}

// k_attn_combine with the output projection: grid (heads, row groups of
// kCombineWoRows Wo rows), one new row. Each block merges head h's chunk
// records into o_h (k_attn_combine's order, in LDS), then adds
// Wo[n][h*hd .. h*hd+hd) . o_h (+ the bias, from head 0) into a.wo_out[n]
// for its rows with float atomics (the order of the per-head additions
// varies between runs). Its Wo loads go out before the records'.
constexpr int kCombineWoRows = 64;
template <int HD4>
__global__ __launch_bounds__(256) void k_attn_combine_wo(AttnArgs a, int nc) {
    constexpr int CPP = 256 / HD4;
    constexpr int WCH = HD4 / 2;          // 16-byte chunks of a head's Wo row slice
    constexpr int WRP = 256 / WCH;        // Wo rows per pass
    constexpr int WPASS = kCombineWoRows / WRP;
    __shared__ float4 st[kAttnSplitMax][HD4];
    __shared__ float sm[kAttnSplitMax], sl[kAttnSplitMax];
    __shared__ float4 oh[HD4];
    const int h = blockIdx.x, c = threadIdx.x % HD4, ch0 = threadIdx.x / HD4;
    const int rows_out = a.wo_rows ? a.wo_rows : a.dim;
    const int cc = threadIdx.x % WCH, rr = threadIdx.x / WCH;
    const int n0 = blockIdx.y * kCombineWoRows;
    const int nrows = max(0, min(kCombineWoRows, rows_out - n0));
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.wo + (size_t)n0 * a.dim + h * (4 * HD4),
                                                nrows > 0 ? ((long long)(nrows - 1) * a.dim + 4 * HD4) * 2 : 0);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.wo_bias + n0, (h == 0 && a.wo_bias) ? (long long)nrows * 4 : 0);
    u32x4 wov[WPASS];
    float wob[WPASS];  // head 0's bias values, loaded with Wo (no load in the epilogue)
#pragma unroll
    for (int q = 0; q < WPASS; q++) {
        const int rl = rr + q * WRP;
        wov[q] = __builtin_amdgcn_raw_buffer_load_b128(rw, rl < nrows ? (rl * a.dim + 8 * cc) * 2 : kOutOfRange, 0,
                                                     kStreamPolicy);
        wob[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, rl * 4, 0, 0));
    }
    const float* rec = a.split_ws + (size_t)h * nc * (4 * HD4 + 2);
    constexpr int NP = (kAttnSplitMax + CPP - 1) / CPP;
    float mc[NP], lc[NP];
    float4 tc[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int ch = ch0 + p * CPP;
        if (ch < nc) {
            const float* r = rec + (size_t)ch * (4 * HD4 + 2);
            mc[p] = r[0];
            lc[p] = r[1];
            tc[p] = make_float4(r[2 + 4 * c], r[3 + 4 * c], r[4 + 4 * c], r[5 + 4 * c]);
            if (c == 0) sm[ch] = mc[p];
        }
    }
    __syncthreads();
    float M = -INFINITY;
    for (int ch = 0; ch < nc; ch++) M = fmaxf(M, sm[ch]);
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int ch = ch0 + p * CPP;
        if (ch < nc) {
            const float w = mc[p] > -INFINITY ? expf(mc[p] - M) : 0.f;
            st[ch][c] = make_float4(w * tc[p].x, w * tc[p].y, w * tc[p].z, w * tc[p].w);
            if (c == 0) sl[ch] = w * lc[p];
        }
    }
    __syncthreads();
    if (threadIdx.x < HD4) {
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.f;
        for (int ch = 0; ch < nc; ch++) {
            const float4 v = st[ch][c];
            L += sl[ch];
            t.x += v.x;
            t.y += v.y;
            t.z += v.z;
            t.w += v.w;
        }
        if (a.recip) {
            const float rs = 1.0f / L;
            t = make_float4(t.x * rs, t.y * rs, t.z * rs, t.w * rs);
        } else {
            t = make_float4(t.x / L, t.y / L, t.z / L, t.w / L);
        }
        oh[c] = t;
    }
    __syncthreads();
    // this thread's 8 head dims (16-byte Wo chunk cc) of o_h
    const float4 t0 = oh[2 * cc], t1 = oh[2 * cc + 1];
    const float o8[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
#pragma unroll
    for (int q = 0; q < WPASS; q++) {
        float v = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) v += bf16_lo(e & 1 ? wov[q][e >> 1] >> 16 : wov[q][e >> 1] & 0xffffu) * o8[e];
        v = seg_sum<WCH>(v);
        const int rl = rr + q * WRP, n = n0 + rl;
        if (cc == 0 && rl < nrows) {
            if (h == 0 && a.wo_bias) v = v + wob[q];
            __hip_atomic_fetch_add(a.wo_out + n, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// 4 waves per (head, row) block when there are enough blocks to fill the
// GPU; 16 waves when the visible context is long and blocks are few, so each
// block keeps more of the KV stream in flight.
enum AttnRoute { kRouteFlash, kRouteSplit, kRouteRows, kRouteLong, kRouteCached16, kRouteCached4, kRouteNone };

// Key chunks of the key-split long-cache attention for a: up to 256 blocks
// in all, at least one load round of keys per chunk; 0 when a cannot split
// (no scratch, more than one new row, scratch too small, one chunk).
static int attn_split_chunks(const AttnArgs& a, int heads, int rows) {
    // one new row of one sequence (for many sequences the one-block-per-
    // (head, row) kernels were faster: XL batch 16 with 2 / 3 / 6 chunks per
    // (head, row) 4,498 / 4,564 / 4,273 tok/s against 5,149)
    if (!a.split_ws || a.new_seq != 1 || rows != 1 || (a.hd != 64 && a.hd != 128)) return 0;
    const int kc = a.hd == 64 ? 64 : 32;  // keys per 4-wave load round
    const long long keys = a.pos_dev ? (long long)a.max_seq : (long long)a.pos_host + a.new_seq;
    // at most 8 chunks per head (Qwen3-shaped step at context 512: 16 / 12 /
    // 10 / 8 / 6 chunks 1,245 / 1,249 / 1,257 / 1,256 / 1,249 tok/s; GPT-2
    // small batch 1 at a 512-token prompt 3,572 -> 3,591 with 8)
    constexpr int max_chunks = 8;
    const int want = std::min(max_chunks, std::max(1, 256 / heads));
    const int nc = (int)std::min<long long>(std::min(kAttnSplitMax, want), (keys + kc - 1) / kc);
    if (nc < 2 || a.split_ws_floats < (long long)heads * nc * (a.hd + 2)) return 0;
    return nc;
}

// The kernel for a: the matrix-core prefill kernel for many new rows per
// sequence, the (key, chunk)-lane kernel for short caches, the online-softmax
// kernel for few (head, row) blocks over a long cache, else the two-pass
// cached kernel (16 waves when blocks are few and the cache long).
static AttnRoute attn_route(const AttnArgs& a, int heads, int rows) {
    // the score-staging kernels hold one f32 per visible key in LDS: at most
    // the cache capacity when the cache length is read on the device, else
    // the known length
    const long long visible = a.pos_dev ? (long long)a.max_seq : (long long)a.pos_host + a.new_seq;
    const bool lds_ok = (size_t)visible * sizeof(float) <= kAttnMaxLdsBytes;
    const int blocks = heads * rows;
    // new rows per sequence from which the matrix-core prefill kernel runs
    constexpr int flash_min = 32;
    const bool aligned = (a.q_stride % 4 == 0) && (a.dim % 4 == 0) && ((a.kv_dim ? a.kv_dim : a.dim) % 4 == 0) &&
                         ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.kc) |
                           reinterpret_cast<uintptr_t>(a.vc) | reinterpret_cast<uintptr_t>(a.out)) % 16 == 0);
    const auto cached = [&] {
        if (!lds_ok) return kRouteNone;
        return (blocks < 1024 && a.max_seq >= 128) ? kRouteCached16 : kRouteCached4;
    };
    // split QKV partials: only the two-pass kernel adds them
    if (a.qkv_part) return cached();
    if (aligned && a.new_seq >= flash_min && (a.hd == 64 || a.hd == 128)) return kRouteFlash;
    // one row over few heads: each head's keys over several CUs
    if (aligned && blocks < 128 && attn_split_chunks(a, heads, rows)) return kRouteSplit;
    if (aligned && a.max_seq <= 256 && (a.hd == 64 || a.hd == 128 || a.hd == 32 || a.hd == 16))
        return kRouteRows;
    // (measured: XL batch 16, 400 blocks, two-pass 25 vs online-softmax
    // 29.4 us per layer)
    if (aligned && (blocks < 128 || !lds_ok) && (a.hd == 64 || a.hd == 128)) return kRouteLong;
    return cached();
}

bool attn_rows_wo_ok(const AttnArgs& a, int heads, int rows) {
    AttnArgs b = a;
    b.wo = nullptr;
    b.split_ws = nullptr;
    return rows == 1 && a.new_seq == 1 && a.kv_heads == 0 && a.hd == 64 && a.max_seq <= 256 &&
           a.dim % 8 == 0 && heads * a.hd == a.dim && attn_route(b, heads, rows) == kRouteRows;
}

int launch_attn_rows_wo(hipStream_t s, const AttnArgs& a, int heads) {
    if (!attn_rows_wo_ok(a, heads, 1) || !a.wo || !a.wo_out || (reinterpret_cast<uintptr_t>(a.wo) % 16) != 0) {
        set_error("attention: the fused output projection needs one new row, head_dim 64, a cache of <= 256 rows");
        return GORCH_HIP_EUNSUPPORTED;
    }
    const size_t lds = (size_t)a.max_seq * sizeof(float);
    const dim3 grid(heads, (a.dim + kWoRows - 1) / kWoRows);
    if (a.max_seq <= 128) hipLaunchKernelGGL((k_attn_rows<16, 8, true, 4, true>), grid, dim3(256), lds, s, a);
    else hipLaunchKernelGGL((k_attn_rows<16, 16, true, 4, true>), grid, dim3(256), lds, s, a);
    count(CNT_ATTENTION);
    return check_launch("attn_rows_wo");
}

bool attn_split_takes_qk(const AttnArgs& a, int heads, int rows) {
    AttnArgs b = a;
    b.k_raw = nullptr;
    return rows == 1 && attn_route(b, heads, rows) == kRouteSplit;
}

bool attn_takes_qkv_part(const AttnArgs& a, int heads, int rows) {
    if (a.new_seq != 1 || a.kv_heads != 0) return false;
    const AttnRoute r = attn_route(a, heads, rows);
    return r == kRouteCached16 || r == kRouteCached4;
}

int launch_attn_cached(hipStream_t s, const AttnArgs& a, int heads, int rows) {
    const long long visible = a.pos_dev ? (long long)a.max_seq : (long long)a.pos_host + a.new_seq;
    const size_t lds = (size_t)visible * sizeof(float);
    if (a.qkv_part && (a.new_seq != 1 || a.kv_heads != 0 || a.qkv_slices < 1 || a.qkv_slices > kMaxPartSlices)) {
        set_error("attention: split QKV partials need one new row per sequence, no grouped KV heads, 1..8 slices");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if (a.out_frag && (rows > 16 || a.wo)) {
        set_error("attention: a fragment-layout output takes at most 16 rows and no fused output projection");
        return GORCH_HIP_EUNSUPPORTED;
    }
    const dim3 grid(heads, rows);
    const AttnRoute route = attn_route(a, heads, rows);
    if (a.wo && route != kRouteSplit) {
        set_error("attention: the fused output projection here needs the key-split path");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if (a.k_raw && (route != kRouteSplit || rows != 1)) {
        set_error("attention: the fused q/k epilogue needs the key-split path (one new row, few heads)");
        return GORCH_HIP_EUNSUPPORTED;
    }
    switch (route) {
        case kRouteFlash: {
            // many new rows per sequence (prefill): the matrix-core kernel,
            // 128 query rows per block sharing each staged K/V tile
            const int batch = rows / a.new_seq;
            const dim3 fg((a.new_seq + 127) / 128, heads, batch);
            if (a.hd == 64) hipLaunchKernelGGL((k_attn_flash<64, 8>), fg, dim3(512), 0, s, a);
            else hipLaunchKernelGGL((k_attn_flash<128, 8>), fg, dim3(512), 0, s, a);
            count(CNT_ATTENTION);
            return check_launch("attn_flash");
        }
        case kRouteRows: {
            // one chunk of KB * UNR keys (KB = 64 NW / HD4) covers the cache:
            // FULL (head dim 128 past 128 rows: 8 waves, 256 keys)
            const int ms = a.max_seq;
            switch (a.hd) {
                case 128:
                    if (ms <= 128) hipLaunchKernelGGL((k_attn_rows<32, 16, true>), grid, dim3(256), lds, s, a);
                    else hipLaunchKernelGGL((k_attn_rows<32, 16, true, 8>), grid, dim3(512), lds, s, a);
                    break;
                case 64:
                    if (ms <= 128) hipLaunchKernelGGL((k_attn_rows<16, 8, true>), grid, dim3(256), lds, s, a);
                    else hipLaunchKernelGGL((k_attn_rows<16, 16, true>), grid, dim3(256), lds, s, a);
                    break;
                case 32: hipLaunchKernelGGL((k_attn_rows<8, 8, true>), grid, dim3(256), lds, s, a); break;
                default: hipLaunchKernelGGL((k_attn_rows<4, 4, true>), grid, dim3(256), lds, s, a); break;
            }
            count(CNT_ATTENTION);
            return check_launch("attn_rows");
        }
        case kRouteSplit: {
            // one new row per sequence: each (head, row)'s keys split over
            // chunks of 4-wave blocks, the chunks' records merged by
            // k_attn_combine
            const int nc = attn_split_chunks(a, heads, rows);
            const dim3 sg(heads, nc, rows), cg(heads, rows);
            if (a.wo) {
                // the output projection fused into the combine (one row)
                const int rows_out = a.wo_rows ? a.wo_rows : a.dim;
                if (rows != 1 || !a.wo_out || a.dim % 8 != 0 || (reinterpret_cast<uintptr_t>(a.wo) % 16) != 0 ||
                    a.dim != heads * a.hd) {
                    set_error("attention: the fused output projection needs one row and 16-byte Wo rows");
                    return GORCH_HIP_EUNSUPPORTED;
                }
                const dim3 wg(heads, (rows_out + kCombineWoRows - 1) / kCombineWoRows);
                if (a.hd == 64) {
                    if (a.k_raw) hipLaunchKernelGGL((k_attn_long<16, 4, 4, true, true>), sg, dim3(256), 0, s, a);
                    else hipLaunchKernelGGL((k_attn_long<16, 4, 4, true>), sg, dim3(256), 0, s, a);
                    hipLaunchKernelGGL((k_attn_combine_wo<16>), wg, dim3(256), 0, s, a, nc);
                } else {
                    if (a.k_raw) hipLaunchKernelGGL((k_attn_long<32, 4, 4, true, true>), sg, dim3(256), 0, s, a);
                    else hipLaunchKernelGGL((k_attn_long<32, 4, 4, true>), sg, dim3(256), 0, s, a);
                    hipLaunchKernelGGL((k_attn_combine_wo<32>), wg, dim3(256), 0, s, a, nc);
                }
                count(CNT_ATTENTION);
                return check_launch("attn_long_split_wo");
            }
            if (a.hd == 64) {
                if (a.k_raw) hipLaunchKernelGGL((k_attn_long<16, 4, 4, true, true>), sg, dim3(256), 0, s, a);
                else hipLaunchKernelGGL((k_attn_long<16, 4, 4, true>), sg, dim3(256), 0, s, a);
                hipLaunchKernelGGL((k_attn_combine<16>), cg, dim3(256), 0, s, a, nc);
            } else {
                if (a.k_raw) hipLaunchKernelGGL((k_attn_long<32, 4, 4, true, true>), sg, dim3(256), 0, s, a);
                else hipLaunchKernelGGL((k_attn_long<32, 4, 4, true>), sg, dim3(256), 0, s, a);
                hipLaunchKernelGGL((k_attn_combine<32>), cg, dim3(256), 0, s, a, nc);
            }
            count(CNT_ATTENTION);
            return check_launch("attn_long_split");
        }
        case kRouteLong:
            // few (head, row) blocks over a long cache without scratch (or
            // several rows): one 16-wave block per (head, row), two 256-key
            // chunks in flight
            if (a.hd == 64) hipLaunchKernelGGL((k_attn_long<16, 16, 4>), grid, dim3(1024), 0, s, a);
            else hipLaunchKernelGGL((k_attn_long<32, 16, 4>), grid, dim3(1024), 0, s, a);
            count(CNT_ATTENTION);
            return check_launch("attn_long");
        case kRouteCached16:
            hipLaunchKernelGGL(k_attn_cached<16>, grid, dim3(1024), lds, s, a);
            count(CNT_ATTENTION);
            return check_launch("attn_cached");
        case kRouteCached4:
            hipLaunchKernelGGL(k_attn_cached<4>, grid, dim3(256), lds, s, a);
            count(CNT_ATTENTION);
            return check_launch("attn_cached");
        default:
            set_error("attention: a cache longer than 16384 visible rows needs head_dim 64 or 128 and 16-byte aligned rows");
            return GORCH_HIP_EUNSUPPORTED;
    }
}

// softmax_metal.go:111-141
__global__ __launch_bounds__(256) void k_causal_softmax(const float* __restrict__ x, float* __restrict__ y,
                                                        int cols, int q_seq, float scale) {
    __shared__ float red[8];
    const int r = blockIdx.x;
    const int limit = (r % q_seq) + (cols - q_seq);
    const float* row = x + (size_t)r * cols;
    float* orow = y + (size_t)r * cols;
    float lmax = -INFINITY;
    for (int j = threadIdx.x; j <= limit && j < cols; j += blockDim.x) lmax = fmaxf(lmax, row[j] * scale);
    const float mx = block_max(lmax, red);
    float lsum = 0.f;
    for (int j = threadIdx.x; j < cols; j += blockDim.x) {
        if (j <= limit) {
            float e = expf(row[j] * scale - mx);
            orow[j] = e;
            lsum += e;
        } else {
            orow[j] = 0.f;
        }
    }
    const float inv = 1.0f / block_sum(lsum, red);
    for (int j = threadIdx.x; j <= limit && j < cols; j += blockDim.x) orow[j] = orow[j] * inv;
}

// nn/attention.go:274-296, in place
__global__ __launch_bounds__(256) void k_softmax_rows(float* x, int cols) {
    __shared__ float red[8];
    float* row = x + (size_t)blockIdx.x * cols;
    float lmax = -INFINITY;
    for (int j = threadIdx.x; j < cols; j += blockDim.x) lmax = fmaxf(lmax, row[j]);
    const float mx = block_max(lmax, red);
    float lsum = 0.f;
    for (int j = threadIdx.x; j < cols; j += blockDim.x) {
        float e = expf(row[j] - mx);
        row[j] = e;
        lsum += e;
    }
    const float sum = block_sum(lsum, red);
    for (int j = threadIdx.x; j < cols; j += blockDim.x) row[j] = row[j] / sum;
}

}  // namespace gh

using namespace gh;

extern "C" int gorch_hip_attention_cached(void* stream, const float* q, const float* k_cache, const float* v_cache,
                                          float* out, int batch, int new_seq, int pos_offset, int heads,
                                          int head_dim, int max_seq, int causal) {
    GH_REQUIRE(batch > 0 && new_seq > 0 && heads > 0 && head_dim > 0 && max_seq > 0,
               "gorch_hip_attention_cached: bad shape");
    GH_REQUIRE(head_dim % 4 == 0 && head_dim <= 256, "gorch_hip_attention_cached: head_dim must be a multiple of 4, <= 256");
    GH_REQUIRE(pos_offset >= 0 && pos_offset + new_seq <= max_seq,
               "gorch_hip_attention_cached: cached sequence length exceeds max_seq");
    GH_SUPPORTED(kv_span_ok(max_seq, (long long)heads * head_dim),
               "gorch_hip_attention_cached: a sequence's cache span (max_seq x dim x 4 bytes) must be below 2 GiB");
    GH_REQUIRE(q && k_cache && v_cache && out, "gorch_hip_attention_cached: null pointer");
    const int dim = heads * head_dim;
    GH_REQUIRE(((uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0, "gorch_hip_attention_cached: cache must be 16-byte aligned");
    // invScale = float32(1.0 / sqrtFloat32(float32(headDim))) (nn/attention.go:348)
    AttnArgs a{q, k_cache, v_cache, out, nullptr, pos_offset, new_seq, dim, head_dim, max_seq, dim, causal ? 1 : 0,
               1.0f / (float)sqrt((double)head_dim)};
    return finish(stream, launch_attn_cached(stream_of(stream), a, heads, batch * new_seq));
}

extern "C" int gorch_hip_causal_softmax(void* stream, const float* x, float* y, int rows, int cols, int q_seq,
                                        float scale) {
    GH_REQUIRE(rows >= 0 && cols > 0 && q_seq > 0 && q_seq <= cols, "gorch_hip_causal_softmax: bad shape");
    if (rows == 0) return GORCH_HIP_OK;
    GH_REQUIRE(x && y, "gorch_hip_causal_softmax: null pointer");
    hipLaunchKernelGGL(k_causal_softmax, dim3(rows), dim3(256), 0, stream_of(stream), x, y, cols, q_seq, scale);
    count(CNT_ATTENTION);
    return finish(stream, check_launch("causal_softmax"));
}

extern "C" int gorch_hip_softmax_rows(void* stream, float* x, int rows, int cols) {
    GH_REQUIRE(rows >= 0 && cols > 0, "gorch_hip_softmax_rows: bad shape");
    if (rows == 0) return GORCH_HIP_OK;
    GH_REQUIRE(x, "gorch_hip_softmax_rows: null pointer");
    hipLaunchKernelGGL(k_softmax_rows, dim3(rows), dim3(256), 0, stream_of(stream), x, cols);
    count(CNT_ATTENTION);
    return finish(stream, check_launch("softmax_rows"));
}

extern "C" int gorch_hip_gqa_attention_cached(void* stream, const float* q, const float* k_cache, const float* v_cache,
                                              float* out, int batch, int new_seq, int pos_offset, int num_q,
                                              int num_kv, int head_dim, int max_seq, int causal) {
    GH_REQUIRE(batch > 0 && new_seq > 0 && num_q > 0 && num_kv > 0 && head_dim > 0 && max_seq > 0,
               "gorch_hip_gqa_attention_cached: bad shape");
    GH_REQUIRE(num_q % num_kv == 0, "gorch/nn: GQA numQueryHeads must be divisible by numKVHeads");
    GH_REQUIRE(head_dim % 4 == 0 && head_dim <= 256,
               "gorch_hip_gqa_attention_cached: head_dim must be a multiple of 4, <= 256");
    GH_REQUIRE(pos_offset >= 0 && pos_offset + new_seq <= max_seq,
               "gorch_hip_gqa_attention_cached: cached sequence length exceeds max_seq");
    GH_SUPPORTED(kv_span_ok(max_seq, (long long)num_kv * head_dim),
               "gorch_hip_gqa_attention_cached: a sequence's cache span (max_seq x kv_dim x 4 bytes) must be below 2 GiB");
    GH_REQUIRE(q && k_cache && v_cache && out, "gorch_hip_gqa_attention_cached: null pointer");
    GH_REQUIRE(((uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0,
               "gorch_hip_gqa_attention_cached: cache must be 16-byte aligned");
    const int qdim = num_q * head_dim;
    AttnArgs a{q, k_cache, v_cache, out, nullptr, pos_offset, new_seq, qdim, head_dim, max_seq, qdim, causal ? 1 : 0,
               (float)(1.0 / sqrt((double)head_dim)), num_kv, num_kv * head_dim, 1};
    return finish(stream, launch_attn_cached(stream_of(stream), a, num_q, batch * new_seq));
}
