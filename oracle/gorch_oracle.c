/*
 * gorch_oracle.c — CPU restatement of gorch's BF16-weight inference path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline.
 * The product never links or calls this file.
 *
 * Each function cites the reference file:line whose semantics it restates.
 * Where the reference calls Apple Accelerate (cblas_sgemm, vvtanhf, vvexpf),
 * whose rounding and summation order are not published, this file uses the
 * C library (tanhf, expf) and a fixed summation order stated at the call;
 * parity at those points is therefore tolerance-based (see the header of
 * tests/test_oracle_pins.py for the pins).
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp).
 */
#include "gorch_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* A1 codec                                                            */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float u2f(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

/* tensor.go:85-94: NaN keeps its top half with the quiet bit forced;
 * everything else rounds to nearest even on the low 16 bits. */
uint16_t orc_f32_to_bf16(float v) {
    uint32_t bits = f2u(v);
    if (((bits >> 23) & 0xffu) == 0xffu && (bits & 0x7fffffu) != 0)
        return (uint16_t)((bits >> 16) | 0x40u);
    uint32_t rounding = 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + rounding) >> 16);
}

/* tensor.go:97-99: exact widening. */
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void orc_f32_to_bf16_slice(const float* in, uint16_t* out, int64_t n) {
#pragma omp parallel for schedule(static) if (n > (1 << 16))
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}

void orc_bf16_to_f32_slice(const uint16_t* in, float* out, int64_t n) {
#pragma omp parallel for schedule(static) if (n > (1 << 16))
    for (int64_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}

/* ------------------------------------------------------------------ */
/* widening of bf16 operands (bf16_matmul.go:147-152)                  */
/* ------------------------------------------------------------------ */

static int g_widen_per_call = 1;
typedef struct { const void* key; int64_t n; float* f32; } widen_entry;
static widen_entry* g_wcache = NULL;
static int g_wcache_len = 0, g_wcache_cap = 0;

void orc_set_widen_per_call(int on) { g_widen_per_call = on; }

/* OpenMP threads for the parallel loops (the CPU baseline's core count;
 * Accelerate picks its own, accelerate/shim.c:8-32). Returns the count now
 * in effect. */
int orc_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
}

void orc_clear_widen_cache(void) {
    for (int i = 0; i < g_wcache_len; i++) free(g_wcache[i].f32);
    free(g_wcache);
    g_wcache = NULL;
    g_wcache_len = g_wcache_cap = 0;
}

/* Returns an f32 view of `p` (n elements). *owned is set when the caller
 * must free it (per-call widening, the reference's behaviour). */
static const float* widen(const void* p, int64_t n, int isBF16, int* owned) {
    *owned = 0;
    if (!isBF16) return (const float*)p;
    if (!g_widen_per_call) {
        for (int i = 0; i < g_wcache_len; i++)
            if (g_wcache[i].key == p && g_wcache[i].n == n) return g_wcache[i].f32;
    }
    float* f = (float*)malloc((size_t)n * sizeof(float));
    orc_bf16_to_f32_slice((const uint16_t*)p, f, n);
    if (g_widen_per_call) {
        *owned = 1;
        return f;
    }
    if (g_wcache_len == g_wcache_cap) {
        g_wcache_cap = g_wcache_cap ? 2 * g_wcache_cap : 64;
        g_wcache = (widen_entry*)realloc(g_wcache, (size_t)g_wcache_cap * sizeof(widen_entry));
    }
    g_wcache[g_wcache_len].key = p;
    g_wcache[g_wcache_len].n = n;
    g_wcache[g_wcache_len].f32 = f;
    g_wcache_len++;
    return f;
}

/* ------------------------------------------------------------------ */
/* f32 sgemm (stands in for accelerate/shim.c:8-32)                    */
/* ------------------------------------------------------------------ */

/* Dot product of two contiguous f32 rows with eight interleaved partial
 * sums (lane j takes k = j mod 8), combined pairwise at the end. Accelerate's
 * summation order is unpublished; this order is fixed and documented. */
static inline float dot8(const float* a, const float* b, int K) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int k = 0;
    for (; k + 8 <= K; k += 8)
        for (int j = 0; j < 8; j++) acc[j] += a[k + j] * b[k + j];
    for (int j = 0; k < K; k++, j++) acc[j] += a[k] * b[k];
    float s01 = acc[0] + acc[1], s23 = acc[2] + acc[3];
    float s45 = acc[4] + acc[5], s67 = acc[6] + acc[7];
    return (s01 + s23) + (s45 + s67);
}

void orc_sgemm(int transA, int transB, int M, int N, int K,
               const float* A, const float* B, float* C) {
    if (!transA && transB) {
        /* A (M,K), B (N,K): row dot row — the Linear layout. */
#pragma omp parallel for collapse(2) schedule(static) if ((int64_t)M * N * K > (1 << 18))
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++)
                C[(int64_t)m * N + n] = dot8(A + (int64_t)m * K, B + (int64_t)n * K, K);
        return;
    }
    /* Other layouts: C[m,:] accumulates over k in increasing order. */
#pragma omp parallel for schedule(static) if ((int64_t)M * N * K > (1 << 18))
    for (int m = 0; m < M; m++) {
        float* c = C + (int64_t)m * N;
        for (int n = 0; n < N; n++) c[n] = 0.0f;
        for (int k = 0; k < K; k++) {
            float a = transA ? A[(int64_t)k * M + m] : A[(int64_t)m * K + k];
            if (!transB) {
                const float* b = B + (int64_t)k * N;
                for (int n = 0; n < N; n++) c[n] += a * b[n];
            } else {
                for (int n = 0; n < N; n++) c[n] += a * B[(int64_t)n * K + k];
            }
        }
    }
}

/* bf16_matmul.go:159-180 (the widen + Accelerate branch). transA && transB
 * is rejected as in the reference (:176-177). */
int orc_matmul_dt(const void* A, const void* B, float* C, int M, int N, int K,
                  int transA, int transB, int aBF16, int bBF16) {
    if (transA && transB) return -1;
    int oa, ob;
    const float* af = widen(A, (int64_t)M * K, aBF16, &oa);
    const float* bf = widen(B, (int64_t)N * K, bBF16, &ob);
    orc_sgemm(transA, transB, M, N, K, af, bf, C);
    if (oa) free((void*)af);
    if (ob) free((void*)bf);
    return 0;
}

/* bf16_matmul.go:185-212: per-batch contiguous GEMMs. */
int orc_batched_matmul_dt(const void* A, const void* B, float* C, int M, int N, int K,
                          int batch, int transA, int transB, int aBF16, int bBF16) {
    if (transA && transB) return -1;
    int oa, ob;
    const float* af = widen(A, (int64_t)batch * M * K, aBF16, &oa);
    const float* bf = widen(B, (int64_t)batch * N * K, bBF16, &ob);
    for (int i = 0; i < batch; i++)
        orc_sgemm(transA, transB, M, N, K, af + (int64_t)i * M * K, bf + (int64_t)i * K * N,
                  C + (int64_t)i * M * N);
    if (oa) free((void*)af);
    if (ob) free((void*)bf);
    return 0;
}

/* nn/module.go:61-88: out = MatMulTransB(x, W) (f32 out), then each row
 * gets the bias added with vDSP_vadd (an exact f32 add per element). */
void orc_linear(const float* x, int M, int K, const void* W, int wBF16,
                const float* bias, int N, float* y) {
    orc_matmul_dt(x, W, y, M, N, K, 0, 1, 0, wBF16);
    if (bias) {
        for (int m = 0; m < M; m++) {
            float* row = y + (int64_t)m * N;
            for (int n = 0; n < N; n++) row[n] = row[n] + bias[n];
        }
    }
}

/* ------------------------------------------------------------------ */
/* elementwise and row ops                                             */
/* ------------------------------------------------------------------ */

/* ops.go:161-179 via binaryOp (ops.go:1012-1027): exact f32 add. */
void orc_add(const float* a, const float* b, float* c, int64_t n) {
    for (int64_t i = 0; i < n; i++) c[i] = a[i] + b[i];
}

/* ops.go:417-443 (CPU branch): inner = 0.7978845608*(x + 0.044715*x^3)
 * in f32, tanh (vForce there, tanhf here), then 0.5*x*(1+t). */
void orc_gelu(const float* x, float* y, int64_t n) {
#pragma omp parallel for schedule(static) if (n > (1 << 16))
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        float x3 = v * v * v;
        float inner = 0.7978845608f * (v + 0.044715f * x3);
        float t = tanhf(inner);
        y[i] = 0.5f * v * (1.0f + t);
    }
}

/* accelerate/shim.c:164-177: s = 1 / (1 + exp(-x)), each step in f32. */
void orc_sigmoid(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float c = -x[i];
        c = expf(c);
        c = c + 1.0f;
        y[i] = 1.0f / c;
    }
}

/* silu.go:45-57 -> accelerate/shim.c:188-191: x * sigmoid(x). */
void orc_silu(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float s;
        orc_sigmoid(&x[i], &s, 1);
        y[i] = x[i] * s;
    }
}

/* silu.go:94-111 -> accelerate/shim.c:200-206: gate * s * val, left to right. */
void orc_swiglu(const float* gate, const float* val, float* y, int64_t n) {
#pragma omp parallel for schedule(static) if (n > (1 << 16))
    for (int64_t i = 0; i < n; i++) {
        float s;
        orc_sigmoid(&gate[i], &s, 1);
        y[i] = gate[i] * s * val[i];
    }
}

/* nn/layernorm.go:61-91: mean and variance accumulated in float64, inv
 * rounded to f32, then ((x - f32(mean)) * inv) * gamma + beta in f32. */
void orc_layernorm(const float* x, int M, int N, const float* gamma, const float* beta,
                   float eps, float* y) {
    for (int i = 0; i < M; i++) {
        const float* row = x + (int64_t)i * N;
        double mean = 0.0;
        for (int j = 0; j < N; j++) mean += (double)row[j];
        mean /= (double)N;
        double var = 0.0;
        for (int j = 0; j < N; j++) {
            double d = (double)row[j] - mean;
            var += d * d;
        }
        var /= (double)N;
        float inv = (float)(1.0 / sqrt(var + (double)eps));
        float fm = (float)mean;
        for (int j = 0; j < N; j++) {
            float normalized = (row[j] - fm) * inv;
            y[(int64_t)i * N + j] = normalized * gamma[j] + beta[j];
        }
    }
}

/* nn/rmsnorm.go:65-79: sum of squares in float64; inv rounded to f32;
 * y = x * inv * gamma (left to right). */
void orc_rmsnorm(const float* x, int M, int N, const float* gamma, float eps, float* y) {
    for (int i = 0; i < M; i++) {
        const float* row = x + (int64_t)i * N;
        double ss = 0.0;
        for (int j = 0; j < N; j++) ss += (double)row[j] * (double)row[j];
        float inv = (float)(1.0 / sqrt(ss / (double)N + (double)eps));
        for (int j = 0; j < N; j++) y[(int64_t)i * N + j] = row[j] * inv * gamma[j];
    }
}

/* nn/attention.go:274-296: row max in f32, exp in float64 of the f32
 * difference rounded back to f32, f32 running sum, then division. */
void orc_softmax_inplace(float* data, int rows, int cols) {
    for (int i = 0; i < rows; i++) {
        float* row = data + (int64_t)i * cols;
        float maxv = row[0];
        for (int j = 1; j < cols; j++)
            if (row[j] > maxv) maxv = row[j];
        float sum = 0.0f;
        for (int j = 0; j < cols; j++) {
            row[j] = (float)exp((double)(row[j] - maxv));
            sum += row[j];
        }
        for (int j = 0; j < cols; j++) row[j] /= sum;
    }
}

/* softmax_metal.go:111-141: staircase-causal softmax; row r may see
 * columns 0..(r mod qSeq) + (cols - qSeq); masked columns stay exactly 0. */
void orc_causal_softmax(const float* x, float* y, int rows, int cols, int qSeq, float scale) {
    int offset = cols - qSeq;
    for (int r = 0; r < rows; r++) {
        int limit = (r % qSeq) + offset;
        const float* row = x + (int64_t)r * cols;
        float* orow = y + (int64_t)r * cols;
        for (int j = 0; j < cols; j++) orow[j] = 0.0f;
        float rowMax = -INFINITY;
        for (int j = 0; j <= limit; j++) {
            float v = row[j] * scale;
            if (v > rowMax) rowMax = v;
        }
        float sum = 0.0f;
        for (int j = 0; j <= limit; j++) {
            float e = (float)exp((double)(row[j] * scale - rowMax));
            orow[j] = e;
            sum += e;
        }
        float inv = 1.0f / sum;
        for (int j = 0; j <= limit; j++) orow[j] *= inv;
    }
}

/* attention_ops.go:64-77: row copy per id. */
void orc_embedding_lookup(const float* weight, int dim, const int* ids, int n, float* out) {
    for (int i = 0; i < n; i++)
        memcpy(out + (int64_t)i * dim, weight + (int64_t)ids[i] * dim, (size_t)dim * sizeof(float));
}

/* nn/rope.go:71-96: invFreq = f32(base^(-2i/hd)); theta = f64(f32(pos)*invFreq)
 * (the product is an f32 multiply); cos/sin in float64 rounded to f32. */
void orc_rope_tables(int headDim, int maxSeq, float base, float* cosT, float* sinT) {
    int half = headDim / 2;
    for (int pos = 0; pos < maxSeq; pos++) {
        for (int i = 0; i < half; i++) {
            float invFreq = (float)pow((double)base, -(double)(2 * i) / (double)headDim);
            float prod = (float)pos * invFreq;
            double theta = (double)prod;
            cosT[pos * half + i] = (float)cos(theta);
            sinT[pos * half + i] = (float)sin(theta);
        }
    }
}

/* nn/rope.go:172-223: Llama half-split (neox=0) or interleaved (neox=1)
 * pair rotation; sign = +1 forward, -1 inverse. */
void orc_rope_apply(const float* x, float* y, int outer, int seqLen, int headDim,
                    int startPos, const float* cosT, const float* sinT, int neox, float sign) {
    int half = headDim / 2;
    for (int o = 0; o < outer; o++) {
        for (int s = 0; s < seqLen; s++) {
            int64_t rowOff = ((int64_t)o * seqLen + s) * headDim;
            int cs = (startPos + s) * half;
            for (int i = 0; i < half; i++) {
                int ia = neox ? 2 * i : i;
                int ib = neox ? 2 * i + 1 : half + i;
                float a = x[rowOff + ia], b = x[rowOff + ib];
                float c = cosT[cs + i];
                float si = sinT[cs + i] * sign;
                y[rowOff + ia] = a * c - b * si;
                y[rowOff + ib] = a * si + b * c;
            }
        }
    }
}

/* index_ops.go:153-186: descending by value. The reference sorts with
 * sort.Slice (not stable); here ties keep the lower index first. */
void orc_topk(const float* x, int B, int V, int k, float* vals, int* idx) {
    for (int b = 0; b < B; b++) {
        const float* row = x + (int64_t)b * V;
        for (int s = 0; s < k; s++) {
            int best = -1;
            for (int j = 0; j < V; j++) {
                int taken = 0;
                for (int t = 0; t < s; t++)
                    if (idx[b * k + t] == j) { taken = 1; break; }
                if (taken) continue;
                if (best < 0 || row[j] > row[best]) best = j;
            }
            idx[b * k + s] = best;
            vals[b * k + s] = row[best];
        }
    }
}

/* model/generate.go:134-144: first maximum wins (strict >). */
int orc_argmax(const float* logits, int n) {
    int maxIdx = 0;
    float maxVal = logits[0];
    for (int i = 1; i < n; i++)
        if (logits[i] > maxVal) { maxVal = logits[i]; maxIdx = i; }
    return maxIdx;
}

/* model/generate.go:247-262 kthLargest: k passes of a selection sort
 * (strict >, first maximum) over a copy; the k-th pass's value. */
float orc_kth_largest(const float* data, int n, int k) {
    float* s = (float*)malloc((size_t)n * sizeof(float));
    memcpy(s, data, (size_t)n * sizeof(float));
    for (int i = 0; i < k; i++) {
        int maxIdx = i;
        for (int j = i + 1; j < n; j++)
            if (s[j] > s[maxIdx]) maxIdx = j;
        float t = s[i];
        s[i] = s[maxIdx];
        s[maxIdx] = t;
    }
    float r = s[k - 1];
    free(s);
    return r;
}

/* model/generate.go:147-243 sample() with the uniform draw r passed in (the
 * reference draws rand.Float64()): scaled = logits / temperature (f32);
 * with 0 < top_k < n every scaled value below kthLargest(scaled, top_k)
 * becomes -inf (:155-163); softmax in f64 of the f32 differences to the
 * maximum (:165-180); with 0 < top_p < 1 the smallest positive probability
 * (first index among equals) is zeroed until the positive ones sum to at most
 * float64(top_p) * 1.5, then all are divided by their sum (:182-229); the
 * token is the first index whose running f64 sum exceeds r, else n - 1
 * (:231-240). probs (may be NULL) receives the final distribution. */
int orc_sample(const float* logits, int n, float temperature, int top_k, float top_p, double r, double* probs_out) {
    if (n <= 0) return -1;
    float* scaled = (float*)malloc((size_t)n * sizeof(float));
    double* probs = (double*)malloc((size_t)n * sizeof(double));
    for (int i = 0; i < n; i++) scaled[i] = logits[i] / temperature;
    if (top_k > 0 && top_k < n) {
        float threshold = orc_kth_largest(scaled, n, top_k);
        for (int i = 0; i < n; i++)
            if (scaled[i] < threshold) scaled[i] = -INFINITY;
    }
    float maxVal = scaled[0];
    for (int i = 1; i < n; i++)
        if (scaled[i] > maxVal) maxVal = scaled[i];
    double sum = 0.0;
    for (int i = 0; i < n; i++) {
        probs[i] = exp((double)(scaled[i] - maxVal));
        sum += probs[i];
    }
    for (int i = 0; i < n; i++) probs[i] /= sum;
    if (top_p > 0.0f && top_p < 1.0f) {
        const double limit = (double)top_p * 1.5;
        for (;;) {
            double cum = 0.0;
            for (int i = 0; i < n; i++)
                if (probs[i] > 0) cum += probs[i];
            if (cum <= limit) break;
            double minP = 1.7976931348623157e308;
            int minI = -1;
            for (int i = 0; i < n; i++)
                if (probs[i] > 0 && probs[i] < minP) { minP = probs[i]; minI = i; }
            if (minI < 0) break;
            probs[minI] = 0.0;
        }
        double resum = 0.0;
        for (int i = 0; i < n; i++) resum += probs[i];
        for (int i = 0; i < n; i++) probs[i] /= resum;
    }
    int tok = n - 1;
    double cumulative = 0.0;
    for (int i = 0; i < n; i++) {
        cumulative += probs[i];
        if (r < cumulative) { tok = i; break; }
    }
    if (probs_out) memcpy(probs_out, probs, (size_t)n * sizeof(double));
    free(scaled);
    free(probs);
    return tok;
}

/* model/qwen/generate.go:94-163 (sampleLogits) with the draw r given: the
 * same scaling, top-k threshold (kthLargestF32 :165-181 is kthLargest's
 * selection, ties counted) and f64 softmax as sample(), then a standard
 * nucleus cut (:121-152): the probabilities in descending order, the shortest
 * prefix whose running sum reaches f64(top_p) kept and divided by its sum,
 * every other probability set to 0; the inverse CDF in index order (:154-162).
 * sort.Slice (:126) is not a stable sort, so the reference leaves the order
 * of equal probabilities open; this restatement orders them by ascending
 * index (the device sampler's order). */
typedef struct {
    double p;
    int i;
} orc_pi;
static int orc_pi_desc(const void* a, const void* b) {
    const orc_pi* x = (const orc_pi*)a;
    const orc_pi* y = (const orc_pi*)b;
    if (x->p > y->p) return -1;
    if (x->p < y->p) return 1;
    return (x->i > y->i) - (x->i < y->i);
}
int orc_sample_nucleus(const float* logits, int n, float temperature, int top_k, float top_p, double r,
                       double* probs_out) {
    if (n <= 0) return -1;
    float* scaled = (float*)malloc((size_t)n * sizeof(float));
    double* probs = (double*)malloc((size_t)n * sizeof(double));
    for (int i = 0; i < n; i++) scaled[i] = logits[i] / temperature;
    if (top_k > 0 && top_k < n) {
        float threshold = orc_kth_largest(scaled, n, top_k);
        for (int i = 0; i < n; i++)
            if (scaled[i] < threshold) scaled[i] = -INFINITY;
    }
    float maxVal = scaled[0];
    for (int i = 1; i < n; i++)
        if (scaled[i] > maxVal) maxVal = scaled[i];
    double sum = 0.0;
    for (int i = 0; i < n; i++) {
        probs[i] = exp((double)(scaled[i] - maxVal));
        sum += probs[i];
    }
    for (int i = 0; i < n; i++) probs[i] /= sum;
    if (top_p > 0.0f && top_p < 1.0f) {
        orc_pi* idx = (orc_pi*)malloc((size_t)n * sizeof(orc_pi));
        for (int i = 0; i < n; i++) {
            idx[i].p = probs[i];
            idx[i].i = i;
        }
        qsort(idx, (size_t)n, sizeof(orc_pi), orc_pi_desc);
        double cum = 0.0;
        int cut = n;
        for (int q = 0; q < n; q++) {
            cum += idx[q].p;
            if (cum >= (double)top_p) {
                cut = q + 1;
                break;
            }
        }
        double resum = 0.0;
        unsigned char* kept = (unsigned char*)calloc((size_t)n, 1);
        for (int q = 0; q < cut; q++) {
            kept[idx[q].i] = 1;
            resum += idx[q].p;
        }
        for (int i = 0; i < n; i++) probs[i] = kept[i] ? probs[i] / resum : 0.0;
        free(kept);
        free(idx);
    }
    int tok = n - 1;
    double cumulative = 0.0;
    for (int i = 0; i < n; i++) {
        cumulative += probs[i];
        if (r < cumulative) {
            tok = i;
            break;
        }
    }
    if (probs_out) memcpy(probs_out, probs, (size_t)n * sizeof(double));
    free(scaled);
    free(probs);
    return tok;
}

/* The device sampler's uniform draws, restated for the tests (this build's
 * own definition; the reference uses math/rand): Philox4x32-10 (Salmon,
 * Moraes, Dror and Shaw, SC 2011) on counter (row, step, 0, 0) with key
 * (seed low, seed high); u = ((x0 >> 5) * 2^26 + (x1 >> 6)) / 2^53. */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

double orc_philox_uniform(uint64_t seed, uint32_t step, uint32_t row) {
    const uint32_t ctr[4] = {row, step, 0u, 0u}, key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t x[4];
    orc_philox4x32_10(ctr, key, x);
    return ((double)(x[0] >> 5) * 67108864.0 + (double)(x[1] >> 6)) / 9007199254740992.0;
}

/* ------------------------------------------------------------------ */
/* KV cache (nn/kvcache.go:14-60)                                      */
/* ------------------------------------------------------------------ */

struct orc_kvcache {
    int layers, dim, max_seq;
    int* len;       /* per-layer token count (the Go slices' lengths / dim) */
    float** keys;   /* [layer] -> [max_seq, dim] */
    float** values;
};

orc_kvcache* orc_kvcache_new(int layers, int dim, int max_seq) {
    orc_kvcache* c = (orc_kvcache*)calloc(1, sizeof(orc_kvcache));
    c->layers = layers;
    c->dim = dim;
    c->max_seq = max_seq;
    c->len = (int*)calloc((size_t)layers, sizeof(int));
    c->keys = (float**)calloc((size_t)layers, sizeof(float*));
    c->values = (float**)calloc((size_t)layers, sizeof(float*));
    for (int l = 0; l < layers; l++) {
        c->keys[l] = (float*)calloc((size_t)max_seq * dim, sizeof(float));
        c->values[l] = (float*)calloc((size_t)max_seq * dim, sizeof(float));
    }
    return c;
}

void orc_kvcache_free(orc_kvcache* c) {
    if (!c) return;
    for (int l = 0; l < c->layers; l++) {
        free(c->keys[l]);
        free(c->values[l]);
    }
    free(c->keys);
    free(c->values);
    free(c->len);
    free(c);
}

/* nn/kvcache.go:47-52: the length of layer 0. */
int orc_kvcache_len(const orc_kvcache* c) {
    if (c->layers == 0 || c->dim == 0) return 0;
    return c->len[0];
}

void orc_kvcache_reset(orc_kvcache* c) {
    for (int l = 0; l < c->layers; l++) c->len[l] = 0;
}

const float* orc_kvcache_keys(const orc_kvcache* c, int layer) { return c->keys[layer]; }
const float* orc_kvcache_values(const orc_kvcache* c, int layer) { return c->values[layer]; }

/* nn/kvcache.go:40-43 */
static void kv_append(orc_kvcache* c, int layer, const float* k, const float* v, int n) {
    int64_t off = (int64_t)c->len[layer] * c->dim;
    memcpy(c->keys[layer] + off, k, (size_t)n * c->dim * sizeof(float));
    memcpy(c->values[layer] + off, v, (size_t)n * c->dim * sizeof(float));
    c->len[layer] += n;
}

/* ------------------------------------------------------------------ */
/* GPT                                                                 */
/* ------------------------------------------------------------------ */

/* nn/attention.go:348-397 for one sequence: q [newSeq, dim] against keys /
 * values [totalSeq, dim] (totalSeq = posOffset + newSeq); writes the
 * per-head attended sum into out [newSeq, dim] (zero-initialised here as
 * g.Zeros does). The causal mask uses absolute positions (:371-379). */
void orc_attention_cached(const float* q, const float* K, const float* V, float* out, int newSeq,
                          int posOffset, int heads, int headDim, int causal) {
    int dim = heads * headDim;
    int totalSeq = posOffset + newSeq;
    float invScale = (float)(1.0 / (double)(float)sqrt((double)(float)headDim));
    float* scores = (float*)malloc((size_t)newSeq * totalSeq * sizeof(float));
    memset(out, 0, (size_t)newSeq * dim * sizeof(float));
    for (int h = 0; h < heads; h++) {
        int headOff = h * headDim;
        for (int i = 0; i < newSeq; i++) {
            const float* qRow = q + (int64_t)i * dim + headOff;
            for (int j = 0; j < totalSeq; j++) {
                const float* kRow = K + (int64_t)j * dim + headOff;
                float sum = 0.0f;
                for (int d = 0; d < headDim; d++) sum += qRow[d] * kRow[d];
                scores[(int64_t)i * totalSeq + j] = sum * invScale;
            }
        }
        if (causal) {
            for (int i = 0; i < newSeq; i++) {
                int absPos = posOffset + i;
                for (int j = absPos + 1; j < totalSeq; j++) scores[(int64_t)i * totalSeq + j] = -1e9f;
            }
        }
        orc_softmax_inplace(scores, newSeq, totalSeq);
        for (int i = 0; i < newSeq; i++) {
            float* outRow = out + (int64_t)i * dim + headOff;
            const float* sRow = scores + (int64_t)i * totalSeq;
            for (int j = 0; j < totalSeq; j++) {
                if (sRow[j] == 0.0f) continue;
                const float* vRow = V + (int64_t)j * dim + headOff;
                float w = sRow[j];
                for (int d = 0; d < headDim; d++) outRow[d] += w * vRow[d];
            }
        }
    }
    free(scores);
}

/* nn/attention.go:313-400 without the Wo projection: the cache already holds
 * the new rows (appended at :339). */
static void mha_cached_core(const float* q, orc_kvcache* cache, int layer, int posOffset,
                            int newSeq, int dim, int heads, float* out) {
    orc_attention_cached(q, cache->keys[layer], cache->values[layer], out, newSeq, posOffset, heads,
                         dim / heads, 1);
}

/* nn/attention.go:80-119 (batched path of MHA.Forward, before Wo):
 * scores = Q_h K_h^T, scaled, -1e9 above the diagonal, softmaxInPlace,
 * then scores @ V_h. */
static void mha_uncached_core(const float* q, const float* k, const float* v, int seq,
                              int dim, int heads, float* out) {
    int hd = dim / heads;
    float* qh = (float*)malloc((size_t)seq * hd * sizeof(float));
    float* kh = (float*)malloc((size_t)seq * hd * sizeof(float));
    float* vh = (float*)malloc((size_t)seq * hd * sizeof(float));
    float* sc = (float*)malloc((size_t)seq * seq * sizeof(float));
    float* oh = (float*)malloc((size_t)seq * hd * sizeof(float));
    float invScale = (float)(1.0 / sqrt((double)hd));
    for (int h = 0; h < heads; h++) {
        for (int s = 0; s < seq; s++)
            for (int d = 0; d < hd; d++) {
                qh[s * hd + d] = q[(int64_t)s * dim + h * hd + d];
                kh[s * hd + d] = k[(int64_t)s * dim + h * hd + d];
                vh[s * hd + d] = v[(int64_t)s * dim + h * hd + d];
            }
        orc_sgemm(0, 1, seq, seq, hd, qh, kh, sc);
        for (int i = 0; i < seq * seq; i++) sc[i] *= invScale;
        for (int i = 0; i < seq; i++)
            for (int j = i + 1; j < seq; j++) sc[i * seq + j] = -1e9f;
        orc_softmax_inplace(sc, seq, seq);
        orc_sgemm(0, 0, seq, hd, seq, sc, vh, oh);
        for (int s = 0; s < seq; s++)
            for (int d = 0; d < hd; d++) out[(int64_t)s * dim + h * hd + d] = oh[s * hd + d];
    }
    free(qh); free(kh); free(vh); free(sc); free(oh);
}

/* One block: nn/transformer.go:53-63 (cached) or :34-48 (uncached). */
static void block_forward(const orc_gpt_weights* w, int l, float* x, int n,
                          orc_kvcache* cache, int posOffset) {
    int d = w->dim, f = 4 * d, wb = w->linear_bf16;
    float* normed = (float*)malloc((size_t)n * d * sizeof(float));
    float* q = (float*)malloc((size_t)n * d * sizeof(float));
    float* k = (float*)malloc((size_t)n * d * sizeof(float));
    float* v = (float*)malloc((size_t)n * d * sizeof(float));
    float* att = (float*)malloc((size_t)n * d * sizeof(float));
    float* proj = (float*)malloc((size_t)n * d * sizeof(float));
    float* h = (float*)malloc((size_t)n * f * sizeof(float));
    float* g = (float*)malloc((size_t)n * f * sizeof(float));

    orc_layernorm(x, n, d, w->ln1_g[l], w->ln1_b[l], 1e-5f, normed);
    orc_linear(normed, n, d, w->wq[l], wb, w->bq[l], d, q);
    orc_linear(normed, n, d, w->wk[l], wb, w->bk[l], d, k);
    orc_linear(normed, n, d, w->wv[l], wb, w->bv[l], d, v);
    if (cache) {
        kv_append(cache, l, k, v, n);
        mha_cached_core(q, cache, l, posOffset, n, d, w->heads, att);
    } else {
        mha_uncached_core(q, k, v, n, d, w->heads, att);
    }
    orc_linear(att, n, d, w->wo[l], wb, w->bo[l], d, proj);
    orc_add(x, proj, x, (int64_t)n * d);

    orc_layernorm(x, n, d, w->ln2_g[l], w->ln2_b[l], 1e-5f, normed);
    orc_linear(normed, n, d, w->w1[l], wb, w->b1[l], f, h);
    orc_gelu(h, g, (int64_t)n * f);
    orc_linear(g, n, f, w->w2[l], wb, w->b2[l], d, proj);
    orc_add(x, proj, x, (int64_t)n * d);

    free(normed); free(q); free(k); free(v); free(att); free(proj); free(h); free(g);
}

static void gpt_trunk(const orc_gpt_weights* w, const int* ids, int n, int posOffset,
                      orc_kvcache* cache, float* logits) {
    int d = w->dim;
    float* x = (float*)malloc((size_t)n * d * sizeof(float));
    float* pe = (float*)malloc((size_t)n * d * sizeof(float));
    int* pos = (int*)malloc((size_t)n * sizeof(int));
    for (int i = 0; i < n; i++) pos[i] = posOffset + i;
    orc_embedding_lookup(w->wte, d, ids, n, x);
    orc_embedding_lookup(w->wpe, d, pos, n, pe);
    orc_add(x, pe, x, (int64_t)n * d);
    for (int l = 0; l < w->layers; l++) block_forward(w, l, x, n, cache, posOffset);
    orc_layernorm(x, n, d, w->lnf_g, w->lnf_b, 1e-5f, pe);
    orc_linear(pe, n, d, w->wlm, w->linear_bf16, w->blm, w->vocab, logits);
    free(x); free(pe); free(pos);
}

/* nn/gpt.go:100-121 */
int orc_gpt_forward_cached(const orc_gpt_weights* w, orc_kvcache* cache,
                           const int* ids, int n, float* logits) {
    int posOffset = orc_kvcache_len(cache);
    if (posOffset + n > w->max_seq) return -1;
    gpt_trunk(w, ids, n, posOffset, cache, logits);
    return 0;
}

/* nn/gpt.go:55-90 */
int orc_gpt_forward(const orc_gpt_weights* w, const int* ids, int n, float* logits) {
    if (n > w->max_seq) return -1;
    gpt_trunk(w, ids, n, 0, NULL, logits);
    return 0;
}

static float top2_gap(const float* row, int n) {
    float a = -INFINITY, b = -INFINITY;
    for (int i = 0; i < n; i++) {
        if (row[i] > a) { b = a; a = row[i]; }
        else if (row[i] > b) b = row[i];
    }
    return a - b;
}

/* model/generate.go:94-131 with Temperature 0 and no stop token. */
int orc_generate_cached(const orc_gpt_weights* w, const int* prompt, int n_prompt,
                        int max_new, int stop_token, int* out_ids, float* step_logits, float* gaps) {
    int V = w->vocab;
    orc_kvcache* cache = orc_kvcache_new(w->layers, w->dim, w->max_seq);
    const int* p = prompt;
    int np = n_prompt;
    if (np > w->max_seq) { p = prompt + (np - w->max_seq); np = w->max_seq; }
    memcpy(out_ids, p, (size_t)np * sizeof(int));
    int n_out = np;
    float* logits = (float*)malloc((size_t)np * V * sizeof(float));
    orc_gpt_forward_cached(w, cache, p, np, logits);
    float* last = (float*)malloc((size_t)V * sizeof(float));
    memcpy(last, logits + (int64_t)(np - 1) * V, (size_t)V * sizeof(float));
    free(logits);
    for (int i = 0; i < max_new; i++) {
        int next = orc_argmax(last, V);
        if (step_logits) memcpy(step_logits + (int64_t)i * V, last, (size_t)V * sizeof(float));
        if (gaps) gaps[i] = top2_gap(last, V);
        /* StopToken (:116-118): the stop token is not kept */
        if (stop_token >= 0 && next == stop_token) break;
        out_ids[n_out++] = next;
        if (orc_kvcache_len(cache) >= w->max_seq) break;
        orc_gpt_forward_cached(w, cache, &next, 1, last);
    }
    free(last);
    orc_kvcache_free(cache);
    return n_out;
}

/* model/generate.go:94-131 with Temperature > 0: each new token from
 * sample() (:105-110), the draw for new token i of sequence `row` being
 * orc_philox_uniform(seed, i, row). Returns the result length. */
int orc_generate_sampled(const orc_gpt_weights* w, const int* prompt, int n_prompt, int max_new, int stop_token,
                         float temperature, int top_k, float top_p, uint64_t seed, int row, int* out_ids) {
    int V = w->vocab;
    orc_kvcache* cache = orc_kvcache_new(w->layers, w->dim, w->max_seq);
    const int* p = prompt;
    int np = n_prompt;
    if (np > w->max_seq) { p = prompt + (np - w->max_seq); np = w->max_seq; }
    memcpy(out_ids, p, (size_t)np * sizeof(int));
    int n_out = np;
    float* logits = (float*)malloc((size_t)np * V * sizeof(float));
    orc_gpt_forward_cached(w, cache, p, np, logits);
    float* last = (float*)malloc((size_t)V * sizeof(float));
    memcpy(last, logits + (int64_t)(np - 1) * V, (size_t)V * sizeof(float));
    free(logits);
    for (int i = 0; i < max_new; i++) {
        int next = orc_sample(last, V, temperature, top_k, top_p, orc_philox_uniform(seed, (uint32_t)i, (uint32_t)row),
                              NULL);
        if (stop_token >= 0 && next == stop_token) break;
        out_ids[n_out++] = next;
        if (orc_kvcache_len(cache) >= w->max_seq) break;
        orc_gpt_forward_cached(w, cache, &next, 1, last);
    }
    free(last);
    orc_kvcache_free(cache);
    return n_out;
}

/* ------------------------------------------------------------------ */
/* GQA (nn/gqa.go:213-363)                                             */
/* ------------------------------------------------------------------ */

/* softmaxRowsAccelerated (nn/gqa.go:367-385): subtract the row max, exp in
 * f32 (vForce), sum, then scale by 1/sum when the sum is positive. */
static void softmax_rows_recip(float* buf, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        float* row = buf + (int64_t)r * cols;
        float maxv = row[0];
        for (int j = 1; j < cols; j++) if (row[j] > maxv) maxv = row[j];
        for (int j = 0; j < cols; j++) row[j] = row[j] - maxv;
        float sum = 0.0f;
        for (int j = 0; j < cols; j++) { row[j] = expf(row[j]); sum += row[j]; }
        if (sum > 0.0f) {
            float inv = 1.0f / sum;
            for (int j = 0; j < cols; j++) row[j] = row[j] * inv;
        }
    }
}

int orc_gqa_forward_cached(const orc_gqa_weights* w, float* k_cache, float* v_cache, int pos_offset,
                           const float* x, int new_seq, float* out) {
    const int S = new_seq, nq = w->num_q, nkv = w->num_kv, hd = w->head_dim, d = w->dim;
    if (nq % nkv != 0) return -1;
    const int g = nq / nkv, qdim = nq * hd, kvdim = nkv * hd, T = pos_offset + S;
    float* q = (float*)malloc((size_t)S * qdim * sizeof(float));
    float* k = (float*)malloc((size_t)S * kvdim * sizeof(float));
    float* v = (float*)malloc((size_t)S * kvdim * sizeof(float));
    /* ProjectQKV (:213-256): projections, per-head RMSNorm, RoPE on Q, K */
    orc_linear(x, S, d, w->wq, w->linear_bf16, w->bq, qdim, q);
    orc_linear(x, S, d, w->wk, w->linear_bf16, w->bk, kvdim, k);
    orc_linear(x, S, d, w->wv, w->linear_bf16, w->bv, kvdim, v);
    if (w->q_norm) orc_rmsnorm(q, S * nq, hd, w->q_norm, w->norm_eps, q);
    if (w->k_norm) orc_rmsnorm(k, S * nkv, hd, w->k_norm, w->norm_eps, k);
    /* (seq, heads, hd) -> (heads, seq, hd) */
    float* qH = (float*)malloc((size_t)S * qdim * sizeof(float));
    float* kH = (float*)malloc((size_t)S * kvdim * sizeof(float));
    for (int s = 0; s < S; s++) {
        for (int h = 0; h < nq; h++)
            memcpy(qH + ((int64_t)h * S + s) * hd, q + (int64_t)s * qdim + h * hd, (size_t)hd * sizeof(float));
        for (int h = 0; h < nkv; h++)
            memcpy(kH + ((int64_t)h * S + s) * hd, k + (int64_t)s * kvdim + h * hd, (size_t)hd * sizeof(float));
    }
    if (w->rope_cos) {
        orc_rope_apply(qH, qH, nq, S, hd, pos_offset, w->rope_cos, w->rope_sin, w->rope_neox, 1.0f);
        orc_rope_apply(kH, kH, nkv, S, hd, pos_offset, w->rope_cos, w->rope_sin, w->rope_neox, 1.0f);
    }
    /* append rotated K and V rows (token, kvDim) at pos_offset (:292-295) */
    for (int s = 0; s < S; s++) {
        for (int h = 0; h < nkv; h++)
            memcpy(k_cache + ((int64_t)(pos_offset + s)) * kvdim + h * hd, kH + ((int64_t)h * S + s) * hd,
                   (size_t)hd * sizeof(float));
        memcpy(v_cache + ((int64_t)(pos_offset + s)) * kvdim, v + (int64_t)s * kvdim, (size_t)kvdim * sizeof(float));
    }
    /* per KV head: scores = invScale * qBlock kHead^T, mask, softmax, @ vHead (:308-352) */
    float invScale = (float)(1.0 / sqrt((double)hd));
    float* kHead = (float*)malloc((size_t)T * hd * sizeof(float));
    float* vHead = (float*)malloc((size_t)T * hd * sizeof(float));
    float* scores = (float*)malloc((size_t)g * S * T * sizeof(float));
    float* attnOut = (float*)malloc((size_t)S * qdim * sizeof(float));
    for (int kv = 0; kv < nkv; kv++) {
        for (int j = 0; j < T; j++) {
            memcpy(kHead + (int64_t)j * hd, k_cache + (int64_t)j * kvdim + kv * hd, (size_t)hd * sizeof(float));
            memcpy(vHead + (int64_t)j * hd, v_cache + (int64_t)j * kvdim + kv * hd, (size_t)hd * sizeof(float));
        }
        const float* qBlock = qH + (int64_t)kv * g * S * hd;
        orc_sgemm(0, 1, g * S, T, hd, qBlock, kHead, scores);
        for (int64_t i = 0; i < (int64_t)g * S * T; i++) scores[i] = invScale * scores[i];
        if (w->causal && S > 1) {
            for (int r = 0; r < g * S; r++) {
                int absPos = pos_offset + r % S;
                for (int j = absPos + 1; j < T; j++) scores[(int64_t)r * T + j] = -INFINITY;
            }
        }
        softmax_rows_recip(scores, g * S, T);
        orc_sgemm(0, 0, g * S, hd, T, scores, vHead, attnOut + (int64_t)kv * g * S * hd);
    }
    /* (heads, seq, hd) -> (seq, heads*hd), then Wo */
    float* concat = (float*)malloc((size_t)S * qdim * sizeof(float));
    for (int h = 0; h < nq; h++)
        for (int s = 0; s < S; s++)
            memcpy(concat + (int64_t)s * qdim + h * hd, attnOut + ((int64_t)h * S + s) * hd, (size_t)hd * sizeof(float));
    orc_linear(concat, S, qdim, w->wo, w->linear_bf16, w->bo, d, out);
    free(q); free(k); free(v); free(qH); free(kH); free(kHead); free(vHead); free(scores); free(attnOut); free(concat);
    return 0;
}

/* ------------------------------------------------------------------ */
/* MoE (nn/moe.go:130-182, softmaxRows :247-268)                       */
/* ------------------------------------------------------------------ */

int orc_moe_forward(const orc_moe_weights* w, const float* x, int M,
                    const float* logits_in, float* out, int* topk_idx, float* topk_w) {
    int E = w->experts, K = w->top_k, d = w->dim, f = w->ffn;
    if (K <= 0 || K > E) return -1;
    float* logits = (float*)malloc((size_t)M * E * sizeof(float));
    if (logits_in) memcpy(logits, logits_in, (size_t)M * E * sizeof(float));
    else orc_linear(x, M, d, w->wr, w->experts_bf16, w->br, E, logits);
    float* tv = (float*)malloc((size_t)M * K * sizeof(float));
    int* ti = (int*)malloc((size_t)M * K * sizeof(int));
    orc_topk(logits, M, E, K, tv, ti);
    /* softmaxRows: max, exp in float64 rounded to f32, f32 sum, divide. */
    float* wts = (float*)malloc((size_t)M * K * sizeof(float));
    for (int i = 0; i < M; i++) {
        const float* row = tv + (int64_t)i * K;
        float maxv = row[0];
        for (int j = 1; j < K; j++) if (row[j] > maxv) maxv = row[j];
        float sum = 0.0f;
        for (int j = 0; j < K; j++) {
            wts[i * K + j] = (float)exp((double)(row[j] - maxv));
            sum += wts[i * K + j];
        }
        for (int j = 0; j < K; j++) wts[i * K + j] /= sum;
    }
    memset(out, 0, (size_t)M * d * sizeof(float));
    int* tok = (int*)malloc((size_t)M * K * sizeof(int));
    float* rw = (float*)malloc((size_t)M * K * sizeof(float));
    for (int e = 0; e < E; e++) {
        /* group (token, slot) pairs routed to e, in token order (:143-149) */
        int cnt = 0;
        for (int t = 0; t < M; t++)
            for (int s = 0; s < K; s++)
                if (ti[t * K + s] == e) { tok[cnt] = t; rw[cnt] = wts[t * K + s]; cnt++; }
        if (cnt == 0) continue;
        float* in = (float*)malloc((size_t)cnt * d * sizeof(float));
        float* gt = (float*)malloc((size_t)cnt * f * sizeof(float));
        float* up = (float*)malloc((size_t)cnt * f * sizeof(float));
        float* hid = (float*)malloc((size_t)cnt * f * sizeof(float));
        float* eo = (float*)malloc((size_t)cnt * d * sizeof(float));
        for (int i = 0; i < cnt; i++)                                   /* Gather */
            memcpy(in + (int64_t)i * d, x + (int64_t)tok[i] * d, (size_t)d * sizeof(float));
        orc_linear(in, cnt, d, w->wgate[e], w->experts_bf16, w->bgate ? w->bgate[e] : NULL, f, gt);
        orc_linear(in, cnt, d, w->wup[e], w->experts_bf16, w->bup ? w->bup[e] : NULL, f, up);
        orc_swiglu(gt, up, hid, (int64_t)cnt * f);
        orc_linear(hid, cnt, f, w->wdown[e], w->experts_bf16, w->bdown ? w->bdown[e] : NULL, d, eo);
        /* weighted = exOut * w; contribution = ScatterAdd(weighted) into
         * zeros; out = out + contribution (:172-179). A token appears at
         * most once per expert, so the contribution row is 0 + weighted. */
        for (int i = 0; i < cnt; i++) {
            float* orow = out + (int64_t)tok[i] * d;
            const float* erow = eo + (int64_t)i * d;
            for (int j = 0; j < d; j++) {
                float weighted = erow[j] * rw[i];
                float contribution = 0.0f + weighted;
                orow[j] = orow[j] + contribution;
            }
        }
        free(in); free(gt); free(up); free(hid); free(eo);
    }
    if (topk_idx) memcpy(topk_idx, ti, (size_t)M * K * sizeof(int));
    if (topk_w) memcpy(topk_w, wts, (size_t)M * K * sizeof(float));
    free(logits); free(tv); free(ti); free(wts); free(tok); free(rw);
    return 0;
}
