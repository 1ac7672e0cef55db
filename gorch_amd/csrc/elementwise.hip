// elementwise.hip — the decode step's pointwise ops, each one HBM pass:
// residual Add (ops.go:161-179; MSL vec_add), bias add (colreduce_metal.go:56-73;
// vec_bias_add), GELU (ops.go:417-443; vec_gelu), SiLU / SwiGLU (silu.go:45-136;
// vec_silu / vec_swiglu) and the embedding row gather (attention_ops.go:64-77),
// plus the fused token + position embedding sum GPT.ForwardCached starts with
// (nn/gpt.go:107-115).
#include "common.h"

namespace gh {

static int grid_1d(int64_t n, int per_thread = 1) {
    int64_t g = (n / per_thread + 255) / 256;
    if (g < 1) g = 1;
    if (g > 16384) g = 16384;
    return (int)g;
}

#define GRID_STRIDE(i, n) \
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (int64_t)gridDim.x * blockDim.x)

__global__ void k_add(const float* __restrict__ a, const float* __restrict__ b, float* c, int64_t n) {
    GRID_STRIDE(i, n) c[i] = a[i] + b[i];
}

__global__ void k_bias_add(float* x, const float* __restrict__ bias, int64_t n, int N) {
    GRID_STRIDE(i, n) x[i] = x[i] + bias[i % N];
}

__global__ void k_gelu(const float* __restrict__ x, float* y, int64_t n) {
    GRID_STRIDE(i, n) y[i] = gelu_tanh(x[i]);
}

__global__ void k_silu(const float* __restrict__ x, float* y, int64_t n) {
    GRID_STRIDE(i, n) {
        float v = x[i];
        y[i] = v * sigmoidf_ref(v);
    }
}

__global__ void k_swiglu(const float* __restrict__ g, const float* __restrict__ v, float* y, int64_t n) {
    GRID_STRIDE(i, n) {
        float gv = g[i];
        y[i] = gv * sigmoidf_ref(gv) * v[i];
    }
}

// out[r, :] = weight[ids[r], :]
__global__ void k_embedding(const float* __restrict__ w, const int* __restrict__ ids, float* out, int dim,
                            int64_t n) {
    GRID_STRIDE(i, n) {
        int64_t r = i / dim;
        int c = (int)(i - r * dim);
        out[i] = w[(size_t)ids[r] * dim + c];
    }
}

// out[b*n + i, :] = wte[ids[b*n + i], :] + wpe[pos + i, :], pos read from
// device memory (the KV-cache length before this forward).
__global__ void k_embed_pos(const float* __restrict__ wte, const float* __restrict__ wpe,
                            const int* __restrict__ ids, const int* __restrict__ pos_dev, float* out,
                            int dim, int n_per_seq, int64_t total) {
    const int pos = *pos_dev;
    GRID_STRIDE(i, total) {
        int64_t r = i / dim;
        int c = (int)(i - r * dim);
        int p = pos + (int)(r % n_per_seq);
        out[i] = wte[(size_t)ids[r] * dim + c] + wpe[(size_t)p * dim + c];
    }
}

int launch_embed_pos(hipStream_t s, const float* wte, const float* wpe, const int* ids, const int* pos_dev,
                     float* out, int dim, int n_per_seq, int rows) {
    int64_t total = (int64_t)rows * dim;
    hipLaunchKernelGGL(k_embed_pos, dim3(grid_1d(total)), dim3(256), 0, s, wte, wpe, ids, pos_dev, out, dim,
                       n_per_seq, total);
    count(CNT_ELEMENTWISE);
    return check_launch("embed_pos");
}

int launch_embedding(hipStream_t s, const float* w, const int* ids, float* out, int dim, int rows) {
    const int64_t total = (int64_t)rows * dim;
    hipLaunchKernelGGL(k_embedding, dim3(grid_1d(total)), dim3(256), 0, s, w, ids, out, dim, total);
    count(CNT_ELEMENTWISE);
    return check_launch("embedding");
}

int launch_swiglu(hipStream_t s, const float* g, const float* v, float* y, int64_t n) {
    if (n == 0) return GORCH_HIP_OK;
    hipLaunchKernelGGL(k_swiglu, dim3(grid_1d(n)), dim3(256), 0, s, g, v, y, n);
    count(CNT_ELEMENTWISE);
    return check_launch("swiglu");
}

}  // namespace gh

using namespace gh;

#define EW_CHECK(n, ...)                                                   \
    GH_REQUIRE((n) >= 0, "negative length");                               \
    if ((n) == 0) return GORCH_HIP_OK;                                     \
    GH_REQUIRE(__VA_ARGS__, "null pointer")

extern "C" int gorch_hip_add(void* stream, const float* a, const float* b, float* c, int64_t n) {
    EW_CHECK(n, a && b && c);
    hipLaunchKernelGGL(k_add, dim3(grid_1d(n)), dim3(256), 0, stream_of(stream), a, b, c, n);
    count(CNT_ELEMENTWISE);
    return finish(stream, check_launch("add"));
}

extern "C" int gorch_hip_bias_add(void* stream, float* x, const float* bias, int M, int N) {
    GH_REQUIRE(M >= 0 && N > 0, "gorch_hip_bias_add: bad shape");
    int64_t n = (int64_t)M * N;
    EW_CHECK(n, x && bias);
    hipLaunchKernelGGL(k_bias_add, dim3(grid_1d(n)), dim3(256), 0, stream_of(stream), x, bias, n, N);
    count(CNT_ELEMENTWISE);
    return finish(stream, check_launch("bias_add"));
}

extern "C" int gorch_hip_gelu(void* stream, const float* x, float* y, int64_t n) {
    EW_CHECK(n, x && y);
    hipLaunchKernelGGL(k_gelu, dim3(grid_1d(n)), dim3(256), 0, stream_of(stream), x, y, n);
    count(CNT_ELEMENTWISE);
    return finish(stream, check_launch("gelu"));
}

extern "C" int gorch_hip_silu(void* stream, const float* x, float* y, int64_t n) {
    EW_CHECK(n, x && y);
    hipLaunchKernelGGL(k_silu, dim3(grid_1d(n)), dim3(256), 0, stream_of(stream), x, y, n);
    count(CNT_ELEMENTWISE);
    return finish(stream, check_launch("silu"));
}

extern "C" int gorch_hip_swiglu(void* stream, const float* gate, const float* value, float* y, int64_t n) {
    EW_CHECK(n, gate && value && y);
    return finish(stream, launch_swiglu(stream_of(stream), gate, value, y, n));
}

extern "C" int gorch_hip_embedding(void* stream, const float* weight, int dim, const int* ids, int n,
                                   float* out) {
    GH_REQUIRE(dim > 0 && n >= 0, "gorch_hip_embedding: bad shape");
    int64_t total = (int64_t)n * dim;
    EW_CHECK(total, weight && ids && out);
    hipLaunchKernelGGL(k_embedding, dim3(grid_1d(total)), dim3(256), 0, stream_of(stream), weight, ids, out, dim,
                       total);
    count(CNT_ELEMENTWISE);
    return finish(stream, check_launch("embedding"));
}
