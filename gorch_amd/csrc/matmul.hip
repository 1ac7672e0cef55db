// matmul.hip — the matmul_dt dispatch (metal_mps_matmul_dt's contract,
// metal/shim.h:99-137) and the fused bf16 Linear entry point.
//
// Routing inside gorch_hip_matmul_dt:
//   - f32 A [M,K] x bf16 B stored [N,K] (transB; the nn.Linear layout,
//     ops.go:788-807 -> bf16_matmul.go:159-173): the MFMA weight-streaming
//     kernel in gemv.hip;
//   - every other transpose/dtype combination: a simple tiled kernel that
//     reads each operand through its own layout and dtype (correct for all
//     shapes; not a hot path of the decode step).
#include <algorithm>

#include "common.h"

namespace gh {

int launch_gemm_bf16w(hipStream_t s, const float* A, const uint16_t* W, const float* bias,
                      const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                      bool act_bf16);

__device__ __forceinline__ float load_op(const void* p, size_t i, int bf16) {
    return bf16 ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16)
                : reinterpret_cast<const float*>(p)[i];
}

// C[b] = opA(A[b]) @ opB(B[b]); 16x16 output tile per block, K staged
// through LDS in 16-wide slabs. Each output sums k in increasing order.
__global__ __launch_bounds__(256) void k_matmul_generic(const void* __restrict__ A,
                                                        const void* __restrict__ B,
                                                        float* __restrict__ C, int M, int N, int K,
                                                        int transA, int transB, int aBF16, int bBF16) {
    __shared__ float As[16][17];
    __shared__ float Bs[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int m = blockIdx.y * 16 + ty, n = blockIdx.x * 16 + tx;
    const size_t bA = (size_t)blockIdx.z * M * K, bB = (size_t)blockIdx.z * K * N;
    float acc = 0.f;
    for (int k0 = 0; k0 < K; k0 += 16) {
        {   // As[ty][tx] = opA(A)[blockIdx.y*16 + ty][k0 + tx]
            int am = blockIdx.y * 16 + ty, ak = k0 + tx;
            float v = 0.f;
            if (am < M && ak < K)
                v = load_op(A, bA + (transA ? (size_t)ak * M + am : (size_t)am * K + ak), aBF16);
            As[ty][tx] = v;
        }
        {   // Bs[ty][tx] = opB(B)[k0 + ty][blockIdx.x*16 + tx]
            int bk = k0 + ty, bn = blockIdx.x * 16 + tx;
            float v = 0.f;
            if (bk < K && bn < N)
                v = load_op(B, bB + (transB ? (size_t)bn * K + bk : (size_t)bk * N + bn), bBF16);
            Bs[ty][tx] = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; kk++) acc += As[ty][kk] * Bs[kk][tx];
        __syncthreads();
    }
    if (m < M && n < N) C[(size_t)blockIdx.z * M * N + (size_t)m * N + n] = acc;
}

static bool linear_fast_ok(const void* x, const void* W, int K) {
    return K % 8 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)W % 16 == 0;
}

}  // namespace gh

using namespace gh;

extern "C" int gorch_hip_linear_bf16_ex(void* stream, const float* x, const uint16_t* W, const float* bias,
                                        const float* residual, float* y, int M, int N, int K, int epilogue,
                                        int flags) {
    GH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gorch_hip_linear_bf16: negative dimension");
    GH_REQUIRE(epilogue == GORCH_HIP_EPI_NONE || epilogue == GORCH_HIP_EPI_GELU,
               "gorch_hip_linear_bf16: unknown epilogue");
    if (M == 0 || N == 0) return GORCH_HIP_OK;
    GH_REQUIRE(x && W && y, "gorch_hip_linear_bf16: null pointer");
    GH_REQUIRE((const void*)x != (const void*)y, "gorch_hip_linear_bf16: x must not alias y");
    if (!linear_fast_ok(x, W, K)) {
        set_error("gorch_hip_linear_bf16: needs K % 8 == 0 and 16-byte aligned x and W");
        return GORCH_HIP_EUNSUPPORTED;
    }
    GH_REQUIRE((flags & ~GORCH_HIP_LINEAR_ACT_BF16) == 0, "gorch_hip_linear_bf16_ex: unknown flag");
    GH_TRY(bf16_gate(stream_of(stream)));
    if (flags & GORCH_HIP_LINEAR_ACT_BF16)
        return finish(stream, launch_gemm_bf16w(stream_of(stream), x, W, bias, residual, OutDesc::plain(y, N), M, N,
                                                K, epilogue, true));
    return finish(stream, launch_linear_bf16(stream_of(stream), x, W, bias, residual, y, M, N, K, epilogue));
}

extern "C" int gorch_hip_linear_bf16(void* stream, const float* x, const uint16_t* W, const float* bias,
                                     const float* residual, float* y, int M, int N, int K, int epilogue) {
    return gorch_hip_linear_bf16_ex(stream, x, W, bias, residual, y, M, N, K, epilogue, 0);
}

extern "C" size_t gorch_hip_packed_bf16_bytes(int N, int K) {
    if (N <= 0 || K <= 0) return 0;
    return packed_bf16_elems(N, K) * sizeof(uint16_t);
}

extern "C" int gorch_hip_pack_bf16(void* stream, const uint16_t* W, uint16_t* Wp, int N, int K) {
    GH_REQUIRE(N >= 0 && K >= 0, "gorch_hip_pack_bf16: negative dimension");
    if (N == 0 || K == 0) return GORCH_HIP_OK;
    GH_REQUIRE(W && Wp, "gorch_hip_pack_bf16: null pointer");
    GH_REQUIRE(K % 8 == 0 && ((uintptr_t)W | (uintptr_t)Wp) % 16 == 0,
               "gorch_hip_pack_bf16: needs K % 8 == 0 and 16-byte aligned buffers");
    return finish(stream, launch_pack_bf16(stream_of(stream), W, Wp, N, K));
}

extern "C" int gorch_hip_linear_bf16_packed(void* stream, const float* x, const uint16_t* Wp, const float* bias,
                                            const float* residual, float* y, int M, int N, int K, int epilogue) {
    GH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gorch_hip_linear_bf16_packed: negative dimension");
    GH_REQUIRE(epilogue == GORCH_HIP_EPI_NONE || epilogue == GORCH_HIP_EPI_GELU,
               "gorch_hip_linear_bf16_packed: unknown epilogue");
    if (M == 0 || N == 0) return GORCH_HIP_OK;
    GH_REQUIRE(M <= 16, "gorch_hip_linear_bf16_packed: M must be <= 16 (decode GEMV)");
    GH_REQUIRE(x && Wp && y, "gorch_hip_linear_bf16_packed: null pointer");
    GH_REQUIRE((const void*)x != (const void*)y, "gorch_hip_linear_bf16_packed: x must not alias y");
    GH_REQUIRE(K % 8 == 0 && ((uintptr_t)x | (uintptr_t)Wp) % 16 == 0,
               "gorch_hip_linear_bf16_packed: needs K % 8 == 0 and 16-byte aligned x and Wp");
    GH_TRY(bf16_gate(stream_of(stream)));
    return finish(stream, launch_linear_packed_od(stream_of(stream), x, Wp, bias, residual, OutDesc::plain(y, N), M,
                                                  N, K, epilogue, LinearExtras{}));
}

// C = 0 for an empty contraction (K == 0), as a kernel rather than a memset
// so that a captured graph holds no memset node
__global__ void k_fill_zero(float* __restrict__ c, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        c[i] = 0.f;
}

namespace gh {

// The matmul_dt routing without the probe gate (the probe itself runs
// through it).
int matmul_dt_raw(hipStream_t s, const void* A, const void* B, float* C, uint32_t M, uint32_t N, uint32_t K,
                  uint32_t batch, int transA, int transB, int aBF16, int bBF16) {
    if (transA && transB) {
        set_error("gorch_hip_matmul_dt: transA && transB is not supported");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if (M == 0 || N == 0 || batch == 0) return GORCH_HIP_OK;
    GH_REQUIRE(A && B && C, "gorch_hip_matmul_dt: null pointer");
    GH_REQUIRE(M < (1u << 30) && N < (1u << 30) && K < (1u << 30) && batch < 65536,
               "gorch_hip_matmul_dt: dimension too large");
    if (K == 0) {
        const size_t n = (size_t)batch * M * N;
        const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
        hipLaunchKernelGGL(k_fill_zero, dim3(blocks), dim3(256), 0, s, C, n);
        count(CNT_ELEMENTWISE);
        return check_launch("fill_zero");
    }
    if (!transA && transB && !aBF16 && bBF16 && linear_fast_ok(A, B, (int)K)) {
        for (uint32_t b = 0; b < batch; b++) {
            const float* a = reinterpret_cast<const float*>(A) + (size_t)b * M * K;
            const uint16_t* w = reinterpret_cast<const uint16_t*>(B) + (size_t)b * N * K;
            if ((uintptr_t)a % 16 != 0) break;
            GH_TRY(launch_linear_bf16(s, a, w, nullptr, nullptr, C + (size_t)b * M * N, (int)M, (int)N, (int)K,
                                      GORCH_HIP_EPI_NONE));
            if (b + 1 == batch) return GORCH_HIP_OK;
        }
    }
    dim3 grid((N + 15) / 16, (M + 15) / 16, batch);
    hipLaunchKernelGGL(k_matmul_generic, grid, dim3(256), 0, s, A, B, C, (int)M, (int)N, (int)K, transA,
                       transB, aBF16, bBF16);
    count(CNT_GENERIC_MATMUL);
    return check_launch("matmul_generic");
}

}  // namespace gh

extern "C" int gorch_hip_matmul_dt(void* stream, const void* A, const void* B, float* C, uint32_t M,
                                   uint32_t N, uint32_t K, int transA, int transB, int aBF16, int bBF16) {
    if (aBF16 || bBF16) GH_TRY(bf16_gate(stream_of(stream)));
    return finish(stream, matmul_dt_raw(stream_of(stream), A, B, C, M, N, K, 1, transA, transB, aBF16, bBF16));
}

extern "C" int gorch_hip_batched_matmul_dt(void* stream, const void* A, const void* B, float* C, uint32_t M,
                                           uint32_t N, uint32_t K, uint32_t batch, int transA, int transB,
                                           int aBF16, int bBF16) {
    if (aBF16 || bBF16) GH_TRY(bf16_gate(stream_of(stream)));
    return finish(stream,
                  matmul_dt_raw(stream_of(stream), A, B, C, M, N, K, batch, transA, transB, aBF16, bBF16));
}
