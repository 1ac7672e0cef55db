// matmul.hip — the matmul_dt dispatch (metal_mps_matmul_dt's contract,
// metal/shim.h:99-137) and the fused bf16 Linear entry point.
//
// Routing inside gorch_hip_matmul_dt:
//   - f32 A [M,K] x bf16 B stored [N,K] (transB; the nn.Linear layout,
//     ops.go:788-807 -> bf16_matmul.go:159-173): the MFMA weight-streaming
//     kernel in gemv.hip;
//   - every other transpose/dtype combination, and every batch of more than
//     one entry: k_matmul_mfma, one launch over the batch, each operand
//     gathered through its own layout and dtype into bf16 matrix-core terms
//     (not a hot path of the decode step).
#include <algorithm>

#include "common.h"

namespace gh {

int launch_gemm_bf16w(hipStream_t s, const float* A, const uint16_t* W, const float* bias,
                      const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                      bool act_bf16);

// C[b] = opA(A[b]) @ opB(B[b]) on the matrix cores for every transpose /
// dtype combination of metal_mps_matmul_dt (one launch for the whole batch,
// blockIdx.z = batch entry). Block tile 64 x 64, K stepped by 32; each
// operand tile is gathered through its own layout into LDS as bf16 terms
// in [row][k] order (NTA / NTB terms: 1 for a bf16 operand, 3 for an f32
// one), then 4 waves (2 x 2, 32 x 32 each) run v_mfma_f32_16x16x32_bf16
// over the term products whose term indices sum to at most 2 (the rest lie
// below f32 rounding), accumulating in f32. Not a hot path of the decode
// step: the gather is per element (bf16 storage is one exact term; f32 is
// hi, the value truncated to bf16, mid, the remainder truncated to bf16, and
// lo, what is left rounded to bf16: x = hi + mid + lo to ~2^-25 relative, so
// f32 x f32 products carry f32-level error).
constexpr int kMmBK = 32, kMmLD = kMmBK + 8;  // LDS row: 40 bf16 (80 bytes)

template <int NTA, int NTB>
__global__ __launch_bounds__(256) void k_matmul_mfma(const void* __restrict__ A, const void* __restrict__ B,
                                                     float* __restrict__ C, int M, int N, int K, int transA,
                                                     int transB) {
    __shared__ __align__(16) uint16_t As[NTA][64][kMmLD];
    __shared__ __align__(16) uint16_t Bs[NTB][64][kMmLD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, r = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const size_t bA = (size_t)blockIdx.z * M * K, bB = (size_t)blockIdx.z * K * N;
    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    // one raw buffer resource per operand over this batch entry (< 2 GiB,
    // host check): elements outside the matrix get an out-of-range offset and
    // read as zero, so all 16 of a thread's element loads go out together (a
    // load under a bounds branch waits for the one before it)
    constexpr int EA = NTA == 1 ? 2 : 4, EB = NTB == 1 ? 2 : 4;
    static_assert(NTA == 1 || NTA == 3, "bf16: one term, f32: three");
    static_assert(NTB == 1 || NTB == 3, "bf16: one term, f32: three");
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(reinterpret_cast<const char*>(A) + bA * EA, (long long)M * K * EA);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(reinterpret_cast<const char*>(B) + bB * EB, (long long)K * N * EB);
    auto ld = [](__amdgpu_buffer_rsrc_t rs, int off, bool half) -> uint32_t {
        return half ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0)
                    : __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
    };
    // the operand's terms: bf16 storage is exact; f32 v = hi + mid + lo (hi
    // and mid truncations, each remainder exact in f32, lo rounded)
    auto terms = [](uint32_t bits, bool half, uint16_t (&t)[3]) {
        if (half) {
            t[0] = (uint16_t)bits;
            t[1] = t[2] = 0;
            return;
        }
        const float v = __uint_as_float(bits);
        const uint32_t u = bits & 0xffff0000u;
        const float r1 = v - __uint_as_float(u);
        const uint32_t u1 = __float_as_uint(r1) & 0xffff0000u;
        t[0] = (uint16_t)(u >> 16);
        t[1] = (uint16_t)(u1 >> 16);
        t[2] = __builtin_bit_cast(uint16_t, (__bf16)(r1 - __uint_as_float(u1)));
    };
    for (int k0 = 0; k0 < K; k0 += kMmBK) {
        // 64 x 32 elements per operand, 8 per thread: thread t takes row
        // t / 4 (of the tile) and k 8 * (t % 4) .. +8, each element read
        // through the operand's stored layout
        const int row = tid >> 2, m = m0 + row, n = n0 + row;
        uint32_t av[8], bv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int k = k0 + 8 * (tid & 3) + e;
            const int oa = (m < M && k < K) ? (transA ? k * M + m : m * K + k) * EA : kOutOfRange;
            const int ob = (n < N && k < K) ? (transB ? n * K + k : k * N + n) * EB : kOutOfRange;
            av[e] = ld(ra, oa, NTA == 1);
            bv[e] = ld(rb, ob, NTB == 1);
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int kk = 8 * (tid & 3) + e;
            uint16_t t[3];
            terms(av[e], NTA == 1, t);
#pragma unroll
            for (int q = 0; q < NTA; q++) As[q][row][kk] = t[q];
            terms(bv[e], NTB == 1, t);
#pragma unroll
            for (int q = 0; q < NTB; q++) Bs[q][row][kk] = t[q];
        }
        __syncthreads();
        bf16x8 af[2][NTA], bfr[2][NTB];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int t = 0; t < NTA; t++)
                af[i][t] = *reinterpret_cast<const bf16x8*>(&As[t][wm * 32 + i * 16 + r][8 * g]);
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int t = 0; t < NTB; t++)
                bfr[j][t] = *reinterpret_cast<const bf16x8*>(&Bs[t][wn * 32 + j * 16 + r][8 * g]);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int ta = 0; ta < NTA; ta++)
#pragma unroll
                    for (int tb = 0; tb < NTB; tb++)
                        if (ta + tb <= 2) acc[i][j] = mfma16x16x32(af[i][ta], bfr[j][tb], acc[i][j]);
        __syncthreads();
    }
    // lane holds rows 4g..4g+3 of column r in each 16 x 16 fragment
    float* Cb = C + (size_t)blockIdx.z * M * N;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn * 32 + j * 16 + r;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = m0 + wm * 32 + i * 16 + 4 * g + v;
                if (m < M && n < N) Cb[(size_t)m * N + n] = acc[i][j][v];
            }
        }
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
    if (batch == 1 && !transA && transB && !aBF16 && bBF16 && linear_fast_ok(A, B, (int)K)) {
        for (uint32_t b = 0; b < batch; b++) {
            const float* a = reinterpret_cast<const float*>(A) + (size_t)b * M * K;
            const uint16_t* w = reinterpret_cast<const uint16_t*>(B) + (size_t)b * N * K;
            if ((uintptr_t)a % 16 != 0) break;
            GH_TRY(launch_linear_bf16(s, a, w, nullptr, nullptr, C + (size_t)b * M * N, (int)M, (int)N, (int)K,
                                      GORCH_HIP_EPI_NONE));
            if (b + 1 == batch) return GORCH_HIP_OK;
        }
    }
    // the kernel's 32-bit buffer offsets: each batch entry below 2 GiB
    if ((unsigned long long)M * K * (aBF16 ? 2 : 4) >= (1ull << 31) ||
        (unsigned long long)K * N * (bBF16 ? 2 : 4) >= (1ull << 31)) {
        set_error("gorch_hip_matmul_dt: an operand of one batch entry is 2 GiB or more");
        return GORCH_HIP_EUNSUPPORTED;
    }
    const dim3 grid((N + 63) / 64, (M + 63) / 64, batch);
    const int tA = transA ? 1 : 0, tB = transB ? 1 : 0, m = (int)M, n = (int)N, k = (int)K;
    if (aBF16 && bBF16) hipLaunchKernelGGL((k_matmul_mfma<1, 1>), grid, dim3(256), 0, s, A, B, C, m, n, k, tA, tB);
    else if (aBF16) hipLaunchKernelGGL((k_matmul_mfma<1, 3>), grid, dim3(256), 0, s, A, B, C, m, n, k, tA, tB);
    else if (bBF16) hipLaunchKernelGGL((k_matmul_mfma<3, 1>), grid, dim3(256), 0, s, A, B, C, m, n, k, tA, tB);
    else hipLaunchKernelGGL((k_matmul_mfma<3, 3>), grid, dim3(256), 0, s, A, B, C, m, n, k, tA, tB);
    count(CNT_GENERIC_MATMUL);
    return check_launch("matmul_mfma");
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
