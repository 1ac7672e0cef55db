// argmax.hip — greedy token choice over logits rows (argmax,
// model/generate.go:134-144): the first maximum wins (strict >). A NaN in
// position 0 makes the reference return 0; a NaN elsewhere is never chosen.
// One 1024-thread block per row; each thread scans a strided slice keeping
// its first best, then a (value, index) tree reduction that prefers the
// larger value and, on ties, the smaller index.
#include "common.h"

namespace gh {

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    // v at index i beats (bv, bi)?  NaN values never beat anything.
    if (v != v) return false;
    if (bv != bv) return true;
    return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ logits, int n, int* __restrict__ out,
                                                 int* __restrict__ out2, const int* __restrict__ step_dev,
                                                 int out2_stride, int* pos_dev, int pos_inc) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const float* row = logits + (size_t)blockIdx.x * n;
    float bv = NAN;
    int bi = 0x7fffffff;
    for (int j = threadIdx.x; j < n; j += blockDim.x) {
        float v = row[j];
        if (better(v, j, bv, bi)) {
            bv = v;
            bi = j;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, 64);
        int oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++)
            if (better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        const float first = row[0];
        int r = (first != first || bi == 0x7fffffff) ? 0 : bi;
        out[blockIdx.x] = r;
        if (out2) out2[(size_t)(*step_dev) * out2_stride + blockIdx.x] = r;
    }
    if (pos_dev && blockIdx.x == 0 && threadIdx.x == 0) {
        // advance the shared cache length once the row's token is chosen
        *pos_dev += pos_inc;
    }
}

// Greedy step helper for the decode engine: rows' tokens go to `next_ids`
// (the next forward's input) and to history[step][row]; step and pos
// (device) advance by one / by pos_inc.
__global__ void k_advance_step(int* step_dev) { *step_dev += 1; }

int launch_argmax(hipStream_t s, const float* logits, int rows, int n, int* out, int* hist, const int* step_dev,
                  int hist_stride, int* pos_dev, int pos_inc) {
    hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(1024), 0, s, logits, n, out, hist, step_dev, hist_stride,
                       pos_dev, pos_inc);
    count(CNT_ARGMAX);
    return check_launch("argmax");
}

int launch_advance_step(hipStream_t s, int* step_dev) {
    hipLaunchKernelGGL(k_advance_step, dim3(1), dim3(1), 0, s, step_dev);
    return check_launch("advance_step");
}

}  // namespace gh

using namespace gh;

extern "C" int gorch_hip_argmax(void* stream, const float* logits, int rows, int n, int* out) {
    GH_REQUIRE(rows >= 0 && n > 0, "gorch_hip_argmax: bad shape");
    if (rows == 0) return GORCH_HIP_OK;
    GH_REQUIRE(logits && out, "gorch_hip_argmax: null pointer");
    return finish(stream, launch_argmax(stream_of(stream), logits, rows, n, out, nullptr, nullptr, 0, nullptr, 0));
}
