// codec.hip — gorch's bf16 codec on device (tensor.go:85-121).
// Widening is an exact 16-bit shift; narrowing is round-to-nearest-even
// with gorch's NaN rule. Both stream 8 elements per thread with 16-byte
// accesses where the pointers allow it.
#include "common.h"

namespace gh {

__global__ __launch_bounds__(256) void k_bf16_to_f32(const uint16_t* __restrict__ in,
                                                     float* __restrict__ out, int64_t n,
                                                     int vec_ok) {
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (vec_ok) {
        int64_t nv = n / 8;
        for (int64_t i = tid; i < nv; i += stride) {
            uint4 w = reinterpret_cast<const uint4*>(in)[i];
            float4 a = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
            float4 b = make_float4(bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w));
            reinterpret_cast<float4*>(out)[2 * i] = a;
            reinterpret_cast<float4*>(out)[2 * i + 1] = b;
        }
        for (int64_t i = nv * 8 + tid; i < n; i += stride) out[i] = __uint_as_float((uint32_t)in[i] << 16);
    } else {
        for (int64_t i = tid; i < n; i += stride) out[i] = __uint_as_float((uint32_t)in[i] << 16);
    }
}

__global__ __launch_bounds__(256) void k_f32_to_bf16(const float* __restrict__ in,
                                                     uint16_t* __restrict__ out, int64_t n,
                                                     int vec_ok) {
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (vec_ok) {
        int64_t nv = n / 8;
        for (int64_t i = tid; i < nv; i += stride) {
            float4 a = reinterpret_cast<const float4*>(in)[2 * i];
            float4 b = reinterpret_cast<const float4*>(in)[2 * i + 1];
            uint4 w;
            w.x = (uint32_t)f32_to_bf16_bits(a.x) | ((uint32_t)f32_to_bf16_bits(a.y) << 16);
            w.y = (uint32_t)f32_to_bf16_bits(a.z) | ((uint32_t)f32_to_bf16_bits(a.w) << 16);
            w.z = (uint32_t)f32_to_bf16_bits(b.x) | ((uint32_t)f32_to_bf16_bits(b.y) << 16);
            w.w = (uint32_t)f32_to_bf16_bits(b.z) | ((uint32_t)f32_to_bf16_bits(b.w) << 16);
            reinterpret_cast<uint4*>(out)[i] = w;
        }
        for (int64_t i = nv * 8 + tid; i < n; i += stride) out[i] = f32_to_bf16_bits(in[i]);
    } else {
        for (int64_t i = tid; i < n; i += stride) out[i] = f32_to_bf16_bits(in[i]);
    }
}

static int grid_for(int64_t work) {
    int64_t g = (work + 255) / 256;
    if (g < 1) g = 1;
    if (g > 8192) g = 8192;
    return (int)g;
}

}  // namespace gh

using namespace gh;

extern "C" int gorch_hip_bf16_to_f32(void* stream, const uint16_t* in, float* out, int64_t n) {
    GH_REQUIRE(n >= 0, "gorch_hip_bf16_to_f32: negative length");
    if (n == 0) return GORCH_HIP_OK;
    GH_REQUIRE(in && out, "gorch_hip_bf16_to_f32: null pointer");
    int vec = ((uintptr_t)in % 16 == 0) && ((uintptr_t)out % 16 == 0);
    hipLaunchKernelGGL(k_bf16_to_f32, dim3(grid_for(vec ? n / 8 + 1 : n)), dim3(256), 0,
                       stream_of(stream), in, out, n, vec);
    count(CNT_CODEC);
    return finish(stream, check_launch("bf16_to_f32"));
}

extern "C" int gorch_hip_f32_to_bf16(void* stream, const float* in, uint16_t* out, int64_t n) {
    GH_REQUIRE(n >= 0, "gorch_hip_f32_to_bf16: negative length");
    if (n == 0) return GORCH_HIP_OK;
    GH_REQUIRE(in && out, "gorch_hip_f32_to_bf16: null pointer");
    int vec = ((uintptr_t)in % 16 == 0) && ((uintptr_t)out % 16 == 0);
    hipLaunchKernelGGL(k_f32_to_bf16, dim3(grid_for(vec ? n / 8 + 1 : n)), dim3(256), 0,
                       stream_of(stream), in, out, n, vec);
    count(CNT_CODEC);
    return finish(stream, check_launch("f32_to_bf16"));
}
