// noalloc.hip — gorch_hip_linear_bf16 for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). The only scratch gorch_hip_linear_bf16
// needs is the K-split partials of a narrow weight over a long K (2..16
// rows, fewer than 128 16-row tiles, K >= 1024), which it takes from a
// per-stream buffer the library allocates on first use. This variant takes
// them from a fixed device array instead.
//
// The array lives in every device's memory until the process ends, one copy
// per GPU at its own address. Host code never uses the array's name as a
// device address: the address of each device's copy is looked up once with
// hipGetSymbolAddress (with that device current) and kept per device.
//
// Every call on a GPU shares that GPU's array. Calls that overlap on one
// GPU (different streams, or threads without ordering between them) race
// on it; calls ordered on one stream do not. The kernels write every
// partial they later read, so nothing needs clearing between calls.
#include <atomic>
#include <mutex>

#include "common.h"

namespace gh {

// S x M x N f32 partials: the split is taken only for fewer than 128 tiles
// (N <= 2032), at most 8 slices and 16 rows: 8 * 16 * 2032 * 4 bytes.
constexpr size_t kNoAllocScratchBytes = (size_t)1 << 20;

static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kNoAllocMaxDevices = 64;
static std::atomic<float*> g_scratch_ptr[kNoAllocMaxDevices];
static std::mutex g_setup_mu;

int noalloc_setup(int device) {
    if (device < 0 || device >= kNoAllocMaxDevices) {
        set_error("gorch_hip_linear_bf16_noalloc: device index out of range");
        return GORCH_HIP_EINVAL;
    }
    if (g_scratch_ptr[device].load(std::memory_order_acquire)) return GORCH_HIP_OK;
    std::lock_guard<std::mutex> lock(g_setup_mu);
    if (g_scratch_ptr[device].load(std::memory_order_acquire)) return GORCH_HIP_OK;
    int cur = -1;
    GH_TRY(check(hipGetDevice(&cur), "hipGetDevice"));
    if (cur != device) {
        set_error("gorch_hip_linear_bf16_noalloc: set-up must run with its device current");
        return GORCH_HIP_EINVAL;
    }
    float* ptr = nullptr;
    GH_TRY(check(hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(scratch)),
                 "hipGetSymbolAddress(scratch)"));
    if (!ptr) {
        set_error("gorch_hip_linear_bf16_noalloc: no device address for the scratch array");
        return GORCH_HIP_ERUNTIME;
    }
    g_scratch_ptr[device].store(ptr, std::memory_order_release);
    return GORCH_HIP_OK;
}

}  // namespace gh

using namespace gh;

extern "C" int gorch_hip_linear_bf16_noalloc(void* stream, const float* x, const uint16_t* W, const float* bias,
                                             const float* residual, float* y, int M, int N, int K, int epilogue) {
    GH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gorch_hip_linear_bf16_noalloc: negative dimension");
    GH_REQUIRE(epilogue == GORCH_HIP_EPI_NONE || epilogue == GORCH_HIP_EPI_GELU,
               "gorch_hip_linear_bf16_noalloc: unknown epilogue");
    if (M == 0 || N == 0) return GORCH_HIP_OK;
    GH_REQUIRE(x && W && y, "gorch_hip_linear_bf16_noalloc: null pointer");
    GH_REQUIRE((const void*)x != (const void*)y, "gorch_hip_linear_bf16_noalloc: x must not alias y");
    if (K % 8 != 0 || ((uintptr_t)x | (uintptr_t)W) % 16 != 0) {
        set_error("gorch_hip_linear_bf16_noalloc: needs K % 8 == 0 and 16-byte aligned x and W");
        return GORCH_HIP_EUNSUPPORTED;
    }
    int dev = 0;
    GH_TRY(check(hipGetDevice(&dev), "hipGetDevice"));
    GH_TRY(noalloc_setup(dev));
    GH_TRY(bf16_gate(stream_of(stream), false));  // the probe allocates: it ran in gorch_hip_init
    LinearExtras ex;
    ex.scratch = g_scratch_ptr[dev].load(std::memory_order_acquire);
    ex.scratch_bytes = kNoAllocScratchBytes;
    return finish(stream, launch_linear_bf16_od(stream_of(stream), x, W, bias, residual, OutDesc::plain(y, N), M, N,
                                                K, epilogue, ex));
}
