// runtime.hip — device selection, errors, memory, copies and dispatch counters. The Metal counterparts are
// metal/shim.m:120-437 (device, queue, buffers) and ops.go:15-78 (counters).
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"

namespace gh {

static thread_local std::string t_error;

void set_error(const std::string& msg) { t_error = msg; }
void clear_error() { t_error.clear(); }

int check(hipError_t e, const char* what) {
    if (e == hipSuccess) return GORCH_HIP_OK;
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? GORCH_HIP_ENOMEM : GORCH_HIP_ERUNTIME;
}

int check_launch(const char* what) { return check(hipGetLastError(), what); }

hipStream_t stream_of(void* s) { return reinterpret_cast<hipStream_t>(s); }

static std::atomic<uint64_t> g_counts[CNT_COUNT];

void count(Counter c) { g_counts[c].fetch_add(1, std::memory_order_relaxed); }

// Scratch for K-split partial sums, one buffer per (device, stream): work on
// one stream is ordered, so consecutive launches on it can share it. A
// buffer only grows outside stream capture (capture then uses the unsplit
// kernel) and is never freed, since a captured graph may still point at it.
namespace {
struct StreamScratch {
    int dev;
    hipStream_t stream;
    void* ptr;
    size_t bytes;
};
std::mutex g_scratch_mu;
std::vector<StreamScratch> g_scratch;
}  // namespace

void* stream_scratch(hipStream_t s, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    StreamScratch* e = nullptr;
    for (auto& w : g_scratch)
        if (w.dev == dev && w.stream == s) e = &w;
    if (e && e->bytes >= bytes) return e->ptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return nullptr;
    }
    const size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (e) {
        e->ptr = p;
        e->bytes = want;
    } else {
        g_scratch.push_back({dev, s, p, want});
    }
    return p;
}

}  // namespace gh

using namespace gh;

extern "C" {

int gorch_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    int ok = 0;
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) == hipSuccess && std::strncmp(p.gcnArchName, "gfx950", 6) == 0)
            ok++;
    }
    return ok;
}

int gorch_hip_init(int device) {
    int n = 0;
    GH_TRY(check(hipGetDeviceCount(&n), "hipGetDeviceCount"));
    GH_REQUIRE(device >= 0 && device < n, "gorch_hip_init: no such device");
    hipDeviceProp_t p;
    GH_TRY(check(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties"));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) {
        set_error(std::string("gorch_hip_init: device is ") + p.gcnArchName + ", this build targets gfx950");
        return GORCH_HIP_EUNSUPPORTED;
    }
    GH_TRY(check(hipSetDevice(device), "hipSetDevice"));
    return GORCH_HIP_OK;
}

const char* gorch_hip_last_error(void) { return t_error.c_str(); }

void* gorch_hip_alloc(size_t bytes) {
    void* p = nullptr;
    if (check(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc")) return nullptr;
    return p;
}

void gorch_hip_release(void* ptr) {
    if (ptr) (void)hipFree(ptr);
}

int gorch_hip_upload(void* stream, void* dst, const void* src, size_t bytes) {
    GH_REQUIRE(dst && src, "gorch_hip_upload: null pointer");
    hipStream_t s = stream_of(stream);
    GH_TRY(check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s), "upload"));
    return check(hipStreamSynchronize(s), "upload sync");
}

int gorch_hip_download(void* stream, void* dst, const void* src, size_t bytes) {
    GH_REQUIRE(dst && src, "gorch_hip_download: null pointer");
    hipStream_t s = stream_of(stream);
    GH_TRY(check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s), "download"));
    return check(hipStreamSynchronize(s), "download sync");
}

int gorch_hip_sync(void* stream) { return check(hipStreamSynchronize(stream_of(stream)), "sync"); }

int gorch_hip_read_dispatch_counts(uint64_t* out, int n) {
    int m = n < CNT_COUNT ? n : CNT_COUNT;
    for (int i = 0; i < m; i++) out[i] = g_counts[i].load(std::memory_order_relaxed);
    return m;
}

void gorch_hip_reset_dispatch_counts(void) {
    for (int i = 0; i < CNT_COUNT; i++) g_counts[i].store(0, std::memory_order_relaxed);
}

}  // extern "C"
