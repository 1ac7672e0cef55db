// runtime.hip — device selection, errors, memory, copies and dispatch counters. The Metal counterparts are
// metal/shim.m:120-437 (device, queue, buffers) and ops.go:15-78 (counters).
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
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
    // buffers this one replaced when it grew (a captured graph may still
    // point at them): freed with it
    std::vector<std::pair<void*, size_t>> retired;
};
std::mutex g_scratch_mu;
std::vector<StreamScratch> g_scratch;
std::atomic<long long> g_scratch_bytes{0};
}  // namespace

long long scratch_bytes_held() { return g_scratch_bytes.load(); }

void release_stream_scratch(hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    for (size_t i = 0; i < g_scratch.size();) {
        if (g_scratch[i].stream == s) {
            (void)hipFree(g_scratch[i].ptr);
            g_scratch_bytes -= (long long)g_scratch[i].bytes;
            for (auto& r : g_scratch[i].retired) {
                (void)hipFree(r.first);
                g_scratch_bytes -= (long long)r.second;
            }
            g_scratch.erase(g_scratch.begin() + (long)i);
        } else {
            i++;
        }
    }
}

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
    g_scratch_bytes += (long long)want;
    if (e) {
        // the smaller buffer stays allocated: a captured graph may point at it
        e->retired.emplace_back(e->ptr, e->bytes);
        e->ptr = p;
        e->bytes = want;
    } else {
        g_scratch.push_back({dev, s, p, want, {}});
    }
    return p;
}

// Dispatch mode (SetMetalAsync, metal_async.go:30-38): on (the default),
// entry points return once their work is queued; off, every compute entry
// point waits for its stream before returning (the Metal shim's per-op
// waitUntilCompleted, metal/shim.m:216-227).
static std::atomic<int> g_async{1};
// gorch_hip_set_deterministic: fixed-order sums only (no float atomics)
static std::atomic<int> g_deterministic{0};

bool deterministic() { return g_deterministic.load(std::memory_order_relaxed) != 0; }

int finish(void* stream, int rc) {
    if (rc != GORCH_HIP_OK || g_async.load(std::memory_order_relaxed)) return rc;
    hipStream_t s = stream_of(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
        (void)hipGetLastError();
        cs = hipStreamCaptureStatusNone;
    }
    if (cs != hipStreamCaptureStatusNone) return rc;  // a captured launch has nothing to wait for yet
    return check(hipStreamSynchronize(s), "sync-mode wait");
}

// ---------------------------------------------------------------- bf16 probe
// runBF16MatMulProbe (bf16_matmul.go:63-112): once per device, a 16x16x16
// bf16 x bf16 and bf16 x f32 product through the matmul path is compared
// with a host f32 product of the same (widened) values; every element must
// agree within 1e-3. A device whose probe fails gets GORCH_HIP_EUNSUPPORTED
// from every bf16 matmul entry point, so the caller takes its CPU path
// (bf16MatMulEligible, :116-119).
constexpr int kMaxDevices = 64;
static std::atomic<int> g_probe[kMaxDevices];  // 0 not run, 1 passed, 2 failed
static std::mutex g_probe_mu;

int matmul_dt_raw(hipStream_t s, const void* A, const void* B, float* C, uint32_t M, uint32_t N, uint32_t K,
                  uint32_t batch, int transA, int transB, int aBF16, int bBF16);

static int run_bf16_probe(int dev) {
    constexpr int n = 16;
    float af[n * n], bf[n * n], aw[n * n], bw[n * n], ref[n * n], got[n * n];
    uint16_t ah[n * n], bh[n * n];
    for (int i = 0; i < n * n; i++) {
        af[i] = (float)(i % 7) * 0.25f - 0.75f;
        bf[i] = (float)((i * 5) % 11) * 0.125f - 0.625f;
        ah[i] = f32_to_bf16_bits(af[i]);
        bh[i] = f32_to_bf16_bits(bf[i]);
        uint32_t ua = (uint32_t)ah[i] << 16, ub = (uint32_t)bh[i] << 16;
        std::memcpy(&aw[i], &ua, 4);
        std::memcpy(&bw[i], &ub, 4);
    }
    // the comparison tolerance; GORCH_HIP_BF16_PROBE_TOL replaces it so a
    // test can make the host-side check reject a correct device result
    float tol = 1e-3f;
    if (const char* e = getenv("GORCH_HIP_BF16_PROBE_TOL")) tol = (float)atof(e);
    char* buf = nullptr;
    hipStream_t s = nullptr;
    int verdict = 2;
    do {
        if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) break;
        if (hipMalloc(&buf, 4096) != hipSuccess) break;
        uint16_t* dA = reinterpret_cast<uint16_t*>(buf);
        uint16_t* dB = dA + n * n;
        float* dBf = reinterpret_cast<float*>(buf + 1024);
        float* dC = reinterpret_cast<float*>(buf + 2048);
        float* dAf = reinterpret_cast<float*>(buf + 3072);
        if (hipMemcpyAsync(dA, ah, sizeof ah, hipMemcpyHostToDevice, s) != hipSuccess ||
            hipMemcpyAsync(dB, bh, sizeof bh, hipMemcpyHostToDevice, s) != hipSuccess ||
            hipMemcpyAsync(dBf, bf, sizeof bf, hipMemcpyHostToDevice, s) != hipSuccess ||
            hipMemcpyAsync(dAf, aw, sizeof aw, hipMemcpyHostToDevice, s) != hipSuccess)
            break;
        bool ok = true;
        // bf16 x bf16 and bf16 x f32 as the reference probes them, then the
        // Linear layout this backend streams (f32 x bf16 stored [N, K])
        for (int pass = 0; pass < 3 && ok; pass++) {
            const float* rb = pass == 1 ? bf : bw;
            for (int i = 0; i < n; i++)
                for (int j = 0; j < n; j++) {
                    float acc = 0.f;
                    for (int k = 0; k < n; k++) acc += aw[i * n + k] * (pass == 2 ? rb[j * n + k] : rb[k * n + j]);
                    ref[i * n + j] = acc;
                }
            const void* A = pass == 2 ? (const void*)dAf : (const void*)dA;
            const void* B = pass == 1 ? (const void*)dBf : (const void*)dB;
            if (matmul_dt_raw(s, A, B, dC, n, n, n, 1, 0, pass == 2, pass != 2, pass != 1) != GORCH_HIP_OK ||
                hipMemcpyAsync(got, dC, sizeof got, hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess) {
                ok = false;
                break;
            }
            for (int i = 0; i < n * n; i++) {
                const float d = ref[i] - got[i];
                if (!(d <= tol && d >= -tol)) ok = false;
            }
        }
        if (ok) verdict = 1;
    } while (false);
    (void)hipGetLastError();
    if (buf) (void)hipFree(buf);
    if (s) {
        release_stream_scratch(s);
        (void)hipStreamDestroy(s);
    }
    g_probe[dev].store(verdict, std::memory_order_release);
    return verdict;
}

int bf16_gate(hipStream_t s, bool may_probe) {
    int dev = 0;
    GH_TRY(check(hipGetDevice(&dev), "hipGetDevice"));
    if (dev < 0 || dev >= kMaxDevices) return GORCH_HIP_OK;
    int v = g_probe[dev].load(std::memory_order_acquire);
    if (v == 0 && !may_probe) {
        set_error("bf16 matmul probe has not run on this device: call gorch_hip_init first");
        return GORCH_HIP_EUNSUPPORTED;
    }
    if (v == 0) {
        // not probed yet (gorch_hip_init runs the probe): probe now unless
        // the caller's stream is being captured into a graph
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &cs) != hipSuccess) (void)hipGetLastError();
        if (cs != hipStreamCaptureStatusNone) {
            set_error("bf16 matmul probe has not run on this device: call gorch_hip_init before capture");
            return GORCH_HIP_EUNSUPPORTED;
        }
        std::lock_guard<std::mutex> lock(g_probe_mu);
        v = g_probe[dev].load(std::memory_order_acquire);
        if (v == 0) v = run_bf16_probe(dev);
    }
    if (v != 1) {
        set_error("bf16 matmul probe failed on this device: use the CPU path");
        return GORCH_HIP_EUNSUPPORTED;
    }
    return GORCH_HIP_OK;
}

// ---------------------------------------------------------------- memory
// Raw allocations are registered so that a release of a pointer this
// library did not hand out, or one already released, does nothing.
static std::mutex g_mem_mu;
static std::unordered_map<void*, size_t> g_raw;

// A buffer handle (metal.Buffer, metal/metal.go:363-422): device memory of
// exactly the requested length, zero-filled, with an optional pinned host
// mirror. Handles are ids that are never reused, so a second release of a
// handle (an explicit call racing a finaliser) is a no-op.
struct Buf {
    void* dev = nullptr;
    void* host = nullptr;
    size_t bytes = 0;
    int device = 0;
    std::mutex mu;
    bool host_valid = true;  // the mirror holds the current contents
    bool dev_valid = true;   // the device copy holds the current contents
    ~Buf() {
        if (dev) (void)hipFree(dev);
        if (host) (void)hipHostFree(host);
    }
};
static std::unordered_map<uintptr_t, std::shared_ptr<Buf>> g_bufs;
static uintptr_t g_next_buf = 1;
static std::atomic<long long> g_live_bytes{0};

static std::shared_ptr<Buf> find_buf(gorch_hip_buf* h) {
    std::lock_guard<std::mutex> lock(g_mem_mu);
    auto it = g_bufs.find(reinterpret_cast<uintptr_t>(h));
    return it == g_bufs.end() ? nullptr : it->second;
}

}  // namespace gh

using namespace gh;

extern "C" {

int gorch_hip_set_async(int on) {
    const int prev = g_async.exchange(on ? 1 : 0);
    // turning async off drains what is queued (SetAsync(false), metal/shim.m:229-242)
    if (prev && !on) return check(hipDeviceSynchronize(), "set_async drain");
    return GORCH_HIP_OK;
}

int gorch_hip_async_enabled(void) { return g_async.load(); }

int gorch_hip_set_deterministic(int on) { return g_deterministic.exchange(on ? 1 : 0); }

int gorch_hip_deterministic_enabled(void) { return g_deterministic.load(); }

int gorch_hip_bf16_matmul_supported(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return 0;
    }
    return bf16_gate(nullptr) == GORCH_HIP_OK ? 1 : 0;
}

int gorch_hip_bf16_probe(void) {
    int dev = 0;
    GH_TRY(check(hipGetDevice(&dev), "hipGetDevice"));
    GH_REQUIRE(dev >= 0 && dev < kMaxDevices, "gorch_hip_bf16_probe: device index out of range");
    std::lock_guard<std::mutex> lock(g_probe_mu);
    return run_bf16_probe(dev) == 1 ? 1 : 0;
}

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
    if (device < kMaxDevices && g_probe[device].load(std::memory_order_acquire) == 0) {
        std::lock_guard<std::mutex> lock(g_probe_mu);
        if (g_probe[device].load(std::memory_order_acquire) == 0) (void)run_bf16_probe(device);
    }
    // The no-allocation entry point's scratch lookup is optional here: a
    // failure leaves that one entry point to retry (and report) on its own
    // first call, and does not fail the library's set-up.
    if (noalloc_setup(device) != GORCH_HIP_OK) clear_error();
    return GORCH_HIP_OK;
}

const char* gorch_hip_last_error(void) { return t_error.c_str(); }

void* gorch_hip_alloc(size_t bytes) {
    void* p = nullptr;
    if (check(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc")) return nullptr;
    std::lock_guard<std::mutex> lock(g_mem_mu);
    g_raw[p] = bytes;
    g_live_bytes += (long long)bytes;
    return p;
}

void gorch_hip_release(void* ptr) {
    if (!ptr) return;
    size_t bytes = 0;
    {
        std::lock_guard<std::mutex> lock(g_mem_mu);
        auto it = g_raw.find(ptr);
        if (it == g_raw.end()) return;  // not ours, or released already
        bytes = it->second;
        g_raw.erase(it);
    }
    g_live_bytes -= (long long)bytes;
    (void)hipFree(ptr);  // waits for work still using it
}

gorch_hip_buf* gorch_hip_buf_new(size_t bytes, int flags) {
    if (flags & ~GORCH_HIP_BUF_HOST_MIRROR) {
        set_error("gorch_hip_buf_new: unknown flag");
        return nullptr;
    }
    auto b = std::make_shared<Buf>();
    b->bytes = bytes;
    if (check(hipGetDevice(&b->device), "hipGetDevice") || check(hipMalloc(&b->dev, bytes ? bytes : 1), "hipMalloc"))
        return nullptr;
    // NewBuffer's contract: zero-filled (metal/metal.go:240-246)
    if (check(hipMemset(b->dev, 0, bytes ? bytes : 1), "hipMemset")) return nullptr;
    if (flags & GORCH_HIP_BUF_HOST_MIRROR) {
        if (check(hipHostMalloc(&b->host, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc")) return nullptr;
        std::memset(b->host, 0, bytes ? bytes : 1);
    }
    std::lock_guard<std::mutex> lock(g_mem_mu);
    const uintptr_t id = g_next_buf++;
    g_bufs[id] = b;
    g_live_bytes += (long long)bytes;
    return reinterpret_cast<gorch_hip_buf*>(id);
}

void gorch_hip_buf_release(gorch_hip_buf* h) {
    std::shared_ptr<Buf> b;
    {
        std::lock_guard<std::mutex> lock(g_mem_mu);
        auto it = g_bufs.find(reinterpret_cast<uintptr_t>(h));
        if (it == g_bufs.end()) return;
        b = std::move(it->second);
        g_bufs.erase(it);
    }
    g_live_bytes -= (long long)b->bytes;
    // the memory goes when the last user of the handle is done with it
}

size_t gorch_hip_buf_len(gorch_hip_buf* h) {
    auto b = find_buf(h);
    return b ? b->bytes : 0;
}

void* gorch_hip_buf_device(void* stream, gorch_hip_buf* h, int will_write) {
    auto b = find_buf(h);
    if (!b) {
        set_error("gorch_hip_buf_device: unknown or released buffer");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(b->mu);
    if (!b->dev_valid) {
        // the host wrote through the mirror: bring the device copy up to date
        hipStream_t s = stream_of(stream);
        if (check(hipMemcpyAsync(b->dev, b->host, b->bytes, hipMemcpyHostToDevice, s), "buf upload") ||
            check(hipStreamSynchronize(s), "buf upload sync"))
            return nullptr;
        b->dev_valid = true;
    }
    if (will_write && b->host) b->host_valid = false;
    return b->dev;
}

void* gorch_hip_buf_host(void* stream, gorch_hip_buf* h, int will_write) {
    auto b = find_buf(h);
    if (!b) {
        set_error("gorch_hip_buf_host: unknown or released buffer");
        return nullptr;
    }
    if (!b->host) {
        set_error("gorch_hip_buf_host: buffer has no host mirror");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(b->mu);
    hipStream_t s = stream_of(stream);
    // the read barrier: work queued on the stream may still write the buffer
    if (check(hipStreamSynchronize(s), "buf host sync")) return nullptr;
    if (!b->host_valid) {
        if (check(hipMemcpy(b->host, b->dev, b->bytes, hipMemcpyDeviceToHost), "buf download")) return nullptr;
        b->host_valid = true;
    }
    if (will_write) b->dev_valid = false;
    return b->host;
}

long long gorch_hip_live_bytes(void) { return g_live_bytes.load(); }

long long gorch_hip_scratch_bytes(void) { return scratch_bytes_held(); }

void gorch_hip_release_stream_scratch(void* stream) {
    hipStream_t s = stream_of(stream);
    (void)hipStreamSynchronize(s);
    release_stream_scratch(s);
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
