// safetensors.hip — safetensors checkpoints straight into device memory
// (gorch's LoadSafetensors / LoadSafetensorsNative, model/safetensors.go:
// 52-130, and the decoders at :132-184).
//
// File format (what the reference parses): 8-byte little-endian header
// length, a JSON object mapping tensor names to {dtype, shape,
// data_offsets} (plus an optional "__metadata__" entry), then the raw
// little-endian tensor bytes, offsets relative to the end of the header.
//
// The host side parses the header once (gorch_hip_st_open) and validates it
// the way the reference's loader fails: unknown dtypes, offsets outside the
// data, a byte count that does not match the shape. Tensors are then read
// on demand: the raw bytes go through a pinned staging buffer to a device
// scratch buffer, and one kernel decodes them into the destination — F32
// copied, F16 and BF16 widened exactly (decodeF16/decodeBF16), BF16 kept
// bit-for-bit in the native mode (decodeBF16Raw), F32 narrowed to BF16 with
// gorch's round-to-nearest-even (f32ToBF16, tensor.go:85-101) — optionally
// transposing a 2-D tensor through LDS tiles (GPT-2's Conv1D weights are
// stored (in, out); a Linear wants (out, in), model/gpt2_loader.go:170-184).
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"

namespace gh {

// ---------------------------------------------------------------- JSON
// The subset a safetensors header uses: objects, arrays, strings (with
// escapes), integers, and other scalars skipped.
namespace {
struct JParser {
    const char* p;
    const char* e;
    std::string err;

    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(char c) {
        ws();
        if (p < e && *p == c) {
            p++;
            return true;
        }
        return false;
    }
    bool fail(const char* what) {
        if (err.empty()) err = what;
        return false;
    }
    bool str(std::string& out) {
        ws();
        if (p >= e || *p != '"') return fail("expected a string");
        p++;
        out.clear();
        while (p < e && *p != '"') {
            char c = *p++;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p >= e) return fail("bad escape");
            c = *p++;
            switch (c) {
                case 'n': out.push_back('\n'); break;
                case 't': out.push_back('\t'); break;
                case 'r': out.push_back('\r'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'u': {
                    if (e - p < 4) return fail("bad \\u escape");
                    unsigned cp = 0;
                    for (int i = 0; i < 4; i++) {
                        const char h = *p++;
                        cp <<= 4;
                        if (h >= '0' && h <= '9') cp |= h - '0';
                        else if (h >= 'a' && h <= 'f') cp |= h - 'a' + 10;
                        else if (h >= 'A' && h <= 'F') cp |= h - 'A' + 10;
                        else return fail("bad \\u escape");
                    }
                    // UTF-8 encode (surrogate pairs are kept as two units)
                    if (cp < 0x80) {
                        out.push_back((char)cp);
                    } else if (cp < 0x800) {
                        out.push_back((char)(0xC0 | (cp >> 6)));
                        out.push_back((char)(0x80 | (cp & 0x3F)));
                    } else {
                        out.push_back((char)(0xE0 | (cp >> 12)));
                        out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
                        out.push_back((char)(0x80 | (cp & 0x3F)));
                    }
                    break;
                }
                default: out.push_back(c); break;  // \" \\ \/
            }
        }
        if (p >= e) return fail("unterminated string");
        p++;
        return true;
    }
    bool integer(long long& v) {
        ws();
        const char* s = p;
        if (p < e && *p == '-') p++;
        if (p >= e || *p < '0' || *p > '9') return fail("expected an integer");
        unsigned long long a = 0;
        while (p < e && *p >= '0' && *p <= '9') {
            const unsigned long long nx = a * 10 + (unsigned)(*p - '0');
            if (nx / 10 != a) return fail("integer overflow");
            a = nx;
            p++;
        }
        if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) return fail("expected an integer");
        if (a > (unsigned long long)INT64_MAX) return fail("integer overflow");
        v = *s == '-' ? -(long long)a : (long long)a;
        return true;
    }
    // skips any value
    bool skip(int depth = 0) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p >= e) return fail("unexpected end");
        if (*p == '"') {
            std::string t;
            return str(t);
        }
        if (*p == '{' || *p == '[') {
            const char close = *p == '{' ? '}' : ']';
            const bool obj = *p == '{';
            p++;
            if (lit(close)) return true;
            do {
                if (obj) {
                    std::string k;
                    if (!str(k) || !lit(':')) return fail("bad object");
                }
                if (!skip(depth + 1)) return false;
            } while (lit(','));
            return lit(close) || fail("bad container");
        }
        while (p < e && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\n' && *p != '\r' &&
               *p != '\t')
            p++;
        return true;
    }
};
}  // namespace

}  // namespace gh

struct gorch_hip_st {
    int fd = -1;
    long long file_bytes = 0, data_start = 0;
    std::vector<gh::StTensor> tensors;  // sorted by name (result.Names)
};

namespace gh {

static int elem_bytes(int dtype) { return dtype == GORCH_HIP_ST_F32 ? 4 : 2; }

static const StTensor* st_find(const gorch_hip_st* f, const char* name) {
    auto it = std::lower_bound(f->tensors.begin(), f->tensors.end(), std::string(name),
                               [](const StTensor& t, const std::string& n) { return t.name < n; });
    return it != f->tensors.end() && it->name == name ? &*it : nullptr;
}

static bool read_at(int fd, void* dst, size_t n, long long off) {
    char* d = static_cast<char*>(dst);
    while (n > 0) {
        const ssize_t r = pread(fd, d, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        d += r;
        n -= (size_t)r;
        off += r;
    }
    return true;
}

// -------------------------------------------------------------- device side
// Decoded value of one stored element (as f32 bits or as 16-bit bits) and
// its encoding for the destination.
enum StMode { kCopy16 = 0, kCopy32, kBf16ToF32, kF16ToF32, kF32ToBf16, kF16ToBf16 };

template <int MODE>
struct StConv;
template <>
struct StConv<kCopy16> {
    using S = uint16_t;
    using D = uint16_t;
    __device__ static D f(S v) { return v; }
};
template <>
struct StConv<kCopy32> {
    using S = uint32_t;
    using D = uint32_t;
    __device__ static D f(S v) { return v; }
};
template <>
struct StConv<kBf16ToF32> {
    using S = uint16_t;
    using D = uint32_t;
    __device__ static D f(S v) { return (uint32_t)v << 16; }
};
template <>
struct StConv<kF16ToF32> {
    using S = uint16_t;
    using D = uint32_t;
    __device__ static D f(S v) { return __float_as_uint((float)__builtin_bit_cast(_Float16, v)); }
};
template <>
struct StConv<kF32ToBf16> {
    using S = uint32_t;
    using D = uint16_t;
    __device__ static D f(S v) { return f32_to_bf16_bits(__uint_as_float(v)); }
};
template <>
struct StConv<kF16ToBf16> {
    using S = uint16_t;
    using D = uint16_t;
    __device__ static D f(S v) { return f32_to_bf16_bits((float)__builtin_bit_cast(_Float16, v)); }
};

template <int MODE>
__global__ __launch_bounds__(256) void k_st_convert(const void* __restrict__ src, void* __restrict__ dst, long long n) {
    using C = StConv<MODE>;
    const auto* s = static_cast<const typename C::S*>(src);
    auto* d = static_cast<typename C::D*>(dst);
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        d[i] = C::f(s[i]);
}

// dst[c][r] = conv(src[r][c]) for src [R, C]: 32x32 tiles through LDS, so
// both the reads and the writes run along rows.
template <int MODE>
__global__ __launch_bounds__(256) void k_st_transpose(const void* __restrict__ src, void* __restrict__ dst, long long R,
                                                      long long C) {
    using Cv = StConv<MODE>;
    __shared__ typename Cv::D tile[32][33];
    const auto* s = static_cast<const typename Cv::S*>(src);
    auto* d = static_cast<typename Cv::D*>(dst);
    const long long r0 = (long long)blockIdx.y * 32, c0 = (long long)blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int j = ty; j < 32; j += 8) {
        const long long r = r0 + j, c = c0 + tx;
        if (r < R && c < C) tile[j][tx] = Cv::f(s[r * C + c]);
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
        const long long c = c0 + j, r = r0 + tx;
        if (c < C && r < R) d[c * R + r] = tile[tx][j];
    }
}

template <int MODE>
static void st_launch(hipStream_t s, const void* raw, void* dst, long long n, bool transpose, long long R, long long C) {
    if (transpose) {
        const dim3 grid((unsigned)((C + 31) / 32), (unsigned)((R + 31) / 32));
        hipLaunchKernelGGL(k_st_transpose<MODE>, grid, dim3(256), 0, s, raw, dst, R, C);
    } else {
        long long g = (n + 255) / 256;
        if (g > 16384) g = 16384;
        if (g < 1) g = 1;
        hipLaunchKernelGGL(k_st_convert<MODE>, dim3((unsigned)g), dim3(256), 0, s, raw, dst, n);
    }
}

// Staging shared by all loads of the process: a pinned host buffer (file
// chunks) and a device buffer holding a tensor's raw bytes. Loads are
// serialised by the mutex and synchronous.
namespace {
std::mutex g_st_mu;
void* g_pinned = nullptr;
size_t g_pinned_bytes = 0;
void* g_raw = nullptr;
size_t g_raw_bytes = 0;
int g_raw_dev = -1;
constexpr size_t kChunk = (size_t)64 << 20;
}  // namespace

int st_load_tensor(hipStream_t s, const gorch_hip_st* f, const char* name, void* dst, int dst_dtype,
                   int transpose) {
    const StTensor* t = st_find(f, name);
    if (!t) {
        set_error(std::string("tensor \"") + name + "\" not found in safetensors");
        return GORCH_HIP_EINVAL;
    }
    if (dst_dtype != GORCH_HIP_ST_F32 && dst_dtype != GORCH_HIP_ST_BF16) {
        set_error("gorch_hip_st_load: destination dtype must be F32 or BF16");
        return GORCH_HIP_EINVAL;
    }
    if (transpose && t->shape.size() != 2) {
        set_error(std::string("gorch_hip_st_load: transpose needs a 2-D tensor: ") + name);
        return GORCH_HIP_EINVAL;
    }
    const long long bytes = t->end - t->begin;
    const long long n = bytes / elem_bytes(t->dtype);
    if (n == 0) return GORCH_HIP_OK;
    if (!dst) {
        set_error("gorch_hip_st_load: null destination");
        return GORCH_HIP_EINVAL;
    }
    std::lock_guard<std::mutex> lock(g_st_mu);
    int dev = 0;
    GH_TRY(check(hipGetDevice(&dev), "hipGetDevice"));
    if (!g_pinned) {
        GH_TRY(check(hipHostMalloc(&g_pinned, kChunk, hipHostMallocDefault), "hipHostMalloc staging"));
        g_pinned_bytes = kChunk;
    }
    if (g_raw_bytes < (size_t)bytes || g_raw_dev != dev) {
        if (g_raw) {
            (void)hipDeviceSynchronize();
            (void)hipFree(g_raw);
        }
        g_raw = nullptr;
        g_raw_bytes = 0;
        GH_TRY(check(hipMalloc(&g_raw, (size_t)bytes), "hipMalloc tensor staging"));
        g_raw_bytes = (size_t)bytes;
        g_raw_dev = dev;
    }
    for (long long off = 0; off < bytes; off += (long long)g_pinned_bytes) {
        const size_t len = (size_t)std::min<long long>((long long)g_pinned_bytes, bytes - off);
        if (!read_at(f->fd, g_pinned, len, f->data_start + t->begin + off)) {
            set_error(std::string("read tensor \"") + name + "\": short read");
            return GORCH_HIP_ERUNTIME;
        }
        GH_TRY(check(hipMemcpyAsync(static_cast<char*>(g_raw) + off, g_pinned, len, hipMemcpyHostToDevice, s),
                     "upload tensor"));
        // the pinned chunk is reused: wait for its copy
        GH_TRY(check(hipStreamSynchronize(s), "upload tensor"));
    }
    const bool tr = transpose != 0;
    const long long R = tr ? t->shape[0] : 0, C = tr ? t->shape[1] : 0;
    const int sd = t->dtype;
    if (dst_dtype == GORCH_HIP_ST_F32) {
        if (sd == GORCH_HIP_ST_F32) st_launch<kCopy32>(s, g_raw, dst, n, tr, R, C);
        else if (sd == GORCH_HIP_ST_BF16) st_launch<kBf16ToF32>(s, g_raw, dst, n, tr, R, C);
        else st_launch<kF16ToF32>(s, g_raw, dst, n, tr, R, C);
    } else {
        if (sd == GORCH_HIP_ST_BF16) st_launch<kCopy16>(s, g_raw, dst, n, tr, R, C);
        else if (sd == GORCH_HIP_ST_F32) st_launch<kF32ToBf16>(s, g_raw, dst, n, tr, R, C);
        else st_launch<kF16ToBf16>(s, g_raw, dst, n, tr, R, C);
    }
    count(CNT_CODEC);
    GH_TRY(check_launch("st_load"));
    // the raw staging buffer is reused by the next load
    return check(hipStreamSynchronize(s), "st_load");
}

const StTensor* st_tensor(const gorch_hip_st* f, const char* name) { return st_find(f, name); }

}  // namespace gh

using namespace gh;

extern "C" gorch_hip_st* gorch_hip_st_open(const char* path) {
    if (!path) {
        set_error("gorch_hip_st_open: null path");
        return nullptr;
    }
    auto* f = new gorch_hip_st();
    auto fail = [&](const std::string& msg) -> gorch_hip_st* {
        set_error(msg);
        if (f->fd >= 0) close(f->fd);
        delete f;
        return nullptr;
    };
    f->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) return fail(std::string("open safetensors: ") + path + ": " + strerror(errno));
    const off_t end = lseek(f->fd, 0, SEEK_END);
    if (end < 0) return fail("open safetensors: cannot size the file");
    f->file_bytes = (long long)end;
    unsigned char lenb[8];
    if (f->file_bytes < 8 || !read_at(f->fd, lenb, 8, 0)) return fail("read header length: file too short");
    unsigned long long hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | lenb[i];
    if (hlen > (unsigned long long)(f->file_bytes - 8) || hlen > ((unsigned long long)1 << 30))
        return fail("read header: header length exceeds the file");
    std::string json((size_t)hlen, '\0');
    if (hlen && !read_at(f->fd, &json[0], (size_t)hlen, 8)) return fail("read header: short read");
    f->data_start = 8 + (long long)hlen;
    const long long data_bytes = f->file_bytes - f->data_start;

    JParser jp{json.data(), json.data() + json.size(), {}};
    if (!jp.lit('{')) return fail("parse safetensors header: not a JSON object");
    if (!jp.lit('}')) {
        do {
            std::string name;
            if (!jp.str(name) || !jp.lit(':')) return fail("parse safetensors header: " + jp.err);
            if (name == "__metadata__") {
                if (!jp.skip()) return fail("parse safetensors header: " + jp.err);
                continue;
            }
            StTensor t;
            t.name = name;
            std::string dt;
            bool have_dt = false, have_shape = false, have_off = false;
            if (!jp.lit('{')) return fail("parse tensor \"" + name + "\" header: not an object");
            if (!jp.lit('}')) {
                do {
                    std::string key;
                    if (!jp.str(key) || !jp.lit(':')) return fail("parse tensor \"" + name + "\" header: " + jp.err);
                    if (key == "dtype") {
                        if (!jp.str(dt)) return fail("parse tensor \"" + name + "\" header: " + jp.err);
                        have_dt = true;
                    } else if (key == "shape" || key == "data_offsets") {
                        std::vector<long long> v;
                        if (!jp.lit('[')) return fail("parse tensor \"" + name + "\" header: bad " + key);
                        if (!jp.lit(']')) {
                            do {
                                long long x;
                                if (!jp.integer(x) || x < 0)
                                    return fail("parse tensor \"" + name + "\" header: bad " + key);
                                v.push_back(x);
                            } while (jp.lit(','));
                            if (!jp.lit(']')) return fail("parse tensor \"" + name + "\" header: bad " + key);
                        }
                        if (key == "shape") {
                            t.shape = v;
                            have_shape = true;
                        } else {
                            if (v.size() != 2) return fail("parse tensor \"" + name + "\" header: bad data_offsets");
                            t.begin = v[0];
                            t.end = v[1];
                            have_off = true;
                        }
                    } else if (!jp.skip()) {
                        return fail("parse tensor \"" + name + "\" header: " + jp.err);
                    }
                } while (jp.lit(','));
                if (!jp.lit('}')) return fail("parse tensor \"" + name + "\" header: bad object");
            }
            if (!have_dt || !have_shape || !have_off)
                return fail("parse tensor \"" + name + "\" header: missing dtype, shape or data_offsets");
            if (dt == "F32") t.dtype = GORCH_HIP_ST_F32;
            else if (dt == "F16") t.dtype = GORCH_HIP_ST_F16;
            else if (dt == "BF16") t.dtype = GORCH_HIP_ST_BF16;
            else return fail("unsupported dtype \"" + dt + "\" for tensor \"" + name + "\"");
            if (t.shape.size() > 8) return fail("tensor \"" + name + "\": more than 8 dimensions");
            long long numel = 1;
            for (long long d : t.shape) {
                if (d != 0 && numel > (INT64_MAX / 8) / d) return fail("tensor \"" + name + "\": shape overflow");
                numel *= d;
            }
            if (t.end < t.begin || t.end > data_bytes)
                return fail("tensor \"" + name + "\": data_offsets outside the file");
            if (t.end - t.begin != numel * elem_bytes(t.dtype))
                return fail("tensor \"" + name + "\": byte count does not match its shape and dtype");
            f->tensors.push_back(std::move(t));
        } while (jp.lit(','));
        if (!jp.lit('}')) return fail("parse safetensors header: bad object");
    }
    std::sort(f->tensors.begin(), f->tensors.end(), [](const StTensor& a, const StTensor& b) { return a.name < b.name; });
    for (size_t i = 1; i < f->tensors.size(); i++)
        if (f->tensors[i].name == f->tensors[i - 1].name)
            return fail("parse safetensors header: duplicate tensor \"" + f->tensors[i].name + "\"");
    return f;
}

extern "C" void gorch_hip_st_close(gorch_hip_st* f) {
    if (!f) return;
    if (f->fd >= 0) close(f->fd);
    delete f;
}

extern "C" int gorch_hip_st_count(const gorch_hip_st* f) { return f ? (int)f->tensors.size() : 0; }

extern "C" const char* gorch_hip_st_name(const gorch_hip_st* f, int i) {
    if (!f || i < 0 || i >= (int)f->tensors.size()) return nullptr;
    return f->tensors[i].name.c_str();
}

extern "C" int gorch_hip_st_info(const gorch_hip_st* f, const char* name, int* dtype, int* ndim, int64_t* shape,
                                 int64_t* nbytes) {
    GH_REQUIRE(f && name, "gorch_hip_st_info: null argument");
    const StTensor* t = st_find(f, name);
    if (!t) {
        set_error(std::string("tensor \"") + name + "\" not found in safetensors");
        return GORCH_HIP_EINVAL;
    }
    if (dtype) *dtype = t->dtype;
    if (ndim) *ndim = (int)t->shape.size();
    if (shape)
        for (size_t i = 0; i < t->shape.size(); i++) shape[i] = t->shape[i];
    if (nbytes) *nbytes = t->end - t->begin;
    return GORCH_HIP_OK;
}

extern "C" int gorch_hip_st_load(void* stream, const gorch_hip_st* f, const char* name, void* dst, int dst_dtype,
                                 int transpose) {
    GH_REQUIRE(f && name, "gorch_hip_st_load: null argument");
    return st_load_tensor(stream_of(stream), f, name, dst, dst_dtype, transpose);
}
