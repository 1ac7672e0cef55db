// common.h — shared device helpers and host error plumbing for libgorch_hip.
//
// gfx950 only: 64-lane wavefronts, bf16 MFMA, hardware f32->bf16 convert.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

#include <cstdio>
#include <string>
#include <vector>

#include "../../include/gorch_hip.h"

namespace gh {

// ---------------------------------------------------------------- host side

// Thread-local last error, returned by gorch_hip_last_error().
void set_error(const std::string& msg);
void clear_error();

// A caller's stream argument (NULL = the device's null stream).
hipStream_t stream_of(void* s);

struct OutDesc;
// Optional fusions of the weight-streaming GEMV (M <= 16):
//   ln_g/ln_b: LayerNorm of each activation row applied as it is loaded;
//   argmax_key: per-row packed (value, index) maximum of the outputs,
//     combined with 64-bit atomicMax into the block's slot of a
//     kArgmaxKeys-entry key array (argmax_slot; all zero before the call).
struct LinearExtras {
    const float* ln_g = nullptr;
    const float* ln_b = nullptr;
    float ln_eps = 1e-5f;
    unsigned long long* argmax_key = nullptr;
    long long x_stride = 0;  // activation row stride in elements (0 = K)
    // LayerNorm row statistics (mean, 1/sqrt(var + eps)) computed by an
    // earlier kernel; null: the GEMV computes them itself
    const float2* ln_stats = nullptr;
    // K split across ksplit blocks: raw partial sums to part[s][m][n]
    // (bias, activation and residual are then applied by the reduction)
    float* part = nullptr;
    // tile-packed GEMV only: K split across ksplit blocks that add their
    // partial sums (slice 0 also the bias) into the output with float
    // atomics; the output holds what they add to (the residual), and the
    // order of the additions varies between runs
    bool accumulate = false;
    // tile-packed GEMV only: the activations come pre-split in the fragment
    // layout (xfrag_index) instead of as f32 rows of x (no fused LayerNorm,
    // x_stride unused)
    const uint16_t* x_frag = nullptr;
    // tile-packed GEMV only: the outputs go to this fragment-layout buffer
    // (as the next GEMV's pre-split activations) instead of the output
    // descriptor (with x_frag; no K split, no argmax)
    uint16_t* out_frag = nullptr;
    int ksplit = 1;
    int kslice = 0;    // K per slice (set by the launcher)
    int split_nt = 0;  // 16-row tiles per block in split mode (0: 4)
    // caller-provided device scratch for the narrow-weight K split (null:
    // the stream's scratch); a split that needs more fails with EINVAL
    float* scratch = nullptr;
    size_t scratch_bytes = 0;
    // one-row register GEMV only: ln_g is an RMSNorm gain (no beta, no mean)
    bool ln_rms = false;
    // one-row register GEMV only: the activation row is [gate | up] of 2K
    // values and the GEMV reads silu(gate) * up
    bool swiglu = false;
    // one-row register GEMV only: W is [gate | up] of 2 * pair_swiglu rows
    // (N = 2 * pair_swiglu); output j = silu(gate_j) * up_j, rows j and
    // pair_swiglu + j computed by one wave (no bias, residual or GELU)
    int pair_swiglu = 0;
};
// Most K slices a K-split partial buffer holds (k_splitk_epilogue, the
// row reducer, the split QKV input of the cached attention).
constexpr int kMaxPartSlices = 8;
// Number of K slices a K-split Linear actually uses for a requested count
// (slices are multiples of 32 wide).
inline int ksplit_slices(int K, int S) {
    const int ks = ((K + S - 1) / S + 31) / 32 * 32;
    return (K + ks - 1) / ks;
}
// sample() (model/generate.go:147-243) per row (sample.hip): the draw is
// u[row], or Philox4x32-10 of (seed, *step, row) when u is null; key (may be
// null) receives a fused-argmax key decoding to the token, err (may be null)
// is set when the top-p candidates exceed the sort's capacity. nucleus: top-p
// as the Qwen loop's sampleLogits (model/qwen/generate.go:121-152).
int launch_sample(hipStream_t s, const float* logits, int rows, int n, float temperature, int top_k, float top_p,
                  const double* u, unsigned long long seed, const int* step, int* out, double* probs,
                  unsigned long long* key, int* err, bool nucleus = false, int* ws = nullptr);
// Workspace for launch_sample's ws (zeroed once at allocation; every call
// leaves it zero): with it, a top-k row's two candidate-search passes run
// over many blocks per row instead of inside the row's one block. Calls that
// share a workspace must not overlap.
size_t sample_ws_bytes(int rows);
int sample_check(int rows, int n, float temperature, int top_k, float top_p);
// Per-(device, stream) scratch for K-split partials; nullptr when it would
// have to grow during stream capture or the allocation fails.
void* stream_scratch(hipStream_t s, size_t bytes);
// Epilogue of a K-split Linear over partials part[S][M][N] (S <= 8).
int launch_splitk_epilogue(hipStream_t s, const float* part, int S, int M, int N, const float* bias,
                           const float* residual, const OutDesc& od, int epilogue);
// Widest row launch_reduce_rows handles.
constexpr int kReduceRowsMaxCols = 2048;
// Row reduction after a K-split Linear: x[m] = x[m] + bias + sum_s part[s][m]
// (slices added in order; S = 0 leaves x as is), then the LayerNorm
// statistics of the new row into stats[m] when stats is not null, and with
// h the normalised row h[m] = LayerNorm(x[m]; ln_g, ln_b) as well; with hf
// (M <= 16) that row goes to hf in the fragment layout (xfrag_index).
int launch_reduce_rows(hipStream_t s, const float* part, int S, const float* bias, float* x, int M, int N,
                       float eps, float2* stats, const float* ln_g = nullptr, const float* ln_b = nullptr,
                       float* h = nullptr, uint16_t* hf = nullptr);
int launch_linear_bf16(hipStream_t s, const float* x, const uint16_t* W, const float* bias,
                       const float* residual, float* y, int M, int N, int K, int epilogue);
// Tile-packed bf16 weights (gemv.hip): element count of the packed copy,
// the pack kernel, and the M <= 16 Linear over it.
size_t packed_bf16_elems(int N, int K);
int launch_pack_bf16(hipStream_t s, const uint16_t* W, uint16_t* Wp, int N, int K);
int launch_linear_packed_od(hipStream_t s, const float* x, const uint16_t* Wp, const float* bias,
                            const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                            const LinearExtras& ex);
// K slices the packed GEMV uses for a K-split of an [N, K] weight.
int packed_split_slices(int K, int N);
int launch_linear_bf16_od(hipStream_t s, const float* x, const uint16_t* W, const float* bias,
                          const float* residual, const OutDesc& od, int M, int N, int K, int epilogue,
                          const LinearExtras& ex);

// Per-device address of the no-allocation entry point's scratch array,
// looked up once per device (gorch_hip_init or that entry point's first
// call on the device).
int noalloc_setup(int device);
// Device bytes held by the per-stream scratch buffers (stream_scratch).
long long scratch_bytes_held();
// Frees the scratch of a stream about to be destroyed (its work finished,
// no graph left that points at it): the library's engines call it for their
// own streams, so a later stream at the same address starts without one.
void release_stream_scratch(hipStream_t s);

// gorch_hip_set_deterministic's setting: no float-atomic sums when true.
bool deterministic();

// End of a compute entry point: in sync mode (gorch_hip_set_async(0)) waits
// for the stream when rc is 0 and the stream is not being captured.
int finish(void* stream, int rc);
// GORCH_HIP_EUNSUPPORTED unless the bf16 matmul probe passed on the current
// device (runs it first if gorch_hip_init has not and may_probe is set; the
// probe allocates).
int bf16_gate(hipStream_t s, bool may_probe = true);

// Dispatch counters (the gorch ReadMetalDispatchCounts analogue).
enum Counter {
    CNT_GEMV = 0,
    CNT_GEMM,
    CNT_GENERIC_MATMUL,
    CNT_ATTENTION,
    CNT_NORM,
    CNT_ELEMENTWISE,
    CNT_MOE,
    CNT_ARGMAX,
    CNT_CODEC,
    CNT_COUNT
};
void count(Counter c);

// Returns 0 or sets the error from a HIP status and returns its code.
int check(hipError_t e, const char* what);
// Checks the last launch on the calling thread.
int check_launch(const char* what);

#define GH_TRY(expr)                 \
    do {                             \
        int _rc = (expr);            \
        if (_rc != 0) return _rc;    \
    } while (0)

#define GH_REQUIRE(cond, msg)                 \
    do {                                      \
        if (!(cond)) {                        \
            ::gh::set_error(msg);             \
            return GORCH_HIP_EINVAL;          \
        }                                     \
    } while (0)

// A configuration the kernels do not handle (the caller's cue for its CPU
// path), as opposed to a bad argument.
#define GH_SUPPORTED(cond, msg)               \
    do {                                      \
        if (!(cond)) {                        \
            ::gh::set_error(msg);             \
            return GORCH_HIP_EUNSUPPORTED;    \
        }                                     \
    } while (0)

// ---------------------------------------------------------------- device side

// Where a Linear's output element (m, n) goes. Columns split into up to
// three segments (the fused QKV projection: Q to a buffer, K and V straight
// into the KV cache). Row m of a segment lands at
//   ptr + (m / rows_per_seq) * seq_stride + (m % rows_per_seq + pos) * row_stride + (n - n_begin)
// where pos is *pos_dev for segments with use_pos set (the cache length
// before this forward), else 0.
struct OutDesc {
    float* ptr[3];
    int n_end[3];
    long long seq_stride[3];
    long long row_stride[3];
    int use_pos[3];
    int nseg;
    int rows_per_seq;
    const int* pos_dev;

    static OutDesc plain(float* y, int N) {
        OutDesc d{};
        d.ptr[0] = y;
        d.n_end[0] = N;
        d.seq_stride[0] = 0;
        d.row_stride[0] = N;
        d.use_pos[0] = 0;
        d.nseg = 1;
        d.rows_per_seq = 1 << 30;
        d.pos_dev = nullptr;
        return d;
    }

    // Segment fields are read as wave-uniform scalars and picked with
    // selects: a runtime-indexed (or select-addressed) kernel argument
    // becomes a per-lane vector load, and every output element would then
    // wait on descriptor loads.
    __device__ static __forceinline__ long long uni(long long v) {
        const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(v & 0xffffffffll));
        const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(v >> 32));
        return (long long)(((unsigned long long)hi << 32) | lo);
    }
    __device__ __forceinline__ float* at(int m, int n) const { return at_p(m, n, pos_dev ? *pos_dev : 0); }
    // pos: the value of *pos_dev, read once by a caller that writes in a
    // loop (a load in its epilogue would wait for its prefetched weights)
    __device__ __forceinline__ float* at_p(int m, int n, int pos) const {
        int seq = 0, r = m;
        if (rows_per_seq < (1 << 30)) {
            seq = m / rows_per_seq;
            r = m - seq * rows_per_seq;
        }
        if (nseg == 1) {
            if (use_pos[0]) r += pos;
            return ptr[0] + seq * seq_stride[0] + (long long)r * row_stride[0] + n;
        }
        const bool s1 = n >= __builtin_amdgcn_readfirstlane(n_end[0]);
        const bool s2 = nseg > 2 && n >= __builtin_amdgcn_readfirstlane(n_end[1]);
        // segment bases as element offsets from ptr[0], so the result keeps
        // the global address space (a pointer rebuilt from integers is
        // generic, and its flat stores wait on LDS traffic too)
        const long long d1 = uni((long long)(ptr[1] - ptr[0])), d2 = uni((long long)(ptr[2] - ptr[0]));
        const long long ss0 = uni(seq_stride[0]), ss1 = uni(seq_stride[1]), ss2 = uni(seq_stride[2]);
        const long long rs0 = uni(row_stride[0]), rs1 = uni(row_stride[1]), rs2 = uni(row_stride[2]);
        const int up0 = __builtin_amdgcn_readfirstlane(use_pos[0]), up1 = __builtin_amdgcn_readfirstlane(use_pos[1]),
                  up2 = __builtin_amdgcn_readfirstlane(use_pos[2]);
        const int ne0 = __builtin_amdgcn_readfirstlane(n_end[0]), ne1 = __builtin_amdgcn_readfirstlane(n_end[1]);
        float* p = ptr[0] + (s2 ? d2 : (s1 ? d1 : 0));
        const int nb = s2 ? ne1 : (s1 ? ne0 : 0);
        const long long ss = s2 ? ss2 : (s1 ? ss1 : ss0);
        const long long rs = s2 ? rs2 : (s1 ? rs1 : rs0);
        const int up = s2 ? up2 : (s1 ? up1 : up0);
        if (up) r += pos;
        return p + seq * ss + (long long)r * rs + (n - nb);
    }
    // at_p split for a writer of many rows per column: col() resolves the
    // segment of column n once, row() adds the row part (same addresses)
    struct Col {
        float* p;
        long long ss, rs;
        int radd;
    };
    __device__ __forceinline__ Col col(int n, int pos) const {
        if (nseg == 1) return Col{ptr[0] + n, seq_stride[0], row_stride[0], use_pos[0] ? pos : 0};
        const bool s1 = n >= __builtin_amdgcn_readfirstlane(n_end[0]);
        const bool s2 = nseg > 2 && n >= __builtin_amdgcn_readfirstlane(n_end[1]);
        const long long d1 = uni((long long)(ptr[1] - ptr[0])), d2 = uni((long long)(ptr[2] - ptr[0]));
        const long long ss0 = uni(seq_stride[0]), ss1 = uni(seq_stride[1]), ss2 = uni(seq_stride[2]);
        const long long rs0 = uni(row_stride[0]), rs1 = uni(row_stride[1]), rs2 = uni(row_stride[2]);
        const int up0 = __builtin_amdgcn_readfirstlane(use_pos[0]), up1 = __builtin_amdgcn_readfirstlane(use_pos[1]),
                  up2 = __builtin_amdgcn_readfirstlane(use_pos[2]);
        const int ne0 = __builtin_amdgcn_readfirstlane(n_end[0]), ne1 = __builtin_amdgcn_readfirstlane(n_end[1]);
        const int nb = s2 ? ne1 : (s1 ? ne0 : 0);
        Col c;
        c.p = ptr[0] + (s2 ? d2 : (s1 ? d1 : 0)) + (n - nb);
        c.ss = s2 ? ss2 : (s1 ? ss1 : ss0);
        c.rs = s2 ? rs2 : (s1 ? rs1 : rs0);
        c.radd = (s2 ? up2 : (s1 ? up1 : up0)) ? pos : 0;
        return c;
    }
    __device__ __forceinline__ float* row(const Col& c, int m) const {
        int seq = 0, r = m;
        if (rows_per_seq < (1 << 30)) {
            seq = m / rows_per_seq;
            r = m - seq * rows_per_seq;
        }
        return c.p + seq * c.ss + (long long)(r + c.radd) * c.rs;
    }
};

// Arguments of the cached-attention kernel (attention.hip).
struct AttnArgs {
    const float* q;      // [rows, q_stride], head h at columns h*hd
    const float* kc;     // [batch][max_seq][dim]
    const float* vc;
    float* out;          // [rows, dim]
    const int* pos_dev;  // cache length before the new rows (device), or null
    int pos_host;        // used when pos_dev is null
    int new_seq, dim, hd, max_seq, q_stride, causal;
    float scale;
    int kv_heads;  // grouped-query attention: KV heads (0 = one per query head)
    int kv_dim;    // cache row stride in floats (0 = dim)
    int recip;     // normalise by multiplying with 1/sum (GQA) instead of dividing
    // not null (at most 16 rows): the output goes here in the fragment
    // layout (xfrag_index, K = dim) instead of to out
    uint16_t* out_frag = nullptr;
    // One new row per sequence (new_seq == 1, no grouped KV heads) whose
    // fused QKV Linear ran split over K: q, k and v of the row are qkv_bias
    // + the qkv_slices partial sums at qkv_part ([slice][row][3 * dim],
    // slices qkv_slice_stride floats apart, added in slice order). The
    // kernel writes k and v into the cache at row pos itself (its block is
    // the only reader of that head's slice in this step); q is not stored.
    const float* qkv_part = nullptr;
    const float* qkv_bias = nullptr;
    int qkv_slices = 0;
    long long qkv_slice_stride = 0;
    // The output projection fused into the one-row attention kernel
    // (launch_attn_rows_wo): wo_out[n] += sum_c wo[n][h*hd + c] * o_h[c]
    // for every head h (+ wo_bias[n] once), wo bf16 [dim][dim] row-major
    const uint16_t* wo = nullptr;
    const float* wo_bias = nullptr;
    float* wo_out = nullptr;
    // key-split path with the output projection (a.wo set): Wo has wo_rows
    // rows (0: dim) of row stride dim; wo_out is first set to wo_resid (or
    // zeros) by the split kernel, then k_attn_combine_wo adds every head's
    // Wo . o_h (+ wo_bias from head 0) with float atomics
    int wo_rows = 0;
    const float* wo_resid = nullptr;
    // Scratch for the key-split long-cache path (one new row, fewer than
    // 128 heads): per (head, key chunk) the chunk's max, weight sum and
    // unnormalised weighted values, hd + 2 floats. Null: one block per head.
    float* split_ws = nullptr;
    long long split_ws_floats = 0;
    // Key-split path only (attn_split_takes_qk): the projection's q/k
    // epilogue in the attention kernel — per-head RMSNorm (q_gain, k_gain,
    // qk_eps; null gain: none), then RoPE at the row's position (rope_cos /
    // rope_sin tables, rope_neox pairing; null: none). a.q holds q before
    // it; k_raw the new row's K before it ([kv heads * hd]): the kernel
    // writes the finished row into the K cache and uses it for that key.
    const float* k_raw = nullptr;
    const float* q_gain = nullptr;
    const float* k_gain = nullptr;
    float qk_eps = 0.f;
    const float* rope_cos = nullptr;
    const float* rope_sin = nullptr;
    int rope_neox = 0;
};
// Key chunks per head of the key-split long-cache attention, at most.
constexpr int kAttnSplitMax = 16;
// True when launch_attn_cached takes the key-split path for a (so it can
// also finish q and k: AttnArgs::k_raw).
bool attn_split_takes_qk(const AttnArgs& a, int heads, int rows);
// The kernel launch_attn_cached picks for a; true when it is the two-pass
// cached kernel, the one that takes split QKV partials.
bool attn_takes_qkv_part(const AttnArgs& a, int heads, int rows);
// One new row of one sequence with the output projection fused (a.wo,
// a.wo_bias, a.wo_out set): launch_attn_rows_wo adds Wo . attention + bias
// into a.wo_out with float atomics (so the order of the per-head additions
// varies between runs). attn_rows_wo_ok: the shapes it takes (the one-pass
// short-cache kernel's).
bool attn_rows_wo_ok(const AttnArgs& a, int heads, int rows);
int launch_attn_rows_wo(hipStream_t s, const AttnArgs& a, int heads);
// LDS the score-staging attention kernels may take (one f32 per visible
// key: 16384 keys); longer caches go to the online-softmax kernel.
constexpr size_t kAttnMaxLdsBytes = 65536;
int launch_attn_cached(hipStream_t s, const AttnArgs& a, int heads, int rows);
// The attention kernels address one sequence's K (or V) rows through a
// buffer resource whose byte span and offsets are 32-bit: a sequence's cache
// of max_seq rows of kv_dim floats must stay below the out-of-range offset
// (0x7fff0000 bytes, just under 2 GiB). Longer caches are refused.
inline bool kv_span_ok(long long max_seq, long long kv_dim) { return max_seq * kv_dim * 4 < 0x7fff0000LL; }

// GQA.forwardCached for one sequence (gqa.hip); pre_gain: an RMSNorm of x
// applied first (the decoder block's), resid: added to the output. ws holds
// gqa_ws(...) bytes.
size_t gqa_ws(int new_seq, int num_q, int num_kv, int hd, int dim);
int gqa_check(const gorch_hip_gqa_weights* w, int S, int pos_offset, int max_seq);
// pos_dev (one-row steps only): the position is read on the device (a
// graph-replayed decode step); pos_offset is then ignored, and shapes whose
// step does not take the key-split attention with the q/k norm and RoPE
// inside return GORCH_HIP_EUNSUPPORTED.
int gqa_core(hipStream_t s, const gorch_hip_gqa_weights* w, const float* x, int S, float* k_cache, float* v_cache,
             int pos_offset, int max_seq, float* out, char* ws, const float* pre_gain, float pre_eps,
             const float* resid, const int* pos_dev = nullptr);
int launch_rmsnorm(hipStream_t s, const float* x, const float* g, float* y, int M, int N, float eps);
// The one-row register GEMV takes K (RMSNorm / SwiGLU prologues need it).
bool gemv_m1_prologue_ok(int K);
// The one-row GEMV can pair the gate and up rows of a [2F, K] weight
// (LinearExtras::pair_swiglu = F).
bool gemv_pair_swiglu_ok(int F, int K);
int launch_swiglu(hipStream_t s, const float* g, const float* v, float* y, int64_t n);

// A tensor entry of a safetensors header (safetensors.hip): dtype
// GORCH_HIP_ST_*, shape, byte range relative to the data section.
struct StTensor {
    std::string name;
    int dtype = -1;
    std::vector<long long> shape;
    long long begin = 0, end = 0;
};
const StTensor* st_tensor(const gorch_hip_st* f, const char* name);
// gorch_hip_st_load without the argument checks of the C entry point.
int st_load_tensor(hipStream_t s, const gorch_hip_st* f, const char* name, void* dst, int dst_dtype, int transpose);

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// bf16 stored in the low half of a 16-bit word -> f32: an exact shift.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// gorch's f32 -> bf16 rounding: NaN keeps its top half with the quiet bit
// set; everything else rounds to nearest even on the dropped 16 bits.
__host__ __device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t bits = __float_as_uint(v);
#else
    uint32_t bits;
    __builtin_memcpy(&bits, &v, 4);
#endif
    if (((bits >> 23) & 0xffu) == 0xffu && (bits & 0x7fffffu) != 0)
        return (uint16_t)((bits >> 16) | 0x40u);
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

// Splits eight f32 values into bf16 hi + bf16 lo with x ~= hi + lo to about
// 2^-16 relative: hi is x truncated to bf16 (exact in f32), lo is the
// remainder rounded to bf16. Two bf16 MFMAs over (hi, lo) against an exact
// bf16 weight reproduce the f32-activation product to ~1e-5 relative.
__device__ __forceinline__ void split_hi_lo(const float (&f)[8], bf16x8& hi, bf16x8& lo) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t u = __float_as_uint(f[i]) & 0xffff0000u;
        float h = __uint_as_float(u);
        hi[i] = __builtin_bit_cast(__bf16, (uint16_t)(u >> 16));
        lo[i] = (__bf16)(f[i] - h);
    }
}

// Fragment layout of up to 16 activation rows of K columns, the tile GEMV's
// MFMA A operand already split: k-step j (columns 32 j .. 32 j + 31) takes
// 2 KB, the bf16 hi parts of lanes 0..63 then their lo parts (split_hi_lo),
// lane 16 g + r holding row r, columns 32 j + 8 g .. 32 j + 8 g + 7. A wave
// reads one k-step as two contiguous 1 KB loads. Rows and columns nobody
// writes keep what the buffer held (zero it once at allocation: columns
// past K must read as zeros; rows past M only feed outputs nobody stores).
__host__ __device__ inline size_t xfrag_bytes(int K) { return (size_t)((K + 31) / 32) * 2048; }
// uint16 index of the hi part of (row m, column k); the lo part is 512 on
__device__ __forceinline__ size_t xfrag_index(int m, int k) {
    return (size_t)(k >> 5) * 1024 + (size_t)((((k >> 3) & 3) * 16 + m) * 8 + (k & 7));
}
// hi/lo bits of one value, as split_hi_lo makes them
__device__ __forceinline__ void split_hi_lo1(float f, uint16_t& hi, uint16_t& lo) {
    const uint32_t u = __float_as_uint(f) & 0xffff0000u;
    hi = (uint16_t)(u >> 16);
    lo = __builtin_bit_cast(uint16_t, (__bf16)(f - __uint_as_float(u)));
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource over [p, p + bytes) (bytes < 2^31): buffer loads at
// offsets >= bytes return zero without touching memory, which lets a kernel
// drop its bounds-check branches (a load under a branch makes the compiler
// wait for every outstanding load before the next use). Word 3 selects the
// 32-bit data format, the gfx9 setting for untyped buffer access. p and
// bytes must be wave-uniform; the size is read back as a scalar so a clamp
// computed on the vector unit does not force a per-lane (waterfall) loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, long long bytes) {
    const int n = __builtin_amdgcn_readfirstlane((int)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, n, 0x00020000);
}
constexpr int kOutOfRange = 0x7fff0000;  // an offset past any resource (+ small immediates)
// Cache policy (the buffer loads' aux bits) for data a launch reads once and
// the next launches do not reuse: GEMV weights, K/V cache rows. 2 is the nt
// (non-temporal) bit; measured faster than the default policy for every
// GEMV shape of the decode path.
#ifndef GH_STREAM_POLICY
#define GH_STREAM_POLICY 2
#endif
constexpr int kStreamPolicy = GH_STREAM_POLICY;

__device__ __forceinline__ floatx4 mfma16x16x32(const bf16x8& a, const bf16x8& b, const floatx4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Greedy-argmax key (model/generate.go:134-144 semantics under atomicMax):
// the high word orders floats, the low word is ~index so ties keep the
// first index. A NaN never wins, except at index 0, where it always wins
// (the reference's loop keeps a leading NaN since no comparison beats it).
__device__ __forceinline__ unsigned long long argmax_pack(float v, int idx) {
    uint32_t b = __float_as_uint(v);
    uint32_t ord;
    if (v != v) ord = idx == 0 ? 0xffffffffu : 0u;
    else ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ int argmax_unpack(unsigned long long key) {
    return (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
}
// Fused-argmax key arrays hold kArgmaxSlots slots of kArgmaxStride keys
// (key[slot * kArgmaxStride + row], rows < 16, all zero between uses): a
// GEMV block combines its rows' maxima into slot blockIdx.x % kArgmaxSlots,
// so the end-of-kernel atomics of hundreds of blocks spread over addresses
// 256 bytes apart instead of queueing on one; the consumer takes the
// maximum over the slots and clears them (argmax_take).
constexpr int kArgmaxSlots = 16, kArgmaxStride = 32, kArgmaxKeys = kArgmaxSlots * kArgmaxStride;
__device__ __forceinline__ unsigned long long* argmax_slot(unsigned long long* key) {
    return key + (blockIdx.x % kArgmaxSlots) * kArgmaxStride;
}
__device__ __forceinline__ unsigned long long argmax_take(unsigned long long* key, int row) {
    unsigned long long v[kArgmaxSlots];
#pragma unroll
    for (int q = 0; q < kArgmaxSlots; q++) v[q] = key[q * kArgmaxStride + row];
    unsigned long long best = 0ull;
#pragma unroll
    for (int q = 0; q < kArgmaxSlots; q++) {
        best = v[q] > best ? v[q] : best;
        key[q * kArgmaxStride + row] = 0ull;
    }
    return best;
}

// tanh-form GELU as gorch computes it (ops.go:417-443), f32 throughout.
__device__ __forceinline__ float gelu_tanh(float x) {
    float x3 = x * x * x;
    float inner = 0.7978845608f * (x + 0.044715f * x3);
    return 0.5f * x * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float sigmoidf_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

// Wavefront (64-lane) reductions on the VALU's DPP lane network, with
// v_readlane for the last step across the four 16-lane rows (a __shfl_xor
// compiles to ds_bpermute, an LDS round trip per step, each waited for).
// All 64 lanes must be active. Every lane returns the same value: within a
// row, lane pairs (i, i^1), (i, i^2), half-row mirrors and row mirrors
// exchange and add partial sums, which gives all 16 lanes the same
// operands in the same order; the rows are then combined as
// (row0 + row1) + (row2 + row3).
constexpr int kDppQuadSwap1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <- lane 7-i within each 8 lanes
constexpr int kDppRowMirror = 0x140;     // lane i <- lane 15-i within each 16 lanes
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Row statistics in f64 (LayerNorm / RMSNorm): a / b with rb = 1/b as one
// product and one FMA correction, and 1/sqrt(v) (v > 0) as the hardware
// reciprocal square root refined by one Newton step. Both are accurate to
// f64 rounding (the quotient's correction is Markstein's), where the
// library's correctly rounded division and square root are dependent
// sequences of ~12 f64 instructions each on the critical path of every
// fused norm; the callers round the result to f32.
__device__ __forceinline__ double div_rcp(double a, double b, double rb) {
    const double q = a * rb;
    return fma(fma(-q, b, a), rb, q);
}
__device__ __forceinline__ double rsqrt_f64(double v) {
    const double y = __builtin_amdgcn_rsq(v);
    return y * fma(-0.5 * v * y, y, 1.5);
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
// Sum over aligned segments of T lanes (T = 4, 8, 16, 32 or 64): every lane
// of a segment returns the segment's sum.
template <int T>
__device__ __forceinline__ float seg_sum(float v) {
    static_assert(T == 4 || T == 8 || T == 16 || T == 32 || T == 64, "segment of 4..64 lanes");
    v += dpp_f<kDppQuadSwap1>(v);
    v += dpp_f<kDppQuadSwap2>(v);
    if constexpr (T >= 8) v += dpp_f<kDppRowHalfMirror>(v);
    if constexpr (T >= 16) v += dpp_f<kDppRowMirror>(v);
    if constexpr (T == 32) {
        const float a = readlane_f(v, 0) + readlane_f(v, 16);
        const float b = readlane_f(v, 32) + readlane_f(v, 48);
        v = (threadIdx.x & 32) ? b : a;
    } else if constexpr (T == 64) {
        v = (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
    }
    return v;
}
__device__ __forceinline__ float wave_sum(float v) { return seg_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppQuadSwap1>(v));
    v = fmaxf(v, dpp_f<kDppQuadSwap2>(v));
    v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppRowMirror>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<kDppQuadSwap1>(v);
    v += dpp_d<kDppQuadSwap2>(v);
    v += dpp_d<kDppRowHalfMirror>(v);
    v += dpp_d<kDppRowMirror>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
// Two f64 sums over the wavefront at once (independent chains, one
// latency); every lane returns both totals.
__device__ __forceinline__ void wave_sum2_d(double& a, double& b) {
    a += dpp_d<kDppQuadSwap1>(a);
    b += dpp_d<kDppQuadSwap1>(b);
    a += dpp_d<kDppQuadSwap2>(a);
    b += dpp_d<kDppQuadSwap2>(b);
    a += dpp_d<kDppRowHalfMirror>(a);
    b += dpp_d<kDppRowHalfMirror>(b);
    a += dpp_d<kDppRowMirror>(a);
    b += dpp_d<kDppRowMirror>(b);
    a = (readlane_d(a, 0) + readlane_d(a, 16)) + (readlane_d(a, 32) + readlane_d(a, 48));
    b = (readlane_d(b, 0) + readlane_d(b, 16)) + (readlane_d(b, 32) + readlane_d(b, 48));
}
// Maximum of a 64-bit key over each row of 16 lanes (all lanes active);
// every lane of the row returns it.
__device__ __forceinline__ unsigned long long row16_max_u64(unsigned long long v) {
    auto dpp_u64 = [](unsigned long long x, auto ctrl_tag) {
        constexpr int C = decltype(ctrl_tag)::value;
        const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)x, C, 0xF, 0xF, false);
        const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(x >> 32), C, 0xF, 0xF, false);
        return ((unsigned long long)hi << 32) | lo;
    };
    unsigned long long o;
    o = dpp_u64(v, std::integral_constant<int, kDppQuadSwap1>{});
    v = o > v ? o : v;
    o = dpp_u64(v, std::integral_constant<int, kDppQuadSwap2>{});
    v = o > v ? o : v;
    o = dpp_u64(v, std::integral_constant<int, kDppRowHalfMirror>{});
    v = o > v ? o : v;
    o = dpp_u64(v, std::integral_constant<int, kDppRowMirror>{});
    v = o > v ? o : v;
    return v;
}
// Maximum of a 64-bit key over the wavefront (all lanes active).
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
    auto step = [](unsigned long long x, unsigned long long y) { return y > x ? y : x; };
    auto dpp_u64 = [](unsigned long long x, auto ctrl_tag) {
        constexpr int C = decltype(ctrl_tag)::value;
        const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)x, C, 0xF, 0xF, false);
        const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(x >> 32), C, 0xF, 0xF, false);
        return ((unsigned long long)hi << 32) | lo;
    };
    v = step(v, dpp_u64(v, std::integral_constant<int, kDppQuadSwap1>{}));
    v = step(v, dpp_u64(v, std::integral_constant<int, kDppQuadSwap2>{}));
    v = step(v, dpp_u64(v, std::integral_constant<int, kDppRowHalfMirror>{}));
    v = step(v, dpp_u64(v, std::integral_constant<int, kDppRowMirror>{}));
    auto rl = [&](int l) {
        return ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), l) << 32) |
               (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, l);
    };
    return step(step(rl(0), rl(16)), step(rl(32), rl(48)));
}

}  // namespace gh
