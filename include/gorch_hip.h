/*
 * gorch_hip.h — C-ABI of the MI355X (gfx950) backend for gorch's BF16-weight
 * inference path: a sibling of gorch's metal/shim.h and accelerate/shim.h.
 *
 * Conventions (mirroring metal/shim.h):
 *   - Plain pointers and sizes only. Device pointers are HBM addresses from
 *     gorch_hip_alloc (or any allocator on the same device).
 *   - Every compute entry point takes `stream` (a hipStream_t passed as
 *     void*; NULL = the current device's null stream) and is asynchronous
 *     on it unless stated; gorch_hip_sync() waits for it (metal_finish /
 *     metal_sync_queue, metal/shim.m:216-242).
 *   - Return code 0 = success. Nonzero = the call did nothing useful and the
 *     caller should take its CPU path (the reference falls back to widen +
 *     Accelerate on rc 1, bf16_matmul.go:124-129); gorch_hip_last_error()
 *     returns a thread-local message for the last failure.
 *   - bf16 tensors are uint16 storage of gorch's bf16 (tensor.go:85-99).
 *   - Row-major, contiguous. A Linear weight is [out, in] = [N, K].
 */
#ifndef GORCH_HIP_H
#define GORCH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GORCH_HIP_OK 0
#define GORCH_HIP_EUNSUPPORTED 1 /* configuration not handled: use the CPU path */
#define GORCH_HIP_EINVAL 2       /* bad argument (shape, null pointer)          */
#define GORCH_HIP_ERUNTIME 3     /* HIP runtime error                           */
#define GORCH_HIP_ENOMEM 4       /* device allocation failed                    */

/* Linear epilogues (applied after the bias add, before the residual add). */
#define GORCH_HIP_EPI_NONE 0
#define GORCH_HIP_EPI_GELU 1 /* tanh-form GELU, ops.go:417-443 */

/* ------------------------------------------------------------------------
 * Device, streams, memory — replaces metal_create_device / queue / buffer
 * (metal/shim.h:15-30, :38-51; Go side metal/metal.go:251-309, :405-422).
 * ---------------------------------------------------------------------- */

/* Selects and initialises `device` for the calling thread (InitMetal,
 * ops.go:93-131). Idempotent. */
int gorch_hip_init(int device);
/* Number of visible gfx950 devices (0 when none). */
int gorch_hip_device_count(void);
/* Thread-local message for the last nonzero return (metal_free_string
 * pattern, metal/shim.m:1018). Never NULL. */
const char* gorch_hip_last_error(void);
/* Device allocation (metal_new_buffer, metal/shim.h:38-41). NULL on
 * failure. gorch_hip_release (metal_release_buffer) ignores NULL and any
 * pointer that is not a live allocation of this library, so a repeated
 * release of the same pointer is harmless until the address is handed out
 * again; it waits for queued work first. Callers that can release from
 * several threads (an explicit Release racing a finaliser) use the buffer
 * handles below, whose release is exactly-once. */
void* gorch_hip_alloc(size_t bytes);
void gorch_hip_release(void* ptr);
/* Bytes held by live allocations and buffers (liveBufferBytes,
 * metal/metal.go:363-368). */
long long gorch_hip_live_bytes(void);
/* Device bytes the library holds for its own scratch: the per-stream
 * K-split partial buffers of gorch_hip_linear_bf16 and the engines, each
 * allocated on a stream's first split launch outside capture and kept (with
 * any it replaced when it grew: a captured graph may point at them) until
 * gorch_hip_release_stream_scratch or the process ends. No counterpart in
 * the reference (Metal's MPSGraph keeps its own scratch); it lets a caller
 * check that a call allocated nothing. */
long long gorch_hip_scratch_bytes(void);
/* No counterpart in the reference: frees the scratch the library holds for
 * `stream` (NULL = the null stream) after waiting for the stream, for a
 * caller about to destroy a stream of its own. No graph captured on that
 * stream may be launched afterwards; the next split launch on it allocates
 * again. The engines release their own streams' scratch when destroyed. */
void gorch_hip_release_stream_scratch(void* stream);

/* Buffer handles (metal.Buffer, metal/metal.go:240-422; Tensor.ToMetal /
 * Data, tensor.go:318-406). Device memory of exactly `bytes`, zero-filled;
 * with GORCH_HIP_BUF_HOST_MIRROR also a pinned host copy, the discrete-GPU
 * stand-in for Metal's unified memory: gorch_hip_buf_host is the Data()
 * read barrier (waits for `stream`, copies the device contents down if a
 * kernel may have written them since), gorch_hip_buf_device brings the
 * device copy up to date after host writes through the mirror. Pass
 * will_write = 1 when the caller (host) or the kernel it is about to queue
 * (device) writes the buffer, so the other copy is refreshed before its next
 * use. Handles are never reused: gorch_hip_buf_release is idempotent and
 * thread-safe (Buffer.Release's CompareAndSwap, metal/metal.go:405-422),
 * and the memory is freed once no call is using it. */
typedef struct gorch_hip_buf gorch_hip_buf;
#define GORCH_HIP_BUF_HOST_MIRROR 1
gorch_hip_buf* gorch_hip_buf_new(size_t bytes, int flags);
void gorch_hip_buf_release(gorch_hip_buf* buf);
size_t gorch_hip_buf_len(gorch_hip_buf* buf);
void* gorch_hip_buf_device(void* stream, gorch_hip_buf* buf, int will_write);
void* gorch_hip_buf_host(void* stream, gorch_hip_buf* buf, int will_write);
/* Host<->device copies, ordered on `stream`; they return after the copy
 * completes (the Data() read barrier, tensor.go:318-323). */
int gorch_hip_upload(void* stream, void* dst_device, const void* src_host, size_t bytes);
int gorch_hip_download(void* stream, void* dst_host, const void* src_device, size_t bytes);
/* Waits for all work on `stream` (metal_finish / metal_sync_queue). */
int gorch_hip_sync(void* stream);
/* Dispatch mode (SetMetalAsync / MetalAsyncEnabled, metal_async.go:30-38):
 * on (the default here), compute entry points return once their work is
 * queued on the stream, and the caller synchronises at read barriers
 * (gorch_hip_sync, gorch_hip_download, gorch_hip_buf_host). Off, every
 * compute entry point waits for its stream before returning (the Metal
 * shim's per-op wait). Turning it off first drains the device. */
int gorch_hip_set_async(int on);
int gorch_hip_async_enabled(void);
/* Run-to-run bit reproducibility. Off (the default), the one-row decode
 * steps of the GPT engine and of the GQA/Qwen block add the output
 * projection into the residual inside the attention kernel with float
 * atomics, one per head, whose order varies between runs (the last bits of
 * the logits can differ; greedy tokens are identical unless two logits tie
 * to that precision). On, those steps run the projection as a GEMV of its
 * own and every sum has a fixed order, as gorch's greedy loop
 * (model/generate.go:134-144). Takes effect at the next launch; a caller's
 * own captured graphs keep the kernels they captured. Returns the previous
 * setting. No counterpart in the reference, whose CPU and Metal paths have
 * no cross-block atomics. */
int gorch_hip_set_deterministic(int on);
int gorch_hip_deterministic_enabled(void);
/* The bf16 matmul self-probe (MetalBF16MatMulSupported / runBF16MatMulProbe,
 * bf16_matmul.go:52-112): a 16x16x16 bf16 x bf16 and bf16 x f32 product
 * through the matmul path against a host f32 product, every element within
 * 1e-3. It runs once per device in gorch_hip_init (or at the first bf16 call
 * on a device that was not initialised). While it has failed, every entry
 * point with bf16 weights returns GORCH_HIP_EUNSUPPORTED, the signal to take
 * the CPU path (bf16MatMulEligible, :116-119). _supported returns 1 when the
 * probe passed on the current device; gorch_hip_bf16_probe runs it again
 * and returns the new verdict. */
int gorch_hip_bf16_matmul_supported(void);
int gorch_hip_bf16_probe(void);
/* Dispatch counters (ReadMetalDispatchCounts / Reset, ops.go:49-78):
 * fills up to `n` slots in the order gemv, gemm, generic_matmul, attention,
 * norm, elementwise, moe, argmax, codec; returns the number of slots. */
int gorch_hip_read_dispatch_counts(uint64_t* out, int n);
void gorch_hip_reset_dispatch_counts(void);

/* ------------------------------------------------------------------------
 * bf16 codec on device (tensor.go:85-121; model/safetensors.go:164-184).
 * ---------------------------------------------------------------------- */
int gorch_hip_bf16_to_f32(void* stream, const uint16_t* in, float* out, int64_t n);
int gorch_hip_f32_to_bf16(void* stream, const float* in, uint16_t* out, int64_t n);

/* ------------------------------------------------------------------------
 * Matmul family.
 * ---------------------------------------------------------------------- */

/* C = opA(A) @ opB(B), C f32 [M,N], f32 accumulation. Stored A is (K,M)
 * if transA else (M,K); stored B is (N,K) if transB else (K,N); aBF16 /
 * bBF16 select bf16 storage per operand. Same arguments and semantics as
 * metal_mps_matmul_dt (metal/shim.h:122-126, metal/shim.m:900), reached
 * from matMulDTGrad / matMulBF16 (bf16_matmul.go:159-180, :217-253).
 * transA && transB returns GORCH_HIP_EUNSUPPORTED (bf16_matmul.go:176). */
int gorch_hip_matmul_dt(void* stream, const void* A, const void* B, float* C,
                        uint32_t M, uint32_t N, uint32_t K,
                        int transA, int transB, int aBF16, int bBF16);

/* Batched variant, matrices packed contiguously per operand
 * (metal_mps_batched_matmul_dt, metal/shim.h:132-137;
 * batchedMatMulDTGrad / batchedMatMulBF16, bf16_matmul.go:185-212, :257-304). */
int gorch_hip_batched_matmul_dt(void* stream, const void* A, const void* B, float* C,
                                uint32_t M, uint32_t N, uint32_t K, uint32_t batch,
                                int transA, int transB, int aBF16, int bBF16);

/* Fused bf16-weight Linear (nn/module.go:61-88 with the op that follows it):
 *   y[m,n] = residual[m,n] + epi( sum_k x[m,k] * W[n,k] + bias[n] )
 * x f32 [M,K]; W bf16 [N,K]; bias f32 [N] or NULL; residual f32 [M,N] or
 * NULL (it may alias y; x must not); epilogue GORCH_HIP_EPI_*. Needs
 * K % 8 == 0 and 16-byte aligned x and W (else GORCH_HIP_EUNSUPPORTED).
 * M <= 16 runs the HBM-streaming GEMV; larger M the tiled MFMA GEMM. Both
 * keep f32-activation accuracy (activations split into two bf16 terms). */
int gorch_hip_linear_bf16(void* stream, const float* x, const uint16_t* W, const float* bias,
                          const float* residual, float* y, int M, int N, int K, int epilogue);

/* Activations rounded to bf16 (RNE) before the matrix cores: the bf16 x bf16
 * -> f32 product of the MPSGraph dtyped path (metal/shim.m:808-857). */
#define GORCH_HIP_LINEAR_ACT_BF16 1
/* gorch_hip_linear_bf16 with flags (GORCH_HIP_LINEAR_ACT_BF16: always the
 * MFMA GEMM, one bf16 MFMA per fragment). */
int gorch_hip_linear_bf16_ex(void* stream, const float* x, const uint16_t* W, const float* bias,
                             const float* residual, float* y, int M, int N, int K, int epilogue, int flags);

/* Device-resident weight format for decode (replaces the row-major bf16
 * buffer gorch's Tensor.ToMetal uploads, tensor.go:388-406, for a weight
 * that only feeds Linear.Forward): ceil(N/16) tiles of ceil(K/32) 1 KB
 * fragments in matrix-core operand order, zero-padded; the values are the
 * weight's bf16 bits unchanged. gorch_hip_packed_bf16_bytes gives the size,
 * gorch_hip_pack_bf16 converts a row-major [N,K] device weight (K % 8 == 0,
 * 16-byte aligned buffers). */
size_t gorch_hip_packed_bf16_bytes(int N, int K);
int gorch_hip_pack_bf16(void* stream, const uint16_t* W, uint16_t* Wp, int N, int K);
/* gorch_hip_linear_bf16 (nn/module.go:61-88) over a packed weight, for
 * decode-sized M (1..16) and K <= 3072: same arguments, semantics and
 * accuracy. */
int gorch_hip_linear_bf16_packed(void* stream, const float* x, const uint16_t* Wp, const float* bias,
                                 const float* residual, float* y, int M, int N, int K, int epilogue);

/* gorch_hip_linear_bf16 that allocates nothing. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results as gorch_hip_linear_bf16; the K-split
 * partials of a narrow weight over a long K come from a fixed 1 MiB device
 * array per GPU instead of a per-stream buffer the library allocates. A call
 * whose split would need more returns GORCH_HIP_EINVAL (the routing never
 * asks for more than 8 slices x 16 rows x 2032 columns). Calls that overlap
 * on one GPU (unordered streams or threads) race on the array; calls ordered
 * on one stream do not. Needs gorch_hip_init on the device first (it looks up
 * the array's address and runs the bf16 probe, which allocates). */
int gorch_hip_linear_bf16_noalloc(void* stream, const float* x, const uint16_t* W, const float* bias,
                                  const float* residual, float* y, int M, int N, int K, int epilogue);

/* ------------------------------------------------------------------------
 * Decode-step ops (the forward halves of gorch's op layer on this path).
 * ---------------------------------------------------------------------- */

/* LayerNorm over the last dim of x [M,N] (nn/layernorm.go:31-91): mean and
 * variance accumulated in f64, y = ((x - mean) * inv) * gamma + beta. */
int gorch_hip_layernorm(void* stream, const float* x, const float* gamma, const float* beta, float* y,
                        int M, int N, float eps);
/* RMSNorm (nn/rmsnorm.go:39-81, RMSNormForwardMetal rmsnorm_metal.go:51):
 * y = x * (1/sqrt(sum(x^2)/N + eps)) * gamma, sum in f64. */
int gorch_hip_rmsnorm(void* stream, const float* x, const float* gamma, float* y, int M, int N, float eps);
/* A decoder block's residual add and the next RMSNorm in one launch
 * (model/qwen/block.go:74-76: h1 = Add(x, attn); NormFFN.Forward(h1)):
 * sum = x + b, y = RMSNorm(sum; gamma). N % 4 == 0, N <= 2048, 16-byte
 * aligned rows; y may not alias x or b. */
int gorch_hip_add_rmsnorm(void* stream, const float* x, const float* b, const float* gamma, float* sum, float* y,
                          int M, int N, float eps);
/* c = a + b (Add, ops.go:161-179; vec_add). */
int gorch_hip_add(void* stream, const float* a, const float* b, float* c, int64_t n);
/* x[m,n] += bias[n] in place (BiasAddInPlaceMetal, colreduce_metal.go:56-73). */
int gorch_hip_bias_add(void* stream, float* x, const float* bias, int M, int N);
/* tanh-form GELU (GELU, ops.go:417-443; vec_gelu). */
int gorch_hip_gelu(void* stream, const float* x, float* y, int64_t n);
/* SiLU and SwiGLU (silu.go:45-136; vec_silu / vec_swiglu). */
int gorch_hip_silu(void* stream, const float* x, float* y, int64_t n);
int gorch_hip_swiglu(void* stream, const float* gate, const float* value, float* y, int64_t n);
/* Row gather out[i,:] = weight[ids[i],:] (EmbeddingLookup, attention_ops.go:64-77);
 * ids is a device int32 array. */
int gorch_hip_embedding(void* stream, const float* weight, int dim, const int* ids, int n, float* out);
/* Attention of new query rows against a KV cache (MHA.ForwardCached's core,
 * nn/attention.go:355-397). q/out [batch*new_seq, heads*head_dim]; caches
 * [batch][max_seq][heads*head_dim] already holding the new rows at
 * positions pos_offset..pos_offset+new_seq-1. causal: query i sees keys
 * 0..pos_offset+i (else all pos_offset+new_seq keys). */
int gorch_hip_attention_cached(void* stream, const float* q, const float* k_cache, const float* v_cache,
                               float* out, int batch, int new_seq, int pos_offset, int heads, int head_dim,
                               int max_seq, int causal);
/* Staircase-causal scaled softmax (CausalSoftmax, softmax_metal.go:68-141):
 * row r sees columns 0..(r mod q_seq)+(cols-q_seq); masked entries are 0. */
int gorch_hip_causal_softmax(void* stream, const float* x, float* y, int rows, int cols, int q_seq, float scale);
/* In-place row softmax (softmaxInPlace, nn/attention.go:274-296). */
int gorch_hip_softmax_rows(void* stream, float* x, int rows, int cols);
/* Row argmax, first maximum wins (argmax, model/generate.go:134-144);
 * out: device int32 [rows]. */
int gorch_hip_argmax(void* stream, const float* logits, int rows, int n, int* out);
/* sample() (model/generate.go:147-243, kthLargest :247-262) for each of
 * `rows` rows of logits [rows, n] (device): scaled = logits / temperature;
 * with 0 < top_k < n the values below the top_k-th largest become -inf;
 * softmax in f64; with 0 < top_p < 1 the smallest positive probabilities go
 * (lowest index first among equals) until the rest sum to at most
 * 1.5 * top_p, then renormalised; the token is the first index whose
 * running sum exceeds the draw u[row] (device f64 in [0, 1); the reference
 * draws rand.Float64()), n - 1 if none. out (device int32 [rows]); probs
 * (device f64 [rows, n], may be NULL) receives the final distribution.
 * EINVAL for temperature <= 0 (the greedy argmax is gorch_hip_argmax) or
 * top_k < 0; EUNSUPPORTED for n > 262144, or top_p in (0, 1) without
 * 1 <= top_k <= 4096 (those candidates are sorted on the device). */
int gorch_hip_sample(void* stream, const float* logits, int rows, int n, float temperature, int top_k, float top_p,
                     const double* u, int* out, double* probs);
/* sampleLogits (model/qwen/generate.go:94-181): gorch_hip_sample with the
 * Qwen loop's nucleus top-p: with 0 < top_p < 1 the probabilities in
 * descending order (equal ones by ascending index: the reference's
 * sort.Slice leaves their order open), the shortest prefix whose running sum
 * reaches top_p kept and divided by its sum, every other probability 0. Same
 * arguments, draws, outputs and return codes as gorch_hip_sample. */
int gorch_hip_sample_nucleus(void* stream, const float* logits, int rows, int n, float temperature, int top_k,
                             float top_p, const double* u, int* out, double* probs);
/* No counterpart in the reference: gorch_hip_sample (nucleus = 0) or
 * gorch_hip_sample_nucleus (nucleus != 0), same arguments, results and return
 * codes, for callers that keep a workspace of
 * gorch_hip_sample_workspace_size(rows) bytes (device memory, zero when first
 * passed; every call leaves it zero): with 0 < top_k <= 4096, top_k < n and
 * n >= 8192, the top-k candidate search's two passes over each row then run
 * on many blocks per row instead of the row's one block (sampling then adds
 * ~21 instead of ~38 us to a GPT-2 small batch-1 decode step). Calls sharing
 * a workspace must not overlap. */
size_t gorch_hip_sample_workspace_size(int rows);
int gorch_hip_sample_with_workspace(void* stream, const float* logits, int rows, int n, float temperature, int top_k,
                                    float top_p, const double* u, int* out, double* probs, int nucleus,
                                    void* workspace);

/* Rotary tables (NewRoPE, nn/rope.go:71-96): cos/sin [max_seq, head_dim/2]
 * device f32, invFreq = f32(base^(-2i/hd)), theta = f64(f32(pos)*invFreq). */
int gorch_hip_rope_tables(void* stream, int head_dim, int max_seq, float base, float* cos_t, float* sin_t);
/* RoPE.Apply / RoPEApplyMetal (nn/rope.go:172-223, rope_metal.go:35-62):
 * x, y [outer, seq_len, head_dim] (may alias); row (o, s) rotated at
 * position start_pos + s; neox selects interleaved pairs; sign +1 forward,
 * -1 inverse. max_seq is the tables' row count. */
int gorch_hip_rope_apply(void* stream, const float* x, float* y, int outer, int seq_len, int head_dim,
                         int start_pos, const float* cos_t, const float* sin_t, int max_seq, int neox, float sign);

/* Grouped-query attention of new query rows against a cache (the
 * per-KV-head loops of GQA.forwardCached, nn/gqa.go:308-352): q/out
 * [batch*new_seq, num_q*head_dim]; caches [batch][max_seq][num_kv*head_dim]
 * holding the (rotated) keys and values up to pos_offset+new_seq; query head
 * h reads KV head h / (num_q/num_kv); softmax rows scaled by 1/sum. */
int gorch_hip_gqa_attention_cached(void* stream, const float* q, const float* k_cache, const float* v_cache,
                                   float* out, int batch, int new_seq, int pos_offset, int num_q, int num_kv,
                                   int head_dim, int max_seq, int causal);

/* GQA module (GQAConfig, nn/gqa.go:64-98), device pointers. Linear weights
 * bf16 [out, in]: wq [num_q*hd, dim], wk/wv [num_kv*hd, dim], wo
 * [dim, num_q*hd]; biases f32 or NULL (= zero, the Bias=false config);
 * q_norm / k_norm: per-head RMSNorm gammas [head_dim] or NULL; rope tables
 * [rope_max_seq, head_dim/2] or NULL (no RoPE). */
typedef struct {
    int dim, num_q, num_kv, head_dim, causal;
    float norm_eps;
    const uint16_t* wq; const float* bq;
    const uint16_t* wk; const float* bk;
    const uint16_t* wv; const float* bv;
    const uint16_t* wo; const float* bo;
    const float* q_norm; const float* k_norm;
    const float* rope_cos; const float* rope_sin;
    int rope_max_seq, rope_neox;
} gorch_hip_gqa_weights;
size_t gorch_hip_gqa_workspace_size(const gorch_hip_gqa_weights* w, int new_seq);
/* GQA.ForwardCached (nn/gqa.go:259-363) for one sequence: x [new_seq, dim]
 * -> out [new_seq, dim]; appends the new (rotated) K and V rows at
 * pos_offset of the caches [max_seq, num_kv*head_dim]. */
int gorch_hip_gqa_forward_cached(void* stream, const gorch_hip_gqa_weights* w, const float* x, int new_seq,
                                 float* k_cache, float* v_cache, int pos_offset, int max_seq, float* out,
                                 void* workspace, size_t workspace_bytes);

/* One Qwen decoder block (model/qwen Block, block.go:27-79; Config,
 * config.go:13-28): attn is the block's GQA (q/k/v biases for AttnBias,
 * q_norm/k_norm for UseQKNorm, the model's shared RoPE tables); norm_attn /
 * norm_ffn: RMSNorm gains [dim] (eps = RMSNormEps); wgate_up: the gate rows
 * then the up rows, one bf16 [2*inter, dim] weight; wdown [dim, inter]. The
 * one-row step fuses Q/K/V into one weight stream when wq, wk, wv (and bq,
 * bk, bv) are consecutive row ranges of one buffer. */
typedef struct {
    gorch_hip_gqa_weights attn;
    const float* norm_attn;
    const float* norm_ffn;
    const uint16_t* wgate_up;
    const uint16_t* wdown;
    int inter;
    float eps;
} gorch_hip_qwen_block;
size_t gorch_hip_qwen_block_workspace_size(const gorch_hip_qwen_block* b, int new_seq);
/* Block.ForwardCached (block.go:71-79) for one sequence, in place on x
 * [new_seq, dim]: x1 = x + GQA(RMSNorm(x)) (the new K/V rows appended at
 * pos_offset of the caches [max_seq, num_kv*head_dim]), x = x1 +
 * down(SwiGLU(gate(h), up(h))) with h = RMSNorm(x1). One-row calls run six
 * launches (norms and SwiGLU fused into the GEMVs' loads, residual adds into
 * their stores). Caller workspace, no allocation. */
int gorch_hip_qwen_block_forward_cached(void* stream, const gorch_hip_qwen_block* b, float* x, int new_seq,
                                        float* k_cache, float* v_cache, int pos_offset, int max_seq,
                                        void* workspace, size_t workspace_bytes);

/* model/qwen Model (qwen.go:12-98) for greedy generation: blocks[0 ..
 * layers) as above (copied; their device weights stay the caller's and
 * must outlive the model; every block needs RoPE tables covering max_seq),
 * embed_bf16 the tied [vocab, dim] bf16 embedding (the LM head, qwen.go:84),
 * embed_f32 its f32 widening (the lookup), norm the final RMSNorm gain.
 * The model owns its KV cache (MaxSeq rows at most, grown as needed),
 * activations and decode state. NULL on failure (gorch_hip_last_error). */
typedef struct gorch_hip_qwen gorch_hip_qwen;
gorch_hip_qwen* gorch_hip_qwen_create(const gorch_hip_qwen_block* blocks, int layers, const uint16_t* embed_bf16,
                                      const float* embed_f32, const float* norm, float eps, int vocab, int max_seq);
void gorch_hip_qwen_destroy(gorch_hip_qwen* m);
/* Generate with a greedy config (model/qwen/generate.go:35-66, Greedy
 * :24-29): a prefill over the host prompt, then one token per step; a token
 * in stop_tokens[0 .. n_stop) ends generation and is not kept; generation
 * also ends after max_new tokens, or once the cache holds max_seq rows (the
 * token chosen then is kept). out_ids (host, n_prompt + max_new ints)
 * receives the prompt and the new tokens, *out_len their count. The argmax
 * is fused into the tied head; flags bit 0 replays each step from a HIP
 * graph that reads the position from device memory (shapes whose
 * attention step cannot, and runs with step_logits, launch each step
 * directly). step_logits (nullable, host [max_new, vocab]): each chosen
 * token's logits. timing_ms (nullable, 4 floats): prefill ms, decode ms,
 * decode forwards run, 1 when the steps were graph-replayed (else 0). Stop
 * tokens are read back every 8 steps. Returns
 * EINVAL for an empty prompt ("qwen: empty prompt", the reference's panic)
 * or one longer than max_seq. Synchronous. */
int gorch_hip_qwen_generate(void* stream, gorch_hip_qwen* m, const int* prompt, int n_prompt, int max_new,
                            const int* stop_tokens, int n_stop, int* out_ids, int* out_len, float* step_logits,
                            float* timing_ms, int flags);
/* Generate with a sampling config (GenerateConfig, model/qwen/generate.go:
 * 12-20, 35-66): temperature 0 is gorch_hip_qwen_generate (top_k, top_p and
 * seed ignored); temperature > 0 chooses each token with sampleLogits
 * (:94-181; gorch_hip_sample_nucleus) over the step's logits on the device,
 * the draw of new token i being the Philox4x32-10 uniform of counter (0, i)
 * under key seed (the reference seeds math/rand; its stream is not
 * reproduced, so runs agree with it given the same draws). Other arguments
 * and outputs as gorch_hip_qwen_generate. EINVAL for a negative or
 * non-finite temperature or top_k < 0; EUNSUPPORTED for top_p in (0, 1)
 * without 1 <= top_k <= 4096, or when values tied at the top-k threshold
 * put more than 4096 candidates in the top-p sort. Synchronous. */
int gorch_hip_qwen_generate_sampled(void* stream, gorch_hip_qwen* m, const int* prompt, int n_prompt, int max_new,
                                    const int* stop_tokens, int n_stop, float temperature, int top_k, float top_p,
                                    unsigned long long seed, int* out_ids, int* out_len, float* step_logits,
                                    float* timing_ms, int flags);

/* ------------------------------------------------------------------------
 * MoE FFN layer (nn.MoE.Forward, nn/moe.go:130-182).
 * ---------------------------------------------------------------------- */

/* Device pointers. Expert weights are stacked per kind: wgate / wup
 * [experts][ffn][dim], wdown [experts][dim][ffn] (bf16, Linear layout);
 * biases [experts][out] f32 or NULL (= zero). wr / br: the router Linear
 * [experts, dim] (bf16) / [experts], or NULL when logits are injected. */
typedef struct {
    int dim, ffn, experts, top_k;
    const uint16_t* wr; const float* br;
    const uint16_t* wgate; const float* bgate;
    const uint16_t* wup; const float* bup;
    const uint16_t* wdown; const float* bdown;
} gorch_hip_moe_weights;

/* Device workspace bytes gorch_hip_moe_forward needs for M tokens. */
size_t gorch_hip_moe_workspace_size(int M, int dim, int ffn, int experts, int top_k);
/* out [M, dim] = MoE(x [M, dim]). logits: injected router logits [M, experts]
 * (device) or NULL to run the router Linear. topk_idx / topk_w (device,
 * nullable) receive the chosen experts [M, top_k] (descending logit, ties
 * to the lower index) and their softmax weights. The workspace is the
 * caller's (no allocation inside; the call is graph-capturable). Top-k is
 * limited to 8, experts to 64, and M * experts and M * top_k * dim to
 * below 2^29 (32-bit buffer offsets). */
int gorch_hip_moe_forward(void* stream, const gorch_hip_moe_weights* w, const float* x, int M,
                          const float* logits, float* out, int* topk_idx, float* topk_w,
                          void* workspace, size_t workspace_bytes);

/* ------------------------------------------------------------------------
 * GPT decode engine (nn.GPT / nn.KVCache / model.generateCached).
 * ---------------------------------------------------------------------- */

/* Host pointers to a GPT's parameters (NewGPT, nn/gpt.go:31-49): Linear
 * weights bf16 [out, in], biases / LayerNorm / embeddings f32, per-layer
 * arrays of `layers` pointers, an untied LM head. */
typedef struct {
    int vocab, dim, heads, layers, max_seq;
    const float* wte;          /* [vocab, dim] */
    const float* wpe;          /* [max_seq, dim] */
    const float* const* ln1_g; const float* const* ln1_b;
    const uint16_t* const* wq; const float* const* bq;
    const uint16_t* const* wk; const float* const* bk;
    const uint16_t* const* wv; const float* const* bv;
    const uint16_t* const* wo; const float* const* bo;
    const float* const* ln2_g; const float* const* ln2_b;
    const uint16_t* const* w1; const float* const* b1;   /* FFN1 [4d, d] */
    const uint16_t* const* w2; const float* const* b2;   /* FFN2 [d, 4d] */
    const float* lnf_g; const float* lnf_b;
    const uint16_t* wlm; const float* blm;               /* LM head [vocab, d] */
} gorch_hip_gpt_weights;

/* ------------------------------------------------------------------------
 * safetensors checkpoints (model/safetensors.go:52-184).
 * ---------------------------------------------------------------------- */

#define GORCH_HIP_ST_F32 0
#define GORCH_HIP_ST_F16 1
#define GORCH_HIP_ST_BF16 2

typedef struct gorch_hip_st gorch_hip_st;
/* Parses and validates the header (LoadSafetensors' checks: unsupported
 * dtype, offsets outside the data, byte count vs shape); tensor data is read
 * on demand. NULL on failure (gorch_hip_last_error). Host-only. */
gorch_hip_st* gorch_hip_st_open(const char* path);
void gorch_hip_st_close(gorch_hip_st* f);
/* Tensor names in sorted order (SafetensorsFile.Names). */
int gorch_hip_st_count(const gorch_hip_st* f);
const char* gorch_hip_st_name(const gorch_hip_st* f, int i);
/* dtype (GORCH_HIP_ST_*), rank, shape (up to 8 dims) and stored bytes;
 * any output may be NULL. */
int gorch_hip_st_info(const gorch_hip_st* f, const char* name, int* dtype, int* ndim, int64_t* shape,
                      int64_t* nbytes);
/* Reads one tensor into device memory `dst` as F32 (F32 copied, F16/BF16
 * widened exactly: decodeF16 / decodeBF16) or BF16 (BF16 bits kept, the
 * native loader's decodeBF16Raw; F32/F16 rounded with f32ToBF16,
 * tensor.go:85-101). transpose: a 2-D [R, C] tensor lands as [C, R] (a
 * GPT-2 Conv1D weight (in, out) as a Linear weight (out, in),
 * model/gpt2_loader.go:170-184). Synchronous. */
int gorch_hip_st_load(void* stream, const gorch_hip_st* f, const char* name, void* dst, int dst_dtype,
                      int transpose);

typedef struct gorch_hip_gpt gorch_hip_gpt;
typedef struct gorch_hip_kvcache gorch_hip_kvcache;

/* Uploads the weights to the current device (gpt.ToMetal, nn/gpt.go:241-257),
 * fusing Wq/Wk/Wv into one [3d, d] weight. NULL on failure. */
gorch_hip_gpt* gorch_hip_gpt_create(const gorch_hip_gpt_weights* w);
/* LoadGPT2 (model/gpt2_loader.go:56-133) from a Hugging Face GPT-2
 * model.safetensors straight into device memory: Conv1D weights transposed
 * on the GPU, c_attn kept as the fused [3d, d] QKV weight (its transpose;
 * the reference splits the same rows into Wq, Wk, Wv), Linear weights in
 * bf16 (BF16 files bit-exact, F32 files rounded with f32ToBF16), embeddings,
 * biases and LayerNorms in f32, the LM head tied to wte (TieLMHeadToEmbedding)
 * as its bf16 rounding with a zero bias. Tensor names with or without the
 * "transformer." prefix. A missing tensor or a size that differs from the
 * configuration fails, as in copyTensor. NULL on failure. */
gorch_hip_gpt* gorch_hip_gpt_load_gpt2(const char* path, int vocab, int dim, int heads, int layers, int max_seq);
void gorch_hip_gpt_free(gorch_hip_gpt* gpt);
/* No counterpart in the reference: frees the engine's tile-packed copies of
 * its weights (made at creation for the 2..16-row decode GEMVs when
 * dim <= 3072: about the bf16 weights' bytes again) and its captured
 * generate step. Steps of 2..16 rows then run the row-major GEMVs (same
 * results to the tested bars, slower: the GPT-2 XL shape at batch 16 and 128
 * new tokens 5,966 -> 4,887 tok/s for 3.1 GB freed); graphs a caller
 * captured before must not be launched afterwards. Returns the bytes freed
 * (0 if none). */
size_t gorch_hip_gpt_drop_packed(gorch_hip_gpt* gpt);
/* KV cache for `batch` independent sequences of up to `capacity` tokens
 * (NewKVCache, nn/kvcache.go:23-36; one reference cache per sequence). */
gorch_hip_kvcache* gorch_hip_kvcache_create(gorch_hip_gpt* gpt, int batch, int capacity);
void gorch_hip_kvcache_free(gorch_hip_kvcache* cache);
int gorch_hip_kvcache_len(const gorch_hip_kvcache* cache);   /* KVCache.Len, nn/kvcache.go:47-52 */
int gorch_hip_kvcache_reset(gorch_hip_kvcache* cache);       /* KVCache.Reset, nn/kvcache.go:55-60 */
/* Copies sequence `seq`'s cached keys/values of `layer` ([len, dim] each;
 * either may be NULL) to host memory. */
int gorch_hip_kvcache_read(const gorch_hip_kvcache* cache, int layer, int seq, float* keys, float* values);
/* GPT.ForwardCached (nn/gpt.go:100-121) for every sequence of the cache:
 * ids host int32 [batch, n]; logits (host, may be NULL) receives
 * [batch*n, vocab]. Appends n tokens to the cache; rc EINVAL when the cache
 * would exceed its capacity (the reference panics). Synchronous. */
int gorch_hip_gpt_forward_cached(void* stream, gorch_hip_gpt* gpt, gorch_hip_kvcache* cache, const int* ids,
                                 int n, float* logits);
/* Greedy generateCached (model/generate.go:94-131, Temperature 0, no stop
 * token) for `batch` prompts of n_prompt tokens (host int32 [batch, n_prompt]).
 * out_ids (host int32, capacity batch*(n_prompt+max_new)) receives each
 * sequence's (MaxSeq-truncated) prompt followed by its new tokens, row length
 * *out_len. step_logits (host, may be NULL): [max_new, batch, vocab], row i
 * = logits that chose token i (forces eager launches). timing_ms (may be
 * NULL): {prefill ms, decode ms, decode forwards}. flags bit 0: replay the
 * decode step from a HIP graph. The engine keeps the KV cache and the
 * captured step graph between calls with the same batch and cache length
 * (capture and instantiation are paid once; decode ms then measures the
 * replays only). Synchronous. */
int gorch_hip_generate_cached(void* stream, gorch_hip_gpt* gpt, const int* prompts, int batch, int n_prompt,
                              int max_new, int* out_ids, int* out_len, float* step_logits, float* timing_ms,
                              int flags);

/* GenerateConfig (model/generate.go:13-42) with UseKVCache (use_kv_cache 1,
 * else GORCH_HIP_EUNSUPPORTED). temperature 0: greedy (top_k / top_p
 * ignored, as the reference). temperature > 0: each new token from sample()
 * (model/generate.go:105-110, 147-243; gorch_hip_sample) over the step's
 * logits, for up to 16 sequences; the uniform draw for new token i of
 * sequence b is Philox4x32-10 of counter (b, i, 0, 0) under key (seed low,
 * seed high), u = ((x0 >> 5) * 2^26 + (x1 >> 6)) / 2^53 (the reference
 * draws math/rand's stream instead). stop_token -1 disables the stop.
 * flags bit 0: replay the decode step from a HIP graph. */
typedef struct {
    int max_new_tokens;
    float temperature;
    int top_k;
    float top_p;
    int stop_token;
    int use_kv_cache;
    int flags;
    unsigned long long seed;
} gorch_hip_generate_config;
/* GenerateWithConfig with UseKVCache (generateCached, model/generate.go:94-131)
 * for `batch` prompts: each sequence stops on its own at stop_token (which
 * is not kept), after max_new_tokens, or once its cache holds MaxSeq tokens.
 * out_ids (host int32 [batch, min(n_prompt, MaxSeq) + max_new_tokens])
 * receives each sequence's (truncated) prompt and new tokens, row b valid up
 * to out_lens[b]. step_logits and timing_ms as gorch_hip_generate_cached
 * (timing_ms[2] counts the decode forwards run: generation ends once every
 * sequence has stopped, checked every 8 steps). Synchronous. */
int gorch_hip_generate(void* stream, gorch_hip_gpt* gpt, const int* prompts, int batch, int n_prompt,
                       const gorch_hip_generate_config* cfg, int* out_ids, int* out_lens, float* step_logits,
                       float* timing_ms);

#ifdef __cplusplus
}
#endif
#endif /* GORCH_HIP_H */
