/*
 * gorch_oracle.h — CPU restatement of gorch's BF16-weight inference path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * path and the CPU baseline that bench.py times beside it. Nothing in the
 * product (gorch_amd/, include/) links, loads or calls it.
 *
 * Every function restates one function of the reference (Go, darwin-only,
 * Apple Accelerate underneath) in plain C; the citation next to each
 * declaration names the reference file:line it follows. Floating-point
 * contraction is disabled when building (-ffp-contract=off) so each
 * statement rounds the way the Go source reads.
 *
 * Pinning (what checks each function independently of its own formula) is
 * listed in oracle/README.md and tested in tests/test_oracle_*.py.
 */
#ifndef GORCH_ORACLE_H
#define GORCH_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- A1: bf16 codec (tensor.go:85-121) ---- */
uint16_t orc_f32_to_bf16(float v);                                   /* tensor.go:85-94   */
float orc_bf16_to_f32(uint16_t h);                                   /* tensor.go:97-99   */
void orc_f32_to_bf16_slice(const float* in, uint16_t* out, int64_t n); /* tensor.go:106-112 */
void orc_bf16_to_f32_slice(const uint16_t* in, float* out, int64_t n); /* tensor.go:115-121 */

/* ---- A3-A6, A8: matmul family ----
 * C = opA(A) @ opB(B); stored A is (K,M) if transA else (M,K); stored B is
 * (N,K) if transB else (K,N). Either operand may be bf16; bf16 operands are
 * widened to a fresh f32 copy first (bf16_matmul.go:147-152, :166), then an
 * f32 sgemm runs (accelerate/shim.c:8-32). Output f32. */
void orc_sgemm(int transA, int transB, int M, int N, int K,
               const float* A, const float* B, float* C);
int orc_matmul_dt(const void* A, const void* B, float* C, int M, int N, int K,
                  int transA, int transB, int aBF16, int bBF16);        /* bf16_matmul.go:159-180 */
int orc_batched_matmul_dt(const void* A, const void* B, float* C, int M, int N, int K,
                          int batch, int transA, int transB, int aBF16, int bBF16); /* :185-212 */

/* Linear.Forward (nn/module.go:61-88): y[M,N] = x[M,K] @ W[N,K]^T + b[N].
 * wBF16 selects a bf16 weight (dtyped branch, nn/module.go:66-67). */
void orc_linear(const float* x, int M, int K, const void* W, int wBF16,
                const float* bias, int N, float* y);

/* When nonzero (the default) a bf16 weight is re-widened on every call, as
 * matMulDTGrad's fallback does; zero keeps one widened copy per weight
 * pointer (the "pre-widened" CPU comparator). */
void orc_set_widen_per_call(int on);
/* OpenMP thread count for the oracle's parallel loops (n <= 0 keeps it);
 * returns the count in effect. */
int orc_set_threads(int n);
void orc_clear_widen_cache(void);

/* ---- elementwise / row ops ---- */
void orc_add(const float* a, const float* b, float* c, int64_t n);   /* ops.go:161-179, :1012-1027 */
void orc_gelu(const float* x, float* y, int64_t n);                  /* ops.go:417-443 */
void orc_sigmoid(const float* x, float* y, int64_t n);               /* accelerate/shim.c:164-177 */
void orc_silu(const float* x, float* y, int64_t n);                  /* silu.go:45-57; shim.c:188-191 */
void orc_swiglu(const float* gate, const float* val, float* y, int64_t n); /* silu.go:94-111; shim.c:200-206 */
void orc_layernorm(const float* x, int M, int N, const float* gamma, const float* beta,
                   float eps, float* y);                              /* nn/layernorm.go:31-91 */
void orc_rmsnorm(const float* x, int M, int N, const float* gamma, float eps,
                 float* y);                                           /* nn/rmsnorm.go:39-81 */
void orc_softmax_inplace(float* data, int rows, int cols);          /* nn/attention.go:274-296 */
void orc_causal_softmax(const float* x, float* y, int rows, int cols, int qSeq,
                        float scale);                                 /* softmax_metal.go:111-141 */
void orc_embedding_lookup(const float* weight, int dim, const int* ids, int n,
                          float* out);                                /* attention_ops.go:64-77 */
void orc_rope_tables(int headDim, int maxSeq, float base, float* cosT, float* sinT); /* nn/rope.go:71-96 */
void orc_rope_apply(const float* x, float* y, int outer, int seqLen, int headDim,
                    int startPos, const float* cosT, const float* sinT, int neox,
                    float sign);                                      /* nn/rope.go:172-223 */
void orc_topk(const float* x, int B, int V, int k, float* vals, int* idx); /* index_ops.go:153-186 */
int orc_argmax(const float* logits, int n);                          /* model/generate.go:134-144 */
float orc_kth_largest(const float* data, int n, int k);             /* model/generate.go:247-262 */
/* model/generate.go:147-243 with the uniform draw r given; probs may be NULL */
int orc_sample(const float* logits, int n, float temperature, int top_k, float top_p, double r, double* probs);
/* model/qwen/generate.go:94-163 (sampleLogits, nucleus top-p) with the draw r given */
int orc_sample_nucleus(const float* logits, int n, float temperature, int top_k, float top_p, double r,
                       double* probs);
/* Philox4x32-10 uniform in [0, 1) for (seed, step, row): the device sampler's draw */
double orc_philox_uniform(uint64_t seed, uint32_t step, uint32_t row);
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* MHA.ForwardCached's attention loops (nn/attention.go:348-397) for one
 * sequence: q [newSeq, dim], K/V [posOffset + newSeq, dim]; out [newSeq, dim]. */
void orc_attention_cached(const float* q, const float* K, const float* V, float* out, int newSeq,
                          int posOffset, int heads, int headDim, int causal);

/* ---- GPT with KV cache (nn/gpt.go, nn/transformer.go, nn/attention.go, nn/kvcache.go) ----
 * Weights: Linear weights are bf16 [out,in] (or f32 when the model is built
 * with linear_bf16 = 0), biases f32, LayerNorm gamma/beta f32, embeddings f32.
 * Per-layer arrays have `layers` entries. */
typedef struct {
    int vocab, dim, heads, layers, max_seq;
    int linear_bf16;           /* 1: Linear weights are uint16 bf16, 0: f32 */
    const float* wte;          /* [vocab, dim] */
    const float* wpe;          /* [max_seq, dim] */
    const float* const* ln1_g; const float* const* ln1_b;
    const void* const* wq; const float* const* bq;
    const void* const* wk; const float* const* bk;
    const void* const* wv; const float* const* bv;
    const void* const* wo; const float* const* bo;
    const float* const* ln2_g; const float* const* ln2_b;
    const void* const* w1; const float* const* b1;   /* FFN1 [4d, d] */
    const void* const* w2; const float* const* b2;   /* FFN2 [d, 4d] */
    const float* lnf_g; const float* lnf_b;
    const void* wlm; const float* blm;               /* LM head [vocab, d] */
} orc_gpt_weights;

typedef struct orc_kvcache orc_kvcache;
orc_kvcache* orc_kvcache_new(int layers, int dim, int max_seq);    /* nn/kvcache.go:23-36 */
void orc_kvcache_free(orc_kvcache* c);
int orc_kvcache_len(const orc_kvcache* c);                           /* nn/kvcache.go:47-52 */
void orc_kvcache_reset(orc_kvcache* c);                              /* nn/kvcache.go:55-60 */
const float* orc_kvcache_keys(const orc_kvcache* c, int layer);
const float* orc_kvcache_values(const orc_kvcache* c, int layer);

/* GPT.ForwardCached (nn/gpt.go:100-121): logits [n, vocab]. Returns 0, or -1
 * when posOffset + n exceeds max_seq (the reference panics). */
int orc_gpt_forward_cached(const orc_gpt_weights* w, orc_kvcache* cache,
                           const int* ids, int n, float* logits);
/* GPT.Forward (nn/gpt.go:86-90) with MHA.Forward's batched path
 * (nn/attention.go:80-119): uncached, logits [n, vocab]. */
int orc_gpt_forward(const orc_gpt_weights* w, const int* ids, int n, float* logits);
/* generateCached, greedy (model/generate.go:94-131). Writes the full result
 * (prompt + new tokens) to out_ids (capacity n_prompt + max_new) and returns
 * its length. If step_logits is non-null, row i receives the logits that
 * chose new token i ([max_new, vocab]). If gaps is non-null, gaps[i] is the
 * top-1 minus top-2 logit of that row. stop_token >= 0 ends generation
 * when it is chosen (it is not appended). */
int orc_generate_cached(const orc_gpt_weights* w, const int* prompt, int n_prompt,
                        int max_new, int stop_token, int* out_ids, float* step_logits, float* gaps);
/* generateCached with Temperature > 0 (model/generate.go:94-131, sample at
 * :105-110): new token i of sequence `row` drawn with
 * orc_philox_uniform(seed, i, row). Returns the result length. */
int orc_generate_sampled(const orc_gpt_weights* w, const int* prompt, int n_prompt, int max_new, int stop_token,
                         float temperature, int top_k, float top_p, uint64_t seed, int row, int* out_ids);

/* ---- GQA with KV cache (nn/gqa.go:213-363) ----
 * Linear weights [out, in] (bf16 when linear_bf16, else f32), biases
 * nullable (= zero); q_norm/k_norm per-head RMSNorm gammas or NULL; RoPE
 * tables [rope_max_seq, head_dim/2] or NULL. */
typedef struct {
    int dim, num_q, num_kv, head_dim, causal, linear_bf16;
    float norm_eps;
    const void *wq, *wk, *wv, *wo;
    const float *bq, *bk, *bv, *bo;
    const float *q_norm, *k_norm;
    const float *rope_cos, *rope_sin;
    int rope_max_seq, rope_neox;
} orc_gqa_weights;
/* GQA.ForwardCached: x [new_seq, dim] -> out [new_seq, dim]; the caches
 * [>= pos_offset+new_seq, num_kv*head_dim] receive the new rows at
 * pos_offset (the reference appends; rows before pos_offset are the
 * existing cache). */
int orc_gqa_forward_cached(const orc_gqa_weights* w, float* k_cache, float* v_cache, int pos_offset,
                           const float* x, int new_seq, float* out);

/* ---- MoE (nn/moe.go:130-182) ----
 * x [M, dim]; router Linear [E, dim] (wr may be null when `logits` is given:
 * injected gate logits [M, E]); expert e: wgate[e], wup[e] [ffn, dim],
 * wdown[e] [dim, ffn] (bf16 when experts_bf16), biases f32 (nullable = 0). */
typedef struct {
    int dim, ffn, experts, top_k;
    int experts_bf16;
    const void* wr; const float* br;
    const void* const* wgate; const float* const* bgate;
    const void* const* wup;   const float* const* bup;
    const void* const* wdown; const float* const* bdown;
} orc_moe_weights;
int orc_moe_forward(const orc_moe_weights* w, const float* x, int M,
                    const float* logits, float* out,
                    int* topk_idx, float* topk_w);

#ifdef __cplusplus
}
#endif
#endif
