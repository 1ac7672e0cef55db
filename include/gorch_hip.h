/*
 * gorch_hip.h — C-ABI of the MI355X (gfx950) backend for gorch's BF16-weight
 * inference path: a sibling of gorch's metal/shim.h and accelerate/shim.h.
 *
 * Conventions (mirroring metal/shim.h):
 *   - Plain pointers and sizes only. Device pointers are HBM addresses from
 *     gorch_hip_alloc (or any allocator on the same device).
 *   - Every compute entry point takes `stream` (a hipStream_t passed as
 *     void*; NULL = the library's stream for the current device) and is
 *     asynchronous on it; gorch_hip_sync() waits for it (metal_finish /
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
 * failure. Release is idempotent for NULL (metal_release_buffer). */
void* gorch_hip_alloc(size_t bytes);
void gorch_hip_release(void* ptr);
/* Host<->device copies, ordered on `stream`; they return after the copy
 * completes (the Data() read barrier, tensor.go:318-323). */
int gorch_hip_upload(void* stream, void* dst_device, const void* src_host, size_t bytes);
int gorch_hip_download(void* stream, void* dst_host, const void* src_device, size_t bytes);
/* Waits for all work on `stream` (metal_finish / metal_sync_queue). */
int gorch_hip_sync(void* stream);
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
 * NULL (it may alias y; x must not); epilogue GORCH_HIP_EPI_*.
 * M <= 16 runs the HBM-streaming GEMV; larger M the MFMA GEMM. */
int gorch_hip_linear_bf16(void* stream, const float* x, const uint16_t* W, const float* bias,
                          const float* residual, float* y, int M, int N, int K, int epilogue);

#ifdef __cplusplus
}
#endif
#endif /* GORCH_HIP_H */
