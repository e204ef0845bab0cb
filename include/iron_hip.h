/*
 * libiron_hip — C ABI of the MI355X (gfx950) kernels behind the IRON operator
 * API (decode/prefill path of Llama-3.2-1B).
 *
 * Conventions
 *  - Every pointer argument is a device pointer (HBM) unless stated. Tensors
 *    are dense row-major; bf16 is passed as its 16-bit pattern.
 *  - `stream` is a hipStream_t (NULL = the legacy default stream). Calls are
 *    stream-ordered and asynchronous; nothing here synchronises the host.
 *  - The library never allocates device memory. Where a kernel needs scratch
 *    the caller passes a workspace sized by the matching *_workspace_bytes().
 *  - Return value: 0 on success, IRON_EINVAL (22) for a rejected argument, or a
 *    hipError_t from the launch. iron_last_error() then describes the failure
 *    (thread-local, valid until the next failing call on that thread).
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to the atassis/IRON tree).
 */
#ifndef IRON_HIP_H
#define IRON_HIP_H

#ifdef __cplusplus
extern "C" {
#endif

#define IRON_HIP_ABI_VERSION 1

/* Error string of the last failing call on this thread. */
const char* iron_last_error(void);
int iron_abi_version(void);

/* Epilogue codes shared by GEMV and GEMM. GELU_TANH is the tanh approximation
 * of iron/operators/gemv/reference.py:69-76; GELU_SIGMOID is x*sigmoid(1.702x)
 * of iron/operators/flm/gemm/reference.py:8-31. */
enum iron_epilogue {
  IRON_EPI_NONE = 0,
  IRON_EPI_GELU_TANH = 1,
  IRON_EPI_SILU = 2,
  IRON_EPI_SIGMOID = 3,
  IRON_EPI_GELU_SIGMOID = 4
};

/* ---------------------------------------------------------------- GEMV ---- */

/* y[b] = epilogue(W[b] . x[b]) for b < batches; W (batches,M,K), x (batches,K),
 * y (batches,M), bf16, fp32 accumulation. K % 8 == 0, W and x 16-byte aligned.
 * Replaces GEMV.get_callable() -> (matrix, vector, output):
 * iron/operators/gemv/op.py:22-159 (arg spec :147-153, batches :145,
 * epilogue :33-36). */
int iron_gemv_bf16(const void* W, const void* x, void* y, int M, int K, int batches, int epilogue,
                   void* stream);

/* Decode-step GEMV with optional fusions (NULL disables each):
 *   norm_w   (K,)  : x is replaced by bf16(x * rsqrt(mean(x^2)+eps) * norm_w)
 *   W2       (M,K) : output is silu(W.x) * (W2.x)  (epilogue must be NONE)
 *   residual (M,)  : added before the final bf16 rounding (may alias y)
 * Fuses the RMSNorm -> GEMV and GEMV -> ElementwiseAdd / SiLU -> Mul steps of
 * the decode runlist iron/applications/llama_3.2_1b/llama_npu.py:459-557 and
 * the SwiGLUDecode sequence iron/operators/swiglu_decode/op.py:56-62. */
int iron_gemv_bf16_fused(const void* W, const void* W2, const void* x, void* y, int M, int K,
                         const void* norm_w, float eps, const void* residual, int epilogue, void* stream);

/* Fused int4 dequant + GEMV, group 32: codes (M,K/2) uint8 (two weights per
 * byte along K, low nibble first), scales (M,K/32) bf16, zero-point 0.
 * is_signed: nibbles are two's complement [-8,7] (else unsigned [0,15]).
 * New fused operator = Dequant (iron/operators/dequant/op.py:20-81) feeding
 * GEMV (iron/operators/gemv/op.py:22-159) without the bf16 round trip. */
int iron_gemv_i4g32(const void* codes, const void* scales, const void* x, void* y, int M, int K, int is_signed,
                    void* stream);

/* int4 counterpart of iron_gemv_bf16_fused (codes2/scales2 = SwiGLU up). */
int iron_gemv_i4g32_fused(const void* codes, const void* scales, const void* codes2, const void* scales2,
                          const void* x, void* y, int M, int K, int is_signed, const void* norm_w, float eps,
                          const void* residual, int epilogue, void* stream);

/* ------------------------------------------------------------- Dequant ---- */

/* Planar int4 -> bf16: out[n,k] = bf16_rne(q[n,k] * scales[n, k/group]),
 * bit-exact. codes (N,K/2) low nibble first. Restates the Dequant contract
 * iron/operators/dequant/reference.py:8-18 for a planar layout. */
int iron_dequant_i4(const void* codes, const void* scales, void* out, int N, int K, int group, int is_signed,
                    void* stream);

/* The reference's own payload layout: per tile, tile_size/2 code bytes then
 * tile_size/group_size bf16 scales (little-endian).
 * Replaces Dequant.get_callable() -> (payload, output):
 * iron/operators/dequant/op.py:77-81, layout dequant/reference.py:68-92. */
int iron_dequant_i4_payload(const void* payload, void* out, long long size, int tile_size, int group_size,
                            int is_signed, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* IRON_HIP_H */
