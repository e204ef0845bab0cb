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
 *    the caller passes a workspace sized by the matching *_workspace_bytes();
 *    only iron_gqa_decode_noalloc uses a fixed array that the library's code
 *    object holds per GPU instead.
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

/* Instrumentation: arm two hipEvent_t (created with timing enabled) for the
 * calling thread's next entry-point call: its kernels record start_event at
 * the first kernel's start and stop_event at the last kernel's end
 * (hipExtLaunchKernel), so their elapsed time is the call's device execution
 * time without the host dispatch before it -- the analogue of the per-dispatch
 * device time the reference benchmarks report (iron/common/test_utils.py:
 * 216-219). Disarmed after that call; NULL, NULL disarms. Results unchanged. */
int iron_time_next_launch(void* start_event, void* stop_event);

/* Device phase trace of the calling thread's next entry-point call: the
 * MI355X counterpart of the reference's per-design trace buffers
 * (trace_size, iron/operators/_trace.py:17-71) that
 * iron/common/tracing_utils.py:49-115 turns into Perfetto JSON and a cycles
 * summary. Kernels with trace points (iron_gqa_decode and its variants,
 * iron_gemv_i4g32 and iron_gemv_i4g32_fused on their fast path,
 * iron_swiglu_decode_i4g32, the bf16 GEMM entry points) write one 64-byte
 * record per workgroup into
 * `buffer` (device memory, 64-byte aligned, zero-filled by the caller), from
 * the workgroup's first thread, at record index = the workgroup's linear id:
 *   uint32 kernel id (1 gqa_decode, 2 gemv_i4, 3 swiglu_decode_i4, 4 gemm_bf16),
 *   uint32 workgroup, uint32 XCC_ID, uint32 HW_ID register,
 *   uint64 stamps[6]: s_memrealtime (100 MHz, one clock for every XCD) when
 *   the workgroup passed each of the kernel's trace points (0 where it did
 *   not reach one).
 * A call whose kernel needs more records than `bytes` holds is refused with
 * IRON_EINVAL before it launches; calls without trace points ignore it. The
 * trace is disarmed by that call; NULL disarms. The buffer must stay allocated
 * until that call's kernels have run (or the trace is disarmed). Outputs are
 * unchanged. */
int iron_trace_next_launch(void* buffer, long long bytes);

/* Epilogue codes shared by GEMV and GEMM. GELU_TANH is the tanh approximation
 * of iron/operators/gemv/reference.py:69-76; GELU_SIGMOID is x*sigmoid(1.702x)
 * of iron/operators/flm/gemm/reference.py:8-31. */
enum iron_epilogue {
  IRON_EPI_NONE = 0,
  IRON_EPI_GELU_TANH = 1,
  IRON_EPI_SILU = 2,
  IRON_EPI_SIGMOID = 3,
  IRON_EPI_GELU_SIGMOID = 4,
  /* OR'ed into the epilogue code of the GEMM entry points: every fp32 -> bf16
   * conversion of the output stage (before the activation and at the store)
   * truncates the mantissa -- rounds toward zero -- instead of rounding to
   * nearest even: flm.GEMM(rounding="floor"), iron/operators/flm/gemm/
   * op.py:105,426-430 and design.py:164-172. */
  IRON_EPI_ROUND_TOWARD_ZERO = 0x100
};

/* ---------------------------------------------------------------- GEMV ---- */

/* y[b] = epilogue(W[b] . x[b]) for b < batches; W (batches,M,K), x (batches,K),
 * y (batches,M), bf16, fp32 accumulation. K % 8 == 0, W and x 16-byte aligned.
 * Replaces GEMV.get_callable() -> (matrix, vector, output):
 * iron/operators/gemv/op.py:22-159 (arg spec :147-153, batches :145,
 * epilogue :33-36). */
int iron_gemv_bf16(const void* W, const void* x, void* y, int M, int K, int batches, int epilogue,
                   void* stream);

/* RMSNorm modes of the fused GEMVs. */
enum iron_norm_mode {
  IRON_NORM_NONE = 0,   /* x used as given */
  IRON_NORM_WEIGHT = 1, /* x -> bf16(x * rsqrt(mean(x^2)+eps) * norm_w), the reference order */
  IRON_NORM_SCALE = 2   /* output rows * rsqrt(mean(x^2)+eps); the norm weight is folded into
                           the matrix columns beforehand (W' = W diag(norm_w)) */
};

/* Decode-step GEMV with optional fusions (NULL disables each):
 *   norm_mode/norm_w : RMSNorm of x (enum iron_norm_mode; norm_w only for mode 1)
 *   W2 (M,K)         : output is silu(W.x) * (W2.x)  (epilogue must be NONE)
 *   residual (M,)    : added before the final bf16 rounding (may alias y)
 *   argmax_keys      : uint64 per 4 output rows (ceil(M/4) of them): the
 *                      largest (value, -row) key of those rows, for
 *                      iron_argmax_select (greedy sampling without a scan)
 * Fuses the RMSNorm -> GEMV and GEMV -> ElementwiseAdd / SiLU -> Mul steps of
 * the decode runlist iron/applications/llama_3.2_1b/llama_npu.py:459-557 and
 * the SwiGLUDecode sequence iron/operators/swiglu_decode/op.py:56-62. */
int iron_gemv_bf16_fused(const void* W, const void* W2, const void* x, void* y, int M, int K, int norm_mode,
                         const void* norm_w, float eps, const void* residual, int epilogue, void* argmax_keys,
                         void* stream);

/* Fused int4 dequant + GEMV, group 32: codes (M,K/2) uint8 (two weights per
 * byte along K, low nibble first), scales (M,K/32) bf16, zero-point 0.
 * is_signed: nibbles are two's complement [-8,7] (else unsigned [0,15]).
 * New fused operator = Dequant (iron/operators/dequant/op.py:20-81) feeding
 * GEMV (iron/operators/gemv/op.py:22-159) without the bf16 round trip. */
int iron_gemv_i4g32(const void* codes, const void* scales, const void* x, void* y, int M, int K, int is_signed,
                    void* stream);

/* Bytes of the workspace of iron_swiglu_decode_i4g32 for hidden E and FFN F
 * (-1 for shapes it does not take). */
long long iron_swiglu_decode_i4g32_workspace_bytes(int E, int F);

/* The decode SwiGLU block in ONE launch, int4 group-32 weights, E = 2048,
 * F = 8192:
 *   h = bf16(silu(Wg xn) * (Wu xn)),  y = bf16(Wd h + residual)
 * with xn as in iron_gemv_i4g32_fused's norm_mode (0 none, 1 RMSNorm with
 * norm_w, 2 outputs scaled by rsqrt(mean(x^2) + eps), norm weight folded into
 * Wg/Wu). Codes (rows, K/2) and scales (rows, K/32) as iron_gemv_i4g32;
 * residual may be NULL, and x, residual and y may alias. y is bit-identical
 * to iron_gemv_i4g32_fused(gate, up, x -> h) then iron_gemv_i4g32_fused(down,
 * h -> y, residual). The 256 workgroups run at once (refused with IRON_EINVAL
 * when the device cannot hold them) and hand h over inside the launch through
 * `workspace` (iron_swiglu_decode_i4g32_workspace_bytes, 256-byte aligned,
 * zero-filled once; its contents carry over between calls, so calls on one
 * workspace must not overlap). Waits are bounded by wait_us microseconds: on
 * timeout, or when the workspace's first 32-bit word (status) is already
 * nonzero, the call ends without writing y and leaves the status word nonzero;
 * zero-fill the workspace before calling again. Replaces the SwiGLUDecode
 * runlist iron/operators/swiglu_decode/op.py:56-62 (GEMV gate, GEMV up, SiLU,
 * ElementwiseMul, GEMV down) and the MLP half of the decode layer
 * iron/applications/llama_3.2_1b/llama_npu.py:534-550 (RMSNorm through the residual add). */
int iron_swiglu_decode_i4g32(const void* gate_codes, const void* gate_scales, const void* up_codes,
                             const void* up_scales, const void* down_codes, const void* down_scales, const void* x,
                             void* y, int E, int F, int is_signed, int norm_mode, const void* norm_w, float eps,
                             const void* residual, void* workspace, unsigned wait_us, void* stream);

/* int4 counterpart of iron_gemv_bf16_fused (codes2/scales2 = SwiGLU up). */
int iron_gemv_i4g32_fused(const void* codes, const void* scales, const void* codes2, const void* scales2,
                          const void* x, void* y, int M, int K, int is_signed, int norm_mode, const void* norm_w,
                          float eps, const void* residual, int epilogue, void* argmax_keys, void* stream);

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

/* Symmetric int4 group-32 quantiser for weight preparation: per 32 weights
 * along K, scale = bf16(max|w| / 7), q = clamp(rint(w / scale), -8, 7); writes
 * codes (N,K/2) (signed, low nibble first) and scales (N,K/32). Produces the
 * format iron_gemv_i4g32 and iron_dequant_i4 consume (no reference
 * counterpart: the reference ships pre-quantized payloads). */
int iron_quantize_i4g32(const void* W, void* codes, void* scales, int N, int K, void* stream);

/* ------------------------------------------------ Norm and elementwise ---- */

/* Row-wise RMSNorm over `cols` (cols % 8 == 0, cols <= 16384):
 *   s = x (+ residual, rounded to bf16); sum_out = s when non-NULL;
 *   out = s * rsqrt(mean(s^2) + eps) [* w]          (w NULL = unweighted)
 * fp32 math, one bf16 rounding. out may alias x; sum_out may alias x.
 * Replaces RMSNorm.get_callable() -> (input, [weight,] output):
 * iron/operators/rms_norm/op.py:19-122, reference rms_norm/reference.py:7-16;
 * with residual it also absorbs ElementwiseAdd (elementwise_add/op.py:12-24). */
int iron_rmsnorm(const void* x, const void* residual, const void* w, void* out, void* sum_out, int rows, int cols,
                 float eps, void* stream);

/* out = a + b, a * b over n bf16 (16-byte aligned). out may alias a or b.
 * Replace ElementwiseAdd / ElementwiseMul.get_callable() -> (a, b, out):
 * iron/operators/elementwise_add/op.py:12-24, elementwise_mul/op.py:12-24. */
/* iron_rmsnorm with the residual operand given as the fp32 partial sums of a
 * split-K GEMM (iron_gemm_nt_partials: `splits` ranges of rows*cols floats,
 * 16-byte aligned; 1 <= splits <= 64): residual = bf16(sum of the ranges in
 * order from 0), then s = bf16(x + residual), sum_out = s, out = norm(s) [* w]
 * as iron_rmsnorm. Bit-identical to iron_gemm_bf16_nt_splitk + iron_rmsnorm.
 * Fuses the GEMM merge into RMSNorm + ElementwiseAdd
 * (iron/operators/rms_norm/op.py:19-122, elementwise_add/op.py:12-24) for
 * the Llama prefill's o_proj and down_proj outputs (llama_npu.py:97-274). */
int iron_rmsnorm_splitk(const void* x, const float* partial, int splits, const void* w, void* out, void* sum_out,
                        int rows, int cols, float eps, void* stream);

int iron_add(const void* a, const void* b, void* out, long long n, void* stream);
int iron_mul(const void* a, const void* b, void* out, long long n, void* stream);

/* out = silu(x). Replaces SiLU.get_callable() -> (input, output):
 * iron/operators/silu/op.py:12-26. */
int iron_silu(const void* x, void* out, long long n, void* stream);

/* out = silu(gate) * up: the SiLU -> ElementwiseMul pair of
 * iron/operators/swiglu_decode/op.py:58-59 in one pass. */
int iron_silu_mul(const void* gate, const void* up, void* out, long long n, void* stream);

/* out = gelu_tanh(x) (iron/operators/gelu/reference.py semantics). */
int iron_gelu(const void* x, void* out, long long n, void* stream);

/* Row softmax over cols (cols % 8 == 0, cols <= 16384) in fp32; columns >=
 * valid_cols are masked to -inf (output 0). valid_cols_dev (device int32,
 * may be NULL) overrides valid_cols at run time (graph-capturable).
 * Replaces Softmax.get_callable() -> (input, output) with its runtime
 * vector-size mask: iron/operators/softmax/op.py:21-97, design.py:74-91. */
int iron_softmax(const void* x, void* out, int rows, int cols, int valid_cols, const int* valid_cols_dev,
                 void* stream);

/* RoPE from a packed angle table (angle_rows, cols) of interleaved [cos, sin]
 * pairs (bf16, or fp32 when angles_fp32); row r uses angle row
 * r / (rows / angle_rows). method 0 rotates the two halves, 1 interleaved
 * pairs. fp32 math, one bf16 rounding; out may alias x.
 * Replaces RoPE.get_callable() -> (input, angles, output):
 * iron/operators/rope/op.py:18-92, reference rope/reference.py:69-102. */
int iron_rope(const void* x, const void* angles, int angles_fp32, void* out, int rows, int cols, int angle_rows,
              int method, void* stream);

/* ----------------------------------------------------------- Attention ---- */

/* Bytes of workspace iron_gqa_decode needs for this shape (-1 if invalid):
 * one arrival counter per KV head (a 128-byte line each), then the per-chunk
 * partial results. iron_gqa_decode needs no initialisation (it zeroes the
 * counters itself before each call); iron_gqa_decode_ex with
 * IRON_GQA_COUNTERS_ZERO skips that and relies on the caller instead: zero-fill
 * the workspace once and let nothing but these calls write to it (every call
 * leaves the counters at zero). Calls that share one workspace must be
 * stream-ordered. */
long long iron_gqa_decode_workspace_bytes(int n_heads, int n_kv_heads, int head_dim, int max_len);

/* Positions per attention chunk (64 or 128) that iron_gqa_decode and its
 * variants take for this shape at position (or hint) pos on this stream's
 * device; -1 if the shape is invalid. The shape of a launch depends on the
 * position, so a caller that captures decode steps into graphs with a device
 * position captures one graph per shape and replays the one this returns for
 * the position at hand. No reference counterpart: it describes a launch.
 * This form answers for calls without IRON_GQA_KV_RESIDENT; the _ex form takes
 * the flags word of iron_gqa_decode_ex (the switch to 128-position chunks
 * comes earlier for resident caches). */
int iron_gqa_decode_chunk_positions(int n_heads, int n_kv_heads, int head_dim, int max_len, int pos, void* stream);
int iron_gqa_decode_chunk_positions_ex(int n_heads, int n_kv_heads, int head_dim, int max_len, int pos, int flags,
                                       void* stream);

/* One GQA decode step (head_dim 64, group n_heads/n_kv_heads in {1,2,4,8}).
 * With n_kv_heads a multiple of 8, on a device whose workgroups with ids
 * congruent mod 8 run on one XCD (iron_xcd_round_robin), it is one kernel
 * launch after a one-wave counter reset (each KV head's chunks run on one
 * XCD, and the last of them to finish merges them there; chunks of 64
 * positions, or of 128 once the active 128-position chunks of all KV heads
 * reach the device's CU count, or half of it with IRON_GQA_KV_RESIDENT:
 * iron_gqa_decode_chunk_positions_ex); otherwise
 * 64-position chunk partials, then a merge kernel:
 *   q' = rope(q, pos), k' = rope(k_new, pos)   (two halves; angles fp32
 *                                               (angle_rows, 64) [cos,sin])
 *   k_cache[:, pos] = k', v_cache[:, pos] = v_new
 *   out[h] = softmax(scale * q'[h] . K[h/G, 0..pos]) V[h/G, 0..pos]  (fp32)
 * q (H,64), k_new/v_new (Hkv,64), caches (Hkv,max_len,64), out (H,64) bf16.
 * pos_dev (device int32, may be NULL) overrides pos at run time; pos is then
 * a hint of the position the call will see (-1: none, taken as max_len - 1),
 * used only to choose the launch shape: every value gives a correct result.
 * A device position outside [0, min(max_len, angle_rows)) cannot be refused
 * before the launch: the call then changes nothing (out, the caches and the
 * workspace's counters keep their contents).
 * Replaces the decode attention runlist (RoPE, StridedCopy, Repeat, GEMV
 * scores, scale Mul, masked Softmax, Transpose, GEMV context) of
 * iron/applications/llama_3.2_1b/llama_npu.py:486-523 and the CPU golden
 * llama_cpu.py:49-148. */
int iron_gqa_decode(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                    const float* angles, int angle_rows, void* out, void* workspace, int n_heads, int n_kv_heads,
                    int head_dim, int max_len, int pos, const int* pos_dev, float scale, void* stream);

/* iron_gqa_decode with flags. IRON_GQA_KV_RESIDENT: the caches stay resident
 * between calls (a decode loop over all layers of a model whose caches fit the
 * 256 MB Infinity Cache), so the K/V reads are ordinary, allocating loads;
 * without it (iron_gqa_decode) they are streaming loads, which are faster when
 * the caches come from HBM on every call. IRON_GQA_COUNTERS_ZERO: the caller
 * keeps the workspace's arrival counters at zero (see
 * iron_gqa_decode_workspace_bytes), so the call skips resetting them (one
 * kernel launch fewer). Results are identical either way; unknown flag bits
 * are rejected (IRON_EINVAL) before anything runs. Same reference interface as
 * iron_gqa_decode (llama_npu.py:486-523). */
#define IRON_GQA_KV_RESIDENT 1
#define IRON_GQA_COUNTERS_ZERO 2
int iron_gqa_decode_ex(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                       const float* angles, int angle_rows, void* out, void* workspace, int n_heads, int n_kv_heads,
                       int head_dim, int max_len, int pos, const int* pos_dev, float scale, int flags, void* stream);

/* iron_gqa_decode without a workspace argument: the counters and partials go
 * to a scratch array the library holds in device memory, one per GPU, for the life of the
 * process (iron_gqa_decode_noalloc_max_bytes(), 4 MiB: at the Llama-3.2-1B
 * shape, 32/8 heads, up to max_len 29056). It allocates nothing, so callers
 * that cannot allocate device memory (code under hipGraph capture, tight
 * serving loops, harnesses that forbid hipMalloc) can use it. Shapes whose
 * iron_gqa_decode_workspace_bytes() exceed the maximum are rejected
 * (IRON_EINVAL) before anything runs. Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) corrupt
 * each other's counters and partials (a call's counter reset can land in the
 * middle of another call); stream-ordered calls are safe, and each first
 * zeroes the array's arrival counters (a one-wave kernel), so nothing carries
 * over from an earlier call. The array's device address is looked up
 * (hipGetSymbolAddress) by the first call on a device or by
 * iron_gqa_decode_noalloc_max_bytes(): make one of them before capturing this
 * call into a hipGraph. Same results as iron_gqa_decode.
 * No counterpart in the reference: it exists for the callers above. */
long long iron_gqa_decode_noalloc_max_bytes(void);
int iron_gqa_decode_noalloc(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                            const float* angles, int angle_rows, void* out, int n_heads, int n_kv_heads, int head_dim,
                            int max_len, int pos, const int* pos_dev, float scale, void* stream);

/* Flash attention over strided Q (H,Sq,64), K/V (Hkv,Skv,64), out (H,Sq,64)
 * (element strides per head and per row; rows 16-byte aligned). Query row i
 * sits at position q_offset+i; with causal it sees keys <= that position.
 * fp32 online softmax. Rows [Sq, out_rows) of out are written as zeros (the
 * MHA operator's padded layout); pass out_rows <= Sq for none. K/V rows are
 * addressed by 32-bit byte offsets from each head's base: seq_kv *
 * kv_row_stride * 2 must stay below 2 GiB. Replaces MHA.get_callable() -> (Q, K, V, O):
 * iron/operators/mha/op.py:21-135, golden mha/reference.py:27-94, and the
 * CPU prefill attention of llama_npu.py:948-990. */
int iron_attention_prefill(const void* q, const void* k, const void* v, void* out, int n_heads, int n_kv_heads,
                           int seq_q, int seq_kv, int head_dim, long long q_head_stride, long long q_row_stride,
                           long long kv_head_stride, long long kv_row_stride, long long o_head_stride,
                           long long o_row_stride, int out_rows, int causal, int q_offset, float scale,
                           void* stream);

/* ---------------------------------------------------------------- GEMM ---- */

/* C = clamp(act(bf16(A . B^T))) on bf16 MFMA, fp32 accumulation:
 * A (M,K), B (N,K) both K-contiguous (K % 64 == 0, K <= 2^21, 16-byte
 * aligned), C (M,N) with row stride ldc. epilogue: enum iron_epilogue (applied after the bf16
 * rounding of the accumulator); has_clamp clamps to [clamp_lo, clamp_hi].
 * Replaces GEMM.get_callable() -> (A, B, C) of iron/operators/gemm/op.py:21-231
 * (b_col_maj=True; other layouts via iron_transpose_bf16 / operand swap) and
 * flm.GEMM of iron/operators/flm/gemm/op.py:64-499 (epilogue + clamp, B packed
 * to (N,K) by pack_B). */
int iron_gemm_bf16_nt(const void* A, const void* B, void* C, int M, int N, int K, long long ldc, int epilogue,
                      int has_clamp, float clamp_lo, float clamp_hi, void* stream);

/* Split-K form of iron_gemm_bf16_nt for shapes whose 128x128 output tiles
 * cannot fill the GPU (prefill projections at short prompts): the K range is
 * cut into `splits` equal parts (splits must divide K/64), each writes fp32
 * partial sums to `workspace` (splits*M*N*4 bytes, 16-byte aligned), and a
 * second kernel sums them in order and applies the same bf16 rounding,
 * epilogue and clamp. Deterministic. iron_gemm_splitk_choose returns the
 * split count this library uses for (M, N, K) with bf16 B (1: no split: the
 * plain kernel's smaller tiles are faster unless K is long);
 * iron_gemm_splitk_workspace_bytes the workspace it needs. */
int iron_gemm_splitk_choose(int M, int N, int K);
long long iron_gemm_splitk_workspace_bytes(int M, int N, int splits);
int iron_gemm_bf16_nt_splitk(const void* A, const void* B, void* C, int M, int N, int K, long long ldc, int epilogue,
                             int has_clamp, float clamp_lo, float clamp_hi, int splits, void* workspace,
                             long long workspace_bytes, void* stream);

/* Fused SwiGLU projection for prefill: H (M, F) = bf16(silu(G) * U) with
 * G = bf16(A . Wg^T), U = bf16(A . Wu^T), one GEMM over Bgu (2F, K) whose rows
 * alternate 64-row blocks of Wg and Wu (rows 128p..128p+63 = Wg rows
 * 64p..64p+63, the next 64 = Wu rows 64p..). F % 64 == 0, K % 64 == 0, H row
 * stride ldh. Bit-identical to two iron_gemm_bf16_nt calls + iron_silu_mul,
 * without writing G and U. Replaces the gate/up GEMMs + SiLU + ElementwiseMul
 * steps of SwiGLUPrefill (iron/operators/swiglu_prefill/op.py:13-115) and of
 * the Llama prefill (llama_npu.py:97-274). */
int iron_gemm_bf16_nt_swiglu(const void* A, const void* Bgu, void* H, int M, int F, int K, long long ldh,
                             void* stream);

/* iron_gemm_bf16_nt with B given as int4-g32 weights and dequantized in the
 * kernel's prologue (no bf16 copy of the weights): B[n][k] = bf16(q * s) with
 * q the nibble of byte codes[n][k/2] (low nibble = even k; two's complement
 * [-8, 7] when is_signed, else [0, 15]) and s = scales[n][k/32] (bf16); the
 * dequantized values are bit-exact, and C is bit-identical to
 * iron_gemm_bf16_nt on them. codes (N, K/2) 16-byte aligned, scales
 * (N, K/32) 4-byte aligned, K % 64 == 0. splits > 1 splits K as
 * iron_gemm_bf16_nt_splitk does (workspace of splits*M*N*4 bytes; unused
 * when splits == 1); iron_gemm_i4g32_splitk_choose returns the split count
 * this library uses for (M, N, K) with int4-g32 B (its tiles are 128x128 or
 * larger, so it splits shorter K than the bf16 policy). No reference
 * counterpart as one operator: it is
 * Dequant (iron/operators/dequant/op.py:20-81) feeding flm.GEMM / GEMM
 * (iron/operators/flm/gemm/op.py:64-499, iron/operators/gemm/op.py:21-231)
 * without the bf16 round trip through memory. */
int iron_gemm_i4g32_nt(const void* A, const void* codes, const void* scales, void* C, int M, int N, int K,
                       long long ldc, int epilogue, int has_clamp, float clamp_lo, float clamp_hi, int is_signed,
                       int splits, void* workspace, long long workspace_bytes, void* stream);
int iron_gemm_i4g32_splitk_choose(int M, int N, int K);

/* First pass of the split-K GEMMs alone, for a consumer that merges the
 * partial sums itself (iron_rmsnorm_splitk, iron_qkv_rope_scatter_splitk):
 * workspace (splits, M, N) fp32 receives A . B^T over each of `splits` equal
 * K ranges (splits >= 1 divides K/64; splits*M*N*4 bytes, 16-byte aligned),
 * with no merge, rounding or epilogue. B is bf16 (N, K) when codes is null,
 * else the int4-g32 weights (codes, scales, is_signed) of iron_gemm_i4g32_nt;
 * exactly one of B and codes is given. The consumers merge the ranges in order
 * with the bf16 rounding of iron_gemm_bf16_nt_splitk, so every result is
 * bit-identical to that GEMM followed by the consumer's plain form. Same
 * reference operators as iron_gemm_bf16_nt / iron_gemm_i4g32_nt; it removes
 * the merge pass (one launch and an M*N bf16 round trip) from the Llama
 * prefill (llama_npu.py:97-274). */
int iron_gemm_nt_partials(const void* A, const void* B, const void* codes, const void* scales, int is_signed,
                          int M, int N, int K, int splits, void* workspace, long long workspace_bytes, void* stream);

/* out (cols, rows) = in (rows, cols)^T, bf16. Layout glue for GEMM's
 * row-major B (the role of iron/operators/transpose/op.py:18-120). */
int iron_transpose_bf16(const void* in, void* out, int rows, int cols, void* stream);

/* ------------------------------------------------------ data movement ---- */

/* out[b] (cols, rows) = in[b] (rows, cols)^T for b < batches (matrices back
 * to back), bf16. Replaces Transpose.get_callable() -> (in, out) of
 * iron/operators/transpose/op.py:16-120 (num_batches). */
int iron_transpose_batched_bf16(const void* in, void* out, int rows, int cols, int batches, void* stream);

/* Repeat-interleave of rows: out row r*repeat+k = x row r (k < repeat), rows of
 * row_bytes bytes (any element type). Replaces Repeat.get_callable() ->
 * (in, out) of iron/operators/repeat/op.py:15-70. */
int iron_repeat_rows(const void* x, void* out, long long rows, long long row_bytes, int repeat, void* stream);

/* Strided copy: out[dst(k)] = in[src(k)] for every element k of two 1-4 D
 * access patterns (sizes, strides, offset, in elements of elem_bytes bytes),
 * split over `channels` along each pattern's last dimension of size >= 1 as
 * the reference splits them (strided_copy/reference.py:9-75). Elements of out
 * outside the output pattern are left as they were. in_addend_dev /
 * out_addend_dev (optional device int32) add a run-time element offset (the
 * *_offset_parameter of a sequence); without them the host checks the
 * patterns against in_len / out_len (elements), with them the kernel skips
 * out-of-range elements. Replaces StridedCopy.get_callable() -> (in, out) of
 * iron/operators/strided_copy/op.py:15-110. */
int iron_strided_copy(const void* in, void* out, int elem_bytes, long long in_len, long long out_len, int ndim_in,
                      const long long* in_sizes, const long long* in_strides, long long in_offset,
                      const int* in_addend_dev, int ndim_out, const long long* out_sizes,
                      const long long* out_strides, long long out_offset, const int* out_addend_dev, int channels,
                      void* stream);

/* --------------------------------------------------------- Llama glue ---- */

/* out[i] = table[ids[i]] (rows of dim bf16; zeros for ids outside [0,vocab)).
 * ids is a device int32 array, so a captured decode graph reads the token it
 * produced. Replaces the host-side embedding of
 * iron/applications/llama_3.2_1b/llama_npu.py:1171-1184. */
int iron_embedding(const void* table, const int* ids, void* out, int n, int dim, int vocab, void* stream);

/* Greedy argmax over n bf16 logits (first index on ties) -> token_out[0].
 * When pos (device int32) is given: history[*pos] = token if *pos <
 * history_cap (history may be NULL), then *pos += 1. Keeps the greedy decode
 * loop on the GPU (the harness samples on the CPU:
 * iron/applications/llama_3.2_1b/llama_inference_harness.py:146-169). */
int iron_argmax_bf16(const void* x, int n, int* token_out, int* pos, int* history, int history_cap, void* stream);

/* Greedy selection from GEMV argmax keys (iron_gemv_*_fused argmax_keys):
 * token_out[0] = row of the largest key; when pos is given, history[*pos] =
 * token (if *pos < history_cap) and *pos += 1; when table is given, x_out =
 * table[token] (dim bf16). One workgroup; replaces the full-vocabulary scan of
 * iron_argmax_bf16 in the decode loop and fuses the next token's embedding. */
int iron_argmax_select(const void* keys, int n_keys, const void* table, int dim, int vocab, void* x_out,
                       int* token_out, int* pos, int* history, int history_cap, void* stream);

/* Prefill scatter: qkv (seq, (H+2Hkv)*64) -> q_out (seq, H*64) rotated,
 * k_cache[:, pos0+s] rotated, v_cache[:, pos0+s] = v (two-halves RoPE with
 * row pos0+s of the fp32 [cos,sin] table; bf16 rounding). Replaces the
 * prefill RoPE + KV copy steps of llama_npu.py:881-947. */
int iron_qkv_rope_scatter(const void* qkv, const float* angles, int angle_rows, void* q_out, void* k_cache,
                          void* v_cache, int seq, int n_heads, int n_kv_heads, int head_dim, int max_len, int pos0,
                          void* stream);

/* iron_qkv_rope_scatter with qkv given as the fp32 partial sums of a split-K
 * GEMM (iron_gemm_nt_partials: `splits` ranges of seq*(H+2Hkv)*64 floats;
 * 1 <= splits <= 64), each element merged as the GEMM's own merge (ranges in
 * order from 0, one bf16 rounding) before the rotation. Bit-identical to
 * iron_gemm_bf16_nt_splitk + iron_qkv_rope_scatter. Same reference steps as
 * iron_qkv_rope_scatter, with the GEMM merge folded in. */
int iron_qkv_rope_scatter_splitk(const float* partial, int splits, const float* angles, int angle_rows, void* q_out,
                                 void* k_cache, void* v_cache, int seq, int n_heads, int n_kv_heads, int head_dim,
                                 int max_len, int pos0, void* stream);

/* 1 when the current device dispatches workgroups whose linear ids agree
 * mod 8 to one XCD (the one-launch merges of iron_gqa_decode and
 * iron_llama_decode_fused rely on it), 0 when it does not or when it cannot
 * be checked now: the first call per device launches a 64-workgroup probe on
 * `stream` and reads its result back, which is not done while `stream` is
 * being captured. The answer is cached per device. No reference counterpart
 * (a property of this GPU that the attention merge needs). */
int iron_xcd_round_robin(void* stream);

/* ------------------------------------------ One-launch decode step ---- */

/* Per-layer device pointers of the one-launch decode step (a device array of
 * n_layers of these): int4-group-32 signed codes (N, K/2) and bf16 scales
 * (N, K/32) of qkv (3072 x 2048, input_layernorm folded in), o (2048 x 2048),
 * gate and up (8192 x 2048, post_attention_layernorm folded in), down
 * (2048 x 8192), and the layer's K/V caches (8, max_len, 64) bf16. */
typedef struct IronDecodeLayer {
  const void* qkv_codes;
  const void* qkv_scales;
  const void* o_codes;
  const void* o_scales;
  const void* gate_codes;
  const void* gate_scales;
  const void* up_codes;
  const void* up_scales;
  const void* down_codes;
  const void* down_scales;
  void* k_cache;
  void* v_cache;
} IronDecodeLayer;

/* Bytes of the exchange area of iron_llama_decode_fused for n_layers (-1 if
 * invalid). */
long long iron_llama_decode_fused_exchange_bytes(int n_layers);

/* One decode step of a Llama-3.2-1B-shaped model (hidden 2048, 32 query / 8
 * KV heads of 64, FFN 8192, int4-g32 linears) in ONE launch, up to the final
 * hidden state: the token selection of iron_argmax_select (keys of the
 * previous head; token, history[*pos], *pos += 1, embedding), then per layer
 * the qkv GEMV (rms scale), the GQA attention of iron_gqa_decode_ex (RoPE,
 * cache append at the new position), o_proj + residual, the SwiGLU pair and
 * down + residual; x_out (2048 bf16) receives the last layer's output.
 * Results are bit-identical to those 82 separate launches while their
 * attention splits the cache into 64-position chunks, as this step always does
 * (max_len / 128 x 8 below the CU count: max_len < 4096 on MI355X); on longer
 * caches the separate attention uses 128-position chunks and the two agree to
 * fp32 rounding of the merge. Stages hand their
 * vectors over inside the launch through `exchange`
 * (iron_llama_decode_fused_exchange_bytes, 256-byte aligned, zero-filled once;
 * contents carry over between calls) tagged with *epoch, which must be
 * nonzero and must change between calls: iron_llama_decode_head advances it.
 * attn_workspace: iron_gqa_decode_workspace_bytes(32, 8, 64, max_len), its
 * counters zero (the kernel leaves them at zero). max_len: a multiple of 64.
 * Every wait inside the launch is bounded by wait_us microseconds: on
 * timeout the launch still ends and *status (device word, zero before the
 * call) becomes nonzero (bits: 1 layer input, 2 position, 4 q/k/v, 8
 * attention output, 16 o_proj output, 32 h); a nonzero
 * *status also makes every later wait give up at once. flags:
 * IRON_GQA_KV_RESIDENT. The launch is a persistent grid of 1024 workgroups
 * that wait for each other: it is refused (IRON_EINVAL) unless the device
 * holds all of them at once (4 per CU on 256 CUs) and iron_xcd_round_robin()
 * holds. Replaces the single fused decode dispatch of
 * iron/applications/llama_3.2_1b/llama_npu.py:459-584 (its runlist minus
 * the LM head). */
int iron_llama_decode_fused(const IronDecodeLayer* layers, int n_layers, const void* keys, int n_keys,
                            const void* embed, int vocab, int* token, int* pos, int* history, int history_cap,
                            const float* angles, int angle_rows, int max_len, float scale, float eps,
                            void* attn_workspace, void* exchange, void* x_out, const unsigned* epoch,
                            unsigned* status, unsigned wait_us, int flags, void* stream);

/* The LM head that ends a one-launch decode step: logits = W' x *
 * rsqrt(mean(x^2) + eps) with argmax keys (iron_gemv_bf16_fused with W, or
 * iron_gemv_i4g32_fused with signed codes/scales, norm_mode 2), and *epoch
 * advanced by one (0 skipped) for the next step's exchange tags. Same
 * reference step as those two (llama_npu.py:559-584). */
int iron_llama_decode_head(const void* W, const void* codes, const void* scales, const void* x, void* logits, int M,
                           int K, float eps, void* argmax_keys, unsigned* epoch, void* stream);

/* -------------------------------------------------- Measurement probes ---- */
/* No counterpart in the reference: they measure the floors that bound the
 * short decode kernels (bench.py --mode floor). */

/* An empty kernel of `workgroups` x 256 threads: the cost of one launch. */
int iron_probe_empty(int workgroups, void* stream);

/* Workgroups iron_probe_read launches for this size (-1 if invalid). */
long long iron_probe_read_workgroups(long long nbytes, int loads_per_lane);

/* Reads nbytes (a multiple of 16, src 16-byte aligned) with 16-byte
 * nontemporal loads, loads_per_lane in {1,2,4,8} in flight per lane, and
 * writes one XOR word per workgroup to sink (sink_words >= the count above):
 * the cost of streaming that many bytes in one launch. */
int iron_probe_read(const void* src, long long nbytes, void* sink, long long sink_words, int loads_per_lane,
                    void* stream);

/* MFMA-only loop: every wave of workgroups x waves_per_workgroup issues
 * mfma_per_wave v_mfma_f32_32x32x16_bf16 over `chains` (1,2,4,8) independent
 * accumulators, register operands only. Per wave w: sink[w] (float) = sum of
 * the accumulators, clocks[4w..4w+3] (uint64) = shader clock (s_memtime)
 * before, after, 100 MHz real-time counter (s_memrealtime) before, after.
 * sink and clocks hold waves_capacity waves. */
int iron_probe_mfma(int workgroups, int waves_per_workgroup, int mfma_per_wave, int chains, void* sink, void* clocks,
                    long long waves_capacity, void* stream);

/* XCD of each workgroup of a launch of `workgroups` x 256 threads (the
 * hardware register XCC_ID, one int per workgroup into ids). The one-launch
 * GQA decode relies on workgroups whose linear ids agree mod 8 sharing an
 * XCD; this shows it on the device at hand. */
int iron_probe_xcc_ids(int workgroups, void* ids, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* IRON_HIP_H */
