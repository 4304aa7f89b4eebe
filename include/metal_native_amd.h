/* C ABI of the MI355X (gfx950) quantized-linear library, libmetal_native_amd.so.
 *
 * Drop-in for MetalNative's quantized-weight linear path.  Every entry point
 * takes plain device pointers, sizes and a HIP stream (as void*; NULL = the
 * null stream), launches asynchronously on that stream and returns a status
 * code.  The status codes keep the numbering of the reference's
 * MetalNativeError (include/metal_native/core/error.h:21-31).  On failure a
 * message is available from mq_last_error() (thread-local), mirroring the
 * MNException text the reference throws (src/ops/matmul.mm:910-934).
 *
 * Storage formats (the reference's, unchanged):
 *   int4 weights   uint8 [N, K/2]: byte j of row n holds k=2j in the low nibble
 *                  and k=2j+1 in the high nibble
 *                  (shaders/matmul_dequant_kernel.metal:37-38,129-139)
 *   int8 weights   int8 [N, K]
 *   scales, zeros  fp16 [N, ceil(K/group_size)], row-major
 *   activations    fp16 [M, K];  output fp16 [M, N] (N/2 columns for SwiGLU)
 * Dequant: w = half(q-8)*s - z (int4), half(q)*s - z (int8), two fp16 roundings
 * (shaders/matmul_dequant_kernel.metal:42-43,47-49).
 */
#ifndef METAL_NATIVE_AMD_H
#define METAL_NATIVE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MQ_API __attribute__((visibility("default")))

/* include/metal_native/core/error.h:21-31 (MetalNativeError) */
enum mq_status {
  MQ_SUCCESS = 0,
  MQ_DEVICE_NOT_FOUND = 1,
  MQ_ALLOCATION_FAILED = 2,
  MQ_KERNEL_COMPILATION_FAILED = 3,
  MQ_INVALID_ARGUMENT = 4,
  MQ_OUT_OF_MEMORY = 5,
  MQ_TIMEOUT_ERROR = 6,
  MQ_INTERNAL_ERROR = 7,
  MQ_NOT_IMPLEMENTED = 8
};

/* include/metal_native/ops/matmul.h:60-63 (QuantType) */
enum mq_quant_type { MQ_QUANT_INT4 = 0, MQ_QUANT_INT8 = 1 };

/* Epilogue applied to the fp32 accumulator before the one fp16 store, numbered
 * like the reference's MatmulEpilogue (include/metal_native/ops/fused_matmul.h:18-24,
 * shaders/matmul_fused_epilogue.metal:97-124):
 *   BIAS       half(acc + float(bias[n]))
 *   BIAS_RELU  half(max(acc + float(bias[n]), 0))
 *   BIAS_SILU  half(v / (1 + exp(-v))), v = acc + float(bias[n])
 *   RESIDUAL   half(acc + float(residual[m * ldr + n]))
 * plus SWIGLU (no MatmulEpilogue counterpart): weight rows [0,N/2) are gate,
 *   [N/2,N) up; output [M, N/2] = half(silu(float(half(gate))) *
 *   float(half(up))), i.e. the reference's dequant_matmul followed by
 *   fast::swiglu (shaders/fused_swiglu.metal:48-84) in one kernel. */
enum mq_epilogue {
  MQ_EPILOGUE_NONE = 0,
  MQ_EPILOGUE_BIAS = 1,
  MQ_EPILOGUE_BIAS_RELU = 2,
  MQ_EPILOGUE_BIAS_SILU = 3,
  MQ_EPILOGUE_RESIDUAL = 4,
  MQ_EPILOGUE_SWIGLU = 5
};

/* Fused dequantize + matmul: out = epi(A . deq(W)^T).
 * Replaces metal_native::dequant_matmul (include/metal_native/ops/matmul.h:77-82,
 * src/ops/matmul.mm:903-1029; bound as _C.dequant_matmul at
 * bindings/bind_ops.cpp:366-382), with the fused epilogues of
 * metal_native::fused_matmul (src/ops/fused_matmul.mm:132-199).  Strides are
 * in elements for A/out/residual and in bytes for the weights (ldw_bytes;
 * K/2 for packed int4 rows, K for int8).  zeros may be NULL (no zero term);
 * bias is read only by the bias epilogues, residual (fp16 [M, N], row stride
 * ldr >= N) only by MQ_EPILOGUE_RESIDUAL; the residual may be the output
 * itself when ldr == ldc (each element is read and then written by one
 * thread).  The kernels that split K across workgroups (the split-K GEMV,
 * the row-block GEMV when the activations exceed LDS, and the prefill GEMM
 * where its output tiles would leave most CUs idle) keep their partial sums
 * and counters in a library workspace per (device, stream), allocated by the
 * first call on that stream that needs it (so that call must not be inside
 * stream capture; under capture the prefill GEMM then keeps one workgroup per
 * tile instead).  Calls on one stream are ordered and share it.  When a
 * larger shape needs more, a new workspace replaces it for later calls; the
 * old one is kept (not freed) until the process ends, so graphs captured
 * earlier on that stream stay valid. */
MQ_API int mq_dequant_matmul(const void* activations, int64_t lda, const void* weights_packed,
                             int64_t ldw_bytes, const void* scales, const void* zeros, void* out,
                             int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t group_size,
                             int32_t quant_type, int32_t epilogue, const void* bias, const void* residual,
                             int64_t ldr, void* stream);

/* mq_dequant_matmul that allocates nothing: no reference counterpart; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * contract and kernels as mq_dequant_matmul; where the split-K decode GEMV
 * runs, its counters and partial sums live in a fixed 8 MiB device array of
 * the library (one per GPU, held until the process ends) instead of the
 * per-stream workspace; the prefill GEMM keeps one workgroup per output tile
 * (no K split) here.  A shape whose split-K partials need more than that
 * returns MQ_INVALID_ARGUMENT with the sizes in mq_last_error().  The first
 * call on a device clears the array's counters with a kernel on the given
 * stream; every call leaves them zero.  Calls that overlap on one GPU share
 * the array and race: keep them stream-ordered. */
MQ_API int mq_dequant_matmul_noalloc(const void* activations, int64_t lda, const void* weights_packed,
                                     int64_t ldw_bytes, const void* scales, const void* zeros, void* out,
                                     int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t group_size,
                                     int32_t quant_type, int32_t epilogue, const void* bias, const void* residual,
                                     int64_t ldr, void* stream);

/* Dequantize to fp16 out[N, K] (row stride ldo elements).
 * flat_groups == 0: per-row groups scales[n, k/g], optional zeros (NULL = no
 *   zero term) -- the fused kernels' dequant (matmul_dequant_kernel.metal:128-162).
 * flat_groups != 0: the standalone kernels' semantics, group index i/g over the
 *   flattened element index and no zero term (shaders/dequantize_kernel.metal:9-163,
 *   dispatched by QuantWeightCache::get_dequantized,
 *   src/memory/quant_weight_cache.mm:65-153); zeros must be NULL. */
MQ_API int mq_dequantize(const void* weights_packed, int64_t ldw_bytes, const void* scales,
                         const void* zeros, void* out, int64_t ldo, int64_t N, int64_t K,
                         int32_t group_size, int32_t quant_type, int32_t flat_groups, void* stream);

/* Residual add + RMSNorm fused into the decode GEMV (M = 1; no reference
 * counterpart: the decode step's glue).  x, delta (may be NULL), norm_weight,
 * resid_out fp16 [K] (16-byte aligned; resid_out must not alias x or delta):
 *   resid_out = half(x + delta);  h = half(resid_out * rsqrt(mean(resid_out^2)
 *   + eps) * norm_weight);  C = epilogue(h . deq(W)^T)  as mq_dequant_matmul.
 * Runs only where the row-block kernel takes the shape
 * (mq_rmsnorm_dequant_matmul_supported); otherwise returns 4 and the caller
 * runs mq_add_rmsnorm_f16 and mq_dequant_matmul. */
MQ_API int mq_rmsnorm_dequant_matmul(const void* x, const void* delta, const void* norm_weight, float eps,
                                     void* resid_out, const void* weights_packed, int64_t ldw_bytes,
                                     const void* scales, const void* zeros, void* C, int64_t N, int64_t K,
                                     int32_t group_size, int32_t quant_type, int32_t epilogue, const void* bias,
                                     void* stream);
MQ_API int mq_rmsnorm_dequant_matmul_supported(int64_t N, int64_t K, int32_t group_size, int32_t quant_type,
                                               int32_t epilogue);

/* Group quantizer, the inverse of the dequant formula (no reference
 * counterpart: the reference has no quantizer and its tests pack weights by
 * hand, tests/cpp/test_dequant_matmul.mm:104-116).  w fp16 [N, K] (row stride
 * ldw elements, 4-byte aligned) -> weights_packed int4 [N, K/2] / int8 [N, K]
 * (row stride ldo_bytes) and scales, zeros fp16 [N, ceil(K/group_size)]:
 *   INT4 (asymmetric): s = half((max-min)/15) (1 if 0),
 *     zp = clamp(rint(-min/s), 0, 15), q = clamp(rint(w/s)+zp, 0, 15),
 *     zeros = half((zp-8)*s); K and group_size even.
 *   INT8 (symmetric): s = half(max|w|/127) (1 if 0),
 *     q = clamp(rint(w/s), -127, 127), zeros = 0.
 * fp32 IEEE steps: bit-identical to the same steps on the host. */
MQ_API int mq_quantize(const void* w, int64_t ldw, void* weights_packed, int64_t ldo_bytes, void* scales,
                       void* zeros, int64_t N, int64_t K, int32_t group_size, int32_t quant_type, void* stream);

/* fp16 matmul route for M <= 8: C[M,N] = A[M,K] . op(B), fp32 accumulation.
 * transpose_b != 0: B is [N, K] (nn.Linear weight, python/metal_native/nn/linear.py:47-49);
 * transpose_b == 0: B is [K, N].  Replaces matmul_vecmat
 * (src/ops/matmul.mm:192-298, shaders/matmul_vecmat_kernel.metal:32-456) following
 * the documented contract C = A @ op(B) (include/metal_native/ops/matmul.h:18-37). */
MQ_API int mq_vecmat_f16(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc,
                         int64_t M, int64_t N, int64_t K, int32_t transpose_b, void* stream);

/* fp32 matmul route for skinny A: C[M,N] = A[M,K] . op(B), all fp32 (any M;
 * rows of A in launches of 8).  Replaces matmul_vecmat_fp32 and
 * matmul_vecmat_batch_fp32 (shaders/matmul_vecmat_kernel.metal:286-369,
 * :462-534, selected at src/ops/matmul.mm:213-225) following the documented
 * contract C = A @ op(B), as mq_vecmat_f16.  Deterministic. */
MQ_API int mq_vecmat_f32(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc,
                         int64_t M, int64_t N, int64_t K, int32_t transpose_b, void* stream);

/* out[i] = half(silu(float(gate[i])) * float(up[i])), i < n.
 * Replaces fast::swiglu (src/future/future_stubs.mm:61-101, bound as
 * _C.fast.swiglu at bindings/bind_ops.cpp:84-93). */
MQ_API int mq_swiglu_f16(const void* gate, const void* up, void* out, int64_t n, void* stream);

/* Decoder glue for the synthetic decode step.  No
 * counterpart on the reference's quantized path: its MiniGPT example
 * (examples/llm_generation.py) does these steps in numpy.
 * add_rmsnorm: per row, x <- half(x + delta) (delta may be NULL), then
 *   out = half(x * rsqrt(mean(x^2) + eps) * weight); x, out fp16 [rows, n].
 * rope_kv: qkv fp16 [heads*D | kv_heads*D | kv_heads*D]; q_out = rope(q);
 *   k_cache[h, pos] = rope(k), v_cache[h, pos] = v (caches fp16
 *   [kv_heads, max_len, D]); cos/sin fp32 [max_len, D] (rotate-half); pos is
 *   a device int64.
 * attention_decode: out[h] = softmax(q[h] . K^T * scale, t <= pos) . V for
 *   one query token, head h reading kv head h / (heads / kv_heads); split
 *   over positions, with per-split partials in the caller's workspace of
 *   mq_attention_decode_workspace_size(heads, head_dim, max_len) bytes. */
MQ_API int mq_add_rmsnorm_f16(void* x, const void* delta, const void* weight, void* out, int64_t rows, int64_t n,
                              float eps, void* stream);
MQ_API int mq_rope_kv_f16(const void* qkv, const float* cos_table, const float* sin_table, const int64_t* pos,
                          void* q_out, void* k_cache, void* v_cache, int32_t heads, int32_t kv_heads,
                          int32_t head_dim, int64_t max_len, void* stream);
MQ_API int64_t mq_attention_decode_workspace_size(int32_t heads, int32_t head_dim, int64_t max_len);
MQ_API int mq_attention_decode_f16(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos,
                                   void* out, int32_t heads, int32_t kv_heads, int32_t head_dim, int64_t max_len,
                                   float scale, void* workspace, int64_t workspace_bytes, void* stream);

/* rope_kv + attention_decode in one launch (head_dim 64 or 128, max_len <=
 * 4096; mq_attention_decode_rope_supported says whether a shape is taken):
 * rotates q and the new k from qkv (layout as rope_kv), writes the new k and
 * v into the caches at pos and returns attention_decode's output (one
 * workgroup per query head; its waves' partial softmax sums are combined in
 * LDS).  A device position outside [0, max_len) writes no cache row and
 * attends over the cache rows that exist: no access outside the caches or
 * the tables (the host must keep positions in range for a meaningful
 * result). */
MQ_API int mq_attention_decode_rope_supported(int32_t heads, int32_t head_dim, int64_t max_len);
MQ_API int mq_attention_decode_rope_f16(const void* qkv, const float* cos_table, const float* sin_table,
                                        const int64_t* pos, void* k_cache, void* v_cache, void* out, int32_t heads,
                                        int32_t kv_heads, int32_t head_dim, int64_t max_len, float scale,
                                        void* stream);

/* Greedy decode tail in one launch (decoder glue, no reference counterpart;
 * replaces torch.argmax + the embedding lookup + the position update of a
 * decode loop): token[0] = argmax(logits[vocab]) in torch.argmax order (NaN
 * above every number, ties to the lowest index), pos[0] += 1, and x[0:d] =
 * embed row token (row stride embed_stride elements).  The workspace of
 * mq_argmax_embed_workspace_size(vocab) bytes starts with a counter that must
 * be zero before the first call; every call leaves it zero.  Calls sharing a
 * workspace must be stream-ordered. */
MQ_API int64_t mq_argmax_embed_workspace_size(int64_t vocab);
MQ_API int mq_argmax_embed_f16(const void* logits, int64_t vocab, const void* embed, int64_t embed_stride, int64_t d,
                               int64_t* token, int64_t* pos, void* x, void* workspace, int64_t workspace_bytes,
                               void* stream);

/* Read probe: a measurement aid with no reference counterpart.  Reads the
 * `bytes` (< 2^31) bytes at p once, in one launch, the fastest way found on
 * gfx950 (one 12-wave workgroup per CU, 4-deep rings of 16-byte
 * non-temporal loads), and writes nothing but an occasional flag into sink
 * (mq_read_probe_sink_size() bytes).  The time of one launch bounds what any
 * kernel that reads the same bytes in one launch can reach; bench.py reports
 * it beside the headline. */
MQ_API int64_t mq_read_probe_sink_size(void);
MQ_API int mq_read_probe(const void* p, int64_t bytes, void* sink, void* stream);

/* Kernel-path override and layout knobs for tests and tuning (no reference
 * counterpart).  Keys: "force_path" (0 automatic, 2 the prefill GEMM family,
 * 3 generic, 6 split-K decode GEMV, 7 row-block decode GEMV, 12 register-
 * streamed decode GEMV: int4, 3 <= M <= 16), "gemv_steps"
 * (K steps per wavefront of the split-K GEMV, 1..8, 0 automatic),
 * "gemv_tiles_per_wg" (row tiles per workgroup: 1, 2 or 4, 0 automatic),
 * "gemm_impl" (prefill GEMM kernel: 0 automatic -- the register-dequant
 * 16x16x32 GEMM (128-row tiles; 64-row tiles for int8 SwiGLU up to M = 64)
 * where its tiles fill the GPU, else the register-operand 32x32x16 kernel
 * where it takes the shape --, 1 always the 16x16x32 tiled kernel, 2 the
 * register-dequant GEMM wherever it takes the shape; all compute the same
 * contract), "gemm_split" (1, the default: the 32x32x16 kernel splits
 * K over several workgroups per output tile where its tiles would leave CUs
 * idle, summing the parts in a fixed order; 0: one workgroup per tile).  A forced path that cannot take the shape falls back
 * to the automatic choice.  Returns MQ_INVALID_ARGUMENT for an unknown key or
 * value. */
MQ_API int mq_set_option(const char* key, int64_t value);

/* Kernel the last successful mq_dequant_matmul / mq_vecmat_f16 /
 * mq_vecmat_f32 call on this thread launched: 2 16x16x32 tiled GEMM, 3
 * generic, 4 vecmat [K,N], 6 split-K decode GEMV, 7 row-block decode GEMV, 8
 * 32x32x16 prefill GEMM, 9 fp32 vecmat, 10 32x32x16 prefill GEMM with K split
 * over workgroups, 11 register-dequant 16x16x32 prefill GEMM, 12
 * register-streamed decode GEMV. */
MQ_API int mq_last_path(void);

MQ_API const char* mq_last_error(void);
MQ_API const char* mq_error_to_string(int code);
MQ_API int mq_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* METAL_NATIVE_AMD_H */
