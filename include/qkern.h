/*
 * qkern.h -- C ABI of the MI355X (gfx950) hot path of the metal-pjrt-plugin
 * JAX PJRT plugin: dense GEMM with a cuBLASLt-style epilogue, group-affine
 * int8/int4 weight-quantized matvec/matmul, and row-wise normalisation
 * (RMSNorm, LayerNorm, softmax).
 *
 * Plain C: device pointers, sizes and small POD descriptors only. A PJRT/XLA
 * integration binds these from its BlasLt and typed-FFI handlers; ctypes
 * binds them in the tests and the benchmark.
 *
 * Conventions
 *  - Every entry point returns a qk_status (absl::StatusCode values). On
 *    failure qk_last_error_message() holds a thread-local message that says
 *    what to change.
 *  - Device errors are sticky: once a launch has failed, every later call
 *    that would launch returns QK_INTERNAL with the first failure's message
 *    until qk_reset_device_error() (reference: metal_pjrt/runtime/
 *    metal_runtime.h:43-53, the sticky Device::error()).
 *  - Streams are hipStream_t passed as void* (NULL = the null stream). The
 *    library launches on that stream only, allocates no device memory and
 *    starts no threads. Plans are immutable after creation and may be used
 *    from any thread.
 *  - Test hook: with QK_FAIL_LAUNCH=n in the environment (read at the first
 *    launch and by qk_reset_device_error), the n-th launch is treated as
 *    failed (reference: METAL_PJRT_FAIL_COMMAND_BUFFER, metal_pjrt/runtime/
 *    metal_runtime.cc:1646-1652).
 */
#ifndef QKERN_H_
#define QKERN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* absl::StatusCode values; the classes the reference uses
 * (metal_pjrt/runtime/metal_runtime.h:33-41). */
typedef enum {
  QK_OK = 0,
  QK_INVALID_ARGUMENT = 3,
  QK_RESOURCE_EXHAUSTED = 8,
  QK_UNIMPLEMENTED = 12,
  QK_INTERNAL = 13,
} qk_status;

/* Element types. F32/F16/BF16 are GEMM and activation types; U8, S8 and
 * U32 hold quantized codes; S32 (or U32) holds the decode position. */
typedef enum {
  QK_F32 = 0,
  QK_F16 = 1,
  QK_BF16 = 2,
  QK_U8 = 3,
  QK_S8 = 4,
  QK_U32 = 5,
  QK_S32 = 6,
} qk_dtype;

/* ------------------------------------------------------------------------
 * Dense GEMM: the BlasLt matmul plan.
 * ---------------------------------------------------------------------- */

typedef enum { QK_ROW_MAJOR = 0, QK_COLUMN_MAJOR = 1 } qk_order;

/* Mirrors gpu::MatrixLayout (XLA stream_executor/gpu/gpu_blas_lt.h), as the
 * reference consumes it in ValidateMatmul (metal_pjrt/blas/
 * blas_lt_support.cc:103-201). The stored matrix is num_rows x num_cols in
 * `order`; leading_dim_stride is the element distance between consecutive
 * rows (row-major) or columns (column-major); batch_stride the element
 * distance between batches (ignored when batch_size is 1). `transpose` must
 * be 0 (the reference refuses transposed layouts,
 * blas_lt_support.cc:112-118). */
typedef struct {
  int32_t dtype; /* qk_dtype: F32, F16 or BF16 */
  int32_t order; /* qk_order */
  int64_t num_rows;
  int64_t num_cols;
  int64_t batch_size;
  int64_t leading_dim_stride;
  int64_t batch_stride;
  int32_t transpose;
  int32_t reserved;
} qk_matrix_layout;

/* Mirrors the fields of gpu::GemmConfig that the reference reads
 * (metal_pjrt/blas/metal_blas.cc:245-287): D = alpha*A*B + beta*C. */
typedef struct {
  qk_matrix_layout lhs, rhs, c, output;
  double alpha_re;
  double alpha_im;
  double beta;
} qk_gemm_config;

/* The twelve gpu::BlasLt::Epilogue values the reference decodes
 * (DecodeEpilogue, metal_pjrt/blas/blas_lt_support.cc:25-83). The integer
 * values are this ABI's own; a binding maps BlasLt::Epilogue by name. */
typedef enum {
  QK_EPILOGUE_DEFAULT = 0,
  QK_EPILOGUE_RELU = 1,
  QK_EPILOGUE_BIAS = 2,
  QK_EPILOGUE_BIAS_THEN_RELU = 3,
  QK_EPILOGUE_GELU = 4,
  QK_EPILOGUE_GELU_WITH_AUX = 5,
  QK_EPILOGUE_BIAS_THEN_GELU = 6,
  QK_EPILOGUE_BIAS_THEN_GELU_WITH_AUX = 7,
  QK_EPILOGUE_SILU = 8,
  QK_EPILOGUE_SILU_WITH_AUX = 9,
  QK_EPILOGUE_BIAS_THEN_SILU = 10,
  QK_EPILOGUE_BIAS_THEN_SILU_WITH_AUX = 11,
} qk_epilogue;

/* Mirrors gpu::BlasLt::MemoryArgs (the buffers ExecuteOnStream binds,
 * metal_pjrt/blas/metal_blas.cc:294-338): device pointers with their sizes
 * in bytes. c may be NULL (D is then read in place when beta != 0); bias
 * and aux are required exactly when the epilogue has them. */
typedef struct {
  const void* a;
  uint64_t a_size;
  const void* b;
  uint64_t b_size;
  const void* c;
  uint64_t c_size;
  void* d;
  uint64_t d_size;
  const void* bias;
  uint64_t bias_size;
  void* aux;
  uint64_t aux_size;
} qk_memory_args;

typedef struct qk_gemm_plan qk_gemm_plan;

/* Replaces MetalBlasLt::GetMatmulPlan (metal_pjrt/blas/metal_blas.cc:
 * 245-287) with ValidateMatmul (blas_lt_support.cc:103-201): validates the
 * configuration exactly as the reference does (same refusals and status
 * classes) and returns an immutable plan. Host only; launches nothing. */
qk_status qk_gemm_plan_create(const qk_gemm_config* config,
                              int32_t epilogue, qk_gemm_plan** plan);

/* Replaces MatmulPlan::ExecuteOnStream (metal_pjrt/blas/metal_blas.cc:
 * 294-338) and its kernels (RunHalfGemm :91-100, RunSteelGemm
 * steel_gemm.cc:163-255, RunGemv gemv.cc:129-196, RunMpsGemm + RunEpilogue
 * metal_blas.cc:114-118,399-423). For each batch, in the row-major view:
 *   v = alpha*op(A)op(B) + beta*C + bias[col];  aux = v;  D = act(v)
 * computed in f32 and rounded once to D's type. */
qk_status qk_gemm_execute(const qk_gemm_plan* plan, void* stream,
                          const qk_memory_args* args);

void qk_gemm_plan_destroy(qk_gemm_plan* plan);

/* Debug string of a plan's row-major problem and chosen kernel
 * (GemmParamsDebugString, metal_pjrt/blas/mps_gemm.h:67). Thread-local
 * storage, valid until the next call on this thread. */
const char* qk_gemm_plan_describe(const qk_gemm_plan* plan);

/* ------------------------------------------------------------------------
 * Typed-FFI style targets. A buffer is an FFI AnyBuffer: data, element
 * type and dimensions (row-major, dense).
 * ---------------------------------------------------------------------- */

#define QK_MAX_RANK 6

typedef struct {
  void* data;
  int32_t dtype; /* qk_dtype */
  int32_t rank;
  int64_t dims[QK_MAX_RANK];
} qk_buffer;

/* Quantized weight packings. */
typedef enum {
  /* 4-bit codes, 8 per uint32 along K: word i of a row holds elements
   * 8i..8i+7, element 8i+j in bits 4j..4j+3. Codes [N, K/8] u32. */
  QK_PACK_U32X8 = 0,
  /* 4-bit codes as the reference's quantize_int4 stores them
   * (examples/llm/qwen3.py:169-196): bytes [N, K/g, g/2] u8, element j of
   * a group in the low nibble of byte j, element j + g/2 in the high
   * nibble. */
  QK_PACK_BYTE_HALFSPLIT = 1,
  /* 8-bit unsigned affine codes, [N, K] (or [N, K/g, g]) u8. */
  QK_PACK_U8 = 2,
  /* 8-bit signed symmetric codes as quantize_int8 stores them
   * (qwen3.py:154-166): [N, K/g, g] (or [N, K]) s8, no offset. */
  QK_PACK_S8_SYM = 3,
} qk_packing;

/* Attributes of the qk$qmatvec / qk$dequantize targets. Per group of
 * `group_size` consecutive inputs of an output row o:
 *   w[o, k] = scale[o, g] * q[o, k] + bias[o, g]     (bias omitted when
 *                                                    has_bias is 0) */
typedef struct {
  int32_t bits;       /* 4 or 8; must agree with packing */
  int32_t group_size; /* 32, 64 or 128 */
  int32_t packing;    /* qk_packing */
  int32_t has_bias;   /* affine offset per group */
} qk_quant_attrs;

/* Target qk$qmatvec: y[m, o] = sum_k x[m, k] * w[o, k] for x [..., K]
 * (M = product of the leading dimensions) in f32, f16 or bf16, with w
 * dequantized on the fly; the sum is formed in f32 and rounded once to x's
 * type into y [..., N]. scales/biases [N, K/g] (trailing 1 allowed) in f32,
 * f16 or bf16. Replaces the reduction fusions XLA emits for _matvec_int8 /
 * _matvec_int4 (examples/llm/qwen3.py:233-267) and, for rows beyond the
 * matvec range, linear()'s dequantize-then-einsum (qwen3.py:218-230).
 * For many rows (65 and up) on few weight rows the library may split K
 * over workgroups; the partial sums then go through a workspace it owns,
 * one per (device, stream), allocated on the first such call on a stream
 * and grown (never freed) when a larger one is needed. Such a call on a
 * stream that is being captured and has no large enough workspace yet
 * takes the unsplit kernel instead. Results do not depend on the split. */
qk_status qk_qmatvec(void* stream, const qk_buffer* x, const qk_buffer* codes,
                     const qk_buffer* scales, const qk_buffer* biases,
                     qk_buffer* y, const qk_quant_attrs* attrs);

/* Target qk$embed: out [tokens..., K] = rows of an embedding table picked
 * by int32 tokens (any shape; indices outside [0, V) are clamped, as a
 * JAX gather clamps them). Quantized (scales given): table = codes of
 * [V, K] in attrs' packing with scales/biases [V, K/g], each picked row
 * dequantized as qk_dequantize does (f32(q)*f32(s) + f32(b), one rounding
 * to out's f32, f16 or bf16). Dense (scales NULL): table [V, K] of out's
 * type, rows copied (16-byte aligned rows). Replaces embed
 * (examples/llm/qwen3.py:270-274): the gather of q4/q, s, b rows and the
 * dequantize of qwen3.py:199-207, or w[tokens]. */
qk_status qk_embed(void* stream, const qk_buffer* tokens,
                   const qk_buffer* table, const qk_buffer* scales,
                   const qk_buffer* biases, qk_buffer* out,
                   const qk_quant_attrs* attrs);

/* Target qk$dequantize: w [N, K] in w's dtype (f32, f16 or bf16), each
 * element computed as f32(q)*f32(scale) + f32(bias) in f32 and rounded once.
 * Replaces dequantize (examples/llm/qwen3.py:199-207). */
qk_status qk_dequantize(void* stream, const qk_buffer* codes,
                        const qk_buffer* scales, const qk_buffer* biases,
                        qk_buffer* w, const qk_quant_attrs* attrs);

/* Quantizes w [N, K] (f32, f16 or bf16, 16-byte aligned) into the codes,
 * scales and offsets qk$qmatvec reads (all outputs, shaped as qk_qmatvec
 * takes them for attrs): int4 affine (U32X8 or BYTE_HALFSPLIT; biases
 * required, has_bias = 1) on the MLX-style grid of quantize_int4
 * (examples/llm/qwen3.py:169-196), or symmetric int8 (S8_SYM; no biases)
 * as quantize_int8 (qwen3.py:154-166). Bit-identical to those float32
 * computations; scales and offsets (one dtype) are stored in f32 or
 * rounded once to f16 / bf16. U8 (affine 8-bit) has no reference
 * quantizer: QK_UNIMPLEMENTED. Replaces the host quantization the
 * reference's load_params does per matrix (qwen3.py:113-128). */
qk_status qk_quantize(void* stream, const qk_buffer* w, qk_buffer* codes,
                      qk_buffer* scales, qk_buffer* biases,
                      const qk_quant_attrs* attrs);

typedef enum {
  QK_ROWNORM_RMS = 0,     /* y = x * rsqrt(mean(x^2) + eps) * gain */
  QK_ROWNORM_LAYER = 1,   /* y = (x - mean) / sqrt(var + eps) * gain + beta */
  QK_ROWNORM_SOFTMAX = 2, /* y = exp(x - max) / sum(exp(x - max)) */
} qk_rownorm_kind;

typedef struct {
  int32_t kind; /* qk_rownorm_kind */
  float eps;
  int32_t has_gain; /* RMS, LAYER: multiply by gain[col] */
  int32_t has_beta; /* LAYER: add beta[col] */
} qk_rownorm_attrs;

/* Target qk$rownorm over the last dimension of x [..., n] (f32, f16 or
 * bf16) into y of the same shape and type, computed in f32 with one
 * rounding at the end. gain/beta are [n] in any float type (NULL when
 * unused). Replaces the reduction fusions of rms_norm
 * (examples/llm/qwen3.py:294-297), jax.nn.softmax (qwen3.py:325,330) and
 * the benchmark's layernorm (bench/jax_bench.py:44-46). */
qk_status qk_rownorm(void* stream, const qk_buffer* x, const qk_buffer* gain,
                     const qk_buffer* beta, qk_buffer* y,
                     const qk_rownorm_attrs* attrs);

/* Attributes of the qk$decode_attention target. */
typedef struct {
  float scale;    /* multiplies q.k; the reference uses head_dim ** -0.5 */
  int32_t window; /* S: cache slots [0, S) are attended where s <= position;
                     0 means the whole cache (Smax) */
} qk_attention_attrs;

/* Workspace bytes qk_decode_attention needs for these shapes: partial
 * (max, sum, accumulator) rows of the split cache window, f32. */
qk_status qk_decode_attention_workspace_size(const qk_buffer* q,
                                             const qk_buffer* k_cache,
                                             const qk_attention_attrs* attrs,
                                             uint64_t* bytes);

/* Target qk$decode_attention: grouped-query attention of one query per
 * sequence against the KV cache, as the one-query branch of the
 * reference's attention() (examples/llm/qwen3.py:322-326) computes it with
 * forward()'s decode mask (qwen3.py:357-358), replacing the reductions XLA
 * emits for it:
 *   q [B, KV, G, D] (or [B, 1, KV, G, D]), k_cache [B, KV, Smax, D],
 *   v_cache [B, KV, D, Smax] (the layouts of init_cache, qwen3.py:
 *   279-291), position: int32 device scalar (1 element, S32 or U32);
 *   t[s] = scale * sum_d q[d] k[s, d] for slots s < window with s <= pos,
 *   p = softmax(t), out[g, d] = sum_s p[s] v[d, s]
 * in f32, rounded once into out (q's shape and type). q, caches and out
 * are all bf16 or all f16; D is 64 or 128; G <= 16; Smax a multiple of 8
 * and at most 2^22; buffers 16-byte aligned. The position is read on the
 * device (a jitted decode loop passes it as a traced value); slots past
 * min(window, pos + 1) take no part, whatever they hold (keys there are
 * not read; values are read in 8-slot units, units wholly past it are
 * not). `workspace` (device memory of at least
 * qk_decode_attention_workspace_size bytes, contents ignored, clobbered)
 * holds the partials of the split window. */
qk_status qk_decode_attention(void* stream, const qk_buffer* q,
                              const qk_buffer* k_cache,
                              const qk_buffer* v_cache,
                              const qk_buffer* position, qk_buffer* out,
                              const qk_attention_attrs* attrs,
                              void* workspace, uint64_t workspace_bytes);

/* qk$decode_attention without a workspace and without any allocation: the
 * split window's partials go to a fixed device scratch of
 * QK_ATTENTION_SCRATCH_BYTES that the library holds on each device it runs
 * on until the process ends. It has no counterpart in the reference; it is
 * for callers that cannot allocate device memory (HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same operands, checks and
 * results as qk_decode_attention; shapes whose partials
 * (qk_decode_attention_workspace_size) exceed the scratch are refused with
 * QK_INVALID_ARGUMENT. The stream must belong to the current device. Every
 * call on one device shares that device's scratch: calls that overlap on
 * one device (different streams, or different threads without ordering)
 * race and give wrong results. Nothing in the scratch needs clearing: each
 * call writes every partial it reads. */
#define QK_ATTENTION_SCRATCH_BYTES (8u << 20)
qk_status qk_decode_attention_noalloc(void* stream, const qk_buffer* q,
                                      const qk_buffer* k_cache,
                                      const qk_buffer* v_cache,
                                      const qk_buffer* position,
                                      qk_buffer* out,
                                      const qk_attention_attrs* attrs);

/* ------------------------------------------------------------------------
 * Status.
 * ---------------------------------------------------------------------- */

/* Message of the last failed call on this thread ("" when none). */
const char* qk_last_error_message(void);

/* QK_OK, or the sticky device error (its message in
 * qk_last_error_message()). Also reads the device status word of every
 * device used so far (a blocking read; synchronize the streams first): a
 * kernel whose bounded wait between producer and consumer waves gave up
 * (after QK_SPIN_LIMIT polls, default 2^20) stores NaN outputs and sets
 * that word, and it becomes the sticky QK_INTERNAL error here. */
qk_status qk_device_error(void);

/* Clears the sticky device error and the device status words, and
 * re-reads QK_FAIL_LAUNCH and QK_SPIN_LIMIT (tests). */
void qk_reset_device_error(void);

/* Library version string. */
const char* qk_version(void);

#ifdef __cplusplus
}
#endif

#endif /* QKERN_H_ */
