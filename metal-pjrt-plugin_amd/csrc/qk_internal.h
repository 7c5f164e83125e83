// Internal interfaces between the C-ABI layer (qk_abi.cpp) and the kernel
// launchers (gemm.hip, qmatvec.hip, rownorm.hip). Host-side only types; no
// torch, no XLA.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/qkern.h"

namespace qk {

// ---------------------------------------------------------------------------
// Errors (qk_abi.cpp).

// Records `msg` as this thread's last error and returns `s`.
qk_status Fail(qk_status s, const std::string& msg);

// Called before every kernel launch: QK_OK, or the sticky device error.
qk_status PreLaunch();

// Called after every kernel launch: counts launches, applies the
// QK_FAIL_LAUNCH test hook, and turns a launch error into the sticky
// device error.
qk_status PostLaunch(const char* kernel);

int DTypeSize(int dtype);

// Polls a bounded flag wait makes before it gives up (QK_SPIN_LIMIT in the
// environment, read with QK_FAIL_LAUNCH; default 2^20, ~70 ms).
int SpinLimit();

// Address of the device status word on the current device (qmatvec.hip),
// or null when it cannot be resolved. Kernels OR kStatus* bits into it.
uint32_t* DeviceStatusWord();

// OR of the status words of every device a kernel has been given one for
// (a blocking read: finished kernels only); clears them when `clear`.
uint32_t ReadDeviceStatusWords(bool clear);

// Compute units of the current device (cached per device).
int DeviceComputeUnits();

// Split-K workspace owned by the library, one per (device, stream): *ws
// takes at least `bytes` of f32 partials, *flags kWsFlagBytes / 4 arrival
// counters (zero between launches). Grown on demand by a new allocation of
// at least twice the size (the old one stays valid for launches already
// queued and for graphs captured from the stream, so all of a stream's
// buffers together stay under twice its largest), never freed before the
// process ends.
// Launches on one stream run in order, so they never use it concurrently;
// a captured graph keeps its capture stream's buffer, so its replays must
// not overlap other launches on that stream. False while the stream is
// being captured and the workspace is too small, or when allocation
// fails: the caller then takes a path without split K.
constexpr size_t kWsFlagBytes = 64 * 1024;
bool StreamWorkspace(hipStream_t stream, size_t bytes, float** ws,
                     uint32_t** flags);

// Workgroups of `kernel` one CU keeps resident with this block size and
// dynamic LDS (cached; at least 1).
int ResidentBlocks(const void* kernel, int block, size_t lds);
const char* DTypeName(int dtype);

// ---------------------------------------------------------------------------
// Dense GEMM, row-major view (the reference's mps::GemmParams,
// metal_pjrt/blas/mps_gemm.h:29-53).

struct Operand {
  const void* ptr = nullptr;
  int64_t ld = 0;            // elements between consecutive stored rows
  int64_t batch_stride = 0;  // elements between batches; 0 broadcasts
  int dtype = QK_F32;
  bool transpose = false;    // used as op(X) = X^T
};

// For each batch b: D = act(alpha op(A) op(B) + beta C + bias[col]),
// aux = the pre-activation value. C shares D's layout.
struct GemmProblem {
  int64_t m = 0, n = 0, k = 0, batch = 1;
  float alpha = 1.f, beta = 0.f;
  Operand a, b, d;
  const void* c = nullptr;  // read when beta != 0 (may equal d.ptr)
  const void* bias = nullptr;
  void* aux = nullptr;
  int act = 0;  // 0 none, 1 ReLU, 2 GELU (tanh), 3 SiLU
};

// Kernel choice for a problem (host only), and its name for debug output.
struct GemmKernelChoice {
  int family = 0;  // 0 MFMA tiles, 1 skinny (few rows / columns)
  int bm = 0, bn = 0, bk = 0;
  int tile = 0;  // tile configuration index (gemm.hip); -1: the f32 tiles
  int split_k = 1;
  std::string name;
};
GemmKernelChoice ChooseGemmKernel(const GemmProblem& p);

// Launches the GEMM. p has been validated; m, n, batch > 0.
qk_status LaunchGemm(const GemmProblem& p, hipStream_t stream);

// The few-row (M <= 8) f16/bf16 NT kernel (gemv.hip): whether it takes the
// problem, and its launch.
bool GemvApplies(const GemmProblem& p);
// At most 4 rows of x against W stored [K][N] (gemv_nn_kernel).
bool GemvNNApplies(const GemmProblem& p);
qk_status LaunchGemv(const GemmProblem& p, hipStream_t stream);

// ---------------------------------------------------------------------------
// Quantized matvec / dequantize (qmatvec.hip).

struct QuantProblem {
  int64_t m = 0, n = 0, k = 0;
  int bits = 4, group = 64, packing = QK_PACK_U32X8;
  bool has_bias = true;
  const void* x = nullptr;
  int x_dtype = QK_BF16;
  const void* codes = nullptr;
  const void* scales = nullptr;
  int scale_dtype = QK_BF16;
  const void* biases = nullptr;
  int bias_dtype = QK_BF16;
  void* y = nullptr;  // y dtype == x dtype; for dequantize, the weights
  int y_dtype = QK_BF16;
  // Embedding gather (qk_embed): output row t is table row rows[t]
  // (clamped to [0, n)), for t < rows_n; null: every row in order.
  const void* rows = nullptr;
  int64_t rows_n = 0;
};

qk_status LaunchQMatvec(const QuantProblem& p, hipStream_t stream);

// Quantized matmul for 5..32 rows of x (qskinny.hip): int4 u32x8 or
// int8, bf16, group 64.
bool QSkinnyApplies(const QuantProblem& p);
qk_status LaunchQSkinny(const QuantProblem& p, hipStream_t stream);
// int4, bf16, group 64, 1..16 rows, K a multiple of 512 up to 4096
// (qstream.hip).
bool QStreamApplies(const QuantProblem& p);
// Row-block rounds each of its waves runs on `cus` CUs.
int QStreamRounds(const QuantProblem& p, int cus);
qk_status LaunchQStream(const QuantProblem& p, hipStream_t stream);

// Quantized matmul for up to 128 rows of x (qmid.hip): int4 u32x8 or
// int8, bf16, group 64, K a multiple of 256.
bool QMidApplies(const QuantProblem& p);
qk_status LaunchQMid(const QuantProblem& p, hipStream_t stream);

// Dequantizing MFMA GEMM (qgemm.hip) for more than four rows of x.
bool QGemmApplies(const QuantProblem& p);
// The register-dequantizing GEMM (qgemm_dma.hip): int4 u32x8 / u8 / s8,
// group 64, bf16 scales, K a multiple of 512, N of 128, 16-byte aligned
// operands; tile and K split chosen per problem.
bool QGemmDmaApplies(const QuantProblem& p);
qk_status LaunchQGemmDma(const QuantProblem& p, hipStream_t stream);
qk_status LaunchQGemm(const QuantProblem& p, hipStream_t stream);
qk_status LaunchDequantize(const QuantProblem& p, hipStream_t stream);
// The quantizer (quantize.hip): w [n, k] of w_dtype into p's codes, scales
// and offsets (outputs; scale and offset dtype p.scale_dtype).
qk_status LaunchQuantize(const QuantProblem& p, const void* w, int w_dtype,
                         hipStream_t stream);

// Dense embedding gather: out[t, :] = table[clamp(rows[t]), :] (k elements
// of esz bytes per row; table rows ld elements apart).
qk_status LaunchRowGather(const void* table, int64_t n, int64_t k, int64_t ld,
                          int esz, const void* rows, int64_t rows_n, void* out,
                          hipStream_t stream);

// ---------------------------------------------------------------------------
// Row normalisation (rownorm.hip).

struct RownormProblem {
  int64_t rows = 0, n = 0;
  int kind = QK_ROWNORM_RMS;
  float eps = 1e-6f;
  const void* x = nullptr;
  void* y = nullptr;
  int dtype = QK_F32;
  const void* gain = nullptr;
  int gain_dtype = QK_F32;
  const void* beta = nullptr;
  int beta_dtype = QK_F32;
};

qk_status LaunchRownorm(const RownormProblem& p, hipStream_t stream);

// ---------------------------------------------------------------------------
// Decode attention (attention.hip).

struct AttentionProblem {
  int64_t b = 0, kv = 0, g = 0, d = 0;  // q [b, kv, g, d]
  int64_t smax = 0, window = 0;         // cache slots, slots read
  float scale = 1.f;
  int dtype = QK_BF16;                  // q, caches and output
  const void* q = nullptr;
  const void* k = nullptr;  // [b, kv, smax, d]
  const void* v = nullptr;  // [b, kv, d, smax]
  const void* pos = nullptr;  // int32 device scalar
  void* out = nullptr;        // [b, kv, g, d]
  // Set by PlanAttention: partials per (b, kv) (runs of 64-slot chunks of
  // the attended window) and the workspace they take.
  int parts = 0;
  uint64_t workspace_bytes = 0;
};

void PlanAttention(AttentionProblem* p);

// Bytes of the fixed device scratch qk_decode_attention_noalloc uses in
// place of a workspace (one copy per device, held until the process ends).
constexpr uint64_t kAttentionScratchBytes = uint64_t{8} << 20;
static_assert(kAttentionScratchBytes == QK_ATTENTION_SCRATCH_BYTES,
              "the scratch size the header states");

// The current device's address of that scratch (resolved with
// hipGetSymbolAddress on the first call per device; allocates nothing).
qk_status AttentionScratch(void** ptr);
qk_status LaunchAttention(const AttentionProblem& p, void* workspace,
                          hipStream_t stream);

}  // namespace qk
