// The C ABI (include/qkern.h): status handling, the BlasLt-style matmul plan
// with the reference's validation, and the typed-FFI style entry points'
// argument checks. Kernels live in gemm.hip, qmatvec.hip and rownorm.hip.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cinttypes>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "qk_internal.h"

// ---------------------------------------------------------------------------
// Status.

namespace qk {
namespace {

thread_local std::string g_last_error;

// Sticky device error (reference: Device::error(), metal_pjrt/runtime/
// metal_runtime.h:43-53): the first failed launch sets it and every later
// launch returns it.
std::mutex g_sticky_mu;
std::atomic<int> g_sticky_status{QK_OK};
std::string g_sticky_message;

// QK_FAIL_LAUNCH test hook (reference: METAL_PJRT_FAIL_COMMAND_BUFFER,
// metal_pjrt/runtime/metal_runtime.cc:1646-1652).
std::atomic<int64_t> g_launches{0};
std::atomic<int64_t> g_fail_at{-1};  // -1: not read yet; 0: disabled
std::once_flag g_env_once;

// QK_SPIN_LIMIT: polls before a bounded flag wait gives up (tests force a
// timeout with 0; every wait still ends).
std::atomic<int> g_spin_limit{1 << 20};

void ReadSpinEnv() {
  const char* v = std::getenv("QK_SPIN_LIMIT");
  int n = 1 << 20;
  if (v != nullptr && *v != '\0') {
    char* end = nullptr;
    long long parsed = std::strtoll(v, &end, 10);
    if (end != v && *end == '\0' && parsed >= 0 && parsed <= (1 << 24))
      n = static_cast<int>(parsed);
  }
  g_spin_limit.store(n);
}

void ReadFailEnv() {
  ReadSpinEnv();
  const char* v = std::getenv("QK_FAIL_LAUNCH");
  int64_t n = 0;
  if (v != nullptr && *v != '\0') {
    char* end = nullptr;
    long long parsed = std::strtoll(v, &end, 10);
    if (end != v && *end == '\0' && parsed > 0) n = parsed;
  }
  g_fail_at.store(n);
}

void SetSticky(qk_status s, const std::string& msg) {
  std::lock_guard<std::mutex> lock(g_sticky_mu);
  if (g_sticky_status.load() == QK_OK) {
    g_sticky_message = msg;
    g_sticky_status.store(s);
  }
}

}  // namespace

int SpinLimit() {
  std::call_once(g_env_once, [] {
    if (g_fail_at.load() < 0) ReadFailEnv();
  });
  return g_spin_limit.load();
}

qk_status Fail(qk_status s, const std::string& msg) {
  g_last_error = msg;
  return s;
}

qk_status PreLaunch() {
  std::call_once(g_env_once, [] {
    if (g_fail_at.load() < 0) ReadFailEnv();
  });
  if (g_sticky_status.load() != QK_OK) {
    std::lock_guard<std::mutex> lock(g_sticky_mu);
    return Fail(static_cast<qk_status>(g_sticky_status.load()),
                "qkern: an earlier GPU launch failed: " + g_sticky_message);
  }
  return QK_OK;
}

qk_status PostLaunch(const char* kernel) {
  const int64_t n = g_launches.fetch_add(1) + 1;
  hipError_t e = hipGetLastError();
  std::string msg;
  if (e != hipSuccess) {
    msg = std::string("launch of ") + kernel + " failed: " +
          hipGetErrorString(e);
  } else if (g_fail_at.load() > 0 && n == g_fail_at.load()) {
    msg = std::string("launch of ") + kernel +
          " failed (injected by QK_FAIL_LAUNCH=" + std::to_string(n) + ")";
  }
  if (msg.empty()) return QK_OK;
  SetSticky(QK_INTERNAL, msg);
  return Fail(QK_INTERNAL, "qkern: " + msg);
}

int DeviceComputeUnits() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount,
                              dev) != hipSuccess ||
        cus <= 0) {
      cus = 256;
    }
    cached[dev] = cus;
  }
  return cached[dev];
}

bool StreamWorkspace(hipStream_t stream, size_t bytes, float** ws,
                     uint32_t** flags) {
  struct Entry {
    int dev;
    hipStream_t stream;
    void* p;
    size_t bytes;
  };
  static std::mutex mu;
  static std::vector<Entry> table;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  const size_t need = kWsFlagBytes + ((bytes + 255) / 256) * 256;
  std::lock_guard<std::mutex> lock(mu);
  Entry* e = nullptr;
  for (auto& t : table)
    if (t.dev == dev && t.stream == stream) e = &t;
  if (e != nullptr && e->bytes >= need) {
    *flags = static_cast<uint32_t*>(e->p);
    *ws = reinterpret_cast<float*>(static_cast<char*>(e->p) + kWsFlagBytes);
    return true;
  }
  // Growing allocates: not while the stream is captured.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess ||
      cap != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return false;
  }
  // At least double the previous size: the replaced buffers (kept alive)
  // then total less than the largest one.
  const size_t size = std::max<size_t>(
      std::max<size_t>(need, size_t{32} << 20), e != nullptr ? 2 * e->bytes : 0);
  // A smaller buffer being replaced is not freed: launches still queued
  // on the stream, and graphs captured from it, keep using it.
  void* p = nullptr;
  if (hipMalloc(&p, size) != hipSuccess ||
      hipMemset(p, 0, kWsFlagBytes) != hipSuccess) {
    if (p != nullptr) (void)hipFree(p);
    (void)hipGetLastError();
    return false;
  }
  if (e == nullptr) {
    table.push_back(Entry{dev, stream, p, size});
  } else {
    e->p = p;
    e->bytes = size;
  }
  *flags = static_cast<uint32_t*>(p);
  *ws = reinterpret_cast<float*>(static_cast<char*>(p) + kWsFlagBytes);
  return true;
}

int ResidentBlocks(const void* kernel, int block, size_t lds) {
  struct Key {
    const void* k;
    int block;
    size_t lds;
    int n;
  };
  static std::mutex mu;
  static Key cache[256];
  static int used = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i) {
    if (cache[i].k == kernel && cache[i].block == block &&
        cache[i].lds == lds) {
      return cache[i].n;
    }
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, lds) !=
          hipSuccess ||
      n < 1) {
    (void)hipGetLastError();
    n = 1;
  }
  if (used < 256) cache[used++] = {kernel, block, lds, n};
  return n;
}

int DTypeSize(int dtype) {
  switch (dtype) {
    case QK_F32:
    case QK_U32:
    case QK_S32:
      return 4;
    case QK_F16:
    case QK_BF16:
      return 2;
    case QK_U8:
    case QK_S8:
      return 1;
  }
  return 0;
}

const char* DTypeName(int dtype) {
  switch (dtype) {
    case QK_F32:
      return "f32";
    case QK_F16:
      return "f16";
    case QK_BF16:
      return "bf16";
    case QK_U8:
      return "u8";
    case QK_S8:
      return "s8";
    case QK_U32:
      return "u32";
    case QK_S32:
      return "s32";
  }
  return "?";
}

}  // namespace qk

using qk::Fail;

// ---------------------------------------------------------------------------
// GEMM plan.

struct qk_gemm_plan {
  qk::GemmProblem p;   // pointers unset
  bool swap = false;   // D^T = B^T A^T: A and B buffers exchanged
  bool bias = false, aux = false;
  int act = 0;
  double beta = 0.0;
  qk::GemmKernelChoice choice;
};

namespace {

struct EpilogueSpec {
  bool bias = false;
  int act = 0;
  bool aux = false;
  bool trivial() const { return !bias && act == 0; }
};

// DecodeEpilogue (reference metal_pjrt/blas/blas_lt_support.cc:25-83).
qk_status DecodeEpilogue(int32_t e, EpilogueSpec* s) {
  if (e < QK_EPILOGUE_DEFAULT || e > QK_EPILOGUE_BIAS_THEN_SILU_WITH_AUX) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: matmul with fused epilogue " + std::to_string(e) +
                    " is not supported");
  }
  static const EpilogueSpec kTable[12] = {
      {false, 0, false}, {false, 1, false}, {true, 0, false},
      {true, 1, false},  {false, 2, false}, {false, 2, true},
      {true, 2, false},  {true, 2, true},   {false, 3, false},
      {false, 3, true},  {true, 3, false},  {true, 3, true},
  };
  *s = kTable[e];
  return QK_OK;
}

std::string LayoutString(const qk_matrix_layout& l) {
  char buf[256];
  std::snprintf(buf, sizeof(buf),
                "{%s %" PRId64 "x%" PRId64 " %s batch=%" PRId64 " ld=%" PRId64
                " batch_stride=%" PRId64 "%s}",
                qk::DTypeName(l.dtype), l.num_rows, l.num_cols,
                l.order == QK_ROW_MAJOR ? "row" : "col", l.batch_size,
                l.leading_dim_stride, l.batch_stride,
                l.transpose ? " T" : "");
  return buf;
}

// gpu::MatrixLayout::Transpose: the same storage viewed transposed.
void TransposeLayout(qk_matrix_layout* l) {
  std::swap(l->num_rows, l->num_cols);
  l->order = l->order == QK_ROW_MAJOR ? QK_COLUMN_MAJOR : QK_ROW_MAJOR;
}

bool IsFloat(int t) { return t == QK_F32 || t == QK_F16 || t == QK_BF16; }

// CheckBlasLtTypes (reference blas_lt_support.cc:85-99).
qk_status CheckTypes(int a, int b, int out) {
  if (IsFloat(a) && a == b && IsFloat(out) && (out == a || out == QK_F32)) {
    return QK_OK;
  }
  return Fail(QK_UNIMPLEMENTED,
              std::string("qkern: matmul ") + qk::DTypeName(a) + " x " +
                  qk::DTypeName(b) + " -> " + qk::DTypeName(out) +
                  " is not supported: both operands must be f32, f16 or "
                  "bf16 of one type, the result that type or f32. Cast the "
                  "operands");
}

}  // namespace

extern "C" qk_status qk_gemm_plan_create(const qk_gemm_config* cfg,
                                         int32_t epilogue,
                                         qk_gemm_plan** out_plan) {
  if (cfg == nullptr || out_plan == nullptr) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: null config or plan pointer");
  }
  *out_plan = nullptr;
  // ValidateMatmul (reference blas_lt_support.cc:103-201), step by step.
  qk_matrix_layout lhs = cfg->lhs, rhs = cfg->rhs, c = cfg->c,
                   out = cfg->output;
  EpilogueSpec epi;
  if (qk_status s = DecodeEpilogue(epilogue, &epi); s != QK_OK) return s;
  if (cfg->alpha_im != 0.0) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: matmul with a complex scale factor is not supported");
  }
  for (const qk_matrix_layout* l : {&lhs, &rhs, &c, &out}) {
    if (l->transpose != 0) {
      return Fail(QK_UNIMPLEMENTED,
                  "qkern: matmul: transposed layout " + LayoutString(*l));
    }
    if (l->order != QK_ROW_MAJOR && l->order != QK_COLUMN_MAJOR) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: matmul: unknown order in " + LayoutString(*l));
    }
    if (l->num_rows < 0 || l->num_cols < 0 || l->batch_size < 0 ||
        l->leading_dim_stride < 0 || l->batch_stride < 0) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: matmul: negative size in " + LayoutString(*l));
    }
  }
  // An operand without a batch dimension is broadcast (batch_stride 0).
  const int64_t batch = std::max(lhs.batch_size, rhs.batch_size);
  lhs.batch_size = rhs.batch_size = batch;
  if (out.batch_size != batch) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: matmul: batch mismatch " + LayoutString(out));
  }
  // Row-major kernels: a column-major output is D^T = B^T A^T.
  const bool swap = out.order == QK_COLUMN_MAJOR;
  if (swap) {
    std::swap(lhs, rhs);
    TransposeLayout(&lhs);
    TransposeLayout(&rhs);
    TransposeLayout(&c);
    TransposeLayout(&out);
  }
  const int64_t m = out.num_rows, n = out.num_cols, k = lhs.num_cols;
  if (lhs.num_rows != m || rhs.num_rows != k || rhs.num_cols != n) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: matmul: inconsistent shapes lhs=" + LayoutString(lhs) +
                    " rhs=" + LayoutString(rhs) + " out=" + LayoutString(out));
  }
  if (qk_status s = CheckTypes(lhs.dtype, rhs.dtype, out.dtype); s != QK_OK) {
    return s;
  }
  if (cfg->beta != 0.0 &&
      (c.dtype != out.dtype || c.order != out.order ||
       c.leading_dim_stride != out.leading_dim_stride ||
       c.batch_stride != out.batch_stride || c.num_rows != out.num_rows ||
       c.num_cols != out.num_cols)) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: matmul adding an operand laid out unlike the result "
                "is not supported (" +
                    LayoutString(c) + " vs " + LayoutString(out) + ")");
  }
  const int t = lhs.dtype;
  constexpr int64_t kMaxInt = 2147483647;
  if (t == QK_F16 || t == QK_BF16) {
    // The f16/bf16 kernels index within a matrix in 32 bits: every
    // dimension and the batch count fit in int32, and every leading
    // dimension in INT32_MAX / 256 elements.
    constexpr int64_t kMaxLd = kMaxInt / 256;
    auto refuse = [&](const char* what, int64_t value, int64_t limit) {
      return Fail(QK_UNIMPLEMENTED,
                  std::string("qkern: ") + qk::DTypeName(t) +
                      " matmul too large: the f16/bf16 matmul kernels index "
                      "in 32 bits, and its " +
                      what + " " + std::to_string(value) + " exceeds " +
                      std::to_string(limit) +
                      ". Split the matmul or use float32");
    };
    if (batch > kMaxInt) return refuse("batch count", batch, kMaxInt);
    for (int64_t dim : {m, n, k}) {
      if (dim > kMaxInt) return refuse("dimension", dim, kMaxInt);
    }
    for (const qk_matrix_layout* l : {&lhs, &rhs, &out}) {
      if (l->leading_dim_stride > kMaxLd) {
        return refuse("leading dimension (elements between rows)",
                      l->leading_dim_stride, kMaxLd);
      }
    }
  } else {
    // The f32 kernels take every dimension and leading dimension as a
    // 32-bit int (row offsets are formed in 64 bits): refuse what does not
    // fit instead of truncating it, as the reference refuses what its
    // kernels cannot index (blas_lt_support.cc:166-199).
    auto refuse = [&](const char* what, int64_t value) {
      return Fail(QK_UNIMPLEMENTED,
                  std::string("qkern: f32 matmul too large: the f32 matmul "
                              "kernels take 32-bit sizes, and its ") +
                      what + " " + std::to_string(value) + " exceeds " +
                      std::to_string(kMaxInt) + ". Split the matmul");
    };
    if (batch > kMaxInt) return refuse("batch count", batch);
    for (int64_t dim : {m, n, k}) {
      if (dim > kMaxInt) return refuse("dimension", dim);
    }
    for (const qk_matrix_layout* l : {&lhs, &rhs, &out}) {
      if (l->leading_dim_stride > kMaxInt) {
        return refuse("leading dimension (elements between rows)",
                      l->leading_dim_stride);
      }
    }
  }

  // The plan (reference GetMatmulPlan, metal_blas.cc:245-287): a row-major
  // matrix is its storage, a column-major one the transpose of it.
  auto operand = [](const qk_matrix_layout& l) {
    qk::Operand o;
    o.ld = l.leading_dim_stride;
    o.batch_stride = l.batch_size > 1 ? l.batch_stride : 0;
    o.dtype = l.dtype;
    o.transpose = l.order == QK_COLUMN_MAJOR;
    return o;
  };
  auto* plan = new qk_gemm_plan;
  plan->p.m = m;
  plan->p.n = n;
  plan->p.k = k;
  plan->p.batch = batch;
  plan->p.alpha = static_cast<float>(cfg->alpha_re);
  plan->p.beta = static_cast<float>(cfg->beta);
  plan->p.a = operand(lhs);
  plan->p.b = operand(rhs);
  plan->p.d = operand(out);
  plan->p.act = epi.act;
  plan->swap = swap;
  plan->bias = epi.bias;
  plan->aux = epi.aux;
  plan->act = epi.act;
  plan->beta = cfg->beta;
  plan->choice = qk::ChooseGemmKernel(plan->p);
  *out_plan = plan;
  return QK_OK;
}

extern "C" void qk_gemm_plan_destroy(qk_gemm_plan* plan) { delete plan; }

extern "C" const char* qk_gemm_plan_describe(const qk_gemm_plan* plan) {
  thread_local std::string s;
  if (plan == nullptr) return "null plan";
  const qk::GemmProblem& p = plan->p;
  char buf[512];
  std::snprintf(
      buf, sizeof(buf),
      "m=%" PRId64 " n=%" PRId64 " k=%" PRId64 " batch=%" PRId64
      " alpha=%g beta=%g a={%s ld=%" PRId64 " bs=%" PRId64 "%s} b={%s ld=%" PRId64
      " bs=%" PRId64 "%s} d={%s ld=%" PRId64 " bs=%" PRId64
      "} swap=%d bias=%d aux=%d act=%d kernel=%s (if 16-byte aligned; "
      "chosen again from the buffers at execute)",
      p.m, p.n, p.k, p.batch, p.alpha, plan->beta, qk::DTypeName(p.a.dtype),
      p.a.ld, p.a.batch_stride, p.a.transpose ? " T" : "",
      qk::DTypeName(p.b.dtype), p.b.ld, p.b.batch_stride,
      p.b.transpose ? " T" : "", qk::DTypeName(p.d.dtype), p.d.ld,
      p.d.batch_stride, plan->swap ? 1 : 0, plan->bias ? 1 : 0,
      plan->aux ? 1 : 0, plan->act, plan->choice.name.c_str());
  s = buf;
  return s.c_str();
}

extern "C" qk_status qk_gemm_execute(const qk_gemm_plan* plan, void* stream,
                                     const qk_memory_args* args) {
  if (plan == nullptr || args == nullptr) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: null plan or memory args");
  }
  qk::GemmProblem p = plan->p;
  // ExecuteOnStream (reference metal_blas.cc:294-338): the operands are
  // exchanged for a column-major output; each must be bound.
  const void* a = plan->swap ? args->b : args->a;
  const void* b = plan->swap ? args->a : args->b;
  const uint64_t a_size = plan->swap ? args->b_size : args->a_size;
  const uint64_t b_size = plan->swap ? args->a_size : args->b_size;
  if (a == nullptr) return Fail(QK_INVALID_ARGUMENT, "qkern: operand A is null");
  if (b == nullptr) return Fail(QK_INVALID_ARGUMENT, "qkern: operand B is null");
  if (args->d == nullptr) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: operand D is null");
  }
  // Shape checks of RunSteelGemm (reference steel_gemm.cc:177-190).
  const int64_t a_cols = p.a.transpose ? p.m : p.k;
  const int64_t b_cols = p.b.transpose ? p.k : p.n;
  if ((p.k > 0 && ((p.m > 0 && p.a.ld < a_cols) ||
                   (p.n > 0 && p.b.ld < b_cols))) ||
      (p.m > 0 && p.d.ld < p.n)) {
    return Fail(QK_INVALID_ARGUMENT,
                std::string("qkern: leading dimension smaller than row "
                            "length: ") +
                    qk_gemm_plan_describe(plan));
  }
  if (p.m == 0 || p.n == 0 || p.batch == 0) return QK_OK;

  // Buffer extents (EpilogueBuffers, reference metal_blas.cc:340-378), for
  // D and aux always, and for A, B and C when their sizes are given.
  auto extent = [&](const qk::Operand& o, int64_t rows, int64_t cols) {
    const int64_t bs = p.batch > 1 ? o.batch_stride : 0;
    return static_cast<uint64_t>((p.batch - 1) * bs + (rows - 1) * o.ld + cols) *
           qk::DTypeSize(o.dtype);
  };
  const uint64_t d_extent = extent(p.d, p.m, p.n);
  if (args->d_size < d_extent) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: matmul: D has " + std::to_string(args->d_size) +
                    " bytes, need " + std::to_string(d_extent));
  }
  if (p.k > 0) {
    const uint64_t ae = p.a.transpose ? extent(p.a, p.k, p.m)
                                      : extent(p.a, p.m, p.k);
    const uint64_t be = p.b.transpose ? extent(p.b, p.n, p.k)
                                      : extent(p.b, p.k, p.n);
    if (a_size != 0 && a_size < ae) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: matmul: A has " + std::to_string(a_size) +
                      " bytes, need " + std::to_string(ae));
    }
    if (b_size != 0 && b_size < be) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: matmul: B has " + std::to_string(b_size) +
                      " bytes, need " + std::to_string(be));
    }
  }
  p.a.ptr = a;
  p.b.ptr = b;
  p.d.ptr = args->d;
  p.c = nullptr;
  if (plan->beta != 0.0) {
    // C shares D's layout (checked at plan creation); without C, D is
    // accumulated in place.
    p.c = args->c != nullptr ? args->c : args->d;
    if (args->c != nullptr && args->c_size != 0 && args->c_size < d_extent) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: matmul: C has " + std::to_string(args->c_size) +
                      " bytes, need " + std::to_string(d_extent));
    }
  }
  const int elem = qk::DTypeSize(p.d.dtype);
  if (plan->bias) {
    if (args->bias == nullptr ||
        args->bias_size < static_cast<uint64_t>(p.n) * elem) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: matmul epilogue: bias buffer (" +
                      std::to_string(args->bias_size) + " bytes) must hold " +
                      std::to_string(p.n) + " elements of " +
                      qk::DTypeName(p.d.dtype));
    }
    p.bias = args->bias;
  }
  if (plan->aux) {
    if (args->aux == nullptr || args->aux_size < d_extent) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: matmul epilogue: aux buffer (" +
                      std::to_string(args->aux_size) +
                      " bytes) smaller than the output (" +
                      std::to_string(d_extent) + " bytes)");
    }
    p.aux = args->aux;
  }
  if (qk_status s = qk::PreLaunch(); s != QK_OK) return s;
  return qk::LaunchGemm(p, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Typed-FFI style targets: argument checks.

namespace {

// Buffers hold at most 2^56 elements: element counts, byte counts and the
// products of two checked sizes below stay far from int64 overflow.
constexpr int64_t kMaxElements = int64_t{1} << 56;

// Element count of b, or -1 when it overflows kMaxElements. Dimensions are
// non-negative (CheckBuffer); a zero dimension gives 0 whatever the others.
int64_t CountElements(const qk_buffer& b) {
  int64_t n = 1;
  bool over = false;
  for (int i = 0; i < b.rank; ++i) {
    if (b.dims[i] == 0) return 0;
    if (__builtin_mul_overflow(n, b.dims[i], &n) || n > kMaxElements) {
      over = true;
      n = 1;
    }
  }
  return over ? -1 : n;
}

// Element count of a buffer CheckBuffer accepted (never overflows).
int64_t NumElements(const qk_buffer& b) { return CountElements(b); }

// a * b for sizes from accepted buffers; -1 when the product overflows
// kMaxElements (such a product never matches an accepted element count).
int64_t MulSizes(int64_t a, int64_t b) {
  int64_t r = 0;
  if (__builtin_mul_overflow(a, b, &r) || r > kMaxElements) return -1;
  return r;
}

std::string BufferString(const qk_buffer& b) {
  std::string s = std::string(qk::DTypeName(b.dtype)) + "[";
  for (int i = 0; i < b.rank; ++i) {
    if (i) s += ",";
    s += std::to_string(b.dims[i]);
  }
  return s + "]";
}

qk_status CheckBuffer(const qk_buffer* b, const char* name, bool allow_null) {
  if (b == nullptr) {
    if (allow_null) return QK_OK;
    return Fail(QK_INVALID_ARGUMENT, std::string("qkern: ") + name +
                                         " buffer descriptor is null");
  }
  if (b->rank < 1 || b->rank > QK_MAX_RANK) {
    return Fail(QK_INVALID_ARGUMENT, std::string("qkern: ") + name +
                                         " has rank " +
                                         std::to_string(b->rank) +
                                         " (1 to 6 supported)");
  }
  for (int i = 0; i < b->rank; ++i) {
    if (b->dims[i] < 0) {
      return Fail(QK_INVALID_ARGUMENT, std::string("qkern: ") + name +
                                           " has a negative dimension");
    }
  }
  if (CountElements(*b) < 0) {
    return Fail(QK_INVALID_ARGUMENT,
                std::string("qkern: ") + name + " has more than 2^56 elements");
  }
  if (b->data == nullptr && NumElements(*b) > 0) {
    return Fail(QK_INVALID_ARGUMENT,
                std::string("qkern: ") + name + " data is null");
  }
  return QK_OK;
}

// Shared checks of qk$qmatvec and qk$dequantize: codes [N, ...] whose
// element count matches N*K in the packing; scales/biases [N, K/g(, 1)].
qk_status CheckQuant(const qk_buffer* codes, const qk_buffer* scales,
                     const qk_buffer* biases, const qk_quant_attrs* attrs,
                     int64_t k, qk::QuantProblem* q) {
  if (attrs == nullptr) return Fail(QK_INVALID_ARGUMENT, "qkern: null attrs");
  if (qk_status s = CheckBuffer(codes, "codes", false); s != QK_OK) return s;
  if (qk_status s = CheckBuffer(scales, "scales", false); s != QK_OK) return s;
  if (qk_status s = CheckBuffer(biases, "biases", true); s != QK_OK) return s;
  const int g = attrs->group_size;
  if (g != 32 && g != 64 && g != 128) {
    return Fail(QK_UNIMPLEMENTED, "qkern: quantization group size " +
                                      std::to_string(g) +
                                      " is not supported (32, 64 or 128)");
  }
  int want_bits = 0, want_dtype = 0;
  int64_t codes_per_elem = 1;
  switch (attrs->packing) {
    case QK_PACK_U32X8:
      want_bits = 4, want_dtype = QK_U32, codes_per_elem = 8;
      break;
    case QK_PACK_BYTE_HALFSPLIT:
      want_bits = 4, want_dtype = QK_U8, codes_per_elem = 2;
      break;
    case QK_PACK_U8:
      want_bits = 8, want_dtype = QK_U8;
      break;
    case QK_PACK_S8_SYM:
      want_bits = 8, want_dtype = QK_S8;
      break;
    default:
      return Fail(QK_UNIMPLEMENTED, "qkern: unknown packing " +
                                        std::to_string(attrs->packing));
  }
  if (attrs->bits != want_bits) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: packing " + std::to_string(attrs->packing) +
                    " holds " + std::to_string(want_bits) + "-bit codes, not " +
                    std::to_string(attrs->bits));
  }
  if (codes->dtype != want_dtype) {
    return Fail(QK_INVALID_ARGUMENT,
                std::string("qkern: codes must be ") +
                    qk::DTypeName(want_dtype) + " for this packing, got " +
                    BufferString(*codes));
  }
  if (attrs->packing == QK_PACK_S8_SYM && attrs->has_bias) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: symmetric int8 codes take no offset (has_bias must "
                "be 0)");
  }
  const int64_t n = codes->dims[0];
  if (k % g != 0) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: K=" + std::to_string(k) +
                    " is not a multiple of the group size " +
                    std::to_string(g));
  }
  if (codes->rank < 2 ||
      NumElements(*codes) * codes_per_elem != MulSizes(n, k)) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: codes " + BufferString(*codes) + " do not hold " +
                    std::to_string(n) + "x" + std::to_string(k) +
                    " codes in this packing");
  }
  if (attrs->packing == QK_PACK_BYTE_HALFSPLIT &&
      !(codes->rank == 3 && codes->dims[1] == k / g &&
        codes->dims[2] == g / 2)) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: half-split int4 codes must be [N, K/g, g/2], got " +
                    BufferString(*codes));
  }
  auto check_sb = [&](const qk_buffer* b, const char* name) -> qk_status {
    if (!IsFloat(b->dtype) || b->dims[0] != n ||
        NumElements(*b) != MulSizes(n, k / g)) {
      return Fail(QK_INVALID_ARGUMENT,
                  std::string("qkern: ") + name + " must be float [N, K/g] = [" +
                      std::to_string(n) + ", " + std::to_string(k / g) +
                      "], got " + BufferString(*b));
    }
    return QK_OK;
  };
  if (qk_status s = check_sb(scales, "scales"); s != QK_OK) return s;
  if (attrs->has_bias) {
    if (biases == nullptr) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: has_bias is set but biases is null");
    }
    if (qk_status s = check_sb(biases, "biases"); s != QK_OK) return s;
  }
  q->n = n;
  q->k = k;
  q->bits = attrs->bits;
  q->group = g;
  q->packing = attrs->packing;
  q->has_bias = attrs->has_bias != 0;
  q->codes = codes->data;
  q->scales = scales->data;
  q->scale_dtype = scales->dtype;
  q->biases = attrs->has_bias ? biases->data : nullptr;
  q->bias_dtype = attrs->has_bias ? biases->dtype : QK_F32;
  return QK_OK;
}

}  // namespace

extern "C" qk_status qk_qmatvec(void* stream, const qk_buffer* x,
                                const qk_buffer* codes,
                                const qk_buffer* scales,
                                const qk_buffer* biases, qk_buffer* y,
                                const qk_quant_attrs* attrs) {
  if (qk_status s = CheckBuffer(x, "x", false); s != QK_OK) return s;
  if (qk_status s = CheckBuffer(y, "y", false); s != QK_OK) return s;
  if (!IsFloat(x->dtype)) {
    return Fail(QK_UNIMPLEMENTED, "qkern: qmatvec input must be f32, f16 or "
                                  "bf16, got " +
                                      BufferString(*x));
  }
  const int64_t k = x->dims[x->rank - 1];
  qk::QuantProblem q;
  if (qk_status s = CheckQuant(codes, scales, biases, attrs, k, &q);
      s != QK_OK) {
    return s;
  }
  const int64_t m = k == 0 ? 0 : NumElements(*x) / k;
  if (y->dtype != x->dtype || y->dims[y->rank - 1] != q.n ||
      NumElements(*y) != MulSizes(m, q.n)) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: qmatvec output must be " +
                    std::string(qk::DTypeName(x->dtype)) + " [..., " +
                    std::to_string(q.n) + "] with x's leading dimensions, got " +
                    BufferString(*y));
  }
  if (k == 0 && q.n > 0) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: qmatvec with K = 0");
  }
  q.m = m;
  q.x = x->data;
  q.x_dtype = x->dtype;
  q.y = y->data;
  q.y_dtype = y->dtype;
  if (m == 0 || q.n == 0) return QK_OK;
  if (qk_status s = qk::PreLaunch(); s != QK_OK) return s;
  return qk::LaunchQMatvec(q, static_cast<hipStream_t>(stream));
}

extern "C" qk_status qk_dequantize(void* stream, const qk_buffer* codes,
                                   const qk_buffer* scales,
                                   const qk_buffer* biases, qk_buffer* w,
                                   const qk_quant_attrs* attrs) {
  if (qk_status s = CheckBuffer(w, "w", false); s != QK_OK) return s;
  if (!IsFloat(w->dtype) || w->rank != 2) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: dequantize output must be float [N, K], got " +
                    BufferString(*w));
  }
  qk::QuantProblem q;
  if (qk_status s = CheckQuant(codes, scales, biases, attrs, w->dims[1], &q);
      s != QK_OK) {
    return s;
  }
  if (w->dims[0] != q.n) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: dequantize output has " +
                                         std::to_string(w->dims[0]) +
                                         " rows, codes have " +
                                         std::to_string(q.n));
  }
  q.y = w->data;
  q.y_dtype = w->dtype;
  if (q.n == 0 || q.k == 0) return QK_OK;
  if (qk_status s = qk::PreLaunch(); s != QK_OK) return s;
  return qk::LaunchDequantize(q, static_cast<hipStream_t>(stream));
}

extern "C" qk_status qk_quantize(void* stream, const qk_buffer* w,
                                 qk_buffer* codes, qk_buffer* scales,
                                 qk_buffer* biases,
                                 const qk_quant_attrs* attrs) {
  if (qk_status s = CheckBuffer(w, "w", false); s != QK_OK) return s;
  if (!IsFloat(w->dtype) || w->rank != 2) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: quantize input must be float [N, K], got " +
                    BufferString(*w));
  }
  qk::QuantProblem q;
  if (qk_status s = CheckQuant(codes, scales, biases, attrs, w->dims[1], &q);
      s != QK_OK) {
    return s;
  }
  if (attrs->packing == QK_PACK_U8) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: quantize makes int4 affine (u32x8, byte_halfsplit) or "
                "symmetric int8 (s8_sym) codes, as the reference's quantizers "
                "do; there is no 8-bit affine quantizer");
  }
  const bool int4 = attrs->bits == 4;
  if (int4 && (!attrs->has_bias || biases == nullptr)) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: int4 quantization writes offsets: pass biases and "
                "has_bias = 1");
  }
  if (w->dims[0] != q.n) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: quantize input has " + std::to_string(w->dims[0]) +
                    " rows, codes have " + std::to_string(q.n));
  }
  if (int4 && biases->dtype != scales->dtype) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: quantize writes scales and offsets of one dtype, got " +
                    BufferString(*scales) + " and " + BufferString(*biases));
  }
  if (reinterpret_cast<uintptr_t>(w->data) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(codes->data) % 4 != 0) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: quantize needs 16-byte aligned weights and 4-byte "
                "aligned codes");
  }
  if (q.n == 0 || q.k == 0) return QK_OK;
  if (qk_status s = qk::PreLaunch(); s != QK_OK) return s;
  return qk::LaunchQuantize(q, w->data, w->dtype,
                            static_cast<hipStream_t>(stream));
}

extern "C" qk_status qk_embed(void* stream, const qk_buffer* tokens,
                              const qk_buffer* table, const qk_buffer* scales,
                              const qk_buffer* biases, qk_buffer* out,
                              const qk_quant_attrs* attrs) {
  if (qk_status s = CheckBuffer(tokens, "tokens", false); s != QK_OK) return s;
  if (qk_status s = CheckBuffer(table, "table", false); s != QK_OK) return s;
  if (qk_status s = CheckBuffer(out, "out", false); s != QK_OK) return s;
  if (tokens->dtype != QK_S32 && tokens->dtype != QK_U32) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: embedding tokens must be int32, got " +
                    BufferString(*tokens));
  }
  // out = tokens' shape + [K]
  bool shape_ok = out->rank == tokens->rank + 1 && IsFloat(out->dtype);
  for (int i = 0; shape_ok && i < tokens->rank; ++i)
    shape_ok = out->dims[i] == tokens->dims[i];
  if (!shape_ok) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: embedding output must be float [" +
                    std::string("tokens..., K], got ") + BufferString(*out) +
                    " for tokens " + BufferString(*tokens));
  }
  const int64_t t = NumElements(*tokens);
  const int64_t k = out->dims[out->rank - 1];
  if (reinterpret_cast<uintptr_t>(tokens->data) % 4 != 0) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: tokens must be 4-byte aligned");
  }
  if (scales == nullptr) {
    // A dense table [V, K]: a plain row gather in the table's type.
    if (table->rank != 2 || table->dtype != out->dtype ||
        table->dims[1] != k) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: dense embedding table must be [V, " +
                      std::to_string(k) + "] of the output type, got " +
                      BufferString(*table));
    }
    if (t == 0 || k == 0) return QK_OK;
    if (table->dims[0] == 0) {
      return Fail(QK_INVALID_ARGUMENT, "qkern: empty embedding table");
    }
    if (qk_status s = qk::PreLaunch(); s != QK_OK) return s;
    return qk::LaunchRowGather(table->data, table->dims[0], k, k,
                               qk::DTypeSize(out->dtype), tokens->data, t,
                               out->data, static_cast<hipStream_t>(stream));
  }
  qk::QuantProblem q;
  if (qk_status s = CheckQuant(table, scales, biases, attrs, k, &q);
      s != QK_OK) {
    return s;
  }
  if (t == 0 || q.k == 0) return QK_OK;
  if (q.n == 0) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: empty embedding table");
  }
  q.y = out->data;
  q.y_dtype = out->dtype;
  q.rows = tokens->data;
  q.rows_n = t;
  if (qk_status s = qk::PreLaunch(); s != QK_OK) return s;
  return qk::LaunchDequantize(q, static_cast<hipStream_t>(stream));
}

extern "C" qk_status qk_rownorm(void* stream, const qk_buffer* x,
                                const qk_buffer* gain, const qk_buffer* beta,
                                qk_buffer* y, const qk_rownorm_attrs* attrs) {
  if (attrs == nullptr) return Fail(QK_INVALID_ARGUMENT, "qkern: null attrs");
  if (qk_status s = CheckBuffer(x, "x", false); s != QK_OK) return s;
  if (qk_status s = CheckBuffer(y, "y", false); s != QK_OK) return s;
  if (attrs->kind < QK_ROWNORM_RMS || attrs->kind > QK_ROWNORM_SOFTMAX) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: unknown rownorm kind " + std::to_string(attrs->kind));
  }
  if (!IsFloat(x->dtype)) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: rownorm input must be f32, f16 or bf16, got " +
                    BufferString(*x));
  }
  if (y->dtype != x->dtype || NumElements(*y) != NumElements(*x) ||
      y->dims[y->rank - 1] != x->dims[x->rank - 1]) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: rownorm output " +
                                         BufferString(*y) +
                                         " must match the input " +
                                         BufferString(*x));
  }
  const int64_t n = x->dims[x->rank - 1];
  qk::RownormProblem r;
  r.n = n;
  r.rows = n == 0 ? 0 : NumElements(*x) / n;
  r.kind = attrs->kind;
  r.eps = attrs->eps;
  r.x = x->data;
  r.y = y->data;
  r.dtype = x->dtype;
  auto vec = [&](const qk_buffer* v, const char* name, bool want,
                 const void** ptr, int* dtype) -> qk_status {
    if (!want) return QK_OK;
    if (attrs->kind == QK_ROWNORM_SOFTMAX) {
      return Fail(QK_INVALID_ARGUMENT,
                  std::string("qkern: softmax takes no ") + name);
    }
    if (v == nullptr) {
      return Fail(QK_INVALID_ARGUMENT,
                  std::string("qkern: rownorm ") + name + " is null");
    }
    if (qk_status s = CheckBuffer(v, name, false); s != QK_OK) return s;
    if (!IsFloat(v->dtype) || NumElements(*v) != n) {
      return Fail(QK_INVALID_ARGUMENT, std::string("qkern: rownorm ") + name +
                                           " must be float [" +
                                           std::to_string(n) + "], got " +
                                           BufferString(*v));
    }
    *ptr = v->data;
    *dtype = v->dtype;
    return QK_OK;
  };
  if (qk_status s = vec(gain, "gain", attrs->has_gain != 0, &r.gain,
                        &r.gain_dtype);
      s != QK_OK) {
    return s;
  }
  if (attrs->has_beta && attrs->kind != QK_ROWNORM_LAYER) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: only layer norm takes a beta (has_beta)");
  }
  if (qk_status s = vec(beta, "beta", attrs->has_beta != 0, &r.beta,
                        &r.beta_dtype);
      s != QK_OK) {
    return s;
  }
  if (r.rows == 0 || r.n == 0) return QK_OK;
  if (qk_status s = qk::PreLaunch(); s != QK_OK) return s;
  return qk::LaunchRownorm(r, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// qk$decode_attention.

namespace {

// Checks of qk$decode_attention's q and key cache and attributes; fills the
// problem's shapes and plan.
qk_status CheckAttentionShapes(const qk_buffer* q, const qk_buffer* k,
                               const qk_attention_attrs* attrs,
                               qk::AttentionProblem* p) {
  if (attrs == nullptr) return Fail(QK_INVALID_ARGUMENT, "qkern: null attrs");
  if (qk_status s = CheckBuffer(q, "q", false); s != QK_OK) return s;
  if (qk_status s = CheckBuffer(k, "k_cache", false); s != QK_OK) return s;
  // q [B, KV, G, D] or the reference's [B, 1, KV, G, D]
  const bool q5 = q->rank == 5 && q->dims[1] == 1;
  if (q->rank != 4 && !q5) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: decode attention q must be [B, KV, G, D] or "
                "[B, 1, KV, G, D], got " +
                    BufferString(*q));
  }
  const int64_t* qd = q5 ? q->dims + 1 : q->dims;
  p->b = q->dims[0];
  p->kv = qd[1];
  p->g = qd[2];
  p->d = qd[3];
  if (q->dtype != QK_BF16 && q->dtype != QK_F16) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: decode attention takes bf16 or f16 q and caches, "
                "got q " +
                    BufferString(*q));
  }
  if (p->d != 64 && p->d != 128) {
    return Fail(QK_UNIMPLEMENTED, "qkern: decode attention head dim " +
                                      std::to_string(p->d) +
                                      " is not supported (64 or 128)");
  }
  if (p->g < 1 || p->g > 16) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: decode attention with " + std::to_string(p->g) +
                    " query heads per KV head is not supported (1 to 16)");
  }
  if (k->rank != 4 || k->dtype != q->dtype || k->dims[0] != p->b ||
      k->dims[1] != p->kv || k->dims[3] != p->d) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: k_cache must be " +
                    std::string(qk::DTypeName(q->dtype)) + " [" +
                    std::to_string(p->b) + ", " + std::to_string(p->kv) +
                    ", Smax, " + std::to_string(p->d) + "], got " +
                    BufferString(*k));
  }
  p->smax = k->dims[2];
  if (p->smax % 8 != 0 || p->smax > (int64_t{1} << 22)) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: decode attention needs a cache length that is a "
                "multiple of 8 and at most 2^22, got " +
                    std::to_string(p->smax));
  }
  const int64_t window = attrs->window == 0 ? p->smax : attrs->window;
  if (window < 0 || window > p->smax) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: attention window " + std::to_string(attrs->window) +
                    " outside the cache length " + std::to_string(p->smax));
  }
  p->window = window;
  p->scale = attrs->scale;
  p->dtype = q->dtype;
  if (p->b > 0 && p->kv > 0 && p->window > 0) qk::PlanAttention(p);
  return QK_OK;
}

}  // namespace

extern "C" qk_status qk_decode_attention_workspace_size(
    const qk_buffer* q, const qk_buffer* k_cache,
    const qk_attention_attrs* attrs, uint64_t* bytes) {
  if (bytes == nullptr) return Fail(QK_INVALID_ARGUMENT, "qkern: null bytes");
  *bytes = 0;
  qk::AttentionProblem p;
  if (qk_status s = CheckAttentionShapes(q, k_cache, attrs, &p); s != QK_OK)
    return s;
  *bytes = p.workspace_bytes;
  return QK_OK;
}

namespace {

// Every check of qk$decode_attention except the workspace's; fills p.
qk_status CheckAttention(const qk_buffer* q, const qk_buffer* k_cache,
                         const qk_buffer* v_cache, const qk_buffer* position,
                         const qk_buffer* out,
                         const qk_attention_attrs* attrs,
                         qk::AttentionProblem* pp) {
  qk::AttentionProblem& p = *pp;
  if (qk_status s = CheckAttentionShapes(q, k_cache, attrs, &p); s != QK_OK)
    return s;
  if (qk_status s = CheckBuffer(v_cache, "v_cache", false); s != QK_OK)
    return s;
  if (qk_status s = CheckBuffer(out, "out", false); s != QK_OK) return s;
  if (v_cache->rank != 4 || v_cache->dtype != p.dtype ||
      v_cache->dims[0] != p.b || v_cache->dims[1] != p.kv ||
      v_cache->dims[2] != p.d || v_cache->dims[3] != p.smax) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: v_cache must be " +
                    std::string(qk::DTypeName(p.dtype)) + " [" +
                    std::to_string(p.b) + ", " + std::to_string(p.kv) +
                    ", " + std::to_string(p.d) + ", " +
                    std::to_string(p.smax) + "], got " +
                    BufferString(*v_cache));
  }
  bool same = out->rank == q->rank && out->dtype == p.dtype;
  for (int i = 0; same && i < q->rank; ++i) same = out->dims[i] == q->dims[i];
  if (!same) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: decode attention output " +
                                         BufferString(*out) +
                                         " must match q " + BufferString(*q));
  }
  if (position == nullptr || position->rank > 1 ||
      (position->rank == 1 && position->dims[0] != 1) ||
      (position->dtype != QK_S32 && position->dtype != QK_U32) ||
      position->data == nullptr) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: decode attention position must be one int32 on the "
                "device");
  }
  if (p.b == 0 || p.kv == 0) return QK_OK;
  if (p.window == 0) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: decode attention over an empty cache window");
  }
  for (const void* ptr : {static_cast<const void*>(q->data),
                          static_cast<const void*>(k_cache->data),
                          static_cast<const void*>(v_cache->data),
                          static_cast<const void*>(out->data)}) {
    if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0) {
      return Fail(QK_INVALID_ARGUMENT,
                  "qkern: decode attention buffers must be 16-byte aligned");
    }
  }
  p.q = q->data;
  p.k = k_cache->data;
  p.v = v_cache->data;
  p.pos = position->data;
  p.out = out->data;
  return QK_OK;
}

}  // namespace

extern "C" qk_status qk_decode_attention(
    void* stream, const qk_buffer* q, const qk_buffer* k_cache,
    const qk_buffer* v_cache, const qk_buffer* position, qk_buffer* out,
    const qk_attention_attrs* attrs, void* workspace,
    uint64_t workspace_bytes) {
  qk::AttentionProblem p;
  if (qk_status s =
          CheckAttention(q, k_cache, v_cache, position, out, attrs, &p);
      s != QK_OK)
    return s;
  if (p.b == 0 || p.kv == 0) return QK_OK;
  if (workspace == nullptr || workspace_bytes < p.workspace_bytes) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: decode attention needs a workspace of " +
                    std::to_string(p.workspace_bytes) + " bytes, got " +
                    std::to_string(workspace_bytes));
  }
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: decode attention workspace must be 16-byte aligned");
  }
  if (qk_status s = qk::PreLaunch(); s != QK_OK) return s;
  return qk::LaunchAttention(p, workspace, static_cast<hipStream_t>(stream));
}

extern "C" qk_status qk_decode_attention_noalloc(
    void* stream, const qk_buffer* q, const qk_buffer* k_cache,
    const qk_buffer* v_cache, const qk_buffer* position, qk_buffer* out,
    const qk_attention_attrs* attrs) {
  qk::AttentionProblem p;
  if (qk_status s =
          CheckAttention(q, k_cache, v_cache, position, out, attrs, &p);
      s != QK_OK)
    return s;
  if (p.b == 0 || p.kv == 0) return QK_OK;
  if (p.workspace_bytes > qk::kAttentionScratchBytes) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: decode attention at these shapes needs " +
                    std::to_string(p.workspace_bytes) +
                    " bytes of partials, more than the fixed scratch of " +
                    std::to_string(qk::kAttentionScratchBytes) +
                    " bytes; call qk_decode_attention with a workspace");
  }
  if (qk_status s = qk::PreLaunch(); s != QK_OK) return s;
  void* scratch = nullptr;
  if (qk_status s = qk::AttentionScratch(&scratch); s != QK_OK) return s;
  return qk::LaunchAttention(p, scratch, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Status entry points.

extern "C" const char* qk_last_error_message(void) {
  return qk::g_last_error.c_str();
}

extern "C" qk_status qk_device_error(void) {
  // Kernels that gave up a bounded wait (their outputs are NaN) set a bit
  // in the device status word; it becomes the sticky error here.
  if (qk::g_sticky_status.load() == QK_OK &&
      (qk::ReadDeviceStatusWords(false) & 1u) != 0u) {
    qk::SetSticky(QK_INTERNAL,
                  "a quantized matmul kernel gave up waiting between its "
                  "producer and consumer waves (its outputs were set to "
                  "NaN)");
  }
  const int s = qk::g_sticky_status.load();
  if (s != QK_OK) {
    std::lock_guard<std::mutex> lock(qk::g_sticky_mu);
    qk::g_last_error = "qkern: " + qk::g_sticky_message;
  }
  return static_cast<qk_status>(s);
}

extern "C" void qk_reset_device_error(void) {
  {
    std::lock_guard<std::mutex> lock(qk::g_sticky_mu);
    qk::g_sticky_message.clear();
    qk::g_sticky_status.store(QK_OK);
  }
  (void)qk::ReadDeviceStatusWords(true);
  qk::g_launches.store(0);
  qk::ReadFailEnv();
  qk::g_last_error.clear();
}

extern "C" const char* qk_version(void) { return "qkern 0.1 gfx950"; }
