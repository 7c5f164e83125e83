// Row-wise RMSNorm, LayerNorm and softmax for gfx950, one pass over HBM.
//
// Replaces the XLA reduction fusions behind the reference's rms_norm
// (examples/llm/qwen3.py:294-297), jax.nn.softmax (qwen3.py:325,330; two
// fusions on the reference) and the benchmark's layernorm
// (bench/jax_bench.py:44-46). Semantics, in f32 with one rounding at the
// end:
//   RMS:     y = x * rsqrt(sum(x^2)/n + eps) * gain
//   LAYER:   mu = sum(x)/n, var = sum((x-mu)^2)/n,
//            y = (x - mu) / sqrt(var + eps) * gain + beta
//   SOFTMAX: y = exp(x - max) / sum(exp(x - max))
//
// Each row is read once into registers with 16-byte loads (a workgroup of
// 256 threads per long row, one wavefront per short row), reduced with
// wavefront butterflies plus one LDS exchange, and written once. Rows too
// long for registers take a looping kernel that reads them again.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct RnArgs {
  const void* x;
  void* y;
  const void* gain;
  const void* beta;
  long long rows;
  int n;
  int kind;
  float eps;
  int gdt, bdt;
  int has_gain, has_beta;
};

constexpr int kThreads = 256;

// Sum over the TPR threads that share a row (TPR = 64 or 256).
template <int TPR>
__device__ __forceinline__ float row_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (TPR == 64) {
    return v;
  } else {
    const int wave = threadIdx.x >> 6;
    __syncthreads();  // red may still be read by a previous reduction
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < TPR / 64; ++w) s += red[w];
    return s;
  }
}
template <int TPR>
__device__ __forceinline__ float row_max(float v, float* red) {
  v = wave_max(v);
  if constexpr (TPR == 64) {
    return v;
  } else {
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < TPR / 64; ++w) s = fmaxf(s, red[w]);
    return s;
  }
}

// V elements per load (16 bytes, or 1 when rows are not 16-byte aligned),
// VPT loads per thread, TPR threads per row.
template <typename T, int V, int VPT, int TPR>
__global__ __launch_bounds__(kThreads) void rownorm_kernel(RnArgs a) {
  __shared__ float red[kThreads / 64];
  constexpr int RPB = kThreads / TPR;  // rows per block
  const int t = threadIdx.x % TPR;
  const long long row = static_cast<long long>(blockIdx.x) * RPB +
                        threadIdx.x / TPR;
  // TPR == 256: the whole block shares the row, so this exit is uniform.
  if (row >= a.rows) return;
  const T* xr = static_cast<const T*>(a.x) + row * a.n;
  T* yr = static_cast<T*>(a.y) + row * a.n;
  const int n = a.n;

  float v[VPT][V];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int base = (t + i * TPR) * V;
    if constexpr (V > 1) {
      if (base < n) {
        union {
          u32x4 u;
          T e[V];
        } q;
        q.u = *reinterpret_cast<const u32x4*>(xr + base);
#pragma unroll
        for (int e = 0; e < V; ++e) v[i][e] = to_f32(q.e[e]);
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) v[i][e] = 0.f;
      }
    } else {
      v[i][0] = base < n ? to_f32(xr[base]) : 0.f;
    }
  }
  auto valid = [&](int i) { return (t + i * TPR) * V < n; };

  float scale = 1.f, shift = 0.f;  // y = (x - shift) * scale (then gain)
  if (a.kind == QK_ROWNORM_RMS) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int e = 0; e < V; ++e) ss += v[i][e] * v[i][e];
    ss = row_sum<TPR>(ss, red);
    scale = rsqrtf(ss / static_cast<float>(n) + a.eps);
  } else if (a.kind == QK_ROWNORM_LAYER) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int e = 0; e < V; ++e) s += v[i][e];
    const float mu = row_sum<TPR>(s, red) / static_cast<float>(n);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (valid(i))
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float d = v[i][e] - mu;
          q += d * d;
        }
    const float var = row_sum<TPR>(q, red) / static_cast<float>(n);
    shift = mu;
    scale = 1.0f / sqrtf(var + a.eps);
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (valid(i))
#pragma unroll
        for (int e = 0; e < V; ++e) mx = fmaxf(mx, v[i][e]);
    mx = row_max<TPR>(mx, red);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (valid(i))
#pragma unroll
        for (int e = 0; e < V; ++e) {
          v[i][e] = expf(v[i][e] - mx);
          s += v[i][e];
        }
    s = row_sum<TPR>(s, red);
    shift = 0.f;
    scale = s;  // divided below
  }

#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    if (!valid(i)) continue;
    const int base = (t + i * TPR) * V;
    float out[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      float o;
      if (a.kind == QK_ROWNORM_SOFTMAX) {
        o = v[i][e] / scale;
      } else {
        o = (v[i][e] - shift) * scale;
        if (a.has_gain) o *= load_any(a.gain, base + e, a.gdt);
        if (a.has_beta) o += load_any(a.beta, base + e, a.bdt);
      }
      out[e] = o;
    }
    if constexpr (V > 1) {
      union {
        u32x4 u;
        T e[V];
      } q;
#pragma unroll
      for (int e = 0; e < V; ++e) q.e[e] = from_f32<T>(out[e]);
      *reinterpret_cast<u32x4*>(yr + base) = q.u;
    } else {
      yr[base] = from_f32<T>(out[0]);
    }
  }
}

// Rows longer than the register kernels take: one block per row, reading
// the row once per statistic.
template <typename T>
__global__ __launch_bounds__(kThreads) void rownorm_long_kernel(RnArgs a) {
  __shared__ float red[kThreads / 64];
  const long long row = blockIdx.x;
  const T* xr = static_cast<const T*>(a.x) + row * a.n;
  T* yr = static_cast<T*>(a.y) + row * a.n;
  const int n = a.n;
  float scale = 1.f, shift = 0.f;
  if (a.kind == QK_ROWNORM_RMS) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kThreads) {
      const float x = to_f32(xr[i]);
      ss += x * x;
    }
    ss = row_sum<kThreads>(ss, red);
    scale = rsqrtf(ss / static_cast<float>(n) + a.eps);
  } else if (a.kind == QK_ROWNORM_LAYER) {
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += kThreads) s += to_f32(xr[i]);
    const float mu = row_sum<kThreads>(s, red) / static_cast<float>(n);
    float q = 0.f;
    for (int i = threadIdx.x; i < n; i += kThreads) {
      const float d = to_f32(xr[i]) - mu;
      q += d * d;
    }
    const float var = row_sum<kThreads>(q, red) / static_cast<float>(n);
    shift = mu;
    scale = 1.0f / sqrtf(var + a.eps);
  } else {
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += kThreads)
      mx = fmaxf(mx, to_f32(xr[i]));
    mx = row_max<kThreads>(mx, red);
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += kThreads)
      s += expf(to_f32(xr[i]) - mx);
    s = row_sum<kThreads>(s, red);
    for (int i = threadIdx.x; i < n; i += kThreads)
      yr[i] = from_f32<T>(expf(to_f32(xr[i]) - mx) / s);
    return;
  }
  for (int i = threadIdx.x; i < n; i += kThreads) {
    float o = (to_f32(xr[i]) - shift) * scale;
    if (a.has_gain) o *= load_any(a.gain, i, a.gdt);
    if (a.has_beta) o += load_any(a.beta, i, a.bdt);
    yr[i] = from_f32<T>(o);
  }
}

template <typename T, int V, int TPR>
qk_status LaunchVpt(const RnArgs& a, hipStream_t st) {
  const int per = TPR * V;  // elements per VPT step
  const long long rpb = kThreads / TPR;
  dim3 grid(static_cast<unsigned>((a.rows + rpb - 1) / rpb)), block(kThreads);
  if (a.n <= per)
    rownorm_kernel<T, V, 1, TPR><<<grid, block, 0, st>>>(a);
  else if (a.n <= 2 * per)
    rownorm_kernel<T, V, 2, TPR><<<grid, block, 0, st>>>(a);
  else if (a.n <= 4 * per)
    rownorm_kernel<T, V, 4, TPR><<<grid, block, 0, st>>>(a);
  else if (a.n <= 8 * per)
    rownorm_kernel<T, V, 8, TPR><<<grid, block, 0, st>>>(a);
  else
    rownorm_kernel<T, V, 16, TPR><<<grid, block, 0, st>>>(a);
  return PostLaunch("rownorm");
}

template <typename T>
qk_status LaunchTyped(const RnArgs& a, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const bool aligned = (reinterpret_cast<uintptr_t>(a.x) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) &&
                       (static_cast<long long>(a.n) * sizeof(T)) % 16 == 0;
  if (aligned) {
    if (a.n <= 64 * V * 4) return LaunchVpt<T, V, 64>(a, st);
    if (a.n <= kThreads * V * 16) return LaunchVpt<T, V, kThreads>(a, st);
  } else {
    if (a.n <= 64 * 4) return LaunchVpt<T, 1, 64>(a, st);
    if (a.n <= kThreads * 16) return LaunchVpt<T, 1, kThreads>(a, st);
  }
  if (a.rows > 0x7fffffff) {
    return Fail(QK_UNIMPLEMENTED, "qkern: rownorm has too many rows");
  }
  rownorm_long_kernel<T><<<dim3(static_cast<unsigned>(a.rows)), kThreads, 0,
                           st>>>(a);
  return PostLaunch("rownorm_long");
}

}  // namespace

qk_status LaunchRownorm(const RownormProblem& p, hipStream_t stream) {
  if (p.n > 0x7fffffff) {
    return Fail(QK_UNIMPLEMENTED, "qkern: rownorm row longer than 2^31");
  }
  if (p.rows > 0x7fffffff) {
    return Fail(QK_UNIMPLEMENTED, "qkern: rownorm has too many rows");
  }
  RnArgs a;
  a.x = p.x;
  a.y = p.y;
  a.gain = p.gain;
  a.beta = p.beta;
  a.rows = p.rows;
  a.n = static_cast<int>(p.n);
  a.kind = p.kind;
  a.eps = p.eps;
  a.gdt = p.gain_dtype;
  a.bdt = p.beta_dtype;
  a.has_gain = p.gain != nullptr;
  a.has_beta = p.beta != nullptr;
  switch (p.dtype) {
    case QK_BF16:
      return LaunchTyped<bf16>(a, stream);
    case QK_F16:
      return LaunchTyped<f16>(a, stream);
    default:
      return LaunchTyped<float>(a, stream);
  }
}

}  // namespace qk
