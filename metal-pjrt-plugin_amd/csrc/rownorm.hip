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
//   SOFTMAX: y = exp(x - max) * (1 / sum(exp(x - max)))
//
// Each row is read once into registers with 16-byte loads, reduced with
// wavefront butterflies (plus one LDS exchange when four waves share a
// row), and written once with 16-byte stores. Rows up to 16 vectors per
// lane of one wavefront take one wavefront each (no barriers); longer rows
// take a 256-thread workgroup; rows too long for registers take a looping
// kernel that reads them again. The kind is a template parameter; gain and
// beta types are chosen per 16-byte vector (a uniform branch).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

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
  float eps;
  int gdt, bdt;
  int has_gain, has_beta;
};

constexpr int kThreads = 256;

// Sum over the TPR threads that share a row (TPR = 64 or 256).
template <int TPR>
__device__ __forceinline__ float row_sum(float v, float* red) {
  if constexpr (TPR == 64) {
    return wave_sum_dpp(v);
  } else {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();  // red may still be read by a previous reduction
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
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
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  }
}

// V consecutive elements starting at element i of a float vector of type
// dtype (qk_dtype), as f32. vec: 16-byte aligned loads are allowed.
template <int V>
__device__ __forceinline__ void load_param(const void* p, int dtype, int i,
                                           bool vec, float* out) {
  if (vec && V > 1) {
    if (dtype == QK_F32) {
#pragma unroll
      for (int h = 0; h < V / 4; ++h) {
        const u32x4 q = *reinterpret_cast<const u32x4*>(
            static_cast<const float*>(p) + i + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) out[4 * h + e] = __uint_as_float(q[e]);
      }
      return;
    }
    if (V % 8 == 0) {
#pragma unroll
      for (int h = 0; h < V / 8; ++h) {
        const u32x4 q = *reinterpret_cast<const u32x4*>(
            static_cast<const uint16_t*>(p) + i + 8 * h);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t bits = (q[e / 2] >> (16 * (e & 1))) & 0xffffu;
          out[8 * h + e] =
              dtype == QK_BF16
                  ? __uint_as_float(bits << 16)
                  : static_cast<float>(__builtin_bit_cast(f16,
                                                          static_cast<uint16_t>(bits)));
        }
      }
      return;
    }
  }
#pragma unroll
  for (int e = 0; e < V; ++e) out[e] = load_any(p, i + e, dtype);
}

// V elements per access (16 bytes, or 1 when rows are not 16-byte
// aligned), VPT accesses per thread, TPR threads per row.
template <typename T, int KIND, int V, int VPT, int TPR>
__global__ __launch_bounds__(kThreads) void rownorm_kernel(RnArgs a) {
  __shared__ float red[kThreads / 64];
  constexpr int RPB = kThreads / TPR;  // rows per block
  const int t = threadIdx.x % TPR;
  const long long row = static_cast<long long>(blockIdx.x) * RPB +
                        threadIdx.x / TPR;
  // TPR == 256: the whole block shares the row, so this exit is uniform;
  // TPR == 64: whole wavefronts exit, and no barrier follows.
  if (row >= a.rows) return;
  const T* xr = static_cast<const T*>(a.x) + row * a.n;
  T* yr = static_cast<T*>(a.y) + row * a.n;
  const int n = a.n;

  union Pack {
    u32x4 u;
    T e[V > 1 ? V : 1];
  };
  float v[VPT][V];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int base = (t + i * TPR) * V;
    if (base < n) {
      if constexpr (V > 1) {
        Pack q;
        q.u = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(xr + base));
#pragma unroll
        for (int e = 0; e < V; ++e) v[i][e] = to_f32(q.e[e]);
      } else {
        v[i][0] = to_f32(xr[base]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) v[i][e] = KIND == QK_ROWNORM_SOFTMAX
                                                ? -INFINITY
                                                : 0.f;
    }
  }

  // Gain and offset are requested right behind x, so their latency hides
  // under the row's own loads instead of following the reduction.
  const bool gvec = V > 1 && (reinterpret_cast<uintptr_t>(a.gain) % 16 == 0);
  const bool bvec = V > 1 && (reinterpret_cast<uintptr_t>(a.beta) % 16 == 0);
  constexpr bool kParams = KIND != QK_ROWNORM_SOFTMAX;
  float g[kParams ? VPT : 1][V], bb[KIND == QK_ROWNORM_LAYER ? VPT : 1][V];
  if constexpr (kParams) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int base = (t + i * TPR) * V;
      if (base >= n) continue;
      if (a.has_gain) load_param<V>(a.gain, a.gdt, base, gvec, g[i]);
      if (KIND == QK_ROWNORM_LAYER && a.has_beta)
        load_param<V>(a.beta, a.bdt, base, bvec, bb[i]);
    }
  }

  float scale = 1.f, shift = 0.f;  // y = (x - shift) * scale (then gain)
  if constexpr (KIND == QK_ROWNORM_RMS) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int e = 0; e < V; ++e) ss += v[i][e] * v[i][e];
    ss = row_sum<TPR>(ss, red);
    scale = rsqrtf(ss / static_cast<float>(n) + a.eps);
  } else if constexpr (KIND == QK_ROWNORM_LAYER) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int e = 0; e < V; ++e) s += v[i][e];
    const float mu = row_sum<TPR>(s, red) / static_cast<float>(n);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      if ((t + i * TPR) * V >= n) continue;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float d = v[i][e] - mu;
        q += d * d;
      }
    }
    const float var = row_sum<TPR>(q, red) / static_cast<float>(n);
    shift = mu;
    scale = 1.0f / sqrtf(var + a.eps);
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int e = 0; e < V; ++e) mx = fmaxf(mx, v[i][e]);
    mx = row_max<TPR>(mx, red);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int e = 0; e < V; ++e) {
        v[i][e] = __expf(v[i][e] - mx);
        s += v[i][e];
      }
    s = row_sum<TPR>(s, red);
    scale = 1.0f / s;
  }

#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int base = (t + i * TPR) * V;
    if (base >= n) continue;
    float out[V];
#pragma unroll
    for (int e = 0; e < V; ++e) out[e] = (v[i][e] - shift) * scale;
    if constexpr (kParams) {
      if (a.has_gain) {
#pragma unroll
        for (int e = 0; e < V; ++e) out[e] *= g[i][e];
      }
      if (KIND == QK_ROWNORM_LAYER && a.has_beta) {
#pragma unroll
        for (int e = 0; e < V; ++e) out[e] += bb[KIND == QK_ROWNORM_LAYER ? i : 0][e];
      }
    }
    if constexpr (V > 1) {
      Pack q;
#pragma unroll
      for (int e = 0; e < V; ++e) q.e[e] = from_f32<T>(out[e]);
      __builtin_nontemporal_store(q.u, reinterpret_cast<u32x4*>(yr + base));
    } else {
      yr[base] = from_f32<T>(out[0]);
    }
  }
}

// Persistent row streamer for rows that fit one wavefront's registers
// (n <= 64 * V * VPT, 16-byte aligned rows): each wave walks rows
// gw, gw + GW, ... with two register buffers, so the next row's loads are
// in flight while the current row is reduced and stored; reads and writes
// of different rows overlap instead of running as two phases. Gain and
// offset are loaded once per wave. Every load and store goes through a
// per-row buffer descriptor whose extent is 0 for rows past the end
// (loads read zeros, stores are dropped), so the loop has no branches
// and the compiler's wait counts follow the two buffers exactly.
//
// SPLIT = 2 (rows of up to 16 vectors per lane, e.g. 4096 f32): two waves
// share a row, each holding half of it (8 vectors per lane), and combine
// their partial sums (or maxima) through LDS; the two row units of a
// workgroup step through their rows together, so the loop's trip count and
// its barriers are uniform across the workgroup (rows past the end go
// through the zero-extent descriptors like any other).
//
// PL: gain and offset in T's type (16-byte aligned) or absent, kept
// packed in registers (LayerNorm of 16-bit rows of 8 vectors per
// lane: one wave per row at two waves per SIMD, no barriers per row).
template <typename T, int KIND, int V, int VPT, int SPLIT = 1, bool PL = false>
__global__ __launch_bounds__(kThreads) void rownorm_stream_kernel(RnArgs a) {
  static_assert(V > 1, "vector rows only");
  static_assert(SPLIT == 1 || SPLIT == 2, "one or two waves per row");
  constexpr int kUnits = kThreads / 64 / SPLIT;  // rows in flight per block
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int unit = __builtin_amdgcn_readfirstlane(wave / SPLIT);
  const int half = __builtin_amdgcn_readfirstlane(wave % SPLIT);
  const int vbase = half * VPT * 64;  // first 16-byte vector of the half
  const long long gw = static_cast<long long>(blockIdx.x) * kUnits + unit;
  const long long GW = static_cast<long long>(gridDim.x) * kUnits;
  __shared__ float xch[SPLIT == 2 ? 2 * 2 * (kThreads / 64) : 1];
  // Combines a wave's partial with its partner's (SPLIT = 2): exchange
  // slot `slot` (0 or 1, for a kind's two reductions) of row parity `par`;
  // alternating parities keep a slot from being rewritten before the
  // partner has read it.
  auto combine = [&](float v, int par, int slot, bool is_max) {
    if constexpr (SPLIT == 1) {
      return v;
    } else {
      float* const x = xch + (par * 2 + slot) * (kThreads / 64);
      if (lane == 0) x[wave] = v;
      __syncthreads();
      const float o = x[wave ^ 1];
      return is_max ? fmaxf(v, o) : v + o;
    }
  };
  const int n = a.n;
  const int row_bytes = n * static_cast<int>(sizeof(T));
  constexpr int kNT = 2;  // nontemporal: streamed once

  constexpr bool kParams = KIND != QK_ROWNORM_SOFTMAX;
  constexpr bool kBeta = KIND == QK_ROWNORM_LAYER;
  static_assert(!PL || (SPLIT == 1 && V == 8), "packed parameters");
  // PL: gain and offset of T's type kept packed (16-byte vectors of V
  // values) and widened when used.
  u32x4 gpk[PL ? VPT : 1], bpk[PL ? VPT : 1];
  if constexpr (PL) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int base = (lane + i * 64) * V;
      const bool in = base < n;
      // absent: gain 1.0, offset 0 (as pairs of T)
      const uint32_t one2 = std::is_same<T, bf16>::value ? 0x3F803F80u
                                                         : 0x3C003C00u;
      gpk[i] = in && a.has_gain ? *reinterpret_cast<const u32x4*>(
                                      static_cast<const T*>(a.gain) + base)
                                : u32x4{one2, one2, one2, one2};
      bpk[i] = in && a.has_beta ? *reinterpret_cast<const u32x4*>(
                                      static_cast<const T*>(a.beta) + base)
                                : u32x4{0u, 0u, 0u, 0u};
    }
  }
  float g[kParams && !PL ? VPT : 1][V], bb[kBeta && !PL ? VPT : 1][V];
  if constexpr (kParams && !PL) {
    const bool gvec = (reinterpret_cast<uintptr_t>(a.gain) % 16 == 0);
    const bool bvec = (reinterpret_cast<uintptr_t>(a.beta) % 16 == 0);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int base = (vbase + lane + i * 64) * V;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        g[i][e] = 1.f;
        if (kBeta) bb[i][e] = 0.f;
      }
      if (base < n) {
        if (a.has_gain) load_param<V>(a.gain, a.gdt, base, gvec, g[i]);
        if (kBeta && a.has_beta)
          load_param<V>(a.beta, a.bdt, base, bvec, bb[kBeta ? i : 0]);
      }
    }
  }

  auto rsrc = [&](const void* base, long long row) {
    const bool ok = row < a.rows;
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(base)) +
            (ok ? row : 0) * row_bytes,
        (short)0, ok ? row_bytes : 0, 0x00020000);
  };
  auto load = [&](long long row, u32x4 (&buf)[VPT]) {
    const auto rs = rsrc(a.x, row);
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      buf[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (vbase + lane + i * 64) * 16,
                                                     0, kNT);
  };
  union Pack {
    u32x4 u;
    T e[V];
  };
  auto process = [&](long long row, const u32x4 (&buf)[VPT], int par) {
    float v[VPT][V];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      Pack q;
      q.u = buf[i];
      const bool in = (vbase + lane + i * 64) * V < n;
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[i][e] = in ? to_f32(q.e[e])
                     : (KIND == QK_ROWNORM_SOFTMAX ? -INFINITY : 0.f);
    }
    float scale = 1.f, shift = 0.f;
    if constexpr (KIND == QK_ROWNORM_RMS) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int e = 0; e < V; ++e) ss += v[i][e] * v[i][e];
      scale = rsqrtf(combine(wave_sum_dpp(ss), par, 0, false) /
                         static_cast<float>(n) +
                     a.eps);
    } else if constexpr (KIND == QK_ROWNORM_LAYER && PL) {
      // 16-bit rows: mean and variance from one reduction of the sums of
      // d = x - x0 and d^2, shifted by the row's first element x0 (a
      // sample of the row, so the two sums do not cancel; 16-bit inputs
      // leave the f32 sums far inside the output's rounding).
      const float x0 = __builtin_bit_cast(
          float, __builtin_amdgcn_readfirstlane(
                     __builtin_bit_cast(int, v[0][0])));
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const bool in = (vbase + lane + i * 64) * V < n;
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float d = in ? v[i][e] - x0 : 0.f;
          s1 += d;
          s2 = fmaf(d, d, s2);
        }
      }
      // two independent DPP reductions (their steps interleave)
      const float inv_n = 1.f / static_cast<float>(n);
      const float m1 = wave_sum_dpp(s1) * inv_n;
      const float m2 = wave_sum_dpp(s2) * inv_n;
      shift = x0 + m1;
      scale = 1.0f / sqrtf(fmaxf(m2 - m1 * m1, 0.f) + a.eps);
    } else if constexpr (KIND == QK_ROWNORM_LAYER) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int e = 0; e < V; ++e) s += v[i][e];
      const float mu =
          combine(wave_sum_dpp(s), par, 0, false) / static_cast<float>(n);
      float q = 0.f;
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const bool in = (vbase + lane + i * 64) * V < n;
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float d = in ? v[i][e] - mu : 0.f;
          q += d * d;
        }
      }
      shift = mu;
      scale = 1.0f / sqrtf(combine(wave_sum_dpp(q), par, 1, false) /
                                static_cast<float>(n) +
                            a.eps);
    } else {
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int e = 0; e < V; ++e) mx = fmaxf(mx, v[i][e]);
      mx = combine(wave_max(mx), par, 0, true);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int e = 0; e < V; ++e) {
          v[i][e] = __expf(v[i][e] - mx);
          s += v[i][e];
        }
      scale = 1.0f / combine(wave_sum_dpp(s), par, 1, false);
    }
    const auto rs = rsrc(a.y, row);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      Pack q;
      float gp[V], bp[V];
      if constexpr (PL) {
        Pack gq, bq;
        gq.u = gpk[i];
        bq.u = bpk[i];
#pragma unroll
        for (int e = 0; e < V; ++e) {
          gp[e] = to_f32(gq.e[e]);
          bp[e] = to_f32(bq.e[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float o = (v[i][e] - shift) * scale;
        if constexpr (PL) {
          o = o * gp[e] + bp[e];
        } else {
          if constexpr (kParams) o *= g[i][e];
          if constexpr (kBeta) o += bb[kBeta ? i : 0][e];
        }
        q.e[e] = from_f32<T>(o);
      }
      // Offsets at or past the row end are dropped by the descriptor.
      __builtin_amdgcn_raw_buffer_store_b128(q.u, rs, (vbase + lane + i * 64) * 16, 0,
                                             kNT);
    }
  };

  u32x4 xa[VPT], xb[VPT];
  load(gw, xa);
  // row - unit is the same for every unit of the block (uniform trip count)
#pragma unroll 1
  for (long long row = gw; row - unit < a.rows; row += 2 * GW) {
    load(row + GW, xb);
    process(row, xa, 0);
    load(row + 2 * GW, xa);
    process(row + GW, xb, 1);
  }
}

// Rows longer than the register kernels take: one block per row, reading
// the row once per statistic.
template <typename T, int KIND>
__global__ __launch_bounds__(kThreads) void rownorm_long_kernel(RnArgs a) {
  __shared__ float red[kThreads / 64];
  const long long row = blockIdx.x;
  const T* xr = static_cast<const T*>(a.x) + row * a.n;
  T* yr = static_cast<T*>(a.y) + row * a.n;
  const int n = a.n;
  float scale = 1.f, shift = 0.f;
  if constexpr (KIND == QK_ROWNORM_RMS) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kThreads) {
      const float x = to_f32(xr[i]);
      ss += x * x;
    }
    ss = row_sum<kThreads>(ss, red);
    scale = rsqrtf(ss / static_cast<float>(n) + a.eps);
  } else if constexpr (KIND == QK_ROWNORM_LAYER) {
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
      s += __expf(to_f32(xr[i]) - mx);
    s = row_sum<kThreads>(s, red);
    const float inv = 1.0f / s;
    for (int i = threadIdx.x; i < n; i += kThreads)
      yr[i] = from_f32<T>(__expf(to_f32(xr[i]) - mx) * inv);
    return;
  }
  for (int i = threadIdx.x; i < n; i += kThreads) {
    float o = (to_f32(xr[i]) - shift) * scale;
    if (a.has_gain) o *= load_any(a.gain, i, a.gdt);
    if (a.has_beta) o += load_any(a.beta, i, a.bdt);
    yr[i] = from_f32<T>(o);
  }
}

template <typename T, int KIND, int V>
qk_status LaunchV(const RnArgs& a, hipStream_t st) {
  constexpr int kSmall = 64 * V * 4, kMid = 64 * V * 8, kWave = 64 * V * 16,
                kBlock = kThreads * V * 16;
  if (a.n <= kSmall) {
    dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
    rownorm_kernel<T, KIND, V, 4, 64><<<grid, kThreads, 0, st>>>(a);
  } else if (a.n <= kMid) {
    dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
    rownorm_kernel<T, KIND, V, 8, 64><<<grid, kThreads, 0, st>>>(a);
  } else if (a.n <= kWave) {
    dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
    rownorm_kernel<T, KIND, V, 16, 64><<<grid, kThreads, 0, st>>>(a);
  } else if (a.n <= kBlock) {
    dim3 grid(static_cast<unsigned>(a.rows));
    rownorm_kernel<T, KIND, V, 16, kThreads><<<grid, kThreads, 0, st>>>(a);
  } else {
    dim3 grid(static_cast<unsigned>(a.rows));
    rownorm_long_kernel<T, KIND><<<grid, kThreads, 0, st>>>(a);
  }
  return PostLaunch("rownorm");
}

// Rows of up to 8 vectors per lane with at least two rows per wave: the
// persistent streamer, two workgroups (eight waves) per CU.
template <typename T, int KIND>
bool LaunchStream(const RnArgs& a, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  // Buffer descriptors take 32-bit extents; rows are at most 64 KB here.
  auto go = [&](auto kernel, int split = 1) {
    const int cus = DeviceComputeUnits();
    // (1..4 workgroups per CU measured within 2% of each other at
    // [4096, 4096].)
    const int per_cu = std::min(
        2, ResidentBlocks(reinterpret_cast<const void*>(kernel), kThreads, 0));
    const long long units = static_cast<long long>(per_cu) * cus *
                            (kThreads / 64 / split);
    if (a.rows < 2 * units) return false;
    kernel<<<dim3(per_cu * cus), kThreads, 0, st>>>(a);
    return true;
  };
  // Rows of 9..16 vectors per lane: two waves per row, 8 vectors each
  // (two 16-vector buffers per wave measured slower than the one-shot
  // kernel).
  if (a.n <= 64 * V * 4) return go(rownorm_stream_kernel<T, KIND, V, 4>);
  // LayerNorm of 16-bit rows (gain and offset held as f32): 8 vectors per
  // lane take 256 VGPRs, one wave per SIMD; two waves of 4 keep two per
  // SIMD ([4096, 4096] bf16: 16.7 -> 14.5 us).
  if constexpr (KIND == QK_ROWNORM_LAYER && V == 8) {
    // Gain and offset each absent (the reference's layernorm has neither)
    // or of x's type and 16-byte aligned: held packed, one wave per row;
    // else two waves of 4 vectors per row with the parameters in f32.
    const int tcode = std::is_same<T, bf16>::value ? QK_BF16 : QK_F16;
    auto packable = [&](bool has, const void* q, int dt) {
      return !has || (dt == tcode && reinterpret_cast<uintptr_t>(q) % 16 == 0);
    };
    const bool packed_params = packable(a.has_gain, a.gain, a.gdt) &&
                               packable(a.has_beta, a.beta, a.bdt) &&
                               std::getenv("QK_ROWNORM_LAYER_SPLIT") == nullptr;
    if (a.n <= 64 * V * 8)
      return packed_params
                 ? go(rownorm_stream_kernel<T, KIND, V, 8, 1, true>)
                 : go(rownorm_stream_kernel<T, KIND, V, 4, 2>, 2);
  }
  if (a.n <= 64 * V * 8) return go(rownorm_stream_kernel<T, KIND, V, 8>);
  if (a.n <= 64 * V * 16)
    return go(rownorm_stream_kernel<T, KIND, V, 8, 2>, 2);
  return false;
}

template <typename T, int KIND>
qk_status LaunchKind(const RnArgs& a, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const bool aligned = (reinterpret_cast<uintptr_t>(a.x) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) &&
                       (static_cast<long long>(a.n) * sizeof(T)) % 16 == 0;
  if (aligned && LaunchStream<T, KIND>(a, st)) return PostLaunch("rownorm");
  return aligned ? LaunchV<T, KIND, V>(a, st) : LaunchV<T, KIND, 1>(a, st);
}

template <typename T>
qk_status LaunchTyped(const RnArgs& a, int kind, hipStream_t st) {
  if (kind == QK_ROWNORM_RMS) return LaunchKind<T, QK_ROWNORM_RMS>(a, st);
  if (kind == QK_ROWNORM_LAYER) return LaunchKind<T, QK_ROWNORM_LAYER>(a, st);
  return LaunchKind<T, QK_ROWNORM_SOFTMAX>(a, st);
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
  a.eps = p.eps;
  a.gdt = p.gain_dtype;
  a.bdt = p.beta_dtype;
  a.has_gain = p.gain != nullptr;
  a.has_beta = p.beta != nullptr;
  switch (p.dtype) {
    case QK_BF16:
      return LaunchTyped<bf16>(a, p.kind, stream);
    case QK_F16:
      return LaunchTyped<f16>(a, p.kind, stream);
    default:
      return LaunchTyped<float>(a, p.kind, stream);
  }
}

}  // namespace qk
