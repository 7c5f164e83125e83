// Device quantizer for gfx950: float weights [N, K] -> the codes, scales
// and offsets qk$qmatvec / qk$dequantize read, for loading a checkpoint
// straight into HBM.
//
// Replaces the reference loader's host quantizers (examples/llm/qwen3.py:
// 154-196, run once per matrix in load_params, qwen3.py:113-128):
//  - int4, MLX-style affine grid per group (quantize_int4): lo / hi of the
//    group; the grid is anchored at the larger-magnitude one (edge, the
//    offset) with step s = +-max(hi - lo, 1e-12) / 15, stretched so that
//    zero also lies on it (s = edge / rint(edge / s) when that is not 0,
//    else offset 0); q = clip(rint((w - b) / s), 0, 15);
//  - int8, symmetric per group (quantize_int8): s = max(max |w|, 1e-12) /
//    127, q = clip(rint(w / s), -127, 127), no offset.
// Every step is the reference's float32 operation in the same order: IEEE
// subtraction, correctly rounded division (__fdiv_rn), round half to even
// (rintf), so codes, scales and offsets are bit-identical to the float32
// numpy restatement. Scales and offsets are stored in f32 or rounded once
// (nearest even) to f16 / bf16.
//
// One thread per group (its 32..128 weights in registers, read as 16-byte
// vectors); each weight's quotient rounded through the reciprocal, with
// the correctly rounded division only near a rounding boundary (one per
// weight made the kernel division-bound: 32 against 28.6 us at 12288 x 4096
// bf16). Eight lanes per group with the extremes reduced across them
// measured slower (the per-group divisions repeat on every lane).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct QzArgs {
  const void* w;
  void* codes;
  void* scales;
  void* biases;
  long long groups;  // n * (k / G)
  int gpr;           // groups per row
};

// rint(fl(x / s)) (fl: the correctly rounded quotient) without a division
// per weight: the hardware reciprocal is within 1 ulp of 1/s, so
// r = x * (1/s) is within 2.5e-7 |r| of x / s, as is fl(x / s). Where r is
// farther than 1e-5 + 1e-6 |r| from a half-integer, rint(r) equals
// rint(fl(x / s)); nearer (rare), the correctly rounded division decides.
__device__ __forceinline__ float RoundQuotient(float x, float s,
                                               float inv) {
  const float r = x * inv;
  const float c = rintf(r);
  const float tol = 1e-5f + 1e-6f * fabsf(r);
  return fabsf(fabsf(r - c) - 0.5f) < tol ? rintf(__fdiv_rn(x, s)) : c;
}

// One thread per group: its G weights in registers, read as 16-byte
// vectors.
template <typename WT, int G, int PACK, typename ST>
__global__ __launch_bounds__(256) void quantize_kernel(QzArgs a) {
  const long long gid =
      static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= a.groups) return;
  constexpr int E = 16 / sizeof(WT);  // weights per 16-byte vector
  const u32x4* src = reinterpret_cast<const u32x4*>(
      static_cast<const WT*>(a.w) + gid * G);
  float v[G];
#pragma unroll
  for (int i = 0; i < G / E; ++i) {
    union {
      u32x4 u;
      WT e[E];
    } p;
    p.u = src[i];
#pragma unroll
    for (int e = 0; e < E; ++e) v[i * E + e] = to_f32(p.e[e]);
  }
  float scale, offset = 0.f;
  int q[G];
  if constexpr (PACK == QK_PACK_S8_SYM) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < G; ++i) amax = fmaxf(amax, fabsf(v[i]));
    scale = __fdiv_rn(fmaxf(amax, 1e-12f), 127.f);
    const float inv = __builtin_amdgcn_rcpf(scale);
#pragma unroll
    for (int i = 0; i < G; ++i)
      q[i] = static_cast<int>(
          fminf(fmaxf(RoundQuotient(v[i], scale, inv), -127.f), 127.f));
  } else {
    float lo = v[0], hi = v[0];
#pragma unroll
    for (int i = 1; i < G; ++i) lo = fminf(lo, v[i]), hi = fmaxf(hi, v[i]);
    const bool neg = fabsf(lo) > fabsf(hi);
    const float width = __fdiv_rn(fmaxf(hi - lo, 1e-12f), 15.f);
    scale = neg ? width : -width;
    const float edge = neg ? lo : hi;
    const float q0 = rintf(__fdiv_rn(edge, scale));
    if (q0 != 0.f) {
      scale = __fdiv_rn(edge, q0);
      offset = edge;
    }
    const float inv = __builtin_amdgcn_rcpf(scale);
#pragma unroll
    for (int i = 0; i < G; ++i)
      q[i] = static_cast<int>(fminf(
          fmaxf(RoundQuotient(v[i] - offset, scale, inv), 0.f), 15.f));
  }
  static_cast<ST*>(a.scales)[gid] = from_f32<ST>(scale);
  if constexpr (PACK != QK_PACK_S8_SYM)
    static_cast<ST*>(a.biases)[gid] = from_f32<ST>(offset);

  if constexpr (PACK == QK_PACK_U32X8) {
    // code 8 i + j in bits 4 j .. 4 j + 3 of word i
    uint32_t* dst = static_cast<uint32_t*>(a.codes) + gid * (G / 8);
#pragma unroll
    for (int i = 0; i < G / 8; ++i) {
      uint32_t wd = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        wd |= static_cast<uint32_t>(q[8 * i + j]) << (4 * j);
      dst[i] = wd;
    }
  } else if constexpr (PACK == QK_PACK_BYTE_HALFSPLIT) {
    // byte j of the group: code j (low nibble), code j + G/2 (high)
    uint32_t* dst = static_cast<uint32_t*>(a.codes) + gid * (G / 8);
#pragma unroll
    for (int i = 0; i < G / 8; ++i) {
      uint32_t wd = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int j = 4 * i + b;
        wd |= static_cast<uint32_t>(q[j] | (q[j + G / 2] << 4)) << (8 * b);
      }
      dst[i] = wd;
    }
  } else {
    uint32_t* dst = static_cast<uint32_t*>(a.codes) + gid * (G / 4);
#pragma unroll
    for (int i = 0; i < G / 4; ++i) {
      uint32_t wd = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b)
        wd |= (static_cast<uint32_t>(q[4 * i + b]) & 0xFFu) << (8 * b);
      dst[i] = wd;
    }
  }
}

template <typename WT, int G, int PACK>
void LaunchS(const QzArgs& a, int sdt, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((a.groups + 255) / 256));
  if (sdt == QK_F32)
    quantize_kernel<WT, G, PACK, float><<<grid, 256, 0, st>>>(a);
  else if (sdt == QK_F16)
    quantize_kernel<WT, G, PACK, f16><<<grid, 256, 0, st>>>(a);
  else
    quantize_kernel<WT, G, PACK, bf16><<<grid, 256, 0, st>>>(a);
}

template <typename WT, int G>
void LaunchP(const QzArgs& a, int packing, int sdt, hipStream_t st) {
  if (packing == QK_PACK_U32X8)
    LaunchS<WT, G, QK_PACK_U32X8>(a, sdt, st);
  else if (packing == QK_PACK_BYTE_HALFSPLIT)
    LaunchS<WT, G, QK_PACK_BYTE_HALFSPLIT>(a, sdt, st);
  else
    LaunchS<WT, G, QK_PACK_S8_SYM>(a, sdt, st);
}

template <typename WT>
void LaunchG(const QzArgs& a, int g, int packing, int sdt, hipStream_t st) {
  if (g == 32)
    LaunchP<WT, 32>(a, packing, sdt, st);
  else if (g == 64)
    LaunchP<WT, 64>(a, packing, sdt, st);
  else
    LaunchP<WT, 128>(a, packing, sdt, st);
}

}  // namespace

qk_status LaunchQuantize(const QuantProblem& p, const void* w, int w_dtype,
                         hipStream_t stream) {
  QzArgs a;
  a.w = w;
  a.codes = const_cast<void*>(p.codes);
  a.scales = const_cast<void*>(p.scales);
  a.biases = const_cast<void*>(p.biases);
  a.gpr = static_cast<int>(p.k / p.group);
  a.groups = p.n * a.gpr;
  if (w_dtype == QK_F32)
    LaunchG<float>(a, p.group, p.packing, p.scale_dtype, stream);
  else if (w_dtype == QK_F16)
    LaunchG<f16>(a, p.group, p.packing, p.scale_dtype, stream);
  else
    LaunchG<bf16>(a, p.group, p.packing, p.scale_dtype, stream);
  return PostLaunch("quantize");
}

}  // namespace qk
