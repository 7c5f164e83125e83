// Group-affine int4/int8 weight-quantized matvec and dequantize for gfx950.
//
// Replaces the reduction fusions XLA emits for the reference's _matvec_int8 /
// _matvec_int4 (examples/llm/qwen3.py:233-267) and its dequantize
// (qwen3.py:199-207). Semantics, per output row o and group g:
//   y[m, o] = sum_g ( scale[o,g] * sum_{k in g} x[m,k] q[o,k]
//                     + bias[o,g] * sum_{k in g} x[m,k] )
// in f32, rounded once to x's type: the reference's per-group factoring
// (qwen3.py:246-250), which equals sum_k x[m,k] (scale*q + bias).
//
// The matvec is bandwidth-bound: every code byte is read once with 16-byte
// loads, codes are widened in registers and the K reduction ends in a
// wavefront butterfly.
//  - A wave owns R output rows; its 64 lanes stride over the rows' 16-byte
//    code chunks (32 int4 or 16 int8 codes), so each lane's x slice is
//    loaded once and reused for all R rows.
//  - bf16 x, 4-bit codes: a code pair (q_a, q_b) sharing a 32-bit word at
//    nibbles s and s+4 becomes the bf16 pair (128+q_a, 128+q_b) with one
//    and-or (0x4300 | q is 128 + q exactly in bf16), and v_dot2_f32_bf16
//    multiplies it with the matching pair of x. The 128 offset is removed
//    per group: s*sum(x(q+128)) + (b - 128 s)*sum(x).
//  - Other types widen codes to f32 and use FMAs.

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <mutex>

#include <algorithm>
#include <cstdint>
#include <string>
#include <type_traits>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {

// The device status word: one per device (each GPU holds its own copy of
// this variable), set by kernels whose bounded waits gave up.
static __device__ uint32_t g_device_status;

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_status_mu;
uint32_t* g_status_ptr[kMaxDevices] = {};
}  // namespace

uint32_t* DeviceStatusWord() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_status_mu);
  if (g_status_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_device_status)) !=
            hipSuccess ||
        ptr == nullptr) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_status_ptr[dev] = static_cast<uint32_t*>(ptr);
  }
  return g_status_ptr[dev];
}

uint32_t ReadDeviceStatusWords(bool clear) {
  std::lock_guard<std::mutex> lock(g_status_mu);
  uint32_t bits = 0;
  int cur = -1;
  for (int dev = 0; dev < kMaxDevices; ++dev) {
    if (g_status_ptr[dev] == nullptr) continue;
    if (cur < 0 && hipGetDevice(&cur) != hipSuccess) cur = 0;
    if (hipSetDevice(dev) != hipSuccess) continue;
    uint32_t v = 0;
    if (hipMemcpy(&v, g_status_ptr[dev], sizeof(v), hipMemcpyDeviceToHost) ==
        hipSuccess)
      bits |= v;
    if (clear) {
      const uint32_t zero = 0;
      (void)hipMemcpy(g_status_ptr[dev], &zero, sizeof(zero),
                      hipMemcpyHostToDevice);
    }
  }
  if (cur >= 0) (void)hipSetDevice(cur);
  (void)hipGetLastError();
  return bits;
}

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;  // waves per workgroup

struct QmvArgs {
  const void* x;
  const uint8_t* codes;
  const void* scales;
  const void* biases;
  void* y;
  int m, n, k;
  int group;
  int sdt, bdt;  // scale / bias dtypes (qk_dtype)
  int has_bias;
  int row_bytes;  // bytes of codes per output row
  const int* gather;  // dequantize: table row of each output row (or null)
  int out_vec;        // dequantize: 16-byte stores of y allowed
};

__device__ __forceinline__ uint32_t PackBf16Pair(float lo, float hi) {
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

// x is bf16: its values are exact in f32, so truncating back is exact.
template <int PACK, int MT, int R>
__global__ __launch_bounds__(kWaves * 64) void qmv_int4_bf16_kernel(
    QmvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int row0 = wave * R;
  if (row0 >= a.n) return;
  const int hg = a.group / 2;  // half group, half-split packing
  const int chunks = a.row_bytes / 16;
  const bf16* X = static_cast<const bf16*>(a.x);

  float acc[MT][R];
#pragma unroll
  for (int mm = 0; mm < MT; ++mm)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[mm][r] = 0.f;

  for (int c = lane; c < chunks; c += 64) {
    // K span of the chunk: u32x8 -> 32 consecutive codes; half-split ->
    // 16 codes at kb and 16 at kb + hg.
    int kb, grp;
    if (PACK == QK_PACK_U32X8) {
      kb = c * 32;
      grp = kb / a.group;
    } else {
      const int byte0 = c * 16;
      grp = byte0 / hg;
      kb = grp * a.group + byte0 % hg;
    }
    u32x4 w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, a.n - 1);
      w[r] = *reinterpret_cast<const u32x4*>(
          a.codes + static_cast<long long>(row) * a.row_bytes + c * 16);
    }
    float s[R], bb[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, a.n - 1);
      const long long gi = static_cast<long long>(row) * (a.k / a.group) + grp;
      s[r] = load_any(a.scales, gi, a.sdt);
      bb[r] = a.has_bias ? load_any(a.biases, gi, a.bdt) : 0.f;
    }
    // Code pairs (128 + q) as bf16x2, pair p = 4*i + s: nibbles s, s+4.
    uint32_t cp[R][16];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int sh = 0; sh < 4; ++sh)
          cp[r][4 * i + sh] = ((w[r][i] >> (4 * sh)) & 0x000F000Fu) | 0x43004300u;

#pragma unroll
    for (int mm = 0; mm < MT; ++mm) {
      if (mm >= a.m) break;
      const bf16* xr = X + static_cast<long long>(mm) * a.k + kb;
      float xf[32];
      if (PACK == QK_PACK_U32X8) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const u32x4 q = *reinterpret_cast<const u32x4*>(xr + 8 * v);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            xf[8 * v + 2 * e] = __uint_as_float(q[e] << 16);
            xf[8 * v + 2 * e + 1] = __uint_as_float(q[e] & 0xffff0000u);
          }
        }
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int v = 0; v < 2; ++v) {
            const u32x4 q =
                *reinterpret_cast<const u32x4*>(xr + h * hg + 8 * v);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              xf[16 * h + 8 * v + 2 * e] = __uint_as_float(q[e] << 16);
              xf[16 * h + 8 * v + 2 * e + 1] =
                  __uint_as_float(q[e] & 0xffff0000u);
            }
          }
      }
      uint32_t xp[16];
      float xs = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int sh = 0; sh < 4; ++sh) {
          int e0, e1;
          if (PACK == QK_PACK_U32X8) {
            e0 = 8 * i + sh;
            e1 = 8 * i + sh + 4;
          } else {
            // Nibble sh: byte 4i + sh/2 of the chunk, low (first half) for
            // even sh; nibble sh + 4: byte 4i + 2 + sh/2.
            e0 = ((sh & 1) ? 16 : 0) + 4 * i + (sh >> 1);
            e1 = ((sh & 1) ? 16 : 0) + 4 * i + 2 + (sh >> 1);
          }
          xp[4 * i + sh] = PackBf16Pair(xf[e0], xf[e1]);
        }
#pragma unroll
      for (int e = 0; e < 32; ++e) xs += xf[e];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = 0.f;
#pragma unroll
        for (int p = 0; p < 16; ++p)
          d = __builtin_amdgcn_fdot2_f32_bf16(AsBf16x2(cp[r][p]),
                                              AsBf16x2(xp[p]), d, false);
        acc[mm][r] += s[r] * d + (bb[r] - 128.f * s[r]) * xs;
      }
    }
  }

#pragma unroll
  for (int mm = 0; mm < MT; ++mm) {
    if (mm >= a.m) break;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(acc[mm][r]);
      if (lane == 0 && row0 + r < a.n)
        static_cast<bf16*>(a.y)[static_cast<long long>(mm) * a.n + row0 + r] =
            from_f32<bf16>(v);
    }
  }
}

// Generic path: any x type, any packing; codes widened to f32, FMAs.
template <typename XT, int PACK, int MT, int R>
__global__ __launch_bounds__(kWaves * 64) void qmv_generic_kernel(QmvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int row0 = wave * R;
  if (row0 >= a.n) return;
  constexpr bool kInt4 = PACK == QK_PACK_U32X8 || PACK == QK_PACK_BYTE_HALFSPLIT;
  constexpr int kCodes = kInt4 ? 32 : 16;  // codes per 16-byte chunk
  const int hg = a.group / 2;
  const int chunks = a.row_bytes / 16;
  const XT* X = static_cast<const XT*>(a.x);

  float acc[MT][R];
#pragma unroll
  for (int mm = 0; mm < MT; ++mm)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[mm][r] = 0.f;

  for (int c = lane; c < chunks; c += 64) {
    int kb, grp;
    if (PACK == QK_PACK_BYTE_HALFSPLIT) {
      const int byte0 = c * 16;
      grp = byte0 / hg;
      kb = grp * a.group + byte0 % hg;
    } else {
      kb = c * kCodes;
      grp = kb / a.group;
    }
    u32x4 w[R];
    float s[R], bb[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, a.n - 1);
      w[r] = *reinterpret_cast<const u32x4*>(
          a.codes + static_cast<long long>(row) * a.row_bytes + c * 16);
      const long long gi = static_cast<long long>(row) * (a.k / a.group) + grp;
      s[r] = load_any(a.scales, gi, a.sdt);
      bb[r] = a.has_bias ? load_any(a.biases, gi, a.bdt) : 0.f;
    }
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) {
      if (mm >= a.m) break;
      const XT* xr = X + static_cast<long long>(mm) * a.k + kb;
      // xf[e]: x at chunk element e (half-split: e >= 16 is the second half).
      float xf[kCodes];
#pragma unroll
      for (int e = 0; e < kCodes; ++e) {
        int off = e;
        if (PACK == QK_PACK_BYTE_HALFSPLIT && e >= 16) off = hg + e - 16;
        xf[e] = to_f32(xr[off]);
      }
      float xs = 0.f;
#pragma unroll
      for (int e = 0; e < kCodes; ++e) xs += xf[e];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t word = w[r][i];
          if (kInt4) {
#pragma unroll
            for (int nib = 0; nib < 8; ++nib) {
              int e;
              if (PACK == QK_PACK_U32X8)
                e = 8 * i + nib;
              else
                e = ((nib & 1) ? 16 : 0) + 4 * i + (nib >> 1);
              d += xf[e] * static_cast<float>((word >> (4 * nib)) & 15u);
            }
          } else {
#pragma unroll
            for (int bt = 0; bt < 4; ++bt) {
              float q;
              if (PACK == QK_PACK_S8_SYM)
                q = static_cast<float>(static_cast<int8_t>(word >> (8 * bt)));
              else
                q = static_cast<float>((word >> (8 * bt)) & 255u);
              d += xf[4 * i + bt] * q;
            }
          }
        }
        acc[mm][r] += s[r] * d + bb[r] * xs;
      }
    }
  }

#pragma unroll
  for (int mm = 0; mm < MT; ++mm) {
    if (mm >= a.m) break;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(acc[mm][r]);
      if (lane == 0 && row0 + r < a.n)
        static_cast<XT*>(a.y)[static_cast<long long>(mm) * a.n + row0 + r] =
            from_f32<XT>(v);
    }
  }
}

// Dequantize: one thread per unit of codes that decodes to runs of 8
// consecutive values of a row: a 4-byte word of 8 int4 codes (U32X8), 8
// int8 codes, or 8 bytes of half-split int4 codes (runs at j and
// j + group / 2). Consecutive lanes load consecutive code bytes and store
// consecutive 16-byte runs (32 for f32 output), so both sides coalesce. A
// run never crosses a group (groups of 32, 64, 128).
// w = f32(q) * f32(scale) rounded, + f32(bias) rounded, then rounded once
// more to the output type (no fused multiply-add).
template <int PACK>
struct DqUnit {
  static constexpr int kBytes = PACK == QK_PACK_U32X8 ? 4 : 8;
  static constexpr int kRuns = PACK == QK_PACK_BYTE_HALFSPLIT ? 2 : 1;
};

template <int PACK, typename OT, int UPT>
__global__ __launch_bounds__(256) void dequant_kernel(QmvArgs a,
                                                     long long total_units) {
  using U = DqUnit<PACK>;
  // Units j * 256 + threadIdx.x of the block's run of 256 UPT (all loads
  // first, then the stores).
  const long long base = static_cast<long long>(blockIdx.x) * 256 * UPT;
  const int upr = a.row_bytes / U::kBytes;
  const int hg = a.group / 2;
  uint32_t w[UPT][2];
  float s[UPT], b[UPT];
  int orow[UPT], kb[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const long long t = min(base + j * 256 + threadIdx.x, total_units - 1);
    orow[j] = static_cast<int>(t / upr);
    // An embedding gather reads table row gather[orow], clamped into
    // range (as a JAX gather clamps out-of-range indices).
    const int row = a.gather == nullptr
                        ? orow[j]
                        : min(max(a.gather[orow[j]], 0), a.n - 1);
    const int byte0 = static_cast<int>(t % upr) * U::kBytes;
    int grp;
    if (PACK == QK_PACK_BYTE_HALFSPLIT) {
      grp = byte0 / hg;
      kb[j] = grp * a.group + byte0 % hg;
    } else {
      kb[j] = PACK == QK_PACK_U32X8 ? 2 * byte0 : byte0;
      grp = kb[j] / a.group;
    }
    const unsigned char* src =
        a.codes + static_cast<long long>(row) * a.row_bytes + byte0;
    if (U::kBytes == 4) {
      w[j][0] = *reinterpret_cast<const uint32_t*>(src);
      w[j][1] = 0;
    } else {
      const uint2 d = *reinterpret_cast<const uint2*>(src);
      w[j][0] = d.x;
      w[j][1] = d.y;
    }
    const long long gi = static_cast<long long>(row) * (a.k / a.group) + grp;
    s[j] = load_any(a.scales, gi, a.sdt);
    b[j] = a.has_bias ? load_any(a.biases, gi, a.bdt) : 0.f;
  }
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    if (base + j * 256 + threadIdx.x >= total_units) break;
    // v[8 r + e]: element e of run r.
    float v[8 * U::kRuns];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float q0, q1 = 0.f;
      if (PACK == QK_PACK_U32X8) {
        q0 = static_cast<float>((w[j][0] >> (4 * e)) & 15u);
      } else {
        const uint32_t byte = (w[j][e >> 2] >> (8 * (e & 3))) & 255u;
        if (PACK == QK_PACK_BYTE_HALFSPLIT) {
          q0 = static_cast<float>(byte & 15u);
          q1 = static_cast<float>(byte >> 4);
        } else if (PACK == QK_PACK_S8_SYM) {
          q0 = static_cast<float>(static_cast<int8_t>(byte));
        } else {
          q0 = static_cast<float>(byte);
        }
      }
      v[e] = __fadd_rn(__fmul_rn(q0, s[j]), b[j]);
      if (U::kRuns == 2) v[8 + e] = __fadd_rn(__fmul_rn(q1, s[j]), b[j]);
    }
    OT* out =
        static_cast<OT*>(a.y) + static_cast<long long>(orow[j]) * a.k + kb[j];
#pragma unroll
    for (int r = 0; r < U::kRuns; ++r) {
      OT* dst = out + r * hg;
      if (a.out_vec) {
        // Whole 16-byte stores: every run starts at a multiple of 8
        // elements.
        constexpr int kPer = 16 / sizeof(OT);
#pragma unroll
        for (int q = 0; q < 8 / kPer; ++q) {
          union {
            u32x4 u;
            OT e[kPer];
          } o;
#pragma unroll
          for (int e = 0; e < kPer; ++e)
            o.e[e] = from_f32<OT>(v[8 * r + kPer * q + e]);
          *reinterpret_cast<u32x4*>(dst + kPer * q) = o.u;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[e] = from_f32<OT>(v[8 * r + e]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Streaming matvec for a few rows of x (M <= 4): the decode hot path.
//
// The grid holds about as many waves as the GPU keeps resident; each wave
// walks output rows gw, gw + GW, ... (GW waves in the grid) and prefetches
// the next row's codes, scales and offsets into registers while it computes
// the current row, so every wave keeps one row of loads in flight. Lane l
// owns the 16-byte chunks l, l + 64, ... of every row, at most CPL of them.
//
// x is staged once per workgroup in LDS in the form the chunks consume:
// for 4-bit codes, bf16 pairs in the order the code words produce them
// (pair 4i + s of a chunk = nibbles s and s + 4 of word i), for 8-bit
// codes, f32 values; plus the sum of x over each chunk. The LDS layout is
// [m][quad][chunk] of 16-byte quads, so the 64 lanes of a wave read
// consecutive quads (no bank conflicts).

constexpr int kStreamThreads = 256;
// s_waitcnt operand: vmcnt(0), expcnt and lgkmcnt left at their maxima.
constexpr int kWaitVmcnt0 = 0x0F70;

template <int PACK>
struct ChunkTraits {
  static constexpr bool kInt4 =
      PACK == QK_PACK_U32X8 || PACK == QK_PACK_BYTE_HALFSPLIT;
  static constexpr int kCodes = kInt4 ? 32 : 16;  // codes per 16 bytes
};

// K offset of chunk c's first element and its group (half-split chunks
// also cover [kb + hg, kb + hg + 16)).
template <int PACK>
__device__ __forceinline__ void ChunkSpan(int c, int group, int* kb,
                                          int* grp) {
  if (PACK == QK_PACK_BYTE_HALFSPLIT) {
    const int hg = group / 2;
    const int byte0 = c * 16;
    *grp = byte0 / hg;
    *kb = *grp * group + byte0 % hg;
  } else {
    *kb = c * ChunkTraits<PACK>::kCodes;
    *grp = *kb / group;
  }
}

// Element (relative to the chunk's kb) of nibble `nib` of word `i`.
template <int PACK>
__device__ __forceinline__ int Int4Elem(int i, int nib, int hg) {
  if (PACK == QK_PACK_U32X8) return 8 * i + nib;
  return ((nib & 1) ? hg : 0) + 4 * i + (nib >> 1);
}

template <int PACK, typename XT>
__device__ __forceinline__ void StageX(const QmvArgs& a, int mt, int cpr,
                                       u32x4* xq, float* xs) {
  const XT* X = static_cast<const XT*>(a.x);
  const int hg = a.group / 2;
  for (int idx = threadIdx.x; idx < mt * cpr; idx += kStreamThreads) {
    const int m = idx / cpr, c = idx % cpr;
    int kb, grp;
    ChunkSpan<PACK>(c, a.group, &kb, &grp);
    const XT* xr = X + static_cast<long long>(m) * a.k + kb;
    u32x4 quad[4];
    float sum = 0.f;
    if constexpr (ChunkTraits<PACK>::kInt4) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int sh = 0; sh < 4; ++sh) {
          const float x0 = to_f32(xr[Int4Elem<PACK>(i, sh, hg)]);
          const float x1 = to_f32(xr[Int4Elem<PACK>(i, sh + 4, hg)]);
          sum += x0 + x1;
          quad[i][sh] = PackBf16Pair(x0, x1);
        }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float xv = to_f32(xr[4 * i + e]);
          sum += xv;
          quad[i][e] = __float_as_uint(xv);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) xq[(m * 4 + i) * cpr + c] = quad[i];
    xs[m * cpr + c] = sum;
  }
}

// Partial dot product of one 16-byte chunk of codes with x (m-th row):
// returns sum_e x_e * q_e, where for 4-bit codes q_e is 128 + code.
template <int PACK>
__device__ __forceinline__ float ChunkDot(const u32x4& w, const u32x4* xq,
                                          int m, int cpr, int c) {
  float d = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 xv = xq[(m * 4 + i) * cpr + c];
    const uint32_t word = w[i];
    if constexpr (ChunkTraits<PACK>::kInt4) {
#pragma unroll
      for (int sh = 0; sh < 4; ++sh) {
        const uint32_t cp = ((word >> (4 * sh)) & 0x000F000Fu) | 0x43004300u;
        const uint32_t xpair = xv[sh];
        d = __builtin_amdgcn_fdot2_f32_bf16(AsBf16x2(cp), AsBf16x2(xpair), d,
                                            false);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float q;
        if (PACK == QK_PACK_S8_SYM)
          q = static_cast<float>(static_cast<int8_t>(word >> (8 * e)));
        else
          q = static_cast<float>((word >> (8 * e)) & 255u);
        d = fmaf(__uint_as_float(xv[e]), q, d);
      }
    }
  }
  return d;
}

// Scale/offset element i: bf16 (the common case, no dtype branch) or any
// float type chosen at run time.
template <bool kBf16SB>
__device__ __forceinline__ float LoadSB(const void* p, long long i, int dt) {
  if constexpr (kBf16SB) return to_f32(static_cast<const bf16*>(p)[i]);
  return load_any(p, i, dt);
}

template <int PACK, typename XT, int MT, int CPL, bool kBf16SB>
__global__ __launch_bounds__(kStreamThreads) void qmv_stream_kernel(
    QmvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int cpr = a.row_bytes / 16;
  u32x4* xq = reinterpret_cast<u32x4*>(smem);
  float* xs = reinterpret_cast<float*>(smem + MT * 4 * cpr * 16);
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * (kStreamThreads / 64) + (threadIdx.x >> 6);
  const int GW = gridDim.x * (kStreamThreads / 64);
  const int groups = a.k / a.group;
  constexpr bool kInt4 = ChunkTraits<PACK>::kInt4;
  // Rows in flight per wave: D slots, D - 1 of them loading while one is
  // computed.
  constexpr int D = CPL <= 2 ? 4 : (CPL <= 4 ? 3 : 2);

  // Codes, scales and offsets of one row for this lane's chunks.
  struct RowRegs {
    u32x4 w[CPL];
    float s[CPL], b[CPL];
  };
  auto load_row = [&](int row, RowRegs& r) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c < cpr) {
        r.w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            a.codes + static_cast<long long>(row) * a.row_bytes + c * 16));
        int kb, grp;
        ChunkSpan<PACK>(c, a.group, &kb, &grp);
        const long long gi = static_cast<long long>(row) * groups + grp;
        r.s[j] = LoadSB<kBf16SB>(a.scales, gi, a.sdt);
        r.b[j] = a.has_bias ? LoadSB<kBf16SB>(a.biases, gi, a.bdt) : 0.f;
      }
    }
  };
  auto compute_row = [&](int row, const RowRegs& r) {
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c >= cpr) continue;
      // 4-bit codes carry +128 (see ChunkDot): fold it into the offset.
      const float boff = kInt4 ? r.b[j] - 128.f * r.s[j] : r.b[j];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m >= a.m) break;
        const float d = ChunkDot<PACK>(r.w[j], xq, m, cpr, c);
        acc[m] = fmaf(r.s[j], d, fmaf(boff, xs[m * cpr + c], acc[m]));
      }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m >= a.m) break;
      const float v = wave_sum(acc[m]);
      if (lane == 0)
        static_cast<XT*>(a.y)[static_cast<long long>(m) * a.n + row] =
            from_f32<XT>(v);
    }
  };

  RowRegs buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int r = gw + d * GW;
    if (r < a.n) load_row(r, buf[d]);  // in flight while x is staged
  }
  StageX<PACK, XT>(a, a.m, cpr, xq, xs);
  __syncthreads();

  for (int row = gw; row < a.n; row += D * GW) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int r = row + d * GW;
      if (r >= a.n) break;
      compute_row(r, buf[d]);
      const int nr = r + D * GW;
      if (nr < a.n) load_row(nr, buf[d]);
    }
  }
}

// x of one 4-bit chunk (group size 64) in registers, as loaded: the 32
// elements of a u32x8 chunk (64 contiguous bytes), or the two 16-element
// runs [kb, kb + 16) and [kb + 32, kb + 48) of a half-split chunk, with
// kb = 64 (c / 2) + 16 (c % 2).
template <int PACK>
__device__ __forceinline__ void LoadXChunk(const bf16* X, int c,
                                           u32x4 (&v)[4]) {
  if constexpr (PACK == QK_PACK_U32X8) {
    const u32x4* src = reinterpret_cast<const u32x4*>(X + 32 * c);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = src[i];
  } else {
    const bf16* base = X + 64 * (c >> 1) + 16 * (c & 1);
    const u32x4* lo = reinterpret_cast<const u32x4*>(base);
    const u32x4* hi = reinterpret_cast<const u32x4*>(base + 32);
    v[0] = lo[0], v[1] = lo[1], v[2] = hi[0], v[3] = hi[1];
  }
}

// The loaded chunk as the bf16 pairs that meet the code pairs (nibbles
// sh, sh + 4) of each code word: xp[i][sh] = (x[e(i, sh)], x[e(i, sh+4)]),
// e as in Int4Elem, one byte permute per pair; returns the chunk's sum.
template <int PACK>
__device__ __forceinline__ float XChunkPairs(const u32x4 (&v)[4],
                                             u32x4 (&xp)[4]) {
  constexpr uint32_t kLoLo = 0x05040100u, kHiHi = 0x07060302u;
  if constexpr (PACK == QK_PACK_U32X8) {
    // v[i] holds x[8i .. 8i + 8) as pairs (x0,x1) (x2,x3) (x4,x5) (x6,x7)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xp[i][0] = __builtin_amdgcn_perm(v[i][2], v[i][0], kLoLo);  // x0, x4
      xp[i][1] = __builtin_amdgcn_perm(v[i][2], v[i][0], kHiHi);  // x1, x5
      xp[i][2] = __builtin_amdgcn_perm(v[i][3], v[i][1], kLoLo);  // x2, x6
      xp[i][3] = __builtin_amdgcn_perm(v[i][3], v[i][1], kHiHi);  // x3, x7
    }
  } else {
    // word i: low nibbles are elements 4i + sh/2 of the low run (even sh)
    // or of the high run (odd sh), high nibbles the same plus 2.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4& L = v[i >> 1];
      const u32x4& H = v[2 + (i >> 1)];
      const int w = 2 * (i & 1);
      xp[i][0] = __builtin_amdgcn_perm(L[w + 1], L[w], kLoLo);
      xp[i][1] = __builtin_amdgcn_perm(H[w + 1], H[w], kLoLo);
      xp[i][2] = __builtin_amdgcn_perm(L[w + 1], L[w], kHiHi);
      xp[i][3] = __builtin_amdgcn_perm(H[w + 1], H[w], kHiHi);
    }
  }
  const uint32_t ones = 0x3F803F80u;  // bf16 (1, 1)
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int sh = 0; sh < 4; ++sh)
      sum = __builtin_amdgcn_fdot2_f32_bf16(AsBf16x2(xp[i][sh]),
                                            AsBf16x2(ones), sum, false);
  return sum;
}

// The decode hot path: M = 1, bf16 x, 4-bit codes, group size 64, bf16
// scales/offsets, rows of 128 k-chunks of 16 bytes (k a multiple of 4096
// for 4-bit codes). Lane l reads chunk 64 j + l for j < CPL, so every
// wave-wide load is 1 KB of contiguous codes. The two lanes of a pair hold
// the two halves of the same groups; one DPP swap hands each lane both
// halves of one group per chunk pair (the even lane the group of the even
// chunk, the odd lane the group of the odd one), so each lane loads one
// scale and one offset per chunk pair. x is held in registers (a lane's
// chunks are the same for every row); codes become (128 + q) bf16 pairs
// with one v_and_or_b32 each; rows are reduced with DPP.
template <int PACK, int CPL, int D>
__global__ __launch_bounds__(kStreamThreads) void qmv_m1_kernel(QmvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int cpr = 64 * CPL;
  constexpr int G = CPL / 2;  // groups per lane
  u32x4* xq = reinterpret_cast<u32x4*>(smem);
  float* xs_lds = reinterpret_cast<float*>(smem + 4 * cpr * 16);
  const int lane = threadIdx.x & 63;
  const int odd = lane & 1;
  // Row indices are wave-uniform: keep them in SGPRs, so a row's loads
  // differ only in their scalar offset.
  const int gw = __builtin_amdgcn_readfirstlane(
      blockIdx.x * (kStreamThreads / 64) + (threadIdx.x >> 6));
  const int GW = gridDim.x * (kStreamThreads / 64);
  constexpr int groups = cpr / 2;
  // Group of chunk 64 j + l is 32 j + l/2; after the swap the lane keeps,
  // for chunk pair t, group 64 t + 32 odd + l/2.
  const int goff = 32 * odd + (lane >> 1);

  // Buffer descriptors (the launcher keeps every extent under 2^31 bytes);
  // per-lane byte offsets are constants, the row offset is scalar.
  const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.codes), (short)0, a.n * a.row_bytes, 0x00020000);
  const int sb_bytes = a.n * groups * 2;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(a.scales), (short)0, sb_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(a.biases), (short)0, a.has_bias ? sb_bytes : 0,
      0x00020000);
  const int cvoff = lane * 16, svoff = goff * 2;
  constexpr int kNonTemporal = 2;  // nt: streamed once

  // Scales and offsets stay raw bf16 bits until used: converting them at
  // load time would make the prefetch wait for its own loads.
  struct Slot {
    u32x4 w[CPL];
    uint16_t s[G], b[G];
  };
  // `skip` (prologue rows past the end) moves the per-lane offsets past
  // every descriptor's extent: such loads return zeros and touch no
  // memory, and every wave issues the same loads (no branch).
  auto load_row = [&](int row, Slot& r, bool skip = false) {
    const int co = skip ? 0 : row * a.row_bytes;
    const int so = skip ? 0 : row * groups * 2;
    const int oob = skip ? 0x7FFF0000 : 0;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      r.w[j] = __builtin_amdgcn_raw_buffer_load_b128(
          crs, cvoff + oob + 1024 * j, co, kNonTemporal);
#pragma unroll
    for (int t = 0; t < G; ++t) {
      r.s[t] = __builtin_amdgcn_raw_buffer_load_b16(srs, svoff + oob + 128 * t,
                                                    so, 0);
      // A descriptor of extent 0 reads zeros when there are no offsets.
      r.b[t] = __builtin_amdgcn_raw_buffer_load_b16(brs, svoff + oob + 128 * t,
                                                    so, 0);
    }
  };

  // x is requested first: loads complete in order, so x can be staged
  // while the rows requested after it are still in flight.
  constexpr int XPT = (cpr + kStreamThreads - 1) / kStreamThreads;
  u32x4 xraw[XPT][4];
#pragma unroll
  for (int q = 0; q < XPT; ++q) {
    const int c = threadIdx.x + q * kStreamThreads;
    if (c < cpr) LoadXChunk<PACK>(static_cast<const bf16*>(a.x), c, xraw[q]);
  }
  Slot buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int r = gw + d * GW;
    load_row(r, buf[d], r >= a.n);
  }
#pragma unroll
  for (int q = 0; q < XPT; ++q) {
    const int c = threadIdx.x + q * kStreamThreads;
    if (c < cpr) {
      u32x4 quad[4];
      xs_lds[c] = XChunkPairs<PACK>(xraw[q], quad);
#pragma unroll
      for (int i = 0; i < 4; ++i) xq[i * cpr + c] = quad[i];
    }
  }
  __syncthreads();
  u32x4 xr[CPL][4];
  float xsum[G];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) xr[j][i] = xq[i * cpr + 64 * j + lane];
  }
#pragma unroll
  for (int t = 0; t < G; ++t) {
    const int g = 64 * t + goff;
    xsum[t] = xs_lds[2 * g] + xs_lds[2 * g + 1];
  }
  const uint32_t kMask = vgpr_const(0x000F000Fu);
  const uint32_t kBias = vgpr_const(0x43004300u);

  // Partial dot product of this lane's chunks with one row.
  auto row_acc = [&](const Slot& r) {
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < G; ++t) {
      float d[2] = {0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * t + jj;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          // Words 2p and 2p+1 shifted together: the bits the low word
          // takes from the high one land above bit 19, outside kMask.
          const uint64_t v = (static_cast<uint64_t>(r.w[j][2 * p + 1]) << 32) |
                             r.w[j][2 * p];
          const uint64_t sv[4] = {v, shr64<4>(v), shr64<8>(v), shr64<12>(v)};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int i = 2 * p + h;
#pragma unroll
            for (int sh = 0; sh < 4; ++sh) {
              const uint32_t word = static_cast<uint32_t>(sv[sh] >> (32 * h));
              const uint32_t cp = (word & kMask) | kBias;
              const uint32_t xp = xr[j][i][sh];
              d[jj] = __builtin_amdgcn_fdot2_f32_bf16(
                  AsBf16x2(cp), AsBf16x2(xp), d[jj], false);
            }
          }
        }
      }
      // Keep the half of the own group, pass the partner its half.
      const float keep = odd ? d[1] : d[0];
      const float give = odd ? d[0] : d[1];
      const float dg = keep + dpp_f32<0xB1>(give);  // swap within lane pairs
      const float sc = __uint_as_float(static_cast<uint32_t>(r.s[t]) << 16);
      const float of = __uint_as_float(static_cast<uint32_t>(r.b[t]) << 16);
      acc = fmaf(sc, dg, fmaf(of - 128.f * sc, xsum[t], acc));
    }
    return acc;
  };

  bf16* Y = static_cast<bf16*>(a.y);
  int row = gw;
  static_assert(D == 2 || D % 4 == 0, "rows are reduced four at a time");
  constexpr int DA = D < 4 ? 4 : D;  // accumulators, padded to fours
  // Reduce one round's partial sums and store rows row + d GW < N.
  auto finish = [&](const float (&acc)[DA]) {
    if (row + GW >= a.n) {  // one row this round (small matrices)
      const float v = wave_sum_dpp(acc[0]);
      if (lane == 0) Y[row] = from_f32<bf16>(v);
    } else {
      // Lane l < 4 gets the total of row row + (q + l) * GW.
#pragma unroll
      for (int q = 0; q < DA; q += 4) {
        const float v = wave_sum4(acc[q], acc[q + 1], acc[q + 2], acc[q + 3],
                                  lane);
        const int rr = row + (q + (lane & 3)) * GW;
        if (lane < 4 && q + lane < D && rr < a.n) Y[rr] = from_f32<bf16>(v);
      }
    }
  };
  if (row + D * GW >= a.n) {
    // All of this wave's rows are in its first slots (one round): each row
    // is computed as soon as its own loads have landed (the loads complete
    // in order), while the later rows are still in flight.
    float acc[DA] = {};
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (row + d * GW < a.n) acc[d] = row_acc(buf[d]);
    finish(acc);
    return;
  }
  // Every wave waits for its first slots here. The loop below then starts
  // from "nothing outstanding", so its waits follow the loop body's own
  // load order; without this, merging the prologue's order makes them
  // wait for whole rounds of prefetch.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  // Steady state: this round's rows and the next round's are all in
  // range, so the prefetch is unconditional (no merge of old and new
  // slot contents that would wait on the loads just issued).
  for (; row + (2 * D - 1) * GW < a.n; row += D * GW) {
    float acc[DA] = {};
#pragma unroll
    for (int d = 0; d < D; ++d) {
      acc[d] = row_acc(buf[d]);
      load_row(row + (d + D) * GW, buf[d]);
    }
#pragma unroll
    for (int q = 0; q < DA; q += 4) {
      const float v = wave_sum4(acc[q], acc[q + 1], acc[q + 2], acc[q + 3],
                                lane);
      if (lane < 4 && q + lane < D) Y[row + (q + lane) * GW] = from_f32<bf16>(v);
    }
  }
  for (; row < a.n; row += D * GW) {
    float acc[DA] = {};
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int r = row + d * GW;
      if (r < a.n) {
        acc[d] = row_acc(buf[d]);
        const int nr = r + D * GW;
        if (nr < a.n) load_row(nr, buf[d]);
      }
    }
    finish(acc);
  }
}

// The int8 decode path: M = 1, bf16 x, u8 or s8 codes, group size 64, bf16
// scales/offsets, k a multiple of 4096 (CPL = k / 1024 16-byte chunks per
// lane, a multiple of 4; 4, 8 or 12 here). Lane l reads chunk 64 j + l, so every wave-wide
// load is 1 KB of contiguous codes; chunk 64 j + l belongs to group
// 16 j + l / 4, so the four lanes of a quad hold the four chunks of the
// same groups. After a two-step DPP transpose inside the quad each lane
// holds the full dot product of one group per four chunks (lane l: chunk
// 4 u + l % 4), so it loads one scale and one offset per four chunks.
// Codes convert exactly to bf16 (integers up to 256; signed codes are
// flipped to q + 128 and the 128 removed per group) and meet x pairs in
// v_dot2_f32_bf16. Rows are reduced four at a time as in the int4 kernel.
template <int PACK, int CPL, int D>
__global__ __launch_bounds__(kStreamThreads) void qmv_m1_i8_kernel(QmvArgs a) {
  static_assert(CPL % 4 == 0, "quads of chunks");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int cpr = 64 * CPL;   // 16-byte chunks per row
  constexpr int U = CPL / 4;      // groups per lane
  constexpr int groups = cpr / 4;
  u32x4* xl = reinterpret_cast<u32x4*>(smem);  // x as loaded, [2 cpr]
  const int lane = threadIdx.x & 63;
  const int q4 = lane & 3;
  const int gw = __builtin_amdgcn_readfirstlane(
      blockIdx.x * (kStreamThreads / 64) + (threadIdx.x >> 6));
  const int GW = gridDim.x * (kStreamThreads / 64);

  const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.codes), (short)0, a.n * a.row_bytes, 0x00020000);
  const int sb_bytes = a.n * groups * 2;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(a.scales), (short)0, sb_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(a.biases), (short)0, a.has_bias ? sb_bytes : 0,
      0x00020000);
  // Lane l keeps, for u < U, the group of chunk 64 (4 u + l % 4) + l:
  // 16 (4 u + l % 4) + l / 4.
  const int cvoff = lane * 16;
  const int svoff = (16 * q4 + (lane >> 2)) * 2;
  constexpr int kNonTemporal = 2;

  struct Slot {
    u32x4 w[CPL];
    uint16_t s[U], b[U];
  };
  auto load_row = [&](int row, Slot& r, bool skip = false) {
    const int co = skip ? 0 : row * a.row_bytes;
    const int so = skip ? 0 : row * groups * 2;
    const int oob = skip ? 0x7FFF0000 : 0;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      r.w[j] = __builtin_amdgcn_raw_buffer_load_b128(
          crs, cvoff + oob + 1024 * j, co, kNonTemporal);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      r.s[u] = __builtin_amdgcn_raw_buffer_load_b16(srs, svoff + oob + 128 * u,
                                                    so, 0);
      r.b[u] = __builtin_amdgcn_raw_buffer_load_b16(brs, svoff + oob + 128 * u,
                                                    so, 0);
    }
  };

  // x first (loads complete in order), then the first rows; x goes through
  // LDS once per workgroup.
  constexpr int XV = 2 * cpr;  // 16-byte vectors of x
  constexpr int XPT = (XV + kStreamThreads - 1) / kStreamThreads;
  u32x4 xraw[XPT];
  const u32x4* X = static_cast<const u32x4*>(a.x);
#pragma unroll
  for (int q = 0; q < XPT; ++q) {
    const int c = threadIdx.x + q * kStreamThreads;
    if (c < XV) xraw[q] = X[c];
  }
  Slot buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int r = gw + d * GW;
    load_row(r, buf[d], r >= a.n);
  }
#pragma unroll
  for (int q = 0; q < XPT; ++q) {
    const int c = threadIdx.x + q * kStreamThreads;
    if (c < XV) xl[c] = xraw[q];
  }
  __syncthreads();
  // The lane's x: chunk 64 j + l covers x[16 (64 j + l) ...], two vectors.
  u32x4 xr[CPL][2];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) xr[j][h] = xl[2 * (64 * j + lane) + h];
  const uint32_t ones = 0x3F803F80u;  // bf16 (1, 1)

  // Quad transpose: lane l gets the quad sum of v[4 u + l % 4].
  auto quad4 = [&](float v0, float v1, float v2, float v3) {
    const bool b0 = lane & 1, b1 = lane & 2;
    const float v01 = (b0 ? v1 : v0) + dpp_f32<0xB1>(b0 ? v0 : v1);
    const float v23 = (b0 ? v3 : v2) + dpp_f32<0xB1>(b0 ? v2 : v3);
    return (b1 ? v23 : v01) + dpp_f32<0x4E>(b1 ? v01 : v23);
  };
  float xsum[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float cs[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float sacc = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          sacc = __builtin_amdgcn_fdot2_f32_bf16(
              AsBf16x2(xr[4 * u + jj][h][e]), AsBf16x2(ones), sacc, false);
      cs[jj] = sacc;
    }
    xsum[u] = quad4(cs[0], cs[1], cs[2], cs[3]);
  }

  // Two codes (bytes of w at 8 c and 8 c + 8) as a bf16 pair.
  auto code2 = [](uint32_t w, int c) {
    const float lo = static_cast<float>((w >> (16 * c)) & 0xFFu);
    const float hi = static_cast<float>((w >> (16 * c + 8)) & 0xFFu);
    const bf16x2 p = {from_f32<bf16>(lo), from_f32<bf16>(hi)};
    return p;
  };
  auto row_acc = [&](const Slot& r) {
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float dj[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = 4 * u + jj;
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t w = r.w[j][i];
          if (PACK == QK_PACK_S8_SYM) w ^= 0x80808080u;
#pragma unroll
          for (int c = 0; c < 2; ++c)
            d = __builtin_amdgcn_fdot2_f32_bf16(
                code2(w, c), AsBf16x2(xr[j][i >> 1][2 * (i & 1) + c]), d,
                false);
        }
        dj[jj] = d;
      }
      const float dg = quad4(dj[0], dj[1], dj[2], dj[3]);
      const float sc = __uint_as_float(static_cast<uint32_t>(r.s[u]) << 16);
      const float of = __uint_as_float(static_cast<uint32_t>(r.b[u]) << 16);
      const float off = PACK == QK_PACK_S8_SYM ? of - 128.f * sc : of;
      acc = fmaf(sc, dg, fmaf(off, xsum[u], acc));
    }
    return acc;
  };

  bf16* Y = static_cast<bf16*>(a.y);
  int row = gw;
  static_assert(D == 2 || D % 4 == 0, "rows are reduced four at a time");
  constexpr int DA = D < 4 ? 4 : D;
  // Reduce one round's partial sums and store rows row + d GW < N.
  auto finish = [&](const float (&acc)[DA]) {
    if (row + GW >= a.n) {
      const float v = wave_sum_dpp(acc[0]);
      if (lane == 0) Y[row] = from_f32<bf16>(v);
    } else {
#pragma unroll
      for (int q = 0; q < DA; q += 4) {
        const float v = wave_sum4(acc[q], acc[q + 1], acc[q + 2], acc[q + 3],
                                  lane);
        const int rr = row + (q + (lane & 3)) * GW;
        if (lane < 4 && q + lane < D && rr < a.n) Y[rr] = from_f32<bf16>(v);
      }
    }
  };
  if (row + D * GW >= a.n) {
    // All of this wave's rows are in its first slots (one round): each row
    // is computed as soon as its own loads have landed.
    float acc[DA] = {};
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (row + d * GW < a.n) acc[d] = row_acc(buf[d]);
    finish(acc);
    return;
  }
  // The loop below starts from "nothing outstanding" (as in qmv_m1_kernel).
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  for (; row + (2 * D - 1) * GW < a.n; row += D * GW) {
    float acc[DA] = {};
#pragma unroll
    for (int d = 0; d < D; ++d) {
      acc[d] = row_acc(buf[d]);
      load_row(row + (d + D) * GW, buf[d]);
    }
#pragma unroll
    for (int q = 0; q < DA; q += 4) {
      const float v = wave_sum4(acc[q], acc[q + 1], acc[q + 2], acc[q + 3],
                                lane);
      if (lane < 4 && q + lane < D) Y[row + (q + lane) * GW] = from_f32<bf16>(v);
    }
  }
  for (; row < a.n; row += D * GW) {
    float acc[DA] = {};
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int r = row + d * GW;
      if (r < a.n) {
        acc[d] = row_acc(buf[d]);
        const int nr = r + D * GW;
        if (nr < a.n) load_row(nr, buf[d]);
      }
    }
    finish(acc);
  }
}

// QK_QMV_WG_PER_CU=<n> sets the workgroups per CU of the streaming
// kernels, within what stays resident (tuning only); 0 when unset.
int QmvWgPerCu() {
  static const int n = [] {
    const char* v = std::getenv("QK_QMV_WG_PER_CU");
    if (v == nullptr || *v < '1' || *v > '9') return 0;
    return std::atoi(v);
  }();
  return n;
}

// QK_QMV_M1_DEPTH=<2|4|8> forces the rows each decode wave keeps in
// flight (tuning only).
int M1DepthForced() {
  static const int d = [] {
    const char* v = std::getenv("QK_QMV_M1_DEPTH");
    if (v == nullptr || *v < '1' || *v > '9') return 0;
    const int x = std::atoi(v);
    return x == 2 || x == 4 || x == 8 ? x : 0;
  }();
  return d;
}

// Workgroups per CU for the M = 1 kernels: the fewest (2..6) for which
// every wave's rows fit its first `depth` slots (one round: each row is
// then computed as soon as it lands, none waits for a ring refill), else
// 2. Measured at 12288 x 4096: 6 per CU (one round) 6.9 us int4 and
// 10.7 us int8 against 7.2 and 11.0 us with 2 (three rounds); where 2
// already give one round (4096 rows), more workgroups only cost.
int SingleRoundWgPerCu(int n, int cus, int depth) {
  const int waves = kStreamThreads / 64;
  for (int wg = 2; wg <= 6; ++wg)
    if (static_cast<int64_t>(cus) * wg * waves * depth >= n) return wg;
  return 2;
}

template <int PACK>
bool LaunchM1(const QmvArgs& a, int cus, hipStream_t stream, qk_status* st) {
  const int cpr = a.row_bytes / 16;
  if (a.m != 1 || a.group != 64 || cpr % 128 != 0) return false;
  // Buffer descriptors cover at most 2^31 bytes of codes.
  if (static_cast<int64_t>(a.n) * a.row_bytes >= (int64_t{1} << 31))
    return false;
  const int cpl = cpr / 64;
  const size_t lds = static_cast<size_t>(cpr) * (64 + 4);
  const int need = (a.n + 3) / 4;
  // About four rows in flight per SIMD: one workgroup per CU with four
  // rows per wave for long matrices of 4096-wide rows, else two
  // workgroups per CU with two rows per wave. Measured on MI355X at the
  // Qwen3-8B decode shapes, this beats full occupancy by 10-20%.
  const bool deep = cpl == 2 && a.n >= 32768;
  const int dflt_depth = deep ? 4 : 2;
  const int dflt_wg = deep ? 1 : SingleRoundWgPerCu(a.n, cus, dflt_depth);
  auto go = [&](auto kernel) {
    const int resident = ResidentBlocks(reinterpret_cast<const void*>(kernel),
                                        kStreamThreads, lds);
    const int per_cu = std::min(QmvWgPerCu() ? QmvWgPerCu() : dflt_wg, resident);
    const int grid = std::max(1, std::min(need, cus * per_cu));
    kernel<<<grid, kStreamThreads, lds, stream>>>(a);
    *st = PostLaunch("qmv_m1");
    return true;
  };
  auto depth = [&](auto k2, auto k4, auto k8, int dflt) {
    const int d = M1DepthForced() ? M1DepthForced() : dflt;
    return d == 2 ? go(k2) : d == 8 ? go(k8) : go(k4);
  };
  switch (cpl) {
    case 2:
      return depth(qmv_m1_kernel<PACK, 2, 2>, qmv_m1_kernel<PACK, 2, 4>,
                   qmv_m1_kernel<PACK, 2, 8>, dflt_depth);
    case 4:
      return depth(qmv_m1_kernel<PACK, 4, 2>, qmv_m1_kernel<PACK, 4, 4>,
                   qmv_m1_kernel<PACK, 4, 8>, dflt_depth);
    case 6:
      return depth(qmv_m1_kernel<PACK, 6, 2>, qmv_m1_kernel<PACK, 6, 4>,
                   qmv_m1_kernel<PACK, 6, 8>, dflt_depth);
    case 8:
      return depth(qmv_m1_kernel<PACK, 8, 2>, qmv_m1_kernel<PACK, 8, 4>,
                   qmv_m1_kernel<PACK, 8, 8>, dflt_depth);
    default:
      return false;
  }
}

template <int PACK>
bool LaunchM1I8(const QmvArgs& a, int cus, hipStream_t stream, qk_status* st) {
  const int cpr = a.row_bytes / 16;  // int8: row_bytes = k
  if (a.m != 1 || a.group != 64 || cpr % 256 != 0) return false;
  if (static_cast<int64_t>(a.n) * a.row_bytes >= (int64_t{1} << 31))
    return false;
  const int cpl = cpr / 64;
  const size_t lds = static_cast<size_t>(2 * cpr) * 16;
  const int need = (a.n + 3) / 4;
  auto go = [&](auto kernel) {
    const int resident = ResidentBlocks(reinterpret_cast<const void*>(kernel),
                                        kStreamThreads, lds);
    const int per_cu = std::min(
        QmvWgPerCu() ? QmvWgPerCu() : SingleRoundWgPerCu(a.n, cus, 2),
        resident);
    const int grid = std::max(1, std::min(need, cus * per_cu));
    kernel<<<grid, kStreamThreads, lds, stream>>>(a);
    *st = PostLaunch("qmv_m1_i8");
    return true;
  };
  switch (cpl) {
    case 4:
      return go(qmv_m1_i8_kernel<PACK, 4, 2>);
    case 8:
      return go(qmv_m1_i8_kernel<PACK, 8, 2>);
    case 12:
      return go(qmv_m1_i8_kernel<PACK, 12, 2>);
    default:
      return false;
  }
}

template <int PACK, typename XT, int MT, bool kBf16SB>
qk_status LaunchStreamMT(QmvArgs a, int cpl, int cus, hipStream_t st) {
  const int cpr = a.row_bytes / 16;
  const size_t lds = static_cast<size_t>(MT) * cpr * (64 + 4);
  const int rows_per_wg = kStreamThreads / 64;
  const int need = (a.n + rows_per_wg - 1) / rows_per_wg;
  // As many workgroups as the GPU keeps resident (each wave then walks
  // its rows with a prefetch), at most one row per wave.
  auto go = [&](auto kernel) {
    const int resident = ResidentBlocks(reinterpret_cast<const void*>(kernel),
                                        kStreamThreads, lds);
    const int per_cu = QmvWgPerCu() ? std::min(QmvWgPerCu(), resident)
                                    : resident;
    const int grid = std::max(1, std::min(need, cus * per_cu));
    kernel<<<grid, kStreamThreads, lds, st>>>(a);
    return PostLaunch("qmv_stream");
  };
  switch (cpl) {
    case 1:
      return go(qmv_stream_kernel<PACK, XT, MT, 1, kBf16SB>);
    case 2:
      return go(qmv_stream_kernel<PACK, XT, MT, 2, kBf16SB>);
    case 4:
      return go(qmv_stream_kernel<PACK, XT, MT, 4, kBf16SB>);
    case 6:
      return go(qmv_stream_kernel<PACK, XT, MT, 6, kBf16SB>);
    default:
      return go(qmv_stream_kernel<PACK, XT, MT, 8, kBf16SB>);
  }
}

// M <= 4 rows; false when this path does not apply (then *st is unset).
template <int PACK, typename XT>
bool LaunchStream(const QmvArgs& a, int cus, hipStream_t stream,
                  qk_status* st) {
  const int cpr = a.row_bytes / 16;
  // The decode case (bf16 x, bf16 scales) gets kernels per row count;
  // everything else runs the four-row kernel with masked rows.
  const bool sb16 = a.sdt == QK_BF16 && (!a.has_bias || a.bdt == QK_BF16);
  const bool fast = sb16 && std::is_same<XT, bf16>::value;
  if constexpr (PACK == QK_PACK_U8 || PACK == QK_PACK_S8_SYM) {
    if (fast && a.m == 1 && LaunchM1I8<PACK>(a, cus, stream, st)) return true;
  }
  int cpl = (cpr + 63) / 64;
  if (cpl > 8 || a.m > 4) return false;
  if (cpl == 3) cpl = 4;
  if (cpl == 5) cpl = 6;
  if (cpl == 7) cpl = 8;
  const int mt = !fast ? 4 : a.m <= 1 ? 1 : a.m <= 2 ? 2 : 4;
  const size_t lds = static_cast<size_t>(mt) * cpr * (64 + 4);
  if (lds > 64 * 1024) return false;
  if (fast && a.m == 1 && ChunkTraits<PACK>::kInt4 && lds <= 64 * 1024 &&
      LaunchM1<PACK>(a, cus, stream, st)) {
    return true;
  }
  if (fast) {
    if (mt == 1)
      *st = LaunchStreamMT<PACK, XT, 1, true>(a, cpl, cus, stream);
    else if (mt == 2)
      *st = LaunchStreamMT<PACK, XT, 2, true>(a, cpl, cus, stream);
    else
      *st = LaunchStreamMT<PACK, XT, 4, true>(a, cpl, cus, stream);
  } else {
    *st = LaunchStreamMT<PACK, XT, 4, false>(a, cpl, cus, stream);
  }
  return true;
}

int RowBytes(const QuantProblem& p) {
  return static_cast<int>(p.bits == 4 ? p.k / 2 : p.k);
}

template <typename XT, int PACK>
qk_status LaunchGeneric(QmvArgs a, int m_total, int xsize, hipStream_t st) {
  constexpr int MT = 4, R = 4;
  const int waves = (a.n + R - 1) / R;
  dim3 grid((waves + kWaves - 1) / kWaves), block(kWaves * 64);
  const char* base_x = static_cast<const char*>(a.x);
  char* base_y = static_cast<char*>(a.y);
  for (int m0 = 0; m0 < m_total; m0 += MT) {
    a.m = m_total - m0 < MT ? m_total - m0 : MT;
    a.x = base_x + static_cast<long long>(m0) * a.k * xsize;
    a.y = base_y + static_cast<long long>(m0) * a.n * xsize;
    qmv_generic_kernel<XT, PACK, MT, R><<<grid, block, 0, st>>>(a);
    if (qk_status s = PostLaunch("qmv_generic"); s != QK_OK) return s;
  }
  return QK_OK;
}

template <int PACK>
qk_status LaunchInt4Bf16(QmvArgs a, int m_total, hipStream_t st) {
  constexpr int R = 4;
  const int waves = (a.n + R - 1) / R;
  dim3 grid((waves + kWaves - 1) / kWaves), block(kWaves * 64);
  const char* base_x = static_cast<const char*>(a.x);
  char* base_y = static_cast<char*>(a.y);
  for (int m0 = 0; m0 < m_total;) {
    const int left = m_total - m0;
    a.x = base_x + static_cast<long long>(m0) * a.k * 2;
    a.y = base_y + static_cast<long long>(m0) * a.n * 2;
    if (left == 1) {
      a.m = 1;
      qmv_int4_bf16_kernel<PACK, 1, R><<<grid, block, 0, st>>>(a);
      m0 += 1;
    } else if (left == 2) {
      a.m = 2;
      qmv_int4_bf16_kernel<PACK, 2, R><<<grid, block, 0, st>>>(a);
      m0 += 2;
    } else {
      a.m = left < 4 ? left : 4;
      qmv_int4_bf16_kernel<PACK, 4, R><<<grid, block, 0, st>>>(a);
      m0 += a.m;
    }
    if (qk_status s = PostLaunch("qmv_int4_bf16"); s != QK_OK) return s;
  }
  return QK_OK;
}

QmvArgs MakeArgs(const QuantProblem& p) {
  QmvArgs a;
  a.x = p.x;
  a.codes = static_cast<const uint8_t*>(p.codes);
  a.scales = p.scales;
  a.biases = p.biases;
  a.y = p.y;
  a.m = static_cast<int>(p.m);
  a.n = static_cast<int>(p.n);
  a.k = static_cast<int>(p.k);
  a.group = p.group;
  a.sdt = p.scale_dtype;
  a.bdt = p.bias_dtype;
  a.has_bias = p.has_bias;
  a.row_bytes = RowBytes(p);
  a.gather = static_cast<const int*>(p.rows);
  a.out_vec = 0;
  return a;
}

qk_status CheckLimits(const QuantProblem& p) {
  if (p.n > 0x7fffffff || p.k > 0x7fffffff || p.m > 0x7fffffff ||
      p.n * (p.k / p.group) > (int64_t{1} << 40)) {
    return Fail(QK_UNIMPLEMENTED, "qkern: quantized matrix too large");
  }
  if (reinterpret_cast<uintptr_t>(p.codes) % 16 != 0) {
    return Fail(QK_INVALID_ARGUMENT,
                "qkern: quantized codes must be 16-byte aligned");
  }
  return QK_OK;
}

}  // namespace

qk_status LaunchQMatvec(const QuantProblem& p, hipStream_t stream) {
  if (qk_status s = CheckLimits(p); s != QK_OK) return s;
  if (reinterpret_cast<uintptr_t>(p.x) % 16 != 0) {
    return Fail(QK_INVALID_ARGUMENT, "qkern: qmatvec x must be 16-byte aligned");
  }
  QmvArgs a = MakeArgs(p);
  const int m = static_cast<int>(p.m);
  // Beyond four rows the reference's linear() (ROWS_MAX = 4,
  // examples/llm/qwen3.py:215-230) dequantizes to x's type and multiplies.
  // Up to 32 rows (int4 and int8) stream through MFMA with the codes kept
  // factored per group (qskinny.hip); 33..64 rows dequantize in registers
  // with K split over the waves of a workgroup (qmid.hip); beyond, and
  // where qmid does not apply, dequantize in registers into the MFMA
  // operands of one GEMM (qgemm_dma.hip, K split over workgroups when
  // the tiles alone would not fill the CUs; other packings qgemm.hip).
  // QK_QGEMM_DMA_MIN_M: fewest rows for the register-dequantizing GEMM
  // (tuning; read at every call).
  const char* dmv = std::getenv("QK_QGEMM_DMA_MIN_M");
  const int dma_min_m = dmv == nullptr ? 33 : std::atoi(dmv);
  // QK_QSTREAM=0 turns the streamed MFMA kernel off, =2 takes it wherever
  // it applies (tuning; read at every call).
  const char* qsv = std::getenv("QK_QSTREAM");
  const bool qstream = qsv == nullptr || *qsv != '0';
  const bool qstream_all = qsv != nullptr && *qsv == '2';
  // The streamed MFMA kernel with x in registers where each of its waves
  // runs at least three row-block rounds (int4, <= 16 rows, K <= 4096: the
  // lm_head, 74 against 118 us at M = 16; 12288 x 4096 11 against 12);
  // with fewer, reading all of x per workgroup costs more than the skinny
  // kernels' single round (8192 x 4096 10 against 8).
  // From two rows on, the MFMA streaming kernels beat the dot-product
  // streams (int8 12288 x 4096: M = 2 / 4 21.3 / 30.5 us on the streams,
  // 14.6 us for M = 5 on the skinny kernel). QK_QMV_MFMA_MIN_M: fewest rows
  // for them (tuning; read at every call).
  const char* mmv = std::getenv("QK_QMV_MFMA_MIN_M");
  const int mfma_min_m = mmv == nullptr ? 2 : std::max(2, std::atoi(mmv));
  if (m >= mfma_min_m && qstream && QStreamApplies(p) &&
      (qstream_all || QStreamRounds(p, DeviceComputeUnits()) >= 3))
    return LaunchQStream(p, stream);
  if (m >= mfma_min_m && QSkinnyApplies(p)) return LaunchQSkinny(p, stream);
  // 33..64 rows: the K-split dequantizing kernel where it applies (int4
  // 12288 x 4096: 21 / 24 us at M = 33 / 64 against 31 for the GEMM).
  const bool mid = m > 4 && QMidApplies(p);
  if (m >= dma_min_m && (m > 64 || !mid) && QGemmDmaApplies(p))
    return LaunchQGemmDma(p, stream);
  if (mid) return LaunchQMid(p, stream);
  if (m > 4 && QGemmApplies(p)) return LaunchQGemm(p, stream);
  if (m <= 4) {
    const int cus = DeviceComputeUnits();
    qk_status st = QK_OK;
    bool done = false;
    if (p.x_dtype == QK_BF16 && p.packing == QK_PACK_U32X8)
      done = LaunchStream<QK_PACK_U32X8, bf16>(a, cus, stream, &st);
    else if (p.x_dtype == QK_BF16 && p.packing == QK_PACK_BYTE_HALFSPLIT)
      done = LaunchStream<QK_PACK_BYTE_HALFSPLIT, bf16>(a, cus, stream, &st);
    else if (p.packing == QK_PACK_U8 || p.packing == QK_PACK_S8_SYM) {
      const bool u8 = p.packing == QK_PACK_U8;
      if (p.x_dtype == QK_BF16)
        done = u8 ? LaunchStream<QK_PACK_U8, bf16>(a, cus, stream, &st)
                  : LaunchStream<QK_PACK_S8_SYM, bf16>(a, cus, stream, &st);
      else if (p.x_dtype == QK_F16)
        done = u8 ? LaunchStream<QK_PACK_U8, f16>(a, cus, stream, &st)
                  : LaunchStream<QK_PACK_S8_SYM, f16>(a, cus, stream, &st);
      else
        done = u8 ? LaunchStream<QK_PACK_U8, float>(a, cus, stream, &st)
                  : LaunchStream<QK_PACK_S8_SYM, float>(a, cus, stream, &st);
    }
    if (done) return st;
  }
  if (p.x_dtype == QK_BF16 && p.packing == QK_PACK_U32X8)
    return LaunchInt4Bf16<QK_PACK_U32X8>(a, m, stream);
  if (p.x_dtype == QK_BF16 && p.packing == QK_PACK_BYTE_HALFSPLIT)
    return LaunchInt4Bf16<QK_PACK_BYTE_HALFSPLIT>(a, m, stream);
#define QK_GENERIC(XT, XS)                                                 \
  switch (p.packing) {                                                     \
    case QK_PACK_U32X8:                                                    \
      return LaunchGeneric<XT, QK_PACK_U32X8>(a, m, XS, stream);           \
    case QK_PACK_BYTE_HALFSPLIT:                                           \
      return LaunchGeneric<XT, QK_PACK_BYTE_HALFSPLIT>(a, m, XS, stream);  \
    case QK_PACK_U8:                                                       \
      return LaunchGeneric<XT, QK_PACK_U8>(a, m, XS, stream);              \
    default:                                                               \
      return LaunchGeneric<XT, QK_PACK_S8_SYM>(a, m, XS, stream);          \
  }
  if (p.x_dtype == QK_BF16) {
    QK_GENERIC(bf16, 2)
  } else if (p.x_dtype == QK_F16) {
    QK_GENERIC(f16, 2)
  } else {
    QK_GENERIC(float, 4)
  }
#undef QK_GENERIC
}

qk_status LaunchDequantize(const QuantProblem& p, hipStream_t stream) {
  if (qk_status s = CheckLimits(p); s != QK_OK) return s;
  QmvArgs a = MakeArgs(p);
  // Every 8-value run starts at a multiple of 8 elements of its row.
  a.out_vec = reinterpret_cast<uintptr_t>(p.y) % 16 == 0 &&
              (p.k * DTypeSize(p.y_dtype)) % 16 == 0;
  const long long rows = p.rows != nullptr ? p.rows_n : p.n;
  const int unit = p.packing == QK_PACK_U32X8 ? 4 : 8;
  const long long units = rows * (a.row_bytes / unit);
  if (units == 0) return QK_OK;  // (the kernel clamps into [0, units))
  // Units per thread: 1 (2 measured level for the int4 embedding gather).
  constexpr int kUpt = 1;
  dim3 block(256), grid(static_cast<unsigned>((units + 256 * kUpt - 1) /
                                             (256 * kUpt)));
  if (units / (256 * kUpt) >= 0x7fffffffLL) {
    return Fail(QK_UNIMPLEMENTED, "qkern: dequantize grid too large");
  }
#define QK_DQ(OT)                                                              \
  switch (p.packing) {                                                         \
    case QK_PACK_U32X8:                                                        \
      dequant_kernel<QK_PACK_U32X8, OT, kUpt><<<grid, block, 0, stream>>>(a, units); \
      break;                                                                   \
    case QK_PACK_BYTE_HALFSPLIT:                                               \
      dequant_kernel<QK_PACK_BYTE_HALFSPLIT, OT, kUpt>                         \
          <<<grid, block, 0, stream>>>(a, units);                              \
      break;                                                                   \
    case QK_PACK_U8:                                                           \
      dequant_kernel<QK_PACK_U8, OT, kUpt><<<grid, block, 0, stream>>>(a, units);    \
      break;                                                                   \
    default:                                                                   \
      dequant_kernel<QK_PACK_S8_SYM, OT, kUpt><<<grid, block, 0, stream>>>(a, units); \
  }
  if (p.y_dtype == QK_BF16) {
    QK_DQ(bf16)
  } else if (p.y_dtype == QK_F16) {
    QK_DQ(f16)
  } else {
    QK_DQ(float)
  }
#undef QK_DQ
  return PostLaunch(p.rows != nullptr ? "embed_dequantize" : "dequantize");
}

namespace {
// One thread per 16-byte chunk of an output row: out[t] = table[rows[t]].
__global__ void row_gather_kernel(const uint8_t* table, long long ld_bytes,
                                  int n, int row_chunks, const int* rows,
                                  long long total, uint8_t* out) {
  const long long t = static_cast<long long>(blockIdx.x) * blockDim.x +
                      threadIdx.x;
  if (t >= total) return;
  const long long orow = t / row_chunks;
  const int c = static_cast<int>(t % row_chunks);
  const int r = min(max(rows[orow], 0), n - 1);
  *reinterpret_cast<u32x4*>(out + (orow * row_chunks + c) * 16) =
      *reinterpret_cast<const u32x4*>(table + r * ld_bytes + c * 16);
}
}  // namespace

qk_status LaunchRowGather(const void* table, int64_t n, int64_t k, int64_t ld,
                          int esz, const void* rows, int64_t rows_n, void* out,
                          hipStream_t stream) {
  const int64_t row_bytes = k * esz;
  if (row_bytes % 16 != 0 || (ld * esz) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(table) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(out) % 16 != 0) {
    return Fail(QK_UNIMPLEMENTED,
                "qkern: embedding gather needs 16-byte aligned tables, "
                "outputs and rows");
  }
  if (n > 0x7fffffff || row_bytes / 16 > 0x7fffffff) {
    return Fail(QK_UNIMPLEMENTED, "qkern: embedding table too large");
  }
  const long long total = rows_n * (row_bytes / 16);
  if (total == 0) return QK_OK;
  row_gather_kernel<<<static_cast<unsigned>((total + 255) / 256), 256, 0,
                      stream>>>(
      static_cast<const uint8_t*>(table), ld * esz, static_cast<int>(n),
      static_cast<int>(row_bytes / 16), static_cast<const int*>(rows), total,
      static_cast<uint8_t*>(out));
  return PostLaunch("embed_gather");
}

}  // namespace qk
