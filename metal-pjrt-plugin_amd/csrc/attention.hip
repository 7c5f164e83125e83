// Decode attention for gfx950: one query per sequence against a KV cache
// window, grouped-query heads, as a split-window (flash-decoding) pair of
// kernels.
//
// Replaces the reductions XLA emits for the one-query branch of the
// reference's attention() (examples/llm/qwen3.py:322-326) with forward()'s
// decode mask (:357-358). Per batch b, KV head h and query head g of that
// KV head, over the cache slots s < window with s <= pos:
//   t[s] = sum_d q[b,h,g,d] * k[b,h,s,d] * scale             (f32)
//   p    = softmax(t)  (masked slots excluded)                 (f32)
//   o[d] = sum_s p[s] * v[b,h,d,s]                             (f32)
// rounded once to the cache type. The cache layouts are the reference's
// init_cache (qwen3.py:279-291): keys [B, KV, Smax, D], values
// [B, KV, D, Smax], each with the reduced axis last.
//
// attn_split_kernel: one wavefront per (b, h, run of cpw 64-slot chunks).
// Scores come from v_mfma_f32_16x16x32 with the query heads as the 16 rows
// (heads past G are zero rows) and 16 slots as columns: lane l reads the 16
// contiguous bytes of key row (slot) l % 16 at head-dim offset 8 (l / 16)
// of each 32-wide step, so a wave instruction covers whole 256-byte key
// rows. The chunk's softmax is folded into a running maximum, sum and
// accumulator (exponentials as exp2 of log2(e)-scaled scores). p goes
// through a wave-private LDS tile into the A operand of a second MFMA
// whose B operand reads 16 contiguous bytes of value row d (8 slots): p is
// split exactly into two bf16 (or f16) parts, hi + lo, so p.v keeps ~2^-17
// relative precision, as f32 arithmetic would. Each wave writes its
// partial (max, sum, accumulator row per head) to the workspace.
// attn_combine_kernel: one wavefront per (b, h, g) rescales the partials
// to the common maximum and divides by the total sum.
//
// Slots past min(window, pos + 1) are never read: the loads use buffer
// descriptors whose extent ends there (or an out-of-range offset), which
// return zeros without touching memory, and their scores are -inf.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <string>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kChunk = 64;        // slots per chunk
constexpr int kPStride = 64 + 4;  // floats per row of the LDS p tile
constexpr int kOut = 0x7FFF0000;  // an offset past every extent
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const void* q;     // [B, KV, G, D]
  const void* k;     // [B, KV, Smax, D]
  const void* v;     // [B, KV, D, Smax]
  const int* pos;    // the query position (device scalar)
  void* out;         // [B, KV, G, D]
  float* part;       // [B*KV][parts][G][D]
  float* ml;         // [B*KV][parts][G][2]: running max (log2 units), sum
  int g, smax, window, parts, cpw;
  float scale_log2;  // scale * log2(e)
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t Rsrc(const void* p,
                                                       long long bytes) {
  const int b = static_cast<int>(std::min<long long>(bytes, 0x7FFFFFFFll));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, b,
                                           0x00020000);
}

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16> {
  typedef bf16x8 V;
  static __device__ __forceinline__ f32x4 run(V a, V b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<f16> {
  typedef f16x8 V;
  static __device__ __forceinline__ f32x4 run(V a, V b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Max over the 16 lanes of a row group (lanes 16i .. 16i + 15).
__device__ __forceinline__ float max16(float v) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <typename T, int D>
__global__ __launch_bounds__(64) void attn_split_kernel(AttnArgs a) {
  using M = Mfma<T>;
  using V = typename M::V;
  constexpr int kSteps = D / 32;  // 32-wide head-dim steps of a score MFMA
  constexpr int kDB = D / 16;     // 16-wide head-dim blocks of the output
  __shared__ __attribute__((aligned(16))) float ptile[16 * kPStride];

  const int lane = threadIdx.x;
  const int bh = blockIdx.y;
  const int w = blockIdx.x;
  const int pos = __builtin_amdgcn_readfirstlane(*a.pos);
  const int valid = min(a.window, pos + 1);  // slots [0, valid) attended
  const int s_begin = w * a.cpw * kChunk;
  if (s_begin >= valid) return;  // the combine reads only partials below
  const int s_end = min(valid, s_begin + a.cpw * kChunk);

  const int r16 = lane & 15, q4 = lane >> 4;
  // q as the A operand: row r16 = head (zero past G), K = head-dim
  // 32 t + 8 q4 .. + 7.
  const auto qrs = Rsrc(static_cast<const T*>(a.q) +
                            static_cast<long long>(bh) * a.g * D,
                        static_cast<long long>(a.g) * D * 2);
  V qf[kSteps];
#pragma unroll
  for (int t = 0; t < kSteps; ++t) {
    const int off = r16 < a.g ? (r16 * D + 32 * t + 8 * q4) * 2 : kOut;
    qf[t] = __builtin_bit_cast(
        V, __builtin_amdgcn_raw_buffer_load_b128(qrs, off, 0, 0));
  }
  // keys of this (b, h) up to the last attended slot; values per row d
  const auto krs = Rsrc(static_cast<const T*>(a.k) +
                            static_cast<long long>(bh) * a.smax * D,
                        static_cast<long long>(valid) * D * 2);
  const auto vrs = Rsrc(static_cast<const T*>(a.v) +
                            static_cast<long long>(bh) * D * a.smax,
                        static_cast<long long>(D) * a.smax * 2);

  float m_run[4], l_run[4];
  f32x4 acc[kDB];
#pragma unroll
  for (int r = 0; r < 4; ++r) m_run[r] = -__builtin_inff(), l_run[r] = 0.f;
#pragma unroll
  for (int db = 0; db < kDB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = s_begin; s0 < s_end; s0 += kChunk) {
    // Loads of the whole chunk first: keys (4 blocks of 16 slots x
    // kSteps), values (2 steps of 32 slots x kDB blocks of 16 rows).
    u32x4 kr[4][kSteps], vr[2][kDB];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < kSteps; ++t)
        kr[j][t] = __builtin_amdgcn_raw_buffer_load_b128(
            krs, ((s0 + 16 * j + r16) * D + 32 * t + 8 * q4) * 2, 0, 0);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int sv = s0 + 32 * u + 8 * q4;  // first of the lane's 8 slots
#pragma unroll
      for (int db = 0; db < kDB; ++db) {
        const int off =
            sv < valid ? ((16 * db + r16) * a.smax + sv) * 2 : kOut;
        vr[u][db] = __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0);
      }
    }
    // Scores: lane l holds heads 4 q4 + r for slot s0 + 16 j + r16.
    f32x4 sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < kSteps; ++t)
        sc[j] = M::run(qf[t], __builtin_bit_cast(V, kr[j][t]), sc[j]);
      const bool in = s0 + 16 * j + r16 < valid;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sc[j][r] = in ? sc[j][r] * a.scale_log2 : -__builtin_inff();
    }
    // Running softmax per head (the lane's rows r).
    float alpha[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float cm = max16(fmaxf(fmaxf(sc[0][r], sc[1][r]),
                                   fmaxf(sc[2][r], sc[3][r])));
      const float mn = fmaxf(m_run[r], cm);
      // mn is finite: the chunk's first slot is attended
      alpha[r] = __builtin_amdgcn_exp2f(m_run[r] - mn);
      m_run[r] = mn;
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sc[j][r] = __builtin_amdgcn_exp2f(sc[j][r] - mn);
        ps += sc[j][r];
      }
      l_run[r] = l_run[r] * alpha[r] + ps;
    }
    // p through LDS into the A layout: row = head, K = 8 slots.
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ptile[(4 * q4 + r) * kPStride + 16 * j + r16] = sc[j][r];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[db][r] *= alpha[r];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float* pr = ptile + r16 * kPStride + 32 * u + 8 * q4;
      const f32x4 p0 = *reinterpret_cast<const f32x4*>(pr);
      const f32x4 p1 = *reinterpret_cast<const f32x4*>(pr + 4);
      V hi, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pv = e < 4 ? p0[e] : p1[e - 4];
        const T h = from_f32<T>(pv);
        hi[e] = h;
        lo[e] = from_f32<T>(pv - to_f32(h));
      }
#pragma unroll
      for (int db = 0; db < kDB; ++db) {
        const V vb = __builtin_bit_cast(V, vr[u][db]);
        acc[db] = M::run(hi, vb, acc[db]);
        acc[db] = M::run(lo, vb, acc[db]);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the tile's reads before next writes
  }

  // Partial of this wave: heads 4 q4 + r < G.
  const long long pidx = static_cast<long long>(bh) * a.parts + w;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int g = 4 * q4 + r;
    const float l_tot = sum16(l_run[r]);
    if (g < a.g) {
      float* pp = a.part + (pidx * a.g + g) * D;
#pragma unroll
      for (int db = 0; db < kDB; ++db) pp[16 * db + r16] = acc[db][r];
      if (r16 == 0) {
        a.ml[(pidx * a.g + g) * 2] = m_run[r];
        a.ml[(pidx * a.g + g) * 2 + 1] = l_tot;
      }
    }
  }
}

// One wavefront per (b, h, g): o = sum_c 2^(m_c - M) acc_c /
// sum_c 2^(m_c - M) l_c over the partials that hold attended slots.
template <typename T, int D>
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnArgs a) {
  const int lane = threadIdx.x;
  const int bhg = blockIdx.x;  // (b * KV + h) * G + g
  const int bh = bhg / a.g, g = bhg % a.g;
  const int pos = __builtin_amdgcn_readfirstlane(*a.pos);
  const int valid = min(a.window, pos + 1);
  const int span = a.cpw * kChunk;
  const int np = valid <= 0 ? 0 : min(a.parts, (valid + span - 1) / span);
  const float* ml = a.ml + static_cast<long long>(bh) * a.parts * a.g * 2;
  float mx = -__builtin_inff();
  for (int c = lane; c < np; c += 64) mx = fmaxf(mx, ml[(c * a.g + g) * 2]);
  mx = wave_max(mx);
  constexpr int kPer = D / 64;
  float num[kPer], den = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) num[i] = 0.f;
  const float* part = a.part + static_cast<long long>(bh) * a.parts * a.g * D;
  for (int c = 0; c < np; ++c) {
    const float wgt = __builtin_amdgcn_exp2f(ml[(c * a.g + g) * 2] - mx);
    den += wgt * ml[(c * a.g + g) * 2 + 1];
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      num[i] += wgt * part[(static_cast<long long>(c) * a.g + g) * D +
                           64 * i + lane];
  }
  // no attended slot: 0 / 0 = NaN, as a softmax over only -inf gives
  T* o = static_cast<T*>(a.out) + static_cast<long long>(bhg) * D;
#pragma unroll
  for (int i = 0; i < kPer; ++i) o[64 * i + lane] = from_f32<T>(num[i] / den);
}

template <typename T, int D>
qk_status Launch(const AttnArgs& a, int bkv, hipStream_t st) {
  attn_split_kernel<T, D><<<dim3(a.parts, bkv), 64, 0, st>>>(a);
  if (qk_status s = PostLaunch("attn_split_kernel"); s != QK_OK) return s;
  attn_combine_kernel<T, D><<<dim3(bkv * a.g), 64, 0, st>>>(a);
  return PostLaunch("attn_combine_kernel");
}

}  // namespace

void PlanAttention(AttentionProblem* p) {
  // Runs of cpw chunks per wave: one chunk each while that keeps the waves
  // under ~2048 (8 per CU), longer runs beyond (fewer partials to combine).
  const int64_t chunks = (p->window + kChunk - 1) / kChunk;
  const int64_t bkv = p->b * p->kv;
  int64_t cpw = 1;
  while (bkv * ((chunks + cpw - 1) / cpw) > 2048 && cpw < chunks) cpw *= 2;
  p->cpw = static_cast<int>(cpw);
  p->parts = static_cast<int>((chunks + cpw - 1) / cpw);
  p->workspace_bytes = static_cast<uint64_t>(bkv) * p->parts * p->g *
                       (p->d + 2) * sizeof(float);
}

// The fixed scratch of qk_decode_attention_noalloc: the partials of the
// split window live here instead of in a caller workspace. Each device holds
// its own copy for the life of the process. Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the
// symbol); it uses the device address hipGetSymbolAddress returns.
static __device__ __align__(256) float scratch[kAttentionScratchBytes /
                                               sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

qk_status AttentionScratch(void** ptr) {
  *ptr = nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    return Fail(QK_INTERNAL, "qkern: no current HIP device for the "
                             "attention scratch");
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    // Resolved once per device, with that device current.
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      return Fail(QK_INTERNAL,
                  std::string("qkern: hipGetSymbolAddress(scratch) failed: ") +
                      hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return QK_OK;
}

qk_status LaunchAttention(const AttentionProblem& p, void* workspace,
                          hipStream_t stream) {
  AttnArgs a;
  a.q = p.q;
  a.k = p.k;
  a.v = p.v;
  a.pos = static_cast<const int*>(p.pos);
  a.out = p.out;
  const int64_t bkv = p.b * p.kv;
  a.part = static_cast<float*>(workspace);
  a.ml = a.part + bkv * p.parts * p.g * p.d;
  a.g = static_cast<int>(p.g);
  a.smax = static_cast<int>(p.smax);
  a.window = static_cast<int>(p.window);
  a.parts = p.parts;
  a.cpw = p.cpw;
  a.scale_log2 = p.scale * kLog2e;
  if (bkv > 65535) {
    return Fail(QK_UNIMPLEMENTED, "qkern: decode attention over " +
                                      std::to_string(bkv) +
                                      " (batch x KV head) pairs exceeds the "
                                      "grid limit 65535");
  }
  const int b = static_cast<int>(bkv);
  if (p.dtype == QK_BF16)
    return p.d == 64 ? Launch<bf16, 64>(a, b, stream)
                     : Launch<bf16, 128>(a, b, stream);
  return p.d == 64 ? Launch<f16, 64>(a, b, stream)
                   : Launch<f16, 128>(a, b, stream);
}

}  // namespace qk
