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
// attn_split_kernel: one workgroup of two wavefronts per (b, h, run of
// 64-slot chunks); the runs cut the attended window (known only on the
// device) into a fixed number of parts, and each wave takes one 32-slot
// half of every chunk, with a running softmax of its own that the two
// merge at the end. Keys and values of a chunk are fetched by LDS DMA as
// whole contiguous 1 KB pieces into one of two LDS stages (the next chunk
// is in flight while one is computed) and read back, swizzled against
// bank conflicts, in the MFMA operand layouts. Scores come from
// v_mfma_f32_16x16x32 with the query heads as the 16 rows (heads past G
// are zero rows) and 16 slots as columns. The chunk's softmax is folded
// into a running maximum, sum and accumulator (exponentials as exp2 of
// log2(e)-scaled scores). p goes through a wave-private LDS tile into the
// A operand of a second MFMA whose B operand is 8 slots of a value row:
// p is split exactly into two bf16 (or f16) parts, hi + lo, so p.v keeps
// ~2^-17 relative precision, as f32 arithmetic would. Each workgroup writes
// its partial (max, sum, accumulator row per head) to the workspace.
// attn_combine_kernel: one workgroup per (b, h, g) and 16 head-dim
// columns rescales the partials to the common maximum and divides by the
// total sum.
//
// Slots past min(window, pos + 1) take no part: keys past it read zeros
// through the descriptor's extent and score -inf; values are fetched in
// 8-slot units, units wholly past it are not read, and the slots past it
// in the last unit are zeroed in LDS before use.

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
constexpr int kPStride = 32 + 4;  // floats per row of a wave's LDS p tile
constexpr int kSplitWaves = 2;    // waves per split workgroup
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
  int g, smax, window, parts;
  float scale_log2;  // scale * log2(e)
};

// The attended window is split into `parts` runs of whole chunks per
// (b, h); both kernels derive the run length from the position read on the
// device, so a short attended prefix of a long window still spreads over
// all parts.
__device__ __forceinline__ int ChunksPerPart(int valid, int parts) {
  const int cv = (valid + kChunk - 1) / kChunk;
  return (cv + parts - 1) / parts;
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

// LDS of one split wave: two stages of a chunk's keys and values, the q
// tile and the p tile. Keys land as their 64 rows of D/8 16-byte units,
// unit c of slot s at position c ^ Swz(s); values as D rows of 8 units
// (64 slots), unit u of row d at u ^ ((d >> 1) & 7). Both swizzles make
// the MFMA operand reads (16 lanes: 16 slots, or 16 rows, at one unit)
// hit 16 distinct 16-byte bank groups.
template <int D>
struct AttnLds {
  static constexpr int kUnits = D / 8;
  static constexpr int kK = kChunk * D * 2;
  static constexpr int kV = D * kChunk * 2;
  static constexpr int kStage = kK + kV;
  static constexpr int kDmaK = kK / 1024;  // 1 KB DMA instructions
  static constexpr int kDmaV = kV / 1024;
  static constexpr int kDma = kDmaK + kDmaV;
  static constexpr int kQ = 16 * D * 2;
  static constexpr int kDmaQ = kQ / 1024;
  static constexpr int kQOff = 2 * kStage;
  static constexpr int kPOff = kQOff + kQ;
  static constexpr int kPTile = 16 * kPStride * 4;  // one per wave
  static constexpr int kBytes = kPOff + kSplitWaves * kPTile;
  static_assert(kDmaK % kSplitWaves == 0 && kDmaV % kSplitWaves == 0 &&
                    kDmaQ % kSplitWaves == 0,
                "the waves share every DMA group evenly");
  static_assert(64 * (8 + 4 * (D / 16)) * 4 <= kStage,
                "the second wave's running state fits in a stage");
  static __device__ __forceinline__ int Swz(int s) {
    return D == 128 ? (s & 15) : ((s >> 1) & 7);
  }
};

template <typename T, int D>
__global__ __launch_bounds__(64 * kSplitWaves) void attn_split_kernel(
    AttnArgs a) {
  using M = Mfma<T>;
  using V = typename M::V;
  using L = AttnLds<D>;
  constexpr int kSteps = D / 32;  // 32-wide head-dim steps of a score MFMA
  constexpr int kDB = D / 16;     // 16-wide head-dim blocks of the output
  constexpr int kDmaW = L::kDma / kSplitWaves;  // DMAs per wave per chunk
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* ptile = reinterpret_cast<float*>(smem + L::kPOff + wv * L::kPTile);
  const int bh = blockIdx.y;
  const int w = blockIdx.x;
  const int pos = __builtin_amdgcn_readfirstlane(*a.pos);
  const int valid = min(a.window, pos + 1);  // slots [0, valid) attended
  const int cpw = ChunksPerPart(valid, a.parts);
  const int s_begin = w * cpw * kChunk;
  if (s_begin >= valid) return;  // the combine reads only partials below
  const int s_end = min(valid, s_begin + cpw * kChunk);
  const int nchunks = (s_end - s_begin + kChunk - 1) / kChunk;

  const T* qb = static_cast<const T*>(a.q) + static_cast<long long>(bh) * a.g * D;
  const T* kb = static_cast<const T*>(a.k) + static_cast<long long>(bh) * a.smax * D;
  const T* vb = static_cast<const T*>(a.v) + static_cast<long long>(bh) * D * a.smax;
  // Keys up to the last attended slot (rows past it read zeros); values
  // of this (b, h) (8-slot units wholly past it are not read).
  DmaRsrc qd, kd, vd;
  qd.make(qb, static_cast<long long>(a.g) * D * 2);
  kd.make(kb, static_cast<long long>(valid) * D * 2);
  vd.make(vb, static_cast<long long>(D) * a.smax * 2);

  // Per-lane DMA offsets within a chunk: key unit p = 64 i + lane is slot
  // p / kUnits, unit (p % kUnits) ^ Swz(slot); value lane covers row
  // 8 i + lane / 8, unit (lane % 8) ^ ((row >> 1) & 7). Wave wv issues
  // pieces i = wv * n / kSplitWaves .. of each group of n. The cache is
  // read once per call: nontemporal.
  auto issue = [&](int chunk) {
    unsigned char* st = smem + (chunk & 1) * L::kStage;
    const int s0 = s_begin + chunk * kChunk;
#pragma unroll
    for (int ii = 0; ii < L::kDmaK / kSplitWaves; ++ii) {
      const int i = wv * (L::kDmaK / kSplitWaves) + ii;
      const int p = 64 * i + lane;
      const int sl = p / L::kUnits;
      const int u = (p % L::kUnits) ^ L::Swz(sl);
      kd.dma_nt(st + 1024 * i, ((s0 + sl) * L::kUnits + u) * 16, 0);
    }
#pragma unroll
    for (int ii = 0; ii < L::kDmaV / kSplitWaves; ++ii) {
      const int i = wv * (L::kDmaV / kSplitWaves) + ii;
      const int d = 8 * i + lane / 8;
      const int u = (lane % 8) ^ ((d >> 1) & 7);
      const int sv = s0 + 8 * u;
      vd.dma_nt(st + L::kK + 1024 * i,
                sv < valid ? (d * a.smax + sv) * 2 : kOut, 0);
    }
  };

  // q first (heads past G read zeros), then the first two chunks.
#pragma unroll
  for (int ii = 0; ii < L::kDmaQ / kSplitWaves; ++ii) {
    const int i = wv * (L::kDmaQ / kSplitWaves) + ii;
    qd.dma(smem + L::kQOff + 1024 * i, (1024 * i + 16 * lane), 0);
  }
  issue(0);
  if (nchunks > 1) issue(1);

  // Wave wv takes slots 32 wv .. 32 wv + 31 of every chunk: score blocks
  // j = 2 wv, 2 wv + 1 and p.v step u = wv; each wave keeps a running
  // softmax of its own, merged with the other's at the end.
  const int r16 = lane & 15, q4 = lane >> 4;
  float m_run[4], l_run[4];
  f32x4 acc[kDB];
#pragma unroll
  for (int r = 0; r < 4; ++r) m_run[r] = -__builtin_inff(), l_run[r] = 0.f;
#pragma unroll
  for (int db = 0; db < kDB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  V qf[kSteps];

  for (int c = 0; c < nchunks; ++c) {
    // Chunk c has landed: own DMA by vmcnt, the other wave's by the barrier.
    if (c + 1 < nchunks)
      __builtin_amdgcn_s_waitcnt(VmcntImm(kDmaW));
    else
      __builtin_amdgcn_s_waitcnt(VmcntImm(0));
    __syncthreads();
    const unsigned char* st = smem + (c & 1) * L::kStage;
    const int s0 = s_begin + c * kChunk;
    if (c == 0) {
      // q as the A operand: row r16 = head (zero past G), K = head-dim
      // 32 t + 8 q4 .. + 7.
#pragma unroll
      for (int t = 0; t < kSteps; ++t) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(
            smem + L::kQOff + (r16 * D + 32 * t + 8 * q4) * 2);
        qf[t] = __builtin_bit_cast(V, r16 < a.g ? v : u32x4{0, 0, 0, 0});
      }
    }
    // The values of slots [valid, next multiple of 8) were fetched with
    // their unit: zero them (a value there may be anything, even NaN, and
    // p = 0 would not cancel it). The wave whose half holds the unit does
    // it; only that wave reads it.
    if (valid - s0 < kChunk && (valid & 7) != 0 &&
        ((valid - s0) >> 5) == wv) {
      const int su = (valid - s0) >> 3;  // unit holding slot valid
      unsigned char* vs = const_cast<unsigned char*>(st) + L::kK;
#pragma unroll
      for (int rr = 0; rr < D / 64; ++rr) {
        const int d = 64 * rr + lane;
        T* row = reinterpret_cast<T*>(vs + d * 128 +
                                      (su ^ ((d >> 1) & 7)) * 16);
        for (int e = valid & 7; e < 8; ++e) row[e] = from_f32<T>(0.f);
      }
    }
    // Scores: lane l holds heads 4 q4 + r for slot s0 + 32 wv + 16 j + r16.
    f32x4 sc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      sc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int sl = 32 * wv + 16 * j + r16;
#pragma unroll
      for (int t = 0; t < kSteps; ++t) {
        const u32x4 kv = *reinterpret_cast<const u32x4*>(
            st + (sl * L::kUnits + ((4 * t + q4) ^ L::Swz(sl))) * 16);
        sc[j] = M::run(qf[t], __builtin_bit_cast(V, kv), sc[j]);
      }
      const bool in = s0 + sl < valid;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sc[j][r] = in ? sc[j][r] * a.scale_log2 : -__builtin_inff();
    }
    // Running softmax per head (the lane's rows r). The second wave's half
    // of the last chunk may hold no attended slot: with nothing attended
    // so far the maximum stays -inf and the shift is taken as 0 (alpha
    // and p are then 0, not NaN).
    float alpha[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float cm = max16(fmaxf(sc[0][r], sc[1][r]));
      const float mn = fmaxf(m_run[r], cm);
      const float sh = mn == -__builtin_inff() ? 0.f : mn;
      alpha[r] = __builtin_amdgcn_exp2f(m_run[r] - sh);
      m_run[r] = mn;
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        sc[j][r] = __builtin_amdgcn_exp2f(sc[j][r] - sh);
        ps += sc[j][r];
      }
      l_run[r] = l_run[r] * alpha[r] + ps;
    }
    // p through the wave's LDS tile into the A layout: row = head, K = 8
    // slots.
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ptile[(4 * q4 + r) * kPStride + 16 * j + r16] = sc[j][r];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[db][r] *= alpha[r];
    {
      const float* pr = ptile + r16 * kPStride + 8 * q4;
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
        const int d = 16 * db + r16;
        const u32x4 vv = *reinterpret_cast<const u32x4*>(
            st + L::kK + d * 128 + ((4 * wv + q4) ^ ((d >> 1) & 7)) * 16);
        const V vbf = __builtin_bit_cast(V, vv);
        acc[db] = M::run(hi, vbf, acc[db]);
        acc[db] = M::run(lo, vbf, acc[db]);
      }
    }
    // Both waves' LDS reads of this stage are done before its refill.
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __syncthreads();
    if (c + 2 < nchunks) issue(c + 2);
  }

  // Merge: the second wave leaves its running state in stage 0 (every DMA
  // has landed and every read of the stages is done at the last barrier);
  // the first rescales both to the common maximum (finite: the part's
  // first slot is attended and lies in the first wave's half).
  float* xs = reinterpret_cast<float*>(smem) + lane;
  if (wv == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      xs[64 * r] = m_run[r];
      xs[64 * (4 + r)] = l_run[r];
#pragma unroll
      for (int db = 0; db < kDB; ++db) xs[64 * (8 + 4 * db + r)] = acc[db][r];
    }
  }
  __syncthreads();
  if (wv == 1) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float m1 = xs[64 * r];
    const float mn = fmaxf(m_run[r], m1);
    const float f0 = __builtin_amdgcn_exp2f(m_run[r] - mn);
    const float f1 = __builtin_amdgcn_exp2f(m1 - mn);
    m_run[r] = mn;
    l_run[r] = l_run[r] * f0 + xs[64 * (4 + r)] * f1;
#pragma unroll
    for (int db = 0; db < kDB; ++db)
      acc[db][r] = acc[db][r] * f0 + xs[64 * (8 + 4 * db + r)] * f1;
  }

  // Partial of this workgroup: heads 4 q4 + r < G.
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

// One workgroup of 256 threads per (b, h, g) and 16 head-dim columns:
// o = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c over the partials
// that hold attended slots. Thread t takes column t % 16 of partials
// c = t / 16, t / 16 + 16, ... (16 partial rows in flight per workgroup,
// 64 contiguous bytes each); the 16 sums per column meet in LDS.
constexpr int kCombineThreads = 256;
constexpr int kCombineCols = 16;
constexpr int kCombineGroups = kCombineThreads / kCombineCols;

template <typename T, int D>
__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(
    AttnArgs a) {
  __shared__ float red[kCombineGroups][kCombineCols + 1];
  __shared__ float dred[kCombineGroups];
  __shared__ float wmax[kCombineThreads / 64];
  const int t = threadIdx.x;
  const int bhg = blockIdx.x;  // (b * KV + h) * G + g
  const int bh = bhg / a.g, g = bhg % a.g;
  const int col = blockIdx.y * kCombineCols + (t % kCombineCols);
  const int cg = t / kCombineCols;
  const float* ml = a.ml + static_cast<long long>(bh) * a.parts * a.g * 2;
  const float* part = a.part + static_cast<long long>(bh) * a.parts * a.g * D;
  // The first kFirst partials of this thread are requested before the
  // position arrives (those past the attended ones are loaded, never
  // used), so the kernel waits for one memory round trip, not three.
  constexpr int kFirst = 8;
  float pm[kFirst], pl[kFirst], pp[kFirst];
#pragma unroll
  for (int i = 0; i < kFirst; ++i) {
    const int c = cg + kCombineGroups * i;
    const bool ok = c < a.parts;
    const long long e = static_cast<long long>(ok ? c : 0) * a.g + g;
    pm[i] = ml[e * 2];
    pl[i] = ml[e * 2 + 1];
    pp[i] = part[e * D + col];
  }
  const int pos = __builtin_amdgcn_readfirstlane(*a.pos);
  const int valid = min(a.window, pos + 1);
  const int span = ChunksPerPart(valid, a.parts) * kChunk;
  const int np = valid <= 0 ? 0 : min(a.parts, (valid + span - 1) / span);
  float mx = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < kFirst; ++i)
    if (cg + kCombineGroups * i < np) mx = fmaxf(mx, pm[i]);
  for (int c = cg + kCombineGroups * kFirst; c < np; c += kCombineGroups)
    mx = fmaxf(mx, ml[(c * a.g + g) * 2]);
  mx = wave_max(mx);
  if ((t & 63) == 0) wmax[t >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  float num = 0.f, den = 0.f;
#pragma unroll
  for (int i = 0; i < kFirst; ++i) {
    if (cg + kCombineGroups * i < np) {
      const float wgt = __builtin_amdgcn_exp2f(pm[i] - mx);
      den += wgt * pl[i];
      num += wgt * pp[i];
    }
  }
#pragma unroll 4
  for (int c = cg + kCombineGroups * kFirst; c < np; c += kCombineGroups) {
    const float wgt = __builtin_amdgcn_exp2f(ml[(c * a.g + g) * 2] - mx);
    den += wgt * ml[(c * a.g + g) * 2 + 1];
    num += wgt * part[(static_cast<long long>(c) * a.g + g) * D + col];
  }
  red[cg][t % kCombineCols] = num;
  if (t % kCombineCols == 0) dred[cg] = den;
  __syncthreads();
  if (cg == 0) {
    float n = 0.f, dsum = 0.f;
#pragma unroll
    for (int i = 0; i < kCombineGroups; ++i) {
      n += red[i][t];
      dsum += dred[i];
    }
    // no attended slot: 0 / 0 = NaN, as a softmax over only -inf gives
    T* o = static_cast<T*>(a.out) + static_cast<long long>(bhg) * D;
    o[col] = from_f32<T>(n / dsum);
  }
}

template <typename T, int D>
qk_status Launch(const AttnArgs& a, int bkv, hipStream_t st) {
  attn_split_kernel<T, D><<<dim3(a.parts, bkv), 64 * kSplitWaves,
                            AttnLds<D>::kBytes, st>>>(a);
  if (qk_status s = PostLaunch("attn_split_kernel"); s != QK_OK) return s;
  attn_combine_kernel<T, D>
      <<<dim3(bkv * a.g, D / kCombineCols), kCombineThreads, 0, st>>>(a);
  return PostLaunch("attn_combine_kernel");
}

}  // namespace

void PlanAttention(AttentionProblem* p) {
  // About 512 split waves in all (two per CU at head dim 128: each holds
  // two 32 KB stages of keys and values in LDS): the attended window of
  // each (b, h) is cut into `parts` runs of whole chunks.
  const int64_t chunks = (p->window + kChunk - 1) / kChunk;
  const int64_t bkv = p->b * p->kv;
  p->parts = static_cast<int>(
      std::max<int64_t>(1, std::min<int64_t>(chunks, (512 + bkv - 1) / bkv)));
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
