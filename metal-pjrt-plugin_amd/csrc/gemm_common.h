// MFMA GEMM building blocks for gfx950 shared by the dense GEMM (gemm.hip)
// and the dequantizing GEMM of the quantized matmul (qgemm.hip): operand
// fragments, LDS tile layouts and loaders, the transposing LDS read, and
// the tiled kernel, whose B operand comes from a pluggable loader.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct GemmArgs {
  const void* a;
  const void* b;
  const void* c;
  void* d;
  const void* bias;
  void* aux;
  int m, n, k;
  int lda, ldb, ldd;
  long long bsa, bsb, bsd;
  float alpha, beta;
  int use_c, has_bias, has_aux, act;
  int out_f32;    // D (and C, bias, aux) are f32; else the input type
  int a_vec, b_vec;  // operand allows 16-byte vector loads
  int out_vec;       // D rows allow 4-element vector stores
  int tiles_m, tiles_n;
  // Quantized B operand (qgemm.hip): b holds the codes; per-group scale
  // and offset (dtypes qk_dtype), group size and bytes of codes per row.
  const void* qscale;
  const void* qbias;
  int qsdt, qbdt, qhas_bias, qgroup, qrow_bytes;
};

constexpr int kGroupM = 8;

// Fragment of 8 consecutive K elements of one row (A) or column (B).
template <typename T>
struct Frag;
template <>
struct Frag<bf16> {
  typedef bf16x8 type;
};
template <>
struct Frag<f16> {
  typedef f16x8 type;
};
template <>
struct Frag<float> {
  struct type {
    f32x4 lo, hi;
  };
};

__device__ __forceinline__ void mma(f32x16& acc, const bf16x8& a,
                                    const bf16x8& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x16& acc, const f16x8& a,
                                    const f16x8& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
}
// f32: lane half h supplies K elements h*8 + j to the j-th 32x32x2 MFMA,
// so the eight MFMAs together cover the 16 K elements of the step.
__device__ __forceinline__ void mma(f32x16& acc, const Frag<float>::type& a,
                                    const Frag<float>::type& b) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.lo[j], b.lo[j], acc, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.hi[j], b.hi[j], acc, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ typename Frag<T>::type lds_frag(const T* p) {
  return *reinterpret_cast<const typename Frag<T>::type*>(p);
}

// Raw 16-byte vector of T.
template <typename T>
struct Vec16 {
  static constexpr int kN = 16 / sizeof(T);
  union {
    u32x4 u;
    T e[kN];
  };
};

// Loads one operand tile of R rows (M or N) x BK into registers and stores
// it K-contiguous into LDS. `kmajor` false: the source is [rows][K]
// (K contiguous); true: the source is [K][rows] (rows contiguous) and the
template <typename T>
__device__ __forceinline__ float ld_out(const void* p, long long i, bool f32) {
  return f32 ? static_cast<const float*>(p)[i]
             : to_f32(static_cast<const T*>(p)[i]);
}
template <typename T>
__device__ __forceinline__ void st_out(void* p, long long i, bool f32,
                                       float v) {
  if (f32)
    static_cast<float*>(p)[i] = v;
  else
    static_cast<T*>(p)[i] = from_f32<T>(v);
}

// ---------------------------------------------------------------------------
// f16/bf16 kernel: every operand tile is copied into LDS in its source
// orientation with 16-byte stores (no transposition on the way in), and
// MFMA fragments are read with ds_read_b128 when the operand is
// K-contiguous, or with the gfx950 transposing read ds_read_b64_tr_b16
// when it is M/N-contiguous (B in the NN layout, A when transposed).
//
// ds_read_b64_tr_b16, per group of 16 lanes: lane s supplies the address of
// 4 consecutive 16-bit elements; lane L receives element L%4 of the chunks
// of lanes L/4, 4 + L/4, 8 + L/4, 12 + L/4. With lane s pointing at
// X[k0 + s/4][r0 + 4*(s%4)] of a K-major tile X[k][r], lane L receives
// X[k0..k0+3][r0 + L]: four consecutive K elements of row r0 + L, the
// MFMA operand layout. Two such reads give the 8 K elements of a
// v_mfma_f32_32x32x16 operand.

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <typename T>
__device__ __forceinline__ u32x2 lds_read_tr(const T* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4*)(const_cast<T*>(p)));
  return __builtin_bit_cast(u32x2, v);
}

// LDS tile of R rows (M or N) x BK: K-contiguous [R][BK + 8] when KCONT,
// else K-major [BK][R + 16] (the source orientation in both cases).
template <typename T, int R, int BK, bool KCONT>
struct TileLayout {
  static constexpr int kLd = KCONT ? BK + 8 : R + 16;
  static constexpr int kElems = KCONT ? R * kLd : BK * kLd;
};

// Global -> registers -> LDS copy of one tile in its source orientation.
template <typename T, int R, int BK, int NT, bool KCONT>
struct DirectLoader {
  static constexpr int VPR = (KCONT ? BK : R) / 8;  // vectors per source row
  static constexpr int NV = R * BK / 8 / NT;        // vectors per thread
  static_assert(NV * NT * 8 == R * BK, "tile does not split evenly");
  u32x4 v[NV];

  // src: operand batch base; the tile covers rows [r0, r0+R) and K
  // [k0, k0+BK); ld is the source row stride (elements).
  __device__ __forceinline__ void load(const T* __restrict__ src, int ld,
                                       int r0, int k0, int rows_total,
                                       int k_total, bool vec_ok, int tid) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int id = tid + i * NT;
      const int sr = id / VPR, sc = (id % VPR) * 8;  // source row / column
      // K-contiguous: source row = tile row, column = k; else row = k.
      const int gr = KCONT ? r0 + sr : k0 + sr;
      const int gc = KCONT ? k0 + sc : r0 + sc;
      const int rlim = KCONT ? rows_total : k_total;
      const int clim = KCONT ? k_total : rows_total;
      const T* p = src + static_cast<long long>(gr) * ld + gc;
      if (vec_ok && gr < rlim && gc + 8 <= clim) {
        v[i] = *reinterpret_cast<const u32x4*>(p);
      } else {
        union {
          u32x4 u;
          T e[8];
        } t;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          t.e[e] = (gr < rlim && gc + e < clim) ? p[e] : T(0);
        v[i] = t.u;
      }
    }
  }

  __device__ __forceinline__ void store(T* lds, int tid) const {
    constexpr int LD = TileLayout<T, R, BK, KCONT>::kLd;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int id = tid + i * NT;
      const int sr = id / VPR, sc = (id % VPR) * 8;
      *reinterpret_cast<u32x4*>(lds + sr * LD + sc) = v[i];
    }
  }
};

// MFMA operand fragment for rows [rb, rb + 32) and K [kb, kb + 16) of an
// LDS tile (see TileLayout); lane l gets row rb + l%32, K kb + 8*(l/32)..+8.
template <typename T, int R, int BK, bool KCONT>
__device__ __forceinline__ typename Frag<T>::type load_frag(const T* lds,
                                                            int rb, int kb,
                                                            int lane) {
  constexpr int LD = TileLayout<T, R, BK, KCONT>::kLd;
  if constexpr (KCONT) {
    return *reinterpret_cast<const typename Frag<T>::type*>(
        lds + (rb + (lane & 31)) * LD + kb + (lane >> 5) * 8);
  } else {
    const int g = lane >> 4, s = lane & 15;
    const T* p = lds + (kb + 8 * (g >> 1) + (s >> 2)) * LD + rb +
                 16 * (g & 1) + 4 * (s & 3);
    const u32x2 lo = lds_read_tr(p);
    const u32x2 hi = lds_read_tr(p + 4 * LD);
    const u32x4 q = {lo[0], lo[1], hi[0], hi[1]};
    return __builtin_bit_cast(typename Frag<T>::type, q);
  }
}


// B operand loaded as stored (dense GEMM): K-contiguous when KCONT.
template <typename T, int BN, int BK, int NT, bool KCONT>
struct DenseB {
  static constexpr bool kKCont = KCONT;
  DirectLoader<T, BN, BK, NT, KCONT> ld;
  const T* src;
  int ldb, n0, n, k, tid;
  bool vec;
  __device__ __forceinline__ DenseB(const GemmArgs& g, long long batch,
                                    int n0_, int tid_)
      : src(static_cast<const T*>(g.b) + batch * g.bsb),
        ldb(g.ldb),
        n0(n0_),
        n(g.n),
        k(g.k),
        tid(tid_),
        vec(g.b_vec != 0) {}
  __device__ __forceinline__ void load(int k0) {
    ld.load(src, ldb, n0, k0, n, k, vec, tid);
  }
  __device__ __forceinline__ void store(T* lds) const { ld.store(lds, tid); }
};

template <typename T, int BM, int BN, int BK, int WM, int WN, bool TA, class BSrc>
__global__ __launch_bounds__(WM* WN * 64) void gemm_tile_kernel(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr bool AK = !TA, BKC = BSrc::kKCont;  // K-contiguous operands
  using LA = TileLayout<T, BM, BK, AK>;
  using LB = TileLayout<T, BN, BK, BKC>;
  static_assert(FM >= 1 && FN >= 1 && BK % 16 == 0, "bad tile");

  // One LDS block: two stages of the A and B tiles during the K loop, the
  // f32 output tile (in row slabs) in the epilogue.
  constexpr int kTileBytes = 2 * (LA::kElems + LB::kElems) * sizeof(T);
  constexpr int kLdo = BN + 4;  // f32 staging row stride
  constexpr int kSlab = WTM;    // output rows staged at a time
  constexpr int kOutBytes = kSlab * kLdo * 4;
  __shared__ __attribute__((aligned(16)))
  unsigned char lds_raw[kTileBytes > kOutBytes ? kTileBytes : kOutBytes];
  T* const lds_base = reinterpret_cast<T*>(lds_raw);
  auto lds_a = [&](int stage) { return lds_base + stage * LA::kElems; };
  auto lds_b = [&](int stage) {
    return lds_base + 2 * LA::kElems + stage * LB::kElems;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int nwg = g.tiles_m * g.tiles_n;
  int bid = blockIdx.x;
  if ((nwg & 7) == 0) bid = (bid & 7) * (nwg >> 3) + (bid >> 3);
  const int group_span = kGroupM * g.tiles_n;
  const int first_m = (bid / group_span) * kGroupM;
  const int gsz = min(g.tiles_m - first_m, kGroupM);
  const int tm = first_m + (bid % group_span) % gsz;
  const int tn = (bid % group_span) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;
  const long long batch = blockIdx.y;

  const T* A = static_cast<const T*>(g.a) + batch * g.bsa;

  DirectLoader<T, BM, BK, NT, AK> la;
  BSrc lb(g, batch, n0, tid);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int ktiles = (g.k + BK - 1) / BK;
  if (ktiles > 0) {
    la.load(A, g.lda, m0, 0, g.m, g.k, g.a_vec, tid);
    lb.load(0);
    la.store(lds_a(0), tid);
    lb.store(lds_b(0));
    __syncthreads();
  }
  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      la.load(A, g.lda, m0, (kt + 1) * BK, g.m, g.k, g.a_vec, tid);
      lb.load((kt + 1) * BK);
    }
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      typename Frag<T>::type fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[i] = load_frag<T, BM, BK, AK>(lds_a(cur), wm * WTM + i * 32,
                                         ks * 16, lane);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[j] = load_frag<T, BN, BK, BKC>(lds_b(cur), wn * WTN + j * 32,
                                          ks * 16, lane);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], fa[i], fb[j]);
    }
    if (more) {
      la.store(lds_a(cur ^ 1), tid);
      lb.store(lds_b(cur ^ 1));
    }
    __syncthreads();
  }

  // Epilogue through LDS, one slab of WTM output rows (one row of waves)
  // at a time: the waves of that row write their f32 accumulators, then
  // all threads apply alpha, beta*C, bias, aux and the activation to four
  // consecutive columns each and store them with one vector store.
  const bool of32 = g.out_f32 != 0;
  const long long dbase = batch * g.bsd;
  float* stage = reinterpret_cast<float*>(lds_raw);
  const bool vec_out = g.out_vec != 0;
#pragma unroll 1
  for (int slab = 0; slab < WM; ++slab) {
    if (wm == slab) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int col = wn * WTN + j * 32 + (lane & 31);
            stage[row * kLdo + col] = acc[i][j][r];
          }
    }
    __syncthreads();
#pragma unroll 1
    for (int q = tid; q < kSlab * BN / 4; q += NT) {
      const int lr = q / (BN / 4), lc = (q % (BN / 4)) * 4;
      const int row = m0 + slab * WTM + lr, col = n0 + lc;
      if (row >= g.m || col >= g.n) continue;
      const float4 a4 = *reinterpret_cast<const float4*>(stage + lr * kLdo + lc);
      float v[4] = {a4.x, a4.y, a4.z, a4.w};
      const long long idx = dbase + static_cast<long long>(row) * g.ldd + col;
      const int cnt = min(4, g.n - col);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (e >= cnt) break;
        float x = g.alpha * v[e];
        if (g.use_c) x += g.beta * ld_out<T>(g.c, idx + e, of32);
        if (g.has_bias) x += ld_out<T>(g.bias, col + e, of32);
        if (g.has_aux) st_out<T>(g.aux, idx + e, of32, x);
        v[e] = act_f32(g.act, x);
      }
      if (vec_out && cnt == 4) {
        if (of32) {
          *reinterpret_cast<float4*>(static_cast<float*>(g.d) + idx) =
              make_float4(v[0], v[1], v[2], v[3]);
        } else {
          union {
            u32x2 u;
            T e[4];
          } o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o.e[e] = from_f32<T>(v[e]);
          *reinterpret_cast<u32x2*>(static_cast<T*>(g.d) + idx) = o.u;
        }
      } else {
        for (int e = 0; e < cnt; ++e) st_out<T>(g.d, idx + e, of32, v[e]);
      }
    }
    __syncthreads();
  }
}


}  // namespace
}  // namespace qk
