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
  // Split K (qgemm_dma.h): K ranges per tile (1: none), the f32 partial
  // tiles and the per-tile arrival counters (zero between launches).
  int ksplit;
  // M tiles per tile group of the workgroup order (qgemm_dma.h; 0: kGroupM)
  int group_m;
  float* ws;
  uint32_t* wsflag;
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
// else K-major [BK][R + 32] (the source orientation in both cases).
template <typename T, int R, int BK, bool KCONT>
struct TileLayout {
  // K-major rows padded by 32 elements: the 16-lane groups of a
  // transposing read then cover all 64 banks (a pad of 16 left 2-way
  // conflicts).
  static constexpr int kLd = KCONT ? BK + 8 : R + 32;
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

// Four consecutive output-type elements as f32 (vector load when `vec`).
template <typename T>
__device__ __forceinline__ void ld_out4(const void* p, long long i, bool f32,
                                        bool vec, int cnt, float (&v)[4]) {
  if (vec && cnt == 4) {
    if (f32) {
      const float4 q = *reinterpret_cast<const float4*>(
          static_cast<const float*>(p) + i);
      v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
    } else {
      union {
        u32x2 u;
        T e[4];
      } q;
      q.u = *reinterpret_cast<const u32x2*>(static_cast<const T*>(p) + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = to_f32(q.e[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = e < cnt ? ld_out<T>(p, i + e, f32) : 0.f;
  }
}
template <typename T>
__device__ __forceinline__ void st_out4(void* p, long long i, bool f32,
                                        bool vec, int cnt, const float (&v)[4]) {
  if (vec && cnt == 4) {
    if (f32) {
      *reinterpret_cast<float4*>(static_cast<float*>(p) + i) =
          make_float4(v[0], v[1], v[2], v[3]);
    } else {
      union {
        u32x2 u;
        T e[4];
      } o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o.e[e] = from_f32<T>(v[e]);
      *reinterpret_cast<u32x2*>(static_cast<T*>(p) + i) = o.u;
    }
  } else {
    for (int e = 0; e < cnt; ++e) st_out<T>(p, i + e, f32, v[e]);
  }
}

// Epilogue through LDS, one slab of WTM output rows (one row of waves) at
// a time: the waves of that row write their f32 accumulators, then all
// threads apply alpha, beta*C, bias, aux and the activation to four
// consecutive columns each and store them with one vector store. Each
// thread keeps the same four columns for the whole tile, so it loads its
// bias once. `lds` holds at least WTM x (BN + 4) floats; the caller has
// synchronised after its last use of it.
template <typename T, int BM, int BN, int WM, int WN>
__device__ __forceinline__ void store_tile(
    const GemmArgs& g, const f32x16 (&acc)[BM / WM / 32][BN / WN / 32],
    unsigned char* lds, int m0, int n0, long long batch, int tid) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int kLdo = BN + 4;  // f32 staging row stride
  constexpr int kQuads = BN / 4;  // column quads per row
  static_assert(NT % kQuads == 0, "a thread's columns must not move");
  constexpr int kRowStep = NT / kQuads;  // rows between a thread's quads
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const bool of32 = g.out_f32 != 0;
  const bool vec = g.out_vec != 0;
  const long long dbase = batch * g.bsd;
  float* stage = reinterpret_cast<float*>(lds);
  const int lc = (tid % kQuads) * 4, lr0 = tid / kQuads;
  const int col = n0 + lc;
  const int cnt = max(0, min(4, g.n - col));
  float bias[4] = {0.f, 0.f, 0.f, 0.f};
  if (g.has_bias && cnt > 0) ld_out4<T>(g.bias, col, of32, false, cnt, bias);
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
            const int c = wn * WTN + j * 32 + (lane & 31);
            stage[row * kLdo + c] = acc[i][j][r];
          }
    }
    __syncthreads();
    if (cnt > 0) {
#pragma unroll 4
      for (int lr = lr0; lr < WTM; lr += kRowStep) {
        const int row = m0 + slab * WTM + lr;
        if (row >= g.m) break;
        const float4 a4 =
            *reinterpret_cast<const float4*>(stage + lr * kLdo + lc);
        float v[4] = {a4.x, a4.y, a4.z, a4.w};
        const long long idx = dbase + static_cast<long long>(row) * g.ldd + col;
        float c4[4] = {0.f, 0.f, 0.f, 0.f};
        if (g.use_c) ld_out4<T>(g.c, idx, of32, vec, cnt, c4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = g.alpha * v[e];
          if (g.use_c) v[e] += g.beta * c4[e];
          if (g.has_bias) v[e] += bias[e];
        }
        if (g.has_aux) st_out4<T>(g.aux, idx, of32, vec, cnt, v);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = act_f32(g.act, v[e]);
        st_out4<T>(g.d, idx, of32, vec, cnt, v);
      }
    }
    __syncthreads();
  }
}

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

  // The K loop ends on a barrier, so the tile stages are free.
  store_tile<T, BM, BN, WM, WN>(g, acc, lds_raw, m0, n0, batch, tid);
}


// ---------------------------------------------------------------------------
// Interior-tile f16/bf16 kernel with a register-staged B source (used by
// the quantized matmul, whose B tile is dequantized on its way into LDS;
// dense operands take the LDS-DMA kernel of gemm_dma.h) for problems whose
// N and K are multiples of the tile (BM = 256 or 128, BN = 256 or 128,
// BK = 64; M too unless MC) and whose operands allow 16-byte loads: no
// bounds checks in the K loop.
//
//  - Four waves (2 x 2), each owning a 128 x BN/2 block of D: 16 (or 8)
//    32x32 accumulators, so one wave per SIMD keeps every MFMA pipe fed.
//  - Global loads are raw buffer loads: one descriptor per operand, one
//    VGPR byte offset per thread and an SGPR offset per vector, so the
//    address arithmetic of the loads is scalar.
//  - The next K tile is in registers during the whole current tile; it is
//    written to the other LDS stage in the last 16-wide K step, its DS
//    writes interleaved one per MFMA; the tile after it is requested right
//    after the barrier, so every global load has one tile of MFMA time to
//    land.
//  - MFMA fragments are double-buffered in registers: the DS reads for
//    K step s + 1 are issued between the MFMAs of step s, one per MFMA
//    (sched_group_barrier), so LDS latency hides under the matrix pipe.
//
// Buffer descriptors take a 32-bit extent, so each operand of one batch
// entry must span less than 2^31 bytes (checked by the launcher).
// VCHK: the whole offset goes in the vector offset, which the descriptor's
// extent checks (rows past the extent read zeros).
template <typename T, int R, int BK, int NT, bool KCONT, bool VCHK = false>
struct BufferLoader {
  static constexpr int VPR = (KCONT ? BK : R) / 8;  // vectors per source row
  static constexpr int RPI = NT / VPR;  // source rows between vector slots
  static constexpr int NV = R * BK / 8 / NT;
  static_assert(NT % VPR == 0 && NV * NT * 8 == R * BK, "bad tile split");
  __amdgpu_buffer_rsrc_t rsrc;
  int voff;  // bytes
  int ld;    // elements
  u32x4 v[NV];
  __device__ __forceinline__ void init(const T* src, long long bytes, int ld_,
                                       int tid) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(src), (short)0,
                                             static_cast<int>(bytes),
                                             0x00020000);
    ld = ld_;
    voff = ((tid / VPR) * ld + (tid % VPR) * 8) * static_cast<int>(sizeof(T));
  }
  // Tile origin: rows r0 (M or N), k0.
  __device__ __forceinline__ void load(int r0, int k0) {
    const int base = KCONT ? r0 * ld + k0 : k0 * ld + r0;  // elements
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int soff = (base + i * RPI * ld) * static_cast<int>(sizeof(T));
      if constexpr (VCHK)
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff + soff, 0, 0);
      else
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, soff, 0);
    }
  }
  __device__ __forceinline__ void store(T* lds, int tid) const {
    constexpr int LD = TileLayout<T, R, BK, KCONT>::kLd;
    T* p = lds + (tid / VPR) * LD + (tid % VPR) * 8;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      *reinterpret_cast<u32x4*>(p + i * RPI * LD) = v[i];
  }
};


// Epilogue straight from the accumulators, for tiles wholly inside D (no
// bounds checks): the lane holding element (row, col) of a 32x32 block
// applies alpha, beta*C, bias, aux and the activation and stores it; the
// 32 lanes of a half-wave write 32 consecutive columns of one row. The
// output type and activation are template arguments, chosen once by
// store_direct, so the per-element code has no branches on them.
// Arithmetic order as store_tile: alpha*acc, + beta*C, + bias.
// MC: rows at or past g.m are neither read (C) nor written (the last M
// tile of a kernel whose M need not be a multiple of BM).
template <typename O, int ACT, int BM, int BN, int WM, int WN, bool MC>
__device__ __forceinline__ void store_direct_t(
    const GemmArgs& g, const f32x16 (&acc)[BM / WM / 32][BN / WN / 32],
    int m0, int n0, long long batch, int lane, int wm, int wn) {
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  const long long dbase = batch * g.bsd;
  const int colb = n0 + wn * WTN + (lane & 31);
  const int rowb = m0 + wm * WTM + 4 * (lane >> 5);
  float bias[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j)
    bias[j] = g.has_bias ? to_f32(static_cast<const O*>(g.bias)[colb + j * 32])
                         : 0.f;
  const O* C = static_cast<const O*>(g.c);
  O* aux = static_cast<O*>(g.aux);
  O* D = static_cast<O*>(g.d);
  // One 32x32 block at a time (16 values per lane, few registers beyond
  // the accumulators); each optional term is one uniform branch around a
  // loop over the block's 16 values.
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const long long base =
          dbase + static_cast<long long>(rowb + i * 32) * g.ldd + colb +
          j * 32;
      auto at = [&](int r) {
        return base + static_cast<long long>(8 * (r >> 2) + (r & 3)) * g.ldd;
      };
      auto live = [&](int r) {
        return !MC || rowb + i * 32 + 8 * (r >> 2) + (r & 3) < g.m;
      };
      float v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = g.alpha * acc[i][j][r];
      if (g.use_c) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (live(r)) v[r] += g.beta * to_f32(C[at(r)]);
      }
      if (g.has_bias) {
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] += bias[j];
      }
      if (g.has_aux) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (live(r)) aux[at(r)] = from_f32<O>(v[r]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (live(r)) D[at(r)] = from_f32<O>(act_f32(ACT, v[r]));
    }
}

template <typename T, int BM, int BN, int WM, int WN, bool MC = false>
__device__ __forceinline__ void store_direct(
    const GemmArgs& g, const f32x16 (&acc)[BM / WM / 32][BN / WN / 32],
    int m0, int n0, long long batch, int lane, int wm, int wn) {
  auto go = [&](auto out) {
    using O = decltype(out);
    switch (g.act) {
      case 1:
        return store_direct_t<O, 1, BM, BN, WM, WN, MC>(g, acc, m0, n0, batch, lane, wm, wn);
      case 2:
        return store_direct_t<O, 2, BM, BN, WM, WN, MC>(g, acc, m0, n0, batch, lane, wm, wn);
      case 3:
        return store_direct_t<O, 3, BM, BN, WM, WN, MC>(g, acc, m0, n0, batch, lane, wm, wn);
      default:
        return store_direct_t<O, 0, BM, BN, WM, WN, MC>(g, acc, m0, n0, batch, lane, wm, wn);
    }
  };
  if (g.out_f32) go(0.f);
  else go(T{});
}

// Store of a tile whose K range may be split over workgroups (K split
// g.ksplit > 1; batch 0 only): workgroup z of output tile `tile` holds the
// sum over K range z in acc. It writes that f32 partial tile to the
// workspace g.ws (slot tile * ksplit + z; values 4 u .. 4 u + 3 of
// fragment q of thread t at float4 ((slot kPer / 4) + 4 q + u) NT + t, so
// the stores are coalesced) through a buffer descriptor with the sc1 cache
// policy (device-coherent: write-through stores, loads that miss stale
// lines), waits for the stores to complete and then counts itself in on
// the tile's arrival counter g.wsflag[tile] (a device-scope atomic; the
// wait, not a device-scope fence, orders "partial, then arrival": a fence
// would write back and invalidate the whole L2). The last to arrive resets
// the counter to zero for the next launch, sums the partials in the order
// z = 0, 1, ... (its own from registers: first when z <= 1, the first
// addition commuting; for z >= 2 the sum restarts from partial 0 and
// reloads its own in place), so the result does not depend on the arrival
// order, and stores the tile with the epilogue. No workgroup waits for
// another. lds_flag: one word of LDS no wave still reads.
template <typename T, int BM, int BN, int WM, int WN, bool MC, int NT>
__device__ __forceinline__ void split_k_store(
    const GemmArgs& g, f32x16 (&acc)[BM / WM / 32][BN / WN / 32], int tile,
    int z, int m0, int n0, int tid, int lane, int wm, int wn,
    uint32_t* lds_flag) {
  constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
  const int nc = g.ksplit;
  if (nc <= 1) {
    store_direct<T, BM, BN, WM, WN, MC>(g, acc, m0, n0, 0, lane, wm, wn);
    return;
  }
  auto slot = [&](int idx) { return tile * nc + idx; };
  constexpr int kPer = FM * FN * 16;
  const __amdgpu_buffer_rsrc_t wsr = __builtin_amdgcn_make_buffer_rsrc(
      g.ws, (short)0, 0x7FFFFFFF, 0x00020000);
  constexpr int kSc1 = 16;
  auto part_off = [&](int sl, int q, int u) {
    return (((sl * (kPer / 4)) + q * 4 + u) * NT + tid) * 16;
  };
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        f32x4 v = {acc[i][j][4 * u], acc[i][j][4 * u + 1],
                   acc[i][j][4 * u + 2], acc[i][j][4 * u + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, v), wsr, part_off(slot(z), i * FN + j, u),
            0, kSc1);
      }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(
        g.wsflag + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = old + 1 == static_cast<uint32_t>(nc);
    if (last)
      __hip_atomic_store(g.wsflag + tile, 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = last;
  }
  __syncthreads();
  if (*lds_flag == 0) return;
  // kChunk fragments at a time, all loads of a chunk issued together (one
  // memory round trip per partial and chunk); two fragments, 32 values: a
  // larger chunk raised the register count of the kernels into spills.
  constexpr int kFrags = FM * FN;
  constexpr int kChunk = kFrags < 2 ? kFrags : 2;
  const int start = z >= 2 ? 1 : 0;
#pragma unroll
  for (int q0 = 0; q0 < kFrags; q0 += kChunk) {
    auto load_into = [&](int idx, float (&v)[kChunk][16]) {
      const int sl = slot(idx);
#pragma unroll
      for (int q = 0; q < kChunk; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const f32x4 l = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         wsr, part_off(sl, q0 + q, u), 0, kSc1));
#pragma unroll
          for (int e = 0; e < 4; ++e) v[q][4 * u + e] = l[e];
        }
    };
    float v[kChunk][16];
    if (z >= 2) {
      load_into(0, v);
#pragma unroll
      for (int q = 0; q < kChunk; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[(q0 + q) / FN][(q0 + q) % FN][r] = v[q][r];
    }
    for (int idx = start; idx < nc; ++idx) {
      if (idx == z && z <= 1) continue;
      load_into(idx, v);
#pragma unroll
      for (int q = 0; q < kChunk; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[(q0 + q) / FN][(q0 + q) % FN][r] += v[q][r];
    }
  }
  store_direct<T, BM, BN, WM, WN, MC>(g, acc, m0, n0, 0, lane, wm, wn);
}

// MC: M need not be a multiple of BM (A rows past M read zeros through the
// descriptor's extent, output rows past M are not stored); AK only.
// DEPTH = 2 keeps two register sets of operand loads in flight, so a
// tile's loads are issued two K tiles of MFMA work before they are stored
// to LDS (for small tiles whose K step is shorter than the load latency).
template <typename T, int BN, bool TA, class BSrc, int NW = 4, int BM = 256,
          int DEPTH = 1, bool MC = false>
__global__ __launch_bounds__(NW * 64) void gemm_fast_kernel(GemmArgs g) {
  constexpr int BK = 64, NT = NW * 64, WM = NW / 2, WN = 2;
  static_assert(BSrc::NT == NT, "B loader built for this workgroup");
  static_assert(DEPTH == 1 || DEPTH == 2, "one or two register sets");
  static_assert(!MC || !TA, "row bounds through the extent of a K-contiguous A");
  constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 32, FN = WTN / 32;
  constexpr bool AK = !TA, BKC = BSrc::kKCont;  // K-contiguous operands
  using LA = TileLayout<T, BM, BK, AK>;
  using LB = TileLayout<T, BN, BK, BKC>;
  constexpr int kTileBytes = 2 * (LA::kElems + LB::kElems) * sizeof(T);
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[kTileBytes];
  T* const base = reinterpret_cast<T*>(lds_raw);
  auto lds_a = [&](int s) { return base + s * LA::kElems; };
  auto lds_b = [&](int s) { return base + 2 * LA::kElems + s * LB::kElems; };

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

  BufferLoader<T, BM, BK, NT, AK, MC> la0, la1;
  la0.init(static_cast<const T*>(g.a) + batch * g.bsa,
           static_cast<long long>(AK ? g.m : g.k) * g.lda * sizeof(T), g.lda,
           tid);
  if constexpr (DEPTH == 2) la1 = la0;
  BSrc lb0(g, batch, tid), lb1 = lb0;

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int ktiles = g.k / BK;  // >= 1
  la0.load(m0, 0);
  lb0.load(n0, 0);
  la0.store(lds_a(0), tid);
  lb0.store(lds_b(0), tid);
  __syncthreads();
  typename Frag<T>::type fa[2][FM], fb[2][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
    fa[0][i] = load_frag<T, BM, BK, AK>(lds_a(0), wm * WTM + i * 32, 0, lane);
#pragma unroll
  for (int j = 0; j < FN; ++j)
    fb[0][j] = load_frag<T, BN, BK, BKC>(lds_b(0), wn * WTN + j * 32, 0, lane);
  // Register set (t - 1) % DEPTH holds tile t.
  la0.load(m0, min(1, ktiles - 1) * BK);
  lb0.load(n0, min(1, ktiles - 1) * BK);
  if constexpr (DEPTH == 2) {
    la1.load(m0, min(2, ktiles - 1) * BK);
    lb1.load(n0, min(2, ktiles - 1) * BK);
  }
  // DS reads per K step (a transposing fragment read is two instructions).
  constexpr int kReads = FM * (AK ? 1 : 2) + FN * (BKC ? 1 : 2);
  auto step = [&](int kt, auto& la, auto& lb) {
    const int cur = kt & 1;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int fc = s & 1, fn = fc ^ 1;
      if (s + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
          fa[fn][i] = load_frag<T, BM, BK, AK>(lds_a(cur), wm * WTM + i * 32,
                                               (s + 1) * 16, lane);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          fb[fn][j] = load_frag<T, BN, BK, BKC>(lds_b(cur), wn * WTN + j * 32,
                                                (s + 1) * 16, lane);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], fa[fc][i], fb[fc][j]);
      if (s + 1 == BK / 16) {
        // Nobody reads the other stage during this tile: its last reader
        // was the previous tile, which ended on a barrier.
        la.store(lds_a(cur ^ 1), tid);
        lb.store(lds_b(cur ^ 1), tid);
        // The registers are free again: request the tile DEPTH + 1 ahead
        // right away (requesting it after the barrier gave ~16% less at
        // 4096^3 with one set).
        const int k2 = min(kt + 1 + DEPTH, ktiles - 1) * BK;
        la.load(m0, k2);
        lb.load(n0, k2);
      }
      // One MFMA, then one DS read (steps 0..2) or one DS write (step 3).
#pragma unroll
      for (int q = 0; q < FM * FN; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (s + 1 < BK / 16 && q < kReads)
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (s + 1 == BK / 16 && q < la.NV + BSrc::NV)
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FM; ++i)
      fa[0][i] = load_frag<T, BM, BK, AK>(lds_a(cur ^ 1), wm * WTM + i * 32, 0,
                                          lane);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      fb[0][j] = load_frag<T, BN, BK, BKC>(lds_b(cur ^ 1), wn * WTN + j * 32,
                                           0, lane);
  };
  if constexpr (DEPTH == 1) {
    for (int kt = 0; kt < ktiles; ++kt) step(kt, la0, lb0);
  } else {
    for (int kt = 0; kt < ktiles; kt += 2) {
      step(kt, la0, lb0);
      if (kt + 1 < ktiles) step(kt + 1, la1, lb1);
    }
  }
  store_direct<T, BM, BN, WM, WN, MC>(g, acc, m0, n0, batch, lane, wm, wn);
}



// ---------------------------------------------------------------------------
// Split-K tile kernel for problems with few output tiles and long K (skinny
// GEMMs, quantized matmuls of 65..255 rows): the KW waves of a workgroup
// each walk a contiguous quarter (for KW = 4) of the K tiles of the same
// BM x BN output tile, through a wave-private LDS stage (a wave's LDS
// operations run in order, so no workgroup barrier is needed in the K
// loop; the next K tile is loaded into registers while the current one is
// used). The KW partial tiles are summed through LDS and the epilogue
// (alpha, beta C, bias, aux, activation) is applied once. BSrc is a B
// loader of the tiled kernel built for 64 threads (one wave).
// A operand loaded as stored (AK: K-contiguous), for the split-K kernel.
template <typename T, int BM, int BK, int NT, bool AK>
struct DenseA {
  static constexpr bool kKCont = AK;
  DirectLoader<T, BM, BK, NT, AK> ld;
  const T* src;
  int lda, m0, m, k, tid;
  bool vec;
  __device__ __forceinline__ DenseA(const GemmArgs& g, long long batch,
                                    int m0_, int tid_)
      : src(static_cast<const T*>(g.a) + batch * g.bsa),
        lda(g.lda),
        m0(m0_),
        m(g.m),
        k(g.k),
        tid(tid_),
        vec(g.a_vec != 0) {}
  __device__ __forceinline__ void load(int k0) {
    ld.load(src, lda, m0, k0, m, k, vec, tid);
  }
  __device__ __forceinline__ void store(T* lds) const { ld.store(lds, tid); }
};

template <typename T, int BM, int BN, int BK, int KW, class ASrc, class BSrc>
__global__ __launch_bounds__(KW * 64) void gemm_splitk_kernel(GemmArgs g) {
  constexpr int NT = KW * 64;
  constexpr int FM = BM / 32, FN = BN / 32;
  constexpr bool AK = ASrc::kKCont, BKC = BSrc::kKCont;
  using LA = TileLayout<T, BM, BK, AK>;
  using LB = TileLayout<T, BN, BK, BKC>;
  constexpr int kWaveBytes = (LA::kElems + LB::kElems) * sizeof(T);
  constexpr int kLdo = BN + 4;
  constexpr int kSumBytes = KW * BM * kLdo * 4;
  __shared__ __attribute__((aligned(16)))
  unsigned char lds_raw[KW * kWaveBytes > kSumBytes ? KW * kWaveBytes
                                                    : kSumBytes];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  T* const lds_a = reinterpret_cast<T*>(lds_raw + wave * kWaveBytes);
  T* const lds_b = lds_a + LA::kElems;

  const int nwg = g.tiles_m * g.tiles_n;
  int bid = blockIdx.x;
  if ((nwg & 7) == 0) bid = (bid & 7) * (nwg >> 3) + (bid >> 3);
  const int tm = bid % g.tiles_m, tn = bid / g.tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const long long batch = blockIdx.y;
  ASrc la(g, batch, m0, lane);
  BSrc lb(g, batch, n0, lane);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int ktiles = (g.k + BK - 1) / BK;
  const int kb = wave * ktiles / KW, ke = (wave + 1) * ktiles / KW;
  if (kb < ke) {
    la.load(kb * BK);
    lb.load(kb * BK);
  }
  for (int kt = kb; kt < ke; ++kt) {
    la.store(lds_a);
    lb.store(lds_b);
    if (kt + 1 < ke) {
      la.load((kt + 1) * BK);
      lb.load((kt + 1) * BK);
    }
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      typename Frag<T>::type fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[i] = load_frag<T, BM, BK, AK>(lds_a, i * 32, ks * 16, lane);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[j] = load_frag<T, BN, BK, BKC>(lds_b, j * 32, ks * 16, lane);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], fa[i], fb[j]);
    }
  }

  // Sum the KW partial tiles: wave w writes its tile to slice w, then all
  // threads add the slices for four consecutive columns and store them
  // with the epilogue.
  __syncthreads();
  float* sum = reinterpret_cast<float*>(lds_raw);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int col = j * 32 + (lane & 31);
        sum[(wave * BM + row) * kLdo + col] = acc[i][j][r];
      }
  __syncthreads();
  const bool of32 = g.out_f32 != 0;
  const bool vec = g.out_vec != 0;
  const long long dbase = batch * g.bsd;
  for (int q = tid; q < BM * BN / 4; q += NT) {
    const int lr = q / (BN / 4), lc = (q % (BN / 4)) * 4;
    const int row = m0 + lr, col = n0 + lc;
    if (row >= g.m || col >= g.n) continue;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < KW; ++w) {
      const float4 p =
          *reinterpret_cast<const float4*>(sum + (w * BM + lr) * kLdo + lc);
      v[0] += p.x, v[1] += p.y, v[2] += p.z, v[3] += p.w;
    }
    const int cnt = min(4, g.n - col);
    const long long idx = dbase + static_cast<long long>(row) * g.ldd + col;
    float c4[4] = {0.f, 0.f, 0.f, 0.f}, b4[4] = {0.f, 0.f, 0.f, 0.f};
    if (g.use_c) ld_out4<T>(g.c, idx, of32, vec, cnt, c4);
    if (g.has_bias) ld_out4<T>(g.bias, col, of32, false, cnt, b4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = g.alpha * v[e];
      if (g.use_c) v[e] += g.beta * c4[e];
      if (g.has_bias) v[e] += b4[e];
    }
    if (g.has_aux) st_out4<T>(g.aux, idx, of32, vec, cnt, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = act_f32(g.act, v[e]);
    st_out4<T>(g.d, idx, of32, vec, cnt, v);
  }
}

}  // namespace
}  // namespace qk
