// Dense GEMM for gfx950 on MFMA, with the cuBLASLt epilogue applied in the
// store. Replaces the reference's steel GEMM (metal_pjrt/blas/
// steel_gemm.cc:163-255, kernels/steel_gemm.metal:334-402) and its MPS f32
// path plus second-pass epilogue (metal_pjrt/blas/metal_blas.cc:102-171).
//
// Design (MI355X-first, not a port of the simdgroup-MMA tiling):
//  - One workgroup computes a BM x BN tile of D. Both operand tiles live in
//    LDS K-contiguous ([rows][BK + pad]), so every MFMA operand fragment is
//    one 16-byte LDS read per lane. An operand stored with K as its slow
//    dimension (B in the NN layout, A when transposed) is transposed on its
//    way from registers into LDS.
//  - Two LDS stages: the next K slab is loaded from HBM into registers
//    while the current one feeds the MFMAs, then written to the other
//    stage; one barrier per K step.
//  - f16/bf16 use v_mfma_f32_32x32x16_{f16,bf16}; f32 uses
//    v_mfma_f32_32x32x2_f32 eight times per 16-wide K step. Accumulation is
//    always f32.
//  - The epilogue (alpha, beta*C, bias[col], aux, ReLU/GELU/SiLU) is
//    applied to the f32 accumulators and rounded once into D's type.
//  - Workgroup ids are remapped so that consecutive tiles share an XCD
//    (the hardware deals workgroups round-robin over the 8 XCDs, each with
//    its own L2) and tiles are visited in groups of GROUP_M tile rows.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>

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
  int tiles_m, tiles_n;
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
// tile is transposed on its way into LDS.
template <typename T, int R, int BK, int NT, bool KMAJOR>
struct TileLoader {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int E = R * BK / NT;  // elements per thread
  static_assert(E % VEC == 0, "tile does not split into 16-byte vectors");
  // Direct: E / VEC vectors along K. Transposing: KSUB source rows (K) of
  // one VEC-wide column group, UNITS times.
  static constexpr int NVEC = E / VEC;
  static constexpr int KSUB = NVEC < 4 ? NVEC : 4;
  static constexpr int UNITS = NVEC / KSUB;
  static_assert(NVEC % KSUB == 0, "bad transposing split");

  Vec16<T> v[NVEC];

  // src points at the operand's batch base; (r0, k0) is the tile origin;
  // rows_total / k_total bound it; ld is the source's row stride.
  __device__ __forceinline__ void load(const T* __restrict__ src, int ld,
                                       int r0, int k0, int rows_total,
                                       int k_total, bool vec_ok, int tid) {
    if constexpr (!KMAJOR) {
      constexpr int VPR = BK / VEC;  // vectors per row
#pragma unroll
      for (int i = 0; i < NVEC; ++i) {
        const int id = tid + i * NT;
        const int r = id / VPR;
        const int c = (id % VPR) * VEC;
        const int gr = r0 + r, gc = k0 + c;
        const T* p = src + static_cast<long long>(gr) * ld + gc;
        if (vec_ok && gr < rows_total && gc + VEC <= k_total) {
          v[i].u = *reinterpret_cast<const u32x4*>(p);
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            v[i].e[e] = (gr < rows_total && gc + e < k_total) ? p[e] : T(0);
        }
      }
    } else {
      constexpr int GPR = R / VEC;  // column groups per source row
#pragma unroll
      for (int u = 0; u < UNITS; ++u) {
        const int id = tid + u * NT;
        const int kb = id / GPR;  // block of KSUB source rows
        const int c = (id % GPR) * VEC;
        const int gc = r0 + c;
#pragma unroll
        for (int s = 0; s < KSUB; ++s) {
          const int gk = k0 + kb * KSUB + s;
          const T* p = src + static_cast<long long>(gk) * ld + gc;
          Vec16<T>& dst = v[u * KSUB + s];
          if (vec_ok && gk < k_total && gc + VEC <= rows_total) {
            dst.u = *reinterpret_cast<const u32x4*>(p);
          } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e)
              dst.e[e] = (gk < k_total && gc + e < rows_total) ? p[e] : T(0);
          }
        }
      }
    }
  }

  // lds is [R][LDK]: row-major, K contiguous.
  template <int LDK>
  __device__ __forceinline__ void store(T* lds, int tid) const {
    if constexpr (!KMAJOR) {
      constexpr int VPR = BK / VEC;
#pragma unroll
      for (int i = 0; i < NVEC; ++i) {
        const int id = tid + i * NT;
        const int r = id / VPR;
        const int c = (id % VPR) * VEC;
        *reinterpret_cast<u32x4*>(lds + r * LDK + c) = v[i].u;
      }
    } else {
      constexpr int GPR = R / VEC;
#pragma unroll
      for (int u = 0; u < UNITS; ++u) {
        const int id = tid + u * NT;
        const int kb = id / GPR;
        const int c = (id % GPR) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          T* dst = lds + (c + e) * LDK + kb * KSUB;
          T tmp[KSUB];
#pragma unroll
          for (int s = 0; s < KSUB; ++s) tmp[s] = v[u * KSUB + s].e[e];
          if constexpr (KSUB * sizeof(T) == 16) {
            *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<u32x4*>(tmp);
          } else if constexpr (KSUB * sizeof(T) == 8) {
            *reinterpret_cast<u32x2*>(dst) = *reinterpret_cast<u32x2*>(tmp);
          } else if constexpr (KSUB * sizeof(T) == 4) {
            *reinterpret_cast<uint32_t*>(dst) =
                *reinterpret_cast<uint32_t*>(tmp);
          } else {
#pragma unroll
            for (int s = 0; s < KSUB; ++s) dst[s] = tmp[s];
          }
        }
      }
    }
  }
};

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

// TA: A is stored [K][M] (column-major op(A)); TB: B is stored [N][K].
template <typename T, int BM, int BN, int BK, int WM, int WN, bool TA, bool TB>
__global__ __launch_bounds__(WM* WN * 64) void gemm_mfma_kernel(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int PAD = 16 / sizeof(T);
  constexpr int LDK = BK + PAD;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  static_assert(FM >= 1 && FN >= 1 && BK % 16 == 0, "bad tile");

  __shared__ __attribute__((aligned(16))) T lds_a[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) T lds_b[2][BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // Tile id: XCD-contiguous remap, then GROUP_M row groups.
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
  const T* B = static_cast<const T*>(g.b) + batch * g.bsb;

  TileLoader<T, BM, BK, NT, TA> la;
  TileLoader<T, BN, BK, NT, !TB> lb;

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
    lb.load(B, g.ldb, n0, 0, g.n, g.k, g.b_vec, tid);
    la.template store<LDK>(lds_a[0], tid);
    lb.template store<LDK>(lds_b[0], tid);
    __syncthreads();
  }
  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      la.load(A, g.lda, m0, (kt + 1) * BK, g.m, g.k, g.a_vec, tid);
      lb.load(B, g.ldb, n0, (kt + 1) * BK, g.n, g.k, g.b_vec, tid);
    }
    const T* sa = lds_a[cur] + (wm * WTM + (lane & 31)) * LDK + (lane >> 5) * 8;
    const T* sb = lds_b[cur] + (wn * WTN + (lane & 31)) * LDK + (lane >> 5) * 8;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      typename Frag<T>::type fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) fa[i] = lds_frag<T>(sa + i * 32 * LDK + ks * 16);
#pragma unroll
      for (int j = 0; j < FN; ++j) fb[j] = lds_frag<T>(sb + j * 32 * LDK + ks * 16);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], fa[i], fb[j]);
    }
    if (more) {
      la.template store<LDK>(lds_a[cur ^ 1], tid);
      lb.template store<LDK>(lds_b[cur ^ 1], tid);
    }
    __syncthreads();
  }

  // Epilogue: lane holds rows 8*(r/4) + 4*(lane/32) + r%4 of column
  // lane%32 of each 32x32 block.
  const bool of32 = g.out_f32 != 0;
  const long long dbase = batch * g.bsd;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = n0 + wn * WTN + j * 32 + (lane & 31);
    if (col >= g.n) continue;
    const float bias = g.has_bias ? ld_out<T>(g.bias, col, of32) : 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) +
                        4 * (lane >> 5) + (r & 3);
        if (row >= g.m) continue;
        const long long idx = dbase + static_cast<long long>(row) * g.ldd + col;
        float v = g.alpha * acc[i][j][r];
        if (g.use_c) v += g.beta * ld_out<T>(g.c, idx, of32);
        if (g.has_bias) v += bias;
        if (g.has_aux) st_out<T>(g.aux, idx, of32, v);
        st_out<T>(g.d, idx, of32, act_f32(g.act, v));
      }
    }
  }
}

struct TileCfg {
  int bm, bn, bk, wm, wn;
};

template <typename T, int BM, int BN, int BK, int WM, int WN>
qk_status Dispatch(const GemmArgs& g, int batch, bool ta, bool tb,
                   hipStream_t stream, const char* name) {
  dim3 grid(g.tiles_m * g.tiles_n, batch);
  dim3 block(WM * WN * 64);
  if (!ta && !tb)
    gemm_mfma_kernel<T, BM, BN, BK, WM, WN, false, false>
        <<<grid, block, 0, stream>>>(g);
  else if (!ta && tb)
    gemm_mfma_kernel<T, BM, BN, BK, WM, WN, false, true>
        <<<grid, block, 0, stream>>>(g);
  else if (ta && !tb)
    gemm_mfma_kernel<T, BM, BN, BK, WM, WN, true, false>
        <<<grid, block, 0, stream>>>(g);
  else
    gemm_mfma_kernel<T, BM, BN, BK, WM, WN, true, true>
        <<<grid, block, 0, stream>>>(g);
  return PostLaunch(name);
}

int64_t CeilDiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace

GemmKernelChoice ChooseGemmKernel(const GemmProblem& p) {
  GemmKernelChoice c;
  const bool half = p.a.dtype != QK_F32;
  const int64_t batch = std::max<int64_t>(p.batch, 1);
  auto tiles = [&](int bm, int bn) {
    return CeilDiv(p.m, bm) * CeilDiv(p.n, bn) * batch;
  };
  if (half) {
    if (tiles(256, 256) >= 192) {
      c.bm = 256, c.bn = 256, c.bk = 64;
    } else if (tiles(128, 128) >= 128) {
      c.bm = 128, c.bn = 128, c.bk = 64;
    } else {
      c.bm = 64, c.bn = 64, c.bk = 64;
    }
  } else {
    if (tiles(128, 128) >= 192) {
      c.bm = 128, c.bn = 128, c.bk = 32;
    } else {
      c.bm = 64, c.bn = 64, c.bk = 32;
    }
  }
  c.name = std::string("gemm_mfma_") + DTypeName(p.a.dtype) + "_" +
           std::to_string(c.bm) + "x" + std::to_string(c.bn) + "x" +
           std::to_string(c.bk) + (p.a.transpose ? "_t" : "_n") +
           (p.b.transpose ? "t" : "n");
  return c;
}

qk_status LaunchGemm(const GemmProblem& p, hipStream_t stream) {
  const GemmKernelChoice c = ChooseGemmKernel(p);
  GemmArgs g;
  g.a = p.a.ptr;
  g.b = p.b.ptr;
  g.c = p.c;
  g.d = const_cast<void*>(p.d.ptr);
  g.bias = p.bias;
  g.aux = p.aux;
  g.m = static_cast<int>(p.m);
  g.n = static_cast<int>(p.n);
  g.k = static_cast<int>(p.k);
  g.lda = static_cast<int>(p.a.ld);
  g.ldb = static_cast<int>(p.b.ld);
  g.ldd = static_cast<int>(p.d.ld);
  const bool batched = p.batch > 1;
  g.bsa = batched ? p.a.batch_stride : 0;
  g.bsb = batched ? p.b.batch_stride : 0;
  g.bsd = batched ? p.d.batch_stride : 0;
  g.alpha = p.alpha;
  g.beta = p.beta;
  g.use_c = p.c != nullptr && p.beta != 0.f;
  g.has_bias = p.bias != nullptr;
  g.has_aux = p.aux != nullptr;
  g.act = p.act;
  g.out_f32 = p.d.dtype == QK_F32;
  const int esz = DTypeSize(p.a.dtype);
  const int vec = 16 / esz;
  auto vec_ok = [&](const Operand& o, long long bs) {
    return (reinterpret_cast<uintptr_t>(o.ptr) % 16 == 0) && o.ld % vec == 0 &&
           bs % vec == 0;
  };
  g.a_vec = vec_ok(p.a, g.bsa);
  g.b_vec = vec_ok(p.b, g.bsb);
  g.tiles_m = static_cast<int>(CeilDiv(p.m, c.bm));
  g.tiles_n = static_cast<int>(CeilDiv(p.n, c.bn));
  if (p.batch > 65535) {
    return Fail(QK_UNIMPLEMENTED, "qkern: matmul batch count " +
                                      std::to_string(p.batch) +
                                      " exceeds the grid limit 65535");
  }
  if (static_cast<int64_t>(g.tiles_m) * g.tiles_n > 0x7fffffff) {
    return Fail(QK_UNIMPLEMENTED, "qkern: matmul has too many tiles");
  }
  const int batch = static_cast<int>(p.batch);
  const bool ta = p.a.transpose, tb = p.b.transpose;
  const char* name = c.name.c_str();
  switch (p.a.dtype) {
    case QK_BF16:
      if (c.bm == 256)
        return Dispatch<bf16, 256, 256, 64, 2, 4>(g, batch, ta, tb, stream, name);
      if (c.bm == 128)
        return Dispatch<bf16, 128, 128, 64, 2, 2>(g, batch, ta, tb, stream, name);
      return Dispatch<bf16, 64, 64, 64, 2, 2>(g, batch, ta, tb, stream, name);
    case QK_F16:
      if (c.bm == 256)
        return Dispatch<f16, 256, 256, 64, 2, 4>(g, batch, ta, tb, stream, name);
      if (c.bm == 128)
        return Dispatch<f16, 128, 128, 64, 2, 2>(g, batch, ta, tb, stream, name);
      return Dispatch<f16, 64, 64, 64, 2, 2>(g, batch, ta, tb, stream, name);
    default:
      if (c.bm == 128)
        return Dispatch<float, 128, 128, 32, 2, 2>(g, batch, ta, tb, stream, name);
      return Dispatch<float, 64, 64, 32, 2, 2>(g, batch, ta, tb, stream, name);
  }
}

}  // namespace qk
