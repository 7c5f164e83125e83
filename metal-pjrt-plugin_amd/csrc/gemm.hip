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
//  - Problems whose N and K are multiples of BN x 64 (any M) with
//    16-byte aligned operands take gemm_dma_kernel (gemm_dma.h): operand tiles go
//    from global memory straight into XOR-swizzled LDS stages, and the
//    epilogue is applied from the accumulators without LDS staging.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <string>

#include "gemm_common.h"
#include "gemm_dma.h"
#include "gemm_f32x3.h"
#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

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

template <typename T, int BM, int BN, int BK, int WM, int WN>
qk_status DispatchTile(const GemmArgs& g, int batch, bool ta, bool tb,
                       hipStream_t stream, const char* name) {
  dim3 grid(g.tiles_m * g.tiles_n, batch);
  dim3 block(WM * WN * 64);
  constexpr int NT = WM * WN * 64;
  using BN_ = DenseB<T, BN, BK, NT, false>;  // B stored [K][N]
  using BT_ = DenseB<T, BN, BK, NT, true>;   // B stored [N][K]
  if (!ta && !tb)
    gemm_tile_kernel<T, BM, BN, BK, WM, WN, false, BN_>
        <<<grid, block, 0, stream>>>(g);
  else if (!ta && tb)
    gemm_tile_kernel<T, BM, BN, BK, WM, WN, false, BT_>
        <<<grid, block, 0, stream>>>(g);
  else if (ta && !tb)
    gemm_tile_kernel<T, BM, BN, BK, WM, WN, true, BN_>
        <<<grid, block, 0, stream>>>(g);
  else
    gemm_tile_kernel<T, BM, BN, BK, WM, WN, true, BT_>
        <<<grid, block, 0, stream>>>(g);
  return PostLaunch(name);
}

template <typename T, int BN, int NW = 4, bool MC = false>
qk_status DispatchFastM(const GemmArgs& g, int batch, bool ta, bool tb,
                        hipStream_t stream, const char* name) {
  dim3 grid(g.tiles_m * g.tiles_n, batch, g.ksplit);
  if (!ta && !tb)
    gemm_dma_kernel<T, BN, false, false, NW, MC><<<grid, NW * 64, 0, stream>>>(g);
  else if (!ta && tb)
    gemm_dma_kernel<T, BN, false, true, NW, MC><<<grid, NW * 64, 0, stream>>>(g);
  else if (ta && !tb)
    gemm_dma_kernel<T, BN, true, false, NW, MC><<<grid, NW * 64, 0, stream>>>(g);
  else
    gemm_dma_kernel<T, BN, true, true, NW, MC><<<grid, NW * 64, 0, stream>>>(g);
  return PostLaunch(name);
}

// 32x32 tiles with sixteen waves over K, A [M][K] and B [N][K] only (both
// K-contiguous: the sixteen wave-private stages of the other layouts do not
// fit the LDS).
template <typename T>
qk_status DispatchSplitKNT16(const GemmArgs& g, int batch, hipStream_t stream,
                             const char* name) {
  dim3 grid(g.tiles_m * g.tiles_n, batch);
  using AN = DenseA<T, 32, 64, 64, true>;
  using BT_ = DenseB<T, 32, 64, 64, true>;
  gemm_splitk_kernel<T, 32, 32, 64, 16, AN, BT_><<<grid, 1024, 0, stream>>>(g);
  return PostLaunch(name);
}

// M a multiple of 256: the kernel without row checks; otherwise the last
// M tile is partly filled.
template <typename T, int BN, int NW = 4>
qk_status DispatchFast(const GemmArgs& g, int batch, bool ta, bool tb,
                       hipStream_t stream, const char* name) {
  if (g.m % 256 == 0)
    return DispatchFastM<T, BN, NW, false>(g, batch, ta, tb, stream, name);
  return DispatchFastM<T, BN, NW, true>(g, batch, ta, tb, stream, name);
}

template <typename T, int BMN, int KW>
qk_status DispatchSplitK(const GemmArgs& g, int batch, bool ta, bool tb,
                         hipStream_t stream, const char* name) {
  dim3 grid(g.tiles_m * g.tiles_n, batch);
  using AN = DenseA<T, BMN, 64, 64, true>;   // A stored [M][K]
  using AT = DenseA<T, BMN, 64, 64, false>;  // A stored [K][M]
  using BN_ = DenseB<T, BMN, 64, 64, false>;
  using BT_ = DenseB<T, BMN, 64, 64, true>;
  constexpr int NT = KW * 64;
  if (!ta && !tb)
    gemm_splitk_kernel<T, BMN, BMN, 64, KW, AN, BN_><<<grid, NT, 0, stream>>>(g);
  else if (!ta && tb)
    gemm_splitk_kernel<T, BMN, BMN, 64, KW, AN, BT_><<<grid, NT, 0, stream>>>(g);
  else if (ta && !tb)
    gemm_splitk_kernel<T, BMN, BMN, 64, KW, AT, BN_><<<grid, NT, 0, stream>>>(g);
  else
    gemm_splitk_kernel<T, BMN, BMN, 64, KW, AT, BT_><<<grid, NT, 0, stream>>>(g);
  return PostLaunch(name);
}

template <int BM, int BN, int NW, bool MC, int KS, int BK>
qk_status DispatchF32x3M(const GemmArgs& g, int batch, bool ta, bool tb,
                         hipStream_t stream, const char* name) {
  dim3 grid(g.tiles_m * g.tiles_n, batch);
  if (!ta && !tb)
    gemm_f32x3_kernel<BM, BN, false, false, NW, MC, KS, BK><<<grid, NW * 64, 0, stream>>>(g);
  else if (!ta && tb)
    gemm_f32x3_kernel<BM, BN, false, true, NW, MC, KS, BK><<<grid, NW * 64, 0, stream>>>(g);
  else if (ta && !tb)
    gemm_f32x3_kernel<BM, BN, true, false, NW, MC, KS, BK><<<grid, NW * 64, 0, stream>>>(g);
  else
    gemm_f32x3_kernel<BM, BN, true, true, NW, MC, KS, BK><<<grid, NW * 64, 0, stream>>>(g);
  return PostLaunch(name);
}

// M a multiple of BM: the kernel without row checks; otherwise the last M
// tile is partly filled.
template <int BM, int BN, int NW, int KS = 1, int BK = 32>
qk_status DispatchF32x3(const GemmArgs& g, int batch, bool ta, bool tb,
                        hipStream_t stream, const char* name) {
  if (g.m % BM == 0)
    return DispatchF32x3M<BM, BN, NW, false, KS, BK>(g, batch, ta, tb, stream,
                                                     name);
  return DispatchF32x3M<BM, BN, NW, true, KS, BK>(g, batch, ta, tb, stream,
                                                  name);
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

// f16/bf16 tile configurations: BM, BN, waves along M, waves along N.
struct HalfTile {
  int bm, bn, wm, wn;
};
constexpr HalfTile kHalfTiles[] = {
    {256, 256, 2, 2},  // 0: 128x128 per wave, one wave per SIMD
    {256, 256, 2, 4},  // 1: 128x64 per wave
    {128, 128, 2, 2},  // 2
    {64, 64, 2, 2},    // 3
    {256, 128, 2, 2},  // 4
    {128, 256, 2, 2},  // 5
    {256, 256, 4, 2},  // 6: interior-tile LDS-DMA kernel (gemm_dma_kernel),
                       //    8 waves of 64 x 128, two per SIMD
    {256, 128, 2, 2},  // 7: interior-tile LDS-DMA kernel, 128 x 64 per wave
    {64, 64, 2, 2},    // 8: split-K, four waves each a quarter of K
    {32, 32, 2, 4},    // 9: split-K for up to 32 rows, eight waves
    {256, 192, 4, 2},  // 10: interior-tile LDS-DMA kernel, 8 waves of 64 x 96
    {32, 32, 2, 8},    // 11: split-K for up to 64 rows, sixteen waves
};
constexpr int kFastTile256 = 6, kFastTile128 = 7, kSplitK = 8, kSplitK32 = 9,
              kFastTile192 = 10, kSplitK32W16 = 11;
// f32 problems on the split-bf16 kernel, and few-row f16/bf16 problems on
// the wide gemv (tile indices below 0: not kHalfTiles entries).
constexpr int kF32x3Tile128 = -2, kF32x3Tile64 = -3, kGemvTile = -4;
constexpr int kNumHalfTiles = sizeof(kHalfTiles) / sizeof(kHalfTiles[0]);

// Cost of a round of 256x192 interior tiles relative to 256x256.
constexpr double kCost192 = 0.95;

// QK_GEMM_TILE=<index into kHalfTiles> forces a configuration (tuning).
int ForcedHalfTile() {
  static const int forced = [] {
    const char* v = std::getenv("QK_GEMM_TILE");
    if (v == nullptr || *v < '0' || *v > '9') return -1;
    const int t = std::atoi(v);
    return t >= 0 && t < kNumHalfTiles ? t : -1;
  }();
  return forced;
}

// Whether the split-bf16 f32 kernel (gemm_f32x3.h) can run the problem
// with bm x bn tiles: f32, any M (the last M tile may be partly filled),
// N a multiple of the tile, K of 32, 16-byte aligned operands and leading
// dimensions, and each operand of one batch entry, with A padded to whole
// tiles, under 2^31 bytes (the extent of a buffer descriptor).
bool F32x3Applies(const GemmProblem& p, int bm, int bn) {
  if (p.a.dtype != QK_F32 || p.m == 0 || p.n % bn != 0 || p.k % 32 != 0 ||
      p.k == 0)
    return false;
  const bool batched = p.batch > 1;
  // elems: the largest element offset a tile can address, plus one
  auto ok = [&](const Operand& o, int64_t elems) {
    const int64_t bs = batched ? o.batch_stride : 0;
    return reinterpret_cast<uintptr_t>(o.ptr) % 16 == 0 && o.ld % 4 == 0 &&
           bs % 4 == 0 && elems * 4 < (int64_t{1} << 31);
  };
  const int64_t mpad = (p.m + bm - 1) / bm * bm;
  return ok(p.a, p.a.transpose ? (p.k - 1) * p.a.ld + mpad
                               : mpad * p.a.ld) &&
         ok(p.b, (p.b.transpose ? p.n : p.k) * p.b.ld);
}

// Whether the interior-tile kernel can run the problem with a BN-wide
// tile: N and K multiples of the tile (any M: the last M tile may be
// partly filled), 16-byte aligned operands and leading dimensions, and
// each operand of one batch entry, with A padded to whole 256-row tiles,
// under 2^31 bytes (the extent of a buffer descriptor).
bool FastApplies(const GemmProblem& p, int bn) {
  if (p.a.dtype == QK_F32 || p.m == 0 || p.n % bn != 0 || p.k % 64 != 0 ||
      p.k == 0)
    return false;
  const int vec = 16 / DTypeSize(p.a.dtype);
  const bool batched = p.batch > 1;
  // elems: the largest element offset a tile can address, plus one
  auto ok = [&](const Operand& o, int64_t elems) {
    const int64_t bs = batched ? o.batch_stride : 0;
    return reinterpret_cast<uintptr_t>(o.ptr) % 16 == 0 && o.ld % vec == 0 &&
           bs % vec == 0 && elems * DTypeSize(o.dtype) < (int64_t{1} << 31);
  };
  const int64_t mpad = CeilDiv(p.m, 256) * 256;
  return ok(p.a, p.a.transpose ? (p.k - 1) * p.a.ld + mpad
                               : mpad * p.a.ld) &&
         ok(p.b, (p.b.transpose ? p.n : p.k) * p.b.ld);
}

GemmKernelChoice ChooseGemmKernel(const GemmProblem& p) {
  GemmKernelChoice c;
  const bool half = p.a.dtype != QK_F32;
  const int64_t batch = std::max<int64_t>(p.batch, 1);
  auto tiles = [&](int bm, int bn) {
    return CeilDiv(p.m, bm) * CeilDiv(p.n, bn) * batch;
  };
  if (half) {
    int t = ForcedHalfTile();
    if ((t == kFastTile256 && !FastApplies(p, 256)) ||
        (t == kFastTile192 && !FastApplies(p, 192)) ||
        (t == kFastTile128 && !FastApplies(p, 128)))
      t = -1;
    if (t == kSplitK32W16 && (p.a.transpose || !p.b.transpose))
      t = kSplitK32;
    const int cus = DeviceComputeUnits();
    if (t < 0) {
      // One 256-row tile per CU: the fewest rounds of resident tiles,
      // weighted by the cost of a round measured on MI355X relative to a
      // round of 256x256 tiles (256x192 ~0.95, 256x128 ~0.67); a width
      // qualifies when it gives at least half the CUs a tile.
      double best = 1e30;
      const struct { int bn, tile; double cost; } cand[] = {
          {256, kFastTile256, 1.0},
          {192, kFastTile192, kCost192},
          {128, kFastTile128, 0.67}};
      for (const auto& c : cand) {
        if (!FastApplies(p, c.bn) || tiles(256, c.bn) < cus / 2) continue;
        const double r =
            c.cost * static_cast<double>(CeilDiv(tiles(256, c.bn), cus));
        if (r < best) best = r, t = c.tile;
      }
    }
    // Too few 256 x 128 tiles to occupy the CUs, more than 64 rows and one
    // batch entry: the same tiles with K split over workgroups (partials
    // summed in K order by the last workgroup of each tile), the largest
    // power-of-two split up to 8 that keeps every workgroup resident (one
    // per CU) with at least 16 K tiles per split; where the split-K 64 x 64
    // kernel below takes one round of workgroups and K is below 8192 that
    // kernel instead. Measured on MI355X (bf16, us, split / previous):
    // 512 x 4096 x 12288 76 / 163, 256 x 4096 x 12288 63 / 78, 256 x 12288
    // x 4096 46 / 72, 384 x 4096 x 4096 36 / 48; 128 x 4096 x 4096 32 / 26
    // (the split-K kernel kept). QK_GEMM_KSPLIT=<s> forces the split where
    // the tiles apply, 0 turns the path off (tuning and tests).
    const bool splitk =
        tiles(64, 64) < 2 * cus && CeilDiv(p.k, 64) >= 16;
    // (A [M][K] against NT weights, at most 128 rows: the split-K kernel
    // also over two rounds, 128 x 12288 x 4096 41 against 49 us.)
    const bool nt_layout = !p.a.transpose && p.b.transpose;
    // (Also 256 x 128 tiles that leave half the CUs idle at K >= 8192:
    // 1024 x 4096 x 12288 split 2.)
    const bool few128 = t == kFastTile128 && p.k >= 8192 &&
                        ForcedHalfTile() < 0;
    if ((t < 0 || few128) && p.batch <= 1 && p.m > 64 &&
        FastApplies(p, 128)) {
      const char* v = std::getenv("QK_GEMM_KSPLIT");
      const int forced = v == nullptr ? -1 : std::atoi(v);
      const int64_t nt = tiles(256, 128), kt = p.k / 64;
      int split = 1;
      if (forced > 0) {
        split = static_cast<int>(std::min<int64_t>(forced, kt));
      } else if (forced < 0 &&
                 (p.k >= 8192 || !splitk ||
                  (tiles(64, 64) > cus &&
                   !(nt_layout && p.m <= 128)))) {
        for (int s2 = 2; s2 <= 8; s2 *= 2)
          if (nt * s2 <= cus && kt / s2 >= 16) split = s2;
      }
      if (split > 1) t = kFastTile128, c.split_k = split;
    }
    // At most eight rows of x against NT weights: the wide gemv
    // (bandwidth-bound on the weights).
    // Few 64x64 tiles and a long K: split K over the waves of each tile
    // (32x32 tiles and eight waves for at most 64 rows or columns: at 33..64
    // rows they give twice the workgroups over the same weight columns;
    // 28 x [64, 1024] x [1024, 6144]^T 312 -> 229 us on MI355X). At most 16
    // rows against NT weights: sixteen waves, twice the loads in flight per
    // workgroup (M = 16 184 -> 168 us; M = 8 173 us against the gemv's 200).
    const bool nt16 = splitk && p.m <= 16 && !p.a.transpose && p.b.transpose;
    // At most four rows of x against NN weights of at least 2^25 values:
    // the NN gemv (one workgroup per 64 columns walking all of K; M = 1
    // 12288 x 4096 23 us, 4096 x 12288 52, against 47 / 68 on the split-K
    // kernel and 26 / 62 for hipBLASLt; at 4096 x 4096 and below level or
    // slower). QK_GEMV_NN=0 turns it off, =2 takes it wherever it applies
    // (tuning and tests, read at every plan).
    const char* gnv = std::getenv("QK_GEMV_NN");
    const bool gemv_nn = (gnv == nullptr ? p.n * p.k >= (int64_t{1} << 25)
                                         : *gnv == '2') &&
                         GemvNNApplies(p);
    if (t < 0 && (GemvApplies(p) || gemv_nn) && !(nt16 && p.m > 6))
      t = kGemvTile;
    if (t == -1 && splitk)
      t = nt16                           ? kSplitK32W16
          : std::min(p.m, p.n) <= 64 ? kSplitK32
                                         : kSplitK;
    if (t == -1) {
      // Rounds of resident tiles on the 256 CUs: one 256x256 tile (8
      // waves) per CU, two 128x128 tiles per CU. Measured on MI355X, a
      // round of 128x128 tiles costs ~0.6 of a round of 256x256 tiles.
      const double r256 = static_cast<double>(CeilDiv(tiles(256, 256), cus));
      const double r128 =
          0.6 * static_cast<double>(CeilDiv(tiles(128, 128), 2 * cus));
      if (tiles(128, 128) < cus)
        t = 3;  // too little work for 128x128 tiles to fill the GPU
      else
        t = r256 <= r128 ? 1 : 2;
    }
    c.tile = t;
    if (t == kGemvTile)
      c.bm = static_cast<int>(p.m), c.bn = 4, c.bk = 512;
    else
      c.bm = kHalfTiles[t].bm, c.bn = kHalfTiles[t].bn, c.bk = 64;
  } else {
    // f32: the split-bf16 kernel on interior tiles (128x128 when those
    // fill the GPU, else 64x64), the f32-MFMA tile kernel otherwise.
    // QK_GEMM_F32=mfma forces the latter (tuning).
    static const bool mfma_only = [] {
      const char* v = std::getenv("QK_GEMM_F32");
      return v != nullptr && std::string(v) == "mfma";
    }();
    const int cus = DeviceComputeUnits();
    c.tile = -1;
    if (!mfma_only && tiles(128, 128) >= cus && F32x3Applies(p, 128, 128)) {
      c.tile = kF32x3Tile128;
      c.bm = 128, c.bn = 128, c.bk = 32;
    } else if (!mfma_only && F32x3Applies(p, 64, 64)) {
      // Four wave groups over 64-wide K tiles when K allows, else two over
      // 32-wide ones; QK_GEMM_F32=x2 forces the latter (tuning).
      static const bool x2 = [] {
        const char* v = std::getenv("QK_GEMM_F32");
        return v != nullptr && std::string(v) == "x2";
      }();
      c.tile = kF32x3Tile64;
      c.bm = 64, c.bn = 64, c.bk = p.k % 64 == 0 && !x2 ? 64 : 32;
    } else if (tiles(128, 128) >= 192) {
      c.bm = 128, c.bn = 128, c.bk = 32;
    } else {
      c.bm = 64, c.bn = 64, c.bk = 32;
    }
  }
  const bool fast = half && (c.tile == kFastTile256 || c.tile == kFastTile192 ||
                             c.tile == kFastTile128);
  const bool splitk =
      c.tile == kSplitK || c.tile == kSplitK32 || c.tile == kSplitK32W16;
  const bool x3 = c.tile == kF32x3Tile128 || c.tile == kF32x3Tile64;
  const bool gemv = c.tile == kGemvTile;
  if (gemv) {
    c.name = std::string(p.b.transpose ? "gemv_nt_" : "gemv_nn_") +
             DTypeName(p.a.dtype) + "_m" +
             std::to_string(p.m) + "_k" + std::to_string(p.k);
    return c;
  }
  c.name = std::string(splitk     ? (c.tile == kSplitK     ? "gemm_splitk4_"
                                     : c.tile == kSplitK32 ? "gemm_splitk8_"
                                                           : "gemm_splitk16_")
                       : x3       ? "gemm_f32x3_"
                       : !half    ? "gemm_mfma_"
                       : fast     ? "gemm_fast_"
                                  : "gemm_tile_") +
           DTypeName(p.a.dtype) + "_" + std::to_string(c.bm) + "x" +
           std::to_string(c.bn) + "x" + std::to_string(c.bk) +
           (c.tile >= 0 ? "_w" + std::to_string(kHalfTiles[c.tile].wm *
                                                kHalfTiles[c.tile].wn)
                        : std::string()) +
           (p.a.transpose ? "_t" : "_n") + (p.b.transpose ? "t" : "n") +
           (c.split_k > 1 ? "_ks" + std::to_string(c.split_k) : std::string());
  return c;
}

template <typename T>
qk_status DispatchHalf(int tile, const GemmArgs& g, int batch, bool ta,
                       bool tb, hipStream_t st, const char* name) {
  switch (tile) {
    case 0:
      return DispatchTile<T, 256, 256, 64, 2, 2>(g, batch, ta, tb, st, name);
    case 1:
      return DispatchTile<T, 256, 256, 64, 2, 4>(g, batch, ta, tb, st, name);
    case 2:
      return DispatchTile<T, 128, 128, 64, 2, 2>(g, batch, ta, tb, st, name);
    case 4:
      return DispatchTile<T, 256, 128, 64, 2, 2>(g, batch, ta, tb, st, name);
    case 5:
      return DispatchTile<T, 128, 256, 64, 2, 2>(g, batch, ta, tb, st, name);
    case kFastTile256:
      return DispatchFast<T, 256, 8>(g, batch, ta, tb, st, name);
    case kFastTile128:
      return DispatchFast<T, 128>(g, batch, ta, tb, st, name);
    case kFastTile192:
      return DispatchFast<T, 192, 8>(g, batch, ta, tb, st, name);
    case kSplitK:
      return DispatchSplitK<T, 64, 4>(g, batch, ta, tb, st, name);
    case kSplitK32:
      return DispatchSplitK<T, 32, 8>(g, batch, ta, tb, st, name);
    case kSplitK32W16:
      return DispatchSplitKNT16<T>(g, batch, st, name);
    default:
      return DispatchTile<T, 64, 64, 64, 2, 2>(g, batch, ta, tb, st, name);
  }
}

qk_status LaunchGemm(const GemmProblem& p, hipStream_t stream) {
  const GemmKernelChoice c = ChooseGemmKernel(p);
  GemmArgs g{};
  g.ksplit = 1;
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
  g.out_vec = (reinterpret_cast<uintptr_t>(p.d.ptr) % 16 == 0) &&
              p.d.ld % 4 == 0 && g.bsd % 4 == 0;
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
  if (c.split_k > 1) {
    // f32 partial tiles in the stream's library workspace; without one
    // (it cannot grow while the stream is captured) one workgroup per tile.
    const size_t bytes = static_cast<size_t>(g.tiles_m) * g.tiles_n *
                         c.split_k * c.bm * c.bn * sizeof(float);
    if (bytes < (size_t{1} << 31) &&
        static_cast<size_t>(g.tiles_m) * g.tiles_n <= kWsFlagBytes / 4 &&
        StreamWorkspace(stream, bytes, &g.ws, &g.wsflag))
      g.ksplit = c.split_k;
  }
  if (c.tile == kGemvTile) return LaunchGemv(p, stream);
  switch (p.a.dtype) {
    case QK_BF16:
      return DispatchHalf<bf16>(c.tile, g, batch, ta, tb, stream, name);
    case QK_F16:
      return DispatchHalf<f16>(c.tile, g, batch, ta, tb, stream, name);
    default:
      if (c.tile == kF32x3Tile128)  // 16 waves in two K-step groups
        return DispatchF32x3<128, 128, 16, 2>(g, batch, ta, tb, stream, name);
      if (c.tile == kF32x3Tile64) {
        // 64x64 tiles: 16 waves in four groups over a 64-wide K tile, or
        // 8 in two over a 32-wide one (ChooseGemmKernel's bk).
        if (c.bk == 64)
          return DispatchF32x3<64, 64, 16, 4, 64>(g, batch, ta, tb, stream,
                                                  name);
        return DispatchF32x3<64, 64, 8, 2>(g, batch, ta, tb, stream, name);
      }
      if (c.bm == 128)
        return Dispatch<float, 128, 128, 32, 2, 2>(g, batch, ta, tb, stream, name);
      return Dispatch<float, 64, 64, 32, 2, 2>(g, batch, ta, tb, stream, name);
  }
}

}  // namespace qk
