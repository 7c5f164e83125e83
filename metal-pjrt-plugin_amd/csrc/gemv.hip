// Few-row f16/bf16 GEMM ("wide gemv") for gfx950: D = act(alpha x W^T +
// beta C + bias) for at most 8 rows of x, with W stored [N][K] (K
// contiguous: the NT layout of a linear layer's weights).
//
// Replaces the reference's wide gemv (metal_pjrt/blas/gemv.cc:68-196,
// kernels/gemv.metal:73-176: 2..8 vectors, K >= 512, NT layout, the GEMM
// store epilogue) for the shapes its ChooseGemv takes. The work is
// bandwidth-bound on W: each wavefront streams whole 1 KB rows of W (lane l
// reads 16-byte chunk l + 64 j of the row, j < K / 512) with every row of
// x held in its registers (the same chunks for every row of W), forms the
// M dot products per row with v_dot2_f32_{bf16,f16}, and reduces D rows x
// M values over the wave four at a time (DPP). The D weight rows of a
// round are requested before the previous round is reduced.
//
// The store applies the BlasLt epilogue of the tiled kernels, in f32, one
// rounding: v = alpha acc (+ beta C) (+ bias[n]); aux = v; D = act(v).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>

#include "gemm_common.h"
#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

constexpr int kGemvThreads = 256;
constexpr int kGemvRows = 4;  // weight rows per wave per round

template <typename T>
__device__ __forceinline__ float Dot8(const u32x4& w, const u32x4& x,
                                      float acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (std::is_same_v<T, bf16>) {
      acc = __builtin_amdgcn_fdot2_f32_bf16(AsBf16x2(w[e]), AsBf16x2(x[e]),
                                            acc, false);
    } else {
      // Through plain values: clang miscompiles a bit cast applied
      // directly to an element of an ext_vector_type.
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      const uint32_t wv = w[e], xv = x[e];
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, wv),
                                   __builtin_bit_cast(h2, xv), acc, false);
    }
  }
  return acc;
}

// M rows of x (M <= 8), CPL = K / 512 chunks of 16 bytes per lane and row.
template <typename T, int M, int CPL>
__global__ __launch_bounds__(kGemvThreads) void gemv_nt_kernel(GemmArgs g) {
  constexpr int D = kGemvRows;
  constexpr int NV = D * M;  // values reduced per round
  constexpr int NV4 = (NV + 3) / 4 * 4;
  const int lane = threadIdx.x & 63;
  const int gw = __builtin_amdgcn_readfirstlane(
      blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6));
  const int GW = gridDim.x * (kGemvThreads / 64);
  const long long batch = blockIdx.y;
  const T* A = static_cast<const T*>(g.a) + batch * g.bsa;
  const T* B = static_cast<const T*>(g.b) + batch * g.bsb;

  // x in registers: chunk lane + 64 j of every row.
  u32x4 xr[M][CPL];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      xr[m][j] = *reinterpret_cast<const u32x4*>(
          A + static_cast<long long>(m) * g.lda + 8 * (lane + 64 * j));

  // Rows of W as one buffer descriptor per batch entry (extent: the rows
  // that exist, so rows past N read zeros without a branch).
  const long long wbytes = (static_cast<long long>(g.n - 1) * g.ldb + g.k) *
                           static_cast<long long>(sizeof(T));
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(B), (short)0,
      static_cast<int>(std::min<long long>(wbytes, 0x7FFFFFFFll)), 0x00020000);
  const int lo = lane * 16;
  auto load = [&](int n0, u32x4 (&w)[D][CPL]) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int n = n0 + d * GW;
      // rows past N: an offset past the extent (zeros, no access)
      const int ro = n < g.n ? n * g.ldb * static_cast<int>(sizeof(T))
                             : 0x7FFF0000;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        w[d][j] = __builtin_amdgcn_raw_buffer_load_b128(wrs, lo + 1024 * j,
                                                        ro, 2);
    }
  };
  using O = T;
  auto store = [&](int m, int n, float v) {
    const long long idx = batch * g.bsd + static_cast<long long>(m) * g.ldd + n;
    v *= g.alpha;
    if (g.out_f32) {
      if (g.use_c) v += g.beta * static_cast<const float*>(g.c)[idx];
      if (g.has_bias) v += static_cast<const float*>(g.bias)[n];
      if (g.has_aux) static_cast<float*>(g.aux)[idx] = v;
      static_cast<float*>(g.d)[idx] = act_f32(g.act, v);
    } else {
      if (g.use_c) v += g.beta * to_f32(static_cast<const O*>(g.c)[idx]);
      if (g.has_bias) v += to_f32(static_cast<const O*>(g.bias)[n]);
      if (g.has_aux) static_cast<O*>(g.aux)[idx] = from_f32<O>(v);
      static_cast<O*>(g.d)[idx] = from_f32<O>(act_f32(g.act, v));
    }
  };

  u32x4 w[D][CPL];
  int n0 = gw;
  if (n0 < g.n) load(n0, w);
  for (; n0 < g.n; n0 += D * GW) {
    float acc[NV4];
#pragma unroll
    for (int v = 0; v < NV4; ++v) acc[v] = 0.f;
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int j = 0; j < CPL; ++j)
          acc[d * M + m] = Dot8<T>(w[d][j], xr[m][j], acc[d * M + m]);
    // The next round's rows are in flight while this one is reduced.
    const int nn = n0 + D * GW;
    if (nn < g.n) load(nn, w);
#pragma unroll
    for (int q = 0; q < NV4; q += 4) {
      const float v = wave_sum4(acc[q], acc[q + 1], acc[q + 2], acc[q + 3],
                                lane);
      const int vi = q + (lane & 3);
      const int d = vi / M, m = vi % M;
      const int n = n0 + d * GW;
      if (lane < 4 && vi < NV && n < g.n) store(m, n, v);
    }
  }
}

template <typename T, int M>
void LaunchM(const GemmArgs& g, int batch, int cpl, int grid,
             hipStream_t st) {
  const dim3 gr(grid, batch);
  switch (cpl) {
    case 1:
      gemv_nt_kernel<T, M, 1><<<gr, kGemvThreads, 0, st>>>(g);
      break;
    case 2:
      gemv_nt_kernel<T, M, 2><<<gr, kGemvThreads, 0, st>>>(g);
      break;
    default:
      gemv_nt_kernel<T, M, 4><<<gr, kGemvThreads, 0, st>>>(g);
      break;
  }
}

template <typename T>
void LaunchT(const GemmArgs& g, int batch, int cpl, int grid, hipStream_t st) {
  switch (g.m) {
    case 1: return LaunchM<T, 1>(g, batch, cpl, grid, st);
    case 2: return LaunchM<T, 2>(g, batch, cpl, grid, st);
    case 3: return LaunchM<T, 3>(g, batch, cpl, grid, st);
    case 4: return LaunchM<T, 4>(g, batch, cpl, grid, st);
    case 5: return LaunchM<T, 5>(g, batch, cpl, grid, st);
    case 6: return LaunchM<T, 6>(g, batch, cpl, grid, st);
    case 7: return LaunchM<T, 7>(g, batch, cpl, grid, st);
    default: return LaunchM<T, 8>(g, batch, cpl, grid, st);
  }
}

}  // namespace

bool GemvApplies(const GemmProblem& p) {
  if (p.a.dtype != QK_BF16 && p.a.dtype != QK_F16) return false;
  if (p.m < 1 || p.m > 8 || p.a.transpose || !p.b.transpose) return false;
  const int64_t cpl = p.k / 512;
  if (p.k % 512 != 0 || (cpl != 1 && cpl != 2 && cpl != 4)) return false;
  // x rows stay in registers: M x K / 512 chunks of 16 bytes per lane.
  if (p.m * cpl > 16) return false;
  const bool batched = p.batch > 1;
  auto aligned = [&](const Operand& o) {
    const int64_t bs = batched ? o.batch_stride : 0;
    return reinterpret_cast<uintptr_t>(o.ptr) % 16 == 0 && o.ld % 8 == 0 &&
           bs % 8 == 0;
  };
  if (!aligned(p.a) || !aligned(p.b)) return false;
  // Weight rows of one batch entry addressed by a 32-bit buffer offset.
  return (p.n - 1) * p.b.ld * 2 + p.k * 2 < (int64_t{1} << 31) &&
         p.n <= (int64_t{1} << 30);
}

qk_status LaunchGemv(const GemmProblem& p, hipStream_t stream) {
  GemmArgs g{};
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
  const int batch = static_cast<int>(p.batch);
  const int cpl = g.k / 512;
  // Rounds of kGemvRows rows per wave; at most 8 waves per SIMD of them.
  const int cus = DeviceComputeUnits();
  const long long waves = (g.n + kGemvRows - 1) / kGemvRows;
  const int grid = static_cast<int>(std::max<long long>(
      1, std::min<long long>((waves + 3) / 4, static_cast<long long>(cus) * 8)));
  if (p.a.dtype == QK_BF16)
    LaunchT<bf16>(g, batch, cpl, grid, stream);
  else
    LaunchT<f16>(g, batch, cpl, grid, stream);
  return PostLaunch("gemv_nt");
}

}  // namespace qk
