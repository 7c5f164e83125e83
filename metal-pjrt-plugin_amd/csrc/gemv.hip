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
#include <cstdlib>
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

// The BlasLt epilogue of one output (m, n) of batch entry `batch`, in f32
// with one rounding: v = alpha acc (+ beta C) (+ bias[n]); aux = v;
// D = act(v).
template <typename T>
__device__ __forceinline__ void GemvStore(const GemmArgs& g, long long batch,
                                          int m, int n, float v) {
  const long long idx = batch * g.bsd + static_cast<long long>(m) * g.ldd + n;
  v *= g.alpha;
  if (g.out_f32) {
    if (g.use_c) v += g.beta * static_cast<const float*>(g.c)[idx];
    if (g.has_bias) v += static_cast<const float*>(g.bias)[n];
    if (g.has_aux) static_cast<float*>(g.aux)[idx] = v;
    static_cast<float*>(g.d)[idx] = act_f32(g.act, v);
  } else {
    if (g.use_c) v += g.beta * to_f32(static_cast<const T*>(g.c)[idx]);
    if (g.has_bias) v += to_f32(static_cast<const T*>(g.bias)[n]);
    if (g.has_aux) static_cast<T*>(g.aux)[idx] = from_f32<T>(v);
    static_cast<T*>(g.d)[idx] = from_f32<T>(act_f32(g.act, v));
  }
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
      if (lane < 4 && vi < NV && n < g.n) GemvStore<T>(g, batch, m, n, v);
    }
  }
}

// NN layout (W stored [K][N], N contiguous), M <= 4 rows of x, K a
// multiple of 512: one workgroup of sixteen waves per 64 output columns
// walks all of K. Lane l holds columns 8 (l % 8) .. + 7 of the
// workgroup's 64 and K rows 4 (l / 8) .. + 3 of its wave's 32-row window
// (the window of wave w in step i: rows 512 i + 32 w ..): per step a lane
// loads four 16-byte pieces of W (each wave-wide load: 8 rows x 128
// contiguous bytes) and, per row of x, the four matching x values (8
// bytes), and accumulates M x 8 column sums in f32 (W and x converted
// exactly, products by FMA; more rows of x exceed the registers of a
// 1024-thread workgroup). The next step's loads are in flight while
// one step is computed. The sixteen row groups of a wave are summed by
// lane shuffles, the eight waves through LDS, and the epilogue is applied
// per output as in the NT gemv.
// LPR lanes per W row piece (8: 128 bytes, 64 columns per workgroup; 4
// lanes, 64-byte pieces, measured at half the bandwidth), NW waves per
// workgroup; a step covers NW * 256 / LPR rows (512 as used).
template <typename T, int M, int LPR = 8, int NW = 16>
__global__ __launch_bounds__(NW * 64) void gemv_nn_kernel(GemmArgs g) {
  constexpr int CW = 8 * LPR;         // columns per workgroup
  constexpr int RW = 4 * (64 / LPR);  // rows per wave per step
  constexpr int RS = NW * RW;         // rows per step
  __shared__ float part[NW][M][CW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane % LPR, r = lane / LPR;
  const int n0 = blockIdx.x * CW;
  const long long batch = blockIdx.y;
  const T* A = static_cast<const T*>(g.a) + batch * g.bsa;
  const T* B = static_cast<const T*>(g.b) + batch * g.bsb;
  // W of one batch entry as a buffer (extent: up to the last row's N
  // values, so columns past N read zeros without a branch).
  const long long wbytes = (static_cast<long long>(g.k - 1) * g.ldb + g.n) *
                           static_cast<long long>(sizeof(T));
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(B), (short)0,
      static_cast<int>(std::min<long long>(wbytes, 0x7FFFFFFFll)), 0x00020000);
  // Columns past N (the last workgroup's tail, whole 16-byte pieces as N
  // is a multiple of 8) read the next row's values, or zeros past the
  // extent; their sums are not stored.
  const int coff = (n0 + 8 * c) * static_cast<int>(sizeof(T));
  const int rstride = g.ldb * static_cast<int>(sizeof(T));
  const int steps = g.k / RS;

  u32x4 w[2][4];
  uint32_t xv[2][M][2];
  auto load = [&](int i, int b) {
    const int k0 = RS * i + RW * wave + 4 * r;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      w[b][u] = __builtin_amdgcn_raw_buffer_load_b128(
          wrs, coff + (k0 + u) * rstride, 0, 2);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint2 v = *reinterpret_cast<const uint2*>(
          A + static_cast<long long>(m) * g.lda + k0);
      xv[b][m][0] = v.x, xv[b][m][1] = v.y;
    }
  };
  float acc[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m][e] = 0.f;
  auto lo16 = [](uint32_t v) { return to_f32(__builtin_bit_cast(T, static_cast<uint16_t>(v & 0xFFFFu))); };
  auto hi16 = [](uint32_t v) { return to_f32(__builtin_bit_cast(T, static_cast<uint16_t>(v >> 16))); };
  auto compute = [&](int b) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float wf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        wf[2 * e] = lo16(w[b][u][e]);
        wf[2 * e + 1] = hi16(w[b][u][e]);
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint32_t xp = xv[b][m][u >> 1];
        const float xs = (u & 1) ? hi16(xp) : lo16(xp);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = fmaf(xs, wf[e], acc[m][e]);
      }
    }
  };
  load(0, 0);
  for (int i = 0; i < steps; i += 2) {
    if (i + 1 < steps) load(i + 1, 1);
    compute(0);
    if (i + 1 >= steps) break;
    if (i + 2 < steps) load(i + 2, 0);
    compute(1);
  }
  // Sum over the 16 row groups of the wave (lane bits 2..5).
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[m][e];
#pragma unroll
      for (int o = LPR; o < 64; o <<= 1) v += __shfl_xor(v, o);
      acc[m][e] = v;
    }
  if (r == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e) part[wave][m][8 * c + e] = acc[m][e];
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < CW * M) {
    const int m = t / CW, j = t % CW;
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < NW; ++q) v += part[q][m][j];
    const int n = n0 + j;
    if (n < g.n) GemvStore<T>(g, batch, m, n, v);
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

bool GemvNNApplies(const GemmProblem& p) {
  if (p.a.dtype != QK_BF16 && p.a.dtype != QK_F16) return false;
  if (p.m < 1 || p.m > 4 || p.a.transpose || p.b.transpose) return false;
  if (p.k % 512 != 0 || p.k == 0 || p.n % 8 != 0 || p.n == 0) return false;
  const bool batched = p.batch > 1;
  // x: 8-byte runs of four values; W: 16-byte runs of eight.
  const int64_t bsa = batched ? p.a.batch_stride : 0;
  const int64_t bsb = batched ? p.b.batch_stride : 0;
  if (reinterpret_cast<uintptr_t>(p.a.ptr) % 8 != 0 || p.a.ld % 4 != 0 ||
      bsa % 4 != 0)
    return false;
  if (reinterpret_cast<uintptr_t>(p.b.ptr) % 16 != 0 || p.b.ld % 8 != 0 ||
      bsb % 8 != 0)
    return false;
  // W of one batch entry addressed by a 32-bit buffer offset.
  return ((p.k - 1) * p.b.ld + p.n + 64) * 2 < (int64_t{1} << 31) &&
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
  if (!p.b.transpose) {
    const dim3 gr(static_cast<unsigned>((g.n + 63) / 64), batch);
    auto go = [&](auto tag) {
      using T = decltype(tag);
      switch (g.m) {
        case 1: gemv_nn_kernel<T, 1><<<gr, 1024, 0, stream>>>(g); break;
        case 2: gemv_nn_kernel<T, 2><<<gr, 1024, 0, stream>>>(g); break;
        case 3: gemv_nn_kernel<T, 3><<<gr, 1024, 0, stream>>>(g); break;
        default: gemv_nn_kernel<T, 4><<<gr, 1024, 0, stream>>>(g); break;
      }
    };
    if (p.a.dtype == QK_BF16)
      go(bf16{});
    else
      go(f16{});
    return PostLaunch("gemv_nn");
  }
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
