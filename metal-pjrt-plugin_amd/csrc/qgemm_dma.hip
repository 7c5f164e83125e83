// Launcher of the register-dequantizing quantized GEMM (qgemm_dma.h): int4
// u32x8, u8 affine and s8 symmetric codes, group 64, bf16 scales and
// offsets, bf16/f16 x; the tile shape and the K split are chosen per
// problem so that the grid fills the CUs.
//
// Serves the reference's dequantize-then-multiply path of linear() for
// rows beyond ROWS_MAX (examples/llm/qwen3.py:218-230) from 33 rows up.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstdio>

#include "gemm_common.h"
#include "qgemm_dma.h"
#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

// Tile shapes: BM x BN, waves WM x (BN / (32 FN)).
struct DmaCfg {
  int bm, bn, wm, fn;
};
constexpr DmaCfg kCfgs[] = {
    {256, 256, 1, 1}, {256, 128, 1, 1}, {256, 192, 1, 1}, {128, 256, 1, 1},
    {128, 128, 1, 1}, {128, 192, 1, 1}, {128, 256, 2, 2}, {128, 128, 2, 1}};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

// A stages: four when they fit the LDS with the code and scale blocks,
// else three; 0 when not even three fit (the layout of QDma).
template <int PACK, int BM, int BN, int WM, int FN>
constexpr int PickStages() {
  constexpr int crow = (PACK == QK_PACK_U32X8 ? 32 : 64) * 2;
  constexpr int nw = WM * BN / (32 * FN);
  constexpr int pad = (BM / 8) % nw != 0 ? 1024 : 0;
  constexpr int b4 = 4 * BM * 128 + 3 * BN * crow + 4 * BN * 16 + pad;
  constexpr int b3 = 3 * BM * 128 + 2 * BN * crow + 4 * BN * 16 + pad;
  return b4 <= 160 * 1024 ? 4 : b3 <= 160 * 1024 ? 3 : 0;
}

template <int PACK, int I>
constexpr int CfgStages() {
  return PickStages<PACK, kCfgs[I].bm, kCfgs[I].bn, kCfgs[I].wm,
                    kCfgs[I].fn>();
}

template <typename T, int PACK, int I>
void LaunchCfg(const GemmArgs& g, int grid, bool mc, hipStream_t st) {
  constexpr DmaCfg c = kCfgs[I];
  constexpr int S = CfgStages<PACK, I>();
  if constexpr (S != 0) {
    constexpr int NT = c.wm * (c.bn / (32 * c.fn)) * 64;
    if (mc)
      qgemm_dma_kernel<T, PACK, c.bm, c.bn, c.wm, c.fn, S, true>
          <<<grid, NT, 0, st>>>(g);
    else
      qgemm_dma_kernel<T, PACK, c.bm, c.bn, c.wm, c.fn, S, false>
          <<<grid, NT, 0, st>>>(g);
  }
}

template <typename T, int PACK>
void LaunchAny(int i, const GemmArgs& g, int grid, bool mc, hipStream_t st) {
  switch (i) {
    case 0: return LaunchCfg<T, PACK, 0>(g, grid, mc, st);
    case 1: return LaunchCfg<T, PACK, 1>(g, grid, mc, st);
    case 2: return LaunchCfg<T, PACK, 2>(g, grid, mc, st);
    case 3: return LaunchCfg<T, PACK, 3>(g, grid, mc, st);
    case 4: return LaunchCfg<T, PACK, 4>(g, grid, mc, st);
    case 5: return LaunchCfg<T, PACK, 5>(g, grid, mc, st);
    case 6: return LaunchCfg<T, PACK, 6>(g, grid, mc, st);
    default: return LaunchCfg<T, PACK, 7>(g, grid, mc, st);
  }
}

template <int PACK>
bool Fits(int i) {
  switch (i) {
    case 0: return CfgStages<PACK, 0>() != 0;
    case 1: return CfgStages<PACK, 1>() != 0;
    case 2: return CfgStages<PACK, 2>() != 0;
    case 3: return CfgStages<PACK, 3>() != 0;
    case 4: return CfgStages<PACK, 4>() != 0;
    case 5: return CfgStages<PACK, 5>() != 0;
    case 6: return CfgStages<PACK, 6>() != 0;
    default: return CfgStages<PACK, 7>() != 0;
  }
}

bool FitsPacking(int packing, int i) {
  switch (packing) {
    case QK_PACK_U32X8: return Fits<QK_PACK_U32X8>(i);
    case QK_PACK_U8: return Fits<QK_PACK_U8>(i);
    default: return Fits<QK_PACK_S8_SYM>(i);
  }
}

}  // namespace

bool QGemmDmaApplies(const QuantProblem& p) {
  if (p.packing != QK_PACK_U32X8 && p.packing != QK_PACK_U8 &&
      p.packing != QK_PACK_S8_SYM)
    return false;
  if (p.x_dtype != QK_BF16 && p.x_dtype != QK_F16) return false;
  if (p.m <= 0 || p.k <= 0 || p.k % 512 != 0 || p.group != 64 ||
      p.scale_dtype != QK_BF16 || (p.has_bias && p.bias_dtype != QK_BF16) ||
      p.n % 128 != 0)
    return false;
  const int64_t row_bytes = p.bits == 4 ? p.k / 2 : p.k;
  if (p.n * row_bytes >= (int64_t{1} << 31) ||
      p.n * (p.k / 64) * 2 >= (int64_t{1} << 31) ||
      (p.m + 256) * p.k * 2 >= (int64_t{1} << 31))
    return false;
  auto al = [](const void* q) {
    return reinterpret_cast<uintptr_t>(q) % 16 == 0;
  };
  return al(p.x) && al(p.codes) && al(p.scales) &&
         (!p.has_bias || al(p.biases));
}

qk_status LaunchQGemmDma(const QuantProblem& p, hipStream_t stream) {
  GemmArgs g{};
  g.a = p.x;
  g.b = p.codes;
  g.d = p.y;
  g.m = static_cast<int>(p.m);
  g.n = static_cast<int>(p.n);
  g.k = static_cast<int>(p.k);
  g.lda = g.k;
  g.ldd = g.n;
  g.alpha = 1.f;
  g.out_vec = 1;
  g.a_vec = g.b_vec = 1;
  g.qscale = p.scales;
  g.qbias = p.biases;
  g.qsdt = p.scale_dtype;
  g.qbdt = p.bias_dtype;
  g.qhas_bias = p.has_bias ? 1 : 0;
  g.qgroup = p.group;
  g.qrow_bytes = static_cast<int>(p.bits == 4 ? p.k / 2 : p.k);
  g.ksplit = 1;

  const int cus = DeviceComputeUnits();
  const int G = g.k / 64;
  // QK_QGEMM_DMA=<shape>,<split> forces a shape of kCfgs and a K split
  // where both apply (tuning and tests; read at every call).
  std::pair<int, int> forced{-1, 0};
  if (const char* v = std::getenv("QK_QGEMM_DMA")) {
    if (std::sscanf(v, "%d,%d", &forced.first, &forced.second) != 2)
      forced.first = -1;
  }
  // Choice (measured on MI355X, int4 and int8, N 4096..151936, K 4096 and
  // 12288, M 33..512): a K tile costs a workgroup about the same time
  // whatever the tile's size (the LDS-DMA pipeline is latency-bound), so
  // the larger tile wins whenever it fills the CUs: 256 x 128 when there
  // are at least 5/8 as many such tiles as CUs; otherwise 128 x 128 (two
  // wave rows) with the largest K split that keeps one workgroup per CU
  // (each split beyond the first costs one memory round trip in the tail).
  // E.g. 12288 x 4096: M = 512 256 x 128 (65 us), M = 128 128 x 128
  // split 2 (32 us); 4096 x 4096: M = 512 128 x 128 split 2 (32 us),
  // M = 128 split 8 (24 us).
  auto valid = [&](int i, int split) {
    const DmaCfg& c = kCfgs[i];
    return FitsPacking(p.packing, i) && g.n % c.bn == 0 && G % split == 0 &&
           G / split >= 8 && (G / split) % 8 == 0;
  };
  auto tiles_of = [&](int i) {
    return static_cast<long long>((g.m + kCfgs[i].bm - 1) / kCfgs[i].bm) *
           (g.n / kCfgs[i].bn);
  };
  int best_i = -1, best_split = 1;
  if (valid(1, 1) && tiles_of(1) * 8 >= static_cast<long long>(cus) * 5) {
    best_i = 1;
  } else if (valid(7, 1)) {
    best_i = 7;
    for (int split = 2; split <= 8; split *= 2)
      if (valid(7, split) && tiles_of(7) * split <= cus &&
          tiles_of(7) <= static_cast<long long>(kWsFlagBytes / 4))
        best_split = split;
  } else {
    for (int i = 0; i < kNumCfgs && best_i < 0; ++i)
      if (valid(i, 1)) best_i = i;
  }
  if (forced.first >= 0 && forced.first < kNumCfgs && forced.second >= 1 &&
      valid(forced.first, forced.second) &&
      (forced.second == 1 ||
       tiles_of(forced.first) <= static_cast<long long>(kWsFlagBytes / 4)))
    best_i = forced.first, best_split = forced.second;
  if (best_i < 0) return Fail(QK_INTERNAL, "qkern: no quantized GEMM tile");
  const DmaCfg& c = kCfgs[best_i];
  g.tiles_m = (g.m + c.bm - 1) / c.bm;
  g.tiles_n = g.n / c.bn;
  if (best_split > 1) {
    const size_t bytes = static_cast<size_t>(g.tiles_m) * g.tiles_n *
                         best_split * c.bm * c.bn * sizeof(float);
    if (bytes >= (size_t{1} << 31) ||
        !StreamWorkspace(stream, bytes, &g.ws, &g.wsflag)) {
      best_split = 1;  // no workspace: one K range per tile
    }
  }
  g.ksplit = best_split;
  if (std::getenv("QK_QGEMM_DMA_TRACE") != nullptr)
    std::fprintf(stderr, "qgemm_dma m=%d n=%d k=%d shape=%d split=%d\n", g.m,
                 g.n, g.k, best_i, best_split);
  const int grid = g.tiles_m * g.tiles_n * best_split;
  const bool mc = g.m % c.bm != 0;
  const bool h = p.x_dtype == QK_F16;
  switch (p.packing) {
    case QK_PACK_U32X8:
      if (h) LaunchAny<f16, QK_PACK_U32X8>(best_i, g, grid, mc, stream);
      else LaunchAny<bf16, QK_PACK_U32X8>(best_i, g, grid, mc, stream);
      break;
    case QK_PACK_U8:
      if (h) LaunchAny<f16, QK_PACK_U8>(best_i, g, grid, mc, stream);
      else LaunchAny<bf16, QK_PACK_U8>(best_i, g, grid, mc, stream);
      break;
    default:
      if (h) LaunchAny<f16, QK_PACK_S8_SYM>(best_i, g, grid, mc, stream);
      else LaunchAny<bf16, QK_PACK_S8_SYM>(best_i, g, grid, mc, stream);
      break;
  }
  return PostLaunch("qgemm_dma");
}

}  // namespace qk
