// Tile shapes of the register-dequantizing quantized GEMM (qgemm_dma.h)
// and their launch, shared by the per-packing translation units
// (qgemm_dma_u4.hip, qgemm_dma_u8.hip, qgemm_dma_s8.hip) and the chooser
// (qgemm_dma.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstring>
#include <type_traits>

#include "qk_internal.h"

namespace qk {

// Tile shapes: BM x BN, waves WM x (BN / (32 FN)).
struct QDmaCfg {
  int bm, bn, wm, fn;
};
constexpr QDmaCfg kQDmaCfgs[] = {
    {256, 128, 1, 1}, {128, 256, 1, 1}, {128, 128, 2, 1}};
constexpr int kQDmaNumCfgs = sizeof(kQDmaCfgs) / sizeof(kQDmaCfgs[0]);

// A stages: the most (up to kQDmaMaxStages) that fit the LDS with the
// code and scale blocks; 0 when not even three fit (the layout of QDma).
constexpr int kQDmaMaxStages = 4;
template <int PACK, int BM, int BN, int WM, int FN>
constexpr int QDmaStages() {
  constexpr int crow = (PACK == QK_PACK_U32X8 ? 32 : 64) * 2;
  constexpr int nw = WM * BN / (32 * FN);
  constexpr int pad = (BM / 8) % nw != 0 ? 1024 : 0;
  int best = 0;
  for (int s = 3; s <= kQDmaMaxStages; ++s)
    if (s * BM * 128 + (s / 2 + 1) * BN * crow + 4 * BN * 16 + pad <=
        160 * 1024)
      best = s;
  return best;
}

template <int PACK, int I>
constexpr int QDmaCfgStages() {
  return QDmaStages<PACK, kQDmaCfgs[I].bm, kQDmaCfgs[I].bn, kQDmaCfgs[I].wm,
                    kQDmaCfgs[I].fn>();
}

inline bool QDmaFits(int packing, int i) {
  auto fits = [&](auto pk) {
    constexpr int P = decltype(pk)::value;
    switch (i) {
      case 0: return QDmaCfgStages<P, 0>() != 0;
      case 1: return QDmaCfgStages<P, 1>() != 0;
      default: return QDmaCfgStages<P, 2>() != 0;
    }
  };
  switch (packing) {
    case QK_PACK_U32X8:
      return fits(std::integral_constant<int, QK_PACK_U32X8>{});
    case QK_PACK_U8:
      return fits(std::integral_constant<int, QK_PACK_U8>{});
    default:
      return fits(std::integral_constant<int, QK_PACK_S8_SYM>{});
  }
}

// One launch of shape `cfg` for codes of one packing; `args` is the
// kernel's argument block (a GemmArgs, copied by bytes: each translation
// unit has its own copy of that type).
void QDmaLaunchU4(int cfg, const void* args, size_t size, int grid, bool mc,
                  bool half, hipStream_t st);
void QDmaLaunchU8(int cfg, const void* args, size_t size, int grid, bool mc,
                  bool half, hipStream_t st);
void QDmaLaunchS8(int cfg, const void* args, size_t size, int grid, bool mc,
                  bool half, hipStream_t st);

}  // namespace qk

// Defines QDmaLaunch<NAME> for packing PACK (in a translation unit that
// includes gemm_common.h and qgemm_dma.h). 128-row tiles are always
// launched with the row check (a check per stored value; M below 128 is
// their usual case).
#define QK_DEFINE_QDMA_LAUNCH(NAME, PACK)                                     \
  namespace qk {                                                             \
  namespace {                                                                \
  template <typename T, int I>                                               \
  void LaunchQDmaCfg(const GemmArgs& g, int grid, bool mc, hipStream_t st) { \
    constexpr QDmaCfg c = kQDmaCfgs[I];                                      \
    constexpr int S = QDmaCfgStages<PACK, I>();                              \
    if constexpr (S != 0) {                                                  \
      constexpr int NT = c.wm * (c.bn / (32 * c.fn)) * 64;                   \
      if (mc || c.bm != 256)                                                 \
        qgemm_dma_kernel<T, PACK, c.bm, c.bn, c.wm, c.fn, S, true>           \
            <<<grid, NT, 0, st>>>(g);                                        \
      else if constexpr (c.bm == 256)                                        \
        qgemm_dma_kernel<T, PACK, c.bm, c.bn, c.wm, c.fn, S, false>          \
            <<<grid, NT, 0, st>>>(g);                                        \
    }                                                                        \
  }                                                                          \
  template <typename T>                                                      \
  void LaunchQDmaT(int cfg, const GemmArgs& g, int grid, bool mc,            \
                   hipStream_t st) {                                         \
    switch (cfg) {                                                           \
      case 0: return LaunchQDmaCfg<T, 0>(g, grid, mc, st);                   \
      case 1: return LaunchQDmaCfg<T, 1>(g, grid, mc, st);                   \
      default: return LaunchQDmaCfg<T, 2>(g, grid, mc, st);                  \
    }                                                                        \
  }                                                                          \
  }                                                                          \
  void NAME(int cfg, const void* args, size_t size, int grid, bool mc,      \
            bool half, hipStream_t st) {                                     \
    GemmArgs g;                                                              \
    static_assert(std::is_trivially_copyable<GemmArgs>::value, "args");     \
    if (size != sizeof(g)) return;                                           \
    std::memcpy(&g, args, sizeof(g));                                        \
    if (half)                                                                \
      LaunchQDmaT<f16>(cfg, g, grid, mc, st);                                \
    else                                                                     \
      LaunchQDmaT<bf16>(cfg, g, grid, mc, st);                               \
  }                                                                          \
  }
