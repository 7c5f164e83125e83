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
#include "qgemm_dma_launch.h"
#include "qk_device.h"
#include "qk_internal.h"

namespace qk {

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
  // QK_QGEMM_DMA=<shape>,<split> forces a shape of kQDmaCfgs and a K
  // split where both apply (tuning and tests; read at every call);
  // QK_QGEMM_DMA_GROUP=<M tiles> the tile group of the workgroup order.
  std::pair<int, int> forced{-1, 0};
  if (const char* v = std::getenv("QK_QGEMM_DMA")) {
    if (std::sscanf(v, "%d,%d", &forced.first, &forced.second) != 2)
      forced.first = -1;
  }
  const long long max_flags = static_cast<long long>(kWsFlagBytes / 4);
  auto tiles_of = [&](int i) {
    return static_cast<long long>((g.m + kQDmaCfgs[i].bm - 1) /
                                  kQDmaCfgs[i].bm) *
           (g.n / kQDmaCfgs[i].bn);
  };
  auto valid = [&](int i, int split) {
    const QDmaCfg& c = kQDmaCfgs[i];
    return i >= 0 && i < kQDmaNumCfgs && QDmaFits(p.packing, i) &&
           g.n % c.bn == 0 && split >= 1 && G % split == 0 &&
           G / split >= 8 && (G / split) % 8 == 0 &&
           (split == 1 || tiles_of(i) <= max_flags);
  };
  // Choice (a sweep on MI355X of every shape and split, int4 and int8,
  // N 4096..151936, K 4096 / 12288, M 33..2048): the kernel's throughput
  // per CU is about the same for every shape at a given number of busy
  // CUs (and falls as more are busy: ~0.95 PFLOP/s with all of them), so
  // what counts is how many CUs work and how little is redone. 128 x 256
  // tiles when there are at least 5/8 as many as CUs (512 x 12288 x 4096:
  // 64 us against 70 for 256 x 128); else 256 x 128 when those fill 5/8
  // (4096 columns); else 128 x 128 (two wave rows) with the largest K
  // split that keeps one workgroup per CU (each partial beyond the first
  // costs the last workgroup a memory round trip): 128 x 12288 x 4096 split
  // 2 (31 us), 128 x 4096 x 4096 split 4 (24 us), 512 x 4096 x 12288
  // split 2 (72 us). 256-row tiles only for more than 128 rows: at M <= 128
  // half their rows are padding (128 x 151936 x 4096, where N is not a
  // multiple of 256: 337 us with 256 x 128 tiles, 273 with 128 x 128;
  // 128 x 32768 x 4096: 82 against 63).
  const long long fill = static_cast<long long>(cus) * 5;
  int best_i = -1, best_split = 1;
  if (valid(1, 1) && tiles_of(1) * 8 >= fill) {
    best_i = 1;
  } else if (valid(0, 1) && g.m > 128 && tiles_of(0) * 8 >= fill) {
    best_i = 0;
  } else if (valid(2, 1)) {
    best_i = 2;
    for (int split = 2; split <= 8; split *= 2)
      if (valid(2, split) && tiles_of(2) * split <= cus) best_split = split;
  } else {
    for (int i = 0; i < kQDmaNumCfgs && best_i < 0; ++i)
      if (valid(i, 1)) best_i = i;
  }
  if (valid(forced.first, forced.second))
    best_i = forced.first, best_split = forced.second;
  if (best_i < 0) return Fail(QK_INTERNAL, "qkern: no quantized GEMM tile");
  const QDmaCfg& c = kQDmaCfgs[best_i];
  g.tiles_m = (g.m + c.bm - 1) / c.bm;
  g.tiles_n = g.n / c.bn;
  const long long tiles = static_cast<long long>(g.tiles_m) * g.tiles_n;
  if (best_split > 1) {
    const size_t bytes = static_cast<size_t>(tiles) * best_split * c.bm *
                         c.bn * sizeof(float);
    if (bytes >= (size_t{1} << 31) ||
        !StreamWorkspace(stream, bytes, &g.ws, &g.wsflag)) {
      best_split = 1;  // no workspace: one workgroup per tile
    }
  }
  g.ksplit = best_split;
  if (const char* v = std::getenv("QK_QGEMM_DMA_GROUP")) {
    g.group_m = std::atoi(v);
  }
  const long long grid = tiles * best_split;
  if (std::getenv("QK_QGEMM_DMA_TRACE") != nullptr)
    std::fprintf(stderr, "qgemm_dma m=%d n=%d k=%d shape=%d split=%d\n",
                 g.m, g.n, g.k, best_i, best_split);
  if (grid > 0x7FFFFFFF) {
    return Fail(QK_UNIMPLEMENTED, "qkern: quantized matmul too large");
  }
  const bool mc = g.m % c.bm != 0;
  const bool h = p.x_dtype == QK_F16;
  switch (p.packing) {
    case QK_PACK_U32X8:
      QDmaLaunchU4(best_i, &g, sizeof(g), static_cast<int>(grid), mc, h,
                   stream);
      break;
    case QK_PACK_U8:
      QDmaLaunchU8(best_i, &g, sizeof(g), static_cast<int>(grid), mc, h,
                   stream);
      break;
    default:
      QDmaLaunchS8(best_i, &g, sizeof(g), static_cast<int>(grid), mc, h,
                   stream);
      break;
  }
  return PostLaunch("qgemm_dma");
}

}  // namespace qk
