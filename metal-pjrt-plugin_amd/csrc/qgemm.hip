// Quantized matmul for more than a few rows of x: y = x @ w^T with w
// dequantized tile by tile inside an MFMA GEMM.
//
// Replaces the reference's path for rows beyond ROWS_MAX (4) in linear()
// (examples/llm/qwen3.py:218-230): w = dequantize(w, x.dtype)
// (qwen3.py:199-207), then einsum("...i,oi->...o", x, w). Here the
// dequantized weights never reach HBM: the GEMM's B-tile loader reads
// 16-byte chunks of codes with their group's scale and offset, forms
// bf16/f16(f32(q)*f32(s) + f32(b)) (the canonical rounding of
// qk$dequantize, unfused) and writes K-contiguous rows into LDS, from
// where the tiled MFMA kernel of gemm_common.h consumes them. Each weight
// byte is read once per M tile.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>

#include "gemm_common.h"
#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

// B tile loader over quantized codes [N][row_bytes]; LDS layout
// [BN][BK + 8], K-contiguous, in the activation type T.
template <int PACK, typename T, int BN, int BK, int NT>
struct QuantB {
  static constexpr bool kKCont = true;
  static constexpr bool kInt4 =
      PACK == QK_PACK_U32X8 || PACK == QK_PACK_BYTE_HALFSPLIT;
  static constexpr int kCodes = kInt4 ? 32 : 16;  // codes per 16 bytes
  static constexpr int CPT = BK / kCodes;         // chunks per tile row
  static constexpr int TOTAL = BN * CPT;
  static constexpr int NC = (TOTAL + NT - 1) / NT;
  static constexpr int LD = BK + 8;

  const uint8_t* codes;
  const void* scales;
  const void* biases;
  int sdt, bdt, has_bias, group, row_bytes, n0, n, tid;
  u32x4 w[NC];
  float s[NC], b[NC];
  int k0_;

  __device__ __forceinline__ QuantB(const GemmArgs& g, long long /*batch*/,
                                    int n0_, int tid_)
      : codes(static_cast<const uint8_t*>(g.b)),
        scales(g.qscale),
        biases(g.qbias),
        sdt(g.qsdt),
        bdt(g.qbdt),
        has_bias(g.qhas_bias),
        group(g.qgroup),
        row_bytes(g.qrow_bytes),
        n0(n0_),
        n(g.n),
        tid(tid_),
        k0_(0) {}

  // Chunk c of a row: first element kb (half-split: also kb + group/2).
  __device__ __forceinline__ void span(int c, int* kb, int* grp) const {
    if (PACK == QK_PACK_BYTE_HALFSPLIT) {
      const int hg = group / 2;
      *grp = (c * 16) / hg;
      *kb = *grp * group + (c * 16) % hg;
    } else {
      *kb = c * kCodes;
      *grp = *kb / group;
    }
  }

  __device__ __forceinline__ void load(int k0) {
    k0_ = k0;
    const int groups = (row_bytes / 16) * kCodes / group;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int id = tid + i * NT;
      w[i] = u32x4{0, 0, 0, 0};
      s[i] = 0.f;
      b[i] = 0.f;
      if (id >= TOTAL) continue;
      const int row = n0 + id / CPT;
      // chunk index within the row: the tile's chunks are the CPT chunks
      // whose first element lies in [k0, k0 + BK)
      const int c = k0 / kCodes +
                    id % CPT;
      if (row >= n || c * 16 >= row_bytes) continue;
      w[i] = *reinterpret_cast<const u32x4*>(
          codes + static_cast<long long>(row) * row_bytes + c * 16);
      int kb, grp;
      span(c, &kb, &grp);
      const long long gi = static_cast<long long>(row) * groups + grp;
      s[i] = load_any(scales, gi, sdt);
      b[i] = has_bias ? load_any(biases, gi, bdt) : 0.f;
    }
  }

  __device__ __forceinline__ void store(T* lds) const {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int id = tid + i * NT;
      if (id >= TOTAL) continue;
      const int r = id / CPT;
      const int c = k0_ / kCodes + id % CPT;
      int kb, grp;
      span(c, &kb, &grp);
      T* dst = lds + r * LD + (kb - k0_);
      auto dq = [&](float q) {
        return from_f32<T>(__fadd_rn(__fmul_rn(q, s[i]), b[i]));
      };
      union Pack8 {
        u32x4 u;
        T e[8];
      };
      if constexpr (PACK == QK_PACK_U32X8) {
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
          Pack8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            o.e[e] = dq(static_cast<float>((w[i][wd] >> (4 * e)) & 15u));
          *reinterpret_cast<u32x4*>(dst + 8 * wd) = o.u;
        }
      } else if constexpr (PACK == QK_PACK_BYTE_HALFSPLIT) {
        const int hg = group / 2;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
          for (int v = 0; v < 2; ++v) {
            Pack8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int byte = 8 * v + e;
              const uint32_t bits = (w[i][byte >> 2] >> (8 * (byte & 3))) >>
                                    (4 * half);
              o.e[e] = dq(static_cast<float>(bits & 15u));
            }
            *reinterpret_cast<u32x4*>(dst + half * hg + 8 * v) = o.u;
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          Pack8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int byte = 8 * v + e;
            const uint32_t word = w[i][byte >> 2] >> (8 * (byte & 3));
            const float q =
                PACK == QK_PACK_S8_SYM
                    ? static_cast<float>(static_cast<int8_t>(word & 255u))
                    : static_cast<float>(word & 255u);
            o.e[e] = dq(q);
          }
          *reinterpret_cast<u32x4*>(dst + 8 * v) = o.u;
        }
      }
    }
  }
};

template <typename T, int PACK, int BM, int BN, int WM, int WN>
qk_status LaunchTileQ(const GemmArgs& g, hipStream_t stream) {
  constexpr int NT = WM * WN * 64;
  dim3 grid(g.tiles_m * g.tiles_n, 1);
  gemm_tile_kernel<T, BM, BN, 64, WM, WN, false, QuantB<PACK, T, BN, 64, NT>>
      <<<grid, NT, 0, stream>>>(g);
  return PostLaunch("qgemm");
}

template <typename T, int PACK>
qk_status LaunchQ(const GemmArgs& g0, int m, int n, hipStream_t stream) {
  GemmArgs g = g0;
  const int cus = DeviceComputeUnits();
  auto ceil_div = [](long long a, long long b) { return (a + b - 1) / b; };
  const long long t128 = ceil_div(m, 128) * ceil_div(n, 128);
  const long long t256 = ceil_div(m, 256) * ceil_div(n, 256);
  int cfg;
  if (m <= 64 || t128 < cus)
    cfg = 3;  // 64x64
  else
    cfg = static_cast<double>(ceil_div(t256, cus)) <=
                  0.6 * static_cast<double>(ceil_div(t128, 2 * cus))
              ? 1
              : 2;
  const int bm = cfg == 1 ? 256 : cfg == 2 ? 128 : 64;
  g.tiles_m = static_cast<int>(ceil_div(m, bm));
  g.tiles_n = static_cast<int>(ceil_div(n, bm));
  if (static_cast<long long>(g.tiles_m) * g.tiles_n > 0x7fffffff) {
    return Fail(QK_UNIMPLEMENTED, "qkern: quantized matmul too large");
  }
  if (cfg == 1) return LaunchTileQ<T, PACK, 256, 256, 2, 4>(g, stream);
  if (cfg == 2) return LaunchTileQ<T, PACK, 128, 128, 2, 2>(g, stream);
  return LaunchTileQ<T, PACK, 64, 64, 2, 2>(g, stream);
}

template <typename T>
qk_status LaunchQPack(const GemmArgs& g, int packing, int m, int n,
                      hipStream_t stream) {
  switch (packing) {
    case QK_PACK_U32X8:
      return LaunchQ<T, QK_PACK_U32X8>(g, m, n, stream);
    case QK_PACK_BYTE_HALFSPLIT:
      return LaunchQ<T, QK_PACK_BYTE_HALFSPLIT>(g, m, n, stream);
    case QK_PACK_U8:
      return LaunchQ<T, QK_PACK_U8>(g, m, n, stream);
    default:
      return LaunchQ<T, QK_PACK_S8_SYM>(g, m, n, stream);
  }
}

}  // namespace

bool QGemmApplies(const QuantProblem& p) {
  if (p.x_dtype != QK_BF16 && p.x_dtype != QK_F16) return false;
  // A k-tile of 64 must hold whole half-split groups.
  if (p.packing == QK_PACK_BYTE_HALFSPLIT && p.group > 64) return false;
  if (p.m > 0x7fffffff || p.n > 0x7fffffff || p.k > 0x7fffffff) return false;
  return reinterpret_cast<uintptr_t>(p.x) % 16 == 0 && p.k % 8 == 0 &&
         reinterpret_cast<uintptr_t>(p.y) % 16 == 0 && p.n % 4 == 0;
}

qk_status LaunchQGemm(const QuantProblem& p, hipStream_t stream) {
  GemmArgs g{};
  g.a = p.x;
  g.b = p.codes;
  g.c = nullptr;
  g.d = p.y;
  g.bias = nullptr;
  g.aux = nullptr;
  g.m = static_cast<int>(p.m);
  g.n = static_cast<int>(p.n);
  g.k = static_cast<int>(p.k);
  g.lda = static_cast<int>(p.k);
  g.ldb = 0;
  g.ldd = static_cast<int>(p.n);
  g.bsa = g.bsb = g.bsd = 0;
  g.alpha = 1.f;
  g.beta = 0.f;
  g.use_c = g.has_bias = g.has_aux = 0;
  g.act = 0;
  g.out_f32 = 0;
  g.a_vec = 1;
  g.b_vec = 1;
  g.out_vec = 1;
  g.qscale = p.scales;
  g.qbias = p.biases;
  g.qsdt = p.scale_dtype;
  g.qbdt = p.bias_dtype;
  g.qhas_bias = p.has_bias ? 1 : 0;
  g.qgroup = p.group;
  g.qrow_bytes = static_cast<int>(p.bits == 4 ? p.k / 2 : p.k);
  if (p.x_dtype == QK_BF16)
    return LaunchQPack<bf16>(g, p.packing, g.m, g.n, stream);
  return LaunchQPack<f16>(g, p.packing, g.m, g.n, stream);
}

}  // namespace qk
