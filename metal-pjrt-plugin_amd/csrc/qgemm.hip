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
#include <cstdlib>
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

// Quantized B operand of the interior-tile kernel (gemm_common.h): weight
// rows n0 .. n0 + BN of a K tile of 64 = one group of 64. Each of the NT
// threads buffer-loads its part of one row's codes (16-byte loads, or one
// 8-byte load for 16 int4 codes; every row's bytes contiguous across its
// TPR threads) and the group's bf16 scale and offset, and writes
// T(f32(q) * f32(s) + f32(b)) (the unfused canonical rounding of
// qk$dequantize) K-contiguously into LDS.
template <int PACK, typename T, int BN, int NT_ = 256>
struct QuantFastB {
  static constexpr bool kKCont = true;
  static constexpr bool kInt4 = PACK == QK_PACK_U32X8;
  static constexpr int NT = NT_, BK = 64;
  static constexpr int TPR = NT / BN;                // threads per row
  static constexpr int KPT = BK / TPR;               // codes per thread
  static constexpr int CBT = kInt4 ? KPT / 2 : KPT;  // code bytes per thread
  static constexpr int NL = CBT >= 16 ? CBT / 16 : 1;  // loads
  static constexpr int NV = KPT * static_cast<int>(sizeof(T)) / 16;
  static constexpr int LD = TileLayout<T, BN, BK, true>::kLd;
  static_assert((CBT == 8 || CBT % 16 == 0) && NV >= 1, "tile split");
  __amdgpu_buffer_rsrc_t crs, srs, brs;
  int row_bytes, G, r, kk0, cvo, svo;
  u32x4 c[NL];
  uint16_t sraw, braw;

  __device__ __forceinline__ QuantFastB(const GemmArgs& g, long long /*b*/,
                                        int tid)
      : row_bytes(g.qrow_bytes), G(g.k / 64), r(tid / TPR),
        kk0((tid % TPR) * KPT) {
    crs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(g.b), (short)0,
                                            g.n * row_bytes, 0x00020000);
    srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(g.qscale),
                                            (short)0, g.n * G * 2, 0x00020000);
    brs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(g.qbias), (short)0, g.qhas_bias ? g.n * G * 2 : 0,
        0x00020000);
    cvo = r * row_bytes + (kInt4 ? kk0 / 2 : kk0);
    svo = r * G * 2;
  }
  __device__ __forceinline__ void load(int n0, int k0) {
    const int so = n0 * row_bytes + (kInt4 ? k0 / 2 : k0);
    if constexpr (CBT == 8) {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(crs, cvo, so, 2);
      c[0] = u32x4{v[0], v[1], 0u, 0u};
    } else {
#pragma unroll
      for (int i = 0; i < NL; ++i)
        c[i] = __builtin_amdgcn_raw_buffer_load_b128(crs, cvo + 16 * i, so, 2);
    }
    const int sg = n0 * G * 2 + (k0 / 64) * 2;
    sraw = __builtin_amdgcn_raw_buffer_load_b16(srs, svo, sg, 0);
    braw = __builtin_amdgcn_raw_buffer_load_b16(brs, svo, sg, 0);  // 0: none
  }
  __device__ __forceinline__ void store(T* lds, int /*tid*/) const {
    const float sc = __uint_as_float(static_cast<uint32_t>(sraw) << 16);
    const float bi = __uint_as_float(static_cast<uint32_t>(braw) << 16);
    T* dst = lds + r * LD + kk0;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      union {
        u32x4 u;
        T e[8];
      } o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = 8 * v + j;  // code index within the thread's run
        float q;
        if constexpr (kInt4) {
          const uint32_t word = c[e / 32][(e % 32) / 8];
          q = static_cast<float>((word >> (4 * (e % 8))) & 15u);
        } else {
          const uint32_t word = c[e / 16][(e % 16) / 4] >> (8 * (e % 4));
          q = PACK == QK_PACK_S8_SYM
                  ? static_cast<float>(static_cast<int8_t>(word & 255u))
                  : static_cast<float>(word & 255u);
        }
        // q * sc is exact in f32 (at most 8 + 8 significant bits), so
        // the fused form rounds exactly as the unfused canonical one.
        o.e[j] = from_f32<T>(fmaf(q, sc, bi));
      }
      *reinterpret_cast<u32x4*>(dst + 8 * v) = o.u;
    }
  }
};

// The interior-tile kernel for any M, N a multiple of 128, group 64, bf16
// scales/offsets; false when it does not apply. Eight waves; tiles of
// 256 x 256, 256 x 128 or 128 x 128 (two workgroups per CU); the last M
// tile may be partly filled (A rows past M read zeros, their outputs are
// not stored).
template <typename T, int PACK>
bool LaunchFastQ(GemmArgs g, int m, int n, hipStream_t stream,
                 qk_status* st) {
  if constexpr (PACK == QK_PACK_BYTE_HALFSPLIT) {
    return false;
  } else {
    if (m <= 0 || n % 128 != 0 || g.k % 64 != 0 || g.k == 0 ||
        g.qgroup != 64 || g.qsdt != QK_BF16 ||
        (g.qhas_bias && g.qbdt != QK_BF16) ||
        static_cast<int64_t>(n) * g.qrow_bytes >= (int64_t{1} << 31) ||
        (static_cast<int64_t>(m) + 256) * g.k * 2 >= (int64_t{1} << 31) ||
        reinterpret_cast<uintptr_t>(g.a) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(g.b) % 16 != 0)
      return false;
    const int cus = DeviceComputeUnits();
    // QK_QGEMM_TILE=1|2|3 forces 256x256 / 256x128 / 128x128 (tuning).
    static const int forced = [] {
      const char* v = std::getenv("QK_QGEMM_TILE");
      return v == nullptr ? 0 : std::atoi(v);
    }();
    // Tile choice, measured at N = 12288, K = 4096 (int4, us): M = 256:
    // 114 / 75 / 63; M = 512: 130 / 82 / 112; M = 1024: 139 / 162 / 187;
    // M = 2048: 271 / 259 / 382 (256x256 / 256x128 / 128x128). The
    // smallest tile whose count still fits one round of CUs; when none
    // does, the fewest rounds times tile size (ties to the larger tile).
    const long long m256 = (m + 255) / 256, m128 = (m + 127) / 128;
    const bool ok[4] = {false, n % 256 == 0, true, true};
    const long long count[4] = {0, m256 * (n / 256), m256 * (n / 128),
                                m128 * (n / 128)};
    const double size[4] = {0, 1.0, 0.5, 0.25};
    int tile = 0;
    for (int t = 1; t <= 3; ++t)
      if (ok[t] && count[t] <= cus) tile = t;
    if (tile == 0) {
      double best = 1e30;
      for (int t = 1; t <= 3; ++t) {
        if (!ok[t]) continue;
        const double c = static_cast<double>((count[t] + cus - 1) / cus) * size[t];
        if (c < best) best = c, tile = t;
      }
    }
    if (forced >= 1 && forced <= 3 && ok[forced]) tile = forced;
    const int bm = tile == 3 ? 128 : 256, bn = tile == 1 ? 256 : 128;
    g.tiles_m = (m + bm - 1) / bm;
    g.tiles_n = n / bn;
    const dim3 grid(g.tiles_m * g.tiles_n);
    // Two register sets of loads in flight (int8 codes in two sets would
    // spill at 256 x 256).
    if (tile == 1)
      gemm_fast_kernel<T, 256, false, QuantFastB<PACK, T, 256, 512>, 8, 256,
                       PACK == QK_PACK_U32X8 ? 2 : 1, true>
          <<<grid, 512, 0, stream>>>(g);
    else if (tile == 2)
      gemm_fast_kernel<T, 128, false, QuantFastB<PACK, T, 128, 512>, 8, 256,
                       2, true><<<grid, 512, 0, stream>>>(g);
    else
      gemm_fast_kernel<T, 128, false, QuantFastB<PACK, T, 128, 512>, 8, 128,
                       2, true><<<grid, 512, 0, stream>>>(g);
    *st = PostLaunch("qgemm_fast");
    return true;
  }
}

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
  qk_status st = QK_OK;
  if (LaunchFastQ<T, PACK>(g0, m, n, stream, &st)) return st;
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
  if (g.k / 64 >= 16) {
    // Few 64x64 tiles and a long K: four waves per tile, each a quarter of
    // the K tiles, reduced through LDS.
    gemm_splitk_kernel<T, 64, 64, 64, 4, DenseA<T, 64, 64, 64, true>,
                       QuantB<PACK, T, 64, 64, 64>>
        <<<dim3(g.tiles_m * g.tiles_n), 256, 0, stream>>>(g);
    return PostLaunch("qgemm_splitk");
  }
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
