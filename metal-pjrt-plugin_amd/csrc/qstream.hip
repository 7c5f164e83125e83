// Quantized matmul for 5..16 rows of x streamed straight into the matrix
// cores: y[M, N] = x[M, K] W^T with W int4 (u32x8 words), bf16 x / scale /
// offset, group size 64, K a multiple of 512 up to 4096 (the batched-decode
// projections and the lm_head of Qwen3-8B). Like qskinny.hip it keeps the
// codes factored per group, as the reference's _matvec_int4 does
// (examples/llm/qwen3.py:233-267: y = s * sum(x q) + b * sum(x) per group),
// which skips the bf16 rounding of the dequantized weights of the
// reference's linear() for more than ROWS_MAX rows (qwen3.py:215-230).
//
// Design (MI355X-first): the codes are read once, as the decode GEMV reads
// them, with no LDS on their path, and x stays in registers.
//  - One workgroup of eight waves per CU. K is cut into KS = K / 512
//    slices of 8 groups; wave w takes slice w % KS of row block
//    (round grid + workgroup) 8 / KS + w / KS, a row block being 16 weight
//    rows (the MFMA's B columns). Its slice of x is loaded once, straight
//    into the A fragments of v_mfma_f32_16x16x32_bf16 (64 VGPRs), with the
//    per-group sums of x. A wave keeps PD row blocks' codes, scales and
//    offsets in flight in registers (24 VGPRs each).
//  - A slice is four 16-byte loads per lane: lane (n = l % 16, q = l / 16)
//    reads chunk 4 j + q of row n's 256 bytes in load j, so every load
//    reads 64 contiguous bytes of each of 16 rows, and lanes q < 2 hold
//    group 2 j, lanes q >= 2 group 2 j + 1 (four words each). Two
//    v_permlane32_swap exchange the halves so that every lane holds two
//    words of each group: each MFMA then multiplies K values of one group
//    only, and its scale applies after it. Lane q holds words
//    {0, 4, 2, 6}[q] + i of both groups; x's fragments follow that order.
//  - Codes become bf16 pairs (128 + q_a, 128 + q_b) with one v_and_or_b32
//    per pair (the two words of a group shifted together by one 64-bit
//    shift); per group tmp = sum x (128 + q) (two MFMAs) and
//    acc += s tmp; the offsets' part, sum over groups of
//    (b - 128 s) sum x, is two f32 MFMAs (16x16x4) per slice.
//  - KS > 1: the waves of a row block add their partial tiles through LDS,
//    one barrier per four rounds, the four rounds' sums spread over the
//    waves; every wave runs the same number of rounds, so the barriers
//    line up.
//  - Rounds past the last row block read zeros through out-of-range
//    per-lane offsets (no memory traffic), so no load is conditional.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kQsWaves = 8;
constexpr int kQsSliceK = 512;  // K per wave slice (8 groups)
constexpr int kQsMaxK = kQsWaves * kQsSliceK;
// Partial tiles are reduced once every kQsRg rounds, from 2 kQsRg buffers.
constexpr int kQsRg = 4;
constexpr int kQsRedBytes = 2 * kQsRg * kQsWaves * 64 * 16;
// An offset past every extent (the launcher bounds the extents below it).
constexpr int kQsSkip = 0x7FF00000;

struct QsArgs {
  const void* x;
  const void* codes;
  const void* scales;
  const void* biases;
  void* y;
  int m, n, k;
  int has_bias;
  int rowblocks;  // ceil(n / 16)
  int rounds;     // row-block rounds of every wave
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t QsRsrc(const void* p,
                                                         int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                           bytes, 0x00020000);
}

// x (8 consecutive bf16) -> the pair order of a code word: (x0, x4),
// (x1, x5), (x2, x6), (x3, x7).
__device__ __forceinline__ u32x4 QsXPairs(const u32x4& v) {
  constexpr uint32_t kLoLo = 0x05040100u, kHiHi = 0x07060302u;
  return u32x4{__builtin_amdgcn_perm(v[2], v[0], kLoLo),
               __builtin_amdgcn_perm(v[2], v[0], kHiHi),
               __builtin_amdgcn_perm(v[3], v[1], kLoLo),
               __builtin_amdgcn_perm(v[3], v[1], kHiHi)};
}

template <int KS, int PD>
__global__ __launch_bounds__(kQsWaves * 64) void qmm_stream_kernel(QsArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char red_lds[kQsRedBytes];
  constexpr int RPW = kQsWaves / KS;  // row blocks per workgroup per round
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sub = wave / KS, kpart = wave % KS;
  const int G = a.k / 64;
  const int n = lane & 15, q = lane >> 4;
  const int row_bytes = a.k / 2;

  const __amdgpu_buffer_rsrc_t crs = QsRsrc(a.codes, a.n * row_bytes);
  const __amdgpu_buffer_rsrc_t srs = QsRsrc(a.scales, a.n * G * 2);
  // An extent of 0 reads zeros: no offsets.
  const __amdgpu_buffer_rsrc_t brs =
      QsRsrc(a.biases, a.has_bias ? a.n * G * 2 : 0);
  const int cvoff = n * row_bytes + kpart * 256 + q * 16;
  const int svoff = n * G * 2 + kpart * 16;

  struct Slot {
    u32x4 c[4];
    u32x4 s, b;
  };
  auto row_block = [&](int round) {
    return (round * static_cast<int>(gridDim.x) +
            static_cast<int>(blockIdx.x)) * RPW + sub;
  };
  auto load = [&](int round, Slot& sl) {
    const int rb = row_block(round);
    const bool ok = round < a.rounds && rb < a.rowblocks;
    // The row offset is scalar; a round past the end moves the per-lane
    // offsets past every extent (the range check covers the per-lane and
    // instruction offsets, not the scalar one).
    const int co = ok ? rb * 16 * row_bytes : 0;
    const int so = ok ? rb * 16 * G * 2 : 0;
    const int skip = ok ? 0 : kQsSkip;
    // Normal cache policy: each load reads half of 16 lines whose other
    // halves the next load reads; nontemporal loads measured 15% slower
    // (the lm_head at 16 rows: 92 against 78 us).
#pragma unroll
    for (int j = 0; j < 4; ++j)
      sl.c[j] = __builtin_amdgcn_raw_buffer_load_b128(
          crs, cvoff + skip + 64 * j, co, 0);
    sl.s = __builtin_amdgcn_raw_buffer_load_b128(srs, svoff + skip, so, 0);
    sl.b = __builtin_amdgcn_raw_buffer_load_b128(brs, svoff + skip, so, 0);
  };

  // The first PD rounds are requested before x (loads complete in order:
  // x is then converted while they land).
  Slot ring[PD];
#pragma unroll
  for (int d = 0; d < PD; ++d) load(d, ring[d]);

  // x of this slice as A fragments: xf[g][i] of lane (m = l % 16, q) holds
  // row m, K (8 kpart + g) 64 + 8 ({0, 4, 2, 6}[q] + i) .. + 7 (zeros past
  // M). xa[t]: the sum of x over group 4 t + q of the slice in row m (the
  // A operand of the offsets' 16x16x4 MFMA).
  bf16x8 xf[8][2];
  float xa[2];
  {
    const int m = n;
    const int base = ((q & 1) ? 4 : 0) + ((q & 2) ? 2 : 0);
    // Rows past M lie past the descriptor's extent: they read zeros, and
    // no load is conditional.
    const __amdgpu_buffer_rsrc_t xrs = QsRsrc(a.x, a.m * a.k * 2);
    const int xoff = (m * a.k + kpart * kQsSliceK + 8 * base) * 2;
    u32x4 xv[8][2];
#pragma unroll
    for (int g = 0; g < 8; ++g)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        xv[g][i] = __builtin_amdgcn_raw_buffer_load_b128(
            xrs, xoff + (g * 64 + 8 * i) * 2, 0, 0);
    // Group sums in named scalars, not an array: a select between array
    // elements by a lane-dependent index would be folded into a dynamically
    // indexed private array (placed in LDS, with every wave reading the
    // dispatch packet for its flat thread index).
    auto group_sum = [&](int g) {
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t pr = xv[g][i][w];
          sum += __uint_as_float(pr << 16) + __uint_as_float(pr & 0xFFFF0000u);
        }
      // The four lanes of row m (q = 0..3) hold the group's 64 elements.
      sum += __shfl_xor(sum, 16, 64);
      return sum + __shfl_xor(sum, 32, 64);
    };
#pragma unroll
    for (int g = 0; g < 8; ++g)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        xf[g][i] = __builtin_bit_cast(bf16x8, QsXPairs(xv[g][i]));
    const bool q1 = (q & 1) != 0, q2 = (q & 2) != 0;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float s0 = group_sum(4 * t), s1 = group_sum(4 * t + 1);
      const float s2 = group_sum(4 * t + 2), s3 = group_sum(4 * t + 3);
      const float lo = q1 ? s1 : s0, hi = q1 ? s3 : s2;
      xa[t] = q2 ? hi : lo;
    }
  }

  const uint32_t kMask = vgpr_const(0x000F000Fu);
  const uint32_t kBias = vgpr_const(0x43004300u);
  bf16* Y = static_cast<bf16*>(a.y);

  // The partial tile of this wave's slice of one row block.
  auto compute = [&](const Slot& sl) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 c = sl.c[j];
      // Lanes 0..31 give words 2, 3 for lanes 32..63's words 0, 1.
      {
        const auto s0 = __builtin_amdgcn_permlane32_swap(c[0], c[2], false,
                                                         false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(c[1], c[3], false,
                                                         false);
        c[0] = s0[0], c[2] = s0[1], c[1] = s1[0], c[3] = s1[1];
      }
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const int g = 2 * j + gg;  // group within the slice
        // Both words of the group shifted together: the bits the low word
        // takes from the high one land above bit 19, outside the mask.
        const uint64_t v = (static_cast<uint64_t>(c[2 * gg + 1]) << 32) |
                           c[2 * gg];
        const uint64_t sv[4] = {v, shr64<4>(v), shr64<8>(v), shr64<12>(v)};
        u32x4 p0, p1;
#pragma unroll
        for (int sh = 0; sh < 4; ++sh) {
          p0[sh] = (static_cast<uint32_t>(sv[sh]) & kMask) | kBias;
          p1[sh] = (static_cast<uint32_t>(sv[sh] >> 32) & kMask) | kBias;
        }
        f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            xf[g][0], __builtin_bit_cast(bf16x8, p0),
            f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            xf[g][1], __builtin_bit_cast(bf16x8, p1), t, 0, 0, 0);
        const uint32_t sw = sl.s[g >> 1];
        const float s =
            __uint_as_float((g & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(s, t[r], acc[r]);
      }
    }
    // Offsets: sum over the slice's groups of (b - 128 s)[n, g] sum x[m, g],
    // as a 16 x 16 x 8 product on the f32 matrix cores (B: lane (n, q)
    // gives group 4 t + q of row n).
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t sw = (q & 2) ? sl.s[2 * t + 1] : sl.s[2 * t];
      const uint32_t bw = (q & 2) ? sl.b[2 * t + 1] : sl.b[2 * t];
      const float s = __uint_as_float((q & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
      const float b = __uint_as_float((q & 1) ? (bw & 0xFFFF0000u) : (bw << 16));
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[t], fmaf(-128.f, s, b), acc,
                                                 0, 0, 0);
    }
    return acc;
  };
  // Lane (n, q) holds rows 4 q + r of column n of the tile.
  auto store = [&](int rb, const f32x4& v) {
    const int col = rb * 16 + n;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * q + r;
      if (m < a.m && col < a.n)
        Y[static_cast<long long>(m) * a.n + col] = from_f32<bf16>(v[r]);
    }
  };
  // Round r's partial tiles go to buffer r % (2 kQsRg); after every
  // kQsRg-th round (and the last) one barrier, then the group's rounds are
  // summed and stored by different waves of their row block (round r by
  // kpart (r % kQsRg) % KS). A buffer is written again 2 kQsRg rounds
  // later, after the next group's barrier, which its readers reach only
  // once they have read it.
  auto finish = [&](int round, const f32x4& acc) {
    if constexpr (KS == 1) {
      const int rb = row_block(round);
      if (rb < a.rowblocks) store(rb, acc);
    } else {
      constexpr int kBuf = kQsWaves * 64 * 16;
      *reinterpret_cast<f32x4*>(red_lds + (round % (2 * kQsRg)) * kBuf +
                                (wave * 64 + lane) * 16) = acc;
      if (round % kQsRg == kQsRg - 1 || round == a.rounds - 1) {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int first = round - round % kQsRg;
#pragma unroll
        for (int g = 0; g < kQsRg; ++g) {
          const int rr = first + g;
          const int rb = row_block(rr);
          if (rr <= round && kpart == g % KS && rb < a.rowblocks) {
            const unsigned char* red = red_lds + (rr % (2 * kQsRg)) * kBuf;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < KS; ++k) {
              const f32x4 o = *reinterpret_cast<const f32x4*>(
                  red + ((sub * KS + k) * 64 + lane) * 16);
#pragma unroll
              for (int r = 0; r < 4; ++r) v[r] += o[r];
            }
            store(rb, v);
          }
        }
      }
    }
  };

  // Every wave runs the same rounds, padded to a multiple of PD: the ring
  // is refilled unconditionally (rounds past the end read zeros), so the
  // compiler's wait counts follow the ring's order instead of draining it.
  const int padded = (a.rounds + PD - 1) / PD * PD;
  for (int r0 = 0; r0 < padded; r0 += PD) {
#pragma unroll
    for (int d = 0; d < PD; ++d) {
      const int round = r0 + d;
      // Padding rounds (the same for every wave) only keep the loads in
      // order; their compute and reduction are skipped.
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if (round < a.rounds) acc = compute(ring[d]);
      load(round + PD, ring[d]);
      if (round < a.rounds) finish(round, acc);
    }
  }
  __builtin_amdgcn_s_waitcnt(VmcntImm(0));
}

}  // namespace

bool QStreamApplies(const QuantProblem& p) {
  return p.m >= 1 && p.m <= 16 && p.bits == 4 &&
         p.packing == QK_PACK_U32X8 && p.group == 64 &&
         p.x_dtype == QK_BF16 && p.scale_dtype == QK_BF16 &&
         (!p.has_bias || p.bias_dtype == QK_BF16) && p.k > 0 &&
         p.k % kQsSliceK == 0 && p.k <= kQsMaxK &&
         (p.k / kQsSliceK & (p.k / kQsSliceK - 1)) == 0 &&
         p.m * p.k * 2 < kQsSkip && p.n > 0 &&
         p.n * (p.k / 2) + 16 * (p.k / 2) < kQsSkip &&
         reinterpret_cast<uintptr_t>(p.x) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.codes) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.scales) % 16 == 0 &&
         (!p.has_bias || reinterpret_cast<uintptr_t>(p.biases) % 16 == 0);
}

namespace {
struct QsGrid {
  int ks, grid, rounds;
};
QsGrid QStreamGrid(const QuantProblem& p, int cus) {
  QsGrid g;
  g.ks = static_cast<int>(p.k / kQsSliceK);  // waves per row block
  const int rpw = kQsWaves / g.ks;
  const int64_t rowblocks = (p.n + 15) / 16;
  g.grid = static_cast<int>(std::max<int64_t>(
      1, std::min<int64_t>(cus, (rowblocks + rpw - 1) / rpw)));
  g.rounds = static_cast<int>((rowblocks + int64_t{g.grid} * rpw - 1) /
                              (int64_t{g.grid} * rpw));
  return g;
}
}  // namespace

int QStreamRounds(const QuantProblem& p, int cus) {
  return QStreamGrid(p, cus).rounds;
}

qk_status LaunchQStream(const QuantProblem& p, hipStream_t stream) {
  QsArgs a;
  a.x = p.x;
  a.codes = p.codes;
  a.scales = p.scales;
  a.biases = p.has_bias ? p.biases : nullptr;
  a.y = p.y;
  a.m = static_cast<int>(p.m);
  a.n = static_cast<int>(p.n);
  a.k = static_cast<int>(p.k);
  a.has_bias = p.has_bias ? 1 : 0;
  a.rowblocks = static_cast<int>((p.n + 15) / 16);
  const QsGrid g = QStreamGrid(p, DeviceComputeUnits());
  a.rounds = g.rounds;
  // Rounds in flight per wave: one for short runs (a deeper ring only adds
  // padding and registers: 12288 x 4096 11.2 against 13.2 us), four for
  // long ones (the lm_head 74 against 82 us).
  const bool deep = g.rounds > 8;
  auto go = [&](auto k1, auto k4) {
    if (deep)
      k4<<<g.grid, kQsWaves * 64, 0, stream>>>(a);
    else
      k1<<<g.grid, kQsWaves * 64, 0, stream>>>(a);
  };
  switch (g.ks) {
    case 1:
      go(qmm_stream_kernel<1, 1>, qmm_stream_kernel<1, 4>);
      break;
    case 2:
      go(qmm_stream_kernel<2, 1>, qmm_stream_kernel<2, 4>);
      break;
    case 4:
      go(qmm_stream_kernel<4, 1>, qmm_stream_kernel<4, 4>);
      break;
    case 8:
      go(qmm_stream_kernel<8, 1>, qmm_stream_kernel<8, 4>);
      break;
    default:
      return Fail(QK_INTERNAL, "qkern: qmm_stream slice count");
  }
  return PostLaunch("qmm_stream");
}

}  // namespace qk
