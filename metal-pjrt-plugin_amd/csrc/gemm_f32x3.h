// f32 GEMM on the bf16 matrix cores: each f32 operand element a is split
// exactly into three bf16 values a = h + m + l (h: a with its mantissa
// truncated to bf16's 7 bits, m: the same of a - h, l = a - h - m, which
// has at most 8 significant bits), and each 32x32 block of the product is
// accumulated in f32 from the six partial products whose magnitude is at
// least 2^-16 of the leading one:
//   h_a h_b + h_a m_b + m_a h_b + h_a l_b + m_a m_b + l_a h_b.
// The dropped terms (m l, l m, l l) are below 2^-23 of |a||b|, under one
// f32 rounding of each product, so the result meets an f32 GEMM's error
// bound; the bf16 MFMA (v_mfma_f32_32x32x16_bf16) has 16x the f32 MFMA's
// rate, so six of them still outrun one f32 MFMA pass. Truncation (never
// rounding up) keeps h finite for every finite a. An infinite or NaN
// element keeps its value in h (a NaN as a quiet NaN) and has m = l = 0;
// so that it enters only the h h term (as in an f32 product) and never
// meets a zero part of the other operand in a cross term (inf * 0 = NaN),
// a workgroup whose loaders saw such an element computes its tile again
// with, in the cross terms, h's infinities and NaNs replaced by zero (the
// common, all-finite case pays only the loaders' check).
//
// Interior tiles (N a multiple of the tile, K of 32, any M: the last M
// tile may be partly filled; 16-byte aligned operands): the operand tiles are read with buffer loads into
// registers, split, and written as three bf16 tiles per operand into LDS
// in the layouts of the bf16 kernels (gemm_common.h TileLayout), so the
// fragment reads and MFMAs are those of the bf16 interior-tile kernel.
// Two LDS stages; the next K tile is loaded while the current one is
// multiplied. The epilogue is applied from the accumulators.
#pragma once

#include <type_traits>

#include "gemm_common.h"

namespace qk {
namespace {

// Three bf16 parts of four f32 values, packed two per dword (element 2i in
// the low half of dword i).
struct Split4 {
  u32x2 h, m, l;
  bool special;  // one of the four is infinite or NaN
};
__device__ __forceinline__ Split4 SplitF32x4(const u32x4& v) {
  uint32_t h[4], m[4], l[4];
  bool special = false;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t u = v[e];
    const uint32_t hb = u & 0xFFFF0000u;
    const float r1 = __uint_as_float(u) - __uint_as_float(hb);
    const uint32_t mb = __float_as_uint(r1) & 0xFFFF0000u;
    const float r2 = r1 - __uint_as_float(mb);
    const bool fin = (u & 0x7F800000u) != 0x7F800000u;
    const bool nan = !fin && (u & 0x007FFFFFu) != 0u;
    special |= !fin;
    h[e] = nan ? 0x7FC00000u : hb;
    m[e] = fin ? mb : 0u;
    l[e] = fin ? __float_as_uint(r2) : 0u;
  }
  constexpr uint32_t kHiHi = 0x07060302u;  // high halves of (lo, hi) words
  Split4 s;
  s.special = special;
  s.h = u32x2{__builtin_amdgcn_perm(h[1], h[0], kHiHi),
              __builtin_amdgcn_perm(h[3], h[2], kHiHi)};
  s.m = u32x2{__builtin_amdgcn_perm(m[1], m[0], kHiHi),
              __builtin_amdgcn_perm(m[3], m[2], kHiHi)};
  s.l = u32x2{__builtin_amdgcn_perm(l[1], l[0], kHiHi),
              __builtin_amdgcn_perm(l[3], l[2], kHiHi)};
  return s;
}

// Global f32 tile (R rows x BK of K, in its source orientation) ->
// registers -> three bf16 tiles in LDS (TileLayout<bf16, R, BK, KCONT>).
// Thread t loads 16-byte vectors t, t + NT, ... of the tile; vector i
// covers source row (t / VPR) + i * RPI, elements 4 (t % VPR) .. + 3.
// VC: the whole offset goes in the vector offset, which the descriptor's
// extent checks (for tiles that run past the operand's last row).
template <int R, int BK, int NT, bool KCONT, bool VC = false>
struct SplitLoader {
  static constexpr int VPR = (KCONT ? BK : R) / 4;  // vectors per row
  static constexpr int RPI = NT / VPR;               // rows between vectors
  static constexpr int NV = R * BK / 4 / NT;
  static_assert(NT % VPR == 0 && NV * NT * 4 == R * BK, "tile split");
  __amdgpu_buffer_rsrc_t rsrc;
  int voff, ld;
  u32x4 v[NV];
  __device__ __forceinline__ void init(const float* src, long long bytes,
                                       int ld_, int tid) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src),
                                             (short)0, static_cast<int>(bytes),
                                             0x00020000);
    ld = ld_;
    voff = ((tid / VPR) * ld + (tid % VPR) * 4) * 4;
  }
  // Tile origin: rows r0 (M or N), k0.
  __device__ __forceinline__ void load(int r0, int k0) {
    const int base = KCONT ? r0 * ld + k0 : k0 * ld + r0;  // elements
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int so = (base + i * RPI * ld) * 4;
      if constexpr (VC)
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff + so, 0, 0);
      else
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, so, 0);
    }
  }
  // Returns whether any of the thread's elements is infinite or NaN.
  __device__ __forceinline__ bool store(bf16* th, bf16* tm, bf16* tl,
                                        int tid) const {
    constexpr int LD = TileLayout<bf16, R, BK, KCONT>::kLd;
    const int o = (tid / VPR) * LD + (tid % VPR) * 4;
    bool special = false;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const Split4 s = SplitF32x4(v[i]);
      special |= s.special;
      const int p = o + i * RPI * LD;
      *reinterpret_cast<u32x2*>(th + p) = s.h;
      *reinterpret_cast<u32x2*>(tm + p) = s.m;
      *reinterpret_cast<u32x2*>(tl + p) = s.l;
    }
    return special;
  }
};

// A fragment with its infinite and NaN bf16 elements replaced by zero.
__device__ __forceinline__ Frag<bf16>::type FiniteOnly(
    const Frag<bf16>::type& f) {
  u32x4 w = __builtin_bit_cast(u32x4, f);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = (w[i] & 0x7F80u) == 0x7F80u ? 0xFFFF0000u : ~0u;
    const uint32_t hi = (w[i] & 0x7F800000u) == 0x7F800000u ? 0x0000FFFFu : ~0u;
    w[i] &= lo & hi;
  }
  return __builtin_bit_cast(Frag<bf16>::type, w);
}

// MC: M need not be a multiple of BM: the A tile's offsets go wholly in
// the range-checked vector offset and the epilogue skips rows past M
// (values fetched for rows past M only reach those rows; a non-finite one
// among them at worst costs the workgroup the masked second pass).
// KS = 2: two groups of NW / 2 waves share the tile, group q taking the
// 16-wide K step q of every K tile (two waves per SIMD for a tile too
// small to keep one wave per SIMD busy); their partial tiles are summed
// through LDS before the epilogue.
template <int BM, int BN, bool TA, bool TB, int NW, bool MC = false,
          int KS = 1, int BK = 32>
__global__ __launch_bounds__(NW * 64) void gemm_f32x3_kernel(GemmArgs g) {
  constexpr int NT = NW * 64, WM = NW / KS / 2, WN = 2;
  static_assert(KS == 1 || KS == BK / 16, "one K step per wave group");
  constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 32, FN = WTN / 32;
  static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0,
                "wave tile");
  constexpr bool AK = !TA, BKC = TB;  // K-contiguous operands
  using LA = TileLayout<bf16, BM, BK, AK>;
  using LB = TileLayout<bf16, BN, BK, BKC>;
  // stage s: [A h | A m | A l | B h | B m | B l]
  constexpr int kStage = 3 * (LA::kElems + LB::kElems);
  __shared__ __attribute__((aligned(16))) bf16 lds[2 * kStage];
  // Set by a loader that stored an infinite or NaN operand element.
  __shared__ int nonfinite;
  auto ta_ = [&](int s, int c) { return lds + s * kStage + c * LA::kElems; };
  auto tb_ = [&](int s, int c) {
    return lds + s * kStage + 3 * LA::kElems + c * LB::kElems;
  };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ks = wave / (WM * WN), wv = wave % (WM * WN);
  const int wm = wv / WN, wn = wv % WN;
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

  SplitLoader<BM, BK, NT, AK, MC> la;
  la.init(static_cast<const float*>(g.a) + batch * g.bsa,
          static_cast<long long>(AK ? g.m : g.k) * g.lda * 4, g.lda, tid);
  SplitLoader<BN, BK, NT, BKC> lb;
  lb.init(static_cast<const float*>(g.b) + batch * g.bsb,
          static_cast<long long>(BKC ? g.n : g.k) * g.ldb * 4, g.ldb, tid);

  f32x16 acc[FM][FN];
  const int ktiles = g.k / BK;  // >= 1
  using F = Frag<bf16>::type;
  // The K loop; MASK: the cross terms use h with its infinities and NaNs
  // replaced by zero. Returns (uniformly) whether any operand element of
  // the workgroup's tiles was infinite or NaN.
  auto run = [&](auto mask_tag) -> bool {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    bool seen = false;
    la.load(m0, 0);
    lb.load(n0, 0);
    seen |= la.store(ta_(0, 0), ta_(0, 1), ta_(0, 2), tid);
    seen |= lb.store(tb_(0, 0), tb_(0, 1), tb_(0, 2), tid);
    {
      const int k1 = min(1, ktiles - 1) * BK;
      la.load(m0, k1);
      lb.load(n0, k1);
    }
    __syncthreads();
    for (int kt = 0; kt < ktiles; ++kt) {
      const int cur = kt & 1;
#pragma unroll
      for (int s = 0; s < BK / 16; ++s) {
        if (KS > 1 && s != ks) continue;
        F fa[3][FM], fb[3][FN];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
#pragma unroll
          for (int i = 0; i < FM; ++i)
            fa[c][i] = load_frag<bf16, BM, BK, AK>(ta_(cur, c),
                                                   wm * WTM + i * 32, s * 16,
                                                   lane);
#pragma unroll
          for (int j = 0; j < FN; ++j)
            fb[c][j] = load_frag<bf16, BN, BK, BKC>(tb_(cur, c),
                                                    wn * WTN + j * 32, s * 16,
                                                    lane);
        }
        // h as it enters the cross terms
        F ax[FM], bx[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          ax[i] = MASK ? FiniteOnly(fa[0][i]) : fa[0][i];
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bx[j] = MASK ? FiniteOnly(fb[0][j]) : fb[0][j];
        // smallest terms first
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            mma(acc[i][j], fa[2][i], bx[j]);
            mma(acc[i][j], fa[1][i], fb[1][j]);
            mma(acc[i][j], ax[i], fb[2][j]);
            mma(acc[i][j], fa[1][i], bx[j]);
            mma(acc[i][j], ax[i], fb[1][j]);
            mma(acc[i][j], fa[0][i], fb[0][j]);
          }
      }
      // Nobody reads the other stage during this tile (its last reader was
      // the previous tile, which ended on a barrier): write the next tile
      // there and request the one after.
      if (kt + 1 < ktiles) {
        seen |=
            la.store(ta_(cur ^ 1, 0), ta_(cur ^ 1, 1), ta_(cur ^ 1, 2), tid);
        seen |=
            lb.store(tb_(cur ^ 1, 0), tb_(cur ^ 1, 1), tb_(cur ^ 1, 2), tid);
        const int k2 = min(kt + 2, ktiles - 1) * BK;
        la.load(m0, k2);
        lb.load(n0, k2);
      }
      __syncthreads();
    }
    if (seen) nonfinite = 1;
    __syncthreads();
    return nonfinite != 0;
  };
  if (tid == 0) nonfinite = 0;  // ordered by the loop's first barrier
  // A workgroup whose tiles hold an infinite or NaN element (rare) runs
  // the loop again with the cross terms masked.
  if (run(std::false_type{})) {
    __syncthreads();  // every wave has read the flag
    run(std::true_type{});
  }
  if constexpr (KS > 1) {
    // Every wave is past the loop's last barrier: the stages are free.
    // Groups 1.. write their partial tiles (lane-linear per accumulator
    // register), group 0 adds them in group order and stores.
    constexpr int kPart = WM * WN * FM * FN * 16 * 64;  // floats per group
    static_assert((KS - 1) * kPart * 4 <= 2 * kStage * 2,
                  "partial tiles fit the stages");
    float* const red = reinterpret_cast<float*>(lds);
    auto at = [&](int q, int i, int j, int r) {
      return (q - 1) * kPart + (((wv * FM + i) * FN + j) * 16 + r) * 64 +
             lane;
    };
    if (ks != 0) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) red[at(ks, i, j, r)] = acc[i][j][r];
    }
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int q = 1; q < KS; ++q)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += red[at(q, i, j, r)];
  }
  store_direct<float, BM, BN, WM, WN, MC>(g, acc, m0, n0, batch, lane, wm,
                                          wn);
}

}  // namespace
}  // namespace qk
