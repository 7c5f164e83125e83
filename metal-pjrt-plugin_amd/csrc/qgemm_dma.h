// Quantized prefill GEMM for gfx950: y = x @ w^T with int4 (u32x8) weight
// codes dequantized in registers, straight into the MFMA B fragments.
//
// Replaces the reference's path for rows beyond ROWS_MAX (4) in linear()
// (examples/llm/qwen3.py:218-230): w = dequantize(w, x.dtype)
// (qwen3.py:199-207), then einsum("...i,oi->...o", x, w). The dequantized
// weights exist only in registers: each B fragment is T(f32(q) * f32(s) +
// f32(b)) (the canonical rounding of qk$dequantize; q * s is exact in f32,
// so one fma rounds as the unfused form), so the result is the dense GEMM
// of x with the dequantized weights, accumulated in f32.
//
// Layout and schedule (the interior-tile scheme of gemm_dma.h):
//  - 256 x BN tiles, K tiles of 64 (one quantization group); every operand
//    reaches LDS by DMA (`buffer_load ... lds`), issued evenly by the
//    waves, in pieces of whole 64- or 128-byte lines (a DMA instruction
//    that touches many lines for few bytes each is what limits a CU's
//    fetch rate, more than the bytes):
//    * A (x rows): S stages (three or four) of 256 rows x 128 bytes, one
//      per K tile; 16-byte chunk c of row r in slot c ^ ((r >> 1) & 7).
//    * Codes: blocks of two K tiles, 64 bytes (128 codes) per weight row,
//      S / 2 + 1 blocks resident; chunk c of row n in slot c ^ ((n >> 2) & 3).
//    * Scales and offsets: blocks of eight K tiles, 16 bytes (eight bf16
//      groups) per row each, two blocks resident.
//    A code (scale) block is fetched with the DMA of its first K tile.
//  - Waves WM x WN, each 256 / WM rows x 32 FN columns
//    (v_mfma_f32_32x32x16): FM = 8 / WM A fragments (16-byte LDS reads) and
//    FN B fragments per K step of 16. A B fragment is lane l's column
//    n = l % 32 at K 8 (l / 32) .. + 7: one 32-bit LDS read of that row's
//    code word, its nibbles split into bytes and converted to f32, one fma
//    each with the row's group scale and offset, and packed to T. Each B
//    fragment feeds FM MFMAs: with WM = 1 the dequantizing VALU work is a
//    third of the MFMA time and no column is dequantized twice in a CU.
//  - One barrier per K tile, as in gemm_dma.h: each wave waits for its own
//    DMA of tile kt + 1 after K step 2; after the barrier the DMA of tile
//    kt + S into the freed stage is issued (with the code or scale block
//    it starts), then the MFMAs of step 3 with the fragment reads of the
//    next tile's step 0.
#pragma once

#include "gemm_common.h"

namespace qk {
namespace {

template <typename T, int BN, int WM, int FN, int S>
struct QDma {
  static constexpr int BM = 256, BK = 64, WTM = BM / WM, FM = WTM / 32;
  static constexpr int WTN = 32 * FN, WN = BN / WTN, NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int CB = 2;           // K tiles per code block
  static constexpr int SBK = 8;          // K tiles per scale block
  static constexpr int kA = BM * 128;    // A stage bytes
  static constexpr int kCRow = 32 * CB;  // code bytes per row per block
  static constexpr int kCB = BN * kCRow; // code block bytes
  static constexpr int kSB = BN * 16;    // scale (offset) block bytes
  // Code blocks resident: block c is fetched at tile 2 c - S into the
  // buffer of block c - NCB, whose last chunk reads (for tile
  // 2 (c - NCB) + 1, at the end of tile 2 (c - NCB)) must come before that
  // tile's barrier: NCB > S / 2. Scale blocks: 8 NSB > S + 6, so two.
  static constexpr int NCB = S / 2 + 1;
  static constexpr int kCOff = S * kA;
  static constexpr int kSOff = kCOff + NCB * kCB;
  static constexpr int kBytes = kSOff + 4 * kSB;  // 2 blocks x (s, b)
  static constexpr int kAI = BM / 8;        // 1 KB A DMA instructions
  static constexpr int kCI = kCB / 1024;    // code block instructions
  static constexpr int kSI = kSB / 1024;    // scale (offset) block instr.
  static constexpr int kNA = kAI / NW;      // A instructions per wave
  static_assert(BN % WTN == 0 && BN % 64 == 0, "tile split");
  static_assert(kAI % NW == 0, "every wave issues the same A DMAs");
  static_assert(kBytes <= 160 * 1024, "LDS");
};

// Eight int4 codes (one u32x8 word: code e in bits 4e .. 4e + 3) as
// T(f32(q) * s + b): the even codes are the bytes of w & 0x0F0F0F0F, the
// odd ones those of (w >> 4) & 0x0F0F0F0F, each converted by one
// v_cvt_f32_ubyteN; one fma each; one v_cvt_pk per pair. The two masks
// are opaque to the compiler (inline asm), which would otherwise fold
// them into a shift and mask per code.
template <typename T>
__device__ __forceinline__ typename Frag<T>::type DequantWord(uint32_t w,
                                                              float s,
                                                              float b) {
  uint32_t lo, hi;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(w));
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(hi) : "v"(w >> 4));
  typedef T T2 __attribute__((ext_vector_type(2)));
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float q0 = static_cast<float>((lo >> (8 * e)) & 0xFFu);
    const float q1 = static_cast<float>((hi >> (8 * e)) & 0xFFu);
    const T2 p = {from_f32<T>(fmaf(q0, s, b)), from_f32<T>(fmaf(q1, s, b))};
    out[e] = __builtin_bit_cast(uint32_t, p);
  }
  return __builtin_bit_cast(typename Frag<T>::type, out);
}

// MC: M need not be a multiple of 256 (A rows past M read zeros through
// the descriptor's extent; their outputs are not stored). K is a multiple
// of 512 (whole scale blocks).
template <typename T, int BN, int WM, int FN, int S, bool MC>
__global__ __launch_bounds__((QDma<T, BN, WM, FN, S>::NT)) void qgemm_dma_kernel(
    GemmArgs g) {
  using C = QDma<T, BN, WM, FN, S>;
  constexpr int FM = C::FM, WN = C::WN, NW = C::NW;
  using F = typename Frag<T>::type;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::kBytes];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int nwg = g.tiles_m * g.tiles_n;
  int bid = blockIdx.x;
  if ((nwg & 7) == 0) bid = (bid & 7) * (nwg >> 3) + (bid >> 3);
  const int group_span = kGroupM * g.tiles_n;
  const int first_m = (bid / group_span) * kGroupM;
  const int gsz = min(g.tiles_m - first_m, kGroupM);
  const int tm = first_m + (bid % group_span) % gsz;
  const int tn = (bid % group_span) / gsz;
  const int m0 = tm * C::BM, n0 = tn * BN;
  const int G = g.k / 64;  // groups (K tiles) per weight row

  DmaRsrc ra, rc, rs, rb;
  ra.make(g.a, static_cast<long long>(g.m) * g.lda * sizeof(T));
  rc.make(g.b, static_cast<long long>(g.n) * g.qrow_bytes);
  rs.make(g.qscale, static_cast<long long>(g.n) * G * 2);
  // An extent of 0 reads zeros: no offsets.
  rb.make(g.qbias, g.qhas_bias ? static_cast<long long>(g.n) * G * 2 : 0);

  // The DMA of K tile kt: its A stage (instruction d fills rows 8 d ..
  // 8 d + 7), then the code block it starts (instruction j: rows 16 j ..
  // 16 j + 15, four 16-byte chunks each) and the scale and offset block it
  // starts (instruction j: 64 rows, 16 bytes each). Wave w takes every
  // NW-th instruction of each kind. `a_st` is the stage's LDS address.
  auto issue = [&](unsigned char* a_st, int kt) {
    const int k0 = kt * 64;
#pragma unroll
    for (int t = 0; t < C::kNA; ++t) {
      const int d = wave + NW * t;
      const int row = 8 * d + lane / 8;
      const int chunk = (lane % 8) ^ ((row >> 1) & 7);
      ra.dma(a_st + d * 1024,
             ((m0 + row) * g.lda + k0 + chunk * 8) *
                 static_cast<int>(sizeof(T)),
             0);
    }
    if (kt % C::CB == 0) {
      unsigned char* cb =
          smem + C::kCOff + ((kt / C::CB) % C::NCB) * C::kCB;
#pragma unroll
      for (int t = 0; t < (C::kCI + NW - 1) / NW; ++t) {
        const int j = wave + NW * t;
        if (j >= C::kCI) break;
        const int row = 16 * j + lane / 4;
        const int chunk = (lane % 4) ^ ((row >> 2) & 3);
        rc.dma(cb + j * 1024,
               (n0 + row) * g.qrow_bytes + k0 / 2 + chunk * 16, 0);
      }
    }
    if (kt % C::SBK == 0) {
      unsigned char* sb =
          smem + C::kSOff + ((kt / C::SBK) & 1) * 2 * C::kSB;
#pragma unroll
      for (int t = 0; t < (2 * C::kSI + NW - 1) / NW; ++t) {
        const int j = wave + NW * t;  // scales first, then offsets
        if (j >= 2 * C::kSI) break;
        const bool off = j >= C::kSI;
        const int jj = off ? j - C::kSI : j;
        const int voff = ((n0 + 64 * jj + lane) * G + kt) * 2;
        if (off)
          rb.dma(sb + C::kSB + jj * 1024, voff, 0);
        else
          rs.dma(sb + jj * 1024, voff, 0);
      }
    }
  };
  // Within a K tile the K steps are taken in a permuted order (the sum
  // over K does not depend on it): K step s gives lane half h = l / 32 the
  // eight K elements 32 h + 8 s .. + 7, so over the four steps a lane's B
  // elements of a row are one 16-byte chunk of codes (32 h / 2 bytes on),
  // read once per tile.
  auto frag_a = [&](const unsigned char* st, int i, int s) {
    const int r = wm * C::WTM + i * 32 + (lane & 31);
    const int c = 4 * (lane >> 5) + s;
    return *reinterpret_cast<const F*>(st + r * 128 +
                                       ((c ^ ((r >> 1) & 7)) << 4));
  };
  // The scale and offset of this lane's column in fragment j, K tile kt.
  auto sb = [&](int j, int kt, float* sc, float* bi) {
    const int n = wn * C::WTN + 32 * j + (lane & 31);
    const unsigned char* p = smem + C::kSOff +
                             ((kt / C::SBK) & 1) * 2 * C::kSB + n * 16 +
                             (kt % C::SBK) * 2;
    *sc = __uint_as_float(static_cast<uint32_t>(
                              *reinterpret_cast<const uint16_t*>(p))
                          << 16);
    *bi = __uint_as_float(static_cast<uint32_t>(
                              *reinterpret_cast<const uint16_t*>(p + C::kSB))
                          << 16);
  };
  // This lane's 16-byte code chunk of fragment j's column in K tile kt
  // (chunk 2 (kt % 2) + l / 32 of the row in code block kt / 2).
  auto codes = [&](int j, int kt) {
    const int n = wn * C::WTN + 32 * j + (lane & 31);
    const int c = (kt % C::CB) * 2 + (lane >> 5);
    return *reinterpret_cast<const u32x4*>(
        smem + C::kCOff + ((kt / C::CB) % C::NCB) * C::kCB + n * C::kCRow +
        ((c ^ ((n >> 2) & 3)) << 4));
  };
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int ktiles = G;  // >= 8
  auto stage = [&](int i) { return smem + i * C::kA; };
#pragma unroll
  for (int t = 0; t < S; ++t) issue(stage(t), t);
  // Tile 0 (with its blocks) has landed: the A DMAs of tiles 1 .. S - 1
  // may still be in flight (the waves' block DMAs, issued with some tiles
  // and not others, only add to what is waited for, never to what is left
  // outstanding).
  __builtin_amdgcn_s_waitcnt(VmcntImm((S - 1) * C::kNA));
  __syncthreads();
  F fa[2][FM], fb[2][FN];
  float scl[FN], bil[FN];
  u32x4 cw[FN];  // code chunks of the current tile
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    sb(j, 0, &scl[j], &bil[j]);
    cw[j] = codes(j, 0);
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = frag_a(stage(0), i, 0);
#pragma unroll
  for (int j = 0; j < FN; ++j) fb[0][j] = DequantWord<T>(cw[j][0], scl[j], bil[j]);

  constexpr int kReads = FM;
  // K tile kt from A stage SLOT = kt % S; tile kt + 1 is in stage
  // (SLOT + 1) % S; after the barrier tile kt + S goes into stage SLOT.
  auto tile = [&](int kt, auto slot_c) {
    constexpr int SLOT = decltype(slot_c)::value;
    unsigned char* cs = stage(SLOT);
    unsigned char* ns = stage((SLOT + 1) % S);
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      const int fc = s & 1, fn = fc ^ 1;
#pragma unroll
      for (int i = 0; i < FM; ++i) fa[fn][i] = frag_a(cs, i, s + 1);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[fn][j] = DequantWord<T>(cw[j][s + 1], scl[j], bil[j]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], fa[fc][i], fb[fc][j]);
#pragma unroll
      for (int q = 0; q < FM * FN; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (q < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    // Tile kt + 1 has landed (own DMA: vmcnt; everyone's: barrier); after
    // the barrier nobody reads cs (step 3 runs from registers), nor the
    // code and scale blocks of tiles before kt + 1.
    __builtin_amdgcn_s_waitcnt(VmcntImm((S - 2) * C::kNA));
    __syncthreads();
    // (Past the last tile the last one is fetched again into the free
    // stage, so that every wait above counts the same DMAs.)
    issue(cs, min(kt + S, ktiles - 1));
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      sb(j, kt + 1, &scl[j], &bil[j]);
      cw[j] = codes(j, kt + 1);
    }
#pragma unroll
    for (int q = 0; q < FM * FN; ++q) {
      const int i = q / FN, j = q % FN;
      mma(acc[i][j], fa[1][i], fb[1][j]);
      if (q < FM) fa[0][q] = frag_a(ns, q, 0);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j)
      fb[0][j] = DequantWord<T>(cw[j][0], scl[j], bil[j]);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  static_assert(S == 3 || S == 4, "unrolled for three or four stages");
  int kt = 0;
  for (; kt + S <= ktiles; kt += S) {
    tile(kt, I0{});
    tile(kt + 1, I1{});
    tile(kt + 2, I2{});
    if constexpr (S == 4) tile(kt + 3, I3{});
  }
  if (kt < ktiles) tile(kt, I0{});
  if (kt + 1 < ktiles) tile(kt + 1, I1{});
  if constexpr (S == 4) {
    if (kt + 2 < ktiles) tile(kt + 2, I2{});
  }
  // No DMA may still be writing this workgroup's LDS when it ends.
  __builtin_amdgcn_s_waitcnt(VmcntImm(0));
  store_direct<T, C::BM, BN, WM, WN, MC>(g, acc, m0, n0, 0, lane, wm, wn);
}

}  // namespace
}  // namespace qk
