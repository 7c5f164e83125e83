// Quantized prefill GEMM for gfx950: y = x @ w^T with int4 (u32x8) or int8
// (u8 affine, s8 symmetric) weight codes dequantized in registers, straight
// into the MFMA B fragments.
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
//  - BM x BN tiles (BM 256 or 128), K tiles of 64 (one quantization
//    group); every operand
//    reaches LDS by DMA (`buffer_load ... lds`), issued evenly by the
//    waves, in pieces of whole 64- or 128-byte lines (a DMA instruction
//    that touches many lines for few bytes each is what limits a CU's
//    fetch rate, more than the bytes):
//    * A (x rows): S stages (three or four) of BM rows x 128 bytes, one
//      per K tile; 16-byte chunk c of row r in slot c ^ ((r >> 1) & 7).
//      When the BM / 8 instructions of a stage do not split evenly over
//      the waves, the waves short of one issue an out-of-range DMA (zeros,
//      no memory access) into a spare 1 KB, so every wave's memory counter
//      counts the same number per stage.
//    * Codes: blocks of two K tiles, 64 bytes (int4, 128 codes) or 128
//      bytes (int8) per weight row, S / 2 + 1 blocks resident; chunk c of
//      row n in slot c ^ ((n >> 2) & 3) (int4) or c ^ (n & 7) (int8).
//    * Scales and offsets: blocks of eight K tiles, 16 bytes (eight bf16
//      groups) per row each, two blocks resident.
//    A code (scale) block is fetched with the DMA of its first K tile.
//  - Waves WM x WN, each BM / WM rows x 32 FN columns
//    (v_mfma_f32_32x32x16): FM = 8 / WM A fragments (16-byte LDS reads) and
//    FN B fragments per K step of 16. A B fragment is lane l's column
//    n = l % 32 at K 8 (l / 32) .. + 7: that row's code word (int4) or
//    two (int8), the codes converted to f32, one fma each with the row's
//    group scale and offset, and packed to T. Each B
//    fragment feeds FM MFMAs: with WM = 1 the dequantizing VALU work is a
//    third of the MFMA time and no column is dequantized twice in a CU.
//  - One barrier per K tile, as in gemm_dma.h: each wave waits for its own
//    DMA of tile kt + 1 after K step 2; after the barrier the DMA of tile
//    kt + S into the freed stage is issued (with the code or scale block
//    it starts), then the MFMAs of step 3 with the fragment reads of the
//    next tile's step 0.
//  - Split K (ksplit > 1, for grids that would otherwise leave CUs idle):
//    workgroup (tile, z) takes K tiles z G / ksplit .. (z + 1) G / ksplit
//    (whole scale blocks), writes its f32 partial tile to the workspace
//    and counts itself in on the tile's arrival counter (a device-scope
//    atomic, once its stores have completed). The last to arrive sums the ksplit
//    partials in the order z = 0, 1, ... (its own from registers), so the
//    result does not depend on the arrival order, resets the counter to
//    zero for the next launch and stores the tile with the epilogue.
#pragma once

#include "gemm_common.h"

namespace qk {
namespace {

template <typename T, int PACK, int BM_, int BN, int WM, int FN, int S>
struct QDma {
  static constexpr bool kInt4 = PACK == QK_PACK_U32X8;
  static constexpr int BM = BM_, BK = 64, WTM = BM / WM, FM = WTM / 32;
  static constexpr int WTN = 32 * FN, WN = BN / WTN, NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int CB = 2;           // K tiles per code block
  static constexpr int SBK = 8;          // K tiles per scale block
  static constexpr int kA = BM * 128;    // A stage bytes
  static constexpr int kCT = kInt4 ? 32 : 64;  // code bytes per row, K tile
  static constexpr int kCRow = kCT * CB; // code bytes per row per block
  static constexpr int kCLanes = kCRow / 16;   // lanes per row in a DMA
  static constexpr int kCRows = 64 / kCLanes;  // rows per code DMA
  static constexpr int kCB = BN * kCRow; // code block bytes
  static constexpr int kSB = BN * 16;    // scale (offset) block bytes
  // Code blocks resident: block c is fetched at tile 2 c - S into the
  // buffer of block c - NCB, whose last chunk reads (for tile
  // 2 (c - NCB) + 1, at the end of tile 2 (c - NCB)) must come before that
  // tile's barrier: NCB > S / 2. Scale blocks: 8 NSB > S + 6, so two.
  static constexpr int NCB = S / 2 + 1;
  static constexpr int kAI = BM / 8;        // 1 KB A DMA instructions
  static constexpr int kNA = (kAI + NW - 1) / NW;  // per wave
  static constexpr bool kPad = kAI % NW != 0;
  static constexpr int kCOff = S * kA;
  static constexpr int kSOff = kCOff + NCB * kCB;
  static constexpr int kDOff = kSOff + 4 * kSB;  // 2 blocks x (s, b)
  static constexpr int kBytes = kDOff + (kPad ? 1024 : 0);
  static constexpr int kCI = kCB / 1024;    // code block instructions
  static constexpr int kSI = kSB / 1024;    // scale (offset) block instr.
  static_assert(BN % WTN == 0 && BN % 64 == 0, "tile split");
  static_assert(BM % (32 * WM) == 0, "wave rows");
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

// Eight int8 codes (bytes 0..3 of w0, then of w1, in K order) as
// T(f32(q) * s + b); u8 codes convert with one v_cvt_f32_ubyteN each, s8
// codes are sign-extended first.
template <typename T, int PACK>
__device__ __forceinline__ typename Frag<T>::type DequantBytes(uint32_t w0,
                                                               uint32_t w1,
                                                               float s,
                                                               float b) {
  typedef T T2 __attribute__((ext_vector_type(2)));
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t w = e < 2 ? w0 : w1;
    const uint32_t b0 = (w >> (16 * (e & 1))) & 0xFFu;
    const uint32_t b1 = (w >> (16 * (e & 1) + 8)) & 0xFFu;
    float q0, q1;
    if constexpr (PACK == QK_PACK_S8_SYM) {
      q0 = static_cast<float>(static_cast<int8_t>(b0));
      q1 = static_cast<float>(static_cast<int8_t>(b1));
    } else {
      q0 = static_cast<float>(b0);
      q1 = static_cast<float>(b1);
    }
    const T2 p = {from_f32<T>(fmaf(q0, s, b)), from_f32<T>(fmaf(q1, s, b))};
    out[e] = __builtin_bit_cast(uint32_t, p);
  }
  return __builtin_bit_cast(typename Frag<T>::type, out);
}

// A lane's codes of one weight row for one K tile: 16 bytes (int4) or 32
// (int8), K 32 (l / 32) .. + 31 of the tile; K step s takes word s (int4)
// or words 2 s and 2 s + 1 (int8).
template <int PACK>
struct QTileCodes {
  static constexpr int kN = PACK == QK_PACK_U32X8 ? 1 : 2;
  u32x4 c[kN];
  template <typename T>
  __device__ __forceinline__ typename Frag<T>::type dq(int s, float sc,
                                                      float bi) const {
    if constexpr (PACK == QK_PACK_U32X8)
      return DequantWord<T>(c[0][s], sc, bi);
    else
      return DequantBytes<T, PACK>(c[kN - 1 > 0 ? s >> 1 : 0][2 * (s & 1)],
                                   c[kN - 1 > 0 ? s >> 1 : 0][2 * (s & 1) + 1],
                                   sc, bi);
  }
};

// f(kt + I, integral_constant<I>) for I = 0 .. N - 1 (the stage index a
// compile-time constant), and the same stopping at the first kt + I past
// kend.
template <int I, int N, typename F>
__device__ __forceinline__ void QTiles(F& f, int kt) {
  if constexpr (I < N) {
    f(kt + I, std::integral_constant<int, I>{});
    QTiles<I + 1, N>(f, kt);
  }
}
template <int I, int N, typename F>
__device__ __forceinline__ void QTilesTail(F& f, int kt, int kend) {
  if constexpr (I < N) {
    if (kt + I < kend) {
      f(kt + I, std::integral_constant<int, I>{});
      QTilesTail<I + 1, N>(f, kt, kend);
    }
  }
}

// MC: M need not be a multiple of BM (A rows past M read zeros through
// the descriptor's extent; their outputs are not stored). K is a multiple
// of 512 (whole scale blocks), and so is every split's K range.
template <typename T, int PACK, int BM, int BN, int WM, int FN, int S,
          bool MC>
__global__ __launch_bounds__((QDma<T, PACK, BM, BN, WM, FN, S>::NT)) void
qgemm_dma_kernel(GemmArgs g) {
  using C = QDma<T, PACK, BM, BN, WM, FN, S>;
  constexpr int FM = C::FM, WN = C::WN, NW = C::NW;
  using F = typename Frag<T>::type;
  using Codes = QTileCodes<PACK>;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::kBytes];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int ntiles = g.tiles_m * g.tiles_n;
  const int G = g.k / 64;  // groups (K tiles) per weight row
  const int splits = g.ksplit;
  const int nwg = ntiles * splits;
  int w = blockIdx.x;
  if ((nwg & 7) == 0) w = (w & 7) * (nwg >> 3) + (w >> 3);
  // Workgroup w = z ntiles + tile takes K range z of the tile, so one
  // XCD's share (consecutive w) takes one K range of neighbouring tiles.
  const int z = w / ntiles;
  const int tile = w - z * ntiles;
  const int kbeg = z * (G / splits), kend = kbeg + G / splits;
  int m0, n0;
  {
    const int gm = g.group_m > 0 ? g.group_m : kGroupM;
    const int group_span = gm * g.tiles_n;
    const int first_m = (tile / group_span) * gm;
    const int gsz = min(g.tiles_m - first_m, gm);
    m0 = (first_m + (tile % group_span) % gsz) * BM;
    n0 = ((tile % group_span) / gsz) * BN;
  }

  DmaRsrc ra, rc, rs, rb;
  ra.make(g.a, static_cast<long long>(g.m) * g.lda * sizeof(T));
  rc.make(g.b, static_cast<long long>(g.n) * g.qrow_bytes);
  rs.make(g.qscale, static_cast<long long>(g.n) * G * 2);
  // An extent of 0 reads zeros: no offsets.
  rb.make(g.qbias, g.qhas_bias ? static_cast<long long>(g.n) * G * 2 : 0);

  // The DMA of K tile kt: its A stage (instruction d fills rows 8 d ..
  // 8 d + 7), then the code block it starts (instruction j: kCRows rows,
  // kCLanes 16-byte chunks each) and the scale and offset block it starts
  // (instruction j: 64 rows, 16 bytes each). Wave w takes every NW-th
  // instruction of each kind. `a_st` is the stage's LDS address.
  auto issue = [&](unsigned char* a_st, int kt) {
    const int k0 = kt * 64;
#pragma unroll
    for (int t = 0; t < C::kNA; ++t) {
      const int d = wave + NW * t;
      if (C::kPad && d >= C::kAI) {
        ra.dma(smem + C::kDOff, 0x7FFF0000, 0);  // zeros, counted alike
      } else {
        const int row = 8 * d + lane / 8;
        const int chunk = (lane % 8) ^ ((row >> 1) & 7);
        ra.dma(a_st + d * 1024,
               ((m0 + row) * g.lda + k0 + chunk * 8) *
                   static_cast<int>(sizeof(T)),
               0);
      }
    }
    if (kt % C::CB == 0) {
      unsigned char* cb =
          smem + C::kCOff + ((kt / C::CB) % C::NCB) * C::kCB;
#pragma unroll
      for (int t = 0; t < (C::kCI + NW - 1) / NW; ++t) {
        const int j = wave + NW * t;
        if (j >= C::kCI) break;
        const int row = C::kCRows * j + lane / C::kCLanes;
        const int chunk =
            (lane % C::kCLanes) ^ (C::kInt4 ? (row >> 2) & 3 : row & 7);
        rc.dma(cb + j * 1024,
               (n0 + row) * g.qrow_bytes + kt * C::kCT + chunk * 16, 0);
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
  // elements of a row are one contiguous run of codes (16 bytes of int4,
  // 32 of int8), read once per tile.
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
  // This lane's codes of fragment j's column in K tile kt: 16-byte chunk
  // 2 (kt % 2) + l / 32 of the row's int4 block, or chunks
  // 4 (kt % 2) + 2 (l / 32) and the next of its int8 block.
  auto codes = [&](int j, int kt) {
    const int n = wn * C::WTN + 32 * j + (lane & 31);
    const unsigned char* row =
        smem + C::kCOff + ((kt / C::CB) % C::NCB) * C::kCB + n * C::kCRow;
    Codes cw;
    if constexpr (C::kInt4) {
      const int c = (kt % C::CB) * 2 + (lane >> 5);
      cw.c[0] = *reinterpret_cast<const u32x4*>(row +
                                                ((c ^ ((n >> 2) & 3)) << 4));
    } else {
      const int c = (kt % C::CB) * 4 + 2 * (lane >> 5);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        cw.c[h] = *reinterpret_cast<const u32x4*>(
            row + (((c + h) ^ (n & 7)) << 4));
    }
    return cw;
  };
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  auto stage = [&](int i) { return smem + i * C::kA; };
#pragma unroll
  for (int t = 0; t < S; ++t) issue(stage(t), kbeg + t);
  // Tile kbeg (with its blocks) has landed: the A DMAs of the next S - 1
  // tiles may still be in flight (the waves' block DMAs, issued with some
  // tiles and not others, only add to what is waited for, never to what is
  // left outstanding).
  __builtin_amdgcn_s_waitcnt(VmcntImm((S - 1) * C::kNA));
  __syncthreads();
  F fa[2][FM], fb[2][FN];
  float scl[FN], bil[FN];
  Codes cw[FN];  // code runs of the current tile
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    sb(j, kbeg, &scl[j], &bil[j]);
    cw[j] = codes(j, kbeg);
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = frag_a(stage(0), i, 0);
#pragma unroll
  for (int j = 0; j < FN; ++j)
    fb[0][j] = cw[j].template dq<T>(0, scl[j], bil[j]);

  constexpr int kReads = FM;
  // K tile kt from A stage SLOT = (kt - kbeg) % S; tile kt + 1 is in stage
  // (SLOT + 1) % S; after the barrier tile kt + S goes into stage SLOT.
  auto tile_step = [&](int kt, auto slot_c) {
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
        fb[fn][j] = cw[j].template dq<T>(s + 1, scl[j], bil[j]);
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
    issue(cs, min(kt + S, kend - 1));
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
      fb[0][j] = cw[j].template dq<T>(0, scl[j], bil[j]);
  };
  static_assert(S >= 3, "at least three stages");
  int kt = kbeg;
  for (; kt + S <= kend; kt += S) QTiles<0, S>(tile_step, kt);
  QTilesTail<0, S - 1>(tile_step, kt, kend);
  // No DMA may still be writing this workgroup's LDS when it ends.
  __builtin_amdgcn_s_waitcnt(VmcntImm(0));
  split_k_store<T, BM, BN, WM, WN, MC, C::NT>(
      g, acc, tile, z, m0, n0, tid, lane, wm, wn,
      reinterpret_cast<uint32_t*>(smem));
}


}  // namespace
}  // namespace qk
