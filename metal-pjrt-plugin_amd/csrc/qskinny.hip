// Quantized matmul for a few rows of x (5 <= M <= 32 as routed; the kernels
// take 1..32): y[M, N] = x[M, K] W^T with W int4 (u32x8 words), bf16 x /
// scale / offset, group size 64: the batched-decode and short-prefill
// shapes. The reference's linear() (examples/llm/qwen3.py:215-230)
// dequantizes W to x's type for more than ROWS_MAX = 4 rows and multiplies;
// this kernel keeps the codes factored as its _matvec_int4 does
// (qwen3.py:233-267: y = s * sum(x q) + b * sum(x) per group), which skips
// the bf16 rounding of the weights and agrees with the dequantized product
// within that rounding.
//
// Design (MI355X-first). The work is HBM-bound (N K / 2 bytes of codes
// against 2 M N K flops), so the codes are streamed once:
//  - A workgroup owns NR = 16 NB weight rows and splits K over its KW waves
//    (reduced through LDS at the end). Each wave walks its K slice in
//    sub-chunks of CG groups: the sub-chunk's codes are read as contiguous
//    row segments (32 CG bytes per row, 16 bytes per lane) and reach the
//    MFMA layout through a wave-private LDS buffer, and so does the
//    sub-chunk's x (16 bytes per lane along a row: with one row per lane,
//    as the MFMA layout has it, every four lanes would touch four rows,
//    which measured ~4x slower to issue) (a wave's LDS
//    operations run in order, so each sub-chunk is written over the last
//    after its final read). Scales, offsets and the sub-chunk's x travel
//    with the codes: the next sub-chunk is requested as a whole while the
//    current one is computed, in consumption order, so the in-order memory
//    counter never waits for data that is not needed yet. Sub-chunks past
//    a wave's slice are requested through out-of-range offsets (zeros, no
//    memory traffic), so no load is conditional.
//  - v_mfma_f32_16x16x32_bf16 with A = 16 rows of x and B = 16 weight rows.
//    Lane l takes the code words 2 (l / 16) and 2 (l / 16) + 1 of a group
//    (one 8-byte LDS read) for the group's two MFMAs, so every MFMA
//    multiplies K values of one group only and the group's scale can be
//    applied after it. x is loaded as the matching 32 bytes per lane.
//  - Codes become bf16 pairs (128 + q_a, 128 + q_b) with one v_and_or_b32
//    (nibbles s and s + 4 of a word; 0x4300 | q is exactly 128 + q); x is
//    permuted with v_perm_b32 into the same K order.
//  - Per group: tmp = sum x (128 + q) and xs = sum x (one MFMA against a
//    constant 1.0 operand, which lands xs in the accumulator layout), then
//    acc += s tmp + (b - 128 s) xs.
//  - Rows past M or N read zeros through buffer descriptors and are not
//    stored.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct SkArgs {
  const void* x;
  const void* codes;
  const void* scales;
  const void* biases;
  void* y;
  int m, n, k;
  int groups;  // k / 64
  int has_bias;
  int chunks;  // 256-K sub-chunks per wave
  uint32_t* status;  // device status word (producer / consumer kernels)
  int spin_limit;    // polls before a flag wait gives up
};

constexpr int kNonTemporal = 2;
constexpr int kOut = 0x7FFF0000;             // an offset past every extent

__device__ __forceinline__ __amdgpu_buffer_rsrc_t Rsrc(const void* p,
                                                       int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                           bytes, 0x00020000);
}

// x (8 consecutive bf16, as loaded) -> the pair order of a code word:
// (x0, x4), (x1, x5), (x2, x6), (x3, x7).
__device__ __forceinline__ bf16x8 XPairs(const u32x4& v) {
  constexpr uint32_t kLoLo = 0x05040100u, kHiHi = 0x07060302u;
  const u32x4 p = {__builtin_amdgcn_perm(v[2], v[0], kLoLo),
                   __builtin_amdgcn_perm(v[2], v[0], kHiHi),
                   __builtin_amdgcn_perm(v[3], v[1], kLoLo),
                   __builtin_amdgcn_perm(v[3], v[1], kHiHi)};
  return __builtin_bit_cast(bf16x8, p);
}

// One u32x8 code word -> bf16 (128 + q) in the same order.
__device__ __forceinline__ bf16x8 CodePairs(uint32_t w, uint32_t mask,
                                            uint32_t bias) {
  const uint64_t v = w;  // the high half is never used
  const u32x4 p = {(w & mask) | bias,
                   (static_cast<uint32_t>(shr64<4>(v)) & mask) | bias,
                   (static_cast<uint32_t>(shr64<8>(v)) & mask) | bias,
                   (static_cast<uint32_t>(shr64<12>(v)) & mask) | bias};
  return __builtin_bit_cast(bf16x8, p);
}

// 8 bytes of int8 codes -> bf16 (exact: integers up to 256 are bf16
// values); signed symmetric codes are first flipped to q + 128.
template <int PACK>
__device__ __forceinline__ bf16x8 CodeBytes(uint32_t w0, uint32_t w1) {
  if (PACK == QK_PACK_S8_SYM) w0 ^= 0x80808080u, w1 ^= 0x80808080u;
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = from_f32<bf16>(static_cast<float>((w0 >> (8 * e)) & 0xFFu));
    r[4 + e] = from_f32<bf16>(static_cast<float>((w1 >> (8 * e)) & 0xFFu));
  }
  return r;
}

// LDS bytes of qmm_skinny_kernel (per wave: codes, scales/offsets and x
// buffers; after the loop, the KW partial tiles).
template <int PACK, int MB, int NB, int KW, int CG>
constexpr int SkinnyLdsBytes() {
  constexpr int GB = PACK == QK_PACK_U32X8 ? 32 : 64;
  constexpr int NR = 16 * NB;
  constexpr int wave = NR * (GB * CG + 16) + 2 * NR * CG * 2 +
                       16 * MB * (CG * 128 + 16);
  constexpr int part = KW * (16 * MB) * (NR + 1) * 4;
  return KW * wave > part ? KW * wave : part;
}
constexpr int kMaxLds = 160 * 1024;

template <int PACK, int MB, int NB, int KW, int CG>
__global__ __launch_bounds__(KW * 64) void qmm_skinny_kernel(SkArgs a) {
  constexpr bool kInt4 = PACK == QK_PACK_U32X8;
  constexpr int GB = kInt4 ? 32 : 64;   // code bytes per group per row
  constexpr int NR = 16 * NB;           // weight rows per workgroup
  constexpr int SEG = GB * CG;          // code bytes per row per sub-chunk
  constexpr int LPR = SEG / 16;         // lanes per row in a code load
  constexpr int RPL = 64 / LPR;         // rows per code load
  constexpr int CL = NR / RPL;          // code loads per sub-chunk
  constexpr int kRow = SEG + 16;        // LDS row stride (padded)
  constexpr int kBuf = NR * kRow;
  // x of one sub-chunk (16 MB rows x CG groups of 128 bytes) is loaded
  // row-contiguously (consecutive lanes, consecutive 16 bytes of one row)
  // and reaches the MFMA layout through the wave's LDS buffer, rows padded
  // by 16 bytes (the 16 rows a fragment read touches fall in distinct
  // banks).
  constexpr int XB = CG * 128;          // x bytes per row per sub-chunk
  constexpr int XLPR = XB / 16;         // lanes per row in an x load
  constexpr int XRPL = 64 / XLPR;       // rows per x load
  constexpr int XL = 16 * MB / XRPL;    // x loads per sub-chunk
  constexpr int kXRow = XB + 16;
  constexpr int kXBuf = 16 * MB * kXRow;
  constexpr int kWaveBytes = kBuf + 2 * NR * CG * 2 + kXBuf;
  static_assert(XL >= 1 && 64 % XLPR == 0, "x tile");
  static_assert(SkinnyLdsBytes<PACK, MB, NB, KW, CG>() <= kMaxLds, "LDS");
  constexpr int kPartBytes = KW * (16 * MB) * (NR + 1) * 4;
  static_assert(CL >= 1 && NR % RPL == 0, "tile");
  __shared__ __attribute__((aligned(16)))
  unsigned char lds[KW * kWaveBytes > kPartBytes ? KW * kWaveBytes
                                                 : kPartBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q16 = lane >> 4, l16 = lane & 15;
  const int n0 = blockIdx.x * NR;
  const int G = a.groups;
  unsigned char* const code_buf = lds + wave * kWaveBytes;
  uint16_t* const sb_buf = reinterpret_cast<uint16_t*>(code_buf + kBuf);
  unsigned char* const x_buf = code_buf + kBuf + 2 * NR * CG * 2;

  const int row_bytes = kInt4 ? a.k / 2 : a.k;
  const auto crs = Rsrc(a.codes, a.n * row_bytes);
  const auto xrs = Rsrc(a.x, a.m * a.k * 2);
  const auto srs = Rsrc(a.scales, a.n * G * 2);
  const auto brs = Rsrc(a.biases, a.has_bias ? a.n * G * 2 : 0);

  // Code loads: load i, lane l -> row RPL i + l / LPR, 16 bytes at
  // 16 (l % LPR) of the row's sub-chunk segment.
  int cvo[CL];
#pragma unroll
  for (int i = 0; i < CL; ++i) {
    const int r = n0 + RPL * i + lane / LPR;
    cvo[i] = r < a.n ? r * row_bytes + 16 * (lane % LPR) : kOut;
  }
  // Scale/offset loads: lane l < NR loads the CG scales and the CG offsets
  // of row l (two loads; one descriptor per array).
  const bool sb_lane = lane < NR;
  const int sb_row = n0 + lane;
  const int svo = (sb_lane && sb_row < a.n) ? sb_row * G * 2 : kOut;
  // x loads: load i, lane l -> row XRPL i + l / XLPR, 16 bytes at
  // 16 (l % XLPR) of the row's sub-chunk segment.
  int xvo[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int r = XRPL * i + lane / XLPR;
    xvo[i] = r < a.m ? r * a.k * 2 + 16 * (lane % XLPR) : kOut;
  }

  struct Chunk {
    u32x4 c[CL];
    uint32_t s[CG / 2], b[CG / 2];
    u32x4 x[XL];
  };
  // `skip`: sub-chunks past the slice read zeros (offsets past the extents).
  auto load = [&](int ch, bool skip, Chunk& t) {
    const int oob = skip ? kOut : 0;
#pragma unroll
    for (int i = 0; i < CL; ++i)
      t.c[i] = __builtin_amdgcn_raw_buffer_load_b128(
          crs, cvo[i] + oob, ch * SEG, kNonTemporal);
    if constexpr (CG == 4) {
      const u32x2 vs = __builtin_amdgcn_raw_buffer_load_b64(srs, svo + oob,
                                                            ch * 8, 0);
      const u32x2 vb = __builtin_amdgcn_raw_buffer_load_b64(brs, svo + oob,
                                                            ch * 8, 0);
      t.s[0] = vs[0], t.s[1] = vs[1], t.b[0] = vb[0], t.b[1] = vb[1];
    } else {
      t.s[0] = __builtin_amdgcn_raw_buffer_load_b32(srs, svo + oob, ch * 4, 0);
      t.b[0] = __builtin_amdgcn_raw_buffer_load_b32(brs, svo + oob, ch * 4, 0);
    }
#pragma unroll
    for (int i = 0; i < XL; ++i)
      t.x[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xvo[i] + oob,
                                                     ch * XB, 0);
  };

  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint32_t kMask = vgpr_const(0x000F000Fu);
  const uint32_t kBias = vgpr_const(0x43004300u);
  const bf16x8 ones = __builtin_bit_cast(
      bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

  auto process = [&](const Chunk& t) {
    // codes and scales into the wave's LDS buffer
#pragma unroll
    for (int i = 0; i < CL; ++i)
      *reinterpret_cast<u32x4*>(code_buf + (RPL * i + lane / LPR) * kRow +
                                16 * (lane % LPR)) = t.c[i];
    if (sb_lane) {  // [scales | offsets][row][group]
      uint32_t* ds = reinterpret_cast<uint32_t*>(sb_buf + lane * CG);
      uint32_t* db = reinterpret_cast<uint32_t*>(sb_buf + (NR + lane) * CG);
#pragma unroll
      for (int h = 0; h < CG / 2; ++h) ds[h] = t.s[h], db[h] = t.b[h];
    }
    // x rows into the wave's x buffer (after this wave's reads of the
    // previous sub-chunk: a wave's LDS operations run in order)
#pragma unroll
    for (int i = 0; i < XL; ++i)
      *reinterpret_cast<u32x4*>(x_buf + (XRPL * i + lane / XLPR) * kXRow +
                                16 * (lane % XLPR)) = t.x[i];
    // Every LDS read of the sub-chunk is issued before any of it is used:
    // one LDS round trip per sub-chunk instead of one per group and row
    // block.
    u32x4 xv[CG][MB][2];
#pragma unroll
    for (int gg = 0; gg < CG; ++gg)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
          xv[gg][mb][t2] = *reinterpret_cast<const u32x4*>(
              x_buf + (16 * mb + l16) * kXRow + gg * 128 + 32 * q16 + 16 * t2);
    using CodeT = typename std::conditional<kInt4, u32x2, u32x4>::type;
    CodeT wv[CG][NB];
    uint32_t sv[NB][CG / 2], bv[NB][CG / 2];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int row = 16 * nb + l16;
#pragma unroll
      for (int gg = 0; gg < CG; ++gg)
        wv[gg][nb] = *reinterpret_cast<const CodeT*>(
            code_buf + row * kRow + gg * GB + (kInt4 ? 8 : 16) * q16);
#pragma unroll
      for (int h = 0; h < CG / 2; ++h) {
        sv[nb][h] = reinterpret_cast<const uint32_t*>(sb_buf + row * CG)[h];
        bv[nb][h] =
            reinterpret_cast<const uint32_t*>(sb_buf + (NR + row) * CG)[h];
      }
    }
#pragma unroll
    for (int gg = 0; gg < CG; ++gg) {
      bf16x8 xa[MB][2];
      f32x4 xs[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        xs[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          // int4: x in the pair order of the code words; int8: as loaded
          xa[mb][t2] = kInt4 ? XPairs(xv[gg][mb][t2])
                             : __builtin_bit_cast(bf16x8, xv[gg][mb][t2]);
          xs[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[mb][t2], ones,
                                                           xs[mb], 0, 0, 0);
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        bf16x8 b0, b1;
        if constexpr (kInt4) {
          b0 = CodePairs(wv[gg][nb][0], kMask, kBias);
          b1 = CodePairs(wv[gg][nb][1], kMask, kBias);
        } else {
          b0 = CodeBytes<PACK>(wv[gg][nb][0], wv[gg][nb][1]);
          b1 = CodeBytes<PACK>(wv[gg][nb][2], wv[gg][nb][3]);
        }
        const int sh = 16 * (gg & 1);
        const float sc = __uint_as_float((sv[nb][gg >> 1] >> sh) << 16);
        const float of = __uint_as_float((bv[nb][gg >> 1] >> sh) << 16);
        // int4 and signed int8 codes enter as q + 128
        const float off = PACK == QK_PACK_U8 ? of : of - 128.f * sc;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              xa[mb][0], b0, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[mb][1], b1, tmp, 0,
                                                        0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[mb][nb][r] =
                fmaf(sc, tmp[r], fmaf(off, xs[mb][r], acc[mb][nb][r]));
        }
      }
    }
  };

  // Two sub-chunks in registers: A and B alternate; every load is issued
  // (past the slice as zeros) so the wait counts follow the ping-pong.
  const int kc0 = wave * a.chunks;
  Chunk A, B;
  load(kc0, false, A);
  for (int c = 0; c < a.chunks; c += 2) {
    load(kc0 + c + 1, c + 1 >= a.chunks, B);
    process(A);
    load(kc0 + c + 2, c + 2 >= a.chunks, A);
    if (c + 1 < a.chunks) process(B);
  }

  // Reduce the KW partial tiles and store rows < M, columns < N.
  __syncthreads();
  float* part = reinterpret_cast<float*>(lds);
  constexpr int TM = 16 * MB, TS = NR + 1;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        part[(wave * TM + 16 * mb + 4 * q16 + r) * TS + 16 * nb + l16] =
            acc[mb][nb][r];
  __syncthreads();
  bf16* Y = static_cast<bf16*>(a.y);
  for (int e = threadIdx.x; e < TM * NR; e += KW * 64) {
    const int r = e / NR, c = e % NR;
    if (r >= a.m || n0 + c >= a.n) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < KW; ++w) v += part[(w * TM + r) * TS + c];
    Y[static_cast<long long>(r) * a.n + n0 + c] = from_f32<bf16>(v);
  }
}

// The eight-wave kernel, or null when its LDS would exceed the limit.
template <int PACK, int MB, int NB, int CG>
auto Skinny8() {
  using K = decltype(&qmm_skinny_kernel<PACK, MB, NB, 4, CG>);
  if constexpr (SkinnyLdsBytes<PACK, MB, NB, 8, CG>() <= kMaxLds)
    return static_cast<K>(&qmm_skinny_kernel<PACK, MB, NB, 8, CG>);
  else
    return static_cast<K>(nullptr);
}

// The streamed form for one or two blocks of 16 rows of x and int4
// (u32x8) or int8 (u8, s8) codes, with the loads and the arithmetic in
// different waves. A workgroup owns NR = 16 NB weight rows and all of K,
// cut into items of four groups (K = 256): x (16 MB rows x 512 bytes),
// codes (NR rows x 128 bytes for int4, 256 for int8) and scale / offset
// dwords. int8 takes MB = 1 only (two row blocks of x would not fit the
// registers at 48 weight rows).
//  - Two producer waves move items (the even and the odd ones) from
//    global memory into a ring of S slots in LDS by LDS DMA, each with up
//    to kFly items in flight (three for int4, two for int8: the most the
//    memory counter of one wave, 63 instructions, can tell apart). A producer never computes, so the
//    memory queue stays full.
//  - NC consumer waves (consumer c takes items c, c + NC, ...) read the
//    items from LDS and compute. A consumer never issues a global load,
//    so it never stalls behind a full memory queue.
//  - Hand-off through LDS words: ready[s] = j + 1 once item j has landed
//    in slot s = j % S, freed[s] = j + 1 once its consumer has read it.
//    Every wait is a bounded spin (the kernel ends even if a flag never
//    comes).
// The arithmetic is that of qmm_skinny_kernel with MB = 1; the consumers'
// partial tiles are summed through LDS at the end. Measured against the
// register-staged kernel at M = 16: 12288 x 4096 11.8 vs 12.5 us, 4096 x
// 12288 13.6 vs 14.7 us (int8 at M = 8, 12288 x 4096: 14.8 vs 16.5 us);
// it is used when every workgroup fits on the GPU at once (the lm_head's
// 3166 row blocks run faster on the register-staged kernel, whose
// workgroups overlap one another). MB = 2 takes 17..32 rows of x (x of an
// item 32 rows x 512 bytes).
template <int PACK, int MB, int NB>
constexpr int WsSlotBytes() {
  // x, codes (whole 1 KB DMA instructions), scales and offsets (two dwords
  // per row, whole 256-byte instructions)
  return 8192 * MB +
         (((PACK == QK_PACK_U32X8 ? 128 : 256) * 16 * NB + 1023) / 1024) *
             1024 +
         2 * ((32 * NB + 63) / 64) * 256;
}
constexpr int kWsConsumers = 8, kWsProducers = 2;

template <int PACK, int MB, int NB>
__global__ __launch_bounds__((kWsConsumers + kWsProducers) * 64) void
qmm_ws_kernel(SkArgs a) {
  constexpr bool kInt4 = PACK == QK_PACK_U32X8;
  constexpr int CB = kInt4 ? 128 : 256;        // code bytes per row and item
  constexpr int NC = kWsConsumers, NP = kWsProducers;
  constexpr int NR = 16 * NB;                  // weight rows per workgroup
  constexpr int TS = NR + 1;                   // partial-tile row stride
  constexpr int TM = 16 * MB;                  // rows of x
  constexpr int kCDma = (NR * CB + 1023) / 1024;
  constexpr int kSDma = (NR * 2 + 63) / 64;
  constexpr int kCOff = 8192 * MB, kSOff = kCOff + kCDma * 1024,
                kBOff = kSOff + kSDma * 256;
  constexpr int kSlot = WsSlotBytes<PACK, MB, NB>();
  constexpr int kDma = 8 * MB + kCDma + 2 * kSDma;  // DMA per item
  constexpr int kFly = 63 / kDma < 3 ? 63 / kDma : 3;  // in flight / producer
  constexpr int S = (150 * 1024) / kSlot;      // ring slots
  static_assert(kBOff + kSDma * 256 == kSlot, "slot layout");
  static_assert(kFly * kDma <= 63, "memory counter");
  static_assert(S >= NP * kFly + 1, "ring depth");
  static_assert(S * kSlot >= NC * TM * TS * 4, "partial tiles fit");
  __shared__ __attribute__((aligned(16))) unsigned char ring[S * kSlot];
  __shared__ uint32_t flags[2 * S + 1];  // ready[S], freed[S], late

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * NR;
  const int G = a.groups;
  const int items = G / 4;
  uint32_t* const ready = flags;
  uint32_t* const freed = flags + S;
  uint32_t* const late = flags + 2 * S;
  if (threadIdx.x < 2 * S + 1) LdsStoreVolatile(flags + threadIdx.x, 0);
  __syncthreads();

  // Bounded waits (a.spin_limit polls, ~70 ms by default): a wave that
  // gives up marks the workgroup late and goes on, so the kernel ends; a
  // late workgroup stores NaN and reports the timeout.
  auto spin_until = [&](const uint32_t* f, uint32_t want) {
    SpinUntil(f, want, a.spin_limit, late);
  };

  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (wave >= NC) {
    // Producer p = wave - NC moves items p, p + NP, ... Lane maps (each
    // DMA writes 16 or 4 bytes per lane at lane * size of its destination;
    // rows past M / N read zeros); 16-byte chunk j of each 128-byte group
    // of a row is stored in place j ^ sw(row), so that the rows of one
    // fragment read fall in distinct banks:
    //  x: 2 rows of 512 bytes per instruction, sw(r) = r & 7;
    //  int4 codes: 8 rows of 128 bytes per instruction, sw(r) = (r / 2) & 7
    //    (the 16 rows of an 8-byte read fall in 16 distinct places);
    //  int8 codes: 4 rows of 256 bytes per instruction, sw(r) = r & 7 (the
    //    8 rows of a 16-byte read pass);
    //  scales / offsets: lane L, row n0 + L / 2, dword L % 2 (groups
    //    4 j + 2 (L % 2) and 4 j + 2 (L % 2) + 1).
    const int p = wave - NC;
    const int row_bytes = kInt4 ? a.k / 2 : a.k;
    DmaRsrc crs, xrs, srs, brs;
    crs.make(a.codes, static_cast<long long>(a.n) * row_bytes);
    xrs.make(a.x, static_cast<long long>(a.m) * a.k * 2);
    srs.make(a.scales, static_cast<long long>(a.n) * G * 2);
    brs.make(a.biases, a.has_bias ? static_cast<long long>(a.n) * G * 2 : 0);
    int xvo[8 * MB];
#pragma unroll
    for (int i = 0; i < 8 * MB; ++i) {
      const int r = 2 * i + lane / 32, q = lane % 32;
      xvo[i] = (r * a.k + ((q & ~7) | ((q & 7) ^ (r & 7))) * 8) * 2;
    }
    int cvo[kCDma];
#pragma unroll
    for (int i = 0; i < kCDma; ++i) {
      constexpr int LPR = CB / 16;  // lanes per code row
      const int rr = (64 / LPR) * i + lane / LPR, q = lane % LPR;
      const int r = n0 + rr;
      const int sw = kInt4 ? (rr >> 1) & 7 : rr & 7;
      cvo[i] = (rr < NR && r < a.n) ? r * row_bytes + ((q ^ sw) << 4) : kOut;
    }
    int svo[kSDma];
#pragma unroll
    for (int i = 0; i < kSDma; ++i) {
      const int rr = (64 * i + lane) / 2;
      svo[i] = (rr < NR && n0 + rr < a.n)
                   ? (n0 + rr) * G * 2 + ((64 * i + lane) % 2) * 4
                   : kOut;
    }
    auto publish = [&](int j) {
      if (lane == 0) LdsStoreVolatile(ready + j % S, j + 1);
    };
    int issued = 0, published = 0;  // own items
    for (int j = p; j < items; j += NP) {
      const int s = j % S;
      unsigned char* slot = ring + s * kSlot;
      if (j >= S && __builtin_amdgcn_readfirstlane(LdsLoadVolatile(
                        freed + s)) != static_cast<uint32_t>(j - S + 1)) {
        // Publish everything in flight before waiting: a consumer of one
        // of those items may be what frees the slot.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        for (; published < issued; ++published) publish(p + NP * published);
        spin_until(freed + s, j - S + 1);
      }
      const int g = 4 * j;
#pragma unroll
      for (int i = 0; i < kCDma; ++i)
        crs.dma_nt(slot + kCOff + i * 1024, cvo[i], g * (CB / 4));
#pragma unroll
      for (int i = 0; i < kSDma; ++i) {
        srs.dma4(slot + kSOff + i * 256, svo[i], g * 2);
        brs.dma4(slot + kBOff + i * 256, svo[i], g * 2);
      }
#pragma unroll
      for (int i = 0; i < 8 * MB; ++i)
        xrs.dma(slot + i * 1024, xvo[i], g * 128);
      ++issued;
      if (issued - published >= kFly) {
        // the oldest own item in flight has landed once at most kFly - 1
        // later ones are outstanding
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kFly - 1) * kDma)
                     : "memory");
        publish(p + NP * published);
        ++published;
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    for (; published < issued; ++published) publish(p + NP * published);
  } else {
    const int q16 = lane >> 4, l16 = lane & 15;
    const uint32_t kMask = vgpr_const(0x000F000Fu);
    const uint32_t kBias = vgpr_const(0x43004300u);
    const bf16x8 ones = __builtin_bit_cast(
        bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    for (int j = wave; j < items; j += NC) {
      const int s = j % S;
      const unsigned char* slot = ring + s * kSlot;
      spin_until(ready + s, j + 1);
      asm volatile("" ::: "memory");  // the slot's reads stay below
      // The item's operands in one LDS round trip: per group, the lane's
      // x chunks 2 (l / 16) and 2 (l / 16) + 1 of row l % 16, its code
      // words 2 (l / 16) and 2 (l / 16) + 1 of each row block, and the
      // group's scale and offset of each row block.
      using CodeT = typename std::conditional<kInt4, u32x2, u32x4>::type;
      u32x4 xv[4][MB][2];
      CodeT wv[4][NB];
      uint32_t sv[2][NB], bv[2][NB];
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            xv[gg][mb][h] = *reinterpret_cast<const u32x4*>(
                slot + (16 * mb + l16) * 512 +
                ((8 * gg + ((2 * q16 + h) ^ (l16 & 7))) << 4));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int r = 16 * nb + l16;
          if constexpr (kInt4) {
            // code words 2 (l / 16), + 1 of the group: 8 bytes of chunk
            // 2 gg + (l / 16) / 2
            const int c = 2 * gg + (q16 >> 1);
            wv[gg][nb] = *reinterpret_cast<const u32x2*>(
                slot + kCOff + r * 128 + ((c ^ ((r >> 1) & 7)) << 4) +
                ((q16 & 1) << 3));
          } else {
            // codes 16 (l / 16) .. + 15 of the group: chunk 4 gg + l / 16
            const int c = 4 * gg + q16;
            wv[gg][nb] = *reinterpret_cast<const u32x4*>(
                slot + kCOff + r * 256 + ((c ^ (r & 7)) << 4));
          }
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int r = 16 * nb + l16;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          sv[h][nb] =
              *reinterpret_cast<const uint32_t*>(slot + kSOff + r * 8 + 4 * h);
          bv[h][nb] =
              *reinterpret_cast<const uint32_t*>(slot + kBOff + r * 8 + 4 * h);
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) LdsStoreVolatile(freed + s, j + 1);
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        // int4: x in the pair order of the code words; int8: as loaded
        bf16x8 x0[MB], x1[MB];
        f32x4 xs[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          x0[mb] = kInt4 ? XPairs(xv[gg][mb][0])
                         : __builtin_bit_cast(bf16x8, xv[gg][mb][0]);
          x1[mb] = kInt4 ? XPairs(xv[gg][mb][1])
                         : __builtin_bit_cast(bf16x8, xv[gg][mb][1]);
          xs[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              x0[mb], ones, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          xs[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1[mb], ones,
                                                           xs[mb], 0, 0, 0);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          bf16x8 b0, b1;
          if constexpr (kInt4) {
            b0 = CodePairs(wv[gg][nb][0], kMask, kBias);
            b1 = CodePairs(wv[gg][nb][1], kMask, kBias);
          } else {
            b0 = CodeBytes<PACK>(wv[gg][nb][0], wv[gg][nb][1]);
            b1 = CodeBytes<PACK>(wv[gg][nb][2], wv[gg][nb][3]);
          }
          const int sh = 16 * (gg & 1);
          const float sc = __uint_as_float((sv[gg >> 1][nb] >> sh) << 16);
          const float of = __uint_as_float((bv[gg >> 1][nb] >> sh) << 16);
          // int4 and signed int8 codes enter as q + 128
          const float off = PACK == QK_PACK_U8 ? of : of - 128.f * sc;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                x0[mb], b0, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1[mb], b1, tmp, 0,
                                                          0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[mb][nb][r] =
                  fmaf(sc, tmp[r], fmaf(off, xs[mb][r], acc[mb][nb][r]));
          }
        }
      }
    }
  }

  // Sum the consumers' partial tiles (the ring is idle: every DMA has
  // landed and been read) and store rows < M, columns < N.
  __syncthreads();
  float* const part = reinterpret_cast<float*>(ring);
  if (wave < NC) {
    const int q16 = lane >> 4, l16 = lane & 15;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          part[(wave * TM + 16 * mb + 4 * q16 + r) * TS + 16 * nb + l16] =
              acc[mb][nb][r];
  }
  __syncthreads();
  bf16* Y = static_cast<bf16*>(a.y);
  const bool bad = LdsLoadVolatile(late) != 0u;  // a wait gave up
  if (threadIdx.x == 0) ReportLate(late, a.status);
  for (int e = threadIdx.x; e < TM * NR; e += (NC + NP) * 64) {
    const int r = e / NR, c = e % NR;
    if (r >= a.m || n0 + c >= a.n) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NC; ++w) v += part[(w * TM + r) * TS + c];
    Y[static_cast<long long>(r) * a.n + n0 + c] =
        from_f32<bf16>(bad ? __builtin_nanf("") : v);
  }
}

// The persistent form of qmm_ws_kernel for int4, one block of 16 rows of
// x, K <= 4096 and more row blocks of 48 weight rows than CUs (the
// lm_head). One workgroup per CU walks row blocks blockIdx.x, blockIdx.x
// + gridDim.x, ...; consumer c takes K ranges (items of four groups) c and
// c + 8 of every row block, so it keeps their x fragments in registers
// after the first row block and only the first row block's items carry x
// (x is read once per workgroup, not once per row block). Per row block,
// each consumer writes its partial tile into one of two LDS buffers and
// counts itself in with an LDS atomic; the last one sums the partials and
// stores, then marks the buffer reusable (done[b]), so the producers
// never wait for a reduction. Hand-off, producers and bounded spins as in
// qmm_ws_kernel. Measured at 151936 x 4096: 94 us against 108 us for the
// register-staged kernel at M = 16, 98 against 107 at M = 8.
constexpr int kWspConsumers = 8;

// s_waitcnt vmcnt(n) for a run-time n in [LO, HI], as a branch tree over
// immediates (the count is an instruction field).
template <int LO, int HI>
__device__ __forceinline__ void WaitVmcnt(int n) {
  if constexpr (LO == HI) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LO) : "memory");
  } else {
    constexpr int MID = (LO + HI) / 2;
    if (n <= MID)
      WaitVmcnt<LO, MID>(n);
    else
      WaitVmcnt<MID + 1, HI>(n);
  }
}

__global__ __launch_bounds__((kWspConsumers + kWsProducers) * 64) void
qmm_wsp_kernel(SkArgs a) {
  constexpr int NC = kWspConsumers, NP = kWsProducers, NB = 3;
  constexpr int NR = 16 * NB;                  // weight rows per block
  constexpr int TS = NR + 4;                   // partial-tile row stride
  constexpr int kCDma = NR * 128 / 1024;       // 6
  constexpr int kSDma = (NR * 2 + 63) / 64;    // 2
  constexpr int kCOff = 8192, kSOff = kCOff + kCDma * 1024,
                kBOff = kSOff + kSDma * 256;
  constexpr int kSlot = kBOff + kSDma * 256;
  constexpr int kDmaW = kCDma + 2 * kSDma;     // a weight item's DMA
  constexpr int kDmaX = kDmaW + 8;             // with its x
  constexpr int kFly = 3;
  constexpr int kPart = NC * 16 * TS;          // floats per buffer
  constexpr int S = (160 * 1024 - 2 * kPart * 4 - 512) / kSlot;
  static_assert(kFly * kDmaX <= 63, "memory counter");
  static_assert(S >= NP * kFly + 1, "ring depth");
  __shared__ __attribute__((aligned(16))) unsigned char ring[S * kSlot];
  __shared__ __attribute__((aligned(16))) float part[2][kPart];
  // ready[S], freed[S], cnt[2], done[2], late
  __shared__ uint32_t flags[2 * S + 5];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = a.groups;
  const int J = G / 4;  // K ranges per row block, <= 2 NC
  const int nrb = (a.n + NR - 1) / NR;
  const int rbs = (nrb - static_cast<int>(blockIdx.x) +
                   static_cast<int>(gridDim.x) - 1) / gridDim.x;
  const int T = rbs * J;  // items
  uint32_t* const ready = flags;
  uint32_t* const freed = flags + S;
  uint32_t* const cnt = flags + 2 * S;
  uint32_t* const done = flags + 2 * S + 2;
  uint32_t* const late = flags + 2 * S + 4;
  if (threadIdx.x < 2 * S + 5) LdsStoreVolatile(flags + threadIdx.x, 0);
  __syncthreads();
  auto block_n0 = [&](int i) {
    return (static_cast<int>(blockIdx.x) + i * static_cast<int>(gridDim.x)) *
           NR;
  };
  // Bounded waits (a.spin_limit polls, ~70 ms by default): a wave that
  // gives up marks the workgroup late and goes on, so the kernel ends; a
  // late workgroup stores NaN and reports the timeout.
  auto spin_until = [&](const uint32_t* f, uint32_t want) {
    SpinUntil(f, want, a.spin_limit, late);
  };

  if (wave >= NC) {
    // Producer p = wave - NC moves items p, p + NP, ...; item t is K range
    // t % J of row block t / J; the first row block's items carry x. Lane
    // maps as in qmm_ws_kernel.
    const int p = wave - NC;
    const int row_bytes = a.k / 2;
    DmaRsrc crs, xrs, srs, brs;
    crs.make(a.codes, static_cast<long long>(a.n) * row_bytes);
    xrs.make(a.x, static_cast<long long>(a.m) * a.k * 2);
    srs.make(a.scales, static_cast<long long>(a.n) * G * 2);
    brs.make(a.biases, a.has_bias ? static_cast<long long>(a.n) * G * 2 : 0);
    int xvo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 2 * i + lane / 32, q = lane % 32;
      xvo[i] = (r * a.k + ((q & ~7) | ((q & 7) ^ (r & 7))) * 8) * 2;
    }
    auto publish = [&](int t) {
      if (lane == 0) LdsStoreVolatile(ready + t % S, t + 1);
    };
    int issued = 0, published = 0;  // own items
    for (int t = p; t < T; t += NP) {
      const int s = t % S;
      unsigned char* slot = ring + s * kSlot;
      if (t >= S && __builtin_amdgcn_readfirstlane(LdsLoadVolatile(
                        freed + s)) != static_cast<uint32_t>(t - S + 1)) {
        // Publish everything in flight before waiting: a consumer of one
        // of those items may be what frees the slot.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        for (; published < issued; ++published) publish(p + NP * published);
        spin_until(freed + s, t - S + 1);
      }
      const int n0 = block_n0(t / J);
      const int g = 4 * (t % J);
#pragma unroll
      for (int i = 0; i < kCDma; ++i) {
        const int rr = 8 * i + lane / 8, r = n0 + rr;
        const int vo =
            r < a.n ? r * row_bytes + (((lane % 8) ^ ((rr >> 1) & 7)) << 4)
                    : kOut;
        crs.dma_nt(slot + kCOff + i * 1024, vo, g * 32);
      }
#pragma unroll
      for (int i = 0; i < kSDma; ++i) {
        const int rr = (64 * i + lane) / 2, r = n0 + rr;
        const int vo = (rr < NR && r < a.n)
                           ? r * G * 2 + ((64 * i + lane) % 2) * 4
                           : kOut;
        srs.dma4(slot + kSOff + i * 256, vo, g * 2);
        brs.dma4(slot + kBOff + i * 256, vo, g * 2);
      }
      if (t < J) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xrs.dma(slot + i * 1024, xvo[i], g * 128);
      }
      ++issued;
      if (issued - published >= kFly) {
        // The oldest own item in flight has landed once only the DMA of
        // the kFly - 1 newer ones is outstanding.
        int newer = 0;
#pragma unroll
        for (int d = 1; d < kFly; ++d)
          newer += p + NP * (published + d) < J ? kDmaX : kDmaW;
        WaitVmcnt<0, 63>(newer);
        publish(p + NP * published);
        ++published;
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    for (; published < issued; ++published) publish(p + NP * published);
    if (lane == 0) ReportLate(late, a.status);
    return;
  }

  // Consumer.
  const int q16 = lane >> 4, l16 = lane & 15;
  const uint32_t kMask = vgpr_const(0x000F000Fu);
  const uint32_t kBias = vgpr_const(0x43004300u);
  const bf16x8 ones = __builtin_bit_cast(
      bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  bf16x8 xk[2][4][2];  // x fragments of K ranges wave and wave + NC
  for (int i = 0; i < rbs; ++i) {
    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = wave + u * NC;
      if (j >= J) continue;
      const int t = i * J + j;
      const int s = t % S;
      const unsigned char* slot = ring + s * kSlot;
      spin_until(ready + s, t + 1);
      asm volatile("" ::: "memory");  // the slot's reads stay below
      if (i == 0) {
        // the lane's x chunks 2 (l / 16) and 2 (l / 16) + 1 of row l % 16
        // for each group, as code-word pairs
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            xk[u][gg][h] = XPairs(*reinterpret_cast<const u32x4*>(
                slot + l16 * 512 +
                ((8 * gg + ((2 * q16 + h) ^ (l16 & 7))) << 4)));
      }
      u32x2 wv[4][NB];
      uint32_t sv[2][NB], bv[2][NB];
#pragma unroll
      for (int gg = 0; gg < 4; ++gg)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int r = 16 * nb + l16;
          const int c = 2 * gg + (q16 >> 1);
          wv[gg][nb] = *reinterpret_cast<const u32x2*>(
              slot + kCOff + r * 128 + ((c ^ ((r >> 1) & 7)) << 4) +
              ((q16 & 1) << 3));
        }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int r = 16 * nb + l16;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          sv[h][nb] =
              *reinterpret_cast<const uint32_t*>(slot + kSOff + r * 8 + 4 * h);
          bv[h][nb] =
              *reinterpret_cast<const uint32_t*>(slot + kBOff + r * 8 + 4 * h);
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) LdsStoreVolatile(freed + s, t + 1);
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        f32x4 xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            xk[u][gg][0], ones, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xk[u][gg][1], ones, xs,
                                                     0, 0, 0);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              xk[u][gg][0], CodePairs(wv[gg][nb][0], kMask, kBias),
              f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              xk[u][gg][1], CodePairs(wv[gg][nb][1], kMask, kBias), tmp, 0,
              0, 0);
          const int sh = 16 * (gg & 1);
          const float sc = __uint_as_float((sv[gg >> 1][nb] >> sh) << 16);
          const float of = __uint_as_float((bv[gg >> 1][nb] >> sh) << 16);
          const float off = of - 128.f * sc;  // codes enter as q + 128
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[nb][r] = fmaf(sc, tmp[r], fmaf(off, xs[r], acc[nb][r]));
        }
      }
    }

    // Row block i: partial tile into buffer b (free once block i - 2 has
    // been summed), count in; the last consumer sums and stores.
    const int b = i & 1;
    if (i >= 2) spin_until(done + b, i - 1);
    float* const pb = part[b];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        pb[(wave * 16 + 4 * q16 + r) * TS + 16 * nb + l16] = acc[nb][r];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    uint32_t old = 0;
    if (lane == 0)
      old = __hip_atomic_fetch_add(cnt + b, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __builtin_amdgcn_readfirstlane(old);
    asm volatile("" ::: "memory");  // the partial tiles' reads stay below
    if (old == NC - 1) {
      // four consecutive columns per lane and step; NaN once a wait of
      // this workgroup gave up
      const int n0 = block_n0(i);
      bf16* Y = static_cast<bf16*>(a.y);
      constexpr int kIt = 4 * NR / 64;
      static_assert(kIt * 64 == 4 * NR, "whole steps");
      f32x4 v[kIt];
#pragma unroll
      for (int it = 0; it < kIt; ++it) {
        const int e = lane + 64 * it;
        const int r = e / (NR / 4), c = 4 * (e % (NR / 4));
        v[it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NC; ++w)
          v[it] += *reinterpret_cast<const f32x4*>(pb + (w * 16 + r) * TS + c);
      }
      // late is read after every partial has been read: a wave that gave
      // up its wait for this buffer set it before writing into the buffer,
      // so a sum that saw such a write also sees late.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const bool bad = LdsLoadVolatile(late) != 0u;
#pragma unroll
      for (int it = 0; it < kIt; ++it) {
        const int e = lane + 64 * it;
        const int r = e / (NR / 4), c = 4 * (e % (NR / 4));
        if (r < a.m) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (n0 + c + q < a.n)
              Y[static_cast<long long>(r) * a.n + n0 + c + q] =
                  from_f32<bf16>(bad ? __builtin_nanf("") : v[it][q]);
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) {
        LdsStoreVolatile(cnt + b, 0);
        LdsStoreVolatile(done + b, i + 1);
      }
    }
  }
  // Once its own work is over, a consumer that finds the workgroup late
  // overwrites a share of all the workgroup's outputs with NaN: a wait that
  // gave up can also leave a row block's partial count wrong, so that the
  // block is never stored. A store that lands after this one read late as
  // 0 after reading its partials, so its sum was complete and correct.
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (LdsLoadVolatile(late) != 0u) {
    bf16* Y = static_cast<bf16*>(a.y);
    const int per_block = a.m * NR;
    for (int e = wave * 64 + lane; e < rbs * per_block; e += NC * 64) {
      const int i = e / per_block, rem = e % per_block;
      const int r = rem / NR, c = block_n0(i) + rem % NR;
      if (c < a.n)
        Y[static_cast<long long>(r) * a.n + c] =
            from_f32<bf16>(__builtin_nanf(""));
    }
  }
  if (lane == 0) ReportLate(late, a.status);
}

}  // namespace

bool QSkinnyApplies(const QuantProblem& p) {
  const int64_t m = p.m;
  const bool int4 = p.bits == 4 && p.packing == QK_PACK_U32X8;
  const bool int8 = p.bits == 8 && (p.packing == QK_PACK_U8 ||
                                    p.packing == QK_PACK_S8_SYM);
  const int64_t row_bytes = int4 ? p.k / 2 : p.k;
  // Above 32 rows the dequantizing qmm_mid_kernel is faster (int4 at
  // 12288 x 4096: M = 33 25.5 vs 29.9 us, M = 64 28.4 vs 38.0 us).
  return m >= 1 && m <= 32 && (int4 || int8) && p.group == 64 &&
         p.x_dtype == QK_BF16 && p.scale_dtype == QK_BF16 &&
         (!p.has_bias || p.bias_dtype == QK_BF16) && p.k % 1024 == 0 &&
         p.k > 0 && p.n > 0 && p.n * row_bytes < (int64_t{1} << 31) &&
         m * p.k * 2 < (int64_t{1} << 31) &&
         p.n * (p.k / 64) * 2 < (int64_t{1} << 31) &&
         reinterpret_cast<uintptr_t>(p.x) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.codes) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.scales) % 8 == 0 &&
         (!p.has_bias || reinterpret_cast<uintptr_t>(p.biases) % 8 == 0);
}

qk_status LaunchQSkinny(const QuantProblem& p, hipStream_t stream) {
  SkArgs a;
  a.x = p.x;
  a.codes = p.codes;
  a.scales = p.scales;
  a.biases = p.has_bias ? p.biases : nullptr;
  a.y = p.y;
  a.m = static_cast<int>(p.m);
  a.n = static_cast<int>(p.n);
  a.k = static_cast<int>(p.k);
  a.groups = a.k / 64;
  a.has_bias = p.has_bias ? 1 : 0;
  a.status = DeviceStatusWord();
  a.spin_limit = SpinLimit();
  if (a.status == nullptr) {
    return Fail(QK_INTERNAL, "qkern: the device status word is unavailable");
  }
  const int cus = DeviceComputeUnits();
  const int mb = (a.m + 15) / 16;
  // Register-staged kernel: sub-chunks of 4 groups (int8: 2, to bound the
  // registers); 32 weight rows per workgroup when that still gives every
  // CU one; eight waves split K (fewer when K is short), each walking
  // k / KW.
  const bool int4 = p.packing == QK_PACK_U32X8;
  // QK_SKINNY_WS=0 turns the streamed kernel off (tuning).
  static const bool ws_off = [] {
    const char* v = std::getenv("QK_SKINNY_WS");
    return v != nullptr && *v == '0';
  }();
  // The streamed kernel when all of its workgroups are resident at once:
  // 16, 32 or 48 weight rows each, the fewest for which one workgroup per
  // CU covers N.
  const int ws_nb = (a.n + 15) / 16 <= cus   ? 1
                    : (a.n + 31) / 32 <= cus ? 2
                    : (a.n + 47) / 48 <= cus ? 3
                                             : 0;
  // int8 with two row blocks of x would not fit the registers at 48 rows.
  if (mb <= (int4 ? 2 : 1) && !ws_off && a.groups % 4 == 0 && ws_nb > 0) {
    const int grid = (a.n + 16 * ws_nb - 1) / (16 * ws_nb);
    constexpr int threads = (kWsConsumers + kWsProducers) * 64;
    auto go = [&](auto k1, auto k2, auto k3) {
      if (ws_nb == 3)
        k3<<<grid, threads, 0, stream>>>(a);
      else if (ws_nb == 2)
        k2<<<grid, threads, 0, stream>>>(a);
      else
        k1<<<grid, threads, 0, stream>>>(a);
    };
#define QK_WS(P, MB) \
  go(qmm_ws_kernel<P, MB, 1>, qmm_ws_kernel<P, MB, 2>, \
     qmm_ws_kernel<P, MB, 3>)
    if (p.packing == QK_PACK_U32X8) {
      if (mb == 1) QK_WS(QK_PACK_U32X8, 1); else QK_WS(QK_PACK_U32X8, 2);
    } else if (p.packing == QK_PACK_U8) {
      QK_WS(QK_PACK_U8, 1);
    } else {
      QK_WS(QK_PACK_S8_SYM, 1);
    }
#undef QK_WS
    return PostLaunch("qmm_ws");
  }
  // The persistent form for the int4 shapes with more 48-row blocks than
  // CUs (the lm_head) and K <= 4096.
  if (int4 && mb == 1 && !ws_off && ws_nb == 0 && a.groups % 4 == 0 &&
      a.groups / 4 <= 2 * kWspConsumers) {
    const int nrb = (a.n + 47) / 48;
    qmm_wsp_kernel<<<std::min(nrb, cus),
                     (kWspConsumers + kWsProducers) * 64, 0, stream>>>(a);
    return PostLaunch("qmm_wsp");
  }
  const int cg = int4 && mb <= 2 ? 4 : 2;
  bool wide = (a.n + 31) / 32 >= cus && mb <= (int4 ? 2 : 1);
  // QK_SKINNY_ROWS=16|32 forces the weight rows per workgroup (tuning).
  static const int forced_rows = [] {
    const char* v = std::getenv("QK_SKINNY_ROWS");
    return v == nullptr ? 0 : std::atoi(v);
  }();
  if (forced_rows == 16) wide = false;
  if (forced_rows == 32 && mb <= (int4 ? 2 : 1)) wide = true;
  // 48 weight rows per workgroup (three row blocks) when that still gives
  // every CU one: x is read once per workgroup, so fewer, taller
  // workgroups read less of it.
  const bool tall = int4 && mb == 1 && (forced_rows == 48 ||
                    (forced_rows == 0 && a.n / 48 >= cus));
  const int nr = tall ? 48 : wide ? 32 : 16;
  const dim3 grid((a.n + nr - 1) / nr);
  // The most waves per workgroup (8, 4 or 2) for which every workgroup is
  // resident at once (no second, partly empty round) and k splits evenly.
  // k8 is null when eight waves would exceed the LDS (not instantiated).
  auto go = [&](auto k8, auto k4, auto k2) {
    auto fits = [&](const void* f, int waves) {
      return f != nullptr && a.k % (waves * 64 * cg) == 0 &&
             static_cast<int64_t>(ResidentBlocks(f, waves * 64, 0)) * cus >=
                 grid.x;
    };
    int kw = 2;
    if (fits(reinterpret_cast<const void*>(k8), 8))
      kw = 8;
    else if (fits(reinterpret_cast<const void*>(k4), 4))
      kw = 4;
    a.chunks = a.k / kw / (64 * cg);  // k % 1024 == 0: kw = 2 always divides
    if (kw == 8)
      k8<<<grid, 8 * 64, 0, stream>>>(a);
    else if (kw == 4)
      k4<<<grid, 4 * 64, 0, stream>>>(a);
    else
      k2<<<grid, 2 * 64, 0, stream>>>(a);
  };
#define QK_SKINNY(P, MB, NB, CG)                                         \
  go(Skinny8<P, MB, NB, CG>(), qmm_skinny_kernel<P, MB, NB, 4, CG>,     \
     qmm_skinny_kernel<P, MB, NB, 2, CG>)
  if (p.packing == QK_PACK_U32X8) {
    switch (mb) {
      case 1:
        if (tall) QK_SKINNY(QK_PACK_U32X8, 1, 3, 4);
        else if (wide) QK_SKINNY(QK_PACK_U32X8, 1, 2, 4);
        else QK_SKINNY(QK_PACK_U32X8, 1, 1, 4);
        break;
      default:  // 17..32 rows
        if (wide) QK_SKINNY(QK_PACK_U32X8, 2, 2, 4);
        else QK_SKINNY(QK_PACK_U32X8, 2, 1, 4);
        break;
    }
  } else if (p.packing == QK_PACK_U8) {
    if (mb == 1) {
      if (wide) QK_SKINNY(QK_PACK_U8, 1, 2, 2);
      else QK_SKINNY(QK_PACK_U8, 1, 1, 2);
    } else {
      QK_SKINNY(QK_PACK_U8, 2, 1, 2);
    }
  } else {
    if (mb == 1) {
      if (wide) QK_SKINNY(QK_PACK_S8_SYM, 1, 2, 2);
      else QK_SKINNY(QK_PACK_S8_SYM, 1, 1, 2);
    } else {
      QK_SKINNY(QK_PACK_S8_SYM, 2, 1, 2);
    }
  }
#undef QK_SKINNY
  return PostLaunch("qmm_skinny");
}

}  // namespace qk
