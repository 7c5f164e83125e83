// Quantized matmul for a medium number of rows of x (33..64 as routed,
// and up to 128 where the register-dequantizing GEMM does not apply):
// y[M, N] = x[M, K] W^T, W int8 (u8 affine or s8 symmetric) or int4 (u32x8
// words), bf16 x / scale / offset, group size 64 — the short-prefill
// shapes. The reference's linear() (examples/llm/qwen3.py:215-230)
// dequantizes W to x's type for more than ROWS_MAX = 4 rows
// (dequantize, qwen3.py:199-207) and multiplies; this kernel does the same
// per weight, in registers, and never writes the dequantized weights.
//
// Design (MI355X-first). At these M the work sits near the ridge point:
// for 128 x 12288 x 4096 int8 the 50 MB of codes take ~7 us at HBM speed
// and the 12.9 GFLOP ~6 us on the matrix cores, and only 1.5 M outputs
// exist, i.e. ~6000 per CU. So:
//  - A workgroup owns NR = 16 NB weight rows and all M rows of x (a
//    16 MB x NR output tile, 128 x 48 for that shape: 256 workgroups, one
//    per CU), and its KW waves split K (each wave a contiguous run of
//    groups). Every weight is loaded and dequantized exactly once, and
//    each wave fetches a distinct slice of x, so no operand byte is
//    fetched twice by a workgroup. The KW partial tiles are summed
//    through LDS at the end.
//  - v_mfma_f32_16x16x32_bf16, A = 16 rows of x, B = 16 weight rows. The
//    K order inside a group is permuted identically for x and W (MFMA
//    sums over K, so only the pairing matters): lane l takes codes
//    16 (l / 16) .. + 15 of the group (one contiguous 16-byte or 8-byte
//    load per weight row) and the matching 32 contiguous bytes of x; codes
//    0..7 of the run feed the group's first MFMA, 8..15 its second.
//  - Weights are dequantized in registers as bf16(q s + b) (one fma per
//    weight, then one rounding to bf16; the reference's XLA program rounds
//    q s and q s + b to bf16 separately, a difference far inside the
//    matmul tolerance).
//  - Loads go straight to registers, the next group in flight while one is
//    computed (each load issued unconditionally; groups past the wave's
//    run read zeros through out-of-range offsets), so the in-order memory
//    counter waits only for the group being consumed.
//  - Rows past M or N read zeros through buffer descriptors and are not
//    stored.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "qk_device.h"
#include "qk_internal.h"

namespace qk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct MdArgs {
  const void* x;
  const void* codes;
  const void* scales;
  const void* biases;
  void* y;
  int m, n, k;
  int groups;  // k / 64
  int has_bias;
  int gpw;     // groups per wave
  uint32_t* status;  // device status word (producer / consumer kernel)
  int spin_limit;    // polls before a flag wait gives up
};

constexpr int kNonTemporal = 2;
constexpr int kOut = 0x7FFF0000;  // an offset past every extent

__device__ __forceinline__ __amdgpu_buffer_rsrc_t Rsrc(const void* p,
                                                       int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                           bytes, 0x00020000);
}

// Eight codes -> bf16(q * s + b). int4: the 8 nibbles of a u32x8 word, code
// j at bits 4 j; int8: 8 bytes (s8: signed).
template <int PACK>
__device__ __forceinline__ bf16x8 Dequant8(uint32_t w0, uint32_t w1, float s,
                                           float b) {
  bf16x8 r;
  if constexpr (PACK == QK_PACK_U32X8) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      r[j] = from_f32<bf16>(
          fmaf(static_cast<float>((w0 >> (4 * j)) & 15u), s, b));
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w = j < 4 ? w0 : w1;
      const uint32_t byte = (w >> (8 * (j & 3))) & 255u;
      const float q = PACK == QK_PACK_S8_SYM
                          ? static_cast<float>(static_cast<int8_t>(byte))
                          : static_cast<float>(byte);
      r[j] = from_f32<bf16>(fmaf(q, s, b));
    }
  }
  return r;
}

template <int PACK, int MB, int NB, int KW>
__global__ __launch_bounds__(KW * 64) void qmm_mid_kernel(MdArgs a) {
  constexpr bool kInt4 = PACK == QK_PACK_U32X8;
  constexpr int GB = kInt4 ? 32 : 64;  // code bytes per group per row
  constexpr int NR = 16 * NB;          // weight rows per workgroup
  constexpr int TM = 16 * MB, TS = NR + 1;
  static_assert(NR <= 64, "one scale DMA per group");
  // A wave's slot for one group: x (TM rows x 128 bytes), codes (NR rows x
  // GB bytes, whole 1 KB DMA instructions), scales and offsets (one dword
  // per row: the group and its neighbour).
  constexpr int kCRows = 1024 / GB;  // code rows per DMA instruction
  constexpr int kCDma = (NR + kCRows - 1) / kCRows;
  constexpr int kXOff = 0, kCOff = TM * 128, kSOff = kCOff + kCDma * 1024,
                kBOff = kSOff + 256, kSlot = kBOff + 256;
  constexpr int kDma = TM / 8 + kCDma + 2;  // DMA instructions per group
  constexpr int kHalfWaves = (KW + 1) / 2;
  constexpr int kPart = kHalfWaves * TM * TS * 4;
  constexpr int kArr = KW * kSlot > kPart ? KW * kSlot : kPart;
  // Ring slots 0 and 1 of every wave (separate arrays: the compiler's wait
  // for an LDS DMA is per array, so reading slot 0 never waits for the DMA
  // into slot 1); after the loop, the partial tiles.
  __shared__ __attribute__((aligned(16))) unsigned char st0[kArr];
  __shared__ __attribute__((aligned(16))) unsigned char st1[kArr];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q16 = lane >> 4, l16 = lane & 15;
  const int n0 = blockIdx.x * NR;
  const int G = a.groups;
  const int row_bytes = kInt4 ? a.k / 2 : a.k;
  const auto crs = Rsrc(a.codes, a.n * row_bytes);
  const auto xrs = Rsrc(a.x, a.m * a.k * 2);
  const auto srs = Rsrc(a.scales, a.n * G * 2);
  const auto brs = Rsrc(a.biases, a.has_bias ? a.n * G * 2 : 0);

  // Every DMA instruction writes 16 (4) bytes per lane at lane * 16 (4) of
  // its destination; the lanes are mapped so that consecutive lanes read
  // consecutive bytes of one row, and rows past M / N read zeros.
  //  x, instruction i: row 8 i + L / 8, 16-byte chunk (L % 8) ^ (L / 8)
  //    into slot L % 8 (the slot of chunk c of row r is c ^ (r & 7)).
  const int xvo = ((lane >> 3) * a.k + ((lane & 7) ^ (lane >> 3)) * 8) * 2;
  //  codes, instruction i: row kCRows i + L / (GB / 16), 16-byte chunk
  //    p ^ sw(row) into slot p = L % (GB / 16), with sw(r) = (r / 2) & 3
  //    for int8 (64-byte rows) and (r / 4) & 1 for int4 (32-byte rows).
  int cvo[kCDma];
#pragma unroll
  for (int i = 0; i < kCDma; ++i) {
    constexpr int LPR = GB / 16;
    const int rr = kCRows * i + lane / LPR;
    const int sw = kInt4 ? ((rr >> 2) & 1) : ((rr >> 1) & 3);
    const int r = n0 + rr;
    cvo[i] = (rr < NR && r < a.n)
                 ? r * row_bytes + (((lane % LPR) ^ sw) << 4)
                 : kOut;
  }
  //  scales / offsets: lane L < NR, row n0 + L, the dword holding groups
  //    g & ~1 and (g & ~1) + 1.
  const int svo = (lane < NR && n0 + lane < a.n) ? (n0 + lane) * G * 2 : kOut;

  const int g0 = wave * a.gpw;
  // DMA group gi of the wave's run into slot (past the run: zeros).
  auto load = [&](int gi, unsigned char* slot) {
    const int oob = gi < a.gpw ? 0 : kOut;
    const int g = g0 + min(gi, a.gpw - 1);
#pragma unroll
    for (int i = 0; i < kCDma; ++i)
      DmaLds16Nt(crs, slot + kCOff + i * 1024, cvo[i] + oob,
                            g * GB);
    DmaLds4(srs, slot + kSOff, svo + oob, (g & ~1) * 2);
    DmaLds4(brs, slot + kBOff, svo + oob, (g & ~1) * 2);
#pragma unroll
    for (int i = 0; i < TM / 8; ++i)
      DmaLds16(xrs, slot + kXOff + i * 1024, xvo + i * 8 * a.k * 2 + oob,
                 g * 128);
  };

  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto process = [&](const unsigned char* slot, int gi) {
    const int odd = (g0 + min(gi, a.gpw - 1)) & 1;
    bf16x8 w[NB][2];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int r = 16 * nb + l16;
      const float sc = __uint_as_float(static_cast<uint32_t>(
          *reinterpret_cast<const uint16_t*>(slot + kSOff + r * 4 + odd * 2))
          << 16);
      const float bi = __uint_as_float(static_cast<uint32_t>(
          *reinterpret_cast<const uint16_t*>(slot + kBOff + r * 4 + odd * 2))
          << 16);
      if constexpr (kInt4) {
        // the lane's 16 codes: bytes 8 (l / 16) .. + 7 of the row
        const int slt = (q16 >> 1) ^ ((r >> 2) & 1);
        const u32x2 c = *reinterpret_cast<const u32x2*>(
            slot + kCOff + r * GB + (slt << 4) + ((q16 & 1) << 3));
        w[nb][0] = Dequant8<PACK>(c[0], 0u, sc, bi);
        w[nb][1] = Dequant8<PACK>(c[1], 0u, sc, bi);
      } else {
        // the lane's 16 codes: chunk l / 16 of the row
        const int slt = q16 ^ ((r >> 1) & 3);
        const u32x4 c = *reinterpret_cast<const u32x4*>(
            slot + kCOff + r * GB + (slt << 4));
        w[nb][0] = Dequant8<PACK>(c[0], c[1], sc, bi);
        w[nb][1] = Dequant8<PACK>(c[2], c[3], sc, bi);
      }
    }
    // All first-half MFMAs, then all second-half ones: the two MFMAs
    // into one accumulator are NB * MB instructions apart. x fragment of
    // row block mb, half h: K chunk 2 (l / 16) + h of the lane's row.
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int r = 16 * mb + l16;
        const int c = 2 * q16 + h;
        const bf16x8 xv = *reinterpret_cast<const bf16x8*>(
            slot + kXOff + r * 128 + ((c ^ (r & 7)) << 4));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              xv, w[nb][h], acc[mb][nb], 0, 0, 0);
      }
  };

  // Two groups in flight (slots 0 and 1 alternate); the memory counter
  // tracks at most 63 operations. The run is padded to an even length with
  // groups past it, which read zeros (codes, x, scales and offsets) and so
  // add nothing: the loop body has no branch (a conditional process makes
  // the compiler's wait-count pass drain every load at the loop head). The
  // scheduling barriers keep each group's DMA ahead of the previous
  // group's arithmetic. A wave's slots are its own, so no workgroup
  // barrier is needed: its LDS reads of a slot are consumed by its MFMAs
  // before it issues the next DMA into that slot.
  //
  // The wait for a slot's DMA is explicit: vmcnt(kDma) after the next
  // group's DMA has been issued means every DMA into the slot about to be
  // read has landed. It is written as asm with a memory clobber (no LDS
  // read moves above it): the compiler's own tracking of LDS DMA cannot be
  // relied on here (its memory operand describes 16 bytes at the wave's
  // base address, not the 1 KB the instruction writes, so reads of other
  // rows of the slot were found to get no wait).
  static_assert(2 * kDma <= 63, "memory counter");
  unsigned char* const sl0 = st0 + wave * kSlot;
  unsigned char* const sl1 = st1 + wave * kSlot;
  load(0, sl0);
  for (int gi = 0; gi < a.gpw; gi += 2) {
    load(gi + 1, sl1);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDma) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    process(sl0, gi);
    load(gi + 2, sl0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDma) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    process(sl1, gi + 1);
  }

  // Sum the KW partial tiles (half of them in each array, after the last
  // DMA, which writes zeros, has landed) and store rows < M, columns < N.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  float* const p0 = reinterpret_cast<float*>(st0);
  float* const p1 = reinterpret_cast<float*>(st1);
  float* const mine = (wave < kHalfWaves ? p0 : p1) +
                      (wave % kHalfWaves) * TM * TS;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        mine[(16 * mb + 4 * q16 + r) * TS + 16 * nb + l16] = acc[mb][nb][r];
  __syncthreads();
  bf16* Y = static_cast<bf16*>(a.y);
  for (int e = threadIdx.x; e < TM * NR; e += KW * 64) {
    const int r = e / NR, c = e % NR;
    if (r >= a.m || n0 + c >= a.n) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < KW; ++w)
      v += (w < kHalfWaves ? p0 : p1)[((w % kHalfWaves) * TM + r) * TS + c];
    Y[static_cast<long long>(r) * a.n + n0 + c] = from_f32<bf16>(v);
  }
}

// The producer / consumer form of qmm_mid_kernel (same slot layout, lane
// maps and arithmetic): two producer waves move whole groups (x TM rows x
// 128 bytes, codes NR rows x GB bytes, scale / offset dwords) from global
// memory into a ring of S slots in LDS by LDS DMA, each with up to three
// groups in flight; NC consumer waves (consumer c takes groups c, c + NC,
// ...) read them from LDS, dequantize and multiply. A consumer never
// issues a global load, so it never stalls behind a full memory queue;
// a producer never computes, so the queue stays full. Hand-off through LDS
// words (ready[s] = g + 1 once group g has landed in slot s = g % S,
// freed[s] = g + 1 once its consumer has read it); every wait is a bounded
// spin. The DMA is inline asm and the flags are read through LDS-typed
// pointers, so the compiler adds no waits for the DMA of its own.
constexpr int kMidConsumers = 4, kMidProducers = 2;

template <int PACK, int MB, int NB>
__global__ __launch_bounds__((kMidConsumers + kMidProducers) * 64) void
qmm_wsmid_kernel(MdArgs a) {
  constexpr int NC = kMidConsumers, NP = kMidProducers;
  constexpr bool kInt4 = PACK == QK_PACK_U32X8;
  constexpr int GB = kInt4 ? 32 : 64;  // code bytes per group per row
  constexpr int NR = 16 * NB;          // weight rows per workgroup
  constexpr int TM = 16 * MB, TS = NR + 1;
  constexpr int kCRows = 1024 / GB;  // code rows per DMA instruction
  constexpr int kCDma = (NR + kCRows - 1) / kCRows;
  constexpr int kXOff = 0, kCOff = TM * 128, kSOff = kCOff + kCDma * 1024,
                kBOff = kSOff + 256, kSlot = kBOff + 256;
  constexpr int kDma = TM / 8 + kCDma + 2;  // DMA instructions per group
  constexpr int kFly = 63 / kDma < 3 ? 63 / kDma : 3;
  constexpr int S = (150 * 1024) / kSlot;
  static_assert(NR <= 64, "one scale DMA per group");
  static_assert(kFly >= 1 && S >= NP * kFly + 1, "ring depth");
  static_assert(S * kSlot >= NC * TM * TS * 4, "partial tiles fit");
  __shared__ __attribute__((aligned(16))) unsigned char ring[S * kSlot];
  __shared__ uint32_t flags[2 * S + 1];  // ready[S], freed[S], late

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q16 = lane >> 4, l16 = lane & 15;
  const int n0 = blockIdx.x * NR;
  const int G = a.groups;
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
    // Producer p = wave - NC moves groups p, p + NP, ... (lane maps as in
    // qmm_mid_kernel).
    const int p = wave - NC;
    const int row_bytes = kInt4 ? a.k / 2 : a.k;
    DmaRsrc crs, xrs, srs, brs;
    crs.make(a.codes, static_cast<long long>(a.n) * row_bytes);
    xrs.make(a.x, static_cast<long long>(a.m) * a.k * 2);
    srs.make(a.scales, static_cast<long long>(a.n) * G * 2);
    brs.make(a.biases, a.has_bias ? static_cast<long long>(a.n) * G * 2 : 0);
    const int xvo = ((lane >> 3) * a.k + ((lane & 7) ^ (lane >> 3)) * 8) * 2;
    int cvo[kCDma];
#pragma unroll
    for (int i = 0; i < kCDma; ++i) {
      constexpr int LPR = GB / 16;
      const int rr = kCRows * i + lane / LPR;
      const int sw = kInt4 ? ((rr >> 2) & 1) : ((rr >> 1) & 3);
      const int r = n0 + rr;
      cvo[i] = (rr < NR && r < a.n)
                   ? r * row_bytes + (((lane % LPR) ^ sw) << 4)
                   : kOut;
    }
    const int svo =
        (lane < NR && n0 + lane < a.n) ? (n0 + lane) * G * 2 : kOut;
    auto publish = [&](int g) {
      if (lane == 0) LdsStoreVolatile(ready + g % S, g + 1);
    };
    int issued = 0, published = 0;  // own groups
    for (int g = p; g < G; g += NP) {
      const int s = g % S;
      unsigned char* slot = ring + s * kSlot;
      if (g >= S && __builtin_amdgcn_readfirstlane(LdsLoadVolatile(
                        freed + s)) != static_cast<uint32_t>(g - S + 1)) {
        // Publish everything in flight before waiting: a consumer of one
        // of those groups may be what frees the slot.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        for (; published < issued; ++published) publish(p + NP * published);
        spin_until(freed + s, g - S + 1);
      }
#pragma unroll
      for (int i = 0; i < kCDma; ++i)
        crs.dma_nt(slot + kCOff + i * 1024, cvo[i], g * GB);
      srs.dma4(slot + kSOff, svo, (g & ~1) * 2);
      brs.dma4(slot + kBOff, svo, (g & ~1) * 2);
#pragma unroll
      for (int i = 0; i < TM / 8; ++i)
        xrs.dma(slot + kXOff + i * 1024, xvo + i * 8 * a.k * 2, g * 128);
      ++issued;
      if (issued - published >= kFly) {
        // the oldest own group in flight has landed once at most kFly - 1
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
    for (int g = wave; g < G; g += NC) {
      const int s = g % S;
      const unsigned char* slot = ring + s * kSlot;
      spin_until(ready + s, g + 1);
      asm volatile("" ::: "memory");  // the slot's reads stay below
      const int odd = g & 1;
      // the group's weights of each row block, dequantized (their reads
      // complete before the slot is released)
      bf16x8 w[NB][2];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int r = 16 * nb + l16;
        const float sc = __uint_as_float(static_cast<uint32_t>(
            *reinterpret_cast<const uint16_t*>(slot + kSOff + r * 4 + odd * 2))
            << 16);
        const float bi = __uint_as_float(static_cast<uint32_t>(
            *reinterpret_cast<const uint16_t*>(slot + kBOff + r * 4 + odd * 2))
            << 16);
        if constexpr (kInt4) {
          const int slt = (q16 >> 1) ^ ((r >> 2) & 1);
          const u32x2 c = *reinterpret_cast<const u32x2*>(
              slot + kCOff + r * GB + (slt << 4) + ((q16 & 1) << 3));
          w[nb][0] = Dequant8<PACK>(c[0], 0u, sc, bi);
          w[nb][1] = Dequant8<PACK>(c[1], 0u, sc, bi);
        } else {
          const int slt = q16 ^ ((r >> 1) & 3);
          const u32x4 c = *reinterpret_cast<const u32x4*>(
              slot + kCOff + r * GB + (slt << 4));
          w[nb][0] = Dequant8<PACK>(c[0], c[1], sc, bi);
          w[nb][1] = Dequant8<PACK>(c[2], c[3], sc, bi);
        }
      }
      bf16x8 xv[2][MB];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int r = 16 * mb + l16;
          const int c = 2 * q16 + h;
          xv[h][mb] = *reinterpret_cast<const bf16x8*>(
              slot + kXOff + r * 128 + ((c ^ (r & 7)) << 4));
        }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) LdsStoreVolatile(freed + s, g + 1);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                xv[h][mb], w[nb][h], acc[mb][nb], 0, 0, 0);
    }
  }

  // Sum the consumers' partial tiles (the ring is idle: every DMA has
  // landed and been read) and store rows < M, columns < N.
  __syncthreads();
  float* const part = reinterpret_cast<float*>(ring);
  if (wave < NC) {
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

}  // namespace

bool QMidApplies(const QuantProblem& p) {
  const bool int4 = p.bits == 4 && p.packing == QK_PACK_U32X8;
  const bool int8 = p.bits == 8 && (p.packing == QK_PACK_U8 ||
                                    p.packing == QK_PACK_S8_SYM);
  const int64_t row_bytes = int4 ? p.k / 2 : p.k;
  return p.m >= 1 && p.m <= 128 && (int4 || int8) && p.group == 64 &&
         p.x_dtype == QK_BF16 && p.scale_dtype == QK_BF16 &&
         (!p.has_bias || p.bias_dtype == QK_BF16) && p.k % 256 == 0 &&
         p.k > 0 && p.n > 0 && p.n * row_bytes < (int64_t{1} << 31) &&
         p.m * p.k * 2 < (int64_t{1} << 31) &&
         p.n * (p.k / 64) * 2 < (int64_t{1} << 31) &&
         reinterpret_cast<uintptr_t>(p.x) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.codes) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.scales) % 4 == 0 &&
         (!p.has_bias || reinterpret_cast<uintptr_t>(p.biases) % 4 == 0);
}

qk_status LaunchQMid(const QuantProblem& p, hipStream_t stream) {
  MdArgs a;
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
  // Four K slices, one wave each (one per SIMD), one workgroup per CU.
  constexpr int KW = 4;
  a.gpw = a.groups / KW;  // k % 256 == 0
  const int cus = DeviceComputeUnits();
  // The widest tile (48, 32 or 16 weight rows) that still gives every CU
  // a workgroup.
  const int nb = (a.n + 47) / 48 >= cus ? 3 : (a.n + 31) / 32 >= cus ? 2 : 1;
  const dim3 grid((a.n + 16 * nb - 1) / (16 * nb));
  const int mb = (a.m + 15) / 16;
  // QK_MID_WS=0 selects the kernel whose waves load their own groups
  // (tuning).
  static const bool ws = [] {
    const char* v = std::getenv("QK_MID_WS");
    return v == nullptr || *v != '0';
  }();
  constexpr int kWsThreads = (kMidConsumers + kMidProducers) * 64;
#define QK_MID_NB(P, MB)                                                  \
  do {                                                                    \
    if (ws && nb == 3)                                                    \
      qmm_wsmid_kernel<P, MB, 3><<<grid, kWsThreads, 0, stream>>>(a);     \
    else if (ws && nb == 2)                                               \
      qmm_wsmid_kernel<P, MB, 2><<<grid, kWsThreads, 0, stream>>>(a);     \
    else if (ws)                                                          \
      qmm_wsmid_kernel<P, MB, 1><<<grid, kWsThreads, 0, stream>>>(a);     \
    else if (nb == 3)                                                     \
      qmm_mid_kernel<P, MB, 3, KW><<<grid, KW * 64, 0, stream>>>(a);      \
    else if (nb == 2)                                                     \
      qmm_mid_kernel<P, MB, 2, KW><<<grid, KW * 64, 0, stream>>>(a);      \
    else                                                                  \
      qmm_mid_kernel<P, MB, 1, KW><<<grid, KW * 64, 0, stream>>>(a);      \
  } while (0)
#define QK_MID(P)                                                         \
  do {                                                                    \
    if (mb <= 4) QK_MID_NB(P, 4);                                         \
    else if (mb <= 6) QK_MID_NB(P, 6);                                    \
    else QK_MID_NB(P, 8);                                                 \
  } while (0)
  if (p.packing == QK_PACK_U32X8)
    QK_MID(QK_PACK_U32X8);
  else if (p.packing == QK_PACK_U8)
    QK_MID(QK_PACK_U8);
  else
    QK_MID(QK_PACK_S8_SYM);
#undef QK_MID
#undef QK_MID_NB
  return PostLaunch("qmm_mid");
}

}  // namespace qk
