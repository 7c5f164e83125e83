// Interior-tile f16/bf16 GEMM whose operand tiles travel from global memory
// straight into LDS (gfx950 `buffer_load_dwordx4 ... lds`), used by the
// dense GEMM for problems whose N and K are multiples of BN x 64 (BN =
// 256, 192 or 128; any M) with 16-byte aligned operands. Replaces the tiled loop
// of the reference's steel GEMM (metal_pjrt/kernels/steel_gemm.metal:
// 180-213) for those shapes; the store applies the same epilogue.
//
// Layout and schedule:
//  - Two LDS stages, each a separate __shared__ array holding the A tile
//    (256 x 64) and the B tile (BN x 64) unpadded. A 16-byte LDS DMA of one
//    wave writes 1024 consecutive bytes (lane L at byte 16 L), so bank
//    conflicts are avoided by choosing which global 16-byte chunk each lane
//    fetches (an XOR swizzle), not by padding:
//      K-contiguous operand (A; B stored [N][K]): row r of 128 bytes holds
//        K chunk c (8 elements) in slot c ^ ((r >> 1) & 7);
//      M/N-contiguous operand (B stored [K][N]; A stored [K][M]): K row k
//        of R elements holds chunk c in slot c ^ 4 (k & 3) (c ^ 2 (k & 3)
//        for 64-element rows).
//    K-contiguous fragments are one 16-byte LDS read per lane; the others
//    are read with the transposing ds_read_b64_tr_b16 (two per fragment).
//    Both read patterns spread each 16-lane group over all 64 banks
//    (rocprofv3 SQ_LDS_BANK_CONFLICT reads 0 at 4096^3).
//  - Four waves (2 x 2), each owning 128 x BN/2 of the tile (32x32
//    blocks, v_mfma_f32_32x32x16_{bf16,f16}), fragments double-buffered in
//    registers with the LDS reads of K step s + 1 interleaved with the
//    MFMAs of step s.
//  - One barrier per K tile, between its K steps 2 and 3: before it each
//    wave waits for its own DMA of the next tile (vmcnt 0), after it no
//    wave reads the current stage any more (step 3's fragments are in
//    registers), so the DMA of tile kt + 2 into the current stage is
//    issued during step 3, one instruction per MFMA, together with the
//    fragment reads of the next stage's first K step. Each DMA has a whole
//    tile of MFMA work to land.
//  - The DMA instructions are written as inline asm: the compiler's
//    wait-count pass would otherwise make the transposing reads of one
//    stage (an intrinsic whose memory operand carries no alias scope)
//    wait for the DMA into the other. Their completion is awaited
//    explicitly before each barrier and before the kernel ends.
//  - The epilogue is applied from the accumulators (store_direct).
//  - K split over workgroups (g.ksplit > 1, one batch entry, for grids
//    whose tiles alone would leave CUs idle): workgroup (tile, z =
//    blockIdx.z) takes K tiles z T / ksplit .. (z + 1) T / ksplit and the
//    partial tiles meet in split_k_store (summed in K order by the last
//    to arrive).
#pragma once

#include "gemm_common.h"

namespace qk {
namespace {

// Swizzles of the 16-byte chunks of an LDS operand row. K-contiguous
// rows of 128 bytes (two per 256-byte bank row): chunk c of row r sits in
// slot c ^ ((r >> 1) & 7), so the 16 rows a 16-lane group reads at one K
// chunk cover all 64 banks once. M/N-contiguous K rows of 256 bytes or
// more (LPR >= 16 chunks, every K row on the same banks): chunk c of K row
// k sits in slot c ^ 4 (k & 3), so the four K rows of a transposing
// 16-lane read (two chunks each, in 16 chunk slots) meet no bank twice;
// 128-byte K rows keep c ^ 2 (k & 3) (two K rows per bank row).
__device__ __forceinline__ constexpr int SwzK(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ constexpr int SwzMN(int k, int lpr) {
  return lpr >= 16 ? (k & 3) << 2 : (k & 3) << 1;
}

// Operand tile of R rows x 64 K, K-contiguous in memory (row stride ld
// elements): R / 32 DMA instructions per wave; instruction i of wave w
// fills rows (4 i + w) * 8 .. + 8.
// VC: the whole offset goes in the vector offset, which the descriptor's
// extent checks (for tiles that run past the operand's last row).
template <typename T, int R, int NW = 4, bool VC = false>
struct DmaK {
  static constexpr int NI = R / (8 * NW);
  static constexpr int kBytes = R * 128;
  DmaRsrc rs;
  int voff, ld;
  __device__ __forceinline__ void init(const T* src, long long bytes, int ld_,
                                       int w, int lane) {
    rs.make(src, bytes);
    ld = ld_;
    voff = ((w * 8 + lane / 8) * ld + ((lane % 8) ^ SwzK(w * 8 + lane / 8)) * 8) *
           static_cast<int>(sizeof(T));
  }
  __device__ __forceinline__ void issue(unsigned char* lds, int r0, int k0,
                                        int w, int i) const {
    const int so = ((r0 + i * 8 * NW) * ld + k0) * static_cast<int>(sizeof(T));
    if constexpr (VC)
      rs.dma(lds + (i * NW + w) * 1024, voff + so, 0);
    else
      rs.dma(lds + (i * NW + w) * 1024, voff, so);
  }
  // Fragment for rows rb .. rb + 31 (rb % 32 == 0), K elements kb + 8 (lane
  // / 32) .. + 7.
  __device__ __forceinline__ static typename Frag<T>::type frag(
      const unsigned char* lds, int rb, int kb, int lane) {
    const int r = rb + (lane & 31);
    const int c = (kb >> 3) + (lane >> 5);
    return *reinterpret_cast<const typename Frag<T>::type*>(
        lds + r * 128 + ((c ^ SwzK(r)) << 4));
  }
};

// Operand tile of 64 K rows x R elements, R-contiguous in memory (K row
// stride ld elements): K row k occupies R * sizeof(T) bytes; a DMA
// instruction covers RPI K rows, instruction i of wave w fills K rows
// (4 i + w) * RPI .. + RPI.
template <typename T, int R, int NW = 4, bool VC = false>
struct DmaMN {
  static constexpr int RB = R * static_cast<int>(sizeof(T));  // row bytes
  static constexpr int LPR = RB / 16;                         // lanes per row
  static constexpr int RPI = 64 / LPR;  // K rows per instruction
  static constexpr int NI = 64 / RPI / NW;
  static constexpr int kBytes = 64 * RB;
  static_assert(LPR >= 8 && 64 % LPR == 0, "row must span 8..64 chunks");
  DmaRsrc rs;
  int voff, ld;
  __device__ __forceinline__ void init(const T* src, long long bytes, int ld_,
                                       int w, int lane) {
    rs.make(src, bytes);
    ld = ld_;
    const int k = w * RPI + lane / LPR;  // k & 3 is the same for every i
    static_assert((NW * RPI) % 4 == 0, "swizzle phase per instruction");
    voff = (k * ld + ((lane % LPR) ^ SwzMN(k, LPR)) * 8) *
           static_cast<int>(sizeof(T));
  }
  __device__ __forceinline__ void issue(unsigned char* lds, int r0, int k0,
                                        int w, int i) const {
    const int so = ((k0 + i * NW * RPI) * ld + r0) * static_cast<int>(sizeof(T));
    if constexpr (VC)
      rs.dma(lds + (i * NW + w) * 1024, voff + so, 0);
    else
      rs.dma(lds + (i * NW + w) * 1024, voff, so);
  }
  // Fragment for columns rb .. rb + 31 and K kb .. kb + 15 with the
  // transposing read (lane s of a 16-lane group addresses K row
  // kb + 8 (g / 2) + s / 4, columns rb + 16 (g % 2) + 4 (s % 4) .. + 3).
  __device__ __forceinline__ static typename Frag<T>::type frag(
      const unsigned char* lds, int rb, int kb, int lane) {
    const int g = lane >> 4, s = lane & 15;
    const int k = kb + 8 * (g >> 1) + (s >> 2);
    const int n = rb + 16 * (g & 1) + 4 * (s & 3);
    const unsigned char* p =
        lds + k * RB + (((n >> 3) ^ SwzMN(k, LPR)) << 4) + (n & 7) * 2;
    const u32x2 lo = lds_read_tr(reinterpret_cast<const T*>(p));
    const u32x2 hi = lds_read_tr(reinterpret_cast<const T*>(p + 4 * RB));
    const u32x4 q = {lo[0], lo[1], hi[0], hi[1]};
    return __builtin_bit_cast(typename Frag<T>::type, q);
  }
};

// A 192-column M/N-contiguous tile as two DmaMN regions, columns 0..127
// (256-byte K rows) and 128..191 (128-byte K rows): 4 + 2 DMA instructions
// per wave. Every 32-column fragment lies in one region.
template <typename T, int NW = 4>
struct DmaMN192 {
  using Lo = DmaMN<T, 128, NW>;
  using Hi = DmaMN<T, 64, NW>;
  static constexpr int NI = Lo::NI + Hi::NI;
  static constexpr int kBytes = Lo::kBytes + Hi::kBytes;
  Lo lo;
  Hi hi;
  __device__ __forceinline__ void init(const T* src, long long bytes, int ld_,
                                       int w, int lane) {
    lo.init(src, bytes, ld_, w, lane);
    hi.init(src, bytes, ld_, w, lane);
  }
  __device__ __forceinline__ void issue(unsigned char* lds, int r0, int k0,
                                        int w, int i) const {
    if (i < Lo::NI)
      lo.issue(lds, r0, k0, w, i);
    else
      hi.issue(lds + Lo::kBytes, r0 + 128, k0, w, i - Lo::NI);
  }
  __device__ __forceinline__ static typename Frag<T>::type frag(
      const unsigned char* lds, int rb, int kb, int lane) {
    // rb is wave-uniform: pick the region without a branch
    const bool h = rb >= 128;
    const int RB = h ? Hi::RB : Lo::RB;
    const unsigned char* base = h ? lds + Lo::kBytes : lds;
    const int g = lane >> 4, s = lane & 15;
    const int k = kb + 8 * (g >> 1) + (s >> 2);
    const int n = (h ? rb - 128 : rb) + 16 * (g & 1) + 4 * (s & 3);
    const unsigned char* p =
        base + k * RB + (((n >> 3) ^ SwzMN(k, RB / 16)) << 4) + (n & 7) * 2;
    const u32x2 lo2 = lds_read_tr(reinterpret_cast<const T*>(p));
    const u32x2 hi2 = lds_read_tr(reinterpret_cast<const T*>(p + 4 * RB));
    const u32x4 q = {lo2[0], lo2[1], hi2[0], hi2[1]};
    return __builtin_bit_cast(typename Frag<T>::type, q);
  }
};


// MC: M need not be a multiple of 256. The A tile's DMA offsets go wholly
// in the range-checked vector offset (rows, or M-contiguous columns, past
// the operand's extent read zeros) and the epilogue skips rows past M;
// values fetched for rows past M (in range of the extent) only reach
// those skipped rows.
template <typename T, int BN, bool TA, bool TB, int NWV = 4, bool MC = false>
__global__ __launch_bounds__(NWV * 64) void gemm_dma_kernel(GemmArgs g) {
  constexpr int BM = 256, BK = 64, WN = 2, WM = NWV / WN;
  constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 32, FN = WTN / 32;
  using LA = std::conditional_t<TA, DmaMN<T, BM, NWV, MC>,
                                DmaK<T, BM, NWV, MC>>;
  using LB = std::conditional_t<
      TB, DmaK<T, BN, NWV>,
      std::conditional_t<BN == 192, DmaMN192<T, NWV>, DmaMN<T, BN, NWV>>>;
  constexpr int kBOff = LA::kBytes;
  constexpr int kStage = LA::kBytes + LB::kBytes;
  constexpr int kDma = LA::NI + LB::NI;  // DMA instructions per wave per tile
  // DMA instructions after each MFMA of the last K step.
  constexpr int kDmaPer = (kDma + FM * FN - 1) / (FM * FN);
  __shared__ __attribute__((aligned(1024))) unsigned char st0[kStage];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[kStage];

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
  const int m0 = tm * BM, n0 = tn * BN;
  const long long batch = blockIdx.y;
  const int ktiles = g.k / BK;  // >= 1
  const int z = blockIdx.z;
  const int kbeg = z * ktiles / g.ksplit;
  const int kend = (z + 1) * ktiles / g.ksplit;  // > kbeg: ksplit <= ktiles

  LA la;
  LB lb;
  la.init(static_cast<const T*>(g.a) + batch * g.bsa,
          static_cast<long long>(TA ? g.k : g.m) * g.lda * sizeof(T), g.lda,
          wave, lane);
  lb.init(static_cast<const T*>(g.b) + batch * g.bsb,
          static_cast<long long>(TB ? g.n : g.k) * g.ldb * sizeof(T), g.ldb,
          wave, lane);
  auto issue_all = [&](unsigned char* st, int k0) {
#pragma unroll
    for (int i = 0; i < LA::NI; ++i) la.issue(st, m0, k0, wave, i);
#pragma unroll
    for (int i = 0; i < LB::NI; ++i) lb.issue(st + kBOff, n0, k0, wave, i);
  };
  typename Frag<T>::type fa[2][FM], fb[2][FN];
  auto frag_a = [&](const unsigned char* st, int i, int kb) {
    return LA::frag(st, wm * WTM + i * 32, kb, lane);
  };
  auto frag_b = [&](const unsigned char* st, int j, int kb) {
    return LB::frag(st + kBOff, wn * WTN + j * 32, kb, lane);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  issue_all(st0, kbeg * BK);
  issue_all(st1, min(kbeg + 1, kend - 1) * BK);
  __builtin_amdgcn_s_waitcnt(VmcntImm(kDma));  // tile 0 has landed
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = frag_a(st0, i, 0);
#pragma unroll
  for (int j = 0; j < FN; ++j) fb[0][j] = frag_b(st0, j, 0);

  // LDS reads per K step (a transposing fragment read is two).
  constexpr int kReads = FM * (TA ? 2 : 1) + FN * (TB ? 1 : 2);
  // Tile kt from stage cs; the next tile is in (or landing in) ns.
  auto tile = [&](unsigned char* cs, unsigned char* ns, int kt) {
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      const int fc = s & 1, fn = fc ^ 1;
#pragma unroll
      for (int i = 0; i < FM; ++i) fa[fn][i] = frag_a(cs, i, (s + 1) * 16);
#pragma unroll
      for (int j = 0; j < FN; ++j) fb[fn][j] = frag_b(cs, j, (s + 1) * 16);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], fa[fc][i], fb[fc][j]);
      // One MFMA, then one DS read.
#pragma unroll
      for (int q = 0; q < FM * FN; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (q < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    // The next tile has landed (own DMA: vmcnt; everyone's: barrier), and
    // after the barrier nobody reads cs: step 3 runs from registers.
    __builtin_amdgcn_s_waitcnt(VmcntImm(0));
    __syncthreads();
    const int k2 = min(kt + 2, kend - 1) * BK;
    // Step 3: each MFMA is followed by kDmaPer DMAs of tile kt + 2 into cs
    // and one fragment read of the next tile's first K step from ns, pinned in
    // that order by scheduling barriers.
#pragma unroll
    for (int q = 0; q < FM * FN; ++q) {
      const int i = q / FN, j = q % FN;
      mma(acc[i][j], fa[1][i], fb[1][j]);
#pragma unroll
      for (int d = q * kDmaPer; d < (q + 1) * kDmaPer; ++d) {
        if (d < LA::NI)
          la.issue(cs, m0, k2, wave, d);
        else if (d < kDma)
          lb.issue(cs + kBOff, n0, k2, wave, d - LA::NI);
      }
      if (q < FM)
        fa[0][q] = frag_a(ns, q, 0);
      else if (q < FM + FN)
        fb[0][q - FM] = frag_b(ns, q - FM, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int kt = kbeg;
  for (; kt + 1 < kend; kt += 2) {
    tile(st0, st1, kt);
    tile(st1, st0, kt + 1);
  }
  if (kt < kend) tile(st0, st1, kt);
  // No DMA may still be writing this workgroup's LDS when it ends.
  __builtin_amdgcn_s_waitcnt(VmcntImm(0));
  if (g.ksplit > 1) {
    __syncthreads();  // every wave is done with st0 (the arrival word)
    split_k_store<T, BM, BN, WM, WN, MC, NWV * 64>(
        g, acc, blockIdx.x, z, m0, n0, tid, lane, wm, wn,
        reinterpret_cast<uint32_t*>(st0));
  } else {
    store_direct<T, BM, BN, WM, WN, MC>(g, acc, m0, n0, batch, lane, wm, wn);
  }
}

}  // namespace
}  // namespace qk
