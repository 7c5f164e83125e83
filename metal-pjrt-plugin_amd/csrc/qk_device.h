// Device-side helpers shared by the gfx950 kernels: element conversion,
// activations, wavefront reductions and LDS DMA.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qk {

typedef __bf16 bf16;
typedef _Float16 f16;

// Element conversions. f32 -> bf16/f16 round to nearest even (the gfx950
// conversion instructions), NaN stays NaN.
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, v))
                         << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) {
  return static_cast<f16>(v);
}
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) {
  return static_cast<bf16>(v);
}

typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Reinterprets 32 bits as two bf16. The argument is a plain value on
// purpose: clang (ROCm 7.2) miscompiles __builtin_bit_cast applied directly
// to an element of an ext_vector_type (it reads element 0 for every index).
__device__ __forceinline__ bf16x2 AsBf16x2(uint32_t u) {
  return __builtin_bit_cast(bf16x2, u);
}

// Loads element i of a float buffer whose type is chosen at run time
// (0 f32, 1 f16, 2 bf16: the qk_dtype values).
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  if (dtype == 2) return to_f32(static_cast<const bf16*>(p)[i]);
  if (dtype == 1) return to_f32(static_cast<const f16*>(p)[i]);
  return static_cast<const float*>(p)[i];
}
__device__ __forceinline__ void store_any(void* p, int64_t i, int dtype,
                                          float v) {
  if (dtype == 2)
    static_cast<bf16*>(p)[i] = from_f32<bf16>(v);
  else if (dtype == 1)
    static_cast<f16*>(p)[i] = from_f32<f16>(v);
  else
    static_cast<float*>(p)[i] = v;
}

// 1 / (1 + e^-t) from the hardware base-2 exponential and reciprocal
// (each within 1 ulp): t = -inf gives 0, t = +inf gives 1, NaN stays NaN.
__device__ __forceinline__ float sigmoid_f32(float t) {
  const float e = __builtin_amdgcn_exp2f(t * -1.4426950408889634f);  // e^-t
  return __builtin_amdgcn_rcpf(1.0f + e);
}

// cuBLASLt epilogue activations, in f32 (the reference's steel_act,
// metal_pjrt/kernels/steel_gemm.metal:57-66): ReLU keeps NaN, GELU is the
// tanh form, SiLU is x / (1 + exp(-x)). Both smooth activations are
// evaluated as x * sigmoid(.): 0.5 (1 + tanh(u)) = 1 / (1 + e^-2u), so
// GELU(x) = x * sigmoid(2u) with u = sqrt(2/pi) (x + 0.044715 x^3). The
// infinities give what the quotient forms give (+inf -> +inf, -inf -> NaN).
__device__ __forceinline__ float act_f32(int act, float x) {
  if (act == 1) return x != x ? x : (x > 0.0f ? x : 0.0f);
  if (act == 2) {
    const float k2 = 2.0f * 0.7978845608028654f;  // 2 sqrt(2/pi)
    return x * sigmoid_f32(k2 * (x + 0.044715f * x * x * x));
  }
  if (act == 3) return x * sigmoid_f32(x);
  return x;
}

// A 32-bit constant held in a VGPR. gfx9 VOP3 instructions (v_and_or_b32,
// v_bfi_b32, ...) take no literal operand and at most one SGPR, so a
// literal mask used by them would be split into two VOP2 instructions.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}

// 64-bit logical right shift by a constant as one v_lshrrev_b64 (the
// compiler would otherwise split it into a funnel shift and a shift).
template <int kS>
__device__ __forceinline__ uint64_t shr64(uint64_t v) {
  uint64_t r;
  asm("v_lshrrev_b64 %0, %1, %2" : "=v"(r) : "i"(kS), "v"(v));
  return r;
}

// Sum over the 64 lanes of a wavefront with DPP row operations (quad
// swaps, half-row and row mirrors) and four lane reads; the result is
// wave-uniform.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl,
                                         0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror: every lane holds its row's sum
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

// Sums of four values over the 64 lanes of a wavefront at once: lane l
// returns the total of value (l & 3). Two quad-transpose steps leave each
// lane with the quad sum of one value, two DPP rotations within rows of
// 16 and two cross-row swaps finish the sum: 10 cross-lane operations in
// all instead of 4 x 8.
__device__ __forceinline__ float wave_sum4(float a0, float a1, float a2,
                                           float a3, int lane) {
  const bool b0 = lane & 1, b1 = lane & 2;
  const float v01 = (b0 ? a1 : a0) + dpp_f32<0xB1>(b0 ? a0 : a1);
  const float v23 = (b0 ? a3 : a2) + dpp_f32<0xB1>(b0 ? a2 : a3);
  float v = (b1 ? v23 : v01) + dpp_f32<0x4E>(b1 ? v01 : v23);
  v += dpp_f32<0x124>(v);  // row_ror:4
  v += dpp_f32<0x128>(v);  // row_ror:8
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// Sum / max over the 64 lanes of a wavefront; every lane gets the result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// LDS DMA (buffer_load ... lds) of 16 or 4 bytes per lane into
// lds + lane * size, as device-only helpers (the address-space cast of the
// LDS pointer is not valid host code). The Nt form reads nontemporally
// (data streamed once).
using LdsPtr = __attribute__((address_space(3))) void*;
__device__ __forceinline__ void DmaLds16(__amdgpu_buffer_rsrc_t r,
                                         unsigned char* lds, int voff,
                                         int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)lds, 16, voff, soff, 0,
                                           0);
}
__device__ __forceinline__ void DmaLds16Nt(__amdgpu_buffer_rsrc_t r,
                                           unsigned char* lds, int voff,
                                           int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)lds, 16, voff, soff, 0,
                                           2);
}
__device__ __forceinline__ void DmaLds4(__amdgpu_buffer_rsrc_t r,
                                        unsigned char* lds, int voff,
                                        int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)lds, 4, voff, soff, 0,
                                           0);
}

// s_waitcnt immediate for vmcnt(n) (expcnt, lgkmcnt not waited).
constexpr int VmcntImm(int n) {
  return (n & 0xF) | (((n >> 4) & 3) << 14) | (7 << 4) | (0xF << 8);
}

// Raw buffer descriptor in SGPRs (base, extent in bytes, raw access) whose
// LDS DMA is issued as inline asm: the compiler's wait-count pass does not
// see it, so it adds no waits of its own for it (it would otherwise make
// LDS reads it cannot tell apart from the DMA's destination wait for every
// DMA in flight); the caller waits explicitly (s_waitcnt vmcnt) before
// reading what a DMA wrote. Lane L's bytes from byte voff + soff of the
// buffer land at lds + L * size.
struct DmaRsrc {
  uint32_t d __attribute__((ext_vector_type(4)));
  __device__ __forceinline__ void make(const void* p, long long bytes) {
    const unsigned long long a = reinterpret_cast<unsigned long long>(p);
    d[0] = static_cast<uint32_t>(a);
    d[1] = static_cast<uint32_t>(a >> 32) & 0xFFFFu;
    d[2] = static_cast<uint32_t>(bytes);
    d[3] = 0x00020000u;
  }
  static __device__ __forceinline__ uint32_t lds_addr(unsigned char* lds) {
    using LdsBytes = __attribute__((address_space(3))) unsigned char*;
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((LdsBytes)lds));
  }
  // 16 bytes per lane.
  __device__ __forceinline__ void dma(unsigned char* lds, int voff,
                                      int soff) const {
    asm volatile(
        "s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
        :
        : "v"(voff), "s"(d), "s"(soff), "s"(lds_addr(lds))
        : "memory", "m0");
  }
  // 16 bytes per lane, nontemporal (data streamed once).
  __device__ __forceinline__ void dma_nt(unsigned char* lds, int voff,
                                         int soff) const {
    asm volatile(
        "s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds"
        :
        : "v"(voff), "s"(d), "s"(soff), "s"(lds_addr(lds))
        : "memory", "m0");
  }
  // 4 bytes per lane.
  __device__ __forceinline__ void dma4(unsigned char* lds, int voff,
                                       int soff) const {
    asm volatile(
        "s_mov_b32 m0, %3\n\tbuffer_load_dword %0, %1, %2 offen lds"
        :
        : "v"(voff), "s"(d), "s"(soff), "s"(lds_addr(lds))
        : "memory", "m0");
  }
};

// Volatile 32-bit LDS accesses (flags polled by other waves of the
// workgroup) through an LDS-typed pointer: as generic pointers they would
// become flat accesses, which count in the memory counter too.
__device__ __forceinline__ uint32_t LdsLoadVolatile(const uint32_t* p) {
  using P = const volatile __attribute__((address_space(3))) uint32_t*;
  return *(P)p;
}
__device__ __forceinline__ void LdsStoreVolatile(uint32_t* p, uint32_t v) {
  using P = volatile __attribute__((address_space(3))) uint32_t*;
  *(P)p = v;
}

// Bit set in the device status word when a wait between the producer and
// consumer waves of a workgroup gave up.
constexpr uint32_t kStatusSpinTimeout = 1u;

// A bounded wait for an LDS flag written by another wave of the workgroup:
// polls until *f == want, at most `limit` polls. A wave that gives up sets
// the workgroup's *late word and goes on, so the kernel still ends; the
// workgroup then stores NaN outputs and reports the timeout through
// ReportLate.
__device__ __forceinline__ void SpinUntil(const uint32_t* f, uint32_t want,
                                          int limit, uint32_t* late) {
  for (int it = 0; it < limit; ++it) {
    if (__builtin_amdgcn_readfirstlane(LdsLoadVolatile(f)) == want) return;
    __builtin_amdgcn_s_sleep(1);
  }
  LdsStoreVolatile(late, 1u);
}

// Called by one lane once the workgroup's waits are over: a workgroup that
// gave up a wait ORs kStatusSpinTimeout into the device status word (a
// global atomic, read back by qk_device_error()).
__device__ __forceinline__ void ReportLate(const uint32_t* late,
                                           uint32_t* status) {
  if (LdsLoadVolatile(late) != 0u)
    __hip_atomic_fetch_or(status, kStatusSpinTimeout, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace qk
