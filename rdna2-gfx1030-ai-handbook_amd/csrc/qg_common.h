// Shared device helpers for the gfx950 quantized-GEMM kernels.
//
// Every file of this library is compiled for gfx950 only (wave64, CDNA4 MFMA,
// 160 KB LDS per CU) with -ffp-contract=off so that the fp32 epilogues keep
// the reference's separate multiply/add rounding.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/qgemm.h"

namespace qg {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}
// fp32 -> bf16 with round-to-nearest-even (NaN stays a quiet NaN); the same
// rule as c10::BFloat16's round_to_nearest_even.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
// Two fp32 -> packed bf16 (a in the low half) with gfx950's v_cvt_pk_bf16_f32:
// round-to-nearest-even, the bits of f32_to_bf16 for every non-NaN input.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
  typedef __bf16 bf16v2 __attribute__((ext_vector_type(2)));
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16v2));
}
// fp32 -> fp16, hardware conversion (round-to-nearest-even, fp16 denormals kept).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Exact decode of an OCP fp8 byte to fp32, bit for bit the construction of the
// reference decoder (rdna2-ops/rdna2_ops/fp8_weight_gemm_v06.py:21-37):
// e4m3fn: exponent 0 -> m * 2^-9; 0x7f / 0xff -> NaN; else (e+120)<<23 | m<<20.
// e5m2:   exponent 0 -> m * 2^-16; exponent 31 -> inf / NaN; else (e+112)<<23 | m<<21.
__device__ __forceinline__ float fp8_to_f32(uint32_t u, bool e5) {
  const uint32_t sign = (u & 128u) << 24;
  uint32_t bits;
  if (e5) {
    const uint32_t e = (u >> 2) & 31u, m = u & 3u;
    bits = ((e + 112u) << 23) | (m << 21);
    if (e == 0) bits = __float_as_uint(static_cast<float>(m) * 0.0000152587890625f);
    if (e == 31) bits = 0x7f800000u | (m << 21);
  } else {
    const uint32_t e = (u >> 3) & 15u, m = u & 7u;
    bits = ((e + 120u) << 23) | (m << 20);
    if (e == 0) bits = __float_as_uint(static_cast<float>(m) * 0.001953125f);
    if (e == 15 && m == 7) bits = 0x7fc00000u;
  }
  return __uint_as_float(bits | sign);
}

// 8 fp8 bytes (2 dwords) -> 8 bf16 / fp16 values in natural order, with
// gfx950's scaled conversions at scale 1: exact for every e4m3 / e5m2 value
// (both formats are subsets of fp16 and bf16), NaN and infinity included.
template <bool F16A, bool E5>
__device__ __forceinline__ i32x4 fp8x8(uint32_t d0, uint32_t d1) {
  i32x4 r;
  if constexpr (F16A) {
    if constexpr (E5) {
      r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(d0, 1.0f, false));
      r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(d0, 1.0f, true));
      r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(d1, 1.0f, false));
      r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(d1, 1.0f, true));
    } else {
      r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, false));
      r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, true));
      r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, false));
      r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, true));
    }
  } else {
    if constexpr (E5) {
      r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(d0, 1.0f, false));
      r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(d0, 1.0f, true));
      r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(d1, 1.0f, false));
      r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(d1, 1.0f, true));
    } else {
      r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, false));
      r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, true));
      r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, false));
      r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, true));
    }
  }
  return r;
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E). Used
// where every index into a register array must be a constant, independent of
// the unroller's size heuristics (a dynamic index sends the array to scratch).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <typename T>
__host__ __device__ __forceinline__ T ceil_div(T a, T b) { return (a + b - 1) / b; }

// Wave-wide reductions (wave64).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Direct global -> LDS copy of 16 bytes per lane (gfx950 global_load_lds_dwordx4).
// The 64 lanes of the wave write 1 KB of LDS: lane i writes bytes
// [lds_addr + 16 i, lds_addr + 16 i + 16). lds_addr must be wave-uniform.
// Issued through inline assembly so that the compiler does not add its own
// conservative vmcnt(0) waits before later LDS reads; the caller waits with
// wait_vm_barrier<N>() instead. M0 is saved and restored around the load.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(gptr)
      : "memory");
}

// Same copy with a wave-uniform 64-bit base in SGPRs and a per-lane 32-bit
// byte offset (global_load_lds_dwordx4 voffset, saddr): advancing along K only
// touches the scalar base.
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(sbase)
      : "memory");
}

// dma16s with the non-temporal hint, for operands streamed once per launch
// (the W4A16 decode's weights: 7.84-7.95 -> 7.43-7.71 us at cfg2 M = 1, one
// box, alternating runs, same bits).
__device__ __forceinline__ void dma16s_nt(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %3 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(sbase)
      : "memory");
}

// 4-byte variant (global_load_lds_dword): lane i writes bytes
// [lds_addr + 4 i, lds_addr + 4 i + 4); lanes outside the exec mask write nothing.
__device__ __forceinline__ void dma4s(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(sbase)
      : "memory");
}

// 2-byte variant (global_load_lds_ushort): lane i writes the element
// zero-extended to 32 bits at [lds_addr + 4 i, lds_addr + 4 i + 4).
__device__ __forceinline__ void dma2s(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_ushort %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(sbase)
      : "memory");
}

// Wait until at most N vector-memory operations of this wave are in flight
// (loads complete in order), drain LDS reads, then barrier the workgroup.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Wait until at most N vector-memory operations of this wave are in flight,
// without a barrier.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Drain this wave's LDS reads, then barrier the workgroup.
__device__ __forceinline__ void wait_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 32-bit LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
  return static_cast<uint32_t>(
      (uintptr_t)((const __attribute__((address_space(3))) char*)(p)));
}

}  // namespace qg
