// Per-row INT8 quantization shared by the quantizer kernels (quant.hip) and
// the MoE routing kernel that quantizes each token's row (moe.hip).
//   step = max(absmax / 127, 1e-20)          (IEEE fp32 division)
//   q = clamp(round(x / step), -127, 127)    (round of the IEEE quotient)
// The step formula and the half-away rounding follow the reference's
// in-tree quantizer rdna2-ops/rdna2_ops/fp8_weight_gemm_v06.py:76-92; the
// half-even mode is the per-token rule of the benchmark (absmax/127, round-half-even).
#pragma once
#include "qg_common.h"
#include "qg_internal.h"

namespace qg {

namespace {

template <int XT>
struct XType;
template <> struct XType<QG_F32> { static constexpr int size = 4; };
template <> struct XType<QG_F16> { static constexpr int size = 2; };
template <> struct XType<QG_BF16> { static constexpr int size = 2; };
template <> struct XType<QG_E4M3> { static constexpr int size = 1; };
template <> struct XType<QG_E5M2> { static constexpr int size = 1; };

template <int XT>
__device__ __forceinline__ float load_x(const char* base, int64_t idx) {
  if constexpr (XT == QG_F32) return reinterpret_cast<const float*>(base)[idx];
  else if constexpr (XT == QG_F16) return f16_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
  else if constexpr (XT == QG_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
  else return fp8_to_f32(reinterpret_cast<const uint8_t*>(base)[idx], XT == QG_E5M2);
}

// Decode the 16/size elements of one 16-byte chunk.
template <int XT>
__device__ __forceinline__ void decode_chunk(const i32x4 c, float* v) {
  constexpr int E = 16 / XType<XT>::size;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t word = static_cast<uint32_t>(c[(e * XType<XT>::size) / 4]);
    if constexpr (XT == QG_F32) v[e] = __uint_as_float(word);
    else if constexpr (XT == QG_F16) v[e] = f16_to_f32(static_cast<uint16_t>(word >> (16 * (e & 1))));
    else if constexpr (XT == QG_BF16) v[e] = bf16_to_f32(static_cast<uint16_t>(word >> (16 * (e & 1))));
    else v[e] = fp8_to_f32((word >> (8 * (e & 3))) & 0xffu, XT == QG_E5M2);
  }
}

template <int MODE>
__device__ __forceinline__ int quant_one(float x, float step) {
#pragma clang fp contract(off)
  const float z = __fdiv_rn(x, step);
  float q;
  if constexpr (MODE == QG_ROUND_HALF_EVEN) {
    q = __builtin_rintf(z);
  } else {
    q = z >= 0.0f ? floorf(z + 0.5f) : ceilf(z - 0.5f);
  }
  q = fminf(fmaxf(q, -127.0f), 127.0f);
  return static_cast<int>(q);
}

// Fast rounding of z = x * rstep (relative error below 1.5 * 2^-23, i.e. below
// 2^-15.5 for |z| < 128): clamp to +-127, then adding 1.5 * 2^23 rounds to the
// nearest integer n, whose two's-complement byte is the low byte of the sum's
// bits. n is the rounded exact quotient, in both modes, unless z lies within
// 2^-13 of a half-integer (|z - n| > 1/2 - 2^-13); such chunks are redone with
// the IEEE quotient.
constexpr float kRoundMagic = 12582912.0f;            // 1.5 * 2^23
constexpr float kRiskyDist = 0.5f - 0.0001220703125f;  // 1/2 - 2^-13

// Quantize the 16-byte chunk `raw` (16 / size elements) with `step` and
// rstep = rcp(step) and, when `store`, write its codes as chunk c of row qr:
// the reciprocal quotient rounds every element unless one of them lies within
// 2^-13 of a half-integer, in which case the chunk is redone with the IEEE
// quotient (so the codes are those of the exact quotient).
// quant_values_store: the same for E (4, 8 or 16) fp32 values already in
// registers (chunk c of E codes).
template <int E, int MODE>
__device__ __forceinline__ void quant_values_store(const float (&v)[E], float step, float rstep, int8_t* qr, int c,
                                                   bool store) {
#pragma clang fp contract(off)
  uint32_t b[E];
  float dmax = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float z = v[e] * rstep;
    const float m = fminf(fmaxf(z, -127.0f), 127.0f) + kRoundMagic;
    dmax = fmaxf(dmax, fabsf(z - (m - kRoundMagic)));
    b[e] = __float_as_uint(m);
  }
  const bool risky = dmax > kRiskyDist;
  if (__builtin_expect(__any(risky), 0)) {
    if (risky) {
#pragma unroll
      for (int e = 0; e < E; ++e) b[e] = static_cast<uint32_t>(quant_one<MODE>(v[e], step));
    }
  }
  // low bytes of 4 words -> one word (byte e of the result = byte 0 of b[e])
  uint32_t packed[E / 4 > 0 ? E / 4 : 1];
#pragma unroll
  for (int w = 0; w < E / 4; ++w) {
    const uint32_t lo = __builtin_amdgcn_perm(b[4 * w + 1], b[4 * w], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(b[4 * w + 3], b[4 * w + 2], 0x04000c0cu);
    packed[w] = lo | hi;
  }
  if (store) {
    if constexpr (E == 4) reinterpret_cast<uint32_t*>(qr)[c] = packed[0];
    else if constexpr (E == 8) reinterpret_cast<uint2*>(qr)[c] = make_uint2(packed[0], packed[1]);
    else reinterpret_cast<uint4*>(qr)[c] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  }
}

template <int XT, int MODE>
__device__ __forceinline__ void quant_chunk_store(const i32x4 raw, float step, float rstep, int8_t* qr, int c,
                                                  bool store) {
  constexpr int E = 16 / XType<XT>::size;
  float v[E];
  decode_chunk<XT>(raw, v);
  quant_values_store<E, MODE>(v, step, rstep, qr, c, store);
}

}  // namespace

}  // namespace qg
