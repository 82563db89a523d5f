// INT8 x INT8 -> INT32 GEMM on gfx950 int8 MFMA with the fused dequant
// epilogue of rdna2-ops/rdna2_ops/int8_gemm.py:19-67 (and the Kitchen eager
// epilogue order of rdna2-ops/rdna2_ops/comfy_int8.py:128-143).
//
// Design (MI355X-first, not a translation of the reference's Triton tiles):
//  * one workgroup per BM x BN output tile, its waves on a WGM x WGN grid;
//    each wave owns a (BM/WGM) x (BN/WGN) sub-tile held in 32x32 int32 MFMA
//    accumulators (v_mfma_i32_32x32x32_i8, 16 accumulator registers each);
//  * operands are A [M, K] and W [N, K], both K-contiguous ("NT"), so every
//    lane feeds the MFMA with 16 contiguous K bytes of one row;
//  * K advances in 128-byte stages (four 32-byte MFMA k-steps). Each stage of
//    A and W is copied straight from HBM into a 2-slot LDS ring with
//    global_load_lds_dwordx4, 8 rows x 128 B (whole cache lines) per wave
//    instruction — the access pattern that sustains the most L2->LDS bandwidth
//    per CU on gfx950;
//  * the direct copy path sustains ~37 B/clk per CU (one 1 KB copy per ~28
//    cycles) whatever the depth in flight, about what a 256 x 192 tile needs at
//    the full MFMA rate, and a wave blocked issuing a copy cannot issue MFMAs.
//    Two pipelines:
//      - 8 waves, two per SIMD, in two groups that alternate every half
//        stage between a burst of MFMAs and reading / copying the next
//        stage ("ping-pong", large problems and the grouped MoE GEMM);
//        their accumulators hold the transposed tile so that each lane owns
//        runs of 4 adjacent output columns (paired conversions, vector LDS
//        staging in the epilogue);
//      - 4 waves (1 per SIMD) stage the whole next stage in registers while
//        the current one computes, two barriers per stage (small tiles, two
//        workgroups per CU); past the end it re-copies the last stage into
//        its own slot (identical bytes) to keep its waits branch-free;
//  * LDS rows are 128 bytes with the 16-byte chunk index XOR-swizzled by
//    ((row >> 1) & 7): the DMA writes whole 1 KB blocks and every group of 16
//    lanes of a fragment read touches 16 distinct 16-byte bank groups;
//  * the linear block id is remapped so that each of the 8 XCDs (round-robin
//    workgroup dispatch) walks one contiguous, GROUP_M-ordered range of tiles,
//    keeping the A rows and W columns it shares in its own L2;
//  * the per-row / per-column scales and the bias reach LDS before the K
//    loop (the 4-wave kernel through registers; the ping-pong kernels by
//    direct copies into one of two parameter buffers) for the epilogue, which
//    is specialised at compile time (output dtype x order) and, for full
//    tiles, stages the rounded tile through LDS so that HBM sees coalesced
//    16-byte row stores.
#include "qg_common.h"
#include "qg_internal.h"

namespace qg {

namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// The MFMA of the ping-pong main loop, W fragment first (transposed
// accumulator): int8 32x32x32 -> int32, or 2-byte 32x32x16 -> fp32. Both take
// a 16-byte fragment per lane (row l & 31, K chunk l >> 5 of the k-step), so
// the ring layout, copies and fragment offsets are the same for both.
struct MfmaI8 {
  using acc_t = i32x16;
  static __device__ __forceinline__ acc_t mfma(const i32x4& w, const i32x4& a, const acc_t& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(w, a, c, 0, 0, 0);
  }
};
template <bool F16>
struct MfmaHalf {
  using acc_t = f32x16;
  static __device__ __forceinline__ acc_t mfma(const i32x4& w, const i32x4& a, const acc_t& c) {
    if constexpr (F16)
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, w), __builtin_bit_cast(f16x8, a), c,
                                                    0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), __builtin_bit_cast(bf16x8, a),
                                                     c, 0, 0, 0);
  }
};

// fp16 / bf16 MFMA whose W fragments arrive as fp8 and are converted in
// registers (fp8x8, exact).
template <bool F16, bool E5_>
struct MfmaHalfF8W : MfmaHalf<F16> {
  static constexpr bool F16A = F16, E5 = E5_;
};

enum EpiMode { EPI_INT = 0, EPI_F = 1, EPI_FMA = 2, EPI_EAGER = 3, EPI_GELU = 4 };

// Tile geometry: BM x BN output tile, WGM x WGN waves, A ring of NA slots and
// W ring of 2 slots of 128-byte K stages, epilogue parameters after the rings.
template <int BM_, int BN_, int WGM_, int WGN_, int NA_>
struct I8Geo {
  static constexpr int BM = BM_, BN = BN_, NA = NA_, WGM = WGM_, WGN = WGN_;
  static constexpr int NW = WGM * WGN, THREADS = 64 * NW;
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // wave sub-tile
  static constexpr int FM = WM / 32, FN = WN / 32;    // 32x32 blocks per wave
  static constexpr int KS = 128;                      // K bytes per stage
  static constexpr int KT = KS / 32;                  // MFMA k-steps per stage
  static constexpr bool W8 = false;                   // W stored as fp8 (1 byte per 2-byte A element)
  static constexpr int STAGE_A = BM * KS, STAGE_B = BN * KS;
  static constexpr int A_SEGS = BM / 8 / NW, B_SEGS = BN / 8 / NW;  // 1 KB copies per wave and stage
  static constexpr int SPW = A_SEGS + B_SEGS;
  static constexpr int RING_B = NA * STAGE_A;
  static constexpr int RING = RING_B + 2 * STAGE_B;
  static constexpr int SC_A = RING;
  static constexpr int SC_B = SC_A + BM * 4;
  static constexpr int SC_BIAS = SC_B + BN * 4;
  static constexpr int LDS_BYTES = SC_BIAS + BN * 4;
  static_assert(NA == 2 || NA == 3, "A ring depth");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave sub-tile of 32x32 blocks");
  static_assert((BM / 8) % NW == 0 && (BN / 8) % NW == 0 && NW % 2 == 0, "copies split evenly over waves");
  static_assert(BM <= THREADS && BN <= THREADS, "one epilogue parameter per thread");
};

// Ping-pong geometry with an fp8 W operand against 2-byte A: a stage holds 64
// K elements, 128 bytes per A row and 64 bytes per W row, so the W ring is
// half the size of the 2-byte one.
template <int BM_, int BN_, int WGM_, int WGN_, int NA_>
struct F8Geo : I8Geo<BM_, BN_, WGM_, WGN_, NA_> {
  using Base = I8Geo<BM_, BN_, WGM_, WGN_, NA_>;
  static constexpr bool W8 = true;
  static constexpr int KSW = Base::KS / 2;  // W bytes per row and stage
  static constexpr int STAGE_B = Base::BN * KSW;
  static constexpr int RING = Base::RING_B + 2 * STAGE_B;
  static constexpr int SC_A = RING;
  static constexpr int SC_B = SC_A + Base::BM * 4;
  static constexpr int SC_BIAS = SC_B + Base::BN * 4;
  static constexpr int LDS_BYTES = SC_BIAS + Base::BN * 4;
};

__device__ __forceinline__ float gelu_tanh(float x) {
#pragma clang fp contract(off)
  // 0.5 * x * (1 + tanh(u)), u = sqrt(2/pi) * (x + 0.044715 * x^3): the
  // tanh approximation of ATen's CPU GeluKernel, evaluated as the identical
  // x * sigmoid(2u) = x / (1 + 2^(-2u log2 e)) with 2u log2 e = x (c0 + c1 x^2),
  // the hardware exp2 and reciprocal. Absolute error a few 1e-7, far below
  // one fp16/bf16 ulp of the result; large +x gives x, large -x gives -0 and
  // -inf gives NaN, as the reference formula does.
  const float c0 = 2.3022082f;   // 2 sqrt(2/pi) log2(e)
  const float c1 = 0.10294324f;  // c0 * 0.044715
  const float p = __builtin_fmaf(c1, x * x, c0);
  const float e = __builtin_amdgcn_exp2f(-(x * p));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// Raw storage bits of bias[col] (fp32, fp16 or bf16) and their fp32 value.
__device__ __forceinline__ uint32_t load_bias_bits(const void* bias, int dtype, int col) {
  if (dtype == QG_F32) return static_cast<const uint32_t*>(bias)[col];
  return static_cast<const uint16_t*>(bias)[col];
}
__device__ __forceinline__ float bias_value(uint32_t bits, int dtype) {
  if (dtype == QG_F32) return __uint_as_float(bits);
  return dtype == QG_F16 ? f16_to_f32(static_cast<uint16_t>(bits)) : bf16_to_f32(static_cast<uint16_t>(bits));
}

template <int OUT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (OUT == QG_F16) return f16_to_f32(f32_to_f16(v));
  else if constexpr (OUT == QG_BF16) return bf16_to_f32(f32_to_bf16(v));
  else return v;
}

template <int OUT>
constexpr int out_size() { return (OUT == QG_F16 || OUT == QG_BF16) ? 2 : 4; }

// Row stride (elements) of a dense kernel's output: out_sm, or N when 0.
__device__ __forceinline__ int64_t out_ld(const I8GemmArgs& p) { return p.out_sm > 0 ? p.out_sm : p.N; }

// Storage bits of one output element.
//   EPI_F:     v = f32(acc) * (sa * sb); v = v + bias           (int8_gemm.py:53-63)
//   EPI_FMA:   v = fma(f32(acc), sa * sb, bias)                 (rounding="fused", :191)
//   EPI_EAGER: t = out(f32(acc) * (sa * sb)); t = out(t + out(bias))  (comfy_int8.py:128-143)
//   EPI_GELU:  EPI_F followed by GELU-tanh in fp32
template <int OUT, int MODE, typename ACC>
__device__ __forceinline__ float epi_value(ACC acc, float sa, float sb, float bv, bool has_bias) {
#pragma clang fp contract(off)
  const float scale = sa * sb;
  const float accf = static_cast<float>(acc);  // exact for int32 |acc| < 2^24, identity for fp32
  float v;
  if constexpr (MODE == EPI_EAGER) {
    v = round_to<OUT>(accf * scale);
    if (has_bias) v = v + round_to<OUT>(bv);
  } else if constexpr (MODE == EPI_FMA) {
    v = has_bias ? __builtin_fmaf(accf, scale, bv) : accf * scale;
  } else {
    v = accf * scale;
    if (has_bias) v = v + bv;
    if constexpr (MODE == EPI_GELU) v = gelu_tanh(v);
  }
  return v;
}
template <int OUT, int MODE>
__device__ __forceinline__ uint32_t epi_bits(int32_t acc, float sa, float sb, float bv, bool has_bias) {
  if constexpr (MODE == EPI_INT) {
    return static_cast<uint32_t>(acc);
  } else {
    const float v = epi_value<OUT, MODE>(acc, sa, sb, bv, has_bias);
    if constexpr (OUT == QG_F32) return __float_as_uint(v);
    else if constexpr (OUT == QG_F16) return f32_to_f16(v);
    else return f32_to_bf16(v);
  }
}

// The residual value of output element (row, col) in fp32 (p.residual non-null).
__device__ __forceinline__ float residual_value(const I8GemmArgs& p, int row, int col) {
  const int64_t idx = static_cast<int64_t>(row) * p.residual_sm + col;
  if (p.residual_dtype == QG_F32) return static_cast<const float*>(p.residual)[idx];
  if (p.residual_dtype == QG_F16) return f16_to_f32(static_cast<const uint16_t*>(p.residual)[idx]);
  return bf16_to_f32(static_cast<const uint16_t*>(p.residual)[idx]);
}

// The residual values of the 4 adjacent output elements (row, col0 .. col0 + 3)
// in fp32, one vector load when they lie in the row and are aligned (columns
// past N read column N - 1: their results are never stored).
__device__ __forceinline__ f32x4 residual_value4(const I8GemmArgs& p, int row, int col0) {
  const int64_t idx = static_cast<int64_t>(row) * p.residual_sm + col0;
  f32x4 r;
  if (col0 + 3 < p.N && (idx & 3) == 0) {
    if (p.residual_dtype == QG_F32) return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p.residual) + idx);
    const uint2 h = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.residual) + idx);
    const bool f16 = p.residual_dtype == QG_F16;
    const uint16_t e[4] = {static_cast<uint16_t>(h.x), static_cast<uint16_t>(h.x >> 16), static_cast<uint16_t>(h.y),
                           static_cast<uint16_t>(h.y >> 16)};
    static_for<0, 4>([&](auto c) {
      constexpr int C = decltype(c)::value;
      r[C] = f16 ? f16_to_f32(e[C]) : bf16_to_f32(e[C]);
    });
    return r;
  }
  static_for<0, 4>([&](auto c) {
    constexpr int C = decltype(c)::value;
    r[C] = residual_value(p, row, min(col0 + C, p.N - 1));
  });
  return r;
}

// The residual scales of output columns col0 .. col0 + 3 (p.residual_scale
// non-null; columns past N take column N - 1's).
__device__ __forceinline__ f32x4 residual_scale4(const I8GemmArgs& p, int col0) {
  if (p.residual_scalar) {
    const float v = p.residual_scale[0];
    return f32x4{v, v, v, v};
  }
  if (col0 + 3 < p.N && (col0 & 3) == 0 && (reinterpret_cast<uintptr_t>(p.residual_scale) & 15) == 0)
    return *reinterpret_cast<const f32x4*>(p.residual_scale + col0);
  f32x4 r;
  static_for<0, 4>([&](auto c) {
    constexpr int C = decltype(c)::value;
    r[C] = p.residual_scale[min(col0 + C, p.N - 1)];
  });
  return r;
}

// The residual term of output element (row, col) (p.residual non-null).
__device__ __forceinline__ float residual_term(const I8GemmArgs& p, int row, int col) {
#pragma clang fp contract(off)
  const int64_t idx = static_cast<int64_t>(row) * p.residual_sm + col;
  float r;
  if (p.residual_dtype == QG_F32) r = static_cast<const float*>(p.residual)[idx];
  else if (p.residual_dtype == QG_F16) r = f16_to_f32(static_cast<const uint16_t*>(p.residual)[idx]);
  else r = bf16_to_f32(static_cast<const uint16_t*>(p.residual)[idx]);
  if (p.residual_scale) r = r * p.residual_scale[p.residual_scalar ? 0 : col];
  return r;
}

// Output bits of one element with the residual term (MODE != EPI_INT / EPI_EAGER).
template <int OUT, int MODE>
__device__ __forceinline__ uint32_t epi_bits_res(const I8GemmArgs& p, int32_t acc, float sa, float sb, float bv,
                                                 bool has_bias, int row, int col) {
#pragma clang fp contract(off)
  float v = epi_value<OUT, MODE>(acc, sa, sb, bv, has_bias);
  v = v + residual_term(p, row, col);
  if constexpr (OUT == QG_F32) return __float_as_uint(v);
  else if constexpr (OUT == QG_F16) return f32_to_f16(v);
  else return f32_to_bf16(v);
}

template <int OUT>
__device__ __forceinline__ void store_elem(void* out, int64_t idx, uint32_t bits) {
  if constexpr (out_size<OUT>() == 4) static_cast<uint32_t*>(out)[idx] = bits;
  else static_cast<uint16_t*>(out)[idx] = static_cast<uint16_t>(bits);
}

// Output tile of this workgroup: the linear block id is remapped so that each
// of the 8 XCDs (round-robin workgroup dispatch) walks one contiguous range of
// tiles, GROUP_M-ordered inside.
template <int BM, int BN>
__device__ __forceinline__ void tile_origin_at(const I8GemmArgs& p, int bid, int& m0, int& n0) {
  const int nbm = ceil_div(p.M, BM), nbn = ceil_div(p.N, BN);
  const int total = nbm * nbn;
  if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  constexpr int GROUP_M = 4;
  const int group = bid / (GROUP_M * nbn);
  const int first = group * GROUP_M;
  const int gm = min(nbm - first, GROUP_M);
  const int in_group = bid - group * GROUP_M * nbn;
  m0 = (first + in_group % gm) * BM;
  n0 = (in_group / gm) * BN;
}
template <int BM, int BN>
__device__ __forceinline__ void tile_origin(const I8GemmArgs& p, int& m0, int& n0) {
  tile_origin_at<BM, BN>(p, static_cast<int>(blockIdx.x), m0, n0);
}

// Copies of one operand: segment i of a wave covers 8 rows starting at row
// 8 (wave + NW i) of the tile. Lane l lands on LDS row 8 (wave + NW i) + (l >> 3),
// physical 16-byte chunk (l & 7), and fetches the logical chunk that the
// swizzle stores there: ((row >> 1) & 7) = 4 (wave & 1) + (l >> 4) for even NW.
// Offsets are 32-bit bytes from the operand base (operands < 2 GiB), recomputed
// per copy from one base row to keep registers for fragments.
template <int NW>
struct CopyPlan {
  uint32_t chunk16;
  int row0;
  __device__ __forceinline__ CopyPlan(int tile_row0, int wave, int lane)
      : chunk16(static_cast<uint32_t>(((lane & 7) ^ (4 * (wave & 1) + (lane >> 4))) << 4)),
        row0(tile_row0 + wave * 8 + (lane >> 3)) {}
  // Copy segment i of K stage s (K bytes [128 s, 128 s + 128)) of rows < rows
  // (clamped) with row stride `stride` into LDS at slot_addr.
  template <int I>
  __device__ __forceinline__ void copy(const char* base, int64_t stride, int rows, int s, uint32_t slot_addr,
                                       int wave) const {
    int r = row0;
    // The opaque copy keeps the compiler from hoisting the loop-invariant
    // offsets out of the K loop (they would be held in registers, or spilled).
    asm volatile("" : "+v"(r));
    const uint32_t row = static_cast<uint32_t>(min(r + 8 * NW * I, rows - 1));
    dma16s(base + static_cast<int64_t>(s) * 128, row * static_cast<uint32_t>(stride) + chunk16,
           slot_addr + (wave + NW * I) * 1024);
  }
};

// Fragment offset in an operand slot: k-step t, lane l reads row (l & 31) of a
// 32-row block, logical chunk 2t + (l >> 5), stored at chunk ^ ((l >> 1) & 7).
__device__ __forceinline__ int frag_offset(int t, int lane) {
  return (lane & 31) * 128 + (((2 * t + (lane >> 5)) ^ ((lane >> 1) & 7)) << 4);
}

// Per-row / per-column epilogue parameters: thread t fetches row m0 + t's scale
// and column n0 + t's scale and bias bits (indices clamped in range; values of
// rows / columns past the edge are never stored).
struct EpiParams {
  float sa = 0.0f, sb = 0.0f;
  uint32_t bias = 0;
};
template <int BM, int BN, int MODE>
__device__ __forceinline__ EpiParams fetch_epi_params(const I8GemmArgs& p, int m0, int n0, int tid) {
  EpiParams e;
  if constexpr (MODE != EPI_INT) {
    if (tid < BM) e.sa = p.a_scale ? p.a_scale[min(m0 + tid, p.M - 1)] : 1.0f;
    if (tid < BN) {
      const int col = min(n0 + tid, p.N - 1);
      e.sb = p.b_scale ? p.b_scale[p.b_scalar ? 0 : col] : 1.0f;
      if (p.bias != nullptr) e.bias = load_bias_bits(p.bias, p.bias_dtype, col);
    }
  }
  return e;
}

// Epilogue. Block (i, j), register r of a lane holds row 32 i + 8 (r >> 2) +
// 4 (l >> 5) + (r & 3) and column 32 j + (l & 31) of the wave sub-tile. The
// caller has drained every copy and passed a barrier after the last LDS read
// of the rings.
template <typename G, int OUT, int MODE, bool RES>
__device__ __forceinline__ void i8_epilogue(const I8GemmArgs& p, const i32x16 (&acc)[G::FM][G::FN], char* smem,
                                            int m0, int n0, int wr, int wc, int wave, int lane, int tid,
                                            const EpiParams& ep) {
#pragma clang fp contract(off)
  float* sa_lds = reinterpret_cast<float*>(smem + G::SC_A);
  float* sb_lds = reinterpret_cast<float*>(smem + G::SC_B);
  uint32_t* bias_lds = reinterpret_cast<uint32_t*>(smem + G::SC_BIAS);
  if constexpr (MODE != EPI_INT) {
    if (tid < G::BM) sa_lds[tid] = ep.sa;
    if (tid < G::BN) {
      sb_lds[tid] = ep.sb;
      bias_lds[tid] = ep.bias;
    }
    __syncthreads();
  }
  const bool has_bias = p.bias != nullptr;
  const int lh = 4 * (lane >> 5);
  const int lcol = lane & 31;
  float sb[G::FN], bv[G::FN], rs[G::FN];
  static_for<0, G::FN>([&](auto j) {
    const int c = wc * G::WN + j * 32 + lcol;
    sb[j] = MODE != EPI_INT ? sb_lds[c] : 0.0f;
    bv[j] = MODE != EPI_INT ? bias_value(bias_lds[c], p.bias_dtype) : 0.0f;
    // the residual scale of this lane's column in block j (loaded once)
    rs[j] = 1.0f;
    if constexpr (RES) {
      if (p.residual_scale) rs[j] = p.residual_scale[p.residual_scalar ? 0 : min(n0 + c, p.N - 1)];
    }
  });
  const bool has_rs = p.residual_scale != nullptr;
  // v + residual (x scale): the fp32 order of residual_term
  auto with_res = [&](float v, int row, int col, float rsc) __attribute__((always_inline)) {
#pragma clang fp contract(off)
    float r = residual_value(p, row, col);
    if (has_rs) r = r * rsc;
    return v + r;
  };
  auto bits_of = [&](float v) __attribute__((always_inline)) -> uint32_t {
    if constexpr (OUT == QG_F32) return __float_as_uint(v);
    else if constexpr (OUT == QG_F16) return f32_to_f16(v);
    else return f32_to_bf16(v);
  };
  // Scales of the 4 rows 32 i + 8 q + lh + (0..3): one aligned LDS vector.
  auto row_scales = [&](int i, int q) -> f32x4 {
    if constexpr (MODE == EPI_INT) return f32x4{0, 0, 0, 0};
    else return *reinterpret_cast<const f32x4*>(sa_lds + wr * G::WM + 32 * i + 8 * q + lh);
  };

  constexpr int ES = out_size<OUT>();
  const int64_t ldo = out_ld(p);
  const bool full = m0 + G::BM <= p.M && n0 + G::BN <= p.N && ((ldo * ES) % 16) == 0 &&
                    (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
  if (full) {
    // Stage the rounded wave sub-tile in LDS (PF blocks of 32 rows per pass, own
    // region of the rings per wave), then write whole 16-byte row chunks.
    constexpr int ROWB = G::WN * ES + 16;                  // padded LDS row pitch
    constexpr int REGION = G::RING / G::NW;
    constexpr int PF = (G::FM * 32 * ROWB <= REGION) ? G::FM : (G::FM / 2 * 32 * ROWB <= REGION) ? G::FM / 2 : 1;
    static_assert(PF * 32 * ROWB <= REGION && G::FM % PF == 0, "epilogue staging does not fit");
    constexpr int CHUNKS = G::WN * ES / 16;                // 16-byte chunks per row
    char* region = smem + wave * REGION;
    char* out = static_cast<char*>(p.out);
    static_for<0, G::FM / PF>([&](auto pass) {
      static_for<0, PF>([&](auto ii) {
        constexpr int i = decltype(pass)::value * PF + decltype(ii)::value;
        // the residual values of block row i, all loads issued before any is
        // used (one memory latency per block row instead of one per element)
        float rv[RES ? 4 : 1][RES ? G::FN : 1][RES ? 4 : 1];
        if constexpr (RES) {
          static_for<0, 4>([&](auto q) {
            static_for<0, G::FN>([&](auto j) {
              static_for<0, 4>([&](auto e) {
                rv[q][j][e] = residual_value(p, m0 + wr * G::WM + 32 * i + 8 * decltype(q)::value + lh +
                                                    decltype(e)::value,
                                             n0 + wc * G::WN + decltype(j)::value * 32 + lcol);
              });
            });
          });
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 sa = row_scales(i, q);
          static_for<0, G::FN>([&](auto j) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              uint32_t bits;
              if constexpr (RES) {
                // v + f32(residual) (x scale), the fp32 order of residual_term
                float r = rv[q][j][e];
                if (has_rs) r = r * rs[j];
                bits = bits_of(epi_value<OUT, MODE>(acc[i][j][4 * q + e], sa[e], sb[j], bv[j], has_bias) + r);
              } else
                bits = epi_bits<OUT, MODE>(acc[i][j][4 * q + e], sa[e], sb[j], bv[j], has_bias);
              char* dstp = region + (ii * 32 + 8 * q + lh + e) * ROWB + (j * 32 + lcol) * ES;
              if constexpr (ES == 4) *reinterpret_cast<uint32_t*>(dstp) = bits;
              else *reinterpret_cast<uint16_t*>(dstp) = static_cast<uint16_t>(bits);
            }
          });
        }
      });
      // LDS accesses of one wave complete in order; the reads below see the writes.
      constexpr int TOTAL = PF * 32 * CHUNKS;
      static_assert(TOTAL % 64 == 0, "whole chunk rounds per lane");
#pragma unroll
      for (int c0 = 0; c0 < TOTAL; c0 += 64) {
        const int c = c0 + lane;
        const int rr = c / CHUNKS, cc = c - rr * CHUNKS;
        const i32x4 v = *reinterpret_cast<const i32x4*>(region + rr * ROWB + cc * 16);
        const int64_t grow = m0 + wr * G::WM + decltype(pass)::value * PF * 32 + rr;
        const int64_t gcol = n0 + wc * G::WN;
        *reinterpret_cast<i32x4*>(out + (grow * ldo + gcol) * ES + cc * 16) = v;
      }
    });
  } else {
    const int row0 = m0 + wr * G::WM + lh;
    const int col0 = n0 + wc * G::WN + lcol;
    static_for<0, G::FM>([&](auto i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 sa = row_scales(i, q);
        static_for<0, G::FN>([&](auto j) {
          const int col = col0 + j * 32;
          if (col < p.N) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int row = row0 + 32 * i + 8 * q + e;
              if (row < p.M)
                store_elem<OUT>(p.out, static_cast<int64_t>(row) * ldo + col,
                                RES ? bits_of(with_res(epi_value<OUT, MODE>(acc[i][j][4 * q + e], sa[e], sb[j],
                                                                            bv[j], has_bias),
                                                       row, col, rs[j]))
                                    : epi_bits<OUT, MODE>(acc[i][j][4 * q + e], sa[e], sb[j], bv[j], has_bias));
            }
          }
        });
      }
    });
  }
}

// 4 waves (2 x 2, one per SIMD), the whole next stage staged in registers.
template <typename G, int WPE, int OUT, int MODE, bool RES>
__global__ __launch_bounds__(G::THREADS, WPE) void k_i8_gemm(I8GemmArgs p) {
#pragma clang fp contract(off)
  static_assert(G::NW == 4, "register-staged pipeline: 4 waves");
  constexpr int NA = G::NA;
  constexpr int READS = G::KT * (G::FM + G::FN);     // fragment reads per stage
  constexpr int GROUPS = G::KT / 2 * G::FM;          // MFMA groups (FN each) per half stage
  __shared__ __attribute__((aligned(1024))) char smem[G::LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int wr = wave >> 1, wc = wave & 1;
  int m0, n0;
  tile_origin<G::BM, G::BN>(p, m0, n0);
  const EpiParams ep = fetch_epi_params<G::BM, G::BN, MODE>(p, m0, n0, tid);

  const CopyPlan<4> ca(m0, wave, lane), cw(n0, wave, lane);
  const uint32_t smem_base = lds_addr_of(smem);
  const int S = p.K / G::KS;
  const char* a_base = reinterpret_cast<const char*>(p.a);
  const char* w_base = reinterpret_cast<const char*>(p.w);
  // A stage s lives in A slot s % NA and W slot s % 2.
  auto dma_a = [&](auto i_c, int s) {
    ca.template copy<decltype(i_c)::value>(a_base, p.a_sm, p.M, s,
                                           smem_base + (NA == 2 ? (s & 1) : s % 3) * G::STAGE_A, wave);
  };
  auto dma_w = [&](auto i_c, int s) {
    cw.template copy<decltype(i_c)::value>(w_base, p.w_sn, p.N, s,
                                           smem_base + G::RING_B + (s & 1) * G::STAGE_B, wave);
  };
  auto dma_stage = [&](int s) {
    static_for<0, G::A_SEGS>([&](auto i) { dma_a(i, s); });
    static_for<0, G::B_SEGS>([&](auto i) { dma_w(i, s); });
  };

  int a_off[G::KT], b_off[G::KT];
#pragma unroll
  for (int t = 0; t < G::KT; ++t) {
    a_off[t] = wr * G::WM * G::KS + frag_offset(t, lane);
    b_off[t] = G::RING_B + wc * G::WN * G::KS + frag_offset(t, lane);
  }

  i32x16 acc[G::FM][G::FN];
  static_for<0, G::FM>([&](auto i) {
    static_for<0, G::FN>([&](auto j) { acc[i][j] = i32x16{}; });
  });

  // Register copies of two stages: [buffer][k-step][block].
  i32x4 fa[2][G::KT][G::FM], fb[2][G::KT][G::FN];

  // Read fragment number r (k-step major, A blocks then W blocks) of the stage
  // held in A slot `abase` and W slot `bbase` (byte offsets from the slot 0
  // positions) into register buffer `buf`.
  auto read_frag = [&](auto r_c, auto buf_c, int abase, int bbase) {
    constexpr int r = decltype(r_c)::value;
    constexpr int buf = decltype(buf_c)::value;
    constexpr int t = r / (G::FM + G::FN), f = r % (G::FM + G::FN);
    if constexpr (f < G::FM)
      fa[buf][t][f] = *reinterpret_cast<const i32x4*>(smem + abase + a_off[t] + f * 32 * G::KS);
    else
      fb[buf][t][f - G::FM] = *reinterpret_cast<const i32x4*>(smem + bbase + b_off[t] + (f - G::FM) * 32 * G::KS);
  };

  if (S > 0) {
    // ---- prologue: stages 0 and 1 in flight, stage 0 into registers, stage 2
    // into the freed slots -----------------------------------------------------
    dma_stage(0);
    if (S > 1) {
      dma_stage(1);
      wait_vm_barrier<G::SPW>();
    } else {
      wait_vm_barrier<0>();
    }
    static_for<0, READS>([&](auto r) { read_frag(r, std::integral_constant<int, 0>{}, 0, 0); });
    wait_lds_barrier();
    dma_stage(min(2, S - 1));

    // ---- steady state, two stages per trip so register buffers are static ----
    //  barrier A  : stage s+1 landed everywhere (copies of stages s+1 and s+2
    //               are in flight here, in that order, so vmcnt(SPW) leaves
    //               only the newer)
    //  first half : MFMAs of k-steps 0..KT/2-1 of stage s; read all of stage
    //               s+1; with a 3-slot A ring, copy A of stage s+3 into the
    //               slot that stage s left (read before the previous barrier B)
    //  barrier B  : every wave holds stage s+1; its W slot (and, with a 2-slot
    //               A ring, its A slot) takes stage s+3
    //  second half: MFMAs of k-steps KT/2..KT-1 with the remaining copies
    auto stage = [&](int s, auto cur_c) {
      constexpr int cur = decltype(cur_c)::value;
      constexpr int nxt = cur ^ 1;
      wait_vm_barrier<G::SPW>();
      const int abase = (NA == 2 ? ((s + 1) & 1) : (s + 1) % 3) * G::STAGE_A;
      const int bbase = ((s + 1) & 1) * G::STAGE_B;
      const int refill_stage = min(s + 3, S - 1);
      static_for<0, GROUPS>([&](auto g) {
        constexpr int t = g / G::FM, i = g % G::FM;
        static_for<0, G::FN>([&](auto j) {
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[cur][t][i], fb[cur][t][j], acc[i][j], 0, 0, 0);
        });
        __builtin_amdgcn_sched_barrier(0);
        constexpr int r0 = g * READS / GROUPS, r1 = (g + 1) * READS / GROUPS;
        static_for<r0, r1>([&](auto r) { read_frag(r, std::integral_constant<int, nxt>{}, abase, bbase); });
        if constexpr (NA == 3) {
          constexpr int d0 = g * G::A_SEGS / GROUPS, d1 = (g + 1) * G::A_SEGS / GROUPS;
          static_for<d0, d1>([&](auto d) { dma_a(d, refill_stage); });
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      wait_lds_barrier();
      constexpr int LATE = (NA == 3 ? 0 : G::A_SEGS) + G::B_SEGS;  // copies after barrier B
      static_for<0, GROUPS>([&](auto g) {
        constexpr int t = G::KT / 2 + g / G::FM, i = g % G::FM;
        constexpr int d0 = g * LATE / GROUPS, d1 = (g + 1) * LATE / GROUPS;
        static_for<d0, d1>([&](auto d) {
          constexpr int di = decltype(d)::value;
          if constexpr (NA == 3) dma_w(d, refill_stage);
          else if constexpr (di < G::A_SEGS) dma_a(d, refill_stage);
          else dma_w(std::integral_constant<int, di - G::A_SEGS>{}, refill_stage);
        });
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, G::FN>([&](auto j) {
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[cur][t][i], fb[cur][t][j], acc[i][j], 0, 0, 0);
        });
        __builtin_amdgcn_sched_barrier(0);
      });
    };
    int s = 0;
    for (; s + 1 < S; s += 2) {
      stage(s, std::integral_constant<int, 0>{});
      stage(s + 1, std::integral_constant<int, 1>{});
    }
    if (s < S) stage(s, std::integral_constant<int, 0>{});
  }

  wait_vm_barrier<0>();  // no copy into LDS in flight; every wave is done reading the rings
  i8_epilogue<G, OUT, MODE, RES>(p, acc, smem, m0, n0, wr, wc, wave, lane, tid, ep);
}

// 8 waves in two groups that share the SIMDs pairwise (waves w and w + 4) and
// alternate roles every half stage ("ping-pong"): while one wave of a SIMD
// issues its whole stage of MFMAs back to back, the other reads its next
// fragments from LDS and issues copies, so a wave waiting on a copy or an LDS
// read never leaves the MFMA pipe idle. Group X (waves 0-3) copies W, group Y
// (waves 4-7) copies A. Phases of stage s:
//   B0(s)  barrier: every wave is done with stage s-1's data
//   P1(s)  X: MFMAs of stage s (fragments read in P2(s-1))
//          Y: read stage s, copy A of stage s+2 into the A slot of stage s-1
//   B1(s)  X: W(s+1) landed (its newest copies), Y: A(s+1) landed (only
//          A(s+2) may still fly) and Y's reads of stage s are complete
//   P2(s)  X: read stage s+1, copy W of stage s+2 into the W slot of stage s
//          Y: MFMAs of stage s
// Nothing past the last stage is copied or read: in the last two stages the
// waits at B1 drain every copy instead.
//
// Accumulator layout: W fragments are the MFMA's first operand, so each 32x32
// block holds the transposed product: register r of lane l is row
// 32 i + (l & 31) and column 32 j + 8 (r >> 2) + 4 (l >> 5) + (r & 3) of the
// wave sub-tile. Every register quad is 4 adjacent columns of one row, which
// the epilogue converts with paired conversions and stores as one vector.

// Copy row offsets per wave of the ping-pong kernels (W copies of waves 0-3,
// A copies of waves 4-7).
template <typename G>
constexpr int pp_copies() { return (G::BM > G::BN ? G::BM : G::BN) / 32; }

// The ping-pong main loop: acc += (A tile x W tile^T) over S stages of 128 K
// bytes, in the transposed layout above. voff[i] is this wave's 32-bit byte
// offset of the row that its copy i fetches (W rows n0 + 8 (gw + 4 i) +
// (l >> 3) for waves 0-3, A rows for waves 4-7), including the swizzled
// chunk; a_base / w_base point at K = 0. park() runs in every wave once its
// first copies, and every copy it issued before them, have landed, and
// before the barrier that opens the loop (the callers finish their epilogue
// parameters there). With `pre`, this wave's stage-0 copies (W(0) for X,
// A(0) for Y) were already issued by pp_prefetch0 (during the previous
// tile's epilogue). On
// return no copy is in flight and every wave has passed the barrier after the
// last read of the rings, so each wave may stage its epilogue in its own part
// of the rings at once (group X's epilogue overlaps group Y's last MFMAs).
// ST > 0: with `pre` and `stores_fly`, the previous tile's epilogue issued at
// least ST vector stores per wave after the stage-0 copies; the prologue waits
// let them stay in flight instead of draining every store first.
// STAMP (the stage-timing instantiation only): the shader-clock counter is
// read at four points of every stage, lane s of stv[P] keeping point P of
// stage s (s < 64): group X before B0, after B0, after its MFMAs, after B1;
// group Y after B0, its LDS reads complete, after B1, after its MFMAs.
template <typename G, typename MF, int ST = 0, bool STAMP = false, bool NTW = false, typename Park>
__device__ __forceinline__ void pp_mainloop(typename MF::acc_t (&acc)[G::FM][G::FN], char* smem, const char* a_base,
                                            const char* w_base, const uint32_t (&voff)[pp_copies<G>()], int S,
                                            int wave, int lane, bool pre, Park&& park, bool stores_fly = false,
                                            uint32_t* stv = nullptr) {
  static_assert(G::NW == 8 && G::NA == 3 && G::KT == 4, "ping-pong geometry");
  constexpr bool W8 = G::W8;
  constexpr int KSW = W8 ? G::KS / 2 : G::KS;             // W bytes per row and stage
  constexpr int XS = G::BN * KSW / 4096, YS = G::BM / 32;  // copies per wave and stage (W by X, A by Y)
  const int wr = wave / G::WGN, wc = wave % G::WGN;
  const bool grp_x = wave < 4;
  const int gw = wave & 3;
  const uint32_t smem_base = lds_addr_of(smem);
  auto copy_w = [&](auto i_c, int s) {
    constexpr int I = decltype(i_c)::value;
    const uint32_t dst = smem_base + G::RING_B + (s & 1) * G::STAGE_B + (gw + 4 * I) * 1024;
    if constexpr (NTW) dma16s_nt(w_base + static_cast<int64_t>(s) * KSW, voff[I], dst);
    else dma16s(w_base + static_cast<int64_t>(s) * KSW, voff[I], dst);
  };
  auto copy_a = [&](auto i_c, int s) {
    constexpr int I = decltype(i_c)::value;
    dma16s(a_base + static_cast<int64_t>(s) * G::KS, voff[I], smem_base + (s % 3) * G::STAGE_A + (gw + 4 * I) * 1024);
  };

  // With fp8 W the two k-steps 2u, 2u + 1 of a 32-element K block u take the
  // K elements {32u + 16h + 0..7} and {32u + 16h + 8..15} from lane half h
  // (A and W alike, so the dot product is the same sum): one 16-byte read of
  // W row chunk 2u + h then serves both k-steps. W rows are 64 bytes, their
  // chunk c stored at c ^ ((row >> 2) & 3) (conflict-free 16-lane reads).
  int a_off[G::KT], b_off[G::KT];
#pragma unroll
  for (int t = 0; t < G::KT; ++t) {
    if constexpr (W8) {
      const int chunk = 4 * (t >> 1) + 2 * (lane >> 5) + (t & 1);
      a_off[t] = wr * G::WM * G::KS + (lane & 31) * 128 + ((chunk ^ ((lane >> 1) & 7)) << 4);
      b_off[t] = G::RING_B + wc * G::WN * KSW + (lane & 31) * KSW +
                 (((2 * (t >> 1) + (lane >> 5)) ^ ((lane >> 2) & 3)) << 4);
    } else {
      a_off[t] = wr * G::WM * G::KS + frag_offset(t, lane);
      b_off[t] = G::RING_B + wc * G::WN * G::KS + frag_offset(t, lane);
    }
  }
  i32x4 fa[G::KT][G::FM], fb[G::KT][G::FN];

  // Read stage s into the fragment registers; with COPY, this wave's copies of
  // stage cs are spread between the k-steps (W copies for X, A copies for Y).
  auto load_phase = [&](auto x_c, auto copy_c, int s, int cs) {
    constexpr bool X = decltype(x_c)::value;
    constexpr bool COPY = decltype(copy_c)::value;
    const int abase = (s % 3) * G::STAGE_A;
    const int bbase = (s & 1) * G::STAGE_B;
    static_for<0, G::KT>([&](auto t_c) {
      constexpr int t = decltype(t_c)::value;
      static_for<0, G::FM>([&](auto i) {
        fa[t][i] = *reinterpret_cast<const i32x4*>(smem + abase + a_off[t] + i * 32 * G::KS);
      });
      if constexpr (!W8) {
        static_for<0, G::FN>([&](auto j) {
          fb[t][j] = *reinterpret_cast<const i32x4*>(smem + bbase + b_off[t] + j * 32 * G::KS);
        });
      } else if constexpr ((t & 1) == 0) {
        static_for<0, G::FN>([&](auto j) {
          const i32x4 raw = *reinterpret_cast<const i32x4*>(smem + bbase + b_off[t] + j * 32 * KSW);
          fb[t][j] = fp8x8<MF::F16A, MF::E5>(static_cast<uint32_t>(raw[0]), static_cast<uint32_t>(raw[1]));
          fb[t + 1][j] = fp8x8<MF::F16A, MF::E5>(static_cast<uint32_t>(raw[2]), static_cast<uint32_t>(raw[3]));
        });
      }
      if constexpr (COPY && X) {
        static_for<t * XS / G::KT, (t + 1) * XS / G::KT>([&](auto d) { copy_w(d, cs); });
      } else if constexpr (COPY) {
        static_for<t * YS / G::KT, (t + 1) * YS / G::KT>([&](auto d) { copy_a(d, cs); });
      }
    });
  };
  auto mfma_phase = [&]() {
    __builtin_amdgcn_s_setprio(1);
    static_for<0, G::KT>([&](auto t) {
      static_for<0, G::FM>([&](auto i) {
        static_for<0, G::FN>([&](auto j) {
          acc[i][j] = MF::mfma(fb[t][j], fa[t][i], acc[i][j]);
        });
      });
    });
    __builtin_amdgcn_s_setprio(0);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  auto stamp = [&](int point, int s) __attribute__((always_inline)) {
    if constexpr (STAMP) {
      const uint32_t t = static_cast<uint32_t>(__builtin_amdgcn_s_memtime());
      stv[point] = lane == (s & 63) ? t : stv[point];
    }
  };

  if (S <= 0) {
    park();
    wait_lds_barrier();
    return;
  }
  // Both groups pass the same barriers: one after the prologue, then B0 and
  // B1 of every stage.
  if (grp_x) {
    // prologue: W(0) landed everywhere, then read stage 0 and copy W(1)
    if (!pre) static_for<0, XS>([&](auto d) { copy_w(d, 0); });
    if (ST > 0 && pre && stores_fly) wait_vm<ST>();  // W(0), issued before the stores
    else wait_vm<0>();
    park();
    wait_lds_barrier();
    if (S > 1) load_phase(T_{}, T_{}, 0, 1);
    else load_phase(T_{}, F_{}, 0, 0);
    for (int s = 0; s < S; ++s) {
      stamp(0, s);
      __builtin_amdgcn_s_barrier();  // B0(s)
      stamp(1, s);
      mfma_phase();
      stamp(2, s);
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");  // B1(s)
      stamp(3, s);
      if (s + 2 < S) load_phase(T_{}, T_{}, s + 1, s + 2);
      else if (s + 1 < S) load_phase(T_{}, F_{}, s + 1, 0);
    }
  } else {
    if (!pre) static_for<0, YS>([&](auto d) { copy_a(d, 0); });
    const bool fly = ST > 0 && pre && stores_fly;  // A(0) issued before the previous tile's stores
    if (S > 1) {
      static_for<0, YS>([&](auto d) { copy_a(d, 1); });
      if (fly) wait_vm<YS + ST>();
      else wait_vm<YS>();
    } else {
      if (fly) wait_vm<ST>();
      else wait_vm<0>();
    }
    park();
    wait_lds_barrier();
    for (int s = 0; s < S; ++s) {
      __builtin_amdgcn_s_barrier();  // B0(s)
      stamp(0, s);
      if (s + 2 < S) {
        load_phase(F_{}, T_{}, s, s + 2);
        if constexpr (STAMP) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          stamp(1, s);
        }
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(YS) : "memory");  // B1(s)
      } else {
        load_phase(F_{}, F_{}, s, 0);
        if constexpr (STAMP) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          stamp(1, s);
        }
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");  // B1(s)
      }
      stamp(2, s);
      mfma_phase();
      stamp(3, s);
    }
  }
}

// Stage-0 copies of the next tile (W(0) by group X into W slot 0, A(0) by group
// Y into A slot 0), issued once pp_mainloop has returned for the current tile:
// the rings are no longer read, and the epilogue stages outside these slots.
template <typename G, bool NTW = false>
__device__ __forceinline__ void pp_prefetch0(char* smem, const char* a_base, const char* w_base,
                                             const uint32_t (&voff)[pp_copies<G>()], int wave) {
  constexpr int XS = G::BN * (G::W8 ? G::KS / 2 : G::KS) / 4096, YS = G::BM / 32;
  const int gw = wave & 3;
  const uint32_t smem_base = lds_addr_of(smem);
  if (wave < 4) {
    static_for<0, XS>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      if constexpr (NTW) dma16s_nt(w_base, voff[I], smem_base + G::RING_B + (gw + 4 * I) * 1024);
      else dma16s(w_base, voff[I], smem_base + G::RING_B + (gw + 4 * I) * 1024);
    });
  } else {
    static_for<0, YS>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      dma16s(a_base, voff[I], smem_base + (gw + 4 * I) * 1024);
    });
  }
}

// Two fp32 values rounded to nearest-even fp16 / bf16 and packed (first in the
// low half) by one paired hardware conversion; bit-identical to f32_to_f16 /
// f32_to_bf16 for every fp32 input, NaNs included.
template <int OUT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const f32x2 v = {a, b};
  if constexpr (OUT == QG_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// 4 adjacent floats 32 j + 8 g + lq .. + 3 of a per-column LDS vector.
__device__ __forceinline__ f32x4 col4(const float* v, int c0) { return *reinterpret_cast<const f32x4*>(v + c0); }

// Epilogue parameters of the dense ping-pong kernel in LDS: BM row scales,
// BN column scales, BN bias values (copied as raw words, fp32 bits or fp16 /
// bf16 bits zero-extended, and widened to fp32 in place before the main loop
// opens), per parameter buffer.
template <typename G>
struct PpParams {
  static constexpr int SA = 0, SB = 4 * G::BM, BIAS = 4 * G::BM + 4 * G::BN;
  static constexpr int BYTES = 4 * G::BM + 8 * G::BN;
};

// Epilogue of the dense ping-pong kernel (transposed accumulators; row
// scales, column scales and bias words in the parameter buffer at pbuf).
// Full tiles are staged per wave in its own part of the rings and leave as
// whole 16-byte row chunks; edge tiles store element-wise.
template <typename G, int OUT, int MODE, bool RES, int STAGE_BASE = 0, int REGION = G::RING / G::NW,
          bool NT = false, typename ACCV = i32x16>
__device__ __forceinline__ void pp_epilogue(const I8GemmArgs& p, const ACCV (&acc)[G::FM][G::FN], char* smem,
                                            const char* pbuf, int m0, int n0, int wr, int wc, int wave, int lane) {
#pragma clang fp contract(off)
  const float* sa_lds = reinterpret_cast<const float*>(pbuf + PpParams<G>::SA);
  const float* sb_lds = reinterpret_cast<const float*>(pbuf + PpParams<G>::SB);
  const float* bv_lds = reinterpret_cast<const float*>(pbuf + PpParams<G>::BIAS);
  const bool has_bias = p.bias != nullptr;
  const int lr = lane & 31, lq = 4 * (lane >> 5);
  float sa[G::FM];
  static_for<0, G::FM>([&](auto i) { sa[i] = MODE != EPI_INT ? sa_lds[wr * G::WM + 32 * i + lr] : 0.0f; });
  // output bits of the 4 columns of quad g of block (i, j): 4 words (4-byte
  // outputs) or 2 packed words (2-byte outputs) in w[0..]
  // row: the quad's output row; col0: its first output column (residual term)
  // the residual term (x scale) of the 4 columns col0 .. col0 + 3 of one row
  auto res_term4 = [&](int row, int col0) __attribute__((always_inline)) -> f32x4 {
#pragma clang fp contract(off)
    f32x4 r = residual_value4(p, row, col0);
    if (p.residual_scale) {
      const f32x4 rs = residual_scale4(p, col0);
      static_for<0, 4>([&](auto c) {
        constexpr int C = decltype(c)::value;
        r[C] = r[C] * rs[C];
      });
    }
    return r;
  };
  auto quad_bits = [&](auto i, auto j, auto g, const f32x4& sb4, const f32x4& bv4, uint32_t (&w)[4], int row,
                       int col0) {
    constexpr int r0 = 4 * decltype(g)::value;
    if constexpr (MODE == EPI_INT) {
      static_for<0, 4>([&](auto c) { w[c] = static_cast<uint32_t>(acc[i][j][r0 + decltype(c)::value]); });
    } else {
      float v[4];
      static_for<0, 4>([&](auto c) {
        constexpr int C = decltype(c)::value;
        v[C] = epi_value<OUT, MODE>(acc[i][j][r0 + C], sa[i], sb4[C], bv4[C], has_bias);
      });
      if constexpr (RES) {
        // v + f32(residual) (x scale), the fp32 order of residual_term
        const f32x4 r = res_term4(row, col0);
        static_for<0, 4>([&](auto c) {
          constexpr int C = decltype(c)::value;
          v[C] = v[C] + r[C];
        });
      }
      if constexpr (out_size<OUT>() == 4) {
        static_for<0, 4>([&](auto c) { w[c] = __float_as_uint(v[c]); });
      } else {
        w[0] = pack2<OUT>(v[0], v[1]);
        w[1] = pack2<OUT>(v[2], v[3]);
      }
    }
  };
  auto params = [&](int c0, f32x4& sb4, f32x4& bv4) {
    sb4 = f32x4{0, 0, 0, 0};
    bv4 = f32x4{0, 0, 0, 0};
    if constexpr (MODE != EPI_INT) {
      sb4 = col4(sb_lds, c0);
      if (has_bias) bv4 = col4(bv_lds, c0);
    }
  };

  constexpr int ES = out_size<OUT>();
  const int64_t ldo = out_ld(p);
  const bool full = m0 + G::BM <= p.M && n0 + G::BN <= p.N && ((ldo * ES) % 16) == 0 &&
                    (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
  if (full) {
    // PF blocks of 32 rows per pass through the wave's staging region
    constexpr int ROWB = G::WN * ES + 16;  // padded LDS row pitch
    constexpr int PF = (G::FM * 32 * ROWB <= REGION) ? G::FM : (G::FM / 2 * 32 * ROWB <= REGION) ? G::FM / 2 : 1;
    static_assert(PF * 32 * ROWB <= REGION && G::FM % PF == 0, "epilogue staging does not fit");
    constexpr int CHUNKS = G::WN * ES / 16;  // 16-byte chunks per row
    char* region = smem + STAGE_BASE + wave * REGION;
    char* out = static_cast<char*>(p.out);
    static_for<0, G::FM / PF>([&](auto pass) {
      static_for<0, G::FN>([&](auto j) {
        static_for<0, 4>([&](auto g) {
          const int c0 = 32 * decltype(j)::value + 8 * decltype(g)::value + lq;  // wave sub-tile column
          f32x4 sb4, bv4;
          params(wc * G::WN + c0, sb4, bv4);
          static_for<0, PF>([&](auto ii) {
            constexpr int i = decltype(pass)::value * PF + decltype(ii)::value;
            uint32_t w[4];
            quad_bits(std::integral_constant<int, i>{}, j, g, sb4, bv4, w, m0 + wr * G::WM + 32 * i + lr,
                      n0 + wc * G::WN + c0);
            char* dst = region + (decltype(ii)::value * 32 + lr) * ROWB + c0 * ES;
            if constexpr (ES == 4) *reinterpret_cast<i32x4*>(dst) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            else *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1]};
          });
        });
      });
      // LDS accesses of one wave complete in order; the reads below see the writes.
      constexpr int TOTAL = PF * 32 * CHUNKS;
      static_assert(TOTAL % 64 == 0, "whole chunk rounds per lane");
#pragma unroll
      for (int c0 = 0; c0 < TOTAL; c0 += 64) {
        const int c = c0 + lane;
        const int rr = c / CHUNKS, cc = c - rr * CHUNKS;
        const i32x4 v = *reinterpret_cast<const i32x4*>(region + rr * ROWB + cc * 16);
        const int64_t grow = m0 + wr * G::WM + decltype(pass)::value * PF * 32 + rr;
        const int64_t gcol = n0 + wc * G::WN;
        i32x4* dst = reinterpret_cast<i32x4*>(out + (grow * ldo + gcol) * ES + cc * 16);
        // NT (the INT8 kernel): non-temporal stores, measured on one box in
        // alternating runs: cfg1 chain 1962-1975 -> 2014-2024 TOPS, cfg0
        // 37.2-37.5 -> 36.5-37.2 us; the 2-byte kernels keep plain stores
        // (FP8 cfg3 and the W4A16 prefill measured the same or 1 % slower)
        if constexpr (NT) __builtin_nontemporal_store(v, dst);
        else *dst = v;
      }
    });
  } else {
    static_for<0, G::FN>([&](auto j) {
      static_for<0, 4>([&](auto g) {
        const int c0 = wc * G::WN + 32 * decltype(j)::value + 8 * decltype(g)::value + lq;  // tile column
        f32x4 sb4, bv4;
        params(c0, sb4, bv4);
        static_for<0, G::FM>([&](auto i) {
          const int row = m0 + wr * G::WM + 32 * decltype(i)::value + lr;
          uint32_t w[4];
          quad_bits(i, j, g, sb4, bv4, w, min(row, p.M - 1), n0 + c0);
          if (row < p.M) {
            static_for<0, 4>([&](auto c) {
              constexpr int C = decltype(c)::value;
              const int col = n0 + c0 + C;
              const uint32_t bits = ES == 4 ? w[C] : (w[C / 2] >> (16 * (C & 1))) & 0xffffu;
              if (col < p.N) store_elem<OUT>(p.out, static_cast<int64_t>(row) * ldo + col, bits);
            });
          }
        });
      });
    });
  }
}

// Persistent: workgroup b computes tiles b, b + gridDim.x, ... (the grid is at
// most one workgroup per CU, and every wave of a workgroup takes the same tiles,
// so all waves pass the same barriers). With 2-byte outputs the next tile's
// stage-0 copies (A slot 0, W slot 0) are issued before the current tile's
// epilogue, which stages in A slots 1-2, so the next tile's first copy latency
// overlaps the epilogue; a barrier after the epilogue keeps the next tile's
// stage-1 copies off the LDS the epilogue still reads. The epilogue
// parameters (row scales, column scales, bias words) are copied straight
// into LDS by the X waves, into one of two parameter buffers (tile parity),
// with the next tile's stage-0 copies: no register loaded from memory is read
// after the epilogue's stores are issued, where the compiler's own wait for
// it would drain those stores before the next main loop.
// The body is shared by the INT8 kernel (MF = MfmaI8, 1-byte operands) and the
// 2-byte kernel (MfmaHalf, fp16 / bf16 operands: a 128-byte stage row holds 64
// K elements, four 32x32x16 k-steps); ES is the operand element size.
//
// STAMP (qg_int8_gemm_stages only): each wave also records the main loop's
// stage stamps (pp_mainloop) and its entry, main-loop exit, epilogue end
// (after its stores completed) and exit, written to p.stamps at the end; the
// values of the last tile a workgroup computed are kept.
template <typename G, int OUT, int MODE, typename MF, int ES, bool RES, bool STAMP = false>
__device__ __forceinline__ void pp_gemm_body(const I8GemmArgs& p) {
#pragma clang fp contract(off)
  constexpr int YS = pp_copies<G>();
  // the next tile's stage-0 prefetch needs 32 staged output rows of a wave to
  // fit in A slots 1-2 (2-byte outputs of the 256-row tiles)
  constexpr bool PREF = out_size<OUT>() == 2 && 32 * (G::WN * 2 + 16) <= (G::NA - 1) * G::STAGE_A / G::NW;
  constexpr int EPI_BASE = PREF ? G::STAGE_A : 0;
  constexpr int EPI_REGION = PREF ? (G::NA - 1) * G::STAGE_A / G::NW : G::RING / G::NW;
  using PP = PpParams<G>;
  __shared__ __attribute__((aligned(1024))) char smem[G::RING + 2 * PP::BYTES];
  static_assert(G::RING + 2 * PP::BYTES <= 160 * 1024, "LDS per CU");
  static_assert(G::BM % 64 == 0 && G::BN % 64 == 0 && G::BM <= 256 && G::BN <= 256,
                "parameter copies: whole waves of the first four");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave / G::WGN, wc = wave % G::WGN;
  const bool grp_x = wave < 4;
  const int total = ceil_div(p.M, G::BM) * ceil_div(p.N, G::BN);
  const int S = p.K * ES / G::KS;
  const char* a_base = reinterpret_cast<const char*>(p.a);
  const char* w_base = reinterpret_cast<const char*>(p.w);

  // Copy i of a wave covers rows 8 (gw + 4 i) .. + 7 of its operand's tile;
  // the 32-bit row offsets (clamped rows, swizzled chunk) are computed once
  // per tile. fp8 W (64-byte stage rows): copy i covers W rows
  // 16 (gw + 4 i) .. + 15, lane l fetching chunk (l & 3) ^ ((l >> 4) & 3) of
  // row l >> 2, which lands at LDS chunk l & 3 of that row (the swizzle the
  // fragment reads expect).
  uint32_t voff[YS];
  auto plan_offsets = [&](int m0_, int n0_) __attribute__((always_inline)) {
    if (G::W8 && grp_x) {
      const int row0 = n0_ + 16 * (wave & 3) + (lane >> 2);
      const uint32_t chunk16 = static_cast<uint32_t>(((lane & 3) ^ ((lane >> 4) & 3)) << 4);
      const uint32_t stride = static_cast<uint32_t>(p.w_sn);  // bytes
      static_for<0, YS>([&](auto i_c) {
        constexpr int I = decltype(i_c)::value;
        voff[I] = static_cast<uint32_t>(min(row0 + 64 * I, p.N - 1)) * stride + chunk16;
      });
      return;
    }
    const CopyPlan<4> plan(grp_x ? n0_ : m0_, wave & 3, lane);
    const int rows = grp_x ? p.N : p.M;
    const uint32_t stride = static_cast<uint32_t>((grp_x ? p.w_sn : p.a_sm) * ES);  // bytes
    static_for<0, YS>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      voff[I] = static_cast<uint32_t>(min(plan.row0 + 32 * I, rows - 1)) * stride + plan.chunk16;
    });
  };

  // epilogue parameters of a tile into parameter buffer `buf`: X wave w
  // copies rows / columns 64 w .. 64 w + 63 (constants where an operand is
  // absent are written directly)
  auto copy_params = [&](int m0_, int n0_, int buf) __attribute__((always_inline)) {
    if constexpr (MODE != EPI_INT) {
      if (!grp_x) return;
      char* const pb = smem + G::RING + buf * PP::BYTES;
      const uint32_t pba = lds_addr_of(pb) + 256 * wave;
      if (64 * wave < G::BM) {
        if (p.a_scale)
          dma4s(p.a_scale, 4u * static_cast<uint32_t>(min(m0_ + 64 * wave + lane, p.M - 1)), pba + PP::SA);
        else
          reinterpret_cast<float*>(pb + PP::SA)[64 * wave + lane] = 1.0f;
      }
      if (64 * wave < G::BN) {
        const uint32_t col = static_cast<uint32_t>(min(n0_ + 64 * wave + lane, p.N - 1));
        if (p.b_scale)
          dma4s(p.b_scale, p.b_scalar ? 0u : 4u * col, pba + PP::SB);
        else
          reinterpret_cast<float*>(pb + PP::SB)[64 * wave + lane] = 1.0f;
        if (p.bias != nullptr) {  // the epilogue reads the bias words only with a bias
          if (p.bias_dtype == QG_F32) dma4s(p.bias, 4u * col, pba + PP::BIAS);
          else dma2s(p.bias, 2u * col, pba + PP::BIAS);
        }
      }
    }
  };

  int t = blockIdx.x;
  int m0, n0;
  tile_origin_at<G::BM, G::BN>(p, t, m0, n0);
  plan_offsets(m0, n0);
  copy_params(m0, n0, 0);
  int buf = 0;
  bool pre = false;
  bool stores_fly = false;
  // lower bound of the full-tile epilogue's 16-byte stores per wave (2-byte
  // outputs; the compiler can only split them into more instructions)
  constexpr int kStoresPerWave = (PREF && !RES) ? G::FM * (G::WN * out_size<OUT>() / 16) / 2 : 0;
  static_assert(kStoresPerWave + pp_copies<G>() < 64, "vmcnt range");
  typename MF::acc_t acc[G::FM][G::FN];
  uint32_t stv[4] = {0, 0, 0, 0};
  uint32_t t_entry = 0, t_loop = 0, t_epi = 0;
  uint64_t rt_entry = 0;
  if constexpr (STAMP) {
    t_entry = static_cast<uint32_t>(__builtin_amdgcn_s_memtime());
    rt_entry = __builtin_amdgcn_s_memrealtime();
  }
  for (;;) {
    // The lane index passes through an opaque copy per tile: lane-derived LDS
    // and global offsets of the main loop and the epilogue are then recomputed
    // per tile instead of being hoisted out of the tile loop (which needs more
    // registers than the main loop leaves free).
    int lane_t = lane;
    asm volatile("" : "+v"(lane_t));
    static_for<0, G::FM>([&](auto i) {
      static_for<0, G::FN>([&](auto j) { acc[i][j] = typename MF::acc_t{}; });
    });
    // the parameter copies complete with the main loop's first waits (issued
    // before the stage-0 copies; K = 0 has no such wait); each X wave then
    // widens the bias words it copied to fp32 in place
    auto park = [&]() __attribute__((always_inline)) {
      if (S <= 0) wait_vm<0>();
      if constexpr (MODE != EPI_INT) {
        if (grp_x && 64 * wave < G::BN && p.bias != nullptr && p.bias_dtype != QG_F32) {
          uint32_t* const bw = reinterpret_cast<uint32_t*>(smem + G::RING + buf * PP::BYTES + PP::BIAS);
          const uint32_t bits = bw[64 * wave + lane];
          bw[64 * wave + lane] = __float_as_uint(bias_value(bits, p.bias_dtype));
        }
      }
    };
    pp_mainloop<G, MF, kStoresPerWave, STAMP>(acc, smem, a_base, w_base, voff, S, wave, lane_t, pre, park,
                                              stores_fly, stv);
    if constexpr (STAMP) t_loop = static_cast<uint32_t>(__builtin_amdgcn_s_memtime());
    const int tn = t + static_cast<int>(gridDim.x);
    const bool more = tn < total;
    int m1 = 0, n1 = 0;
    if (more) {
      tile_origin_at<G::BM, G::BN>(p, tn, m1, n1);
      plan_offsets(m1, n1);
      copy_params(m1, n1, buf ^ 1);
      if (PREF && S > 0) pp_prefetch0<G>(smem, a_base, w_base, voff, wave);
    }
    // the full-tile epilogue of 2-byte outputs issues kStoresPerWave 16-byte
    // stores per wave (no other vector memory operation) after the next
    // tile's stage-0 copies
    stores_fly = PREF && m0 + G::BM <= p.M && n0 + G::BN <= p.N && ((out_ld(p) * out_size<OUT>()) % 16) == 0 &&
                 (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
    pp_epilogue<G, OUT, MODE, RES, EPI_BASE, EPI_REGION, ES == 1>(p, acc, smem, smem + G::RING + buf * PP::BYTES,
                                                                  m0, n0, wr, wc, wave, lane_t);
    if constexpr (STAMP) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      t_epi = static_cast<uint32_t>(__builtin_amdgcn_s_memtime());
    }
    if (!more) break;
    wait_lds_barrier();
    t = tn;
    m0 = m1;
    n0 = n1;
    buf ^= 1;
    pre = PREF && S > 0;
  }
  if constexpr (STAMP) {
    const uint64_t rt_exit = __builtin_amdgcn_s_memrealtime();
    const uint32_t t_exit = static_cast<uint32_t>(__builtin_amdgcn_s_memtime());
    uint32_t* o = p.stamps + (static_cast<size_t>(blockIdx.x) * G::NW + wave) * kStampWords;
    static_for<0, 4>([&](auto q) { o[decltype(q)::value * 64 + lane] = stv[decltype(q)::value]; });
    if (lane == 0) {
      o[256] = t_entry;
      o[257] = t_loop;
      o[258] = t_epi;
      o[259] = t_exit;
      o[260] = static_cast<uint32_t>(rt_entry);
      o[261] = static_cast<uint32_t>(rt_exit);
      o[262] = __builtin_amdgcn_s_getreg((4 << 0) | (0 << 6) | (31 << 11));  // HW_ID (CU, SIMD, SE)
      o[263] = static_cast<uint32_t>(S);
    }
  }
}

template <typename G, int OUT, int MODE, bool RES>
__global__ __launch_bounds__(G::THREADS, 1) void k_i8_gemm_pp(I8GemmArgs p) {
  pp_gemm_body<G, OUT, MODE, MfmaI8, 1, RES>(p);
}

// Stage-timing instantiation of the ping-pong INT8 GEMM (fp16 output, order
// F): the same schedule with shader-clock stamps (qg_int8_gemm_stages).
template <typename G>
__global__ __launch_bounds__(G::THREADS, 1) void k_i8_gemm_pp_stages(I8GemmArgs p) {
  pp_gemm_body<G, QG_F16, EPI_F, MfmaI8, 1, false, true>(p);
}

// fp16 / bf16 A [M, K] and W [N, K] (K a multiple of 64, 16-byte aligned
// rows): out = f32(acc) * (1 * w_scale[n]) + bias in order F, one rounding.
// Serves the fp8 weight-only GEMM on large grids, after an exact fp8 -> 2-byte
// decode of W.
template <typename G, int OUT, bool F16A>
__global__ __launch_bounds__(G::THREADS, 1) void k_h16_gemm_pp(I8GemmArgs p) {
  pp_gemm_body<G, OUT, EPI_F, MfmaHalf<F16A>, 2, false>(p);
}

// fp16 / bf16 A [M, K] against fp8 (e4m3fn or e5m2) W [N, K] (K a multiple of
// 64, 16-byte aligned rows): W stages stay fp8 in LDS and each fragment is
// converted exactly to A's type in registers; the products, fp32 accumulation
// and order-F epilogue are those of k_h16_gemm_pp on the decoded weight.
template <typename G, int OUT, bool F16A, bool E5>
__global__ __launch_bounds__(G::THREADS, 1) void k_f8w_gemm_pp(I8GemmArgs p) {
  pp_gemm_body<G, OUT, EPI_F, MfmaHalfF8W<F16A, E5>, 2, false>(p);
}

// Raw buffer resources (stride 0, range checked against num_records bytes):
// the gfx9 descriptor word 3 (32-bit data format), and an offset that no
// buffer this library builds reaches (their num_records stay at or below
// it), so a store at it is dropped by the range check.
constexpr int kBufferWord3 = 0x00020000;
constexpr uint32_t kOobOffset = 0x7FFFFFF0u;

__device__ __forceinline__ float silu(float g) {
#pragma clang fp contract(off)
  // g / (1 + e^-g) with the hardware exp2 and reciprocal (a few ulps)
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

// Candidate work items per workgroup of the grouped kernel: their table
// entries are copied into LDS at the start (launch_i8_moe_gemm rejects plans
// that would need more).
constexpr int kMoeItems = 512;

// Grouped (MoE) INT8 GEMM on the ping-pong main loop, persistent. Work items
// are the device tile table's tiles in use (tile 0's spare field holds their
// number) x ceil(N / G::BN) column tiles: tile t = {expert e (< 0: none), first
// routed row m0, end of the expert's valid rows}. Each XCD takes one
// contiguous range of items and workgroup b (XCD b & 7) every (gridDim.x /
// 8)-th item of its range, skipping table entries that name no tile. A row of
// routed row r is row_token[r] (or r); W and b_scale start at expert e.
// Epilogues (v = f32(acc) * (sa[r] * sb[e, n]), order F):
//   QG_MOE_EPI_I32       out int32 [M, N] = acc (routed rows)
//   QG_MOE_EPI_SILU_MUL  columns 32 b .. 32 b + 15 are the gate and
//                        32 b + 16 .. 32 b + 31 the up rows of features
//                        16 b .. 16 b + 15: out bf16 [M, N / 2] = silu(g) * u
//                        (in the transposed layout the gate and up values of
//                        a feature sit in the same lane, registers r and r + 8)
//   QG_MOE_EPI_ROUTE     out bf16 [slots, N] row row_slot[r] = v * row_weight[r]
// As in the dense persistent body, the next item's stage-0 copies (A slot 0,
// W slot 0) are issued before the current item's epilogue, which stages its
// bf16 rows 32 at a time in A slots 1-2, and a barrier after the epilogue
// keeps the next item's stage-1 copies off the LDS the epilogue still reads.
// The staged epilogue's stores are buffer stores whose lanes without a valid
// target get an offset past the buffer's range, which the hardware drops:
// every wave issues the same number of them per item, so the next main loop
// lets them fly past its stage-0 waits.
// No item-boundary step waits for memory: the table entries of a workgroup's
// candidate items are copied into LDS at the start; the row_token values of
// item i + 1's rows are copied into LDS at item i - 1's prefetch point (after
// its main loop) and read at item i's, where they give item i + 1's A copy
// offsets and the copies of its epilogue parameters (row scale, routing
// weight, output row, column scale) straight into LDS (token and parameter
// buffers alternate by item parity). Every such copy lands before the next
// main loop's first barrier (the X waves wait for all their copies at each
// stage). No register loaded from memory is read after the epilogue's
// stores are issued: the compiler's own wait for it would drain the stores.
template <typename G, int MOE>
__global__ __launch_bounds__(G::THREADS, 1) void k_i8_moe_pp(I8GemmArgs p) {
#pragma clang fp contract(off)
  constexpr int YS = pp_copies<G>();
  constexpr int YA = G::BM / 32;                                    // A copies per Y wave and stage
  constexpr int EPI_BASE = G::STAGE_A;                              // A slots 1-2
  constexpr int EPI_REGION = (G::NA - 1) * G::STAGE_A / G::NW;     // bytes per wave
  // parameter buffer: row scales, routing weights, output rows, column scales
  constexpr int P_SA = 0, P_RW = 4 * G::BM, P_DST = 8 * G::BM, P_SB = 12 * G::BM;
  constexpr int PSZ = 12 * G::BM + 4 * G::BN;
  // the expert weights' copies carry the non-temporal hint: cfg4 forward
  // 288.1-289.3 -> 284.4-285.2 us (alternating processes, one box); the
  // dense kernels keep plain copies (the cfg1 chain measured 3.5 % slower
  // with the hint)
  constexpr bool NTW = true;
  constexpr int TAB = G::RING + 2 * PSZ;    // candidate table, kMoeItems x {e, m0, m_end, n0}
  constexpr int TOK = TAB + 16 * kMoeItems;  // two token buffers of BM rows
  __shared__ __attribute__((aligned(1024))) char smem[TOK + 8 * G::BM];
  static_assert(TOK + 8 * G::BM <= 160 * 1024, "LDS per CU");
  static_assert(G::BM % 64 == 0 && G::BN % 64 == 0 && G::BM <= 256 && G::BN <= 256,
                "parameter copies: whole waves of the first four");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave / G::WGN, wc = wave % G::WGN;
  const bool grp_x = wave < 4;

  const int ncol = ceil_div(p.N, G::BN);
  const int used = min(max(p.tiles[3], 0), p.tiles_max) * ncol;
  const int per_xcd = (used + 7) >> 3;
  const int slots = static_cast<int>(gridDim.x) >> 3;  // the grid is a multiple of 8
  const int first = (static_cast<int>(blockIdx.x) & 7) * per_xcd;
  const int last = min(first + per_xcd, used);
  const int S = p.K / G::KS;
  const int item0 = first + (static_cast<int>(blockIdx.x) >> 3);
  const int nitems = item0 < last ? min(ceil_div(last - item0, slots), kMoeItems) : 0;

  // candidate c = item item0 + c slots: {e, m0, m_end, n0}, e = -1 where its
  // table entry names no tile or a tile outside the operands
  i32x4* const tab = reinterpret_cast<i32x4*>(smem + TAB);
  for (int c = tid; c < nitems; c += G::THREADS) {
    const int w = item0 + c * slots;
    const int tile = w / ncol, ct = w - tile * ncol;
    const int e_ = p.tiles[4 * tile], m0_ = p.tiles[4 * tile + 1], mend_ = p.tiles[4 * tile + 2];
    const bool ok = e_ >= 0 && e_ < p.n_experts && m0_ >= 0 && m0_ < p.M && mend_ > m0_ && mend_ <= p.M;
    tab[c] = i32x4{ok ? e_ : -1, m0_, mend_, ct * G::BN};
  }
  __syncthreads();
  auto next_valid = [&](int c) {
    while (c < nitems && __builtin_amdgcn_readfirstlane(tab[c][0]) < 0) ++c;
    return c;
  };
  auto entry = [&](int c, int& e_, int& m0_, int& mend_, int& n0_) {
    const i32x4 t = tab[c];
    e_ = __builtin_amdgcn_readfirstlane(t[0]);
    m0_ = __builtin_amdgcn_readfirstlane(t[1]);
    mend_ = __builtin_amdgcn_readfirstlane(t[2]);
    n0_ = __builtin_amdgcn_readfirstlane(t[3]);
  };
  int cur = next_valid(0);
  if (cur >= nitems) return;
  int e = 0, m0 = 0, m_end = 0, n0 = 0;
  entry(cur, e, m0, m_end, n0);
  int nxt = next_valid(cur + 1);
  int e1 = 0, m1 = 0, mend1 = 0, n1 = 0;
  if (nxt < nitems) entry(nxt, e1, m1, mend1, n1);

  // row_token values of an item's rows (entry j: row min(m0 + j, M - 1)),
  // copied into token buffer `buf` by the X waves (each 64 rows)
  auto copy_tokens = [&](int m0_, int buf) __attribute__((always_inline)) {
    if (p.row_token == nullptr || !grp_x || 64 * wave >= G::BM) return;
    dma4s(p.row_token, 4u * static_cast<uint32_t>(min(m0_ + 64 * wave + lane, p.M - 1)),
          lds_addr_of(smem + TOK + buf * 4 * G::BM) + 256 * wave);
  };
  // A row of routed row m0_ + j (j < BM; the row clamped to M - 1)
  auto src_row = [&](int m0_, int j, int buf) {
    const int r = min(m0_ + j, p.M - 1);
    if (p.row_token == nullptr) return min(r, p.a_rows - 1);
    const int tok = reinterpret_cast<const int*>(smem + TOK + buf * 4 * G::BM)[r - m0_];
    return min(max(tok, 0), p.a_rows - 1);
  };
  uint32_t voff[YS];
  auto plan_offsets = [&](int m0_, int n0_, int buf) __attribute__((always_inline)) {
    const CopyPlan<4> plan(grp_x ? n0_ : m0_, wave & 3, lane);
    static_for<0, YS>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      if (grp_x) {
        voff[I] = static_cast<uint32_t>(min(plan.row0 + 32 * I, p.N - 1)) * static_cast<uint32_t>(p.w_sn) +
                  plan.chunk16;
      } else if constexpr (I < YA) {
        const int src = src_row(m0_, plan.row0 - m0_ + 32 * I, buf);
        voff[I] = static_cast<uint32_t>(src) * static_cast<uint32_t>(p.a_sm) + plan.chunk16;
      }
    });
  };
  // epilogue parameters of an item, copied into parameter buffer `buf` by the
  // X waves (each 64 rows / columns)
  auto copy_params = [&](int e_, int m0_, int n0_, int buf) __attribute__((always_inline)) {
    if constexpr (MOE != QG_MOE_EPI_I32) {
      if (!grp_x) return;
      const uint32_t pb = lds_addr_of(smem + G::RING + buf * PSZ) + 256 * wave;
      if (64 * wave < G::BM) {
        const int r = min(m0_ + 64 * wave + lane, p.M - 1);
        dma4s(p.a_scale, 4u * static_cast<uint32_t>(src_row(m0_, 64 * wave + lane, buf)), pb + P_SA);
        if constexpr (MOE == QG_MOE_EPI_ROUTE) {
          dma4s(p.row_weight, 4u * static_cast<uint32_t>(r), pb + P_RW);
          dma4s(p.row_slot, 4u * static_cast<uint32_t>(r), pb + P_DST);
        }
      }
      if (64 * wave < G::BN)
        dma4s(p.b_scale + static_cast<int64_t>(e_) * p.N,
              4u * static_cast<uint32_t>(min(n0_ + 64 * wave + lane, p.N - 1)), pb + P_SB);
    }
  };
  const char* a_base = reinterpret_cast<const char*>(p.a);
  auto w_base = [&](int e_) { return reinterpret_cast<const char*>(p.w) + static_cast<int64_t>(e_) * p.w_estride; };
  // tokens of the first two items, then the first item's offsets and parameters
  copy_tokens(m0, 0);
  if (nxt < nitems) copy_tokens(m1, 1);
  wait_vm<0>();
  __syncthreads();
  plan_offsets(m0, n0, 0);
  copy_params(e, m0, n0, 0);

  // bf16 outputs whose rows take whole 16-byte chunks are staged per wave, 32
  // rows at a time, and written as row chunks; int32 (test) output goes
  // element-wise
  constexpr bool STAGED = MOE != QG_MOE_EPI_I32;
  constexpr int OCOLS = MOE == QG_MOE_EPI_SILU_MUL ? G::WN / 2 : G::WN;  // output columns per wave row
  constexpr int ROWB = OCOLS * 2 + 16;
  constexpr int CH = OCOLS * 2 / 16;
  static_assert(32 * ROWB <= EPI_REGION, "staging region");
  static_assert((32 * CH) % 64 == 0, "whole chunk rounds per lane");
  const int out_cols = MOE == QG_MOE_EPI_SILU_MUL ? p.N / 2 : p.N;
  // ST: the staged epilogue's 16-byte stores per wave and item
  constexpr int ST = STAGED ? G::FM * (32 * CH / 64) : 0;
  static_assert(ST + YS + 4 < 64, "vmcnt range");
  const int64_t out_bytes = static_cast<int64_t>(p.out_rows) * p.out_sm * 2;
  const bool staged = STAGED && (out_cols % 8) == 0 && (p.out_sm % 8) == 0 &&
                      (reinterpret_cast<uintptr_t>(p.out) & 15) == 0 && out_bytes <= kOobOffset;
  // raw buffer over out (num_records in bytes, below kOobOffset)
  const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      p.out, 0, static_cast<int>(staged ? out_bytes : 0), kBufferWord3);
  char* const region = smem + EPI_BASE + wave * EPI_REGION;

  bool pre = false;
  int buf = 0;
  i32x16 acc[G::FM][G::FN];
  for (;;) {
    // lane-derived offsets recomputed per item instead of hoisted (registers)
    int lane_t = lane;
    asm volatile("" : "+v"(lane_t));
    static_for<0, G::FM>([&](auto i) {
      static_for<0, G::FN>([&](auto j) { acc[i][j] = i32x16{}; });
    });
    // the parameter copies complete with the main loop's first waits (issued
    // before the stage-0 copies); K = 0 has no such wait
    auto park = [&]() __attribute__((always_inline)) {
      if (S <= 0) wait_vm<0>();
    };
    pp_mainloop<G, MfmaI8, ST, false, NTW>(acc, smem, a_base, w_base(e), voff, S, wave, lane_t, pre, park, staged);

    // the next item: its copy offsets, parameter copies and stage-0 copies
    // ahead of this item's epilogue, then the tokens of the item after it
    const bool more = nxt < nitems;
    int nn = nitems, e2 = 0, m2 = 0, mend2 = 0, n2 = 0;
    if (more) {
      plan_offsets(m1, n1, buf ^ 1);
      copy_params(e1, m1, n1, buf ^ 1);
      if (S > 0) pp_prefetch0<G, NTW>(smem, a_base, w_base(e1), voff, wave);
      nn = next_valid(nxt + 1);
      if (nn < nitems) {
        entry(nn, e2, m2, mend2, n2);
        copy_tokens(m2, buf);  // this item's tokens are no longer read
      }
    }

    // ---- epilogue of this item ----------------------------------------------
    const char* const pbuf = smem + G::RING + buf * PSZ;
    const float* sa_lds = reinterpret_cast<const float*>(pbuf + P_SA);
    const float* rw_lds = reinterpret_cast<const float*>(pbuf + P_RW);
    const int* dst_lds = reinterpret_cast<const int*>(pbuf + P_DST);
    const float* sb_lds = reinterpret_cast<const float*>(pbuf + P_SB);
    const int lr = lane_t & 31, lq = 4 * (lane_t >> 5);
    static_for<0, G::FM>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      const int rl_i = wr * G::WM + 32 * i + lr;  // row in the tile
      const float sa = sa_lds[rl_i];
      const float rwv = MOE == QG_MOE_EPI_ROUTE ? rw_lds[rl_i] : 0.0f;
      static_for<0, G::FN>([&](auto j_c) {
        constexpr int j = decltype(j_c)::value;
        if constexpr (MOE == QG_MOE_EPI_I32) {
          static_for<0, 4>([&](auto g_c) {
            constexpr int g = decltype(g_c)::value;
            const int row = m0 + rl_i;
            static_for<0, 4>([&](auto c) {
              const int n = n0 + wc * G::WN + 32 * j + 8 * g + lq + decltype(c)::value;
              if (row < m_end && n < p.N)
                static_cast<int32_t*>(p.out)[static_cast<int64_t>(row) * p.out_sm + n] =
                    acc[i][j][4 * g + decltype(c)::value];
            });
          });
        } else if constexpr (MOE == QG_MOE_EPI_SILU_MUL) {
          static_for<0, 2>([&](auto g_c) {
            constexpr int g = decltype(g_c)::value;
            const f32x4 sbg = col4(sb_lds, wc * G::WN + 32 * j + 8 * g + lq);
            const f32x4 sbu = col4(sb_lds, wc * G::WN + 32 * j + 8 * (g + 2) + lq);
            float h[4];
            static_for<0, 4>([&](auto c) {
              constexpr int C = decltype(c)::value;
              const float gv = static_cast<float>(acc[i][j][4 * g + C]) * (sa * sbg[C]);
              const float uv = static_cast<float>(acc[i][j][4 * (g + 2) + C]) * (sa * sbu[C]);
              h[C] = silu(gv) * uv;
            });
            const int fl = 16 * j + 8 * g + lq;  // feature in the wave's output columns
            if (staged) {
              *reinterpret_cast<u32x2*>(region + lr * ROWB + fl * 2) =
                  u32x2{pack2<QG_BF16>(h[0], h[1]), pack2<QG_BF16>(h[2], h[3])};
            } else {
              const int row = m0 + rl_i;
              const int f0 = (n0 + wc * G::WN) / 2 + fl;
              if (row < m_end) {
                static_for<0, 4>([&](auto c) {
                  if (f0 + decltype(c)::value < out_cols)
                    static_cast<uint16_t*>(p.out)[static_cast<int64_t>(row) * p.out_sm + f0 + decltype(c)::value] =
                        f32_to_bf16(h[decltype(c)::value]);
                });
              }
            }
          });
        } else {
          static_for<0, 4>([&](auto g_c) {
            constexpr int g = decltype(g_c)::value;
            const int cl = wc * G::WN + 32 * j + 8 * g + lq;  // tile column
            const f32x4 sb4 = col4(sb_lds, cl);
            float y[4];
            static_for<0, 4>([&](auto c) {
              constexpr int C = decltype(c)::value;
              const float v = static_cast<float>(acc[i][j][4 * g + C]) * (sa * sb4[C]);
              y[C] = v * rwv;
            });
            if (staged) {
              *reinterpret_cast<u32x2*>(region + lr * ROWB + (32 * j + 8 * g + lq) * 2) =
                  u32x2{pack2<QG_BF16>(y[0], y[1]), pack2<QG_BF16>(y[2], y[3])};
            } else {
              const int d = dst_lds[rl_i];
              if (m0 + rl_i < m_end && d >= 0 && d < p.out_rows) {
                static_for<0, 4>([&](auto c) {
                  const int n = n0 + cl + decltype(c)::value;
                  if (n < p.N)
                    static_cast<uint16_t*>(p.out)[static_cast<int64_t>(d) * p.out_sm + n] =
                        f32_to_bf16(y[decltype(c)::value]);
                });
              }
            }
          });
        }
      });
      if constexpr (STAGED) {
        if (staged) {
          // LDS accesses of one wave complete in order: the reads see this
          // pass's writes, and the next pass's writes follow these reads
          const int col0 = (MOE == QG_MOE_EPI_SILU_MUL ? (n0 + wc * G::WN) / 2 : n0 + wc * G::WN);
#pragma unroll
          for (int c0 = 0; c0 < 32 * CH; c0 += 64) {
            const int c = c0 + lane_t;
            const int rr = c / CH, cc = c - rr * CH;
            const int rl = wr * G::WM + 32 * i + rr;
            const int row = m0 + rl;
            const int d = MOE == QG_MOE_EPI_ROUTE ? dst_lds[rl] : row;
            const int col = col0 + cc * 8;
            const bool ok = row < m_end && d >= 0 && d < p.out_rows && col + 8 <= out_cols;
            const uint32_t off = ok ? static_cast<uint32_t>((static_cast<int64_t>(d) * p.out_sm + col) * 2) : kOobOffset;
            const i32x4 v = *reinterpret_cast<const i32x4*>(region + rr * ROWB + cc * 16);
            __builtin_amdgcn_raw_buffer_store_b128(v, out_rsrc, off, 0, 0);
          }
        }
      }
    });
    if (!more) break;
    wait_lds_barrier();
    cur = nxt;
    e = e1;
    m0 = m1;
    m_end = mend1;
    n0 = n1;
    nxt = nn;
    e1 = e2;
    m1 = m2;
    mend1 = mend2;
    n1 = n2;
    buf ^= 1;
    pre = S > 0;
  }
}

// CUs of an MI355X (gfx950): the persistent grid size.
constexpr int kPersistentCUs = 256;

template <typename G, int WPE, int OUT, int MODE, bool RES = false>
hipError_t launch_tile(const I8GemmArgs& p, hipStream_t stream) {
  static_assert(G::LDS_BYTES * WPE <= 160 * 1024, "LDS per CU");
  const int blocks = ceil_div(p.M, G::BM) * ceil_div(p.N, G::BN);
  if constexpr (G::NW == 4)
    hipLaunchKernelGGL((k_i8_gemm<G, WPE, OUT, MODE, RES>), dim3(blocks), dim3(G::THREADS), 0, stream, p);
  else  // persistent: at most one workgroup per CU (LDS), a multiple of the 8 XCDs
    hipLaunchKernelGGL((k_i8_gemm_pp<G, OUT, MODE, RES>), dim3(blocks < kPersistentCUs ? blocks : kPersistentCUs),
                       dim3(G::THREADS), 0, stream, p);
  return hipGetLastError();
}

template <typename G, int WPE, int OUT>
hipError_t launch_mode(const I8GemmArgs& p, hipStream_t stream) {
  // Orders F and E coincide for fp32 output (no intermediate rounding).
  // residual term (qg_w8a8_linear_ex): its own instantiations, so the plain
  // kernels carry no residual code
  if (p.residual) {
    if (p.epi & QG_EPI_GELU_TANH) return launch_tile<G, WPE, OUT, EPI_GELU, true>(p, stream);
    if (p.epi & QG_EPI_ORDER_FUSED_FMA) return launch_tile<G, WPE, OUT, EPI_FMA, true>(p, stream);
    return launch_tile<G, WPE, OUT, EPI_F, true>(p, stream);
  }
  if (p.epi & QG_EPI_GELU_TANH) return launch_tile<G, WPE, OUT, EPI_GELU>(p, stream);
  if (p.epi & QG_EPI_ORDER_FUSED_FMA) return launch_tile<G, WPE, OUT, EPI_FMA>(p, stream);
  if constexpr (OUT != QG_F32) {
    if (p.epi & QG_EPI_ORDER_EAGER) return launch_tile<G, WPE, OUT, EPI_EAGER>(p, stream);
  }
  return launch_tile<G, WPE, OUT, EPI_F>(p, stream);
}

template <typename G, int WPE>
hipError_t launch_variant(const I8GemmArgs& p, hipStream_t stream) {
  if (p.a_scale == nullptr) return launch_tile<G, WPE, QG_I32, EPI_INT>(p, stream);
  if (p.out_dtype == QG_F16) return launch_mode<G, WPE, QG_F16>(p, stream);
  if (p.out_dtype == QG_BF16) return launch_mode<G, WPE, QG_BF16>(p, stream);
  return launch_mode<G, WPE, QG_F32>(p, stream);
}

}  // namespace

hipError_t launch_i8_moe_gemm(const I8GemmArgs& p, hipStream_t stream) {
  // 192-row tiles: expert segments of ~512-576 rows (cfg4) fill 3 tiles
  using G = I8Geo<QG_MOE_TILE_ROWS, 256, 2, 4, 3>;
  static_assert(G::LDS_BYTES <= 160 * 1024, "LDS per CU");
  // persistent: at most one workgroup per CU, a multiple of the 8 XCDs
  const long items = static_cast<long>(p.tiles_max) * ceil_div(p.N, G::BN);
  if (items == 0) return hipSuccess;
  const int blocks = items < kPersistentCUs ? static_cast<int>((items + 7) & ~7L) : kPersistentCUs;
  // candidate items per workgroup: its share of one XCD's contiguous range
  const long per_xcd = (items + 7) / 8, slots = blocks / 8;
  if ((per_xcd + slots - 1) / slots > kMoeItems) return hipErrorInvalidValue;
  switch (p.moe_epi) {
    case QG_MOE_EPI_I32:
      hipLaunchKernelGGL((k_i8_moe_pp<G, QG_MOE_EPI_I32>), dim3(blocks), dim3(G::THREADS), 0, stream, p);
      break;
    case QG_MOE_EPI_SILU_MUL:
      hipLaunchKernelGGL((k_i8_moe_pp<G, QG_MOE_EPI_SILU_MUL>), dim3(blocks), dim3(G::THREADS), 0, stream, p);
      break;
    default:
      hipLaunchKernelGGL((k_i8_moe_pp<G, QG_MOE_EPI_ROUTE>), dim3(blocks), dim3(G::THREADS), 0, stream, p);
  }
  return hipGetLastError();
}

hipError_t launch_i8_gemm_stages(const I8GemmArgs& p, hipStream_t stream) {
  using G = I8Geo<256, 192, 4, 2, 3>;
  const int tiles = ceil_div(p.M, G::BM) * ceil_div(p.N, G::BN);
  if (tiles == 0) return hipSuccess;
  hipLaunchKernelGGL((k_i8_gemm_pp_stages<G>), dim3(tiles < kPersistentCUs ? tiles : kPersistentCUs),
                     dim3(G::THREADS), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_i8_gemm(const I8GemmArgs& p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  // 256x192 tiles tile every benchmark shape into whole multiples of the 256
  // CUs (4096x3072 -> 256 tiles, x9216 -> 768, x12288 -> 1024). Smaller
  // problems use 128x128 tiles so that more CUs get work.
  const long big = static_cast<long>(ceil_div(p.M, 256)) * ceil_div(p.N, 192);
  if (big >= 192) return launch_variant<I8Geo<256, 192, 4, 2, 3>, 1>(p, stream);
  return launch_variant<I8Geo<128, 128, 2, 2, 2>, 2>(p, stream);
}

namespace {

// Tail split of a persistent launch of BM x BN tiles. When the tiles take more
// than one round of kPersistentCUs workgroups and the last round would run
// one big tile per busy CU while the rest wait, columns [0, n1) keep the big
// tiles in whole rounds and columns [n1, N) run as a single round of 128 x 128
// tiles (a third of a 256 x 192 tile's work each), so the last round takes
// about half the time. Returns n1, or 0 for no split (whole rounds already,
// a single round, or a remainder that needs more than one round of small
// tiles).
template <int BM, int BN>
int tail_split_cols(int M, int N) {
  const long nbm = ceil_div(M, BM), nbn = ceil_div(N, BN);
  const long tiles = nbm * nbn;
  if (tiles <= kPersistentCUs || tiles % kPersistentCUs == 0) return 0;
  const long c1 = tiles / kPersistentCUs * kPersistentCUs / nbm;  // column tiles in whole rounds
  if (c1 <= 0 || c1 >= nbn) return 0;
  const int n1 = static_cast<int>(c1) * BN;
  const long rem = static_cast<long>(ceil_div(M, 128)) * ceil_div(N - n1, 128);
  return rem <= kPersistentCUs ? n1 : 0;
}

// Columns [n1, N) of p as a problem of its own: W rows, column scales, bias
// values and output columns start at n1, and the output keeps p's row stride.
// w_es: bytes per W element.
I8GemmArgs column_slice(const I8GemmArgs& p, int n1, int w_es) {
  I8GemmArgs q = p;
  q.N = p.N - n1;
  q.w = p.w + static_cast<int64_t>(n1) * p.w_sn * w_es;
  if (p.b_scale != nullptr && !p.b_scalar) q.b_scale = p.b_scale + n1;
  if (p.bias != nullptr) q.bias = static_cast<const char*>(p.bias) + static_cast<int64_t>(n1) * (p.bias_dtype == QG_F32 ? 4 : 2);
  const int out_es = (p.out_dtype == QG_F16 || p.out_dtype == QG_BF16) ? 2 : 4;
  q.out = static_cast<char*>(p.out) + static_cast<int64_t>(n1) * out_es;
  q.out_sm = p.out_sm > 0 ? p.out_sm : p.N;
  return q;
}

template <typename G>
hipError_t launch_h16_geo(const I8GemmArgs& p, bool f16a, hipStream_t stream) {
  static_assert(G::LDS_BYTES <= 160 * 1024, "LDS per CU");
  const int tiles = ceil_div(p.M, G::BM) * ceil_div(p.N, G::BN);
  if (tiles == 0) return hipSuccess;
  const dim3 grid(tiles < kPersistentCUs ? tiles : kPersistentCUs);
#define QG_H16(OUT)                                                                                   \
  do {                                                                                                \
    if (f16a) hipLaunchKernelGGL((k_h16_gemm_pp<G, OUT, true>), grid, dim3(G::THREADS), 0, stream, p); \
    else hipLaunchKernelGGL((k_h16_gemm_pp<G, OUT, false>), grid, dim3(G::THREADS), 0, stream, p);    \
  } while (0)
  if (p.out_dtype == QG_F16) QG_H16(QG_F16);
  else if (p.out_dtype == QG_BF16) QG_H16(QG_BF16);
  else QG_H16(QG_F32);
#undef QG_H16
  return hipGetLastError();
}

}  // namespace

hipError_t launch_h16_gemm(const I8GemmArgs& p, bool f16a, hipStream_t stream) {
  using Big = I8Geo<256, 192, 4, 2, 3>;
  const int n1 = tail_split_cols<Big::BM, Big::BN>(p.M, p.N);
  if (n1 == 0) return launch_h16_geo<Big>(p, f16a, stream);
  I8GemmArgs head = p;
  head.N = n1;
  head.out_sm = p.out_sm > 0 ? p.out_sm : p.N;
  const hipError_t e = launch_h16_geo<Big>(head, f16a, stream);
  if (e != hipSuccess) return e;
  return launch_h16_geo<I8Geo<128, 128, 4, 2, 3>>(column_slice(p, n1, 2), f16a, stream);
}

hipError_t launch_f8w_gemm(const I8GemmArgs& p, bool f16a, bool e5, hipStream_t stream) {
  using G = F8Geo<256, 192, 4, 2, 3>;
  static_assert(G::LDS_BYTES <= 160 * 1024, "LDS per CU");
  const int tiles = ceil_div(p.M, G::BM) * ceil_div(p.N, G::BN);
  if (tiles == 0) return hipSuccess;
  const dim3 grid(tiles < kPersistentCUs ? tiles : kPersistentCUs);
#define QG_F8W(OUT, F16, E5)                                                                             \
  hipLaunchKernelGGL((k_f8w_gemm_pp<G, OUT, F16, E5>), grid, dim3(G::THREADS), 0, stream, p)
#define QG_F8W_OUT(OUT)                  \
  do {                                   \
    if (f16a && e5) QG_F8W(OUT, true, true);        \
    else if (f16a) QG_F8W(OUT, true, false);        \
    else if (e5) QG_F8W(OUT, false, true);          \
    else QG_F8W(OUT, false, false);                 \
  } while (0)
  if (p.out_dtype == QG_F16) QG_F8W_OUT(QG_F16);
  else if (p.out_dtype == QG_BF16) QG_F8W_OUT(QG_BF16);
  else QG_F8W_OUT(QG_F32);
#undef QG_F8W_OUT
#undef QG_F8W
  return hipGetLastError();
}

}  // namespace qg
