// INT8 x INT8 -> INT32 GEMM on gfx950 int8 MFMA with the fused dequant
// epilogue of rdna2-ops/rdna2_ops/int8_gemm.py:19-67 (and the Kitchen eager
// epilogue order of rdna2-ops/rdna2_ops/comfy_int8.py:128-143).
//
// Design (MI355X-first, not a translation of the reference's Triton tiles):
//  * one 256-thread workgroup (4 waves, 2x2) per BM x BN output tile; each wave
//    owns a (BM/2) x (BN/2) sub-tile held in 16x16 int32 MFMA accumulators;
//  * operands are A [M, K] and W [N, K], both K-contiguous ("NT"), so every
//    lane feeds v_mfma_i32_16x16x64_i8 with 16 contiguous K bytes;
//  * K advances in 128-byte stages (two 64-byte MFMA sub-steps). Each stage
//    of A and W is copied straight from HBM into a 2-slot LDS ring with
//    global_load_lds_dwordx4, 8 rows x 128 B (whole cache lines) per wave
//    instruction — the access pattern that sustains the most L2->LDS bandwidth
//    per CU on gfx950;
//  * software pipeline: a stage is read from LDS into registers while the
//    MFMAs of the previous stage run; as soon as every wave holds it, its slot
//    is refilled two stages ahead, so two stages (2 x 56 KB) stay in flight
//    behind the MFMAs;
//  * LDS rows are 128 bytes with the 16-byte chunk index XOR-swizzled by
//    (row & 7): the DMA writes and the fragment reads (8 consecutive lanes =
//    8 distinct 16-byte bank groups) are bank-conflict free;
//  * the linear block id is remapped so that each of the 8 XCDs (round-robin
//    workgroup dispatch) walks one contiguous, GROUP_M-ordered range of tiles,
//    keeping the A rows and W columns it shares in its own L2;
//  * the epilogue is specialised at compile time (output dtype x order) and,
//    for full tiles, stages the rounded tile through LDS so that HBM sees
//    coalesced 16-byte row stores.
#include "qg_common.h"
#include "qg_internal.h"

namespace qg {

namespace {

enum EpiMode { EPI_INT = 0, EPI_F = 1, EPI_FMA = 2, EPI_EAGER = 3, EPI_GELU = 4 };

template <int BM, int BN>
struct I8Tile {
  static constexpr int WM = BM / 2, WN = BN / 2;  // wave sub-tile
  static constexpr int FM = WM / 16, FN = WN / 16;  // 16x16 fragments per wave
  static constexpr int KS = 128;                   // K bytes per stage (2 MFMA sub-steps)
  static constexpr int STAGE_A = BM * KS, STAGE_B = BN * KS;
  static constexpr int STAGE = STAGE_A + STAGE_B;
  static constexpr int NST = 2;                    // LDS ring depth
  static constexpr int SEGS = (BM + BN) / 8;       // 1 KB DMA segments (8 rows x 128 B)
  static constexpr int SPW = SEGS / 4;             // segments per wave
  static constexpr int LDS_BYTES = NST * STAGE;
  static_assert(BM % 32 == 0 && BN % 32 == 0, "tile must split into 2x2 waves of 16-multiples");
  static_assert(SEGS % 4 == 0, "DMA segments must divide over 4 waves");
  static_assert(SPW <= 2 * FM, "DMA issue is spread over the second-half fragment rows");
};

__device__ __forceinline__ float gelu_tanh(float x) {
#pragma clang fp contract(off)
  // 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3))), in the operation
  // order of ATen's CPU GeluKernel (tanh approximation). tanh(u) is evaluated
  // as 1 - 2 / (exp(2u) + 1) with the hardware exp2 and reciprocal: absolute
  // error a few 1e-7, far below one fp16/bf16 ulp of the result.
  const float kBeta = 0.7978845608028654f;
  const float kKappa = 0.044715f;
  const float x_cube = x * x * x;
  const float inner = kBeta * (x + kKappa * x_cube);
  const float e = __builtin_amdgcn_exp2f(inner * 2.8853900817779268f);  // exp(2u) = 2^(2u log2 e)
  const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
  return 0.5f * x * (1.0f + t);
}

__device__ __forceinline__ float load_bias(const void* bias, int dtype, int col) {
  if (dtype == QG_F32) return static_cast<const float*>(bias)[col];
  const uint16_t b = static_cast<const uint16_t*>(bias)[col];
  return dtype == QG_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

template <int OUT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (OUT == QG_F16) return f16_to_f32(f32_to_f16(v));
  else if constexpr (OUT == QG_BF16) return bf16_to_f32(f32_to_bf16(v));
  else return v;
}

template <int OUT>
constexpr int out_size() { return (OUT == QG_F16 || OUT == QG_BF16) ? 2 : 4; }

// Storage bits of one output element.
//   EPI_F:     v = f32(acc) * (sa * sb); v = v + bias           (int8_gemm.py:53-63)
//   EPI_FMA:   v = fma(f32(acc), sa * sb, bias)                 (rounding="fused", :191)
//   EPI_EAGER: t = out(f32(acc) * (sa * sb)); t = out(t + out(bias))  (comfy_int8.py:128-143)
//   EPI_GELU:  EPI_F followed by GELU-tanh in fp32
template <int OUT, int MODE>
__device__ __forceinline__ uint32_t epi_bits(int32_t acc, float sa, float sb, float bv, bool has_bias) {
#pragma clang fp contract(off)
  if constexpr (MODE == EPI_INT) {
    return static_cast<uint32_t>(acc);
  } else {
    const float scale = sa * sb;
    const float accf = static_cast<float>(acc);
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
    if constexpr (OUT == QG_F32) return __float_as_uint(v);
    else if constexpr (OUT == QG_F16) return f32_to_f16(v);
    else return f32_to_bf16(v);
  }
}

template <int OUT>
__device__ __forceinline__ void store_elem(void* out, int64_t idx, uint32_t bits) {
  if constexpr (out_size<OUT>() == 4) static_cast<uint32_t*>(out)[idx] = bits;
  else static_cast<uint16_t*>(out)[idx] = static_cast<uint16_t>(bits);
}

template <int BM, int BN, int WPE, int OUT, int MODE>
__global__ __launch_bounds__(256, WPE) void k_i8_gemm(I8GemmArgs p) {
#pragma clang fp contract(off)
  using T = I8Tile<BM, BN>;
  __shared__ __attribute__((aligned(1024))) char smem[T::LDS_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int wr = wave >> 1, wc = wave & 1;

  // ---- tile order: XCD-contiguous ranges, GROUP_M-swizzled inside ---------
  const int nbm = ceil_div(p.M, BM), nbn = ceil_div(p.N, BN);
  const int total = nbm * nbn;
  int bid = blockIdx.x;
  if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  constexpr int GROUP_M = 4;
  const int group = bid / (GROUP_M * nbn);
  const int first = group * GROUP_M;
  const int gm = min(nbm - first, GROUP_M);
  const int in_group = bid - group * GROUP_M * nbn;
  const int m0 = (first + in_group % gm) * BM;
  const int n0 = (in_group / gm) * BN;

  // ---- DMA plan: this wave copies SPW 1 KB segments per stage --------------
  // Segment seg = wave + 4 i covers 8 rows: A rows for seg < BM/8, W rows
  // after. Lane l lands on LDS row (l >> 3) of the segment, physical chunk
  // (l & 7), and fetches the logical chunk that the swizzle stores there.
  // Offsets are 32-bit bytes from the operand base (operands < 2 GiB); they are
  // recomputed per copy from two base rows to keep registers for fragments.
  constexpr int A_SEGS_PER_WAVE = BM / 32;  // i < this: A segment
  static_assert((BM / 8) % 4 == 0 && (BN / 8) % 4 == 0, "segments split evenly over waves");
  const int srow = lane >> 3;
  const uint32_t schunk16 = static_cast<uint32_t>(((lane & 7) ^ srow) << 4);
  const int row_a = m0 + wave * 8 + srow;
  const int row_w = n0 + wave * 8 + srow;
  const uint32_t smem_base = lds_addr_of(smem);
  const int S = p.K / T::KS;
  const char* a_base = reinterpret_cast<const char*>(p.a);
  const char* w_base = reinterpret_cast<const char*>(p.w);
  auto dma = [&](auto i_c, int s) {
    constexpr int i = decltype(i_c)::value;
    const int64_t k = static_cast<int64_t>(s) * T::KS;
    const uint32_t slot = smem_base + (s & 1) * T::STAGE;
    // The opaque copy keeps the compiler from hoisting the 14 loop-invariant
    // offsets out of the K loop (they would be held in registers, or spilled).
    int ra = row_a, rw = row_w;
    asm volatile("" : "+v"(ra), "+v"(rw));
    if constexpr (i < A_SEGS_PER_WAVE) {
      const uint32_t row = static_cast<uint32_t>(min(ra + 32 * i, p.M - 1));
      dma16s(a_base + k, row * static_cast<uint32_t>(p.a_sm) + schunk16,
             slot + (wave + 4 * i) * 1024);
    } else {
      constexpr int iw = i - A_SEGS_PER_WAVE;
      const uint32_t row = static_cast<uint32_t>(min(rw + 32 * iw, p.N - 1));
      dma16s(w_base + k, row * static_cast<uint32_t>(p.w_sn) + schunk16,
             slot + T::STAGE_A + (wave + 4 * iw) * 1024);
    }
  };

  // Fragment read offsets of this lane (sub-step h reads logical chunks 4h..4h+3).
  int a_off[2], b_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int lo = (lane & 15) * T::KS + ((((h << 2) | (lane >> 4)) ^ (lane & 7)) << 4);
    a_off[h] = wr * T::WM * T::KS + lo;
    b_off[h] = T::STAGE_A + wc * T::WN * T::KS + lo;
  }

  i32x4 acc[T::FM][T::FN];
  static_for<0, T::FM>([&](auto i) {
    static_for<0, T::FN>([&](auto j) { acc[i][j] = i32x4{0, 0, 0, 0}; });
  });

  // Register copies of two stages: [buffer][sub-step][fragment].
  i32x4 fa[2][2][T::FM], fb[2][2][T::FN];

  if (S > 0) {
    // ---- prologue: stages 0 and 1 in flight, stage 0 into registers, stage 2
    // into the freed slot ------------------------------------------------------
    static_for<0, T::SPW>([&](auto i) { dma(i, 0); });
    if (S > 1) {
      static_for<0, T::SPW>([&](auto i) { dma(i, 1); });
      wait_vm_barrier<T::SPW>();
    } else {
      wait_vm_barrier<0>();
    }
    static_for<0, 2>([&](auto h) {
      static_for<0, T::FM>([&](auto i) {
        fa[0][h][i] = *reinterpret_cast<const i32x4*>(smem + a_off[h] + i * 16 * T::KS);
      });
      static_for<0, T::FN>([&](auto j) {
        fb[0][h][j] = *reinterpret_cast<const i32x4*>(smem + b_off[h] + j * 16 * T::KS);
      });
    });
    wait_lds_barrier();
    static_for<0, T::SPW>([&](auto i) { dma(i, min(2, S - 1)); });

    // ---- steady state, two stages per trip so register buffers are static ----
    //  barrier A  : stage s+1 landed everywhere
    //  first half : MFMAs of (s, sub-step 0); read all of stage s+1
    //  barrier B  : every wave holds stage s+1; its slot takes stage s+3
    //  second half: MFMAs of (s, sub-step 1) with the refill copies between them
    // Stages s+2 and s+3 are in flight behind the second half. Past the end the
    // last stage is re-copied into the free slot (never read) so that no branch
    // splits the MFMA chain, and next-stage reads run unconditionally on a
    // valid slot (their values are dead after the last stage).
    auto stage = [&](int s, auto cur_c) {
      constexpr int cur = decltype(cur_c)::value;
      constexpr int nxt = cur ^ 1;
      if (s + 2 < S) wait_vm_barrier<T::SPW>();
      else wait_vm_barrier<0>();
      const char* nbase = smem + ((s + 1) & 1) * T::STAGE;
      static_for<0, T::FM>([&](auto i) {
        static_for<0, T::FN>([&](auto j) {
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[cur][0][i], fb[cur][0][j], acc[i][j], 0, 0, 0);
        });
        __builtin_amdgcn_sched_barrier(0);
        fa[nxt][0][i] = *reinterpret_cast<const i32x4*>(nbase + a_off[0] + i * 16 * T::KS);
        fa[nxt][1][i] = *reinterpret_cast<const i32x4*>(nbase + a_off[1] + i * 16 * T::KS);
        if constexpr (i + 2 < T::FN) {
          fb[nxt][0][i] = *reinterpret_cast<const i32x4*>(nbase + b_off[0] + i * 16 * T::KS);
          fb[nxt][1][i] = *reinterpret_cast<const i32x4*>(nbase + b_off[1] + i * 16 * T::KS);
        }
      });
      static_for<(T::FN >= 2 ? T::FN - 2 : 0), T::FN>([&](auto j) {
        fb[nxt][0][j] = *reinterpret_cast<const i32x4*>(nbase + b_off[0] + j * 16 * T::KS);
        fb[nxt][1][j] = *reinterpret_cast<const i32x4*>(nbase + b_off[1] + j * 16 * T::KS);
      });
      wait_lds_barrier();
      const int refill_stage = min(s + 3, S - 1);
      static_for<0, T::FM>([&](auto i) {
        if constexpr (2 * i < T::SPW) dma(std::integral_constant<int, 2 * i>{}, refill_stage);
        if constexpr (2 * i + 1 < T::SPW) dma(std::integral_constant<int, 2 * i + 1>{}, refill_stage);
        static_for<0, T::FN>([&](auto j) {
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[cur][1][i], fb[cur][1][j], acc[i][j], 0, 0, 0);
        });
      });
    };
    int s = 0;
    for (; s + 1 < S; s += 2) {
      stage(s, std::integral_constant<int, 0>{});
      stage(s + 1, std::integral_constant<int, 1>{});
    }
    if (s < S) stage(s, std::integral_constant<int, 0>{});
  }

  // ---- epilogue -------------------------------------------------------------
  // Lane holds rows 4*(lane>>4)+r, column lane&15 of each 16x16 fragment.
  const int row0 = m0 + wr * T::WM + 4 * (lane >> 4);
  const int col0 = n0 + wc * T::WN + (lane & 15);
  const bool has_bias = p.bias != nullptr;
  float sa[T::FM][4], sb[T::FN], bv[T::FN];
  static_for<0, T::FM>([&](auto i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + i * 16 + r;
      sa[i][r] = (MODE != EPI_INT && row < p.M) ? p.a_scale[row] : 0.0f;
    }
  });
  static_for<0, T::FN>([&](auto j) {
    const int col = col0 + j * 16;
    const bool ok = MODE != EPI_INT && col < p.N;
    sb[j] = ok ? p.b_scale[p.b_scalar ? 0 : col] : 0.0f;
    bv[j] = (ok && has_bias) ? load_bias(p.bias, p.bias_dtype, col) : 0.0f;
  });

  constexpr int ES = out_size<OUT>();
  const bool full = m0 + BM <= p.M && n0 + BN <= p.N && ((static_cast<int64_t>(p.N) * ES) % 16) == 0 &&
                    (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
  if (full) {
    // Stage the rounded wave sub-tile in LDS (PF fragment rows per pass, own
    // region per wave), then write whole 16-byte row chunks.
    constexpr int ROWB = T::WN * ES + 16;                  // padded LDS row pitch
    constexpr int REGION = T::LDS_BYTES / 4;
    constexpr int PF = (T::FM * 16 * ROWB <= REGION) ? T::FM : T::FM / 2;
    static_assert(PF * 16 * ROWB <= REGION && T::FM % PF == 0, "epilogue staging does not fit");
    constexpr int CHUNKS = T::WN * ES / 16;                // 16-byte chunks per row
    char* region = smem + wave * REGION;
    const int lrow = 4 * (lane >> 4);
    const int lcol = (lane & 15) * ES;
    char* out = static_cast<char*>(p.out);
    wait_vm_barrier<0>();  // no copy into LDS in flight; every wave is done reading the ring
    static_for<0, T::FM / PF>([&](auto pass) {
      static_for<0, PF>([&](auto ii) {
        constexpr int i = decltype(pass)::value * PF + decltype(ii)::value;
        static_for<0, T::FN>([&](auto j) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t bits = epi_bits<OUT, MODE>(acc[i][j][r], sa[i][r], sb[j], bv[j], has_bias);
            char* dstp = region + (ii * 16 + lrow + r) * ROWB + j * 16 * ES + lcol;
            if constexpr (ES == 4) *reinterpret_cast<uint32_t*>(dstp) = bits;
            else *reinterpret_cast<uint16_t*>(dstp) = static_cast<uint16_t>(bits);
          }
        });
      });
      // LDS accesses of one wave complete in order; the reads below see the writes.
      constexpr int TOTAL = PF * 16 * CHUNKS;
      static_assert(TOTAL % 64 == 0, "whole chunk rounds per lane");
#pragma unroll
      for (int c0 = 0; c0 < TOTAL; c0 += 64) {
        const int c = c0 + lane;
        const int rr = c / CHUNKS, cc = c - rr * CHUNKS;
        const i32x4 v = *reinterpret_cast<const i32x4*>(region + rr * ROWB + cc * 16);
        const int64_t grow = m0 + wr * T::WM + decltype(pass)::value * PF * 16 + rr;
        const int64_t gcol = n0 + wc * T::WN;
        *reinterpret_cast<i32x4*>(out + (grow * p.N + gcol) * ES + cc * 16) = v;
      }
    });
  } else {
    static_for<0, T::FN>([&](auto j) {
      const int col = col0 + j * 16;
      if (col < p.N) {
        static_for<0, T::FM>([&](auto i) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = row0 + i * 16 + r;
            if (row < p.M)
              store_elem<OUT>(p.out, static_cast<int64_t>(row) * p.N + col,
                              epi_bits<OUT, MODE>(acc[i][j][r], sa[i][r], sb[j], bv[j], has_bias));
          }
        });
      }
    });
  }
}

template <int BM, int BN, int WPE, int OUT, int MODE>
hipError_t launch_tile(const I8GemmArgs& p, hipStream_t stream) {
  const int blocks = ceil_div(p.M, BM) * ceil_div(p.N, BN);
  hipLaunchKernelGGL((k_i8_gemm<BM, BN, WPE, OUT, MODE>), dim3(blocks), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int BM, int BN, int WPE, int OUT>
hipError_t launch_mode(const I8GemmArgs& p, hipStream_t stream) {
  // Orders F and E coincide for fp32 output (no intermediate rounding).
  if (p.epi & QG_EPI_GELU_TANH) return launch_tile<BM, BN, WPE, OUT, EPI_GELU>(p, stream);
  if (p.epi & QG_EPI_ORDER_FUSED_FMA) return launch_tile<BM, BN, WPE, OUT, EPI_FMA>(p, stream);
  if constexpr (OUT != QG_F32) {
    if (p.epi & QG_EPI_ORDER_EAGER) return launch_tile<BM, BN, WPE, OUT, EPI_EAGER>(p, stream);
  }
  return launch_tile<BM, BN, WPE, OUT, EPI_F>(p, stream);
}

template <int BM, int BN, int WPE>
hipError_t launch_variant(const I8GemmArgs& p, hipStream_t stream) {
  if (p.a_scale == nullptr) return launch_tile<BM, BN, WPE, QG_I32, EPI_INT>(p, stream);
  if (p.out_dtype == QG_F16) return launch_mode<BM, BN, WPE, QG_F16>(p, stream);
  if (p.out_dtype == QG_BF16) return launch_mode<BM, BN, WPE, QG_BF16>(p, stream);
  return launch_mode<BM, BN, WPE, QG_F32>(p, stream);
}

}  // namespace

hipError_t launch_i8_gemm(const I8GemmArgs& p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  // 256x192 tiles tile every BASELINE shape into whole multiples of the 256
  // CUs (4096x3072 -> 256 tiles, x9216 -> 768, x12288 -> 1024). Smaller
  // problems use 128x128 tiles so that more CUs get work.
  const long big = static_cast<long>(ceil_div(p.M, 256)) * ceil_div(p.N, 192);
  if (big >= 192) return launch_variant<256, 192, 1>(p, stream);
  return launch_variant<128, 128, 2>(p, stream);
}

}  // namespace qg
