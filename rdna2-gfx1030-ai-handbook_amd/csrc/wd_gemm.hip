// Tiled weight-decode GEMM for gfx950: out = A @ dequant(W)^T (+ bias), with
// A [M, K] fp16 / bf16 and W either INT4 groups (the W4 storage of
// include/qgemm.h) or OCP fp8 (e4m3fn / e5m2) with an optional per-channel
// scale. Serves the large-M shapes of int4_linear_a16
// (rdna2-ops/rdna2_ops/int4_weight_gemm_v07.py:540-564) and fp8_weight_gemm's
// fused path (rdna2-ops/rdna2_ops/fp8_weight_gemm_v06.py:49-73, :195-206).
//
// Design:
//  * one 512-thread workgroup (2 x 4 waves) per 128 x 128 output tile (FP8 on
//    large grids: 256 x 128); each wave owns 64 x 32 (128 x 32) as 4 x 2
//    (8 x 2) fragments of v_mfma_f32_16x16x32_{bf16,f16};
//  * K advances in 128-wide stages. The activation stage (128 rows x 256 B)
//    is copied HBM -> LDS with global_load_lds_dwordx4 into a 2-slot ring,
//    as two 128-byte-row halves with the 16-byte chunk index XOR-swizzled by
//    ((row >> 1) & 3) ^ 4 (row & 1). The fragment reads of a 16 x 16 x 32
//    step (rows 0-15 at one logical chunk per lane quarter, quarters 2 and 3
//    in the second half) measured 4 bank-conflict cycles per ds_read_b128
//    with an XOR by (row & 7) or by ((row >> 1) & 7) and none with this one;
//  * weights never touch LDS: each lane loads its column's words / bytes for
//    the next stage into registers while the current stage computes, and
//    expands them in registers right before the MFMA (nibble -> 128 + u or
//    256 + 4u with one v_perm + one v_and_or per register; fp8 -> bf16/fp16
//    with v_cvt_scalef32_pk_*_fp8 at scale 1, exact);
//  * W4: each group's MFMA sum is taken separately; total += s * (acc - zb *
//    rowsum) with the row sums from an MFMA against ones (fp32, exact
//    products). FP8: out = acc * scale[n] + bias[n] (fp32).
// One barrier per stage: at the top of stage s every wave waits for its own
// copies of stage s (LDS) and its weight registers (vmcnt(0)), then the
// workgroup barrier makes the whole stage visible and guarantees that the
// other slot is free; stage s+1 is issued right after and overlaps stage s's
// MFMAs. Two stages per loop iteration with the weight register sets swapped
// (no register copy, which would wait for the loads of stage s+1 at the end of
// stage s): 126 -> 117 us for cfg3 N = 3072, 577 -> 558 us for the cfg2
// prefill.
#include "qg_common.h"
#include "qg_internal.h"

namespace qg {

namespace {

constexpr int kKS = 128;  // K elements per stage

enum WdFormat { WD_W4_UINT4 = 0, WD_W4_GENERIC = 1, WD_FP8_E4M3 = 2, WD_FP8_E5M2 = 3 };

// 8 waves as 2 x 4, 64 x 32 outputs each: half the accumulators and weight
// registers of a 2 x 2 grid of 64 x 64 (two or three waves per SIMD instead
// of one for W4; measured 1.26x on the cfg2 prefill, 1.1x on cfg3 N 3072);
// 4 x 2 loads every weight column in four waves and is slower still.
constexpr int kWdWavesM = 2;


template <bool F16A>
__device__ __forceinline__ f32x4 mfma16(const i32x4& a, const i32x4& b, const f32x4& c) {
  if constexpr (F16A)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ T load_at(const void* base, uint32_t byte_off) {
  return *reinterpret_cast<const T*>(static_cast<const char*>(base) + byte_off);
}

// Word f (0..15) of a 128-wide stage feeds MFMA step j from lane group q; each
// step stays inside one W4 group (same rule as the decode kernels).
template <int G, bool KN>
__device__ __forceinline__ int word_of(int q, int j) {
  if constexpr (!KN && G == 128) return 4 * q + j;
  else if constexpr (!KN && G == 64) return 8 * (j >> 1) + 2 * q + (j & 1);
  else return 4 * j + q;
}

// Natural-order nibble expansion (register i = K elements 2i, 2i+1).
template <bool F16A>
__device__ __forceinline__ i32x4 unpack_nat(uint32_t w, const uint32_t (&sel)[4], uint32_t mask,
                                            uint32_t magic2) {
  const uint32_t lo = F16A ? w << 4 : w;
  const uint32_t hi = F16A ? w : w >> 4;
  i32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t t = __builtin_amdgcn_perm(hi, lo, sel[i]);
    r[i] = static_cast<int>((t & mask) | magic2);
  }
  return r;
}

__device__ __forceinline__ void nat_selectors(bool high, uint32_t (&sel)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t b0 = high ? (4u + 3u - i) : static_cast<uint32_t>(i);
    const uint32_t b2 = high ? (3u - i) : (4u + i);
    sel[i] = 0x0C000C00u | (b2 << 16) | b0;
  }
}

__device__ __forceinline__ float bias_at(const void* bias, int dtype, int col) {
  if (dtype == QG_F32) return static_cast<const float*>(bias)[col];
  const uint16_t b = static_cast<const uint16_t*>(bias)[col];
  return dtype == QG_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

__device__ __forceinline__ void put_out(void* out, int dtype, int64_t idx, float v) {
  if (dtype == QG_F32) static_cast<float*>(out)[idx] = v;
  else if (dtype == QG_F16) static_cast<uint16_t*>(out)[idx] = f32_to_f16(v);
  else static_cast<uint16_t*>(out)[idx] = f32_to_bf16(v);
}

// Weight registers of one stage for one wave: FN column tiles.
template <int FMT, int FN>
struct StageW {
  static constexpr int R = (FMT >= WD_FP8_E4M3) ? 8 : 4;  // 32-bit words per lane per tile
  uint32_t w[FN][R];
  uint32_t gs[FN][4], gz[FN][4];  // W4: raw scale / zero words per group slot
};

// TBM x TBN output tile, NWM x NWN waves: each wave owns 16 kFM rows x 16 kFN
// columns, kFM = TBM / 16 / NWM, kFN = TBN / 16 / NWN.
template <int FMT, int G, bool KN, bool F16A, int NWM, int NWN, int TBM, int TBN>
__global__ __launch_bounds__(64 * NWM * NWN, 1) void k_wd_gemm(WdArgs p) {
#pragma clang fp contract(off)
  constexpr int NW = NWM * NWN;
  constexpr int kFM = TBM / 16 / NWM, kFN = TBN / 16 / NWN;
  constexpr int kBM = TBM, kBN = TBN;
  constexpr int kHalf = kBM * 128;  // bytes of one 64-wide K half of an activation stage
  constexpr int kStage = 2 * kHalf;
  constexpr int kSegs = kBM / 4;    // 1 KB DMA segments (8 rows x 128 B) per stage
  static_assert(kFM >= 1 && kFN >= 1 && kSegs % NW == 0, "tile / wave grid");
  constexpr bool W4 = FMT <= WD_W4_GENERIC;
  constexpr bool UINT4 = FMT == WD_W4_UINT4;
  constexpr int SPS = W4 ? kKS / G : 1;         // W4 groups per stage
  constexpr int STEPS_PER_GROUP = 4 / SPS;
  constexpr float MAGIC = F16A ? 256.0f : 128.0f;
  constexpr float UNIT = F16A ? 4.0f : 1.0f;
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = wave / NWN, wc = wave % NWN;
  const int col = lane & 15, q = lane >> 4;

  // ---- tile order: XCD-contiguous ranges, GROUP_M-swizzled inside --------
  const int nbm = ceil_div(p.M, kBM), nbn = ceil_div(p.N, kBN);
  const int total_tiles = nbm * nbn;
  int bid = blockIdx.x;
  if ((total_tiles & 7) == 0) bid = (bid & 7) * (total_tiles >> 3) + (bid >> 3);
  constexpr int GROUP_M = 8;
  const int group = bid / (GROUP_M * nbn);
  const int first = group * GROUP_M;
  const int gm = min(nbm - first, GROUP_M);
  const int in_group = bid - group * GROUP_M * nbn;
  const int m0 = (first + in_group % gm) * kBM;
  const int n0 = (in_group / gm) * kBN;

  // ---- activation DMA plan: kSegs segments (8 rows x 128 B) per stage ------
  const int srow = lane >> 3;
  const uint32_t smem_base = lds_addr_of(smem);
  const char* a_base = reinterpret_cast<const char*>(p.a);
  const int S = p.K / kKS;
  const uint32_t a_stride = static_cast<uint32_t>(2 * p.a_sm);
  auto dma_stage = [&](int s) __attribute__((always_inline)) {
    const uint32_t slot = smem_base + (s & 1) * kStage;
    static_for<0, kSegs / NW>([&](auto i) {
      const int seg = wave + NW * i;
      const int h = seg / (kBM / 8), rb = seg % (kBM / 8);
      const int row = rb * 8 + srow;
      const uint32_t lc = static_cast<uint32_t>((lane & 7) ^ ((row >> 1) & 3) ^ (4 * (row & 1)));
      int rg = min(m0 + row, p.M - 1);
      asm volatile("" : "+v"(rg));
      // a 32-bit product (the compiler would otherwise fold it into a 64-bit
      // multiply-add and keep the per-segment constants in register pairs)
      uint32_t roff;
      asm("v_mul_lo_u32 %0, %1, %2" : "=v"(roff) : "v"(rg), "s"(a_stride));
      const uint32_t voff = roff + 128u * h + 16u * lc;
      dma16s(a_base + static_cast<int64_t>(s) * 256, voff, slot + h * kHalf + rb * 1024);
    });
  };

  // ---- weight loads of one stage ----------------------------------------
  int ncol[kFN];
  static_for<0, kFN>([&](auto t) { ncol[t] = min(n0 + wc * 16 * kFN + 16 * t + col, p.N - 1); });
  const int KW = p.K >> 3;
  auto load_w = [&](StageW<FMT, kFN>& sw, int s) __attribute__((always_inline)) {
    static_for<0, kFN>([&](auto t) {
      const uint32_t n = static_cast<uint32_t>(ncol[t]);
      if constexpr (!W4) {
        const uint32_t off = n * static_cast<uint32_t>(p.w8_sn) + 128u * s + 32u * q;
        const i32x4 v0 = load_at<i32x4>(p.w8, off);
        const i32x4 v1 = load_at<i32x4>(p.w8, off + 16);
        static_for<0, 4>([&](auto e) {
          sw.w[t][e] = static_cast<uint32_t>(v0[int(e)]);
          sw.w[t][4 + e] = static_cast<uint32_t>(v1[int(e)]);
        });
      } else {
        const int kw0 = 16 * s;
        auto woff = [&](int kw) __attribute__((always_inline)) -> uint32_t {
          return KN ? 4u * (static_cast<uint32_t>(kw) * p.N + n) : 4u * (n * KW + kw);
        };
        if constexpr (!KN && G == 128) {
          const i32x4 v = load_at<i32x4>(p.w4, woff(kw0 + 4 * q));
          static_for<0, 4>([&](auto j) { sw.w[t][j] = static_cast<uint32_t>(v[int(j)]); });
        } else if constexpr (!KN && G == 64) {
          const uint2 v0 = load_at<uint2>(p.w4, woff(kw0 + 2 * q));
          const uint2 v1 = load_at<uint2>(p.w4, woff(kw0 + 8 + 2 * q));
          sw.w[t][0] = v0.x;
          sw.w[t][1] = v0.y;
          sw.w[t][2] = v1.x;
          sw.w[t][3] = v1.y;
        } else {
          static_for<0, 4>([&](auto j) { sw.w[t][j] = load_at<uint32_t>(p.w4, woff(kw0 + word_of<G, KN>(q, j))); });
        }
        static_for<0, SPS>([&](auto g) {
          const uint32_t gi = n * p.ng + s * SPS + g;
          if constexpr (UINT4) {
            sw.gs[t][g] = load_at<uint32_t>(p.scales, 4u * (gi >> 1));
            sw.gz[t][g] = load_at<uint32_t>(p.zeros, 4u * (n * p.zw + ((s * SPS + g) >> 3)));
          } else {
            sw.gs[t][g] = load_at<uint32_t>(p.scales, p.scale_f32 ? 4u * gi : 4u * (gi >> 1));
            sw.gz[t][g] = (p.flags & QG_W4_ZEROS_PACKED)
                              ? load_at<uint32_t>(p.zeros, 4u * (n * p.zw + ((s * SPS + g) >> 3)))
                              : load_at<uint32_t>(p.zeros, 4u * gi);
          }
        });
      }
    });
  };

  // ---- fragment read offsets (rows of this wave, per fragment f) -----------
  // chunk f = word_of(q, j) of the stage: half f >> 3, logical 16-byte chunk f & 7
  uint32_t a_row_off[kFM];
  static_for<0, kFM>([&](auto f) {
    const int r = wr * 16 * kFM + 16 * f + col;
    a_row_off[f] = static_cast<uint32_t>(r * 128);
  });
  const int rsw = ((col >> 1) & 3) ^ (4 * (col & 1));  // swizzle of every row this lane reads

  uint32_t sel[4], umask = F16A ? 0x00F000F0u : 0x000F000Fu, umagic = F16A ? 0x5C005C00u : 0x43004300u;
  nat_selectors(W4 && !UINT4 && (p.flags & QG_W4_ORDER_HIGH), sel);
  asm volatile("" : "+v"(umask), "+v"(umagic));
  const uint32_t wxor = (W4 && !UINT4 && (p.flags & QG_W4_SIGNED_NIBBLES)) ? 0x88888888u : 0u;
  const uint32_t ones2 = F16A ? 0x3C003C00u : 0x3F803F80u;
  const i32x4 ones = {static_cast<int>(ones2), static_cast<int>(ones2), static_cast<int>(ones2),
                      static_cast<int>(ones2)};

  f32x4 acc[kFM][kFN];
  f32x4 tot[W4 ? kFM : 1][W4 ? kFN : 1];
  f32x4 asum[kFM];
  static_for<0, kFM>([&](auto f) {
    static_for<0, kFN>([&](auto t) { acc[f][t] = f32x4{0, 0, 0, 0}; });
  });
  if constexpr (W4) {
    static_for<0, kFM>([&](auto f) {
      static_for<0, kFN>([&](auto t) { tot[f][t] = f32x4{0, 0, 0, 0}; });
    });
  }

  // Stage s computes from `cur` and loads stage s + 1 into `nxt`; the loop
  // runs two stages per iteration with the register sets swapped, so no
  // weight registers are copied (a copy would wait for the loads just issued).
  auto stage = [&](int s, StageW<FMT, kFN>& cur, StageW<FMT, kFN>& nxt) __attribute__((always_inline)) {
    wait_vm_barrier<0>();  // stage s landed everywhere; slot (s+1)&1 is free
    if (s + 1 < S) {
      dma_stage(s + 1);
      load_w(nxt, s + 1);
    }
    const char* const sbuf = smem + (s & 1) * kStage;
    static_for<0, 4>([&](auto j) {
      if constexpr (W4 && j % STEPS_PER_GROUP == 0) {
        static_for<0, kFM>([&](auto f) {
          asum[f] = f32x4{0, 0, 0, 0};
          static_for<0, kFN>([&](auto t) { acc[f][t] = f32x4{0, 0, 0, 0}; });
        });
      }
      // activation fragments of step j
      const int fw = W4 ? word_of<G, KN>(q, j) : 4 * q + j;
      const uint32_t chunk_off = static_cast<uint32_t>((fw >> 3) * kHalf + (((fw & 7) ^ rsw) << 4));
      i32x4 af[kFM];
      static_for<0, kFM>([&](auto f) {
        af[f] = *reinterpret_cast<const i32x4*>(sbuf + a_row_off[f] + chunk_off);
      });
      if constexpr (W4) static_for<0, kFM>([&](auto f) { asum[f] = mfma16<F16A>(af[f], ones, asum[f]); });
      static_for<0, kFN>([&](auto t) {
        i32x4 b;
        if constexpr (W4) b = unpack_nat<F16A>(cur.w[t][j] ^ wxor, sel, umask, umagic);
        else b = fp8x8<F16A, FMT == WD_FP8_E5M2>(cur.w[t][2 * j], cur.w[t][2 * j + 1]);
        static_for<0, kFM>([&](auto f) { acc[f][t] = mfma16<F16A>(af[f], b, acc[f][t]); });
      });
      if constexpr (W4 && j % STEPS_PER_GROUP == STEPS_PER_GROUP - 1) {
        constexpr int gi = j / STEPS_PER_GROUP;
        static_for<0, kFN>([&](auto t) {
          const int g = s * SPS + gi;
          const uint32_t i = static_cast<uint32_t>(ncol[t]) * p.ng + g;
          float sc, zb;
          const uint32_t rs = cur.gs[t][gi], rz = cur.gz[t][gi];
          if constexpr (UINT4) {
            sc = __uint_as_float((i & 1u) ? (rs & 0xFFFF0000u) : (rs << 16));
            zb = MAGIC + UNIT * static_cast<float>((rz >> ((g & 7) * 4)) & 15u);
          } else {
            sc = p.scale_f32 ? __uint_as_float(rs) : __uint_as_float((i & 1u) ? (rs & 0xFFFF0000u) : (rs << 16));
            const bool packed = p.flags & QG_W4_ZEROS_PACKED;
            const int z = packed ? static_cast<int>((rz >> ((g & 7) * 4)) & 15u) : static_cast<int>(rz);
            const int zu = (p.flags & QG_W4_SIGNED_NIBBLES) ? (packed ? (z ^ 8) : z + 8) : z;
            zb = MAGIC + UNIT * static_cast<float>(zu);
          }
          sc = sc / UNIT;
          static_for<0, kFM>([&](auto f) {
            static_for<0, 4>([&](auto e) {
              const float v = __builtin_fmaf(-zb, asum[f][int(e)], acc[f][t][int(e)]);
              tot[f][t][int(e)] = __builtin_fmaf(sc, v, tot[f][t][int(e)]);
            });
          });
        });
      }
    });
  };
  StageW<FMT, kFN> w0, w1;
  if (S > 0) {
    dma_stage(0);
    load_w(w0, 0);
  }
  for (int s = 0; s < S; s += 2) {
    stage(s, w0, w1);
    if (s + 1 < S) stage(s + 1, w1, w0);
  }

  // ---- epilogue -------------------------------------------------------------
  static_for<0, kFN>([&](auto t) {
    const int nn = n0 + wc * 16 * kFN + 16 * t + col;
    if (nn < p.N) {
      const float bv = p.bias ? bias_at(p.bias, p.bias_dtype, nn) : 0.0f;
      const float ws = (!W4 && p.w_scale) ? p.w_scale[nn] : 1.0f;
      static_for<0, kFM>([&](auto f) {
        static_for<0, 4>([&](auto e) {
          const int row = m0 + wr * 16 * kFM + 16 * f + 4 * q + e;
          if (row < p.M) {
            float v;
            if constexpr (W4) v = tot[f][t][int(e)];
            else {
              v = acc[f][t][int(e)];
              if (p.w_scale) v = v * ws;
            }
            if (p.bias) v = v + bv;
            put_out(p.out, p.out_dtype, static_cast<int64_t>(row) * p.N + nn, v);
          }
        });
      });
    }
  });
}

template <int FMT, int G, bool KN, int TBM, int TBN>
hipError_t launch_wd_tile(const WdArgs& p, hipStream_t stream) {
  const int tiles = ceil_div(p.M, TBM) * ceil_div(p.N, TBN);
  constexpr int NWM = kWdWavesM, NWN = 8 / kWdWavesM;
  if (p.a_f16)
    hipLaunchKernelGGL((k_wd_gemm<FMT, G, KN, true, NWM, NWN, TBM, TBN>), dim3(tiles), dim3(64 * NWM * NWN), 0,
                       stream, p);
  else
    hipLaunchKernelGGL((k_wd_gemm<FMT, G, KN, false, NWM, NWN, TBM, TBN>), dim3(tiles), dim3(64 * NWM * NWN), 0,
                       stream, p);
  return hipGetLastError();
}

// Columns of the W4 tiled kernel's 128-row tile for an M x N output and group G.
int wd_w4_tile_n(int M, int N, int G) {
  if (G == 32) return 64;
  const long tiles = static_cast<long>(ceil_div(M, 128)) * ceil_div(N, 128);
  return tiles < (G == 64 ? 192 : 256) ? 64 : 128;
}

// W4 tile width: 128 x 64 tiles where 128 x 128 tiles would leave CUs idle
// (M = 512, N = 4096: 78.5 -> 52.7 us at group 128, 116 -> 69 us at group 64;
// M = 1061, N = 3072, 216 tiles: 62.8 -> 58.8 us at group 128, while group 64
// keeps 128 columns there, 90 against 102 us), and always for group 32, whose
// 128 x 128 form needs 319 VGPRs (63 spilled: 289 -> 171 us at M = 1061).
template <int FMT, int G, bool KN>
hipError_t launch_wd_t(const WdArgs& p, hipStream_t stream) {
  if constexpr (G == 32) {
    return launch_wd_tile<FMT, G, KN, 128, 64>(p, stream);
  } else {
    if (wd_w4_tile_n(p.M, p.N, G) == 64) return launch_wd_tile<FMT, G, KN, 128, 64>(p, stream);
    return launch_wd_tile<FMT, G, KN, 128, 128>(p, stream);
  }
}

// dst[r, k] = src[r * s_r + k * s_k] (16-bit) for k < K, 0 for K <= k < k_pad.
__global__ void k_pack_rows_u16(const uint16_t* src, int64_t s_r, int64_t s_k, int64_t rows, int64_t K,
                                uint16_t* dst, int64_t k_pad) {
  const int64_t total = rows * k_pad;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / k_pad, k = i % k_pad;
    dst[i] = k < K ? src[r * s_r + k * s_k] : static_cast<uint16_t>(0);
  }
}

// out[n, k] = decode(w[n * w_sn + k * w_sk]) in out_dtype: every finite OCP
// fp8 value is exact in fp16, fp32 and bf16 (bit construction of fp8_to_f32).
__global__ void k_fp8_decode(const uint8_t* w, int64_t w_sn, int64_t w_sk, int64_t n, int64_t K, int e5,
                             void* out, int out_dtype) {
  const int64_t total = n * K;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / K, k = i % K;
    put_out(out, out_dtype, i, fp8_to_f32(w[r * w_sn + k * w_sk], e5 != 0));
  }
}

// The same for unit K stride, 16-byte aligned rows and output: one thread per
// 16 bytes (one 16-byte load, 16 outputs in 2- or 4-byte vector stores).
template <int OUT>
__global__ __launch_bounds__(256) void k_fp8_decode16(const uint8_t* w, int64_t w_sn, int n, int K, int e5,
                                                      void* out) {
  const int cpr = K >> 4;  // 16-byte chunks per row (< 2^27)
  const int chunks = n * cpr;
  for (int ci = blockIdx.x * blockDim.x + threadIdx.x; ci < chunks; ci += gridDim.x * blockDim.x) {
    const int r = ci / cpr, c = ci - r * cpr;
    const uint4 v = *reinterpret_cast<const uint4*>(w + static_cast<int64_t>(r) * w_sn + 16 * c);
    const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
    const int64_t o0 = static_cast<int64_t>(r) * K + 16 * c;
    if constexpr (OUT == QG_F32) {
      float* o = static_cast<float*>(out) + o0;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        reinterpret_cast<float4*>(o)[q] =
            make_float4(fp8_to_f32(wd[q] & 0xffu, e5), fp8_to_f32((wd[q] >> 8) & 0xffu, e5),
                        fp8_to_f32((wd[q] >> 16) & 0xffu, e5), fp8_to_f32(wd[q] >> 24, e5));
    } else {
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const float a = fp8_to_f32((wd[e >> 2] >> (8 * (e & 3))) & 0xffu, e5);
        const float b = fp8_to_f32((wd[e >> 2] >> (8 * ((e + 1) & 3))) & 0xffu, e5);
        const uint32_t ha = OUT == QG_F16 ? f32_to_f16(a) : f32_to_bf16(a);
        const uint32_t hb = OUT == QG_F16 ? f32_to_f16(b) : f32_to_bf16(b);
        h[e >> 1] = ha | (hb << 16);
      }
      uint4* o = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + o0);
      o[0] = make_uint4(h[0], h[1], h[2], h[3]);
      o[1] = make_uint4(h[4], h[5], h[6], h[7]);
    }
  }
}

unsigned grid_for(int64_t total) {
  const int64_t blocks = ceil_div<int64_t>(total, 256);
  return static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
}

}  // namespace

hipError_t launch_pack_rows_u16(const uint16_t* src, int64_t s_r, int64_t s_k, int64_t rows, int64_t K,
                                uint16_t* dst, int64_t k_pad, hipStream_t stream) {
  if (rows * k_pad == 0) return hipSuccess;
  hipLaunchKernelGGL(k_pack_rows_u16, dim3(grid_for(rows * k_pad)), dim3(256), 0, stream, src, s_r, s_k, rows,
                     K, dst, k_pad);
  return hipGetLastError();
}

hipError_t launch_fp8_decode(const uint8_t* w, int64_t w_sn, int64_t w_sk, int64_t n, int64_t K, int e5,
                             void* out, int out_dtype, hipStream_t stream) {
  if (n * K == 0) return hipSuccess;
  const bool vec = w_sk == 1 && K % 16 == 0 && w_sn % 16 == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0 && n * K < (int64_t(1) << 31);
  if (vec) {
    const int64_t chunks = n * K / 16;
    const unsigned grid = static_cast<unsigned>(chunks / 256 + 1 < 65536 ? chunks / 256 + 1 : 65536);
    const int ni = static_cast<int>(n), ki = static_cast<int>(K);
    if (out_dtype == QG_F32)
      hipLaunchKernelGGL(k_fp8_decode16<QG_F32>, dim3(grid), dim3(256), 0, stream, w, w_sn, ni, ki, e5, out);
    else if (out_dtype == QG_F16)
      hipLaunchKernelGGL(k_fp8_decode16<QG_F16>, dim3(grid), dim3(256), 0, stream, w, w_sn, ni, ki, e5, out);
    else
      hipLaunchKernelGGL(k_fp8_decode16<QG_BF16>, dim3(grid), dim3(256), 0, stream, w, w_sn, ni, ki, e5, out);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_fp8_decode, dim3(grid_for(n * K)), dim3(256), 0, stream, w, w_sn, w_sk, n, K, e5, out,
                     out_dtype);
  return hipGetLastError();
}

// FP8: 256 x 128 tiles (wave tile 128 x 32; 1.3x fewer bytes per MFMA than
// 128 x 128, one workgroup per CU for its 128 KB of activation ring) once the
// grid has at least four of them per CU: 397 us against 474 us for cfg3's
// N = 12288, while N = 3072 (1.5 such tiles per CU) stays faster at 128 x 128
// (117 us against 131 us). 256 x 256 spills and W4 does not fit either.
hipError_t launch_wd_fp8(const WdArgs& p, hipStream_t stream) {
  const int64_t wide_tiles = static_cast<int64_t>(ceil_div(p.M, 256)) * ceil_div(p.N, 128);
  if (p.M >= 256 && wide_tiles >= 4 * 256)
    return p.fp8_e5 ? launch_wd_tile<WD_FP8_E5M2, 128, false, 256, 128>(p, stream)
                    : launch_wd_tile<WD_FP8_E4M3, 128, false, 256, 128>(p, stream);
  return p.fp8_e5 ? launch_wd_tile<WD_FP8_E5M2, 128, false, 128, 128>(p, stream)
                  : launch_wd_tile<WD_FP8_E4M3, 128, false, 128, 128>(p, stream);
}

hipError_t launch_wd_w4(const WdArgs& p, hipStream_t stream) {
  const bool kn = p.flags & QG_W4_LAYOUT_KN;
  const bool uint4 = !p.scale_f32 && p.flags == QG_W4_ZEROS_PACKED;
  switch (p.group) {
    case 128:
      if (uint4 && !kn) return launch_wd_t<WD_W4_UINT4, 128, false>(p, stream);
      return kn ? launch_wd_t<WD_W4_GENERIC, 128, true>(p, stream) : launch_wd_t<WD_W4_GENERIC, 128, false>(p, stream);
    case 64:
      return kn ? launch_wd_t<WD_W4_GENERIC, 64, true>(p, stream) : launch_wd_t<WD_W4_GENERIC, 64, false>(p, stream);
    default:
      return kn ? launch_wd_t<WD_W4_GENERIC, 32, true>(p, stream) : launch_wd_t<WD_W4_GENERIC, 32, false>(p, stream);
  }
}

}  // namespace qg
