// W4A8 GEMM on gfx950 int8 MFMA: int4_linear_a8 of
// rdna2-ops/rdna2_ops/int4_weight_gemm_v07.py:476-537. Every method of the
// reference computes the same numbers (_linear_dot4 :181-217,
// _linear_dot4_split :220-256, _linear_dot4_words :288-322, _linear_dot8
// :325-353); they differ only in how the integer group sums are formed:
//
//   integer: out[m, n] = sum_g sum_{k in g} a[m, k] (q[n, k] - z[n, g])   int32
//   float:   total = 0; for g ascending: total = total + f32(acc_g) * s[n, g]
//            (two fp32 roundings, no FMA: enable_fp_fusion=False)
//            out = total * sa[m]; out = out + f32(bias[n])                  fp32
//
// acc_g is exact (|acc_g| <= 128 * 15 * 128 < 2^24, so f32(acc_g) is exact too).
//
// Design (not a translation of the reference's dot4 / dot8 Triton tiles):
//  * one 128 x 128 output tile per workgroup of 4 waves; wave w owns output
//    columns 32 w .. 32 w + 31 for all 128 rows: four 32x32 int32 blocks of
//    v_mfma_i32_32x32x32_i8 with the weight fragment as the first operand, so
//    a lane holds row 32 i + (l & 31) and 4 adjacent columns per register
//    quad (columns 8 (r >> 2) + 4 (l >> 5) + (r & 3));
//  * A stages (128 rows x 128 K bytes) are copied HBM -> LDS with
//    global_load_lds_dwordx4 into a 2-slot ring in the INT8 GEMM's layout
//    (128-byte rows, 16-byte chunks XOR-swizzled by (row >> 1) & 7); each lane
//    loads the packed words of its own weight row for the next stage into
//    registers (no weight byte is shared between waves), and its zero points;
//  * a word of 8 nibbles becomes two dwords of signed bytes q - z without any
//    borrow between bytes: with u, zu the unsigned nibble and zero point,
//    ((u | 0x80) - zu) ^ 0x80 per byte (128 + u - zu never goes below 113, and
//    flipping bit 7 turns the excess-128 value into two's complement), then
//    two v_perm_b32 interleave the even and odd nibbles back into K order.
//    The MFMA sums a (q - z) exactly, against the A fragment as it lies in LDS;
//  * when a group ends its exact int32 sum is folded into the fp32 total in
//    the reference's order (the stage's scales are staged in LDS as
//    [group][column] and read as 4-column vectors) or into an int32 total;
//  * prepared centred int8 weights (method dot4_prepared) are loaded as 16
//    bytes per lane and k-step and need no expansion.
#include "qg_common.h"
#include "qg_internal.h"

namespace qg {

namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 128;
constexpr int kStage = 128;                       // K bytes per stage
constexpr int kSlotA = kBM * kStage;              // 16 KB per A slot

// NW waves own 32 output columns each: a 128 x 32 NW tile, one A stage in LDS
// shared by all of them.
template <int NW>
struct W8Geo {
  static constexpr int BN = 32 * NW, THREADS = 64 * NW;
  static constexpr int SLOT_S = 4 * BN * 4;       // <= 4 groups x BN fp32 scales
  static constexpr int LDS = 2 * kSlotA + 2 * SLOT_S;
  static_assert(16 % NW == 0, "A copies split evenly over the waves");
};

// Output tile of this workgroup (same XCD-aware, GROUP_M-ordered walk as the
// INT8 GEMM).
template <int kBN>
__device__ __forceinline__ void w4a8_tile(int M, int N, int& m0, int& n0) {
  const int nbm = ceil_div(M, kBM), nbn = ceil_div(N, kBN);
  const int total = nbm * nbn;
  int bid = blockIdx.x;
  if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  constexpr int GROUP_M = 4;
  const int group = bid / (GROUP_M * nbn);
  const int first = group * GROUP_M;
  const int gm = min(nbm - first, GROUP_M);
  const int in_group = bid - group * GROUP_M * nbn;
  m0 = (first + in_group % gm) * kBM;
  n0 = (in_group / gm) * kBN;
}

// Fragment offset in an A slot: k-step t, lane l reads row (l & 31) of a
// 32-row block, logical chunk 2t + (l >> 5), stored at chunk ^ ((l >> 1) & 7).
__device__ __forceinline__ int a_frag_offset(int t, int lane) {
  return (lane & 31) * kStage + (((2 * t + (lane >> 5)) ^ ((lane >> 1) & 7)) << 4);
}

// Weight registers of one stage: 4 k-steps of a lane's 16 K bytes (2 packed
// words, or 16 prepared bytes), and the stage's per-group zero points as
// loaded (the packed word or the int32), decoded only where the stage
// computes so that no wait for these loads is needed before then.
template <bool PREP>
struct WStage {
  uint32_t w[4][PREP ? 4 : 2];
  uint32_t zraw[4];
};
template <bool PREP>
__device__ __forceinline__ void settle_stage(WStage<PREP>& b) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int e = 0; e < (PREP ? 4 : 2); ++e) asm volatile("" : "+v"(b.w[t][e]));
    if constexpr (!PREP) asm volatile("" : "+v"(b.zraw[t]));
  }
}

template <int G, bool PREP, bool INTEGER, int NW, bool VEC, bool FULLK>
__global__ __launch_bounds__(64 * NW, NW == 4 ? 2 : 1) void k_w4a8(W4A8Args p) {
#pragma clang fp contract(off)
  constexpr int GK = G / 32;      // k-steps per group
  constexpr int GS = kStage / G;  // groups per stage
  constexpr int kBN = W8Geo<NW>::BN;
  constexpr int kSlotS = W8Geo<NW>::SLOT_S;
  constexpr int NA = 16 / NW;     // A copies (1 KB each) per wave and stage
  __shared__ __attribute__((aligned(1024))) char smem[W8Geo<NW>::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, lr = lane & 31;
  int m0, n0;
  w4a8_tile<kBN>(p.M, p.N, m0, n0);
  const int KT = p.K / 32;                 // k-steps
  const int S = ceil_div(p.K, kStage);     // stages
  const uint32_t smem_base = lds_addr_of(smem);

  // ---- A copies: copy I of this wave covers tile rows 8 (wave + NW I) .. + 7;
  // lane l fetches logical chunk (l & 7) ^ ((row >> 1) & 7) of its row, rows
  // clamped into A, and in a last partial stage chunks past K fetch chunk 0
  // (their LDS bytes are never read).
  const uint32_t chunk = static_cast<uint32_t>(((lane & 7) ^ (4 * (wave & 1) + (lane >> 4))) << 4);
  const uint32_t klast = static_cast<uint32_t>(p.K - (S - 1) * kStage);
  uint32_t aoff[NA];
  for (int i = 0; i < NA; ++i)
    aoff[i] = static_cast<uint32_t>(min(m0 + wave * 8 + (lane >> 3) + 8 * NW * i, p.M - 1)) *
              static_cast<uint32_t>(p.a_sm);
  const char* a_base = reinterpret_cast<const char*>(p.a);
  auto copy_a = [&](int s, int slot) __attribute__((always_inline)) {
    const uint32_t ch = (!FULLK && s == S - 1 && chunk >= klast) ? 0u : chunk;
#pragma unroll
    for (int i = 0; i < NA; ++i)
      dma16s(a_base + static_cast<int64_t>(s) * kStage, aoff[i] + ch,
             smem_base + slot * kSlotA + (wave + NW * i) * 1024);
  };

  // ---- this lane's weight row (output column n0 + 32 wave + (l & 31))
  const int nw = min(n0 + 32 * wave + lr, p.N - 1);
  const bool kn = p.flags & QG_W4_LAYOUT_KN;
  const bool sgn = p.flags & QG_W4_SIGNED_NIBBLES;
  const bool zpk = p.flags & QG_W4_ZEROS_PACKED;
  const bool high = p.flags & QG_W4_ORDER_HIGH;
  // packed word (K index 8 j .. 8 j + 7) of this row: base + j * kstride
  const uint32_t* wrow = p.w + (kn ? static_cast<int64_t>(nw) : static_cast<int64_t>(nw) * (p.K / 8));
  const int64_t kstride = kn ? p.N : 1;
  const uint32_t xmask = sgn ? 0x88888888u : 0u;  // signed nibble q & 15 -> q + 8
  // K order from the even-nibble bytes (lo) and odd-nibble bytes (hi):
  // low order lo = (k0 k2 k4 k6), hi = (k1 k3 k5 k7); high order lo =
  // (k7 k5 k3 k1), hi = (k6 k4 k2 k0); v_perm_b32(hi, lo, sel) picks bytes
  // 0-3 of lo and 4-7 of hi
  const uint32_t sel0 = high ? 0x02060307u : 0x05010400u;  // k0 k1 k2 k3
  const uint32_t sel1 = high ? 0x00040105u : 0x07030602u;  // k4 k5 k6 k7

  auto load_w = [&](int s, WStage<PREP>& b) __attribute__((always_inline)) {
    static_for<0, 4>([&](auto t_c) {
      constexpr int t = decltype(t_c)::value;
      const int kt = min(s * 4 + t, KT - 1);  // k-steps past K load valid, unused data
      if constexpr (PREP) {
        const i32x4 v = *reinterpret_cast<const i32x4*>(p.w8 + static_cast<int64_t>(nw) * p.w8_sn + kt * 32 + 16 * h);
        static_for<0, 4>([&](auto e) { b.w[t][e] = static_cast<uint32_t>(v[decltype(e)::value]); });
      } else if constexpr (!VEC) {
        const int64_t j = 4 * kt + 2 * h;
        b.w[t][0] = wrow[j * kstride];
        b.w[t][1] = wrow[(j + 1) * kstride];
      } else if constexpr (t < 2) {
        // nk rows, 16-byte aligned: two 16-byte loads per lane and stage (words
        // 16 s + 4 h + 8 t .. + 3 of the lane's row, clamped into the row: a
        // clamped load only feeds k-steps past K), regrouped in compute()
        const int o = min(16 * s + 4 * h + 8 * t, p.K / 8 - 4);
        const i32x4 v = *reinterpret_cast<const i32x4*>(wrow + o);
        b.w[2 * t][0] = static_cast<uint32_t>(v[0]);
        b.w[2 * t][1] = static_cast<uint32_t>(v[1]);
        b.w[2 * t + 1][0] = static_cast<uint32_t>(v[2]);
        b.w[2 * t + 1][1] = static_cast<uint32_t>(v[3]);
      }
    });
    if constexpr (!PREP) {
      static_for<0, GS>([&](auto gi_c) {
        constexpr int gi = decltype(gi_c)::value;
        const int g = min(s * GS + gi, p.ng - 1);
        b.zraw[gi] = zpk ? static_cast<const uint32_t*>(p.zeros)[static_cast<int64_t>(nw) * p.zw + (g >> 3)]
                         : static_cast<uint32_t>(static_cast<const int32_t*>(p.zeros)[static_cast<int64_t>(nw) * p.ng + g]);
      });
    }
  };
  // Group gi of stage s: the unsigned zero point of this lane's row replicated
  // into the 4 bytes of a dword.
  auto zero_bytes = [&](int s, int gi, uint32_t zraw) __attribute__((always_inline)) {
    const int g = min(s * GS + gi, p.ng - 1);
    int zu;
    if (zpk) {
      const int z = static_cast<int>((zraw >> (4 * (g & 7))) & 15u);
      zu = sgn ? (z ^ 8) : z;
    } else {
      const int z = static_cast<int>(zraw);
      zu = sgn ? z + 8 : z;
    }
    return static_cast<uint32_t>(zu) * 0x01010101u;
  };

  // ---- scales of a stage: thread t covers column t % BN and the stage's
  // groups t / BN and t / BN + 2 (clamped; only valid ones are stored)
  const int scol = tid & (kBN - 1), sg0 = tid / kBN;
  const int scn = min(n0 + scol, p.N - 1);
  // (the raw bits are kept until parked: a bf16 value is widened there, so
  // nothing waits for these loads before the stage's MFMAs)
  auto load_scales = [&](int s, uint32_t (&sc)[2]) __attribute__((always_inline)) {
    if constexpr (!INTEGER) {
      static_for<0, 2>([&](auto j_c) {
        constexpr int j = decltype(j_c)::value;
        const int gi = min(sg0 + 2 * j, GS - 1);
        const int g = min(s * GS + gi, p.ng - 1);
        const int64_t i = static_cast<int64_t>(scn) * p.ng + g;
        sc[j] = p.scale_f32 ? static_cast<const uint32_t*>(p.scales)[i]
                            : static_cast<uint32_t>(static_cast<const uint16_t*>(p.scales)[i]);
      });
    }
  };
  auto park_scales = [&](int slot, const uint32_t (&sc)[2]) __attribute__((always_inline)) {
    if constexpr (!INTEGER) {
      float* dst = reinterpret_cast<float*>(smem + 2 * kSlotA + slot * kSlotS);
      static_for<0, 2>([&](auto j_c) {
        constexpr int j = decltype(j_c)::value;
        const int gi = sg0 + 2 * j;
        if (gi < GS) dst[gi * kBN + scol] = p.scale_f32 ? __uint_as_float(sc[j]) : bf16_to_f32(static_cast<uint16_t>(sc[j]));
      });
    }
  };

  i32x16 acc[4];
  float tot[4][16];
  int itot[4][16];
  static_for<0, 4>([&](auto i) {
    static_for<0, 16>([&](auto r) {
      tot[i][r] = 0.0f;
      itot[i][r] = 0;
    });
  });

  // Fold the finished group gi of the stage in slot `slot` into the totals.
  auto flush = [&](int slot, int gi) __attribute__((always_inline)) {
    const float* scl = reinterpret_cast<const float*>(smem + 2 * kSlotA + slot * kSlotS) + gi * kBN;
    f32x4 s4q[4];
    static_for<0, 4>([&](auto q) {
      s4q[q] = f32x4{0, 0, 0, 0};
      if constexpr (!INTEGER) s4q[q] = *reinterpret_cast<const f32x4*>(scl + 32 * wave + 8 * q + 4 * h);
    });
    static_for<0, 4>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      static_for<0, 4>([&](auto q_c) {
        constexpr int q = decltype(q_c)::value;
        const f32x4 s4 = s4q[q];
        static_for<0, 4>([&](auto c_c) {
          constexpr int c = decltype(c_c)::value;
          const int v = acc[i][4 * q + c];
          if constexpr (INTEGER) itot[i][4 * q + c] += v;
          else tot[i][4 * q + c] = tot[i][4 * q + c] + static_cast<float>(v) * s4[c];
          // Pin the fold here: otherwise instruction selection may defer it
          // past the next group's MFMAs, keeping every group's sums live.
          if constexpr (FULLK) {
            if constexpr (INTEGER) asm volatile("" : "+v"(itot[i][4 * q + c]));
            else asm volatile("" : "+v"(tot[i][4 * q + c]));
          }
        });
      });
    });
  };

  // MFMAs of stage s (A in slot s & 1, weights in b).
  auto compute = [&](int s, const WStage<PREP>& b_in) __attribute__((always_inline)) {
    const int slot = s & 1;
    const char* abase = smem + slot * kSlotA;
    // VEC: lane half h loaded words 4 h .. 4 h + 3 and 8 + 4 h .. 11 + 4 h of
    // the stage (b_in.w[0..3] = those 8 words in order); k-step t needs words
    // 4 t + 2 h, + 1. Each half keeps the pairs it holds and swaps the other
    // two with the lane 32 away.
    WStage<PREP> b = b_in;
    uint32_t zbs[GS];
    if constexpr (!PREP) static_for<0, GS>([&](auto gi) { zbs[gi] = zero_bytes(s, gi, b_in.zraw[gi]); });
    if constexpr (VEC) {
      const uint32_t* r = &b_in.w[0][0];  // r[0..3] = first load, r[4..7] = second
      uint32_t snd[4], got[4];
      snd[0] = h ? r[0] : r[2];
      snd[1] = h ? r[1] : r[3];
      snd[2] = h ? r[4] : r[6];
      snd[3] = h ? r[5] : r[7];
      static_for<0, 4>([&](auto i) { got[i] = static_cast<uint32_t>(__shfl_xor(static_cast<int>(snd[i]), 32, 64)); });
      b.w[0][0] = h ? got[0] : r[0];
      b.w[0][1] = h ? got[1] : r[1];
      b.w[1][0] = h ? r[2] : got[0];
      b.w[1][1] = h ? r[3] : got[1];
      b.w[2][0] = h ? got[2] : r[4];
      b.w[2][1] = h ? got[3] : r[5];
      b.w[3][0] = h ? r[6] : got[2];
      b.w[3][1] = h ? r[7] : got[3];
    }
    auto read_a = [&](auto t_c, i32x4 (&af)[4]) __attribute__((always_inline)) {
      constexpr int t = decltype(t_c)::value;
      static_for<0, 4>([&](auto i_c) {
        constexpr int i = decltype(i_c)::value;
        af[i] = *reinterpret_cast<const i32x4*>(abase + i * 32 * kStage + a_frag_offset(t, lane));
      });
    };
    // k-step t's weight fragment: 16 bytes of q - z (or the prepared bytes)
    auto weight_frag = [&](auto t_c) __attribute__((always_inline)) {
      constexpr int t = decltype(t_c)::value;
      if constexpr (PREP) {
        return i32x4{static_cast<int>(b.w[t][0]), static_cast<int>(b.w[t][1]), static_cast<int>(b.w[t][2]),
                     static_cast<int>(b.w[t][3])};
      } else {
        const uint32_t zb = zbs[t / GK];
        auto expand = [&](uint32_t word, uint32_t& d0, uint32_t& d1) __attribute__((always_inline)) {
          const uint32_t x = word ^ xmask;
          const uint32_t lo = (((x & 0x0F0F0F0Fu) | 0x80808080u) - zb) ^ 0x80808080u;
          const uint32_t hi = ((((x >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - zb) ^ 0x80808080u;
          d0 = __builtin_amdgcn_perm(hi, lo, sel0);
          d1 = __builtin_amdgcn_perm(hi, lo, sel1);
        };
        uint32_t d[4];
        expand(b.w[t][0], d[0], d[1]);
        expand(b.w[t][1], d[2], d[3]);
        return i32x4{static_cast<int>(d[0]), static_cast<int>(d[1]), static_cast<int>(d[2]), static_cast<int>(d[3])};
      }
    };
    auto mfmas = [&](auto t_c, const i32x4& wf, const i32x4 (&af)[4]) __attribute__((always_inline)) {
      constexpr int t = decltype(t_c)::value;
      static_for<0, 4>([&](auto i_c) {
        constexpr int i = decltype(i_c)::value;
        if constexpr (t % GK == 0) acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf, af[i], i32x16{}, 0, 0, 0);
        else acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf, af[i], acc[i], 0, 0, 0);
      });
    };
    if constexpr (FULLK) {
      // Four k-steps, software-pipelined by hand: k-step t + 1's A fragments
      // are read and its weight fragment expanded while k-step t's MFMAs run,
      // and nothing moves across k-steps (the compiler would otherwise hoist
      // every read of the stage and run out of registers).
      i32x4 af[2][4];
      read_a(std::integral_constant<int, 0>{}, af[0]);
      i32x4 wf = weight_frag(std::integral_constant<int, 0>{});
      static_for<0, 4>([&](auto t_c) {
        constexpr int t = decltype(t_c)::value;
        i32x4 wn = wf;
        if constexpr (t + 1 < 4) read_a(std::integral_constant<int, t + 1>{}, af[(t + 1) & 1]);
        mfmas(t_c, wf, af[t & 1]);
        if constexpr (t + 1 < 4) wn = weight_frag(std::integral_constant<int, t + 1>{});
        if constexpr ((t + 1) % GK == 0) flush(slot, t / GK);
        wf = wn;
        __builtin_amdgcn_sched_barrier(0);
      });
    } else {
      static_for<0, 4>([&](auto t_c) {
        constexpr int t = decltype(t_c)::value;
        if (s * 4 + t < KT) {
          i32x4 af[4];
          read_a(t_c, af);
          const i32x4 wf = weight_frag(t_c);
          mfmas(t_c, wf, af);
          if constexpr ((t + 1) % GK == 0) flush(slot, t / GK);
        }
      });
    }
  };

  // ---- pipeline: stage s + 1's copies and loads are issued before stage s
  // computes; one barrier per stage.
  WStage<PREP> wb[2] = {};  // zero: the settle step touches every zero-point slot
  uint32_t sc[2] = {0u, 0u};
  copy_a(0, 0);
  load_w(0, wb[0]);
  load_scales(0, sc);
  wait_vm<0>();
  park_scales(0, sc);
  wait_lds_barrier();
  auto stage = [&](int s, auto cur_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(cur_c)::value;
    // This stage's weight registers landed before the last barrier (its wait
    // is inline assembly, which the compiler's wait insertion cannot see):
    // touch them before the next stage's loads are issued, so that the
    // compiler's own wait for them falls here, where it is free, and not
    // behind the new loads.
    settle_stage(wb[cur]);
    if (s + 1 < S) {
      copy_a(s + 1, (s + 1) & 1);
      load_w(s + 1, wb[cur ^ 1]);
      load_scales(s + 1, sc);
    }
    compute(s, wb[cur]);
    if (s + 1 < S) {
      wait_vm<0>();
      park_scales((s + 1) & 1, sc);
    }
    wait_vm_barrier<0>();  // stage s + 1 landed everywhere; slot s & 1 free
  };
  int s = 0;
  for (; s + 1 < S; s += 2) {
    stage(s, std::integral_constant<int, 0>{});
    stage(s + 1, std::integral_constant<int, 1>{});
  }
  if (s < S) stage(s, std::integral_constant<int, 0>{});

  // ---- output: row m0 + 32 i + (l & 31), columns n0 + 32 wave + 8 q + 4 h + c.
  // The row scales and the bias values are loaded before the first store (a
  // load after a store to a possibly aliasing address would wait for it).
  const bool vec = (p.N % 4) == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
  float sa[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float bv[4][4];
  if constexpr (!INTEGER) {
    static_for<0, 4>([&](auto i) { sa[i] = p.a_scale[min(m0 + 32 * decltype(i)::value + lr, p.M - 1)]; });
    // all raw values first, then the widening (no wait between loads)
    uint32_t braw[4][4] = {};
    auto bias_cols = [&](auto load) __attribute__((always_inline)) {
      static_for<0, 4>([&](auto q_c) {
        constexpr int q = decltype(q_c)::value;
        static_for<0, 4>([&](auto c_c) {
          constexpr int c = decltype(c_c)::value;
          braw[q][c] = load(min(n0 + 32 * wave + 8 * q + 4 * h + c, p.N - 1));
        });
      });
    };
    if (p.bias != nullptr) {
      if (p.bias_dtype == QG_F32) bias_cols([&](int col) { return static_cast<const uint32_t*>(p.bias)[col]; });
      else bias_cols([&](int col) { return static_cast<uint32_t>(static_cast<const uint16_t*>(p.bias)[col]); });
    }
    static_for<0, 4>([&](auto q) {
      static_for<0, 4>([&](auto c) {
        const uint32_t r = braw[decltype(q)::value][decltype(c)::value];
        bv[q][c] = p.bias_dtype == QG_F32   ? __uint_as_float(r)
                   : p.bias_dtype == QG_F16 ? f16_to_f32(static_cast<uint16_t>(r))
                                            : bf16_to_f32(static_cast<uint16_t>(r));
      });
    });
  }
  const bool has_bias = p.bias != nullptr;
  static_for<0, 4>([&](auto i_c) {
    constexpr int i = decltype(i_c)::value;
    const int row = m0 + 32 * i + lr;
    if (row >= p.M) return;
    static_for<0, 4>([&](auto q_c) {
      constexpr int q = decltype(q_c)::value;
      const int col0 = n0 + 32 * wave + 8 * q + 4 * h;
      uint32_t bits[4];
      static_for<0, 4>([&](auto c_c) {
        constexpr int c = decltype(c_c)::value;
        if constexpr (INTEGER) {
          bits[c] = static_cast<uint32_t>(itot[i][4 * q + c]);
        } else {
          float y = tot[i][4 * q + c] * sa[i];
          if (has_bias) y = y + bv[q][c];
          bits[c] = __float_as_uint(y);
        }
      });
      uint32_t* orow = static_cast<uint32_t*>(p.out) + static_cast<int64_t>(row) * p.N;
      if (vec && col0 + 4 <= p.N) {
        *reinterpret_cast<i32x4*>(orow + col0) =
            i32x4{static_cast<int>(bits[0]), static_cast<int>(bits[1]), static_cast<int>(bits[2]),
                  static_cast<int>(bits[3])};
      } else {
        static_for<0, 4>([&](auto c_c) {
          constexpr int c = decltype(c_c)::value;
          if (col0 + c < p.N) orow[col0 + c] = bits[c];
        });
      }
    });
  });
}

// ---- waves of 128 rows x 16 columns (K a multiple of 128, packed weights)
//
// The same arithmetic and fold order as k_w4a8 on v_mfma_i32_16x16x32_i8:
// wave w owns output columns 16 w .. 16 w + 15 of a 128 x 16 NW tile over all
// 128 rows (eight 16 x 16 int32 blocks, weights as the first operand). Half
// the columns per wave keeps the nibble expansion and fold per MAC and
// doubles the LDS fragment reads; at <= 168 registers three 4-wave
// workgroups share a CU, so a grid too small to fill the CUs with the 4-wave
// form's 128 x 128 tiles gets twice the tiles and up to three independent
// waves per SIMD (waves of one workgroup meet at every stage's barrier and so
// run their folds and MFMAs in step: an 8-wave form measured slower).
//
// A k-step is 32 K (one g32 group, half a g64 one, a quarter of g128): lane
// l = 16 kg + c supplies 8 bytes of K [32 t + 8 kg, 32 t + 8 kg + 8) of
// weight column 16 w + c (one packed word, expanded to q - z) and of
// activation row 16 b + c; the block result holds columns 16 w + 4 kg .. + 3
// of row 16 b + c in its 4 registers.
template <int G, bool INTEGER, int NW>
__global__ __launch_bounds__(64 * NW, NW == 4 ? 3 : 1) void k_w4a8_n16(W4A8Args p) {
#pragma clang fp contract(off)
  constexpr int BN = 16 * NW;                  // 64 or 128 columns
  constexpr int GK = G / 32;                   // k-steps per group
  constexpr int GS = kStage / G;               // groups per stage
  constexpr int NA = 16 / NW;                  // A copies (1 KB) per wave and stage
  constexpr int SLOT_S = 4 * BN * 4;           // <= 4 groups x BN fp32 scales
  __shared__ __attribute__((aligned(1024))) char smem[2 * kSlotA + 2 * SLOT_S];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kg = lane >> 4;
  int m0, n0;
  w4a8_tile<BN>(p.M, p.N, m0, n0);
  const int S = p.K / kStage;                  // the launcher guarantees K % 128 == 0
  const uint32_t smem_base = lds_addr_of(smem);

  // ---- A copies: as k_w4a8 (rows 8 (wave + NW i) + (l >> 3), chunk swizzle)
  const uint32_t chunk = static_cast<uint32_t>(((lane & 7) ^ (4 * (wave & 1) + (lane >> 4))) << 4);
  uint32_t aoff[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i)
    aoff[i] = static_cast<uint32_t>(min(m0 + wave * 8 + (lane >> 3) + 8 * NW * i, p.M - 1)) *
              static_cast<uint32_t>(p.a_sm);
  const char* a_base = reinterpret_cast<const char*>(p.a);
  auto copy_a = [&](int s, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NA; ++i)
      dma16s(a_base + static_cast<int64_t>(s) * kStage, aoff[i] + chunk, smem_base + slot * kSlotA + (wave + NW * i) * 1024);
  };

  // ---- this lane's weight column and its packed words: k-step t of stage s
  // is word 16 s + 4 t + kg of the column (nk: consecutive words of a row;
  // kn: words N apart)
  const int nw = min(n0 + 16 * wave + c16, p.N - 1);
  const bool kn = p.flags & QG_W4_LAYOUT_KN;
  const bool sgn = p.flags & QG_W4_SIGNED_NIBBLES;
  const bool zpk = p.flags & QG_W4_ZEROS_PACKED;
  const bool high = p.flags & QG_W4_ORDER_HIGH;
  const uint32_t* wcol = p.w + (kn ? static_cast<int64_t>(nw) : static_cast<int64_t>(nw) * (p.K / 8));
  const int64_t kstride = kn ? p.N : 1;
  const uint32_t xmask = sgn ? 0x88888888u : 0u;
  const uint32_t sel0 = high ? 0x02060307u : 0x05010400u;
  const uint32_t sel1 = high ? 0x00040105u : 0x07030602u;

  struct Stage {
    uint32_t w[4];
    uint32_t zraw[4];
  };
  auto load_w = [&](int s, Stage& b) __attribute__((always_inline)) {
    static_for<0, 4>([&](auto t) { b.w[decltype(t)::value] = wcol[(16 * s + 4 * decltype(t)::value + kg) * kstride]; });
    static_for<0, GS>([&](auto gi_c) {
      constexpr int gi = decltype(gi_c)::value;
      const int g = min(s * GS + gi, p.ng - 1);
      b.zraw[gi] = zpk ? static_cast<const uint32_t*>(p.zeros)[static_cast<int64_t>(nw) * p.zw + (g >> 3)]
                       : static_cast<uint32_t>(static_cast<const int32_t*>(p.zeros)[static_cast<int64_t>(nw) * p.ng + g]);
    });
  };
  auto zero_bytes = [&](int s, int gi, uint32_t zraw) __attribute__((always_inline)) {
    const int g = min(s * GS + gi, p.ng - 1);
    int zu;
    if (zpk) {
      const int z = static_cast<int>((zraw >> (4 * (g & 7))) & 15u);
      zu = sgn ? (z ^ 8) : z;
    } else {
      const int z = static_cast<int>(zraw);
      zu = sgn ? z + 8 : z;
    }
    return static_cast<uint32_t>(zu) * 0x01010101u;
  };
  // a packed word (8 K in order) -> 8 signed bytes q - z in K order
  auto expand = [&](uint32_t word, uint32_t zb) __attribute__((always_inline)) {
    const uint32_t x = word ^ xmask;
    const uint32_t lo = (((x & 0x0F0F0F0Fu) | 0x80808080u) - zb) ^ 0x80808080u;
    const uint32_t hi = ((((x >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - zb) ^ 0x80808080u;
    const uint64_t d0 = __builtin_amdgcn_perm(hi, lo, sel0);
    const uint64_t d1 = __builtin_amdgcn_perm(hi, lo, sel1);
    return static_cast<int64_t>(d0 | (d1 << 32));
  };

  // ---- scales of a stage: thread t covers column t % BN, group t / BN
  const int scol = tid & (BN - 1), sg = tid / BN;
  const int scn = min(n0 + scol, p.N - 1);
  auto load_scales = [&](int s, uint32_t& sc) __attribute__((always_inline)) {
    if constexpr (!INTEGER) {
      const int g = min(s * GS + min(sg, GS - 1), p.ng - 1);
      const int64_t i = static_cast<int64_t>(scn) * p.ng + g;
      sc = p.scale_f32 ? static_cast<const uint32_t*>(p.scales)[i]
                       : static_cast<uint32_t>(static_cast<const uint16_t*>(p.scales)[i]);
    }
  };
  auto park_scales = [&](int slot, uint32_t sc) __attribute__((always_inline)) {
    if constexpr (!INTEGER) {
      float* dst = reinterpret_cast<float*>(smem + 2 * kSlotA + slot * SLOT_S);
      if (sg < GS) dst[sg * BN + scol] = p.scale_f32 ? __uint_as_float(sc) : bf16_to_f32(static_cast<uint16_t>(sc));
    }
  };

  i32x4 acc[8];
  float tot[8][4];
  int itot[8][4];
  static_for<0, 8>([&](auto b) {
    static_for<0, 4>([&](auto r) {
      tot[b][r] = 0.0f;
      itot[b][r] = 0;
    });
  });
  // fold the finished group gi of the stage in slot `slot` (pinned in place,
  // as in k_w4a8's full-K body)
  auto flush = [&](int slot, int gi) __attribute__((always_inline)) {
    f32x4 s4 = {0, 0, 0, 0};
    if constexpr (!INTEGER)
      s4 = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(smem + 2 * kSlotA + slot * SLOT_S) +
                                           gi * BN + 16 * wave + 4 * kg);
    static_for<0, 8>([&](auto b_c) {
      constexpr int b = decltype(b_c)::value;
      static_for<0, 4>([&](auto r_c) {
        constexpr int r = decltype(r_c)::value;
        const int v = acc[b][r];
        if constexpr (INTEGER) {
          itot[b][r] += v;
          asm volatile("" : "+v"(itot[b][r]));
        } else {
          tot[b][r] = tot[b][r] + static_cast<float>(v) * s4[r];
          asm volatile("" : "+v"(tot[b][r]));
        }
      });
    });
  };
  // activation fragment of block b, k-step t: row 16 b + c16, K bytes
  // [32 t + 8 kg, + 8) = half (kg & 1) of logical chunk 2 t + (kg >> 1)
  auto read_a = [&](const char* abase, auto t_c, int64_t (&af)[8]) __attribute__((always_inline)) {
    constexpr int t = decltype(t_c)::value;
    static_for<0, 8>([&](auto b_c) {
      constexpr int b = decltype(b_c)::value;
      const int row = 16 * b + c16;
      const int off = row * kStage + ((((2 * t + (kg >> 1)) ^ ((row >> 1) & 7))) << 4) + 8 * (kg & 1);
      af[b] = *reinterpret_cast<const int64_t*>(abase + off);
    });
  };

  // MFMAs of stage s: k-step t + 1's fragments are read and its weight word
  // expanded under k-step t's MFMAs; nothing moves across k-steps.
  auto compute = [&](int s, const Stage& b_in) __attribute__((always_inline)) {
    const int slot = s & 1;
    const char* abase = smem + slot * kSlotA;
    uint32_t zbs[GS];
    static_for<0, GS>([&](auto gi) { zbs[gi] = zero_bytes(s, gi, b_in.zraw[gi]); });
    int64_t af[2][8];
    read_a(abase, std::integral_constant<int, 0>{}, af[0]);
    int64_t wf = expand(b_in.w[0], zbs[0]);
    static_for<0, 4>([&](auto t_c) {
      constexpr int t = decltype(t_c)::value;
      int64_t wn = wf;
      if constexpr (t + 1 < 4) read_a(abase, std::integral_constant<int, t + 1>{}, af[(t + 1) & 1]);
      static_for<0, 8>([&](auto b_c) {
        constexpr int b = decltype(b_c)::value;
        if constexpr (t % GK == 0) acc[b] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wf, af[t & 1][b], i32x4{}, 0, 0, 0);
        else acc[b] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wf, af[t & 1][b], acc[b], 0, 0, 0);
      });
      if constexpr (t + 1 < 4) wn = expand(b_in.w[t + 1], zbs[(t + 1) / GK]);
      if constexpr ((t + 1) % GK == 0) flush(slot, t / GK);
      wf = wn;
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // ---- pipeline: stage s + 1's copies and loads are issued before stage s
  // computes (this stage's registers touched first, see k_w4a8); one barrier
  // per stage
  Stage wb[2] = {};  // zero: the settle step touches every zero-point slot
  uint32_t sc = 0u;
  copy_a(0, 0);
  load_w(0, wb[0]);
  load_scales(0, sc);
  wait_vm<0>();
  park_scales(0, sc);
  wait_lds_barrier();
  auto settle = [&](Stage& b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      asm volatile("" : "+v"(b.w[i]));
      asm volatile("" : "+v"(b.zraw[i]));
    }
  };
  auto stage = [&](int s, auto cur_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(cur_c)::value;
    settle(wb[cur]);
    if (s + 1 < S) {
      copy_a(s + 1, (s + 1) & 1);
      load_w(s + 1, wb[cur ^ 1]);
      load_scales(s + 1, sc);
    }
    compute(s, wb[cur]);
    if (s + 1 < S) {
      wait_vm<0>();
      park_scales((s + 1) & 1, sc);
    }
    wait_vm_barrier<0>();  // stage s + 1 landed everywhere; slot s & 1 free
  };
  int s = 0;
  for (; s + 1 < S; s += 2) {
    stage(s, std::integral_constant<int, 0>{});
    stage(s + 1, std::integral_constant<int, 1>{});
  }
  if (s < S) stage(s, std::integral_constant<int, 0>{});

  // ---- output: row m0 + 16 b + c16, columns n0 + 16 wave + 4 kg + r. The
  // row scales and the bias are loaded before the first store.
  const int col0 = n0 + 16 * wave + 4 * kg;
  const bool vec = (p.N % 4) == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
  float sa[8];
  float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (!INTEGER) {
    static_for<0, 8>([&](auto b) { sa[b] = p.a_scale[min(m0 + 16 * decltype(b)::value + c16, p.M - 1)]; });
    uint32_t braw[4] = {};
    if (p.bias != nullptr) {
      if (p.bias_dtype == QG_F32)
        static_for<0, 4>([&](auto r) { braw[r] = static_cast<const uint32_t*>(p.bias)[min(col0 + decltype(r)::value, p.N - 1)]; });
      else
        static_for<0, 4>([&](auto r) {
          braw[r] = static_cast<const uint16_t*>(p.bias)[min(col0 + decltype(r)::value, p.N - 1)];
        });
    }
    static_for<0, 4>([&](auto r) {
      const uint32_t x = braw[r];
      bv[r] = p.bias_dtype == QG_F32   ? __uint_as_float(x)
              : p.bias_dtype == QG_F16 ? f16_to_f32(static_cast<uint16_t>(x))
                                       : bf16_to_f32(static_cast<uint16_t>(x));
    });
  }
  const bool has_bias = p.bias != nullptr;
  static_for<0, 8>([&](auto b_c) {
    constexpr int b = decltype(b_c)::value;
    const int row = m0 + 16 * b + c16;
    if (row >= p.M) return;
    uint32_t bits[4];
    static_for<0, 4>([&](auto r_c) {
      constexpr int r = decltype(r_c)::value;
      if constexpr (INTEGER) {
        bits[r] = static_cast<uint32_t>(itot[b][r]);
      } else {
        float y = tot[b][r] * sa[b];
        if (has_bias) y = y + bv[r];
        bits[r] = __float_as_uint(y);
      }
    });
    uint32_t* orow = static_cast<uint32_t*>(p.out) + static_cast<int64_t>(row) * p.N;
    if (vec && col0 + 4 <= p.N) {
      *reinterpret_cast<i32x4*>(orow + col0) = i32x4{static_cast<int>(bits[0]), static_cast<int>(bits[1]),
                                                     static_cast<int>(bits[2]), static_cast<int>(bits[3])};
    } else {
      static_for<0, 4>([&](auto r_c) {
        constexpr int r = decltype(r_c)::value;
        if (col0 + r < p.N) orow[col0 + r] = bits[r];
      });
    }
  });
}

// 4 waves (two workgroups per CU): 8 waves on 128 x 256 tiles halve the A
// bytes per MAC but took 187 us against 145 us on (4096, 3072, 3072) g128 and
// 105 against 82 us on (1061, 3072, 3072) g32 (one workgroup per CU: the
// per-stage barrier then stalls every wave of the CU at once).
constexpr int kW4A8Waves = 4;

template <int G, bool PREP>
hipError_t launch_g(const W4A8Args& p, hipStream_t stream) {
  constexpr int NW = kW4A8Waves;
  const int blocks = ceil_div(p.M, kBM) * ceil_div(p.N, W8Geo<NW>::BN);
  // nk words with 16-byte aligned rows (K % 32 == 0 makes every row a
  // multiple of 16 bytes): 16-byte weight loads
  const bool vec = !PREP && !(p.flags & QG_W4_LAYOUT_KN) && (reinterpret_cast<uintptr_t>(p.w) & 15) == 0;
  // K a multiple of the 128-byte stage: every stage holds four k-steps, and
  // the stage body is one straight-line block the compiler can schedule
  // across k-steps (fragment reads and nibble expansion under the MFMAs)
  const bool fullk = (p.K % kStage) == 0;
  const dim3 grid(blocks), block(W8Geo<NW>::THREADS);
#define QG_W4A8(INT, V)                                                                                 \
  do {                                                                                                \
    if (fullk) hipLaunchKernelGGL((k_w4a8<G, PREP, INT, NW, V, true>), grid, block, 0, stream, p);   \
    else hipLaunchKernelGGL((k_w4a8<G, PREP, INT, NW, V, false>), grid, block, 0, stream, p);        \
  } while (0)
  if (p.integer) {
    if (vec) QG_W4A8(true, true);
    else QG_W4A8(true, false);
  } else {
    if (vec) QG_W4A8(false, true);
    else QG_W4A8(false, false);
  }
#undef QG_W4A8
  return hipGetLastError();
}

constexpr int kN16Waves = 4;

template <int G>
hipError_t launch_n16(const W4A8Args& p, hipStream_t stream) {
  constexpr int NW = kN16Waves;
  const int blocks = ceil_div(p.M, kBM) * ceil_div(p.N, 16 * NW);
  const dim3 grid(blocks), block(64 * NW);
  if (p.integer) hipLaunchKernelGGL((k_w4a8_n16<G, true, NW>), grid, block, 0, stream, p);
  else hipLaunchKernelGGL((k_w4a8_n16<G, false, NW>), grid, block, 0, stream, p);
  return hipGetLastError();
}

// The 16-column form where the 4-wave grid leaves the CUs short of waves: at
// most 128 of its 128 x 128 tiles, or at most 256 with g32, whose four folds
// per stage make the vector ALU the bound (one MI355X, both kernels in one
// run: M 512 x N 3072 x K 3072 all groups 15-28 % faster, M 1061 g32 8-13 %;
// M 1061 g64 / g128, M 2048, M 4096 and N 9216 slower).
bool use_n16(const W4A8Args& p) {
  if (p.w8 != nullptr || p.K <= 0 || p.K % kStage != 0) return false;
  const int64_t tiles = static_cast<int64_t>(ceil_div(p.M, kBM)) * ceil_div(p.N, W8Geo<kW4A8Waves>::BN);
  return tiles <= 128 || (tiles <= 256 && p.group == 32);
}

template <bool PREP>
hipError_t launch_p(const W4A8Args& p, hipStream_t stream) {
  if (!PREP && use_n16(p)) {
    if (p.group == 32) return launch_n16<32>(p, stream);
    if (p.group == 64) return launch_n16<64>(p, stream);
    return launch_n16<128>(p, stream);
  }
  if (p.group == 32) return launch_g<32, PREP>(p, stream);
  if (p.group == 64) return launch_g<64, PREP>(p, stream);
  return launch_g<128, PREP>(p, stream);
}

}  // namespace

hipError_t launch_w4a8_gemm(const W4A8Args& p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  return p.w8 != nullptr ? launch_p<true>(p, stream) : launch_p<false>(p, stream);
}

}  // namespace qg
