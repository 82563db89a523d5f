// W4A16 group-dequant GEMM, INT4 weight packing and unpacking for gfx950.
//
// Reference behaviour: rdna2-ops/rdna2_ops/int4_weight_gemm_v07.py
//   PackedInt4 storage (:20-46), pack_int4 / _pack_weight (:103-133, :413-430),
//   unpack_int4 / _unpack_weight (:136-151, :450-458), int4_linear_a16 (:540-564).
//
// Arithmetic of the GEMM (MI355X design, not the reference's dot2 tiles):
//   y[m,n] = sum_g s[n,g] * ( sum_{k in g} a[m,k] * (MAGIC + u[n,k])
//                              - (MAGIC + z[n,g]) * sum_{k in g} a[m,k] ) (+ bias[n])
// where u is the unsigned nibble (signed storage: u = q + 8) and z the unsigned
// zero point. Each nibble becomes an exact 16-bit float with one AND-OR:
// bf16 128 + u (nibble in mantissa bits 0-3), fp16 256 + 4u (nibble in
// mantissa bits 4-7; the factor 4 is folded into the group scale), so the
// bf16/fp16 MFMA sees exact weights and accumulates exact products in fp32;
// the per-row group sums come from a second MFMA against a fragment of ones.
// The group scale is applied once per group in fp32 — more accurate than
// rounding every dequantised weight to fp16 as the reference's dot2 path does.
#include "qg_common.h"
#include "qg_internal.h"

namespace qg {

namespace {

typedef short i16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------- fragments
// MFMA v_mfma_f32_16x16x32_{bf16,f16}: lane l supplies row / column (l & 15)
// and the 8 consecutive K values of chunk (l >> 4); the accumulator holds rows
// 4 (l >> 4) + i, column l & 15.
template <bool F16A>
__device__ __forceinline__ f32x4 mfma16(const i32x4& a, const i32x4& b, const f32x4& c) {
  if constexpr (F16A)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// One packed word (8 nibbles = 8 consecutive K) -> 4 registers of 16-bit
// floats MAGIC + u in natural K order (register i = elements 2i, 2i+1), so the
// activation fragment is used exactly as it lies in memory.
//   low order : nibble e at bits 4e       -> element e = low nibble of byte e/2 (even e)
//   high order: nibble e at bits 28 - 4e  -> element e = high nibble of byte 3 - e/2 (even e)
// v_perm_b32 gathers byte i of w and of w >> 4 into the two halves, one AND-OR
// keeps the nibbles and inserts the exponent.
// bf16: nibbles land in bits 0-3 of each half (bytes of w and w >> 4);
// fp16: in bits 4-7 (bytes of w << 4 and w).
template <bool F16A>
__device__ __forceinline__ i32x4 unpack_word(uint32_t w, const uint32_t (&sel)[4]) {
  const uint32_t lo = F16A ? w << 4 : w;
  const uint32_t hi = F16A ? w : w >> 4;
  constexpr uint32_t mask = F16A ? 0x00F000F0u : 0x000F000Fu;
  constexpr uint32_t magic2 = F16A ? 0x5C005C00u : 0x43004300u;  // fp16 256 / bf16 128
  i32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t t = __builtin_amdgcn_perm(hi, lo, sel[i]);
    r[i] = static_cast<int>((t & mask) | magic2);
  }
  return r;
}

// v_perm selectors: combined bytes 0-3 = lo, 4-7 = hi (lo/hi: the two shifted
// copies of the word); 0x0C = zero byte.
__device__ __forceinline__ void unpack_selectors(bool high, uint32_t (&sel)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // low : half 0 <- byte i of w (low nibble = element 2i),
    //       half 1 <- byte i of w>>4 (its low nibble = element 2i+1)
    // high: half 0 <- byte 3-i of w>>4 (high nibble of byte 3-i = element 2i),
    //       half 1 <- byte 3-i of w (low nibble = element 2i+1)
    const uint32_t b0 = high ? (4u + 3u - i) : static_cast<uint32_t>(i);
    const uint32_t b2 = high ? (3u - i) : (4u + i);
    sel[i] = 0x0C000C00u | (b2 << 16) | b0;
  }
}

__device__ __forceinline__ float load_bias(const void* bias, int dtype, int col) {
  if (dtype == QG_F32) return static_cast<const float*>(bias)[col];
  const uint16_t b = static_cast<const uint16_t*>(bias)[col];
  return dtype == QG_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

__device__ __forceinline__ void store_out(void* out, int dtype, int64_t idx, float v) {
  if (dtype == QG_F32) static_cast<float*>(out)[idx] = v;
  else if (dtype == QG_F16) static_cast<uint16_t*>(out)[idx] = f32_to_f16(v);
  else static_cast<uint16_t*>(out)[idx] = f32_to_bf16(v);
}

// Scale and unsigned zero point of group g of column n, in the units of the
// expanded weights: weight value = (zb_unit * u + magic) with zb = magic +
// unit * zu and s = scale / unit (unit 4 for fp16, 1 otherwise; exact).
struct GroupParams {
  float s, zb;
};

__device__ __forceinline__ GroupParams group_params(const W4Args& p, int n, int g, float magic,
                                                    float unit = 1.0f) {
  const int ng = p.K / p.group;
  GroupParams r;
  const int64_t i = static_cast<int64_t>(n) * ng + g;
  r.s = p.scale_f32 ? static_cast<const float*>(p.scales)[i]
                    : bf16_to_f32(static_cast<const uint16_t*>(p.scales)[i]);
  int zu;
  if (p.flags & QG_W4_ZEROS_PACKED) {
    const int zw = (ng + 7) >> 3;
    const uint32_t word = static_cast<const uint32_t*>(p.zeros)[static_cast<int64_t>(n) * zw + (g >> 3)];
    zu = static_cast<int>((word >> ((g & 7) * 4)) & 15u);
    if (p.flags & QG_W4_SIGNED_NIBBLES) zu ^= 8;
  } else {
    zu = static_cast<const int32_t*>(p.zeros)[i];
    if (p.flags & QG_W4_SIGNED_NIBBLES) zu += 8;
  }
  r.zb = magic + unit * static_cast<float>(zu);
  r.s = r.s / unit;
  return r;
}

// ------------------------------------------------------------- skinny kernel
// Small M (decode): one 256-thread workgroup per 16 output columns x 16*FM
// rows. The K axis is cut into 128-wide chunks; wave w takes chunks
// w, w+4, w+8, ... so the four waves stream each weight row front to back
// together. Per chunk a lane loads its column's 4 words (16 bytes, one
// dwordx4 in the nk / group-128 layout) and its rows' activations straight
// from memory; no LDS staging, DEPTH chunks in flight per wave. The four
// partial tiles are summed through LDS in a fixed order (deterministic).
//
// Word f of a chunk feeds MFMA step j from lane group q, with f chosen so
// that each step stays inside one quantisation group:
//   nk, G=128: f = 4q + j (one dwordx4 per lane)
//   nk, G=64 : f = 8 (j / 2) + 2q + (j % 2) (two dwordx2)
//   G=32, kn : f = 4j + q (four dwords)
template <int G, bool KN>
__device__ __forceinline__ int word_of(int q, int j) {
  if constexpr (!KN && G == 128) return 4 * q + j;
  else if constexpr (!KN && G == 64) return 8 * (j >> 1) + 2 * q + (j & 1);
  else return 4 * j + q;
}

template <int FM, int SPC>
struct SkinnyChunk {
  uint32_t w[4];
  i32x4 a[FM][4];
  GroupParams gp[SPC];
};

template <int FM, int G, bool KN, bool F16A, int DEPTH>
__global__ __launch_bounds__(256) void k_w4_skinny(W4Args p) {
#pragma clang fp contract(off)
  constexpr int SPC = 128 / G;                  // groups per chunk
  constexpr int STEPS_PER_GROUP = 4 / SPC;
  constexpr float MAGIC = F16A ? 256.0f : 128.0f;
  constexpr float UNIT = F16A ? 4.0f : 1.0f;
  const uint32_t ones2 = F16A ? 0x3C003C00u : 0x3F803F80u;

  __shared__ float red[4][FM * 16][17];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * 16 * FM;
  const int n = min(n0 + col, p.N - 1);
  const int C = ceil_div(p.K, 128);
  const int KW = p.K >> 3;  // words per column

  uint32_t sel[4];
  unpack_selectors(p.flags & QG_W4_ORDER_HIGH, sel);
  const uint32_t wxor = (p.flags & QG_W4_SIGNED_NIBBLES) ? 0x88888888u : 0u;
  const i32x4 ones = {static_cast<int>(ones2), static_cast<int>(ones2), static_cast<int>(ones2),
                      static_cast<int>(ones2)};

  const uint32_t* wcol = KN ? p.w + n : p.w + static_cast<int64_t>(n) * KW;
  const int64_t wstride = KN ? p.N : 1;

  auto load = [&](SkinnyChunk<FM, SPC>& ch, int c) {
    const int kw0 = c * 16;
    const int steps = min(4, (p.K - c * 128) >> 5);
    if constexpr (!KN && G == 128) {
      const i32x4 v = *reinterpret_cast<const i32x4*>(wcol + kw0 + 4 * q);
      static_for<0, 4>([&](auto j) { ch.w[j] = static_cast<uint32_t>(v[int(j)]); });
    } else if constexpr (!KN && G == 64) {
      const uint2 v0 = *reinterpret_cast<const uint2*>(wcol + kw0 + 2 * q);
      ch.w[0] = v0.x;
      ch.w[1] = v0.y;
      if (steps > 2) {
        const uint2 v1 = *reinterpret_cast<const uint2*>(wcol + kw0 + 8 + 2 * q);
        ch.w[2] = v1.x;
        ch.w[3] = v1.y;
      } else {
        ch.w[2] = ch.w[3] = 0;
      }
    } else {
      static_for<0, 4>([&](auto j) {
        ch.w[j] = j < steps ? wcol[(kw0 + word_of<G, KN>(q, j)) * wstride] : 0u;
      });
    }
    static_for<0, SPC>([&](auto g) {
      if (g * (G / 32) < steps) ch.gp[g] = group_params(p, n, c * SPC + g, MAGIC, UNIT);
    });
    static_for<0, FM>([&](auto f) {
      const int row = m0 + 16 * f + col;
      const uint16_t* arow = p.a + static_cast<int64_t>(min(row, p.M - 1)) * p.a_sm + c * 128;
      static_for<0, 4>([&](auto j) {
        i32x4 v = {0, 0, 0, 0};
        if (row < p.M && j < steps)
          v = *reinterpret_cast<const i32x4*>(arow + 8 * word_of<G, KN>(q, j));
        ch.a[f][j] = v;
      });
    });
  };

  f32x4 total[FM], acc[FM], asum[FM];
  static_for<0, FM>([&](auto f) { total[f] = f32x4{0, 0, 0, 0}; });

  auto compute = [&](const SkinnyChunk<FM, SPC>& ch, int c) {
    const int steps = min(4, (p.K - c * 128) >> 5);
    static_for<0, 4>([&](auto j) {
      if (j < steps) {
        if constexpr (j % STEPS_PER_GROUP == 0) {
          static_for<0, FM>([&](auto f) {
            acc[f] = f32x4{0, 0, 0, 0};
            asum[f] = f32x4{0, 0, 0, 0};
          });
        }
        const i32x4 b = unpack_word<F16A>(ch.w[j] ^ wxor, sel);
        static_for<0, FM>([&](auto f) {
          acc[f] = mfma16<F16A>(ch.a[f][j], b, acc[f]);
          asum[f] = mfma16<F16A>(ch.a[f][j], ones, asum[f]);
        });
        if constexpr (j % STEPS_PER_GROUP == STEPS_PER_GROUP - 1) {
          const GroupParams gp = ch.gp[j / STEPS_PER_GROUP];
          static_for<0, FM>([&](auto f) {
            static_for<0, 4>([&](auto i) {
              const float t = acc[f][int(i)] - gp.zb * asum[f][int(i)];
              total[f][int(i)] = total[f][int(i)] + gp.s * t;
            });
          });
        }
      }
    });
  };

  SkinnyChunk<FM, SPC> buf[DEPTH];
  static_for<0, DEPTH>([&](auto d) {
    if (wave + 4 * d < C) load(buf[d], wave + 4 * d);
  });
  for (int base = wave; base < C; base += 4 * DEPTH) {
    static_for<0, DEPTH>([&](auto d) {
      const int c = base + 4 * d;
      if (c < C) {
        compute(buf[d], c);
        if (c + 4 * DEPTH < C) load(buf[d], c + 4 * DEPTH);
      }
    });
  }

  static_for<0, FM>([&](auto f) {
    static_for<0, 4>([&](auto i) { red[wave][16 * f + 4 * q + i][col] = total[f][int(i)]; });
  });
  __syncthreads();
  for (int e = threadIdx.x; e < FM * 256; e += 256) {
    const int r = e >> 4, cc = e & 15;
    const int row = m0 + r, nn = n0 + cc;
    if (row < p.M && nn < p.N) {
      float v = red[0][r][cc];
      v = v + red[1][r][cc];
      v = v + red[2][r][cc];
      v = v + red[3][r][cc];
      if (p.bias) v = v + load_bias(p.bias, p.bias_dtype, nn);
      store_out(p.out, p.out_dtype, static_cast<int64_t>(row) * p.N + nn, v);
    }
  }
}

// ------------------------------------------------------------ pack / unpack
// One thread per (column n, octet of 8 groups): the zero points of an octet
// share one packed word. Rule of _pack_weight (int4_weight_gemm_v07.py:103-133)
// with fp32 IEEE division and round-half-even; the scale is rounded to the
// storage dtype first when that is bf16, and an all-zero group (scale 0) gets
// scale 1.
__device__ __forceinline__ float load_w(const void* w, int dt, int64_t i) {
  if (dt == QG_F32) return static_cast<const float*>(w)[i];
  const uint16_t b = static_cast<const uint16_t*>(w)[i];
  return dt == QG_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

__global__ void k_w4_pack(W4PackArgs p) {
  const int ng = p.K / p.group;
  const int octs = (ng + 7) >> 3;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= static_cast<int64_t>(p.N) * octs) return;
  const int n = static_cast<int>(t / octs), o = static_cast<int>(t % octs);
  const bool sgn = p.flags & QG_W4_SIGNED_NIBBLES;
  const bool high = p.flags & QG_W4_ORDER_HIGH;
  const bool kn = p.flags & QG_W4_LAYOUT_KN;
  uint32_t zword = 0;
  for (int g = o * 8; g < min(ng, o * 8 + 8); ++g) {
    const int64_t base = static_cast<int64_t>(n) * p.w_sn + static_cast<int64_t>(g) * p.group * p.w_sk;
    float lo = 0.0f, hi = 0.0f, amax = 0.0f;
    for (int r = 0; r < p.group; ++r) {
      const float x = load_w(p.w, p.w_dtype, base + r * p.w_sk);
      lo = fminf(lo, x);
      hi = fmaxf(hi, x);
      amax = fmaxf(amax, fabsf(x));
    }
    float s = p.symmetric ? __fdiv_rn(amax, 7.0f) : __fdiv_rn(hi - lo, 15.0f);
    if (p.scale_dtype == QG_BF16) s = bf16_to_f32(f32_to_bf16(s));
    const bool empty = s == 0.0f;
    if (empty) s = 1.0f;
    int zu = 8;  // unsigned zero point; symmetric codes are centred on 8
    if (!p.symmetric) zu = static_cast<int>(fminf(fmaxf(__builtin_rintf(__fdiv_rn(-lo, s)), 0.0f), 15.0f));
    const bool signed_empty = sgn && !p.symmetric && empty;  // reference: q = zero = 0
    if (signed_empty) zu = 8;
    int sum = 0;
    for (int wi = 0; wi < p.group / 8; ++wi) {
      uint32_t word = 0;
      for (int e = 0; e < 8; ++e) {
        const float x = load_w(p.w, p.w_dtype, base + (wi * 8 + e) * p.w_sk);
        const float r = __builtin_rintf(__fdiv_rn(x, s));
        int qu;
        if (p.symmetric) qu = static_cast<int>(fminf(fmaxf(r, -7.0f), 7.0f)) + 8;
        else qu = static_cast<int>(fminf(fmaxf(r + static_cast<float>(zu), 0.0f), 15.0f));
        if (signed_empty) qu = 8;
        const int stored = sgn ? qu - 8 : qu;
        sum += stored;
        const int shift = high ? 28 - 4 * e : 4 * e;
        word |= static_cast<uint32_t>(stored & 15) << shift;
      }
      const int64_t kw = static_cast<int64_t>(g) * (p.group / 8) + wi;
      if (kn) p.data[kw * p.N + n] = static_cast<int32_t>(word);
      else p.data[static_cast<int64_t>(n) * (p.K / 8) + kw] = static_cast<int32_t>(word);
    }
    const int64_t gi = static_cast<int64_t>(n) * ng + g;
    if (p.scale_dtype == QG_F32) static_cast<float*>(p.scales)[gi] = s;
    else static_cast<uint16_t*>(p.scales)[gi] = f32_to_bf16(s);
    const int zstored = sgn ? zu - 8 : zu;
    if (p.flags & QG_W4_ZEROS_PACKED) zword |= static_cast<uint32_t>(zstored & 15) << (4 * (g & 7));
    else static_cast<int32_t*>(p.zeros)[gi] = zstored;
    if (p.sums) p.sums[gi] = sum;
  }
  if (p.flags & QG_W4_ZEROS_PACKED) static_cast<int32_t*>(p.zeros)[static_cast<int64_t>(n) * octs + o] = static_cast<int32_t>(zword);
}

// out[n, k] = (q - z) (int8) or (q - z) * s rounded once to the output dtype
// (_unpack_weight, int4_weight_gemm_v07.py:136-151).
__global__ void k_w4_unpack(W4Args p) {
  const int64_t total = static_cast<int64_t>(p.N) * p.K;
  const int ng = p.K / p.group;
  const bool sgn = p.flags & QG_W4_SIGNED_NIBBLES;
  const bool high = p.flags & QG_W4_ORDER_HIGH;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int n = static_cast<int>(i / p.K), k = static_cast<int>(i % p.K);
    const int64_t kw = k >> 3;
    const uint32_t word = static_cast<uint32_t>(
        (p.flags & QG_W4_LAYOUT_KN) ? p.w[kw * p.N + n] : p.w[static_cast<int64_t>(n) * (p.K >> 3) + kw]);
    const int e = k & 7;
    int u = static_cast<int>((word >> (high ? 28 - 4 * e : 4 * e)) & 15u);
    if (sgn) u ^= 8;
    const GroupParams gp = group_params(p, n, k / p.group, 0.0f);
    const int cen = u - static_cast<int>(gp.zb);
    if (p.out_dtype == QG_I8) {
      static_cast<int8_t*>(p.out)[i] = static_cast<int8_t>(cen);
    } else {
      const float v = static_cast<float>(cen) * gp.s;
      store_out(p.out, p.out_dtype, i, v);
    }
    (void)ng;
  }
}

template <int FM, int G, bool KN, bool F16A>
hipError_t launch_skinny_t(const W4Args& p, hipStream_t stream) {
  constexpr int DEPTH = FM == 1 ? 4 : 2;
  dim3 grid(ceil_div(p.N, 16), ceil_div(p.M, 16 * FM));
  hipLaunchKernelGGL((k_w4_skinny<FM, G, KN, F16A, DEPTH>), grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int FM, bool F16A>
hipError_t launch_skinny_g(const W4Args& p, hipStream_t stream) {
  const bool kn = p.flags & QG_W4_LAYOUT_KN;
  switch (p.group) {
    case 128: return kn ? launch_skinny_t<FM, 128, true, F16A>(p, stream) : launch_skinny_t<FM, 128, false, F16A>(p, stream);
    case 64: return kn ? launch_skinny_t<FM, 64, true, F16A>(p, stream) : launch_skinny_t<FM, 64, false, F16A>(p, stream);
    default: return kn ? launch_skinny_t<FM, 32, true, F16A>(p, stream) : launch_skinny_t<FM, 32, false, F16A>(p, stream);
  }
}

template <bool F16A>
hipError_t launch_skinny(const W4Args& p, hipStream_t stream) {
  if (p.M <= 16) return launch_skinny_g<1, F16A>(p, stream);
  if (p.M <= 32) return launch_skinny_g<2, F16A>(p, stream);
  return launch_skinny_g<4, F16A>(p, stream);
}

}  // namespace

hipError_t launch_w4a16(const W4Args& p, hipStream_t stream) {
  return p.a_f16 ? launch_skinny<true>(p, stream) : launch_skinny<false>(p, stream);
}

hipError_t launch_w4_pack(const W4PackArgs& p, hipStream_t stream) {
  const int64_t threads = static_cast<int64_t>(p.N) * ceil_div(p.K / p.group, 8);
  const int64_t blocks = ceil_div<int64_t>(threads, 256);
  hipLaunchKernelGGL(k_w4_pack, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_w4_unpack(const W4Args& p, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(p.N) * p.K;
  int64_t blocks = ceil_div<int64_t>(total, 256);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_w4_unpack, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace qg
