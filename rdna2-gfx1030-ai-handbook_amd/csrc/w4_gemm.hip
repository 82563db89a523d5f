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
// mask / magic2 come from unpack_consts(): held in registers so that each
// register costs one v_perm_b32 and one v_and_or_b32 (a VOP3 instruction
// cannot take the literals directly on gfx9).
template <bool F16A>
__device__ __forceinline__ i32x4 unpack_word(uint32_t w, const uint32_t (&sel)[4], uint32_t mask,
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

template <bool F16A>
__device__ __forceinline__ void unpack_consts(uint32_t& mask, uint32_t& magic2) {
  mask = F16A ? 0x00F000F0u : 0x000F000Fu;
  magic2 = F16A ? 0x5C005C00u : 0x43004300u;  // fp16 256 / bf16 128
  asm volatile("" : "+v"(mask), "+v"(magic2));
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
// expanded weights (value = magic + unit * u): zb = magic + unit * zu and
// s = scale / unit (unit 4 for fp16, 1 for bf16; exact).
struct GroupParams {
  float s, zb;
};

// Raw storage words of a group's scale and zero point. Both are read as
// aligned dwords whatever the storage dtype, so the loads are unconditional
// (no data-dependent control flow around them); the dtype and packing are
// resolved afterwards by decode_group().
struct GroupRaw {
  uint32_t s, z;
};

__device__ __forceinline__ GroupRaw load_group(const W4Args& p, int n, int g) {
  const uint32_t i = static_cast<uint32_t>(n) * p.ng + g;
  const uint32_t sb = p.scale_f32 ? 4u * i : 4u * (i >> 1);
  const uint32_t zb = (p.flags & QG_W4_ZEROS_PACKED)
                          ? 4u * (static_cast<uint32_t>(n) * p.zw + (g >> 3))
                          : 4u * i;
  GroupRaw r;
  r.s = *reinterpret_cast<const uint32_t*>(static_cast<const char*>(p.scales) + sb);
  r.z = *reinterpret_cast<const uint32_t*>(static_cast<const char*>(p.zeros) + zb);
  return r;
}

// UINT4: storage known at compile time to be bf16 scales, packed unsigned
// zero points (the benchmark's uint4 format); otherwise resolved from p.flags.
template <bool UINT4 = false>
__device__ __forceinline__ GroupParams decode_group(const W4Args& p, GroupRaw raw, int n, int g,
                                                    float magic, float unit) {
  const uint32_t i = static_cast<uint32_t>(n) * p.ng + g;
  if constexpr (UINT4) {
    GroupParams r;
    r.s = __uint_as_float((i & 1u) ? (raw.s & 0xFFFF0000u) : (raw.s << 16)) / unit;
    r.zb = magic + unit * static_cast<float>((raw.z >> ((g & 7) * 4)) & 15u);
    return r;
  }
  const uint32_t sbits = p.scale_f32 ? raw.s : ((i & 1u) ? (raw.s & 0xFFFF0000u) : (raw.s << 16));
  const bool packed = p.flags & QG_W4_ZEROS_PACKED;
  const bool sgn = p.flags & QG_W4_SIGNED_NIBBLES;
  const int z = packed ? static_cast<int>((raw.z >> ((g & 7) * 4)) & 15u) : static_cast<int>(raw.z);
  const int zu = sgn ? (packed ? (z ^ 8) : z + 8) : z;
  GroupParams r;
  r.s = __uint_as_float(sbits) / unit;
  r.zb = magic + unit * static_cast<float>(zu);
  return r;
}

__device__ __forceinline__ GroupParams group_params(const W4Args& p, int n, int g, float magic,
                                                    float unit = 1.0f) {
  return decode_group(p, load_group(p, n, g), n, g, magic, unit);
}

// ------------------------------------------------------------- skinny kernel
// Small M (decode): one workgroup of WAVES waves per 16*CT output columns x
// 16*FM rows. The K axis is cut into 128-wide chunks; wave w takes chunks
// w, w+WAVES, ... so the waves stream each weight row front to back
// together. Per chunk a lane loads, for each of its CT column tiles, its
// column's 4 words (16 bytes, one dwordx4 in the nk / group-128 layout), and
// once the activation fragments of its rows, which all CT tiles share (as
// does the MFMA against ones that yields the per-row group sums). No LDS
// staging; DEPTH chunks in flight per wave. The WAVES partial tiles are summed
// through LDS in a fixed order (deterministic).
//
// Every load is unconditional, addressed with a 32-bit byte offset from a
// wave-uniform base and clamped into its tensor: activation rows past M
// repeat row M-1 (they only reach output rows that are not stored), columns
// past N repeat column N-1, steps past K re-read the last valid words, and
// refills past a wave's last chunk re-read that chunk (a cache hit); such
// groups are computed with scale 0. Conditional loads, or branches around
// the MFMAs, would make the compiler wait for all outstanding loads (or copy
// the accumulators) at every join.
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

template <int FM, int CT, int SPC>
struct SkinnyChunk {
  uint32_t w[CT][4];
  i32x4 a[FM][4];
  GroupRaw gr[CT][SPC];
};

template <typename T>
__device__ __forceinline__ T load_at(const void* base, uint32_t byte_off) {
  return *reinterpret_cast<const T*>(static_cast<const char*>(base) + byte_off);
}
template <int FM, int CT, int G, bool KN, bool F16A, int DEPTH, int WAVES, bool UINT4>
__global__ __launch_bounds__(64 * WAVES) void k_w4_skinny(W4Args p) {
#pragma clang fp contract(off)
  constexpr int SPC = 128 / G;                  // groups per chunk
  constexpr int STEPS_PER_GROUP = 4 / SPC;
  constexpr float MAGIC = F16A ? 256.0f : 128.0f;
  constexpr float UNIT = F16A ? 4.0f : 1.0f;
  const uint32_t ones2 = F16A ? 0x3C003C00u : 0x3F803F80u;

  __shared__ float red[WAVES][FM * 16][CT * 16 + 1];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16 * CT;
  const int m0 = blockIdx.y * 16 * FM;
  int ncol[CT];
  static_for<0, CT>([&](auto t) { ncol[t] = min(n0 + 16 * t + col, p.N - 1); });
  const int C = ceil_div(p.K, 128);
  const int KW = p.K >> 3;  // words per column
  // last chunk of this wave (a wave without chunks re-reads chunk 0)
  const int clast = wave < C ? wave + WAVES * ((C - 1 - wave) / WAVES) : 0;

  uint32_t sel[4];
  unpack_selectors(p.flags & QG_W4_ORDER_HIGH, sel);
  const uint32_t wxor = (!UINT4 && (p.flags & QG_W4_SIGNED_NIBBLES)) ? 0x88888888u : 0u;
  uint32_t umask, umagic;
  unpack_consts<F16A>(umask, umagic);
  const i32x4 ones = {static_cast<int>(ones2), static_cast<int>(ones2), static_cast<int>(ones2),
                      static_cast<int>(ones2)};

  // byte offset of word kw of column n
  auto woff = [&](int n, int kw) __attribute__((always_inline)) -> uint32_t {
    return KN ? 4u * (static_cast<uint32_t>(kw) * p.N + n) : 4u * (static_cast<uint32_t>(n) * KW + kw);
  };
  uint32_t arow_off[FM];
  static_for<0, FM>([&](auto f) {
    arow_off[f] = 2u * static_cast<uint32_t>(min(m0 + 16 * f + col, p.M - 1)) * static_cast<uint32_t>(p.a_sm);
  });

  auto load = [&](SkinnyChunk<FM, CT, SPC>& ch, int c) __attribute__((always_inline)) {
    const int kw0 = c * 16;
    static_for<0, CT>([&](auto t) {
      const int n = ncol[t];
      if constexpr (!KN && G == 128) {
        const i32x4 v = load_at<i32x4>(p.w, woff(n, kw0 + 4 * q));
        static_for<0, 4>([&](auto j) { ch.w[t][j] = static_cast<uint32_t>(v[int(j)]); });
      } else if constexpr (!KN && G == 64) {
        const uint2 v0 = load_at<uint2>(p.w, woff(n, kw0 + 2 * q));
        const uint2 v1 = load_at<uint2>(p.w, woff(n, min(kw0 + 8 + 2 * q, KW - 2)));
        ch.w[t][0] = v0.x;
        ch.w[t][1] = v0.y;
        ch.w[t][2] = v1.x;
        ch.w[t][3] = v1.y;
      } else {
        static_for<0, 4>([&](auto j) {
          ch.w[t][j] = load_at<uint32_t>(p.w, woff(n, min(kw0 + word_of<G, KN>(q, j), KW - 1)));
        });
      }
      static_for<0, SPC>([&](auto g) { ch.gr[t][g] = load_group(p, n, min(c * SPC + g, p.ng - 1)); });
    });
    static_for<0, FM>([&](auto f) {
      static_for<0, 4>([&](auto j) {
        const int k = min(c * 128 + 8 * word_of<G, KN>(q, j), p.K - 8);
        ch.a[f][j] = load_at<i32x4>(p.a, arow_off[f] + 2u * k);
      });
    });
  };

  f32x4 total[CT][FM], acc[CT][FM], asum[FM];
  static_for<0, CT>([&](auto t) {
    static_for<0, FM>([&](auto f) { total[t][f] = f32x4{0, 0, 0, 0}; });
  });

  // Straight-line: all 4 steps of every scheduled chunk run on (clamped)
  // data; a group that does not exist — past K, or a refill past the wave's
  // last chunk — gets scale 0 and adds exactly 0 (inputs are finite).
  auto compute = [&](const SkinnyChunk<FM, CT, SPC>& ch, int c) __attribute__((always_inline)) {
    const bool live = c <= clast;
    static_for<0, 4>([&](auto j) {
      {
        if constexpr (j % STEPS_PER_GROUP == 0) {
          static_for<0, FM>([&](auto f) {
            asum[f] = f32x4{0, 0, 0, 0};
            static_for<0, CT>([&](auto t) { acc[t][f] = f32x4{0, 0, 0, 0}; });
          });
        }
        static_for<0, FM>([&](auto f) { asum[f] = mfma16<F16A>(ch.a[f][j], ones, asum[f]); });
        static_for<0, CT>([&](auto t) {
          const i32x4 b = unpack_word<F16A>(UINT4 ? ch.w[t][j] : ch.w[t][j] ^ wxor, sel, umask, umagic);
          static_for<0, FM>([&](auto f) { acc[t][f] = mfma16<F16A>(ch.a[f][j], b, acc[t][f]); });
        });
        if constexpr (j % STEPS_PER_GROUP == STEPS_PER_GROUP - 1) {
          constexpr int gi = j / STEPS_PER_GROUP;
          static_for<0, CT>([&](auto t) {
            GroupParams gp = decode_group<UINT4>(p, ch.gr[t][gi], ncol[t], c * SPC + gi, MAGIC, UNIT);
            if (!live || c * SPC + gi >= p.ng) gp.s = 0.0f;
            static_for<0, FM>([&](auto f) {
              static_for<0, 4>([&](auto i) {
                const float v = __builtin_fmaf(-gp.zb, asum[f][int(i)], acc[t][f][int(i)]);
                total[t][f][int(i)] = __builtin_fmaf(gp.s, v, total[t][f][int(i)]);
              });
            });
          });
        }
      }
    });
  };

  SkinnyChunk<FM, CT, SPC> buf[DEPTH];
  static_for<0, DEPTH>([&](auto d) { load(buf[d], min(wave + WAVES * d, clast)); });
  for (int base = wave; base <= clast; base += WAVES * DEPTH) {
    static_for<0, DEPTH>([&](auto d) {
      const int c = base + WAVES * d;
      compute(buf[d], c);
      load(buf[d], min(c + WAVES * DEPTH, clast));
    });
  }

  static_for<0, CT>([&](auto t) {
    static_for<0, FM>([&](auto f) {
      static_for<0, 4>([&](auto i) { red[wave][16 * f + 4 * q + i][16 * t + col] = total[t][f][int(i)]; });
    });
  });
  __syncthreads();
  for (int e = threadIdx.x; e < FM * CT * 256; e += 64 * WAVES) {
    const int r = e / (16 * CT), cc = e % (16 * CT);
    const int row = m0 + r, nn = n0 + cc;
    if (row < p.M && nn < p.N) {
      float v = red[0][r][cc];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) v = v + red[w][r][cc];
      if (p.bias) v = v + load_bias(p.bias, p.bias_dtype, nn);
      store_out(p.out, p.out_dtype, static_cast<int64_t>(row) * p.N + nn, v);
    }
  }
}

// ------------------------------------------------------------- decode kernel
// M <= 16 (token decode), the HBM-bound shape. One workgroup of WAVES waves
// per 16*CT output columns; wave w owns a contiguous range of 128-wide K
// chunks (at most CH, 4 or 8). At the start each wave copies its
// activation slice [rows, 128 * chunks] into its own LDS region (one 16-byte
// load and one 16-byte LDS store per lane per row and 512 K), storing every
// 8-element group in the order (0 2 4 6 1 3 5 7). In that order a weight
// word needs only 7 VALU operations to become 4 MFMA registers:
//   E = even nibbles as bytes, O = odd nibbles as bytes (one AND, one
//   shift+AND), then 4 v_perm_b32 that pair two nibble bytes with the
//   exponent byte of the magic number (bf16 0x43.. = 128 + u, fp16 0x5C.. =
//   256 + 4u with the nibble placed in bits 4-7).
// The activation fragments (ds_read_b128) and the MFMA against ones that
// yields the row sums per group are shared by the CT column tiles. All
// weight, scale and zero-point loads of a wave are issued before its first
// MFMA (the chunk range is at most CH long), unconditionally and
// clamped as in the skinny kernel; the WAVES partial tiles are summed through
// LDS in a fixed order.
constexpr int kDecodeChunks = 4;  // chunks per wave with 8 waves (K <= 4096)

template <bool F16A, bool UINT4>
struct Unpack7 {
  uint32_t mask_e, magic4, sel_a, sel_b, sh_e, sh_o;
  __device__ __forceinline__ void init(bool high) {
    mask_e = F16A ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    magic4 = F16A ? 0x5C5C5C5Cu : 0x43434343u;
    // result bytes (low to high): nibble byte, magic, nibble byte, magic;
    // combined source bytes 0-3 = E or O, 4-7 = magic. High order keeps the
    // nibbles of each word in reverse, so its selectors read bytes 3..0 and
    // the even / odd roles of the two nibbles of a byte swap.
    sel_a = high ? 0x04020403u : 0x04010400u;
    sel_b = high ? 0x04000401u : 0x04030402u;
    // E = nibbles 0,2,4,6 and O = nibbles 1,3,5,7, each moved to the
    // nibble position of its byte that the magic expects (bits 0-3 for bf16,
    // 4-7 for fp16)
    const uint32_t s_lo = F16A ? 4u : 0u, s_hi = F16A ? 0u : 4u;
    sh_e = high ? s_hi : s_lo;
    sh_o = high ? s_lo : s_hi;
    asm volatile("" : "+v"(mask_e), "+s"(magic4), "+s"(sel_a), "+s"(sel_b), "+s"(sh_e), "+s"(sh_o));
  }
  __device__ __forceinline__ uint32_t shifted(uint32_t w, uint32_t sh, bool lo_role) const {
    // bf16: bits 0-3 <- (w >> sh); fp16: bits 4-7 <- (w << sh)
    return F16A ? (w << sh) : (w >> sh);
  }
  __device__ __forceinline__ i32x4 operator()(uint32_t w) const {
    uint32_t e, o;
    if constexpr (UINT4) {  // low order known at compile time
      e = F16A ? (w << 4) & mask_e : w & mask_e;
      o = F16A ? w & mask_e : (w >> 4) & mask_e;
    } else {
      e = shifted(w, sh_e, true) & mask_e;
      o = shifted(w, sh_o, false) & mask_e;
    }
    i32x4 r;
    r[0] = static_cast<int>(__builtin_amdgcn_perm(magic4, e, sel_a));
    r[1] = static_cast<int>(__builtin_amdgcn_perm(magic4, e, sel_b));
    r[2] = static_cast<int>(__builtin_amdgcn_perm(magic4, o, sel_a));
    r[3] = static_cast<int>(__builtin_amdgcn_perm(magic4, o, sel_b));
    return r;
  }
};

// 8 consecutive 16-bit activations (4 registers) -> order (0 2 4 6 1 3 5 7).
__device__ __forceinline__ i32x4 even_odd(const i32x4& v) {
  i32x4 r;
  r[0] = static_cast<int>(__builtin_amdgcn_perm(v[1], v[0], 0x05040100u));
  r[1] = static_cast<int>(__builtin_amdgcn_perm(v[3], v[2], 0x05040100u));
  r[2] = static_cast<int>(__builtin_amdgcn_perm(v[1], v[0], 0x07060302u));
  r[3] = static_cast<int>(__builtin_amdgcn_perm(v[3], v[2], 0x07060302u));
  return r;
}

template <int CT, int SPC, bool UINT4>
struct DecodeChunk {
  uint32_t w[CT][4];
  GroupRaw gr[CT][UINT4 ? 1 : SPC];  // UINT4: scales / zero points come in one batch
};

// RP: activation rows held per slab (1, 4 or 16; rows past M repeat row M-1).
// CH: 128-wide K chunks per wave (4 or 8).
template <int RP, int CT, int G, bool KN, bool F16A, int WAVES, bool UINT4, int CH>
__global__ __launch_bounds__(64 * WAVES) void k_w4_decode(W4Args p) {
#pragma clang fp contract(off)
  constexpr int SPC = 128 / G;                  // groups per chunk
  constexpr int STEPS_PER_GROUP = 4 / SPC;
  static_assert(CH == 4 || CH == 8, "chunks per wave");
  constexpr int ROWB = CH * 128 * 2 + 16;       // LDS bytes per activation row (padded)
  constexpr float MAGIC = F16A ? 256.0f : 128.0f;
  constexpr float UNIT = F16A ? 4.0f : 1.0f;
  const uint32_t ones2 = F16A ? 0x3C003C00u : 0x3F803F80u;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16 * CT;
  const int m0 = blockIdx.y * RP;
  int ncol[CT];
  static_for<0, CT>([&](auto t) { ncol[t] = min(n0 + 16 * t + col, p.N - 1); });
  const int C = ceil_div(p.K, 128);
  const int KW = p.K >> 3;
  const int cpw = ceil_div(C, WAVES);           // <= CH (checked by the launcher)
  const int c0 = min(wave * cpw, C - 1);
  const int nch = max(0, min(cpw, C - wave * cpw));  // chunks of this wave

  Unpack7<F16A, UINT4> unpack;
  unpack.init(!UINT4 && (p.flags & QG_W4_ORDER_HIGH));
  // signed storage: q & 15 with q in [-8, 7] -> unsigned u = q + 8 = nibble ^ 8
  const uint32_t wxor = (!UINT4 && (p.flags & QG_W4_SIGNED_NIBBLES)) ? 0x88888888u : 0u;
  const i32x4 ones = {static_cast<int>(ones2), static_cast<int>(ones2), static_cast<int>(ones2),
                      static_cast<int>(ones2)};
  auto woff = [&](int n, int kw) __attribute__((always_inline)) -> uint32_t {
    return KN ? 4u * (static_cast<uint32_t>(kw) * p.N + n) : 4u * (static_cast<uint32_t>(n) * KW + kw);
  };

  // ---- 1. this wave's activation slice (issued first: it is needed first):
  // CH 128-wide chunks = CH / 4 16-byte loads per lane and row
  constexpr int AV = CH / 4;
  i32x4 av[RP][AV];
  static_for<0, AV>([&](auto h) {
    const int k = min(c0 * 128 + 512 * h + 8 * lane, p.K - 8);
    static_for<0, RP>([&](auto r) {
      const uint32_t roff = 2u * static_cast<uint32_t>(min(m0 + r, p.M - 1)) * static_cast<uint32_t>(p.a_sm);
      av[r][h] = load_at<i32x4>(p.a, roff + 2u * k);
    });
  });

  // ---- 2. every weight / scale / zero load of this wave, in chunk order ----
  // UINT4 (group 128: chunk c is group c; launcher: CH chunks per wave and
  // ng % CH == 0): the wave's CH groups start at a multiple of CH, so CH / 4
  // 8-byte loads hold their bf16 scales and one word their zero points
  // (nibbles 4 * (g0 % 8) + 4 cl). Waves past K read an aligned in-range set.
  uint2 s4[CT][CH / 4];
  uint32_t z8[CT];
  const int g0 = min(c0, (p.ng - 1) & ~(CH - 1));
  if constexpr (UINT4) {
    static_for<0, CT>([&](auto t) {
      static_for<0, CH / 4>([&](auto h) {
        s4[t][h] = load_at<uint2>(p.scales, 2u * (static_cast<uint32_t>(ncol[t]) * p.ng + g0 + 4 * h));
      });
      z8[t] = load_at<uint32_t>(p.zeros, 4u * (static_cast<uint32_t>(ncol[t]) * p.zw + (g0 >> 3)));
    });
  }
  DecodeChunk<CT, SPC, UINT4> ch[CH];
  static_for<0, CH>([&](auto cl) {
    const int c = min(c0 + cl, C - 1);
    const int kw0 = c * 16;
    static_for<0, CT>([&](auto t) {
      const int n = ncol[t];
      if constexpr (!KN && G == 128) {
        const i32x4 v = load_at<i32x4>(p.w, woff(n, kw0 + 4 * q));
        static_for<0, 4>([&](auto j) { ch[cl].w[t][j] = static_cast<uint32_t>(v[int(j)]); });
      } else if constexpr (!KN && G == 64) {
        const uint2 v0 = load_at<uint2>(p.w, woff(n, kw0 + 2 * q));
        const uint2 v1 = load_at<uint2>(p.w, woff(n, min(kw0 + 8 + 2 * q, KW - 2)));
        ch[cl].w[t][0] = v0.x;
        ch[cl].w[t][1] = v0.y;
        ch[cl].w[t][2] = v1.x;
        ch[cl].w[t][3] = v1.y;
      } else {
        static_for<0, 4>([&](auto j) {
          ch[cl].w[t][j] = load_at<uint32_t>(p.w, woff(n, min(kw0 + word_of<G, KN>(q, j), KW - 1)));
        });
      }
      if constexpr (!UINT4)
        static_for<0, SPC>([&](auto g) { ch[cl].gr[t][g] = load_group(p, n, min(c * SPC + g, p.ng - 1)); });
    });
  });

  // keep every load above this point: the scheduler would otherwise sink
  // them next to their first use to save registers and serialise the latency
  __builtin_amdgcn_sched_barrier(0);

  // ---- 3. activations -> this wave's LDS rows, even/odd order --------------
  char* const abase = smem + wave * RP * ROWB;
  static_for<0, RP>([&](auto r) {
    static_for<0, AV>([&](auto h) {
      *reinterpret_cast<i32x4*>(abase + r * ROWB + 1024 * h + 16 * lane) = even_odd(av[r][h]);
    });
  });

  f32x4 total[CT], acc[CT], asum;
  static_for<0, CT>([&](auto t) { total[t] = f32x4{0, 0, 0, 0}; });
  const char* const arow = abase + min(col, RP - 1) * ROWB;
  // accumulator registers that hold real rows: all 4 for RP >= 4, only
  // register 0 (row 0, lanes 0-15) for a single activation row
  constexpr int NI = RP == 1 ? 1 : 4;

  // UINT4: decode the wave's group scales / zero points once
  float gs[CT][CH], gz[CT][CH];
  if constexpr (UINT4) {
    static_for<0, CT>([&](auto t) {
      const uint32_t zs = z8[t] >> (4 * (g0 & 7));
      static_for<0, CH>([&](auto cl) {
        const uint32_t sw = ((cl >> 1) & 1) ? s4[t][cl >> 2].y : s4[t][cl >> 2].x;
        gs[t][cl] = __uint_as_float((cl & 1) ? (sw & 0xFFFF0000u) : (sw << 16)) / UNIT;
        if (cl >= nch) gs[t][cl] = 0.0f;
        gz[t][cl] = MAGIC + UNIT * static_cast<float>((zs >> (4 * cl)) & 15u);
      });
    });
  }

  // ---- 4. chunks in order, each as soon as its loads have landed -----------
  static_for<0, CH>([&](auto cl) {
    const int c = c0 + cl;
    const bool live = cl < nch;
    static_for<0, 4>([&](auto j) {
      if constexpr (j % STEPS_PER_GROUP == 0) {
        asum = f32x4{0, 0, 0, 0};
        static_for<0, CT>([&](auto t) { acc[t] = f32x4{0, 0, 0, 0}; });
      }
      const i32x4 af = *reinterpret_cast<const i32x4*>(arow + 2 * (cl * 128 + 8 * word_of<G, KN>(q, j)));
      asum = mfma16<F16A>(af, ones, asum);
      static_for<0, CT>([&](auto t) {
        acc[t] = mfma16<F16A>(af, unpack(UINT4 ? ch[cl].w[t][j] : ch[cl].w[t][j] ^ wxor), acc[t]);
      });
      if constexpr (j % STEPS_PER_GROUP == STEPS_PER_GROUP - 1) {
        constexpr int gi = j / STEPS_PER_GROUP;
        static_for<0, CT>([&](auto t) {
          GroupParams gp;
          if constexpr (UINT4) {
            gp.s = gs[t][cl];
            gp.zb = gz[t][cl];
          } else {
            gp = decode_group<false>(p, ch[cl].gr[t][gi], ncol[t], c * SPC + gi, MAGIC, UNIT);
            if (!live || c * SPC + gi >= p.ng) gp.s = 0.0f;
          }
          static_for<0, NI>([&](auto i) {
            const float v = __builtin_fmaf(-gp.zb, asum[int(i)], acc[t][int(i)]);
            total[t][int(i)] = __builtin_fmaf(gp.s, v, total[t][int(i)]);
          });
        });
      }
    });
  });

  // ---- 5. fixed-order reduction of the WAVES partial tiles -----------------
  __syncthreads();  // every wave is done with its activation slice
  float* red = reinterpret_cast<float*>(smem);  // [WAVES][16][16*CT + 1]
  constexpr int RS = 16 * CT + 1;
  static_for<0, CT>([&](auto t) {
    static_for<0, 4>([&](auto i) { red[(wave * 16 + 4 * q + i) * RS + 16 * t + col] = total[t][int(i)]; });
  });
  __syncthreads();
  for (int e = threadIdx.x; e < RP * 16 * CT; e += 64 * WAVES) {
    const int r = e / (16 * CT), cc = e % (16 * CT);
    const int row = m0 + r, nn = n0 + cc;
    if (row < p.M && nn < p.N) {
      float v = red[r * RS + cc];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) v = v + red[(w * 16 + r) * RS + cc];
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
// (_unpack_weight, int4_weight_gemm_v07.py:136-151). One thread per 4 packed
// words of a column (32 K elements: K and the group are multiples of 32, so
// they share one group): the scale and zero point are read once and the 32
// outputs leave as 8- to 32-byte stores (element stores when `vec` is 0, an
// output base that does not allow them). Threads walk the quads in storage
// order (n fastest for the kn layout), so word loads are coalesced.
// One packed word: 8 K values of a column, centred (u - zero point) and, for
// floating outputs, scaled (exact fp32 product, one rounding to the output).
template <int OUT>
__device__ __forceinline__ void unpack_word_store(uint32_t word, bool high, bool sgn, int zu, float s, void* out,
                                                  int64_t o0, int vec) {
  if (sgn) word ^= 0x88888888u;  // q & 15 with q in [-8, 7] -> u = q + 8
  int cen[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) cen[e] = static_cast<int>((word >> (high ? 28 - 4 * e : 4 * e)) & 15u) - zu;
  if constexpr (OUT == QG_I8) {
    uint32_t b[2] = {0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e >> 2] |= (static_cast<uint32_t>(cen[e]) & 0xffu) << (8 * (e & 3));
    int8_t* o = static_cast<int8_t*>(out) + o0;
    if (vec) *reinterpret_cast<uint2*>(o) = make_uint2(b[0], b[1]);
    else for (int e = 0; e < 8; ++e) o[e] = static_cast<int8_t>(cen[e]);
  } else if constexpr (OUT == QG_F32) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = static_cast<float>(cen[e]) * s;
    float* o = static_cast<float*>(out) + o0;
    if (vec) {
      reinterpret_cast<float4*>(o)[0] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4*>(o)[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      for (int e = 0; e < 8; ++e) o[e] = v[e];
    }
  } else {
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float a = static_cast<float>(cen[e]) * s, b = static_cast<float>(cen[e + 1]) * s;
      if constexpr (OUT == QG_F16) h[e >> 1] = f32_to_f16(a) | (static_cast<uint32_t>(f32_to_f16(b)) << 16);
      else h[e >> 1] = f32x2_to_bf16x2(a, b);
    }
    uint16_t* o = static_cast<uint16_t*>(out) + o0;
    if (vec) *reinterpret_cast<uint4*>(o) = make_uint4(h[0], h[1], h[2], h[3]);
    else for (int e = 0; e < 8; ++e) o[e] = static_cast<uint16_t>(h[e >> 1] >> (16 * (e & 1)));
  }
}

// kn layout: one thread per 4 packed words of a column (32 consecutive K, one
// group lookup), 64 contiguous output bytes per thread.
template <int OUT>
__global__ __launch_bounds__(256) void k_w4_unpack(W4Args p, int vec) {
  const int KW = p.K >> 3, KQ = KW >> 2;  // words and word quads per column
  const int quads = p.N * KQ;              // < 2^28 (N K < 2^31)
  const bool kn = p.flags & QG_W4_LAYOUT_KN;
  const bool sgn = p.flags & QG_W4_SIGNED_NIBBLES;
  const bool high = p.flags & QG_W4_ORDER_HIGH;
  for (int qi = blockIdx.x * blockDim.x + threadIdx.x; qi < quads; qi += gridDim.x * blockDim.x) {
    int n, kq;
    if (kn) {
      kq = qi / p.N;
      n = qi - kq * p.N;
    } else {
      n = qi / KQ;
      kq = qi - n * KQ;
    }
    const int kw0 = 4 * kq;
    uint32_t word[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      word[j] = p.w[kn ? static_cast<int64_t>(kw0 + j) * p.N + n : static_cast<int64_t>(n) * KW + kw0 + j];
    const GroupParams gp = group_params(p, n, (8 * kw0) / p.group, 0.0f);
    const int64_t base = static_cast<int64_t>(n) * p.K + 8 * kw0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      unpack_word_store<OUT>(word[j], high, sgn, static_cast<int>(gp.zb), gp.s, p.out, base + 8 * j, vec);
  }
}

// nk layout: a wave takes 256 consecutive packed words and lane l words
// base + 64 j + l (j < 4), so each load (4 bytes per lane) and each store (8
// values per lane) of the wave is contiguous, with four loads in flight per
// lane. Word i of the weight holds K values [8 i, 8 i + 8) of the output's flat
// [N, K] order; its group's scale and zero point come from the small scale /
// zero arrays (cache hits).
template <int OUT>
__global__ __launch_bounds__(256) void k_w4_unpack_nk(W4Args p, int vec) {
  const int KW = p.K >> 3;
  const int words = p.N * KW;  // < 2^28 (N K < 2^31)
  const bool sgn = p.flags & QG_W4_SIGNED_NIBBLES;
  const bool high = p.flags & QG_W4_ORDER_HIGH;
  const int lane = threadIdx.x & 63;
  for (int base = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 256; base < words; base += gridDim.x * 1024) {
    const int w0 = base + lane;
    uint32_t word[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) word[j] = p.w[min(w0 + 64 * j, words - 1)];
    int n = w0 / KW, kw = w0 - n * KW;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int wi = w0 + 64 * j;
      if (wi < words) {
        const GroupParams gp = group_params(p, n, (8 * kw) / p.group, 0.0f);
        unpack_word_store<OUT>(word[j], high, sgn, static_cast<int>(gp.zb), gp.s, p.out, 8 * static_cast<int64_t>(wi),
                               vec);
      }
      kw += 64;
      while (kw >= KW) {
        kw -= KW;
        ++n;
      }
    }
  }
}

template <int FM, int CT, int G, bool KN, bool F16A>
hipError_t launch_skinny_t(const W4Args& p, hipStream_t stream) {
  // chunks in flight per wave; groups of 64 / 32 hold 2 / 4 scale and zero
  // words per column and chunk, so they keep half as many (no spills)
  constexpr int DEPTH = G == 128 ? ((FM * CT <= 2) ? 4 : 2) : ((FM * CT <= 2) ? 2 : 1);
  constexpr int WAVES = 8;
  dim3 grid(ceil_div(p.N, 16 * CT), ceil_div(p.M, 16 * FM));
  constexpr int kUint4Flags = QG_W4_ZEROS_PACKED;
  if (G == 128 && !KN && !p.scale_f32 && p.flags == kUint4Flags)
    hipLaunchKernelGGL((k_w4_skinny<FM, CT, G, KN, F16A, DEPTH, WAVES, (G == 128 && !KN)>), grid,
                       dim3(64 * WAVES), 0, stream, p);
  else
    hipLaunchKernelGGL((k_w4_skinny<FM, CT, G, KN, F16A, DEPTH, WAVES, false>), grid, dim3(64 * WAVES), 0,
                       stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Single-row W4A16 decode (M = 1) on the benchmark's uint4 storage: unsigned
// nibbles, low order, [N, K/8] words, bf16 scales, packed uint4 zero points,
// group 128, bf16 activations, K a multiple of 512 up to 4096.
//
// Workgroup = 32 columns (n0 = 32 b), 8 waves; wave w owns K range
// [512 w, 512 w + 512) (groups 4 w .. 4 w + 3) of all 32 columns. Every
// operand reaches LDS by direct global -> LDS copies issued at the start
// (nothing else is in flight, so the waits are exact vmcnt counts):
//   activations  the wave's 512 values (1 KB), then reordered in place to
//                (0 2 4 6 1 3 5 7) per 8 for the 7-op nibble unpack;
//   scales       8 B per column (groups 4 w .. 4 w + 3), one 4-byte copy per lane;
//   zero points  the packed word holding those groups, lanes 0-31;
//   weights      8 non-temporal copies (each byte is read once per call) of
//                4 columns x 256 B (two whole cache lines per column): copy
//                i, lane L lands in 16-byte slot 64 i + L =
//                c * 16 + (k ^ (c & 14)), c = 4 i + L / 16 the local column and
//                k the 16-byte chunk of its 256 B. The XOR makes the MFMA-layout
//                reads below (lane (col, q) -> chunk 4 g + q of column col)
//                hit distinct banks for each group of 32 lanes.
// Columns 0-15 (copies 0-3) are computed while columns 16-31 still arrive.
// Per group g: v_mfma_f32_16x16x32_bf16 of the activations (A, all 16 rows
// the same vector) with 128 + u (B, exact bf16), plus one MFMA against ones
// for the group's activation sum; y += s (acc - (128 + z) sum) in fp32. The 8
// waves' partial columns are summed through LDS in wave order.
constexpr int kGemv1Region = 8192 + 1024 + 256 + 128;  // LDS bytes per wave
constexpr int kGemv1Lds = 8 * kGemv1Region + 8 * 32 * 4;

__global__ __launch_bounds__(512) void k_w4_gemv1(W4Args p) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(1024))) char smem[kGemv1Lds];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 32;
  const bool live = 512 * wave < p.K;  // waves past K contribute zero
  char* const region = smem + wave * kGemv1Region;
  char* const wt = region;             // weights, 32 columns x 256 B
  char* const at = region + 8192;      // activations, 512 bf16
  char* const st = region + 9216;      // scales [column][4] bf16
  char* const zt = region + 9472;      // zero-point words [column]
  float total[2] = {0.0f, 0.0f};
  if (live) {
    const int KW = p.K >> 3;
    dma16s(p.a, 1024u * wave + 16u * lane, lds_addr_of(at));
    {
      const int c = min(n0 + (lane >> 1), p.N - 1);
      dma4s(p.scales, 2u * (static_cast<uint32_t>(c) * p.ng + 4 * wave) + 4u * (lane & 1), lds_addr_of(st));
    }
    if (lane < 32) {
      const int c = min(n0 + lane, p.N - 1);
      dma4s(p.zeros, 4u * (static_cast<uint32_t>(c) * p.zw + (wave >> 1)), lds_addr_of(zt));
    }
    static_for<0, 8>([&](auto i) {
      const int c = 4 * i + (lane >> 4);
      const int k = (lane & 15) ^ (c & 14);
      const int n = min(n0 + c, p.N - 1);
      dma16s_nt(p.w, 4u * (static_cast<uint32_t>(n) * KW + 64 * wave + 4 * k), lds_addr_of(wt + 1024 * i));
    });
    wait_vm<8>();  // activations, scales, zero points (the 8 weight copies may fly)
    {
      char* const a16 = at + 16 * lane;
      *reinterpret_cast<i32x4*>(a16) = even_odd(*reinterpret_cast<const i32x4*>(a16));
    }
    const int col = lane & 15, q = lane >> 4;
    Unpack7<false, true> unpack;
    unpack.init(false);
    uint32_t ones2 = 0x3F803F80u;  // bf16 (1, 1)
    asm volatile("" : "+v"(ones2));
    const i32x4 ones = {static_cast<int>(ones2), static_cast<int>(ones2), static_cast<int>(ones2),
                        static_cast<int>(ones2)};
    // activation sums of the wave's 4 groups (column independent)
    f32x4 asum[4];
    static_for<0, 4>([&](auto g) {
      asum[g] = f32x4{0, 0, 0, 0};
      static_for<0, 4>([&](auto j) {
        const i32x4 af = *reinterpret_cast<const i32x4*>(at + 2 * (128 * g + 32 * q + 8 * j));
        asum[g] = mfma16<false>(af, ones, asum[g]);
      });
    });
    static_for<0, 2>([&](auto t) {
      if constexpr (t == 0) wait_vm<4>();
      else wait_vm<0>();
      const int c = 16 * t + col;
      const uint32_t zword = *reinterpret_cast<const uint32_t*>(zt + 4 * c) >> (16 * (wave & 1));
      static_for<0, 4>([&](auto g) {
        const int k = 4 * g + q;
        const i32x4 wv = *reinterpret_cast<const i32x4*>(wt + 16 * (c * 16 + (k ^ (c & 14))));
        f32x4 acc = {0, 0, 0, 0};
        static_for<0, 4>([&](auto j) {
          const i32x4 af = *reinterpret_cast<const i32x4*>(at + 2 * (128 * g + 32 * q + 8 * j));
          acc = mfma16<false>(af, unpack(static_cast<uint32_t>(wv[int(j)])), acc);
        });
        const float s = bf16_to_f32(*reinterpret_cast<const uint16_t*>(st + 8 * c + 2 * g));
        const float zb = 128.0f + static_cast<float>((zword >> (4 * g)) & 15u);
        total[t] = __builtin_fmaf(s, __builtin_fmaf(-zb, asum[g][0], acc[0]), total[t]);
      });
    });
  }
  // ---- partial columns of the 8 waves (row 0 sits in lanes 0-15, register 0)
  float* red = reinterpret_cast<float*>(smem + 8 * kGemv1Region);
  if (lane < 16) {
    red[wave * 32 + lane] = total[0];
    red[wave * 32 + 16 + lane] = total[1];
  }
  __syncthreads();
  if (threadIdx.x < 32) {
    float v = red[threadIdx.x];
#pragma unroll
    for (int w = 1; w < 8; ++w) v = v + red[w * 32 + threadIdx.x];
    const int n = n0 + threadIdx.x;
    if (n < p.N) {
      if (p.bias) v = v + load_bias(p.bias, p.bias_dtype, n);
      store_out(p.out, p.out_dtype, n, v);
    }
  }
}

// The single-row kernel's operand contract (see k_w4_gemv1).
bool gemv1_applies(const W4Args& p) {
  const uintptr_t align = reinterpret_cast<uintptr_t>(p.w) | reinterpret_cast<uintptr_t>(p.a);
  return p.M == 1 && !p.a_f16 && p.group == 128 && !p.scale_f32 && p.flags == QG_W4_ZEROS_PACKED &&
         p.K % 512 == 0 && p.K <= 4096 && (align & 15) == 0 &&
         ((reinterpret_cast<uintptr_t>(p.scales) | reinterpret_cast<uintptr_t>(p.zeros)) & 3) == 0;
}

template <int FM, int CT, bool F16A>
hipError_t launch_skinny_g(const W4Args& p, hipStream_t stream) {
  const bool kn = p.flags & QG_W4_LAYOUT_KN;
  switch (p.group) {
    case 128: return kn ? launch_skinny_t<FM, CT, 128, true, F16A>(p, stream) : launch_skinny_t<FM, CT, 128, false, F16A>(p, stream);
    case 64: return kn ? launch_skinny_t<FM, CT, 64, true, F16A>(p, stream) : launch_skinny_t<FM, CT, 64, false, F16A>(p, stream);
    default: return kn ? launch_skinny_t<FM, CT, 32, true, F16A>(p, stream) : launch_skinny_t<FM, CT, 32, false, F16A>(p, stream);
  }
}

template <int RP, int CT, int G, bool KN, bool F16A, bool UINT4, int WAVES = 8, int CH = kDecodeChunks>
hipError_t launch_decode_t(const W4Args& p, hipStream_t stream) {
  const size_t a_bytes = static_cast<size_t>(WAVES) * RP * (CH * 256 + 16);
  const size_t red_bytes = static_cast<size_t>(WAVES) * 16 * (16 * CT + 1) * 4;
  const size_t lds = a_bytes > red_bytes ? a_bytes : red_bytes;
  dim3 grid(ceil_div(p.N, 16 * CT), ceil_div(p.M, RP));
  hipLaunchKernelGGL((k_w4_decode<RP, CT, G, KN, F16A, WAVES, UINT4, CH>), grid, dim3(64 * WAVES), lds, stream, p);
  return hipGetLastError();
}

template <int RP, int CT, bool F16A>
hipError_t launch_decode_g(const W4Args& p, hipStream_t stream) {
  const bool kn = p.flags & QG_W4_LAYOUT_KN;
  switch (p.group) {
    case 128: {
      const int cpw = ceil_div(ceil_div(p.K, 128), 8);
      if (!kn && !p.scale_f32 && p.flags == QG_W4_ZEROS_PACKED && p.ng % 4 == 0 && cpw == kDecodeChunks)
        return launch_decode_t<RP, CT, 128, false, F16A, true>(p, stream);
      return kn ? launch_decode_t<RP, CT, 128, true, F16A, false>(p, stream)
                : launch_decode_t<RP, CT, 128, false, F16A, false>(p, stream);
    }
    case 64:
      return kn ? launch_decode_t<RP, 2, 64, true, F16A, false>(p, stream)
                : launch_decode_t<RP, 2, 64, false, F16A, false>(p, stream);
    default:  // group 32: one column tile per wave past one row (4 scale / zero words per chunk)
      return kn ? launch_decode_t<RP, (RP > 1 ? 1 : 2), 32, true, F16A, false>(p, stream)
                : launch_decode_t<RP, (RP > 1 ? 1 : 2), 32, false, F16A, false>(p, stream);
  }
}

template <bool F16A>
hipError_t launch_skinny(const W4Args& p, hipStream_t stream) {
  const int C = ceil_div(p.K, 128);
  if (p.M <= 16 && ceil_div(C, 8) <= kDecodeChunks) {
    // column tiles of 16 per workgroup, all sharing each activation fragment:
    // two for 1-4 rows (cfg2, 448 workgroups: 2-4 rows 9.5-9.7 us against
    // 10.0-10.1 us with four), four for 5-16 rows (11.2-11.4 us against 12.9 us
    // with two)
    if (p.M == 1) {
      if (gemv1_applies(p)) {
        hipLaunchKernelGGL(k_w4_gemv1, dim3(ceil_div(p.N, 32)), dim3(512), 0, stream, p);
        return hipGetLastError();
      }
      return launch_decode_g<1, 2, F16A>(p, stream);
    }
    if (p.M <= 4) return launch_decode_g<4, 2, F16A>(p, stream);
    return launch_decode_g<16, 4, F16A>(p, stream);
  }
  if (p.M <= 16) return launch_skinny_g<1, 4, F16A>(p, stream);
  if (p.M <= 32) return launch_skinny_g<2, 1, F16A>(p, stream);
  return launch_skinny_g<4, 1, F16A>(p, stream);
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
  const int64_t quads = static_cast<int64_t>(p.N) * (p.K / 32);  // K % 32 == 0 (group multiple)
  if (quads == 0) return hipSuccess;
  int64_t blocks = ceil_div<int64_t>(quads, 256);
  if (blocks > 65536) blocks = 65536;
  const int es = p.out_dtype == QG_I8 ? 1 : p.out_dtype == QG_F32 ? 4 : 2;
  const int vec = (reinterpret_cast<uintptr_t>(p.out) % (8 * es)) == 0 ? 1 : 0;  // rows of K % 32 == 0
  const dim3 grid(static_cast<unsigned>(blocks));
  if (!(p.flags & QG_W4_LAYOUT_KN)) {
    int64_t wblocks = ceil_div<int64_t>(quads * 4, 1024);  // 256 words per wave, 4 waves
    const dim3 wgrid(static_cast<unsigned>(wblocks < 65536 ? wblocks : 65536));
    switch (p.out_dtype) {
      case QG_I8: hipLaunchKernelGGL(k_w4_unpack_nk<QG_I8>, wgrid, dim3(256), 0, stream, p, vec); break;
      case QG_F32: hipLaunchKernelGGL(k_w4_unpack_nk<QG_F32>, wgrid, dim3(256), 0, stream, p, vec); break;
      case QG_F16: hipLaunchKernelGGL(k_w4_unpack_nk<QG_F16>, wgrid, dim3(256), 0, stream, p, vec); break;
      default: hipLaunchKernelGGL(k_w4_unpack_nk<QG_BF16>, wgrid, dim3(256), 0, stream, p, vec); break;
    }
    return hipGetLastError();
  }
  switch (p.out_dtype) {
    case QG_I8: hipLaunchKernelGGL(k_w4_unpack<QG_I8>, grid, dim3(256), 0, stream, p, vec); break;
    case QG_F32: hipLaunchKernelGGL(k_w4_unpack<QG_F32>, grid, dim3(256), 0, stream, p, vec); break;
    case QG_F16: hipLaunchKernelGGL(k_w4_unpack<QG_F16>, grid, dim3(256), 0, stream, p, vec); break;
    default: hipLaunchKernelGGL(k_w4_unpack<QG_BF16>, grid, dim3(256), 0, stream, p, vec); break;
  }
  return hipGetLastError();
}

// Plain read floor: the bytes are split evenly over the waves of a grid of
// four 512-thread workgroups per CU; each wave reads its contiguous share as
// whole 1 KB non-temporal requests (16 bytes per lane; 6.03 against 6.31-6.34
// us without the hint for the cfg2 weight bytes), 4 issued back to back per round,
// folds them into one word and stores it only if it equals a constant (so the
// loads stay live). Of the shapes measured for a 30.5 MB read on MI355X (256
// to 4096 workgroups of 4 to 16 waves, 4 to 16 requests per round, register
// loads and direct-to-LDS copies, all without the hint), this one and its
// neighbours were the fastest (6.2-6.3 us); two workgroups per CU with 8
// requests per round, the shape of the W4A16 decode, took 6.8 us.
__global__ __launch_bounds__(512) void k_read_floor(const char* src, uint64_t bytes, uint64_t share,
                                                    uint32_t* sink) {
  constexpr int LPW = 4;
  const int lane = threadIdx.x & 63;
  const uint64_t wave = static_cast<uint64_t>(blockIdx.x) * 8 + (threadIdx.x >> 6);
  const uint64_t start = wave * share;
  const uint64_t end = start + share < bytes ? start + share : bytes;
  int x = 0;
  for (uint64_t o = start; o < end; o += LPW * 1024) {
    i32x4 v[LPW];
    static_for<0, LPW>([&](auto i) {
      const uint64_t off = o + 1024u * decltype(i)::value + 16u * lane;
      v[i] = off < end ? __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(src + off)) : i32x4{0, 0, 0, 0};
    });
    static_for<0, LPW>([&](auto i) { x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3]; });
  }
  if (x == 0x5eed1e55) sink[0] = static_cast<uint32_t>(x);
}

hipError_t launch_read_floor(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream) {
  constexpr uint64_t kWaves = 4 * 256 * 8;  // four workgroups of 8 waves per CU
  const uint64_t share = ((bytes + kWaves - 1) / kWaves + 1023) / 1024 * 1024;
  const uint64_t waves = (bytes + share - 1) / share;
  hipLaunchKernelGGL(k_read_floor, dim3(static_cast<unsigned>((waves + 7) / 8)), dim3(512), 0, stream,
                     static_cast<const char*>(src), static_cast<uint64_t>(bytes), share, sink);
  return hipGetLastError();
}

}  // namespace qg
