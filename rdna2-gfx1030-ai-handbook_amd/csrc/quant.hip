// Per-row dynamic INT8 quantizer and the strided int8 row packer.
//
// quant: one row per workgroup of NW waves (absmax: a wave reduction, then one
// LDS exchange across the waves).
//   step = max(absmax / 127, 1e-20)          (IEEE fp32 division)
//   q = clamp(round(x / step), -127, 127)    (round of the IEEE quotient)
// Rows of up to 8 waves x 64 lanes x 6 16-byte chunks (24576 fp16) are loaded
// into registers once, all loads in flight together, and quantized from there.
// NW is the smallest of 1, 2, 4, 8 that leaves at most 3 chunks per lane and NCH
// the chunks per lane the row needs: the row's loads are spread over more
// waves (more requests in flight per CU, shorter per-wave chains) — 25 us
// instead of 34 us for 4096 x 12288 fp16. The quotient is
// formed as x * rcp(step) (a few ulps from x / step); only when that lands
// within 2^-12 of a rounding boundary (n + 1/2) is the IEEE division done, so
// the rounded result is always that of the exact quotient. Longer or strided
// rows take a two-pass kernel (pass 2 re-reads the row from L2).
// The step formula and the half-away rounding follow the reference's
// in-tree quantizer rdna2-ops/rdna2_ops/fp8_weight_gemm_v06.py:76-92; the
// half-even mode is the per-token rule of the benchmark (absmax/127, round-half-even).
#include "qg_common.h"
#include "qg_internal.h"
#include "qg_quant.h"

namespace qg {

namespace {

// Register-resident rows: thread t of the workgroup holds chunks t + 64 NW i,
// i < NCH.
template <int XT, int MODE, int NW, int NCH>
__global__ __launch_bounds__(64 * NW) void k_quant_rows_reg(const char* x, int64_t x_sm, int M, int K, int8_t* q,
                                                            int64_t q_sm, int k_pad, float* step_out) {
#pragma clang fp contract(off)
  constexpr int ES = XType<XT>::size;
  constexpr int E = 16 / ES;
  constexpr int T = 64 * NW;
  __shared__ float s_amax[NW];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int row = blockIdx.x;
  const char* xr = x + static_cast<int64_t>(row) * x_sm * ES;
  int8_t* qr = q + static_cast<int64_t>(row) * q_sm;
  const int chunks = K / E;
  i32x4 raw[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = t + T * i;
    raw[i] = c < chunks ? reinterpret_cast<const i32x4*>(xr)[c] : i32x4{0, 0, 0, 0};
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    float v[E];
    decode_chunk<XT>(raw[i], v);
#pragma unroll
    for (int e = 0; e < E; ++e) amax = fmaxf(amax, fabsf(v[e]));
  }
  amax = wave_max(amax);
  if constexpr (NW > 1) {
    if (lane == 0) s_amax[wave] = amax;
    __syncthreads();
    amax = s_amax[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) amax = fmaxf(amax, s_amax[w]);
  }
  const float step = fmaxf(amax / 127.0f, 1.0e-20f);
  const float rstep = __builtin_amdgcn_rcpf(step);
  // Up to 3 chunks the decoded elements stay live (at most 48 registers);
  // longer rows are decoded again rather than hold every element.
  if constexpr (NCH > 3) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) asm volatile("" : "+v"(raw[i]));
  }
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = t + T * i;
    quant_chunk_store<XT, MODE>(raw[i], step, rstep, qr, c, c < chunks);
  }
  for (int k = K + t; k < k_pad; k += T) qr[k] = 0;
  if (t == 0) step_out[row] = step;
}

template <int XT, int MODE, bool VEC>
__global__ __launch_bounds__(256) void k_quant_rows(const char* x, int64_t x_sm, int64_t x_sk,
                                                    int M, int K, int8_t* q, int64_t q_sm,
                                                    int k_pad, float* step_out) {
#pragma clang fp contract(off)
  constexpr int ES = XType<XT>::size;
  constexpr int E = 16 / ES;  // elements per 16-byte chunk
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const char* xr = x + static_cast<int64_t>(row) * x_sm * ES;
  int8_t* qr = q + static_cast<int64_t>(row) * q_sm;

  float amax = 0.0f;
  if constexpr (VEC) {
    const int chunks = K / E;
    for (int c = lane; c < chunks; c += 64) {
      const i32x4 raw = reinterpret_cast<const i32x4*>(xr)[c];
      float v[E];
      decode_chunk<XT>(raw, v);
#pragma unroll
      for (int e = 0; e < E; ++e) amax = fmaxf(amax, fabsf(v[e]));
    }
  } else {
    for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(load_x<XT>(xr, k * x_sk)));
  }
  amax = wave_max(amax);
  const float step = fmaxf(amax / 127.0f, 1.0e-20f);

  if constexpr (VEC) {
    const int chunks = K / E;
    for (int c = lane; c < chunks; c += 64) {
      const i32x4 raw = reinterpret_cast<const i32x4*>(xr)[c];
      float v[E];
      decode_chunk<XT>(raw, v);
      uint32_t packed[E / 4 > 0 ? E / 4 : 1] = {};
#pragma unroll
      for (int e = 0; e < E; ++e)
        packed[e / 4] |= (static_cast<uint32_t>(quant_one<MODE>(v[e], step)) & 0xffu) << (8 * (e & 3));
      if constexpr (E == 4) reinterpret_cast<uint32_t*>(qr)[c] = packed[0];
      else if constexpr (E == 8) reinterpret_cast<uint2*>(qr)[c] = make_uint2(packed[0], packed[1]);
      else reinterpret_cast<uint4*>(qr)[c] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    }
  } else {
    for (int k = lane; k < K; k += 64)
      qr[k] = static_cast<int8_t>(quant_one<MODE>(load_x<XT>(xr, k * x_sk), step));
  }
  for (int k = K + lane; k < k_pad; k += 64) qr[k] = 0;
  if (lane == 0) step_out[row] = step;
}

template <int XT, int MODE>
hipError_t launch_quant_t(const void* x, int64_t x_sm, int64_t x_sk, int64_t M, int64_t K,
                          int8_t* q, int64_t q_sm, int64_t k_pad, float* step, hipStream_t stream) {
  constexpr int ES = XType<XT>::size;
  constexpr int E = 16 / ES;
  const uintptr_t xa = reinterpret_cast<uintptr_t>(x), qa = reinterpret_cast<uintptr_t>(q);
  const bool vec = x_sk == 1 && (xa % 16) == 0 && ((x_sm * ES) % 16) == 0 && (K % E) == 0 &&
                   (qa % E) == 0 && (q_sm % E) == 0;
  const dim3 grid(static_cast<unsigned>(ceil_div<int64_t>(M, 4)));
  const char* xp = static_cast<const char*>(x);
  const int64_t chunks = K / E;  // 16-byte chunks per row
  const int m = static_cast<int>(M), k = static_cast<int>(K), kp = static_cast<int>(k_pad);
  if (vec && chunks <= 64 * 8 * 6) {
    const dim3 rows(static_cast<unsigned>(M));  // one row per workgroup
    // NW: the smallest of 1, 2, 4, 8 with at most 3 chunks per lane (3 waves of
    // 2 chunks for 257-384: 4096 x 3072 fp16 9.3 against 9.6 us with 2 of 3);
    // NCH: the chunks per lane that row needs (1 to 3; 6 past 1536 chunks)
#define QG_QUANT_REG(NW, NCH)                                                                   \
  hipLaunchKernelGGL((k_quant_rows_reg<XT, MODE, NW, NCH>), rows, dim3(64 * NW), 0, stream, xp, \
                     x_sm, m, k, q, q_sm, kp, step)
    if (chunks <= 64) QG_QUANT_REG(1, 1);
    else if (chunks <= 128) QG_QUANT_REG(1, 2);
    else if (chunks <= 192) QG_QUANT_REG(1, 3);
    else if (chunks <= 256) QG_QUANT_REG(2, 2);
    else if (chunks <= 384) QG_QUANT_REG(3, 2);
    else if (chunks <= 512) QG_QUANT_REG(4, 2);
    else if (chunks <= 768) QG_QUANT_REG(4, 3);
    else if (chunks <= 1024) QG_QUANT_REG(8, 2);
    else if (chunks <= 1536) QG_QUANT_REG(8, 3);
    else QG_QUANT_REG(8, 6);
#undef QG_QUANT_REG
    return hipGetLastError();
  }
  if (vec)
    hipLaunchKernelGGL((k_quant_rows<XT, MODE, true>), grid, dim3(256), 0, stream, xp, x_sm, x_sk,
                       static_cast<int>(M), static_cast<int>(K), q, q_sm, static_cast<int>(k_pad), step);
  else
    hipLaunchKernelGGL((k_quant_rows<XT, MODE, false>), grid, dim3(256), 0, stream, xp, x_sm, x_sk,
                       static_cast<int>(M), static_cast<int>(K), q, q_sm, static_cast<int>(k_pad), step);
  return hipGetLastError();
}

template <int MODE>
hipError_t launch_quant_mode(const void* x, int x_dtype, int64_t x_sm, int64_t x_sk, int64_t M,
                             int64_t K, int8_t* q, int64_t q_sm, int64_t k_pad, float* step,
                             hipStream_t stream) {
  switch (x_dtype) {
    case QG_F32: return launch_quant_t<QG_F32, MODE>(x, x_sm, x_sk, M, K, q, q_sm, k_pad, step, stream);
    case QG_F16: return launch_quant_t<QG_F16, MODE>(x, x_sm, x_sk, M, K, q, q_sm, k_pad, step, stream);
    case QG_BF16: return launch_quant_t<QG_BF16, MODE>(x, x_sm, x_sk, M, K, q, q_sm, k_pad, step, stream);
    case QG_E4M3: return launch_quant_t<QG_E4M3, MODE>(x, x_sm, x_sk, M, K, q, q_sm, k_pad, step, stream);
    case QG_E5M2: return launch_quant_t<QG_E5M2, MODE>(x, x_sm, x_sk, M, K, q, q_sm, k_pad, step, stream);
    default: return hipErrorInvalidValue;
  }
}

// ConvRot prologue + per-row quantizer: every group of G consecutive K
// values of the row is rotated by the normalised Hadamard matrix H_G / sqrt(G)
// (Sylvester order: (H x)_i = sum_j (-1)^popcount(i & j) x_j), then the row is
// quantized as above. One row per workgroup of 256 threads: the row is held in
// LDS as fp32 (K <= QG_ROT_MAX_K), transformed in place by the fast
// Walsh-Hadamard butterflies (log2 G stages of (a, b) -> (a + b, a - b) on
// pairs h apart inside aligned blocks of 2 h), scaled by the fp32 value of
// 1 / sqrt(G) (exact for G = 4^j, e.g. 256), then reduced and quantized. The
// butterflies form the same sums as the dense product with H in another
// order, so the rotated values agree with it to a few fp32 ulps.
template <int XT, int MODE>
__global__ __launch_bounds__(256) void k_rot_quant_rows(const char* x, int64_t x_sm, int K, int G, float inv_sqrt_g,
                                                        int8_t* q, int64_t q_sm, int k_pad, float* step_out) {
#pragma clang fp contract(off)
  constexpr int ES = XType<XT>::size;
  __shared__ float v[QG_ROT_MAX_K];
  __shared__ float s_amax[4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int row = blockIdx.x;
  const char* xr = x + static_cast<int64_t>(row) * x_sm * ES;
  int8_t* qr = q + static_cast<int64_t>(row) * q_sm;
  for (int k = t; k < K; k += 256) v[k] = load_x<XT>(xr, k);
  for (int lh = 0; (1 << lh) < G; ++lh) {
    const int h = 1 << lh;
    __syncthreads();
    for (int b = t; b < K / 2; b += 256) {
      const int i = ((b >> lh) << (lh + 1)) | (b & (h - 1));
      const float a = v[i], c = v[i + h];
      v[i] = a + c;
      v[i + h] = a - c;
    }
  }
  __syncthreads();
  float amax = 0.0f;
  for (int k = t; k < K; k += 256) {
    const float r = v[k] * inv_sqrt_g;
    v[k] = r;
    amax = fmaxf(amax, fabsf(r));
  }
  amax = wave_max(amax);
  if (lane == 0) s_amax[wave] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(s_amax[0], s_amax[1]), fmaxf(s_amax[2], s_amax[3]));
  const float step = fmaxf(amax / 127.0f, 1.0e-20f);
  for (int k = t; k < K; k += 256) qr[k] = static_cast<int8_t>(quant_one<MODE>(v[k], step));
  for (int k = K + t; k < k_pad; k += 256) qr[k] = 0;
  if (t == 0) step_out[row] = step;
}

// Register-resident form of k_rot_quant_rows for K a multiple of 512 (up to
// QG_ROT_MAX_K) and groups of 8 to 512: one row per workgroup of NW = min(8,
// K / 512) waves; lane t of the workgroup holds, in each of NS slots, the 8
// consecutive values 8 (s 64 NW + t) .. + 7 of the row as fp32. A group of G
// values is G / 8 consecutive lanes of one slot (aligned), so the butterfly
// stages h = 1, 2, 4 pair registers of a lane, and the stages h = 8 .. G / 2
// pair register e of lanes h / 8 apart (__shfl_xor): the lower element of a
// pair becomes a + c and the upper a - c, with a the lower and c the upper
// value — the operations, operands and stage order of the LDS form, so the
// results are the same bits. Lanes past K hold zeros (whole groups, K % G ==
// 0) and store nothing. Then the scale by fp32(1 / sqrt(G)), the row's absmax
// (wave reduction, one LDS exchange) and the shared quantizer of
// k_quant_rows_reg (reciprocal quotient, IEEE redo near half-integers).
template <int XT, int MODE, int NS>
__global__ __launch_bounds__(512) void k_rot_quant_rows_reg(const char* x, int64_t x_sm, int K, int G,
                                                            float inv_sqrt_g, int8_t* q, int64_t q_sm, int k_pad,
                                                            float* step_out) {
#pragma clang fp contract(off)
  constexpr int ES = XType<XT>::size;
  __shared__ float s_amax[8];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int nt = blockDim.x;
  const int row = blockIdx.x;
  const char* xr = x + static_cast<int64_t>(row) * x_sm * ES;
  int8_t* qr = q + static_cast<int64_t>(row) * q_sm;
  float v[NS][8];
  bool live[NS];
  // loads of every slot first, then their decoding
  i32x4 raw[NS][ES == 4 ? 2 : 1];
  static_for<0, NS>([&](auto s_c) {
    constexpr int S = decltype(s_c)::value;
    const int base = 8 * (S * nt + t);
    live[S] = base < K;
    const int b = live[S] ? base : 0;  // lanes past K read the row's first values (unused)
    static_for<0, (ES == 4 ? 2 : 1)>([&](auto h) {
      raw[S][decltype(h)::value] =
          *reinterpret_cast<const i32x4*>(xr + static_cast<int64_t>(b) * ES + 16 * decltype(h)::value);
    });
  });
  static_for<0, NS>([&](auto s_c) {
    constexpr int S = decltype(s_c)::value;
    if constexpr (ES == 4) {
      decode_chunk<XT>(raw[S][0], v[S]);
      decode_chunk<XT>(raw[S][1], v[S] + 4);
    } else {
      decode_chunk<XT>(raw[S][0], v[S]);
    }
    if (!live[S]) {
      static_for<0, 8>([&](auto e) { v[S][decltype(e)::value] = 0.0f; });
    }
  });
  // butterflies inside a lane: h = 1, 2, 4
  static_for<0, NS>([&](auto s_c) {
    constexpr int S = decltype(s_c)::value;
    static_for<0, 3>([&](auto lh_c) {
      constexpr int h = 1 << decltype(lh_c)::value;
      if (h < G) {
        static_for<0, 8>([&](auto i_c) {
          constexpr int i = decltype(i_c)::value;
          if constexpr ((i & h) == 0) {
            const float a = v[S][i], c = v[S][i + h];
            v[S][i] = a + c;
            v[S][i + h] = a - c;
          }
        });
      }
    });
  });
  // butterflies across lanes: h = 8 d for lane distance d = 1 .. G / 16
  for (int d = 1; 8 * d < G; d <<= 1) {
    const bool upper = (lane & d) != 0;
    static_for<0, NS>([&](auto s_c) {
      constexpr int S = decltype(s_c)::value;
      static_for<0, 8>([&](auto e_c) {
        constexpr int e = decltype(e_c)::value;
        const float self = v[S][e];
        const float other = __shfl_xor(self, d, 64);
        v[S][e] = upper ? other - self : self + other;
      });
    });
  }
  float amax = 0.0f;
  static_for<0, NS>([&](auto s_c) {
    constexpr int S = decltype(s_c)::value;
    static_for<0, 8>([&](auto e_c) {
      constexpr int e = decltype(e_c)::value;
      const float r = v[S][e] * inv_sqrt_g;
      v[S][e] = r;
      amax = fmaxf(amax, fabsf(r));
    });
  });
  amax = wave_max(amax);
  if (lane == 0) s_amax[wave] = amax;
  __syncthreads();
  amax = s_amax[0];
  for (int w = 1; w < nt / 64; ++w) amax = fmaxf(amax, s_amax[w]);
  const float step = fmaxf(amax / 127.0f, 1.0e-20f);
  const float rstep = __builtin_amdgcn_rcpf(step);
  static_for<0, NS>([&](auto s_c) {
    constexpr int S = decltype(s_c)::value;
    quant_values_store<8, MODE>(v[S], step, rstep, qr, S * nt + t, live[S]);
  });
  for (int k = K + t; k < k_pad; k += nt) qr[k] = 0;
  if (t == 0) step_out[row] = step;
}

// The register form's contract (K % 512 == 0, groups 8 .. 512, 16-byte
// aligned rows); its slot count per lane (at most 4: the launcher's largest
// instantiation).
static_assert(QG_ROT_MAX_K <= 4 * 512 * 8, "register ConvRot form: at most 4 slots of 8 values per lane");
inline int rot_reg_slots(const void* x, int x_dtype, int64_t x_sm, int64_t K, int G, int8_t* q, int64_t q_sm) {
  const int es = x_dtype == QG_F32 ? 4 : 2;
  if (K % 512 != 0 || K > QG_ROT_MAX_K || G < 8 || G > 512) return 0;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_sm * es) % 16 != 0) return 0;
  if ((reinterpret_cast<uintptr_t>(q) & 7) != 0 || q_sm % 8 != 0) return 0;
  const int64_t nw = K / 512 < 8 ? K / 512 : 8;
  return static_cast<int>((K + 512 * nw - 1) / (512 * nw));
}

template <int MODE>
hipError_t launch_rot_quant_mode(const void* x, int x_dtype, int64_t x_sm, int64_t M, int64_t K, int G,
                                 float inv_sqrt_g, int8_t* q, int64_t q_sm, int64_t k_pad, float* step,
                                 hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(M));
  const char* xp = static_cast<const char*>(x);
  const int k = static_cast<int>(K), kp = static_cast<int>(k_pad);
  const int ns = rot_reg_slots(x, x_dtype, x_sm, K, G, q, q_sm);
  if (ns > 0) {
    const dim3 block(static_cast<unsigned>(64 * (K / 512 < 8 ? K / 512 : 8)));
#define QG_ROT_REG(XT, NS)                                                                                      \
  hipLaunchKernelGGL((k_rot_quant_rows_reg<XT, MODE, NS>), grid, block, 0, stream, xp, x_sm, k, G, inv_sqrt_g, q, \
                     q_sm, kp, step)
#define QG_ROT_REG_NS(XT)                  \
  do {                                     \
    if (ns == 1) QG_ROT_REG(XT, 1);        \
    else if (ns == 2) QG_ROT_REG(XT, 2);   \
    else if (ns == 3) QG_ROT_REG(XT, 3);   \
    else QG_ROT_REG(XT, 4);                \
  } while (0)
    if (x_dtype == QG_F32) QG_ROT_REG_NS(QG_F32);
    else if (x_dtype == QG_F16) QG_ROT_REG_NS(QG_F16);
    else QG_ROT_REG_NS(QG_BF16);
#undef QG_ROT_REG_NS
#undef QG_ROT_REG
    return hipGetLastError();
  }
  switch (x_dtype) {
    case QG_F32:
      hipLaunchKernelGGL((k_rot_quant_rows<QG_F32, MODE>), grid, dim3(256), 0, stream, xp, x_sm, k, G, inv_sqrt_g, q,
                         q_sm, kp, step);
      break;
    case QG_F16:
      hipLaunchKernelGGL((k_rot_quant_rows<QG_F16, MODE>), grid, dim3(256), 0, stream, xp, x_sm, k, G, inv_sqrt_g, q,
                         q_sm, kp, step);
      break;
    case QG_BF16:
      hipLaunchKernelGGL((k_rot_quant_rows<QG_BF16, MODE>), grid, dim3(256), 0, stream, xp, x_sm, k, G, inv_sqrt_g,
                         q, q_sm, kp, step);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_pack_rows_i8(const int8_t* src, int64_t s_r, int64_t s_k,
                                                      int64_t rows, int64_t K, int8_t* dst,
                                                      int64_t k_pad) {
  const int64_t total = rows * k_pad;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / k_pad, k = i - r * k_pad;
    dst[i] = k < K ? src[r * s_r + k * s_k] : static_cast<int8_t>(0);
  }
}

}  // namespace

hipError_t launch_quant_rows(const void* x, int x_dtype, int64_t x_sm, int64_t x_sk, int64_t M,
                             int64_t K, int8_t* q, int64_t q_sm, int64_t k_pad, float* step,
                             int rounding, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  if (rounding == QG_ROUND_HALF_EVEN)
    return launch_quant_mode<QG_ROUND_HALF_EVEN>(x, x_dtype, x_sm, x_sk, M, K, q, q_sm, k_pad, step, stream);
  return launch_quant_mode<QG_ROUND_HALF_AWAY>(x, x_dtype, x_sm, x_sk, M, K, q, q_sm, k_pad, step, stream);
}

hipError_t launch_rot_quant_rows(const void* x, int x_dtype, int64_t x_sm, int64_t M, int64_t K, int group,
                                 int8_t* q, int64_t q_sm, int64_t k_pad, float* step, int rounding,
                                 hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const float inv_sqrt_g = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(group)));
  if (rounding == QG_ROUND_HALF_EVEN)
    return launch_rot_quant_mode<QG_ROUND_HALF_EVEN>(x, x_dtype, x_sm, M, K, group, inv_sqrt_g, q, q_sm, k_pad, step,
                                                     stream);
  return launch_rot_quant_mode<QG_ROUND_HALF_AWAY>(x, x_dtype, x_sm, M, K, group, inv_sqrt_g, q, q_sm, k_pad, step,
                                                   stream);
}

hipError_t launch_pack_rows_i8(const int8_t* src, int64_t s_r, int64_t s_k, int64_t rows, int64_t K,
                               int8_t* dst, int64_t k_pad, hipStream_t stream) {
  const int64_t total = rows * k_pad;
  if (total == 0) return hipSuccess;
  const int64_t blocks = ceil_div<int64_t>(total, 256);
  const unsigned grid = static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
  hipLaunchKernelGGL(k_pack_rows_i8, dim3(grid), dim3(256), 0, stream, src, s_r, s_k, rows, K, dst, k_pad);
  return hipGetLastError();
}

}  // namespace qg
