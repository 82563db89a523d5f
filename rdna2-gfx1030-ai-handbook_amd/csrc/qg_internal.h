// Host-side launch interface shared by the translation units of the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qg {

// Canonical INT8 GEMM operands: A [M, K] and W [N, K] (B = W^T), both with
// unit K stride, 16-byte aligned rows and K % 64 == 0 (zero padded).
struct I8GemmArgs {
  const int8_t* a;
  int64_t a_sm;
  const int8_t* w;
  int64_t w_sn;
  int M, N, K;
  const float* a_scale;  // nullptr: int32 output
  const float* b_scale;
  int b_scalar;
  const void* bias;      // nullptr or [N] of bias_dtype
  int bias_dtype;
  void* out;             // [M, N], row stride out_sm (0: N)
  int out_dtype;
  int epi;
  // Optional residual term of the epilogue (nullptr: none): after the scale /
  // bias / activation steps, v += f32(residual[row * residual_sm + col])
  // (* residual_scale[col], or residual_scale[0] when residual_scalar), in
  // fp32 before the one rounding to out_dtype. residual_dtype QG_F32 / F16 / BF16.
  const void* residual;
  int residual_dtype;
  int64_t residual_sm;
  const float* residual_scale;
  int residual_scalar;
  // Grouped (MoE) mode (launch_i8_moe_gemm): M is the number of routed rows,
  // tiles [tiles_max][4] = {expert (< 0: none), first row, end of valid rows, -};
  // A row of routed row r is row_token[r] (r when null, < a_rows); expert e's
  // weights start w_estride bytes after expert e-1's, its scales N floats.
  const int* tiles;
  int tiles_max;
  const int* row_token;
  int a_rows;
  int64_t w_estride;
  const float* row_weight;
  const int* row_slot;
  int64_t out_sm;  // row stride of out in elements (the dense kernels read 0 as N)
  int out_rows;   // rows of out (routed rows, or tokens * top_k for the route epilogue)
  int n_experts;
  int moe_epi;
  // Stage-timing instantiation only (launch_i8_gemm_stages): per wave of
  // workgroup b, kStampWords words at stamps + (8 b + wave) * kStampWords.
  uint32_t* stamps;
};

// Stage timing of the ping-pong INT8 GEMM (qg_int8_gemm_stages): words per
// wave = 4 stamp points x 64 stages (lane s holds stage s, s < 64) + 16
// (kernel entry, main-loop exit, epilogue end, exit in shader-clock cycles;
// entry and exit in 100 MHz ticks; the hardware id; the stage count).
constexpr int kStampWords = 4 * 64 + 16;
hipError_t launch_i8_gemm_stages(const I8GemmArgs& p, hipStream_t stream);

hipError_t launch_i8_gemm(const I8GemmArgs& p, hipStream_t stream);
hipError_t launch_i8_moe_gemm(const I8GemmArgs& p, hipStream_t stream);
// 2-byte (fp16 / bf16) A and W on the ping-pong main loop; p.a_sm / p.w_sn /
// p.K in elements, a_scale null (1), b_scale per column or null (1).
hipError_t launch_h16_gemm(const I8GemmArgs& p, bool f16a, hipStream_t stream);
// Plain streaming read of `bytes` (a multiple of 16) at a 16-byte aligned src.
hipError_t launch_read_floor(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream);
// MFMA clock probe (qg_mfma_clock): kMfmaClockWorkgroups workgroups of 8 waves,
// out[2 * (8 b + w) + {0, 1}] = shader-clock cycles and 100 MHz ticks of wave w
// of workgroup b.
constexpr int kMfmaClockWorkgroups = 256;
hipError_t launch_mfma_clock(int mode, int iters, uint32_t* out, hipStream_t stream);
// fp16 / bf16 A against fp8 W converted in registers (fp8 W stages in LDS).
hipError_t launch_f8w_gemm(const I8GemmArgs& p, bool f16a, bool e5, hipStream_t stream);

// MoE routing and dispatch: see include/qgemm.h (qg_moe_dispatch).
struct MoeDispatchArgs {
  const float* logits;
  int64_t l_sm;
  int T, E, top_k, pad;
  int* experts;       // [T, top_k]
  float* weights;     // [T, top_k]
  int* counts;        // [3 E]: counts, offsets, cursors
  int* row_token;     // [rows_max]
  float* row_weight;  // [rows_max]
  int* row_slot;      // [rows_max]
  int rows_max;
  int* tiles;         // [tiles_max][4]
  int tiles_max;
  int tile_rows;
  // optional (x != nullptr): the routing kernel also quantizes each token's
  // row of x (bf16 [T, H], row stride x_sm elements) to xq (int8, row stride
  // xq_sm) and xs (fp32 step per token), half even; H % 8 == 0, H <= 2048
  const uint16_t* x;
  int64_t x_sm;
  int H;
  int8_t* xq;
  int64_t xq_sm;
  float* xs;
};
// Largest hidden size whose rows the routing kernel quantizes (one wave per
// token, 4 chunks of 8 bf16 per lane).
constexpr int kMoeRouteQuantMaxH = 2048;
hipError_t launch_moe_dispatch(const MoeDispatchArgs& p, hipStream_t stream);
// out[t, n] = bf16(sum over k of y[t * top_k + k, n]) (fp32 sum in k order)
hipError_t launch_moe_combine(const uint16_t* y, int T, int top_k, int H, uint16_t* out, int64_t out_sm,
                              hipStream_t stream);

// dst[r, k] = src[r * s_r + k * s_k] for k < K, 0 for K <= k < k_pad.
hipError_t launch_pack_rows_i8(const int8_t* src, int64_t s_r, int64_t s_k,
                               int64_t rows, int64_t K, int8_t* dst,
                               int64_t k_pad, hipStream_t stream);

// Per-row INT8 quantizer; columns [K, k_pad) of q are written as zeros.
// Per-row quantizer after a ConvRot rotation of every group of `group` K values
// (normalised Hadamard, group a power of two in [2, 1024] dividing K,
// K <= QG_ROT_MAX_K, unit K stride).
hipError_t launch_rot_quant_rows(const void* x, int x_dtype, int64_t x_sm, int64_t M, int64_t K, int group,
                                 int8_t* q, int64_t q_sm, int64_t k_pad, float* step, int rounding,
                                 hipStream_t stream);
hipError_t launch_quant_rows(const void* x, int x_dtype, int64_t x_sm,
                             int64_t x_sk, int64_t M, int64_t K, int8_t* q,
                             int64_t q_sm, int64_t k_pad, float* step,
                             int rounding, hipStream_t stream);

// W4A16 GEMM / unpack operands (see include/qgemm.h for the storage flags).
struct W4Args {
  const uint16_t* a;     // activations [M, K] fp16 / bf16, unit K stride
  int64_t a_sm;
  int a_f16;             // 1: fp16 activations, 0: bf16
  int M, N, K;
  const uint32_t* w;     // packed words, [N, K/8] or [K/8, N]
  int flags;             // qg_w4_flags
  int group;             // 32, 64 or 128
  int ng;                // groups per row, K / group
  int zw;                // packed zero-point words per row, ceil(ng / 8)
  const void* scales;    // [N, K/G] fp32 or bf16
  int scale_f32;
  const void* zeros;     // int32 [N, K/G] or packed uint4 [N, ceil(K/G/8)]
  const void* bias;      // nullptr or [N] of bias_dtype
  int bias_dtype;
  void* out;             // [M, N] contiguous (unpack: [N, K])
  int out_dtype;
};

// W4A8 GEMM operands (int4_linear_a8; see include/qgemm.h, qg_w4a8_gemm).
struct W4A8Args {
  const int8_t* a;       // activations int8 [M, K], row stride a_sm bytes
  int64_t a_sm;
  int M, N, K;
  const uint32_t* w;     // packed words ([N, K/8] or [K/8, N] per flags), or
  const int8_t* w8;      // prepared centred int8 weights [N, K] (row stride w8_sn)
  int64_t w8_sn;
  int flags;             // qg_w4_flags
  int group;             // 32, 64 or 128
  int ng;                // K / group
  int zw;                // packed zero-point words per row, ceil(ng / 8)
  const void* scales;    // [N, K/G] fp32 or bf16
  int scale_f32;
  const void* zeros;     // int32 [N, K/G] or packed uint4 [N, ceil(K/G/8)]
  const float* a_scale;  // [M] (float output)
  const void* bias;      // nullptr or [N] of bias_dtype
  int bias_dtype;
  void* out;             // int32 (integer) or fp32 [M, N] contiguous
  int integer;
};
hipError_t launch_w4a8_gemm(const W4A8Args& p, hipStream_t stream);

struct W4PackArgs {
  const void* w;         // [N, K] fp32 / fp16 / bf16, strides in elements
  int w_dtype;
  int64_t w_sn, w_sk;
  int N, K, group, symmetric, flags;
  int32_t* data;
  void* scales;
  int scale_dtype;       // QG_F32 or QG_BF16
  void* zeros;
  int32_t* sums;         // nullptr or [N, K/G]
};

// Tiled weight-decode GEMM (M large): A [M, K] fp16 / bf16 (unit K stride,
// 16-byte aligned rows, K % 128 == 0) times INT4 or fp8 weights.
struct WdArgs {
  const uint16_t* a;
  int64_t a_sm;
  int a_f16;
  int M, N, K;
  // INT4 weights (same storage fields as W4Args)
  const uint32_t* w4;
  int flags, group, ng, zw;
  const void* scales;
  int scale_f32;
  const void* zeros;
  // fp8 weights [N, K] with row stride w8_sn (bytes, multiple of 16)
  const uint8_t* w8;
  int64_t w8_sn;
  int fp8_e5;
  const float* w_scale;  // nullptr or per-channel [N]
  const void* bias;
  int bias_dtype;
  void* out;  // [M, N] contiguous
  int out_dtype;
};

hipError_t launch_wd_w4(const WdArgs& p, hipStream_t stream);
hipError_t launch_pack_rows_u16(const uint16_t* src, int64_t s_r, int64_t s_k, int64_t rows, int64_t K,
                                uint16_t* dst, int64_t k_pad, hipStream_t stream);
hipError_t launch_fp8_decode(const uint8_t* w, int64_t w_sn, int64_t w_sk, int64_t n, int64_t K, int e5,
                             void* out, int out_dtype, hipStream_t stream);
hipError_t launch_wd_fp8(const WdArgs& p, hipStream_t stream);

hipError_t launch_w4a16(const W4Args& p, hipStream_t stream);
hipError_t launch_w4_pack(const W4PackArgs& p, hipStream_t stream);
hipError_t launch_w4_unpack(const W4Args& p, hipStream_t stream);

}  // namespace qg
