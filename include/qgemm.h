/*
 * qgemm.h — C ABI of the MI355X (gfx950) quantized-weight GEMM library
 * (librdna2_qgemm.so).
 *
 * Conventions (mirroring the reference's only native ABI,
 * rdna2-ops/rdna2_ops/csrc/group_norm_silu.hip:283-321, loaded by ctypes in
 * rdna2-ops/rdna2_ops/normalization.py:16-27):
 *   - every entry point returns an int that is a hipError_t value; 0 = success;
 *   - bad arguments return hipErrorInvalidValue (1) BEFORE any HIP call, so
 *     argument validation is testable without a GPU;
 *   - all pointers are device pointers owned by the caller; outputs and
 *     workspace are allocated by the caller (query *_workspace_bytes first);
 *   - launches are asynchronous on `stream` (a hipStream_t, NULL = default);
 *   - the library allocates nothing, never synchronises and keeps no mutable
 *     global state; concurrent calls need distinct workspace;
 *   - strides are in ELEMENTS of the tensor they describe;
 *   - dtype codes: QG_F32 = 0, QG_F16 = 1, QG_BF16 = 2 (same numbering as
 *     normalization.py:14), then QG_I32, QG_I8, QG_U8, QG_E4M3, QG_E5M2.
 */
#ifndef RDNA2_QGEMM_H
#define RDNA2_QGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum qg_dtype {
  QG_F32 = 0,
  QG_F16 = 1,
  QG_BF16 = 2,
  QG_I32 = 3,
  QG_I8 = 4,
  QG_U8 = 5,
  QG_E4M3 = 6, /* OCP float8 e4m3fn (torch.float8_e4m3fn) */
  QG_E5M2 = 7  /* OCP float8 e5m2 (torch.float8_e5m2) */
};

/* Epilogue flags of the INT8 GEMM (bit field). */
enum qg_epilogue {
  /* order F (default, 0): v = f32(acc) * (sa[m] * sb[n]); v = v + f32(bias[n]);
   *   act(v); one RNE rounding to out dtype.  int8_gemm.py:53-63, :191. */
  QG_EPI_ORDER_FUSED_FMA = 1, /* rounding="fused": v = fma(f32(acc), sa*sb, bias)
                                 (int8_gemm.py:191 enable_fp_fusion=True) */
  QG_EPI_ORDER_EAGER = 2,     /* Kitchen eager order E: t = out(f32(acc)*(sa*sb));
                                 t = out(f32(t) + f32(out(bias))) (comfy_int8.py:128-143) */
  QG_EPI_GELU_TANH = 4        /* GELU(tanh approximation) in fp32 before the final
                                 rounding (new; benchmark configuration 1) */
};

/* Rounding mode of the per-row INT8 quantizer. */
enum qg_rounding {
  QG_ROUND_HALF_EVEN = 0, /* q = rint(x / step)        (round half to even) */
  QG_ROUND_HALF_AWAY = 1  /* q = floor(z+.5) | ceil(z-.5) (fp8_weight_gemm_v06.py:87-90) */
};

/* W4 storage flags (bit field). */
enum qg_w4_flags {
  QG_W4_SIGNED_NIBBLES = 1, /* stored nibble = q & 15 with q in [-8,7] and int32
                               zero points in the same signed coordinates
                               (reference PackedInt4, int4_weight_gemm_v07.py:49-82);
                               otherwise nibble and zero point are unsigned uint4 */
  QG_W4_ORDER_HIGH = 2,     /* nibble i of a word at bits 28-4i (order="high") */
  QG_W4_LAYOUT_KN = 4,      /* words are [K/8, N] (layout="kn") instead of [N, K/8] */
  QG_W4_ZEROS_PACKED = 8    /* zero points are uint4 packed 8 per int32 along the
                               group axis, [N, ceil((K/G)/8)], group g at bits
                               4*(g%8) of word g/8; else int32 [N, K/G] */
};

/* Error string of a returned status. Mirrors rdna2_hip_error_string
 * (group_norm_silu.hip:319-321). */
const char* qg_error_string(int status);

/* Library build identity: "gfx950 <git-less source digest>". */
const char* qg_version(void);

/* ---------------------------------------------------------------------------
 * Per-row dynamic INT8 quantizer.
 * Replaces: Kitchen eager.quantize_int8_rowwise (third-party comfy_kitchen
 *   0.2.40, called at rdna2-ops/rdna2_ops/comfy_int8.py:122 and
 *   int8_gemm.py:255) and the in-tree Triton _quant_rows
 *   (rdna2-ops/rdna2_ops/fp8_weight_gemm_v06.py:76-92).
 * step[m] = max(absmax(x[m,:]) / 127, 1e-20) (IEEE fp32 division);
 * q[m,k] = clamp(round(x[m,k] / step[m]), -127, 127) with IEEE division.
 * x_dtype: QG_F32 / QG_F16 / QG_BF16 / QG_E4M3 / QG_E5M2 (fp8 decoded exactly
 * first, as fp8_weight_gemm_v06.py:83-84). q is [m, k] with row stride q_sm.
 * ------------------------------------------------------------------------- */
int qg_quant_rows_i8(const void* x, int x_dtype, int64_t x_sm, int64_t x_sk,
                     int64_t m, int64_t k, int8_t* q, int64_t q_sm, float* step,
                     int rounding, void* stream);

/* ---------------------------------------------------------------------------
 * INT8 x INT8 -> INT32 GEMM with an optional fused dequant epilogue.
 * Replaces: _int8_dot_dequant / _int8_dot_dequant_wrapped + _launch
 *   (rdna2-ops/rdna2_ops/int8_gemm.py:19-123, :152-192), i.e. the entry
 *   points int8_matmul (:195-200) and int8_gemm_dequant (:203-214).
 * a: [m, k] int8 with strides (a_sm, a_sk); b: [k, n] int8 with strides
 * (b_sk, b_sn) — the MOSS call passes weight.T, i.e. b_sk = 1, b_sn = k.
 * a_scale == NULL: integer GEMM, out_dtype must be QG_I32.
 * Otherwise a_scale: [m] fp32, b_scale: [n] fp32 (b_scale_numel == n) or a
 * scalar (b_scale_numel == 1); bias: NULL or [n] of bias_dtype
 * (QG_F32/QG_F16/QG_BF16); out_dtype QG_F32 / QG_F16 / QG_BF16.
 * out: [m, n] contiguous. Non-canonical strides or k % 128 != 0 are packed into
 * the workspace first (see qg_int8_gemm_workspace_bytes).
 * k must be <= 131071 (int8_gemm.py:142-143); each (packed) operand must be
 * smaller than 2 GiB.
 * ------------------------------------------------------------------------- */
size_t qg_int8_gemm_workspace_bytes(const void* a, int64_t a_sm, int64_t a_sk,
                                    const void* b, int64_t b_sk, int64_t b_sn,
                                    int64_t m, int64_t n, int64_t k);
int qg_int8_gemm(const int8_t* a, int64_t a_sm, int64_t a_sk, const int8_t* b,
                 int64_t b_sk, int64_t b_sn, int64_t m, int64_t n, int64_t k,
                 const float* a_scale, const float* b_scale,
                 int64_t b_scale_numel, const void* bias, int bias_dtype,
                 void* out, int out_dtype, int epilogue, void* workspace,
                 size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * W8A8 linear: per-token activation quantize prologue + INT8 GEMM + epilogue
 * in one call: out = epi(quant(x) @ w.T).
 * Replaces: the MOSS candidate body quantize_int8_rowwise -> int8_gemm_dequant
 *   (rdna2-ops/rdna2_ops/int8_gemm.py:254-259) and the FP8 "int8" method
 *   (fp8_weight_gemm_v06.py:181-193).
 * x: [m, k] (x_dtype QG_F32/QG_F16/QG_BF16, row stride x_sm, unit k stride);
 * w: [n, k] int8 row-major (row stride w_sn); w_scale [n] or scalar.
 * The workspace holds the int8 activations ([m, round_up(k, 128)]), their fp32
 * steps ([m]) and, when w is not canonical ([n, k] with unit k stride,
 * 16-byte aligned rows and k % 128 == 0), a zero-padded packed copy of w; its
 * size comes from qg_w8a8_linear_workspace_bytes.
 * ------------------------------------------------------------------------- */
size_t qg_w8a8_linear_workspace_bytes(const int8_t* w, int64_t w_sn, int64_t m,
                                      int64_t n, int64_t k);
int qg_w8a8_linear(const void* x, int x_dtype, int64_t x_sm, int64_t m,
                   int64_t k, const int8_t* w, int64_t w_sn, int64_t n,
                   const float* w_scale, int64_t w_scale_numel,
                   const void* bias, int bias_dtype, void* out, int out_dtype,
                   int rounding, int epilogue, void* workspace,
                   size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * ConvRot prologue: per-row INT8 quantization after rotating every group of
 * rot_group consecutive K values by the normalised Hadamard matrix
 * H / sqrt(rot_group) (Sylvester order, H[i][j] = (-1)^popcount(i & j)).
 * Replaces, as an opt-in fused path: Kitchen's _build_hadamard +
 *   _rotate_activation + quantize_int8_rowwise of the MOSS linear
 *   (rdna2-ops/rdna2_ops/comfy_int8.py:112-122; every MOSS call uses
 *   convrot=True, convrot_groupsize=256). Kitchen rotates with a dense fp32
 *   matmul; this library uses the fast Walsh-Hadamard butterflies, which form
 *   the same sums in another order (agreement to a few fp32 ulps, so codes can
 *   differ by 1 where the quotient is within a few ulps of a rounding tie).
 * x: [m, k] QG_F32 / QG_F16 / QG_BF16, unit K stride, row stride x_sm >= k;
 * rot_group a power of two in [2, 1024] dividing k; k <= QG_ROT_MAX_K.
 * q [m, k] (row stride q_sm >= k), step [m]: as qg_quant_rows_i8 on the
 * rotated rows.
 * ------------------------------------------------------------------------- */
#define QG_ROT_MAX_K 16384
int qg_rot_quant_rows_i8(const void* x, int x_dtype, int64_t x_sm, int64_t m,
                         int64_t k, int rot_group, int8_t* q, int64_t q_sm,
                         float* step, int rounding, void* stream);

/* ---------------------------------------------------------------------------
 * W8A8 linear with the opt-in MOSS fusion: qg_w8a8_linear plus an optional
 * ConvRot prologue (rot_group > 0, see qg_rot_quant_rows_i8) and an optional
 * residual epilogue term.
 * Replaces, as an opt-in fused path: the MOSS int8_linear body
 *   (rdna2-ops/rdna2_ops/comfy_int8.py:98-145: ConvRot, quantizer, GEMM,
 *   scaling, bias, Kitchen's _apply_residual).
 * residual: NULL or [m, n] (row stride residual_sm >= n) of residual_dtype
 * (QG_F32 / QG_F16 / QG_BF16); residual_scale: NULL, one value or [n] fp32.
 * The epilogue adds f32(residual) (* residual_scale) in fp32 after the scale,
 * bias and activation steps and before the single rounding to out_dtype, so
 * fp32 outputs equal the fp32 sequence scale -> + bias -> + residual bit for
 * bit. Not with QG_EPI_ORDER_EAGER. The workspace is that of qg_w8a8_linear
 * (qg_w8a8_linear_workspace_bytes).
 * ------------------------------------------------------------------------- */
int qg_w8a8_linear_ex(const void* x, int x_dtype, int64_t x_sm, int64_t m,
                      int64_t k, const int8_t* w, int64_t w_sn, int64_t n,
                      const float* w_scale, int64_t w_scale_numel,
                      const void* bias, int bias_dtype, int rot_group,
                      const void* residual, int residual_dtype,
                      int64_t residual_sm, const float* residual_scale,
                      int64_t residual_scale_numel, void* out, int out_dtype,
                      int rounding, int epilogue, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Allocation-free W8A8 linear: qg_w8a8_linear without a workspace argument.
 * No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the workspace is a file-scope device array of
 * QG_W8A8_NOALLOC_SCRATCH_BYTES (64 MiB) per GPU, held until the process
 * ends; the call makes no hipMalloc / hipFree or other allocation. The caller
 * still passes inputs and outputs, as for qg_w8a8_linear (same arguments, same
 * results, bit for bit). Limit: qg_w8a8_linear_workspace_bytes(w, w_sn, m, n, k)
 * must not exceed QG_W8A8_NOALLOC_SCRATCH_BYTES (cfg1's K = 12288 down
 * projection at m = 4096 needs 50.3 MB), else hipErrorInvalidValue before any
 * HIP call. The stream must belong to the current device
 * (hipErrorInvalidDevice otherwise). Every call on one GPU shares that GPU's
 * array: calls that overlap in time on one GPU (other streams, other host
 * threads) race and must be serialised by the caller. The first call on a
 * device looks up the array's address (hipGetSymbolAddress); make it outside
 * graph capture.
 * ------------------------------------------------------------------------- */
#define QG_W8A8_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int qg_w8a8_linear_noalloc(const void* x, int x_dtype, int64_t x_sm, int64_t m,
                           int64_t k, const int8_t* w, int64_t w_sn, int64_t n,
                           const float* w_scale, int64_t w_scale_numel,
                           const void* bias, int bias_dtype, void* out,
                           int out_dtype, int rounding, int epilogue,
                           void* stream);

/* ---------------------------------------------------------------------------
 * INT4 weight storage (W4).
 * A W4 weight [n, k] quantised in groups of G = group_size (32, 64 or 128)
 * consecutive K values per output row n:
 *   data   int32 words, 8 nibbles each: [n, k/8] ("nk") or [k/8, n]
 *          (QG_W4_LAYOUT_KN); nibble e of a word holds K index 8*word + e at
 *          bits 4e, or 28-4e with QG_W4_ORDER_HIGH;
 *   scales [n, k/G] fp32 or bf16;
 *   zeros  [n, k/G] int32, or uint4 packed (QG_W4_ZEROS_PACKED);
 *   weight = (q - zero) * scale.
 * QG_W4_SIGNED_NIBBLES selects the reference PackedInt4 coordinates
 * (int4_weight_gemm_v07.py:20-82): q in [-8, 7] stored as q & 15, zero points
 * in the same signed coordinates. Without it nibbles and zero points are
 * unsigned uint4 (benchmark configuration 2: flags = QG_W4_ZEROS_PACKED,
 * bf16 scales, G = 128).
 * Shape contract (int4_weight_gemm_v07.py:436-440): n, k > 0, k % G == 0,
 * n * k < 2^31.
 * ------------------------------------------------------------------------- */

/* Quantise and pack a floating [n, k] weight (strides w_sn, w_sk > 0; w_dtype
 * QG_F32/QG_F16/QG_BF16).
 * Replaces: pack_int4 / _pack_weight (int4_weight_gemm_v07.py:103-133, :413-430),
 *   which must equal pack_int4_cpu (:49-82).
 * Per group, fp32 IEEE division and round-half-to-even throughout:
 *   symmetric:  s = absmax / 7, q = clamp(round(x / s), -7, 7), zero = 0;
 *   asymmetric: lo = min(min x, 0), hi = max(max x, 0), s = (hi - lo) / 15,
 *               zu = clamp(round(-lo / s), 0, 15),
 *               q = clamp(round(x / s) + zu, 0, 15) (unsigned coordinates);
 * s is rounded to scales_dtype before it is used; a group whose s is 0 gets
 * s = 1 (and, in signed coordinates, q = zero = 0, :74-75).
 * sums: NULL or [n, k/G] int32, the per-group sum of the stored codes. */
int qg_w4_pack(const void* w, int w_dtype, int64_t w_sn, int64_t w_sk, int64_t n,
               int64_t k, int group_size, int symmetric, int flags, int32_t* data,
               void* scales, int scales_dtype, void* zeros, int32_t* sums,
               void* stream);

/* Decode a W4 weight to out [n, k] contiguous: (q - zero) * scale rounded once
 * to out_dtype (QG_F16 / QG_F32 / QG_BF16), or the centred integers q - zero
 * (QG_I8).
 * Replaces: unpack_int4 / _unpack_weight (int4_weight_gemm_v07.py:136-151,
 *   :450-458). */
int qg_w4_unpack(const int32_t* data, int64_t n, int64_t k, int group_size,
                 int flags, const void* scales, int scales_dtype,
                 const void* zeros, void* out, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * W4A16 linear: out[m, n] = sum_k a[m, k] * ((q[n,k] - zero[n,g]) * scale[n,g])
 * (+ bias[n]), fp32 accumulation, one rounding to out_dtype.
 * Replaces: int4_linear_a16 (int4_weight_gemm_v07.py:540-564) with its
 *   _linear_dot2 kernel (:365-387) and its default dequant method (:549-554).
 * Decode shapes and smaller prefill grids apply each group scale to the exact
 * group partial sum (closer to the exact product than the reference, which
 * rounds every dequantised weight to fp16 first). Prefill grids of more than
 * 64 rows (K a multiple of 64) with at least T output tiles of 256 x 192 —
 * T = 192 at group 128, 64 at group 64, 1 at group 32 — take the reference's
 * dequant formulation instead: W is dequantised once into the
 * workspace, (q - z) * s in fp32 rounded to the activation dtype, then a
 * 2-byte MFMA GEMM with fp32 accumulation runs on it; the workspace is then
 * 2 * n * k bytes (16-byte aligned), reported by
 * qg_w4a16_gemm_workspace_bytes (0 on the other shapes), and required.
 * a: [m, k] QG_F16 or QG_BF16, unit K stride, row stride a_sm (a multiple of 8
 * elements, 16-byte aligned base); w: 16-byte aligned; out: [m, n] contiguous
 * QG_F16 / QG_BF16 / QG_F32; bias NULL or [n] of bias_dtype; m * n < 2^31. */
size_t qg_w4a16_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int group_size,
                                     int flags);
int qg_w4a16_gemm(const void* a, int a_dtype, int64_t a_sm, int64_t m, int64_t k,
                  const int32_t* w, int64_t n, int group_size, int flags,
                  const void* scales, int scales_dtype, const void* zeros,
                  const void* bias, int bias_dtype, void* out, int out_dtype,
                  void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * W4A8 linear on the int8 MFMA, integer-exact group sums:
 *   acc_g[m, n] = sum_{k in group g} a[m, k] * (q[n, k] - zero[n, g])  (exact)
 *   integer: out int32 [m, n] = sum_g acc_g
 *   float:   total = 0; for g = 0, 1, ...: total = total + f32(acc_g) * scale[n, g]
 *            (separate fp32 roundings); out fp32 = total * a_scale[m] (+ bias[n])
 * Replaces: int4_linear_a8 (int4_weight_gemm_v07.py:476-537) — every method
 *   (dot4, dot4_split, dot4_words, dot8 :181-353) computes these numbers; with
 *   prepared != NULL the weights are the caller's centred int8 q - zero [n, k]
 *   (row stride prepared_sn bytes, method dot4_prepared) and w / zeros are unused.
 * a: int8 [m, k], row stride a_sm (a multiple of 16 bytes, 16-byte aligned
 * base); w: the W4 storage above (16-byte aligned); a_scale fp32 [m] (float
 * output); bias NULL or [n] of bias_dtype; out [m, n] contiguous; m * n < 2^31,
 * k * 128 * 15 < 2^31 (int4_weight_gemm_v07.py:493). */
int qg_w4a8_gemm(const int8_t* a, int64_t a_sm, int64_t m, int64_t k, const int32_t* w, int64_t n,
                 int group_size, int flags, const void* scales, int scales_dtype, const void* zeros,
                 const int8_t* prepared, int64_t prepared_sn, const float* a_scale, const void* bias,
                 int bias_dtype, void* out, int integer, void* stream);

/* ---------------------------------------------------------------------------
 * FP8 (OCP e4m3fn / e5m2) weights.
 * ------------------------------------------------------------------------- */

/* Decode fp8 storage w [n, k] (strides w_sn, w_sk in bytes = elements) to
 * out [n, k] contiguous in out_dtype (QG_F16 / QG_F32 / QG_BF16); exact for
 * every finite value, 0x7f / 0xff (e4m3fn) decode to NaN, e5m2 keeps inf/NaN.
 * Replaces: decode_fp8_weight / _decode_weight / _decode_bits
 *   (rdna2-ops/rdna2_ops/fp8_weight_gemm_v06.py:21-46, :109-124). */
int qg_fp8_decode(const uint8_t* w, int w_dtype, int64_t w_sn, int64_t w_sk,
                  int64_t n, int64_t k, void* out, int out_dtype, void* stream);

/* FP8 weight-only linear: out[m, n] = (sum_k a[m, k] * decode(w[n, k])) *
 * w_scale[n] + bias[n]; fp32 accumulation, scale and bias applied in fp32 in
 * that order, one rounding to out_dtype. w_scale NULL = unscaled (the
 * reference's storage); bias NULL or [n] of bias_dtype.
 * Replaces: the fused path _fp8_linear of fp8_weight_gemm
 *   (fp8_weight_gemm_v06.py:49-73, :195-206), whose products and fp32
 *   accumulation it performs exactly; benchmark configuration 3 adds the
 *   per-channel scale (s = absmax / 448).
 * a: [m, k] QG_F16 / QG_BF16 with strides (a_sm, a_sk); w: [n, k] with strides
 * (w_sn, w_sk); out: [m, n] contiguous QG_F16 / QG_BF16 / QG_F32. Operands that
 * are not canonical (unit K stride, 16-byte aligned rows, k % 128 == 0) are
 * packed, zero-padded, into the workspace (qg_fp8w_gemm_workspace_bytes).
 * From 192 output tiles of 256 x 192 on (and 2 * m * k < 2^31) the GEMM runs
 * the 2-byte MFMA on W fragments converted exactly to the activation dtype in
 * registers (every fp8 value is exact in fp16 and bf16): the same fp32
 * products and epilogue, another summation order, no extra workspace. */
size_t qg_fp8w_gemm_workspace_bytes(const void* a, int64_t a_sm, int64_t a_sk,
                                    const uint8_t* w, int64_t w_sn, int64_t w_sk,
                                    int64_t m, int64_t n, int64_t k);
int qg_fp8w_gemm(const void* a, int a_dtype, int64_t a_sm, int64_t a_sk, int64_t m,
                 int64_t k, const uint8_t* w, int w_dtype, int64_t w_sn,
                 int64_t w_sk, int64_t n, const float* w_scale, const void* bias,
                 int bias_dtype, void* out, int out_dtype, void* workspace,
                 size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * MoE prefill with grouped INT8 GEMMs (benchmark configuration 4).
 * No counterpart in the reference repository (it has no MoE kernel); the
 * stages follow the benchmark's CPU formulation: softmax + top-k routing, tokens
 * sorted and padded per expert, per-expert INT8 GEMMs with a SiLU * mul
 * epilogue, scatter-add with the routing weights.
 * ------------------------------------------------------------------------- */

/* Routed rows per grouped-GEMM tile (the dispatch builds its tile table in
 * units of this many rows). */
#define QG_MOE_TILE_ROWS 192

/* int32 words of the dispatch's counts workspace per expert. */
#define QG_MOE_COUNTS_PER_EXPERT 259

/* Epilogues of qg_moe_grouped_gemm; v = f32(acc) * (a_scale[row] * b_scale[e, n]). */
enum qg_moe_epilogue {
  QG_MOE_EPI_I32 = 0,      /* out int32 [rows, n] = acc */
  QG_MOE_EPI_SILU_MUL = 1, /* W rows 32b..32b+15 are gate rows and 32b+16..32b+31 the
                              up rows of features 16b..16b+15:
                              out bf16 [rows, n / 2] = silu(v_gate) * v_up */
  QG_MOE_EPI_ROUTE = 2     /* out bf16 [tokens * top_k, n], row row_slot[r]
                              = v * row_weight[r] */
};

/* Upper bounds of the routed rows and tiles of a dispatch (sizes of the
 * row_* and tiles arrays): rows_max = tokens * top_k + n_experts * (pad - 1),
 * tiles_max = ceil(rows_max / QG_MOE_TILE_ROWS) + n_experts. */
int qg_moe_sizes(int64_t tokens, int n_experts, int top_k, int pad, int64_t* rows_max, int64_t* tiles_max);

/* Routing and dispatch. logits: fp32 [tokens, n_experts] (row stride l_sm),
 * n_experts <= 64, 1 <= top_k <= n_experts, pad >= 1.
 * experts int32 [tokens, top_k]: the top_k experts by logit (descending;
 *   equal logits: lower index first); weights fp32 [tokens, top_k]: their
 *   softmax probabilities over all experts (not renormalised).
 * Routed rows grouped by expert (expert 0 first), each expert's segment
 * padded to a multiple of pad rows: row_token (token, -1 for padding),
 * row_weight (0 for padding), row_slot (t * top_k + k, -1 for padding), each
 * [rows_max]; inside a segment the rows are in slot order (t * top_k + k
 * ascending), so the dispatch is deterministic; rows past the last segment
 * are padding too.
 * tiles int32 [tiles_max][4] = {expert (-1: unused), first row, end of the
 * expert's valid rows, 0}; tiles[0][3] = number of tiles in use (the used
 * tiles come first). counts: int32 workspace [QG_MOE_COUNTS_PER_EXPERT *
 * n_experts]: per-expert counts, segment offsets and first tiles, then the
 * sort's per-block histograms. Two launches, no host synchronisation and no
 * memset (capturable in a graph). */
int qg_moe_dispatch(const float* logits, int64_t l_sm, int64_t tokens, int n_experts, int top_k, int pad,
                    int32_t* experts, float* weights, int32_t* counts, int32_t* row_token,
                    float* row_weight, int32_t* row_slot, int64_t rows_max, int32_t* tiles,
                    int64_t tiles_max, void* stream);

/* qg_moe_dispatch that also quantizes x for the gate/up GEMM, in the same
 * routing launch: x bf16 [tokens, hidden] (row stride x_sm elements, 16-byte
 * aligned rows) -> xq int8 (row stride xq_sm, 8-byte aligned rows) and xs
 * fp32 [tokens], bit-identical to qg_quant_rows_i8(x, QG_BF16, ...,
 * QG_ROUND_HALF_EVEN). hidden % 8 == 0 and hidden <= 2048 (one wave per token
 * holds its row); anything else returns hipErrorInvalidValue and the caller
 * runs qg_moe_dispatch and qg_quant_rows_i8. This build's own (benchmark
 * configuration 4 has no counterpart in the reference): the quantization's
 * loads overlap the routing's latency-bound shuffles instead of a launch of
 * their own. */
int qg_moe_dispatch_qx(const float* logits, int64_t l_sm, int64_t tokens, int n_experts, int top_k, int pad,
                       int32_t* experts, float* weights, int32_t* counts, int32_t* row_token,
                       float* row_weight, int32_t* row_slot, int64_t rows_max, int32_t* tiles,
                       int64_t tiles_max, const void* x, int64_t x_sm, int64_t hidden, int8_t* xq,
                       int64_t xq_sm, float* xs, void* stream);

/* Grouped INT8 GEMM over the dispatch's tile table: for each routed row r of
 * expert e, acc[r, n] = sum_k a[src(r), k] * w[e, n, k] with src(r) =
 * row_token[r] (row_token NULL: r itself), then the epilogue. a: int8
 * [a_rows, k] (row stride a_sm); w: int8 [n_experts][n, k] (row stride w_sn,
 * expert stride w_estride bytes); a_scale fp32 indexed like a's rows;
 * b_scale fp32 [n_experts, n]. k % 128 == 0, 16-byte aligned rows;
 * QG_MOE_EPI_SILU_MUL needs n % 32 == 0. out: out_rows rows (>= rows_max, or
 * tokens * top_k for QG_MOE_EPI_ROUTE) of row stride out_sm (elements). Tile
 * entries naming an expert >= n_experts or rows outside [0, rows_max) are
 * skipped, row_token entries are clamped into [0, a_rows) and route rows
 * outside [0, out_rows) are not written. At most 131072 work items
 * (tiles_max * ceil(n / 256)); more return hipErrorInvalidValue. */
int qg_moe_grouped_gemm(const int8_t* a, int64_t a_sm, int64_t a_rows, const int32_t* row_token,
                        int64_t rows_max, int64_t k, const int8_t* w, int64_t w_sn, int64_t w_estride,
                        int64_t n, int n_experts, const int32_t* tiles, int64_t tiles_max,
                        const float* a_scale, const float* b_scale, const float* row_weight,
                        const int32_t* row_slot, int epilogue, void* out, int64_t out_sm,
                        int64_t out_rows, void* stream);

/* out bf16 [tokens, hidden] (row stride out_sm) = bf16(sum over k of
 * y[t * top_k + k, :]) with y bf16 [tokens * top_k, hidden] contiguous; the
 * fp32 sum runs in k order (deterministic). */
int qg_moe_combine(const void* y, int64_t tokens, int top_k, int64_t hidden, void* out, int64_t out_sm,
                   void* stream);

/* ---------------------------------------------------------------------------
 * Plain HBM read (a measurement aid; no counterpart in the reference): reads
 * `bytes` bytes at src (16-byte aligned, bytes a multiple of 16) once, split
 * evenly over four 512-thread workgroups per CU, as whole 1 KB non-temporal
 * wave requests with 4 in flight per wave (the W4A16 decode streams its
 * weights with the same hint), and folds them into one word; sink (one uint32)
 * is written only if that word equals a fixed constant. Its time is the floor
 * a weight-streaming kernel such as the W4A16 decode is measured against.
 * ------------------------------------------------------------------------- */
int qg_read_floor(const void* src, size_t bytes, uint32_t* sink, void* stream);

/* ---------------------------------------------------------------------------
 * MFMA clock probe (a measurement aid; no counterpart in the reference): 256
 * workgroups of 8 waves (two per SIMD) each issue `iters` (1 .. 2^22) rounds of
 * six independent v_mfma_i32_32x32x32_i8 back to back; mode 0 keeps the
 * operands constant, mode 1 cycles them through random fragments, mode 2 adds
 * the INT8 GEMM's LDS fragment reads (two A and three W 1 KB reads per six
 * MFMAs). out (uint32 [256 * 8 * 2]): per wave, the shader-clock cycles
 * (s_memtime) and the 100 MHz real-time ticks (s_memrealtime) of its loop.
 * Their ratio is the shader clock that MFMA load sustains under the board's
 * power limit; cycles / (6 * iters) is the issue interval per MFMA of a wave.
 * ------------------------------------------------------------------------- */
int qg_mfma_clock(int mode, int iters, uint32_t* out, void* stream);

/* ---------------------------------------------------------------------------
 * Stage timing of the INT8 GEMM (a measurement aid; no counterpart in the
 * reference): the persistent ping-pong kernel that qg_int8_gemm runs for grids
 * of >= 192 tiles of 256 x 192, with fp16 output and order F (acc * (sa * sw)
 * + bias), instantiated with shader-clock stamps. Operands canonical: a int8
 * [m, k] and w int8 [n, k] row-major, 16-byte aligned, k a multiple of 128;
 * a_scale [m], w_scale [n] fp32; bias_f16 [n] or NULL; out_f16 [m, n].
 * stamps (uint32, at least min(tiles, 256) * 8 * 272 words): per wave w of
 * workgroup b, 272 words at (8 b + w) * 272 — words 64 P + s hold point P of
 * stage s (s < 64) of the last tile the workgroup ran: waves 0-3 before the
 * stage's first barrier, after it, after their MFMAs, after the second
 * barrier; waves 4-7 after the first barrier, their LDS reads complete,
 * after the second barrier, after their MFMAs; then word 256 entry, 257
 * main-loop exit, 258 epilogue end (its stores complete), 259 exit (shader-
 * clock cycles), 260 / 261 entry / exit in 100 MHz ticks, 262 the hardware
 * id, 263 the stage count.
 * ------------------------------------------------------------------------- */
int qg_int8_gemm_stages(const int8_t* a, const int8_t* w, int64_t m, int64_t n, int64_t k, const float* a_scale,
                        const float* w_scale, const void* bias_f16, void* out_f16, uint32_t* stamps,
                        size_t stamp_words, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RDNA2_QGEMM_H */
