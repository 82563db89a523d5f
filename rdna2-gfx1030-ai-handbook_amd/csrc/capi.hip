// extern "C" entry points of librdna2_qgemm.so (declared in include/qgemm.h).
//
// Argument validation happens here, before any HIP call, and returns
// hipErrorInvalidValue like the reference's native ABI
// (rdna2-ops/rdna2_ops/csrc/group_norm_silu.hip:298-317). The library never
// allocates: non-canonical operands are packed into caller workspace.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "../../include/qgemm.h"
#include "qg_internal.h"

namespace {

constexpr int64_t kMaxK = 131071;  // int32 accumulator bound, int8_gemm.py:142-143
constexpr int64_t kIntMax = 2147483647;

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The GEMM kernel streams K in 128-byte stages and addresses an operand with
// 32-bit byte offsets from its base.
constexpr int64_t kStageK = 128;
constexpr int64_t kMaxOperandBytes = int64_t(1) << 31;
// Work items of one grouped (MoE) GEMM launch: 256 workgroups x 512 table
// entries each.
constexpr int64_t kMoeMaxItems = 131072;

// An operand of `rows` rows (row stride s_row, element stride s_k) can be read
// in place by the GEMM kernel.
inline bool canonical_rows(const void* p, int64_t s_row, int64_t s_k, int64_t rows, int64_t k) {
  return s_k == 1 && (s_row % 16) == 0 && aligned16(p) && (k % kStageK) == 0 &&
         (rows - 1) * s_row + k < kMaxOperandBytes;
}

inline bool float_dtype(int d) { return d == QG_F32 || d == QG_F16 || d == QG_BF16; }

struct I8Plan {
  bool pack_a, pack_b;
  int64_t kp;
  size_t a_bytes, b_bytes;
  size_t total() const { return a_bytes + b_bytes; }
};

I8Plan plan_i8(const void* a, int64_t a_sm, int64_t a_sk, const void* b, int64_t b_sk,
               int64_t b_sn, int64_t m, int64_t n, int64_t k) {
  I8Plan pl;
  pl.kp = round_up(k, kStageK);
  // B = W^T: W [n, k] has row stride b_sn and element stride b_sk.
  pl.pack_a = !canonical_rows(a, a_sm, a_sk, m, k);
  pl.pack_b = !canonical_rows(b, b_sn, b_sk, n, k);
  pl.a_bytes = pl.pack_a ? static_cast<size_t>(round_up(m * pl.kp, 256)) : 0;
  pl.b_bytes = pl.pack_b ? static_cast<size_t>(round_up(n * pl.kp, 256)) : 0;
  return pl;
}

bool valid_epilogue(int epi) {
  if (epi & ~(QG_EPI_ORDER_FUSED_FMA | QG_EPI_ORDER_EAGER | QG_EPI_GELU_TANH)) return false;
  if ((epi & QG_EPI_ORDER_EAGER) && (epi & (QG_EPI_ORDER_FUSED_FMA | QG_EPI_GELU_TANH))) return false;
  return true;
}

bool valid_gemm_shape(int64_t m, int64_t n, int64_t k, int64_t a_sm, int64_t a_sk, int64_t b_sk,
                      int64_t b_sn) {
  if (m < 0 || n < 0 || k < 0 || k > kMaxK || m > kIntMax || n > kIntMax) return false;
  if (a_sm < 0 || a_sk < 0 || b_sk < 0 || b_sn < 0) return false;
  if (m * n > (int64_t(1) << 40)) return false;
  return true;
}

}  // namespace

extern "C" const char* qg_error_string(int status) {
  return hipGetErrorString(static_cast<hipError_t>(status));
}

extern "C" const char* qg_version(void) { return "librdna2_qgemm gfx950 1"; }

extern "C" int qg_read_floor(const void* src, size_t bytes, uint32_t* sink, void* stream) {
  if (bytes % 16 != 0 || bytes >= (size_t(1) << 40)) return hipErrorInvalidValue;
  if (bytes == 0) return hipSuccess;
  if (!src || !sink || !aligned16(src)) return hipErrorInvalidValue;
  return qg::launch_read_floor(src, bytes, sink, static_cast<hipStream_t>(stream));
}

extern "C" int qg_mfma_clock(int mode, int iters, uint32_t* out, void* stream) {
  if (mode < 0 || mode > 2 || iters < 1 || iters > (1 << 22) || !out) return hipErrorInvalidValue;
  return qg::launch_mfma_clock(mode, iters, out, static_cast<hipStream_t>(stream));
}

extern "C" int qg_quant_rows_i8(const void* x, int x_dtype, int64_t x_sm, int64_t x_sk, int64_t m,
                                int64_t k, int8_t* q, int64_t q_sm, float* step, int rounding,
                                void* stream) {
  if (m < 0 || k < 0 || m > kIntMax || k > kIntMax || x_sm < 0 || x_sk < 0 || q_sm < k)
    return hipErrorInvalidValue;
  if (!(float_dtype(x_dtype) || x_dtype == QG_E4M3 || x_dtype == QG_E5M2)) return hipErrorInvalidValue;
  if (rounding != QG_ROUND_HALF_EVEN && rounding != QG_ROUND_HALF_AWAY) return hipErrorInvalidValue;
  if (m == 0) return hipSuccess;
  if (!q || !step || (k > 0 && !x)) return hipErrorInvalidValue;
  return qg::launch_quant_rows(x, x_dtype, x_sm, x_sk, m, k, q, q_sm, k, step, rounding,
                               static_cast<hipStream_t>(stream));
}

namespace {
bool valid_rot_group(int g, int64_t k) {
  return g >= 2 && g <= 1024 && (g & (g - 1)) == 0 && k % g == 0 && k <= QG_ROT_MAX_K;
}
}  // namespace

extern "C" int qg_rot_quant_rows_i8(const void* x, int x_dtype, int64_t x_sm, int64_t m, int64_t k,
                                    int rot_group, int8_t* q, int64_t q_sm, float* step, int rounding,
                                    void* stream) {
  if (m < 0 || k < 1 || m > kIntMax || x_sm < k || q_sm < k) return hipErrorInvalidValue;
  if (!float_dtype(x_dtype) || !valid_rot_group(rot_group, k)) return hipErrorInvalidValue;
  if (rounding != QG_ROUND_HALF_EVEN && rounding != QG_ROUND_HALF_AWAY) return hipErrorInvalidValue;
  if (m == 0) return hipSuccess;
  if (!x || !q || !step) return hipErrorInvalidValue;
  return qg::launch_rot_quant_rows(x, x_dtype, x_sm, m, k, rot_group, q, q_sm, k, step, rounding,
                                   static_cast<hipStream_t>(stream));
}

extern "C" size_t qg_int8_gemm_workspace_bytes(const void* a, int64_t a_sm, int64_t a_sk,
                                               const void* b, int64_t b_sk, int64_t b_sn,
                                               int64_t m, int64_t n, int64_t k) {
  if (!valid_gemm_shape(m, n, k, a_sm, a_sk, b_sk, b_sn)) return 0;
  return plan_i8(a, a_sm, a_sk, b, b_sk, b_sn, m, n, k).total();
}

namespace {

int int8_gemm_impl(const int8_t* a, int64_t a_sm, int64_t a_sk, const int8_t* b, int64_t b_sk,
                   int64_t b_sn, int64_t m, int64_t n, int64_t k, const float* a_scale,
                   const float* b_scale, int64_t b_scale_numel, const void* bias, int bias_dtype,
                   void* out, int out_dtype, int epilogue, void* workspace, size_t workspace_bytes,
                   hipStream_t stream) {
  if (!valid_gemm_shape(m, n, k, a_sm, a_sk, b_sk, b_sn)) return hipErrorInvalidValue;
  if (!valid_epilogue(epilogue)) return hipErrorInvalidValue;
  const bool dequant = a_scale != nullptr;
  if (dequant) {
    if (!float_dtype(out_dtype)) return hipErrorInvalidValue;
    if (!b_scale || (b_scale_numel != 1 && b_scale_numel != n)) return hipErrorInvalidValue;
    if (bias && !float_dtype(bias_dtype)) return hipErrorInvalidValue;
  } else {
    if (out_dtype != QG_I32 || b_scale || bias || epilogue != 0) return hipErrorInvalidValue;
  }
  if (m == 0 || n == 0) return hipSuccess;
  if (!out || (k > 0 && (!a || !b))) return hipErrorInvalidValue;
  const I8Plan pl = plan_i8(a, a_sm, a_sk, b, b_sk, b_sn, m, n, k);
  if (pl.total() > 0 && (!workspace || workspace_bytes < pl.total() || !aligned16(workspace)))
    return hipErrorInvalidValue;
  if (m * pl.kp >= kMaxOperandBytes || n * pl.kp >= kMaxOperandBytes) return hipErrorInvalidValue;

  qg::I8GemmArgs p{};
  p.M = static_cast<int>(m);
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(pl.kp);
  char* ws = static_cast<char*>(workspace);
  if (pl.pack_a) {
    int8_t* pa = reinterpret_cast<int8_t*>(ws);
    hipError_t e = qg::launch_pack_rows_i8(a, a_sm, a_sk, m, k, pa, pl.kp, stream);
    if (e != hipSuccess) return e;
    p.a = pa;
    p.a_sm = pl.kp;
  } else {
    p.a = a;
    p.a_sm = a_sm;
  }
  if (pl.pack_b) {
    int8_t* pb = reinterpret_cast<int8_t*>(ws + pl.a_bytes);
    hipError_t e = qg::launch_pack_rows_i8(b, b_sn, b_sk, n, k, pb, pl.kp, stream);
    if (e != hipSuccess) return e;
    p.w = pb;
    p.w_sn = pl.kp;
  } else {
    p.w = b;
    p.w_sn = b_sn;
  }
  p.a_scale = a_scale;
  p.b_scale = b_scale;
  p.b_scalar = b_scale_numel == 1;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.out = out;
  p.out_dtype = out_dtype;
  p.epi = epilogue;
  return qg::launch_i8_gemm(p, stream);
}

}  // namespace

extern "C" int qg_int8_gemm(const int8_t* a, int64_t a_sm, int64_t a_sk, const int8_t* b,
                            int64_t b_sk, int64_t b_sn, int64_t m, int64_t n, int64_t k,
                            const float* a_scale, const float* b_scale, int64_t b_scale_numel,
                            const void* bias, int bias_dtype, void* out, int out_dtype,
                            int epilogue, void* workspace, size_t workspace_bytes, void* stream) {
  return int8_gemm_impl(a, a_sm, a_sk, b, b_sk, b_sn, m, n, k, a_scale, b_scale, b_scale_numel,
                        bias, bias_dtype, out, out_dtype, epilogue, workspace, workspace_bytes,
                        static_cast<hipStream_t>(stream));
}

extern "C" int qg_int8_gemm_stages(const int8_t* a, const int8_t* w, int64_t m, int64_t n, int64_t k,
                                   const float* a_scale, const float* w_scale, const void* bias_f16, void* out_f16,
                                   uint32_t* stamps, size_t stamp_words, void* stream) {
  if (m <= 0 || n <= 0 || k <= 0 || k > kMaxK || m > kIntMax || n > kIntMax) return hipErrorInvalidValue;
  if (!a || !w || !a_scale || !w_scale || !out_f16 || !stamps) return hipErrorInvalidValue;
  if (!canonical_rows(a, k, 1, m, k) || !canonical_rows(w, k, 1, n, k) || !aligned16(out_f16))
    return hipErrorInvalidValue;
  if (m * k >= kMaxOperandBytes || n * k >= kMaxOperandBytes) return hipErrorInvalidValue;
  const int64_t tiles = ((m + 255) / 256) * ((n + 191) / 192);
  const int64_t grid = tiles < 256 ? tiles : 256;
  if (stamp_words < static_cast<size_t>(grid * 8 * qg::kStampWords)) return hipErrorInvalidValue;
  qg::I8GemmArgs p{};
  p.a = a;
  p.a_sm = k;
  p.w = w;
  p.w_sn = k;
  p.M = static_cast<int>(m);
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(k);
  p.a_scale = a_scale;
  p.b_scale = w_scale;
  p.bias = bias_f16;
  p.bias_dtype = QG_F16;
  p.out = out_f16;
  p.out_dtype = QG_F16;
  p.stamps = stamps;
  return qg::launch_i8_gemm_stages(p, static_cast<hipStream_t>(stream));
}

namespace {
// Workspace of the W8A8 linear: int8 activations [m, kp], fp32 steps [m], then
// a packed copy of W when W is not canonical ([n, k] row-major, 16-byte rows,
// k % 64 == 0).
struct W8A8Plan {
  int64_t kp;
  size_t act_bytes, step_bytes;
  I8Plan w;
  size_t total() const { return act_bytes + step_bytes + w.b_bytes; }
};
W8A8Plan plan_w8a8(const void* w, int64_t w_sn, int64_t m, int64_t n, int64_t k) {
  W8A8Plan pl;
  pl.kp = round_up(k, kStageK);
  pl.act_bytes = static_cast<size_t>(round_up(m * pl.kp, 256));
  pl.step_bytes = static_cast<size_t>(round_up(m * 4, 256));
  pl.w = plan_i8(nullptr, pl.kp, 1, w, 1, w_sn, m, n, k);
  pl.w.a_bytes = 0;
  return pl;
}
}  // namespace

extern "C" size_t qg_w8a8_linear_workspace_bytes(const int8_t* w, int64_t w_sn, int64_t m,
                                                 int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k < 0 || k > kMaxK || w_sn < 0) return 0;
  return plan_w8a8(w, w_sn, m, n, k).total();
}

namespace {

// Validation and launches of the W8A8 linear into a given workspace: shared by
// qg_w8a8_linear (caller workspace) and qg_w8a8_linear_noalloc (the library's
// scratch array). `capacity` is the workspace size.
// Optional ConvRot rotation / residual term (qg_w8a8_linear_ex): rot_group 0 =
// no rotation; residual nullptr = no residual term.
struct W8A8Extra {
  int rot_group = 0;
  const void* residual = nullptr;
  int residual_dtype = 0;
  int64_t residual_sm = 0;
  const float* residual_scale = nullptr;
  int64_t residual_scale_numel = 0;
};

int w8a8_linear_run(const void* x, int x_dtype, int64_t x_sm, int64_t m, int64_t k, const int8_t* w,
                    int64_t w_sn, int64_t n, const float* w_scale, int64_t w_scale_numel, const void* bias,
                    int bias_dtype, void* out, int out_dtype, int rounding, int epilogue, char* ws,
                    size_t capacity, hipStream_t s, const W8A8Extra& ex = W8A8Extra{}) {
  if (m < 0 || n < 0 || k < 0 || k > kMaxK || x_sm < 0 || w_sn < 0) return hipErrorInvalidValue;
  if (ex.rot_group != 0 && (!valid_rot_group(ex.rot_group, k) || x_sm < k)) return hipErrorInvalidValue;
  if (ex.residual) {
    if (!float_dtype(ex.residual_dtype) || ex.residual_sm < n || (epilogue & QG_EPI_ORDER_EAGER))
      return hipErrorInvalidValue;
    if (ex.residual_scale && ex.residual_scale_numel != 1 && ex.residual_scale_numel != n)
      return hipErrorInvalidValue;
  }
  if (m > kIntMax || n > kIntMax || m * n > (int64_t(1) << 40)) return hipErrorInvalidValue;
  if (!float_dtype(x_dtype) || !float_dtype(out_dtype)) return hipErrorInvalidValue;
  if (rounding != QG_ROUND_HALF_EVEN && rounding != QG_ROUND_HALF_AWAY) return hipErrorInvalidValue;
  if (!valid_epilogue(epilogue)) return hipErrorInvalidValue;
  if (!w_scale || (w_scale_numel != 1 && w_scale_numel != n)) return hipErrorInvalidValue;
  if (bias && !float_dtype(bias_dtype)) return hipErrorInvalidValue;
  if (m == 0 || n == 0) return hipSuccess;
  if (!out || (k > 0 && (!x || !w))) return hipErrorInvalidValue;
  const W8A8Plan pl = plan_w8a8(w, w_sn, m, n, k);
  if (!ws || capacity < pl.total() || !aligned16(ws)) return hipErrorInvalidValue;
  if (m * pl.kp >= kMaxOperandBytes || n * pl.kp >= kMaxOperandBytes) return hipErrorInvalidValue;
  int8_t* xq = reinterpret_cast<int8_t*>(ws);
  float* xs = reinterpret_cast<float*>(ws + pl.act_bytes);
  hipError_t e = ex.rot_group
                     ? qg::launch_rot_quant_rows(x, x_dtype, x_sm, m, k, ex.rot_group, xq, pl.kp, pl.kp, xs,
                                                 rounding, s)
                     : qg::launch_quant_rows(x, x_dtype, x_sm, 1, m, k, xq, pl.kp, pl.kp, xs, rounding, s);
  if (e != hipSuccess) return e;
  qg::I8GemmArgs p{};
  p.residual = ex.residual;
  p.residual_dtype = ex.residual_dtype;
  p.residual_sm = ex.residual_sm;
  p.residual_scale = ex.residual_scale;
  p.residual_scalar = ex.residual_scale_numel == 1;
  p.M = static_cast<int>(m);
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(pl.kp);
  p.a = xq;
  p.a_sm = pl.kp;
  if (pl.w.pack_b) {
    int8_t* pw = reinterpret_cast<int8_t*>(ws + pl.act_bytes + pl.step_bytes);
    e = qg::launch_pack_rows_i8(w, w_sn, 1, n, k, pw, pl.kp, s);
    if (e != hipSuccess) return e;
    p.w = pw;
    p.w_sn = pl.kp;
  } else {
    p.w = w;
    p.w_sn = w_sn;
  }
  p.a_scale = xs;
  p.b_scale = w_scale;
  p.b_scalar = w_scale_numel == 1;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.out = out;
  p.out_dtype = out_dtype;
  p.epi = epilogue;
  return qg::launch_i8_gemm(p, s);
}

}  // namespace

extern "C" int qg_w8a8_linear(const void* x, int x_dtype, int64_t x_sm, int64_t m, int64_t k,
                              const int8_t* w, int64_t w_sn, int64_t n, const float* w_scale,
                              int64_t w_scale_numel, const void* bias, int bias_dtype, void* out,
                              int out_dtype, int rounding, int epilogue, void* workspace,
                              size_t workspace_bytes, void* stream) {
  return w8a8_linear_run(x, x_dtype, x_sm, m, k, w, w_sn, n, w_scale, w_scale_numel, bias, bias_dtype, out,
                         out_dtype, rounding, epilogue, static_cast<char*>(workspace), workspace_bytes,
                         static_cast<hipStream_t>(stream));
}

extern "C" int qg_w8a8_linear_ex(const void* x, int x_dtype, int64_t x_sm, int64_t m, int64_t k,
                                 const int8_t* w, int64_t w_sn, int64_t n, const float* w_scale,
                                 int64_t w_scale_numel, const void* bias, int bias_dtype, int rot_group,
                                 const void* residual, int residual_dtype, int64_t residual_sm,
                                 const float* residual_scale, int64_t residual_scale_numel, void* out,
                                 int out_dtype, int rounding, int epilogue, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  W8A8Extra ex;
  ex.rot_group = rot_group;
  ex.residual = residual;
  ex.residual_dtype = residual_dtype;
  ex.residual_sm = residual_sm;
  ex.residual_scale = residual_scale;
  ex.residual_scale_numel = residual_scale_numel;
  return w8a8_linear_run(x, x_dtype, x_sm, m, k, w, w_sn, n, w_scale, w_scale_numel, bias, bias_dtype, out,
                         out_dtype, rounding, epilogue, static_cast<char*>(workspace), workspace_bytes,
                         static_cast<hipStream_t>(stream), ex);
}

// --------------------------------------------------------------------------
// Allocation-free W8A8 linear. Its workspace (the int8 activations, their
// steps and a packed weight when the weight is not canonical) lives in this
// file-scope device array: one copy per GPU, at its own address on each, held
// until the process ends. Every byte a call reads from it is written by the
// same call first (the quantizer writes the K padding, the packer whole padded
// rows), so nothing has to be cleared between calls; calls that overlap in time
// on one GPU share the array and race.
namespace {

static __device__ __align__(256) char scratch[QG_W8A8_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::atomic<char*> g_scratch_addr[kMaxScratchDevices];
std::mutex g_scratch_lock;

// The device address of `scratch` on `device`, looked up once per device with
// that device current (host code never passes the array's own name: on the
// host it is a stand-in symbol, not a device address).
hipError_t scratch_address(int device, char** addr) {
  if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
  char* p = g_scratch_addr[device].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    p = g_scratch_addr[device].load(std::memory_order_relaxed);
    if (p == nullptr) {
      int current = -1;
      hipError_t e = hipGetDevice(&current);
      if (e != hipSuccess) return e;
      if (current != device) return hipErrorInvalidDevice;
      void* sym = nullptr;
      e = hipGetSymbolAddress(&sym, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return e;
      if (sym == nullptr) return hipErrorInvalidSymbol;
      p = static_cast<char*>(sym);
      g_scratch_addr[device].store(p, std::memory_order_release);
    }
  }
  *addr = p;
  return hipSuccess;
}

}  // namespace

extern "C" int qg_w8a8_linear_noalloc(const void* x, int x_dtype, int64_t x_sm, int64_t m, int64_t k,
                                      const int8_t* w, int64_t w_sn, int64_t n, const float* w_scale,
                                      int64_t w_scale_numel, const void* bias, int bias_dtype, void* out,
                                      int out_dtype, int rounding, int epilogue, void* stream) {
  // argument errors before any HIP call (the workspace check needs the plan)
  if (m < 0 || n < 0 || k < 0 || k > kMaxK || w_sn < 0) return hipErrorInvalidValue;
  if (m == 0 || n == 0) return hipSuccess;
  if (plan_w8a8(w, w_sn, m, n, k).total() > QG_W8A8_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;
  // the scratch of the device the stream runs on, which must be the current one
  hipStream_t s = static_cast<hipStream_t>(stream);
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  if (s != nullptr) {
    hipDevice_t stream_device = -1;
    e = hipStreamGetDevice(s, &stream_device);
    if (e != hipSuccess) return e;
    if (stream_device != device) return hipErrorInvalidDevice;
  }
  char* ws = nullptr;
  e = scratch_address(device, &ws);
  if (e != hipSuccess) return e;
  return w8a8_linear_run(x, x_dtype, x_sm, m, k, w, w_sn, n, w_scale, w_scale_numel, bias, bias_dtype, out,
                         out_dtype, rounding, epilogue, ws, QG_W8A8_NOALLOC_SCRATCH_BYTES, s);
}

// --------------------------------------------------------------------------
// W4 (INT4 weight) storage and the W4A16 GEMM.
namespace {

constexpr int kW4Flags = QG_W4_SIGNED_NIBBLES | QG_W4_ORDER_HIGH | QG_W4_LAYOUT_KN | QG_W4_ZEROS_PACKED;
// Above this many rows the W4A16 GEMM uses the tiled kernel.
constexpr int64_t kW4TiledMinRows = 64;

// int4_weight_gemm_v07.py:436-440: group 32/64/128 dividing K, nonempty, N*K < 2^31.
bool valid_w4_shape(int64_t n, int64_t k, int group, int flags) {
  if (group != 32 && group != 64 && group != 128) return false;
  if (n <= 0 || k <= 0 || k % group != 0 || n * k >= (int64_t(1) << 31)) return false;
  return (flags & ~kW4Flags) == 0;
}

}  // namespace

extern "C" int qg_w4_pack(const void* w, int w_dtype, int64_t w_sn, int64_t w_sk, int64_t n,
                          int64_t k, int group_size, int symmetric, int flags, int32_t* data,
                          void* scales, int scales_dtype, void* zeros, int32_t* sums, void* stream) {
  if (!valid_w4_shape(n, k, group_size, flags)) return hipErrorInvalidValue;
  if (!float_dtype(w_dtype) || (scales_dtype != QG_F32 && scales_dtype != QG_BF16)) return hipErrorInvalidValue;
  if (w_sn <= 0 || w_sk <= 0 || symmetric < 0 || symmetric > 1) return hipErrorInvalidValue;
  if ((n - 1) * w_sn + (k - 1) * w_sk >= (int64_t(1) << 40)) return hipErrorInvalidValue;
  if (!w || !data || !scales || !zeros) return hipErrorInvalidValue;
  qg::W4PackArgs p{};
  p.w = w;
  p.w_dtype = w_dtype;
  p.w_sn = w_sn;
  p.w_sk = w_sk;
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(k);
  p.group = group_size;
  p.symmetric = symmetric;
  p.flags = flags;
  p.data = data;
  p.scales = scales;
  p.scale_dtype = scales_dtype;
  p.zeros = zeros;
  p.sums = sums;
  return qg::launch_w4_pack(p, static_cast<hipStream_t>(stream));
}

extern "C" int qg_w4_unpack(const int32_t* data, int64_t n, int64_t k, int group_size, int flags,
                            const void* scales, int scales_dtype, const void* zeros, void* out,
                            int out_dtype, void* stream) {
  if (!valid_w4_shape(n, k, group_size, flags)) return hipErrorInvalidValue;
  if (scales_dtype != QG_F32 && scales_dtype != QG_BF16) return hipErrorInvalidValue;
  if (!(float_dtype(out_dtype) || out_dtype == QG_I8)) return hipErrorInvalidValue;
  if (!data || !scales || !zeros || !out) return hipErrorInvalidValue;
  qg::W4Args p{};
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(k);
  p.w = reinterpret_cast<const uint32_t*>(data);
  p.flags = flags;
  p.group = group_size;
  p.ng = static_cast<int>(k / group_size);
  p.zw = (p.ng + 7) / 8;
  p.scales = scales;
  p.scale_f32 = scales_dtype == QG_F32;
  p.zeros = zeros;
  p.out = out;
  p.out_dtype = out_dtype;
  return qg::launch_w4_unpack(p, static_cast<hipStream_t>(stream));
}

namespace {

// Prefill grids (more than kW4TiledMinRows rows, K a multiple of the
// 64-element stage) with at least as many tiles of 256 x 192 as the dequant
// formulation needs to beat the fused tiled kernel at that group size: W is
// dequantised once into the workspace as the activation dtype, (q - z) * s in
// fp32 rounded once (the reference's dequant method,
// int4_weight_gemm_v07.py:549-554), then the 2-byte ping-pong GEMM runs on
// it. Group 128: 192 tiles (the INT8 kernel's large-grid rule); group 64: 64
// tiles (1061 x 3072 x 3072, 80 tiles: 54-58 us against 74-89 us); group 32:
// every grid (its four group folds per 128-wide stage make the tiled kernel
// 2-3x slower: 57-60 against 129-169 us at 1061 x 3072, 71-80 against 86-112
// us at 512 x 4096, 44 tiles). Returns the workspace bytes (0: the fused
// tiled kernel).
size_t w4_prefill_bytes(int64_t m, int64_t n, int64_t k, int group_size) {
  const int64_t tiles = ((m + 255) / 256) * ((n + 191) / 192);
  const int64_t min_tiles = group_size == 32 ? 1 : group_size == 64 ? 64 : 192;
  if (m <= kW4TiledMinRows || k % 64 != 0 || tiles < min_tiles) return 0;
  if (2 * n * k >= kMaxOperandBytes) return 0;
  return static_cast<size_t>(round_up(2 * n * k, 256));
}

}  // namespace

extern "C" size_t qg_w4a16_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int group_size,
                                                int flags) {
  if (!valid_w4_shape(n, k, group_size, flags) || m < 0 || m > kIntMax) return 0;
  return w4_prefill_bytes(m, n, k, group_size);
}

extern "C" int qg_w4a8_gemm(const int8_t* a, int64_t a_sm, int64_t m, int64_t k, const int32_t* w, int64_t n,
                            int group_size, int flags, const void* scales, int scales_dtype, const void* zeros,
                            const int8_t* prepared, int64_t prepared_sn, const float* a_scale, const void* bias,
                            int bias_dtype, void* out, int integer, void* stream) {
  if (!valid_w4_shape(n, k, group_size, flags)) return hipErrorInvalidValue;
  if (m < 0 || m > kIntMax || m * n >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  // the integer bound of int4_weight_gemm_v07.py:493 (k * 128 * 15 < 2^31)
  if (k * 128 * 15 >= (int64_t(1) << 31) || (integer != 0 && integer != 1)) return hipErrorInvalidValue;
  if (scales_dtype != QG_F32 && scales_dtype != QG_BF16) return hipErrorInvalidValue;
  if (bias && !float_dtype(bias_dtype)) return hipErrorInvalidValue;
  // activation rows are copied as 16-byte chunks
  if (a_sm < k || a_sm % 16 != 0) return hipErrorInvalidValue;
  if (prepared && (prepared_sn < k || prepared_sn % 16 != 0)) return hipErrorInvalidValue;
  if (m == 0) return hipSuccess;
  if (!a || !aligned16(a) || !out || (!integer && !a_scale)) return hipErrorInvalidValue;
  if (prepared ? (!aligned16(prepared) || (n - 1) * prepared_sn + k >= kMaxOperandBytes)
               : (!w || !zeros || !aligned16(w)))
    return hipErrorInvalidValue;
  if (!integer && !scales) return hipErrorInvalidValue;
  // activation addresses are 32-bit byte offsets from the base
  if ((m - 1) * a_sm + k >= kMaxOperandBytes) return hipErrorInvalidValue;
  qg::W4A8Args p{};
  p.a = a;
  p.a_sm = a_sm;
  p.M = static_cast<int>(m);
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(k);
  p.w = reinterpret_cast<const uint32_t*>(w);
  p.w8 = prepared;
  p.w8_sn = prepared_sn;
  p.flags = flags;
  p.group = group_size;
  p.ng = static_cast<int>(k / group_size);
  p.zw = (p.ng + 7) / 8;
  p.scales = scales;
  p.scale_f32 = scales_dtype == QG_F32;
  p.zeros = zeros;
  p.a_scale = a_scale;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.out = out;
  p.integer = integer;
  return qg::launch_w4a8_gemm(p, static_cast<hipStream_t>(stream));
}

extern "C" int qg_w4a16_gemm(const void* a, int a_dtype, int64_t a_sm, int64_t m, int64_t k,
                             const int32_t* w, int64_t n, int group_size, int flags,
                             const void* scales, int scales_dtype, const void* zeros,
                             const void* bias, int bias_dtype, void* out, int out_dtype,
                             void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_w4_shape(n, k, group_size, flags)) return hipErrorInvalidValue;
  if (m < 0 || m > kIntMax || m * n >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  if (a_dtype != QG_F16 && a_dtype != QG_BF16) return hipErrorInvalidValue;
  if (scales_dtype != QG_F32 && scales_dtype != QG_BF16) return hipErrorInvalidValue;
  if (!float_dtype(out_dtype) || (bias && !float_dtype(bias_dtype))) return hipErrorInvalidValue;
  // activation rows are read as 16-byte vectors
  if (a_sm < k || a_sm % 8 != 0) return hipErrorInvalidValue;
  if (m == 0) return hipSuccess;
  if (!a || !w || !scales || !zeros || !out) return hipErrorInvalidValue;
  if (!aligned16(a) || !aligned16(w)) return hipErrorInvalidValue;
  // activation addresses are 32-bit byte offsets from the base
  if ((m - 1) * a_sm + k >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  qg::W4Args p{};
  p.a = static_cast<const uint16_t*>(a);
  p.a_sm = a_sm;
  p.a_f16 = a_dtype == QG_F16;
  p.M = static_cast<int>(m);
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(k);
  p.w = reinterpret_cast<const uint32_t*>(w);
  p.flags = flags;
  p.group = group_size;
  p.ng = static_cast<int>(k / group_size);
  p.zw = (p.ng + 7) / 8;
  p.scales = scales;
  p.scale_f32 = scales_dtype == QG_F32;
  p.zeros = zeros;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.out = out;
  p.out_dtype = out_dtype;
  // prefill grids past the group's tile threshold: dequantise W into the
  // workspace, then the 2-byte ping-pong GEMM (out = acc + bias, one rounding)
  const size_t need = w4_prefill_bytes(m, n, k, group_size);
  if (need > 0) {
    if (!workspace || workspace_bytes < need || !aligned16(workspace)) return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    qg::W4Args u = p;
    u.out = workspace;
    u.out_dtype = a_dtype;
    hipError_t e = qg::launch_w4_unpack(u, s);
    if (e != hipSuccess) return e;
    qg::I8GemmArgs g{};
    g.a = static_cast<const int8_t*>(a);
    g.a_sm = a_sm;
    g.w = static_cast<const int8_t*>(workspace);
    g.w_sn = k;
    g.M = p.M;
    g.N = p.N;
    g.K = p.K;
    g.a_scale = nullptr;
    g.b_scale = nullptr;
    g.b_scalar = 0;
    g.bias = bias;
    g.bias_dtype = bias_dtype;
    g.out = out;
    g.out_dtype = out_dtype;
    g.epi = 0;
    return qg::launch_h16_gemm(g, p.a_f16 != 0, s);
  }
  // large M: the tiled kernel (activation rows staged in LDS, 128-wide K stages)
  if (m > kW4TiledMinRows && k % 128 == 0) {
    qg::WdArgs t{};
    t.a = p.a;
    t.a_sm = p.a_sm;
    t.a_f16 = p.a_f16;
    t.M = p.M;
    t.N = p.N;
    t.K = p.K;
    t.w4 = p.w;
    t.flags = p.flags;
    t.group = p.group;
    t.ng = p.ng;
    t.zw = p.zw;
    t.scales = p.scales;
    t.scale_f32 = p.scale_f32;
    t.zeros = p.zeros;
    t.bias = bias;
    t.bias_dtype = bias_dtype;
    t.out = out;
    t.out_dtype = out_dtype;
    return qg::launch_wd_w4(t, static_cast<hipStream_t>(stream));
  }
  return qg::launch_w4a16(p, static_cast<hipStream_t>(stream));
}

// --------------------------------------------------------------------------
// FP8 weights.
namespace {

bool fp8_dtype(int d) { return d == QG_E4M3 || d == QG_E5M2; }

// Operands of the tiled kernel: unit K stride, 16-byte aligned rows, K a
// multiple of the 128-wide stage; anything else is packed into workspace.
struct Fp8Plan {
  bool pack_a, pack_w;
  bool pingpong;  // large grid: the ping-pong GEMM with fp8 W stages converted in registers
  int64_t kp;
  size_t a_bytes, w_bytes;
  size_t total() const { return a_bytes + w_bytes; }
};

Fp8Plan plan_fp8(const void* a, int64_t a_sm, int64_t a_sk, const void* w, int64_t w_sn, int64_t w_sk,
                 int64_t m, int64_t n, int64_t k) {
  Fp8Plan pl;
  pl.kp = round_up(k, kStageK);
  // In place only when every row's byte offset fits the kernels' 32-bit
  // offsets: the span of the last row ends below 2 GiB.
  pl.pack_a = !(a_sk == 1 && a_sm % 8 == 0 && aligned16(a) && k % kStageK == 0 &&
                2 * ((m - 1) * a_sm + k) < kMaxOperandBytes);
  pl.pack_w = !(w_sk == 1 && w_sn % 16 == 0 && aligned16(w) && k % kStageK == 0 &&
                (n - 1) * w_sn + k < kMaxOperandBytes);
  pl.a_bytes = pl.pack_a ? static_cast<size_t>(round_up(2 * m * pl.kp, 256)) : 0;
  pl.w_bytes = pl.pack_w ? static_cast<size_t>(round_up(n * pl.kp, 256)) : 0;
  // >= 192 tiles of 256 x 192 (the INT8 kernel's large-grid rule): the
  // ping-pong GEMM, fp8 W converted exactly to A's 2-byte type in registers
  const int64_t tiles = ((m + 255) / 256) * ((n + 191) / 192);
  pl.pingpong = tiles >= 192 && 2 * m * pl.kp < kMaxOperandBytes;
  return pl;
}

bool valid_fp8_shape(int64_t m, int64_t n, int64_t k, int64_t a_sm, int64_t a_sk, int64_t w_sn, int64_t w_sk) {
  if (m < 0 || n < 0 || k < 0 || m > kIntMax || n > kIntMax || k > kIntMax) return false;
  if (a_sm < 0 || a_sk < 0 || w_sn < 0 || w_sk < 0) return false;
  return m * n < (int64_t(1) << 40);
}

}  // namespace

extern "C" int qg_fp8_decode(const uint8_t* w, int w_dtype, int64_t w_sn, int64_t w_sk, int64_t n, int64_t k,
                             void* out, int out_dtype, void* stream) {
  if (!fp8_dtype(w_dtype) || !float_dtype(out_dtype)) return hipErrorInvalidValue;
  if (n < 0 || k < 0 || w_sn < 0 || w_sk < 0 || n * k >= (int64_t(1) << 40)) return hipErrorInvalidValue;
  if (n == 0 || k == 0) return hipSuccess;
  if (!w || !out) return hipErrorInvalidValue;
  return qg::launch_fp8_decode(w, w_sn, w_sk, n, k, w_dtype == QG_E5M2, out, out_dtype,
                               static_cast<hipStream_t>(stream));
}

extern "C" size_t qg_fp8w_gemm_workspace_bytes(const void* a, int64_t a_sm, int64_t a_sk, const uint8_t* w,
                                               int64_t w_sn, int64_t w_sk, int64_t m, int64_t n, int64_t k) {
  if (!valid_fp8_shape(m, n, k, a_sm, a_sk, w_sn, w_sk)) return 0;
  return plan_fp8(a, a_sm, a_sk, w, w_sn, w_sk, m, n, k).total();
}

extern "C" int qg_fp8w_gemm(const void* a, int a_dtype, int64_t a_sm, int64_t a_sk, int64_t m, int64_t k,
                            const uint8_t* w, int w_dtype, int64_t w_sn, int64_t w_sk, int64_t n,
                            const float* w_scale, const void* bias, int bias_dtype, void* out, int out_dtype,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_fp8_shape(m, n, k, a_sm, a_sk, w_sn, w_sk)) return hipErrorInvalidValue;
  if ((a_dtype != QG_F16 && a_dtype != QG_BF16) || !fp8_dtype(w_dtype)) return hipErrorInvalidValue;
  if (!float_dtype(out_dtype) || (bias && !float_dtype(bias_dtype))) return hipErrorInvalidValue;
  if (m == 0 || n == 0) return hipSuccess;
  if (!out || (k > 0 && (!a || !w))) return hipErrorInvalidValue;
  const Fp8Plan pl = plan_fp8(a, a_sm, a_sk, w, w_sn, w_sk, m, n, k);
  if (pl.total() > 0 && (!workspace || workspace_bytes < pl.total() || !aligned16(workspace)))
    return hipErrorInvalidValue;
  // 32-bit byte offsets inside the kernel
  if (2 * m * pl.kp >= kMaxOperandBytes * 2 || n * pl.kp >= kMaxOperandBytes) return hipErrorInvalidValue;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  qg::WdArgs p{};
  p.M = static_cast<int>(m);
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(pl.kp);
  p.a_f16 = a_dtype == QG_F16;
  if (pl.pack_a) {
    uint16_t* pa = reinterpret_cast<uint16_t*>(ws);
    hipError_t e = qg::launch_pack_rows_u16(static_cast<const uint16_t*>(a), a_sm, a_sk, m, k, pa, pl.kp, s);
    if (e != hipSuccess) return e;
    p.a = pa;
    p.a_sm = pl.kp;
  } else {
    p.a = static_cast<const uint16_t*>(a);
    p.a_sm = a_sm;
  }
  if (pl.pack_w) {
    int8_t* pw = reinterpret_cast<int8_t*>(ws + pl.a_bytes);
    hipError_t e = qg::launch_pack_rows_i8(reinterpret_cast<const int8_t*>(w), w_sn, w_sk, n, k, pw, pl.kp, s);
    if (e != hipSuccess) return e;
    p.w8 = reinterpret_cast<const uint8_t*>(pw);
    p.w8_sn = pl.kp;
  } else {
    p.w8 = w;
    p.w8_sn = w_sn;
  }
  p.fp8_e5 = w_dtype == QG_E5M2;
  p.w_scale = w_scale;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.out = out;
  p.out_dtype = out_dtype;
  if (pl.pingpong && k > 0) {
    // every fp8 value is exact in fp16 and bf16: the 2-byte ping-pong GEMM with
    // the W fragments converted in registers (same fp32 products, order F)
    qg::I8GemmArgs g{};
    g.a = reinterpret_cast<const int8_t*>(p.a);
    g.a_sm = p.a_sm;
    g.w = reinterpret_cast<const int8_t*>(p.w8);
    g.w_sn = p.w8_sn;
    g.M = p.M;
    g.N = p.N;
    g.K = p.K;
    g.a_scale = nullptr;
    g.b_scale = w_scale;
    g.b_scalar = 0;
    g.bias = bias;
    g.bias_dtype = bias_dtype;
    g.out = out;
    g.out_dtype = out_dtype;
    g.epi = 0;
    return qg::launch_f8w_gemm(g, p.a_f16 != 0, p.fp8_e5 != 0, s);
  }
  return qg::launch_wd_fp8(p, s);  // k == 0: no stage, out = bias (or 0)
}

// ------------------------------------------------------------------- MoE
namespace {

bool moe_sizes(int64_t tokens, int n_experts, int top_k, int pad, int64_t* rows_max, int64_t* tiles_max) {
  if (tokens < 0 || n_experts < 1 || n_experts > 64 || top_k < 1 || top_k > n_experts || pad < 1 || pad > 4096)
    return false;
  const int64_t rows = tokens * top_k + static_cast<int64_t>(n_experts) * (pad - 1);
  if (rows >= (int64_t(1) << 30)) return false;
  *rows_max = rows;
  *tiles_max = (rows + QG_MOE_TILE_ROWS - 1) / QG_MOE_TILE_ROWS + n_experts;
  return true;
}

}  // namespace

extern "C" int qg_moe_sizes(int64_t tokens, int n_experts, int top_k, int pad, int64_t* rows_max,
                            int64_t* tiles_max) {
  if (!rows_max || !tiles_max) return hipErrorInvalidValue;
  return moe_sizes(tokens, n_experts, top_k, pad, rows_max, tiles_max) ? hipSuccess : hipErrorInvalidValue;
}

namespace {

// Argument checks and arguments of qg_moe_dispatch (x fields left empty).
hipError_t moe_dispatch_args(const float* logits, int64_t l_sm, int64_t tokens, int n_experts, int top_k, int pad,
                             int32_t* experts, float* weights, int32_t* counts, int32_t* row_token,
                             float* row_weight, int32_t* row_slot, int64_t rows_max, int32_t* tiles,
                             int64_t tiles_max, qg::MoeDispatchArgs* out) {
  int64_t need_rows = 0, need_tiles = 0;
  if (!moe_sizes(tokens, n_experts, top_k, pad, &need_rows, &need_tiles)) return hipErrorInvalidValue;
  if (rows_max < need_rows || tiles_max < need_tiles || rows_max >= (int64_t(1) << 30) ||
      tiles_max >= (int64_t(1) << 30))
    return hipErrorInvalidValue;
  if (l_sm < n_experts || (tokens > 0 && (!logits || !experts || !weights))) return hipErrorInvalidValue;
  if (!counts || !row_token || !row_weight || !row_slot || !tiles) return hipErrorInvalidValue;
  if (tokens * l_sm >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  qg::MoeDispatchArgs p{};
  p.logits = logits;
  p.l_sm = l_sm;
  p.T = static_cast<int>(tokens);
  p.E = n_experts;
  p.top_k = top_k;
  p.pad = pad;
  p.experts = experts;
  p.weights = weights;
  p.counts = counts;
  p.row_token = row_token;
  p.row_weight = row_weight;
  p.row_slot = row_slot;
  p.rows_max = static_cast<int>(rows_max);
  p.tiles = tiles;
  p.tiles_max = static_cast<int>(tiles_max);
  p.tile_rows = QG_MOE_TILE_ROWS;
  *out = p;
  return hipSuccess;
}

}  // namespace

extern "C" int qg_moe_dispatch(const float* logits, int64_t l_sm, int64_t tokens, int n_experts, int top_k,
                               int pad, int32_t* experts, float* weights, int32_t* counts, int32_t* row_token,
                               float* row_weight, int32_t* row_slot, int64_t rows_max, int32_t* tiles,
                               int64_t tiles_max, void* stream) {
  qg::MoeDispatchArgs p{};
  const hipError_t e = moe_dispatch_args(logits, l_sm, tokens, n_experts, top_k, pad, experts, weights, counts,
                                         row_token, row_weight, row_slot, rows_max, tiles, tiles_max, &p);
  if (e != hipSuccess) return e;
  return qg::launch_moe_dispatch(p, static_cast<hipStream_t>(stream));
}

extern "C" int qg_moe_dispatch_qx(const float* logits, int64_t l_sm, int64_t tokens, int n_experts, int top_k,
                                  int pad, int32_t* experts, float* weights, int32_t* counts, int32_t* row_token,
                                  float* row_weight, int32_t* row_slot, int64_t rows_max, int32_t* tiles,
                                  int64_t tiles_max, const void* x, int64_t x_sm, int64_t hidden, int8_t* xq,
                                  int64_t xq_sm, float* xs, void* stream) {
  qg::MoeDispatchArgs p{};
  const hipError_t e = moe_dispatch_args(logits, l_sm, tokens, n_experts, top_k, pad, experts, weights, counts,
                                         row_token, row_weight, row_slot, rows_max, tiles, tiles_max, &p);
  if (e != hipSuccess) return e;
  if (hidden <= 0 || hidden % 8 != 0 || hidden > qg::kMoeRouteQuantMaxH || x_sm < hidden || x_sm % 8 != 0 ||
      xq_sm < hidden || xq_sm % 8 != 0)
    return hipErrorInvalidValue;
  if (tokens > 0 && (!x || !xq || !xs || (reinterpret_cast<uintptr_t>(x) & 15) != 0 ||
                     (reinterpret_cast<uintptr_t>(xq) & 7) != 0))
    return hipErrorInvalidValue;
  if (tokens * x_sm >= (int64_t(1) << 40) || tokens * xq_sm >= (int64_t(1) << 40)) return hipErrorInvalidValue;
  p.x = static_cast<const uint16_t*>(x);
  p.x_sm = x_sm;
  p.H = static_cast<int>(hidden);
  p.xq = xq;
  p.xq_sm = xq_sm;
  p.xs = xs;
  return qg::launch_moe_dispatch(p, static_cast<hipStream_t>(stream));
}

extern "C" int qg_moe_grouped_gemm(const int8_t* a, int64_t a_sm, int64_t a_rows, const int32_t* row_token,
                                   int64_t rows_max, int64_t k, const int8_t* w, int64_t w_sn, int64_t w_estride,
                                   int64_t n, int n_experts, const int32_t* tiles, int64_t tiles_max,
                                   const float* a_scale, const float* b_scale, const float* row_weight,
                                   const int32_t* row_slot, int epilogue, void* out, int64_t out_sm,
                                   int64_t out_rows, void* stream) {
  if (epilogue < QG_MOE_EPI_I32 || epilogue > QG_MOE_EPI_ROUTE) return hipErrorInvalidValue;
  if (a_rows < 1 || rows_max < 1 || k < 1 || n < 1 || n_experts < 1 || tiles_max < 0) return hipErrorInvalidValue;
  if (k % kStageK != 0 || a_sm < k || a_sm % 16 != 0 || w_sn < k || w_sn % 16 != 0 || w_estride < n * w_sn ||
      w_estride % 16 != 0)
    return hipErrorInvalidValue;
  if (!a || !w || !tiles || !out || !aligned16(a) || !aligned16(w)) return hipErrorInvalidValue;
  // 32-bit byte offsets from the A base and from each expert's W base
  if (a_rows * a_sm >= kMaxOperandBytes || n * w_sn >= kMaxOperandBytes || rows_max >= (int64_t(1) << 30) ||
      tiles_max >= (int64_t(1) << 24))
    return hipErrorInvalidValue;
  if (!row_token && a_rows < rows_max) return hipErrorInvalidValue;
  const int64_t out_cols = epilogue == QG_MOE_EPI_SILU_MUL ? n / 2 : n;
  if (out_sm < out_cols) return hipErrorInvalidValue;
  // rows of out: every routed row (int32 / SiLU*mul) or every slot (route)
  if (out_rows < 1 || out_rows >= (int64_t(1) << 30) || out_rows * out_sm >= (int64_t(1) << 31) ||
      (epilogue != QG_MOE_EPI_ROUTE && out_rows < rows_max))
    return hipErrorInvalidValue;
  if (epilogue != QG_MOE_EPI_I32 && (!a_scale || !b_scale)) return hipErrorInvalidValue;
  if (epilogue == QG_MOE_EPI_SILU_MUL && n % 32 != 0) return hipErrorInvalidValue;
  if (epilogue == QG_MOE_EPI_ROUTE && (!row_weight || !row_slot)) return hipErrorInvalidValue;
  // work items (tiles x 256-column tiles): each workgroup holds its share's
  // table entries in LDS (launch_i8_moe_gemm checks the same bound)
  if (tiles_max * ((n + 255) / 256) > kMoeMaxItems) return hipErrorInvalidValue;
  if (tiles_max == 0) return hipSuccess;
  qg::I8GemmArgs p{};
  p.a = a;
  p.a_sm = a_sm;
  p.w = w;
  p.w_sn = w_sn;
  p.M = static_cast<int>(rows_max);
  p.N = static_cast<int>(n);
  p.K = static_cast<int>(k);
  p.a_scale = a_scale;
  p.b_scale = b_scale;
  p.out = out;
  p.tiles = tiles;
  p.tiles_max = static_cast<int>(tiles_max);
  p.row_token = row_token;
  p.a_rows = static_cast<int>(a_rows);
  p.w_estride = w_estride;
  p.row_weight = row_weight;
  p.row_slot = row_slot;
  p.out_sm = out_sm;
  p.out_rows = static_cast<int>(out_rows);
  p.n_experts = n_experts;
  p.moe_epi = epilogue;
  return qg::launch_i8_moe_gemm(p, static_cast<hipStream_t>(stream));
}

extern "C" int qg_moe_combine(const void* y, int64_t tokens, int top_k, int64_t hidden, void* out, int64_t out_sm,
                              void* stream) {
  if (tokens < 0 || top_k < 1 || hidden < 1 || out_sm < hidden) return hipErrorInvalidValue;
  if (tokens == 0) return hipSuccess;
  if (!y || !out || tokens * top_k * hidden >= (int64_t(1) << 31) || tokens * out_sm >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  return qg::launch_moe_combine(static_cast<const uint16_t*>(y), static_cast<int>(tokens), top_k,
                                static_cast<int>(hidden), static_cast<uint16_t*>(out), out_sm,
                                static_cast<hipStream_t>(stream));
}
