// INT8 x INT8 -> INT32 GEMM on gfx950 int8 MFMA with the fused dequant
// epilogue of rdna2-ops/rdna2_ops/int8_gemm.py:19-67 (and the Kitchen eager
// epilogue order of rdna2-ops/rdna2_ops/comfy_int8.py:128-143).
//
// Design (MI355X-first, not a translation of the reference's Triton tiles):
//  * one 256-thread workgroup (4 waves, 2x2) per BM x BN output tile; each wave
//    owns a (BM/2) x (BN/2) sub-tile held in 16x16 int32 MFMA accumulators;
//  * operands are A [M, K] and W [N, K], both K-contiguous ("NT"), so every
//    lane feeds v_mfma_i32_16x16x64_i8 with 16 contiguous K bytes;
//  * K advances in 64-byte stages; each stage of A and W is copied straight
//    from HBM into LDS with global_load_lds_dwordx4 (no VGPR staging) into a
//    4-deep ring, so three stages are in flight while one is consumed;
//  * LDS rows are 64 bytes with the 16-byte chunk index XOR-swizzled by
//    (row >> 1) & 3, which makes both the DMA writes and the MFMA fragment
//    reads (8 consecutive lanes = 8 distinct 16-byte bank groups) conflict free;
//  * the linear block id is remapped so that each of the 8 XCDs (round-robin
//    workgroup dispatch) walks one contiguous, GROUP_M-ordered range of tiles,
//    keeping the A rows and W columns it shares in its own L2.
#include "qg_common.h"
#include "qg_internal.h"

namespace qg {

namespace {

template <int BM, int BN>
struct I8Tile {
  static constexpr int WM = BM / 2, WN = BN / 2;  // wave sub-tile
  static constexpr int FM = WM / 16, FN = WN / 16;  // 16x16 fragments per wave
  static constexpr int KS = 64;                    // K bytes per stage
  static constexpr int STAGE_A = BM * KS, STAGE_B = BN * KS;
  static constexpr int STAGE = STAGE_A + STAGE_B;
  static constexpr int NST = 4;                    // LDS ring depth
  static constexpr int SEGS = (BM + BN) / 16;      // 1 KB DMA segments per stage
  static constexpr int SEG_PER_WAVE = SEGS / 4;
  static_assert(BM % 32 == 0 && BN % 32 == 0, "tile must split into 2x2 waves of 16-multiples");
  static_assert(SEGS % 4 == 0, "DMA segments must divide over 4 waves");
};

__device__ __forceinline__ float gelu_tanh(float x) {
#pragma clang fp contract(off)
  // 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3))), evaluated in the
  // operation order of ATen's CPU GeluKernel (tanh approximation).
  const float kBeta = 0.7978845608028654f;
  const float kKappa = 0.044715f;
  const float x_cube = x * x * x;
  const float inner = kBeta * (x + kKappa * x_cube);
  return 0.5f * x * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float load_bias(const void* bias, int dtype, int col) {
  if (dtype == QG_F32) return static_cast<const float*>(bias)[col];
  const uint16_t b = static_cast<const uint16_t*>(bias)[col];
  return dtype == QG_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

// Round an fp32 value to the output dtype and back (identity for fp32).
__device__ __forceinline__ float round_to(float v, int dtype) {
  if (dtype == QG_F16) return f16_to_f32(f32_to_f16(v));
  if (dtype == QG_BF16) return bf16_to_f32(f32_to_bf16(v));
  return v;
}

__device__ __forceinline__ void store_out(void* out, int dtype, int64_t idx, float v) {
  if (dtype == QG_F32) static_cast<float*>(out)[idx] = v;
  else if (dtype == QG_F16) static_cast<uint16_t*>(out)[idx] = f32_to_f16(v);
  else static_cast<uint16_t*>(out)[idx] = f32_to_bf16(v);
}

// Epilogue of one 16x16 fragment: this lane holds rows row..row+3 of column
// col. Order F (default): v = f32(acc) * (sa * sb); v = v + bias; act; round.
__device__ __forceinline__ void store_frag(const I8GemmArgs& p, const i32x4 acc, int row, int col) {
#pragma clang fp contract(off)
  if (col >= p.N) return;
  if (p.a_scale == nullptr) {
    int32_t* out = static_cast<int32_t*>(p.out);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (row + r < p.M) out[static_cast<int64_t>(row + r) * p.N + col] = acc[r];
    return;
  }
  const float sb = p.b_scalar ? p.b_scale[0] : p.b_scale[col];
  const bool has_bias = p.bias != nullptr;
  const float bv = has_bias ? load_bias(p.bias, p.bias_dtype, col) : 0.0f;
  const bool fused_fma = (p.epi & QG_EPI_ORDER_FUSED_FMA) != 0;
  const bool eager = (p.epi & QG_EPI_ORDER_EAGER) != 0;
  const bool gelu = (p.epi & QG_EPI_GELU_TANH) != 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (row + r >= p.M) continue;
    const float scale = p.a_scale[row + r] * sb;
    const float accf = static_cast<float>(acc[r]);
    float v;
    if (eager) {
      v = round_to(accf * scale, p.out_dtype);
      if (has_bias) v = v + round_to(bv, p.out_dtype);
    } else if (fused_fma && has_bias) {
      v = __builtin_fmaf(accf, scale, bv);
    } else {
      v = accf * scale;
      if (has_bias) v = v + bv;
    }
    if (gelu) v = gelu_tanh(v);
    store_out(p.out, p.out_dtype, static_cast<int64_t>(row + r) * p.N + col, v);
  }
}

template <int BM, int BN, int WPE>
__global__ __launch_bounds__(256, WPE) void k_i8_gemm(I8GemmArgs p) {
#pragma clang fp contract(off)
  using T = I8Tile<BM, BN>;
  __shared__ __attribute__((aligned(1024))) char smem[T::NST * T::STAGE];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
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

  // ---- DMA plan: this wave copies SEG_PER_WAVE 1 KB segments per stage ------
  // Segment lane i lands on LDS row (i >> 2) of the segment, physical chunk
  // (i & 3); it fetches the logical chunk that the swizzle stores there.
  const char* src[T::SEG_PER_WAVE];
  uint32_t dst[T::SEG_PER_WAVE];
  {
    const int srow = lane >> 2;
    const int schunk = (lane & 3) ^ ((lane >> 3) & 3);
#pragma unroll
    for (int i = 0; i < T::SEG_PER_WAVE; ++i) {
      const int seg = wave + 4 * i;
      if (seg < BM / 16) {
        const int row = min(m0 + seg * 16 + srow, p.M - 1);
        src[i] = reinterpret_cast<const char*>(p.a) + static_cast<int64_t>(row) * p.a_sm + schunk * 16;
        dst[i] = seg * 1024;
      } else {
        const int sb = seg - BM / 16;
        const int col = min(n0 + sb * 16 + srow, p.N - 1);
        src[i] = reinterpret_cast<const char*>(p.w) + static_cast<int64_t>(col) * p.w_sn + schunk * 16;
        dst[i] = T::STAGE_A + sb * 1024;
      }
    }
  }
  const uint32_t smem_base = lds_addr_of(smem);
  auto issue = [&](int s, int slot) {
    const int64_t koff = static_cast<int64_t>(s) * T::KS;
#pragma unroll
    for (int i = 0; i < T::SEG_PER_WAVE; ++i)
      dma16(src[i] + koff, smem_base + slot * T::STAGE + dst[i]);
  };

  // Fragment read offset of this lane inside a 16-row block (same for A and W).
  const int lane_off = (lane & 15) * T::KS + (((lane >> 4) ^ ((lane >> 1) & 3)) << 4);

  i32x4 acc[T::FM][T::FN];
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < T::FN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

  const int S = p.K / T::KS;
#pragma unroll
  for (int s = 0; s < T::NST - 1; ++s)
    if (s < S) issue(s, s);

  for (int s = 0; s < S; ++s) {
    const int ahead = min(S - 1 - s, T::NST - 2);
    if (ahead >= 2) wait_vm_barrier<2 * T::SEG_PER_WAVE>();
    else if (ahead == 1) wait_vm_barrier<T::SEG_PER_WAVE>();
    else wait_vm_barrier<0>();
    if (s + T::NST - 1 < S) issue(s + T::NST - 1, (s + T::NST - 1) % T::NST);

    const char* base = smem + (s % T::NST) * T::STAGE;
    i32x4 af[T::FM], bf[T::FN];
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
      af[i] = *reinterpret_cast<const i32x4*>(base + (wr * T::WM + i * 16) * T::KS + lane_off);
#pragma unroll
    for (int j = 0; j < T::FN; ++j)
      bf[j] = *reinterpret_cast<const i32x4*>(base + T::STAGE_A + (wc * T::WN + j * 16) * T::KS + lane_off);
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
      for (int j = 0; j < T::FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
  }

  // ---- epilogue: lane holds rows 4*(lane>>4)+r, column lane&15 of each frag --
  const int row0 = m0 + wr * T::WM + 4 * (lane >> 4);
  const int col0 = n0 + wc * T::WN + (lane & 15);
  static_for<0, T::FN>([&](auto j) {
    static_for<0, T::FM>([&](auto i) { store_frag(p, acc[i][j], row0 + i * 16, col0 + j * 16); });
  });
}

template <int BM, int BN, int WPE>
hipError_t launch_tile(const I8GemmArgs& p, hipStream_t stream) {
  const int blocks = ceil_div(p.M, BM) * ceil_div(p.N, BN);
  hipLaunchKernelGGL((k_i8_gemm<BM, BN, WPE>), dim3(blocks), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_i8_gemm(const I8GemmArgs& p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  // 256x192 tiles tile every BASELINE shape into whole multiples of the 256
  // CUs (4096x3072 -> 256 tiles, x9216 -> 768, x12288 -> 1024). Smaller
  // problems use 128x128 tiles so that more CUs get work.
  const long big = static_cast<long>(ceil_div(p.M, 256)) * ceil_div(p.N, 192);
  if (big >= 192) return launch_tile<256, 192, 1>(p, stream);
  return launch_tile<128, 128, 2>(p, stream);
}

}  // namespace qg
