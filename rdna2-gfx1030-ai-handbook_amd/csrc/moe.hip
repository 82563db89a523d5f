// MoE prefill routing, dispatch and combine on gfx950 (BASELINE configuration
// 4; the reference repository has no MoE kernel). The grouped INT8 GEMM that
// runs between dispatch and combine is k_i8_moe_pp in int8_gemm.hip.
//
//   init     zero the per-expert counters, mark every routed row as padding
//            and every tile as empty (no memset node: safe under graph capture)
//   route    one wave per token, lane e = expert e: softmax over the experts
//            in fp32 and the top_k experts by logit (ties: lower index)
//   count    a stable counting sort of the tokens * top_k slots in three
//   plan     steps: per-block expert histograms (blocks of kSortBlock slots,
//   scatter  LDS atomics); one workgroup turns them into per-expert segments
//            padded to `pad` rows, each block's first row per expert and the
//            table of tile_rows-row tiles of the grouped GEMM (tile 0's spare
//            field holds the number of tiles in use); then every slot's row =
//            its block's base + earlier waves of the block + its rank among
//            equal experts of its 64-slot step (six ballots). Rows inside a
//            segment are in slot order, so the dispatch is deterministic
//   combine  out[t] = bf16(sum over k of y[t * top_k + k]) in k order (fp32)
#include "qg_common.h"
#include "qg_internal.h"

namespace qg {

namespace {

constexpr int kSortBlock = 1024;      // slots per sort block (at least)
constexpr int kMaxSortBlocks = 256;

__global__ __launch_bounds__(256) void k_moe_init(MoeDispatchArgs p) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < p.rows_max; i += stride) {
    p.row_token[i] = -1;
    p.row_slot[i] = -1;
    p.row_weight[i] = 0.0f;
  }
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < p.tiles_max; i += stride) {
    p.tiles[4 * i] = -1;
    p.tiles[4 * i + 1] = 0;
    p.tiles[4 * i + 2] = 0;
    p.tiles[4 * i + 3] = 0;
  }
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < 3 * p.E; i += 256) p.counts[i] = 0;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, kWave);
  return v;
}

__global__ __launch_bounds__(256) void k_moe_route(MoeDispatchArgs p) {
#pragma clang fp contract(off)
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= p.T) return;  // whole wave
  const int e = threadIdx.x & 63;
  const bool live = e < p.E;
  const float l = live ? p.logits[static_cast<int64_t>(t) * p.l_sm + e] : -__builtin_inff();
  const float mx = wave_max(l);
  const float ex = live ? __builtin_amdgcn_exp2f((l - mx) * 1.4426950408889634f) : 0.0f;
  const float prob = __fdiv_rn(ex, wave_sum(ex));
  bool taken = false;
  for (int k = 0; k < p.top_k; ++k) {
    const bool cand_ok = live && !taken;
    const float cand = cand_ok ? l : -__builtin_inff();
    const float mk = wave_max(cand);
    uint64_t win = __ballot(cand_ok && cand == mk);
    if (win == 0) win = __ballot(cand_ok);  // NaN logits: lowest free expert
    const int w = static_cast<int>(__builtin_ctzll(win));
    if (e == w) {
      taken = true;
      p.experts[static_cast<int64_t>(t) * p.top_k + k] = e;
      p.weights[static_cast<int64_t>(t) * p.top_k + k] = prob;
    }
  }
}

// Lanes of the wave whose value of e (< 64) equals this lane's, among the
// lanes in `valid`.
__device__ __forceinline__ uint64_t match_expert(int e, uint64_t valid) {
  uint64_t m = valid;
#pragma unroll
  for (int b = 0; b < 6; ++b) {
    const uint64_t bal = __ballot((e >> b) & 1);
    m &= ((e >> b) & 1) ? bal : ~bal;
  }
  return m;
}

// counts layout: [0, E) counts, [E, 2E) segment offsets, [2E, 3E) spare,
// then [kMaxSortBlocks][E] per-block histograms / first rows (the workspace
// holds (3 + 256) E ints).
__host__ __device__ __forceinline__ int sort_block_size(int slots) {
  const int b = (ceil_div(slots, kMaxSortBlocks) + 255) / 256 * 256;
  return b > kSortBlock ? b : kSortBlock;
}

__global__ __launch_bounds__(256) void k_moe_count(MoeDispatchArgs p) {
  __shared__ int hist[64];
  const int slots = p.T * p.top_k;
  const int bs = sort_block_size(slots);
  const int b = blockIdx.x;
  if (threadIdx.x < 64) hist[threadIdx.x] = 0;
  __syncthreads();
  const int s_end = min(slots, (b + 1) * bs);
  for (int s = b * bs + threadIdx.x; s < s_end; s += 256) atomicAdd(&hist[p.experts[s]], 1);
  __syncthreads();
  if (threadIdx.x < p.E) p.counts[3 * p.E + b * p.E + threadIdx.x] = hist[threadIdx.x];
}

// sum over blocks b' in [0, nb) of the block histograms of expert (tid & 63),
// four threads per expert (tid >> 6 picks b' modulo 4), reduced in LDS
__device__ __forceinline__ int sum_block_hist(const int* bh, int E, int nb, int (*part)[64]) {
  const int e = threadIdx.x & 63, q = threadIdx.x >> 6;
  int c = 0;
  if (e < E)
    for (int b = q; b < nb; b += 4) c += bh[b * E + e];
  part[q][e] = c;
  __syncthreads();
  const int r = part[0][e] + part[1][e] + part[2][e] + part[3][e];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(256) void k_moe_plan(MoeDispatchArgs p) {
  __shared__ int part[4][64];
  __shared__ int off[64], cnt[64];
  const int e = threadIdx.x;
  const int slots = p.T * p.top_k;
  const int nb = ceil_div(slots, sort_block_size(slots));
  const int c = sum_block_hist(p.counts + 3 * p.E, p.E, nb, part);
  if (e < 64) cnt[e] = c;
  __syncthreads();
  if (e == 0) {
    int o = 0, tl = 0;
    for (int i = 0; i < p.E; ++i) {
      const int padded = (cnt[i] + p.pad - 1) / p.pad * p.pad;
      off[i] = o;
      o += padded;
      tl += (padded + p.tile_rows - 1) / p.tile_rows;
    }
    p.tiles[3] = min(tl, p.tiles_max);  // tiles in use (tile 0's spare field)
  }
  __syncthreads();
  if (e < p.E) {
    p.counts[e] = cnt[e];
    p.counts[p.E + e] = off[e];
    int tile0 = 0;
    for (int i = 0; i < e; ++i) tile0 += ((cnt[i] + p.pad - 1) / p.pad * p.pad + p.tile_rows - 1) / p.tile_rows;
    const int padded = (cnt[e] + p.pad - 1) / p.pad * p.pad;
    const int nt = (padded + p.tile_rows - 1) / p.tile_rows;
    for (int j = 0; j < nt && tile0 + j < p.tiles_max; ++j) {
      int* td = p.tiles + 4 * (tile0 + j);
      td[0] = e;
      td[1] = off[e] + j * p.tile_rows;
      td[2] = off[e] + cnt[e];
    }
  }
}

__global__ __launch_bounds__(256) void k_moe_scatter(MoeDispatchArgs p) {
  __shared__ int part[4][64];
  __shared__ int hist[4][64];
  const int slots = p.T * p.top_k;
  const int bs = sort_block_size(slots);
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // wave w takes slots [b bs + w bs/4, b bs + (w+1) bs/4)
  const int per_wave = bs / 4;
  const int s_begin = b * bs + wave * per_wave, s_end = min(slots, s_begin + per_wave);
  // this block's first row per expert: segment offset + earlier blocks
  const int before = sum_block_hist(p.counts + 3 * p.E, p.E, b, part);
  hist[wave][lane] = 0;
  __syncthreads();
  for (int s = s_begin + lane; s < s_end; s += 64) atomicAdd(&hist[wave][p.experts[s]], 1);
  __syncthreads();
  if (threadIdx.x < p.E) {
    const int e = threadIdx.x;
    int base = p.counts[p.E + e] + before;
    for (int w = 0; w < 4; ++w) {
      const int h = hist[w][e];
      hist[w][e] = base;
      base += h;
    }
  }
  __syncthreads();
  const uint64_t lower = (uint64_t(1) << lane) - 1;
  for (int s0 = s_begin; s0 < s_end; s0 += 64) {
    const int s = s0 + lane;
    const bool ok = s < s_end;
    const int e = ok ? p.experts[s] : 0;
    const float w = ok ? p.weights[s] : 0.0f;
    const uint64_t same = match_expert(e, __ballot(ok));
    const int pos = hist[wave][e] + __builtin_popcountll(same & lower);
    if (ok && pos >= 0 && pos < p.rows_max) {
      p.row_token[pos] = s / p.top_k;
      p.row_weight[pos] = w;
      p.row_slot[pos] = s;
    }
    // the last lane of each group advances its expert's cursor (the LDS
    // accesses of one wave complete in order)
    if (ok && (same >> lane) == 1) hist[wave][e] += __builtin_popcountll(same);
  }
}

// 8 columns (16 bytes) per thread when H % 8 == 0 and rows are aligned,
// one column per thread otherwise.
template <bool VEC>
__global__ __launch_bounds__(256) void k_moe_combine(const uint16_t* y, int T, int top_k, int H, uint16_t* out,
                                                     int64_t out_sm) {
#pragma clang fp contract(off)
  constexpr int V = VEC ? 8 : 1;
  const int per_row = H / V;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(T) * per_row) return;
  const int t = static_cast<int>(i / per_row), c = static_cast<int>(i % per_row) * V;
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  for (int k = 0; k < top_k; ++k) {
    const uint16_t* row = y + (static_cast<int64_t>(t) * top_k + k) * H + c;
    if constexpr (VEC) {
      const i32x4 w = *reinterpret_cast<const i32x4*>(row);
#pragma unroll
      for (int v = 0; v < 8; ++v)
        acc[v] = acc[v] + bf16_to_f32(static_cast<uint16_t>(static_cast<uint32_t>(w[v >> 1]) >> (16 * (v & 1))));
    } else {
      acc[0] = acc[0] + bf16_to_f32(row[0]);
    }
  }
  uint16_t* o = out + static_cast<int64_t>(t) * out_sm + c;
  if constexpr (VEC) {
    i32x4 w;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      w[v] = static_cast<int>(static_cast<uint32_t>(f32_to_bf16(acc[2 * v])) |
                              (static_cast<uint32_t>(f32_to_bf16(acc[2 * v + 1])) << 16));
    *reinterpret_cast<i32x4*>(o) = w;
  } else {
    o[0] = f32_to_bf16(acc[0]);
  }
}

}  // namespace

hipError_t launch_moe_dispatch(const MoeDispatchArgs& p, hipStream_t stream) {
  if (p.E > 64) return hipErrorInvalidValue;
  const int64_t init_items = p.rows_max > p.tiles_max ? p.rows_max : p.tiles_max;
  int64_t blocks = ceil_div<int64_t>(init_items, 256);
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(k_moe_init, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
  if (p.T == 0) return hipGetLastError();
  hipLaunchKernelGGL(k_moe_route, dim3(static_cast<unsigned>(ceil_div(p.T, 4))), dim3(256), 0, stream, p);
  const int slots = p.T * p.top_k;
  const int nb = ceil_div(slots, sort_block_size(slots));  // <= kMaxSortBlocks
  hipLaunchKernelGGL(k_moe_count, dim3(static_cast<unsigned>(nb)), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(k_moe_plan, dim3(1), dim3(256), 0, stream, p);  // 4 threads per expert
  hipLaunchKernelGGL(k_moe_scatter, dim3(static_cast<unsigned>(nb)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_moe_combine(const uint16_t* y, int T, int top_k, int H, uint16_t* out, int64_t out_sm,
                              hipStream_t stream) {
  if (T == 0 || H == 0) return hipSuccess;
  const bool vec = H % 8 == 0 && out_sm % 8 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  const int64_t items = static_cast<int64_t>(T) * (vec ? H / 8 : H);
  const dim3 grid(static_cast<unsigned>(ceil_div<int64_t>(items, 256)));
  if (vec) hipLaunchKernelGGL(k_moe_combine<true>, grid, dim3(256), 0, stream, y, T, top_k, H, out, out_sm);
  else hipLaunchKernelGGL(k_moe_combine<false>, grid, dim3(256), 0, stream, y, T, top_k, H, out, out_sm);
  return hipGetLastError();
}

}  // namespace qg
