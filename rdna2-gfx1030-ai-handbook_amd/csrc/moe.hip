// MoE prefill routing, dispatch and combine on gfx950 (benchmark configuration
// 4; the reference repository has no MoE kernel). The grouped INT8 GEMM that
// runs between dispatch and combine is k_i8_moe_pp in int8_gemm.hip.
//
// The dispatch is a stable counting sort of the tokens * top_k routed slots
// by expert, in two launches over sort blocks of tb consecutive tokens
// (tb * top_k slots, at most kMaxSortBlocks blocks):
//   route    one wave per token, lane e = expert e: softmax over the experts
//            in fp32 and the top_k experts by logit (ties: lower index); the
//            block counts its slots per expert (LDS atomics) into its
//            histogram
//   scatter  every block derives the plan from all histograms: expert
//            counts, segments padded to `pad` rows (wave-wide scans, lane =
//            expert), its own first row per expert; block 0 writes the table
//            of tile_rows-row tiles of the grouped GEMM (tile 0's spare field
//            holds the number of tiles in use, unused tiles are empty); the
//            padding rows and the rows past the last segment are marked empty
//            (no memset node: safe under graph capture). Then every slot's
//            row = its block's first row + earlier waves of the block + its
//            rank among equal experts of its 64-slot step (six ballots). Rows
//            inside a segment are in slot order: the dispatch is deterministic
//   combine  out[t] = bf16(sum over k of y[t * top_k + k]) in k order (fp32)
#include "qg_common.h"
#include "qg_internal.h"
#include "qg_quant.h"

namespace qg {

namespace {

constexpr int kMaxSortBlocks = 256;
constexpr int kRouteWaves = 16;  // waves (tokens in flight) per routing block

// Tokens per sort block: blocks of tb tokens, at most kMaxSortBlocks of them.
__host__ __device__ __forceinline__ int sort_block_tokens(int T) {
  const int tb = ceil_div(T, kMaxSortBlocks);
  return tb > 0 ? tb : 1;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, kWave);
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, kWave);
    if (lane >= o) v += u;
  }
  return v;
}

// counts layout: [0, E) counts, [E, 2E) segment offsets, [2E, 3E) first tile
// of each expert, then [kMaxSortBlocks][E] per-block histograms (the
// workspace holds (3 + 256) E ints).
// QX: the wave also quantizes token t's row of x (the per-token activation
// quantization of the gate/up GEMM, bit-identical to k_quant_rows_reg): its
// loads are issued before the routing, which they overlap, and the codes are
// formed and stored after it.
template <bool QX>
__global__ __launch_bounds__(kRouteWaves * 64) void k_moe_route(MoeDispatchArgs p) {
#pragma clang fp contract(off)
  constexpr int kQxChunks = kMoeRouteQuantMaxH / 8 / 64;  // 16-byte chunks per lane
  __shared__ int hist[64];
  const int tb = sort_block_tokens(p.T);
  const int b = blockIdx.x;
  if (threadIdx.x < 64) hist[threadIdx.x] = 0;
  __syncthreads();
  const int e = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool live = e < p.E;
  const int t_end = min(p.T, (b + 1) * tb);
  for (int t = b * tb + wave; t < t_end; t += kRouteWaves) {
    // the logit of a clamped lane, replaced below: an unconditional load, so
    // the row's loads issued after it stay in flight while the routing waits
    // for the logit only (loads complete in order)
    const float l_raw = p.logits[static_cast<int64_t>(t) * p.l_sm + min(e, p.E - 1)];
    i32x4 xr[kQxChunks];
    if constexpr (QX) {
      asm volatile("" ::: "memory");
      // unconditional loads of clamped chunks (a conditional load would make
      // the compiler wait for every load at the join); chunks past the row are
      // zeroed where they are used
      const i32x4* row = reinterpret_cast<const i32x4*>(p.x + static_cast<int64_t>(t) * p.x_sm);
      const int last = (p.H >> 3) - 1;
#pragma unroll
      for (int i = 0; i < kQxChunks; ++i) xr[i] = row[min(e + 64 * i, last)];
    }
    const float l = live ? l_raw : -__builtin_inff();
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
        atomicAdd(&hist[e], 1);
      }
    }
    if constexpr (QX) {
      const int chunks = p.H >> 3;
#pragma unroll
      for (int i = 0; i < kQxChunks; ++i)
        if (e + 64 * i >= chunks) xr[i] = i32x4{0, 0, 0, 0};
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < kQxChunks; ++i) {
        float v[8];
        decode_chunk<QG_BF16>(xr[i], v);
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
      }
      amax = wave_max(amax);
      const float step = fmaxf(amax / 127.0f, 1.0e-20f);
      const float rstep = __builtin_amdgcn_rcpf(step);
      int8_t* qr = p.xq + static_cast<int64_t>(t) * p.xq_sm;
#pragma unroll
      for (int i = 0; i < kQxChunks; ++i) {
        const int c = e + 64 * i;
        quant_chunk_store<QG_BF16, QG_ROUND_HALF_EVEN>(xr[i], step, rstep, qr, c, c < chunks);
      }
      if (e == 0) p.xs[t] = step;
    }
  }
  __syncthreads();
  if (threadIdx.x < p.E) p.counts[3 * p.E + b * p.E + threadIdx.x] = hist[threadIdx.x];
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

// Every workgroup (256 threads, one per sort block) first derives the whole
// plan from the sort blocks' histograms [nb][E]: thread (q = tid >> 6,
// e = tid & 63) sums expert e's entries of blocks q, q + 4, ... (all, and
// those before this block); wave 0 then turns the expert counts into padded
// segments and tiles with wave-wide scans (lane = expert). Block 0 writes the
// counts, offsets and the tile table; the padding rows of expert e are
// marked empty by block e mod nb, the rows past the last segment by all
// blocks in turn. Then the block scatters its slots.
__global__ __launch_bounds__(256) void k_moe_scatter(MoeDispatchArgs p) {
  __shared__ int hist[4][64];
  __shared__ int part[4][64], prior[4][64];
  __shared__ int seg[64], cnt_s[64], pad_s[64], tile0_s[64], ntile_s[64];
  __shared__ int totals[2];  // rows and tiles of all segments
  const int slots = p.T * p.top_k;
  const int tb = sort_block_tokens(p.T);
  const int nb = ceil_div(p.T, tb);  // 0 without tokens (one workgroup runs)
  const int nbl = nb > 0 ? nb : 1;
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int* bh = p.counts + 3 * p.E;
  // wave w takes slots [b bs + w pw, b bs + (w+1) pw) of the block; the first
  // 64-slot step's experts and weights are fetched before the plan
  const int bs = tb * p.top_k;
  const int pw = ceil_div(bs, 4);
  const int blk_end = min(slots, (b + 1) * bs);
  const int s_begin = min(blk_end, b * bs + wave * pw), s_end = min(blk_end, s_begin + pw);
  const bool ok0 = s_begin + lane < s_end;
  const int e0 = ok0 ? p.experts[s_begin + lane] : 0;
  const float w0 = ok0 ? p.weights[s_begin + lane] : 0.0f;

  // ---- plan ------------------------------------------------------------------
  {
    const int e = lane, q = wave;
    int tot = 0, bef = 0;
    if (e < p.E) {
      // kBatch independent loads in flight per round (a dependent sum would
      // wait one memory latency per block)
      constexpr int kBatch = 32;
      for (int bb0 = q; bb0 < nb; bb0 += 4 * kBatch) {
        int v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int bb = bb0 + 4 * u;
          v[u] = bb < nb ? bh[bb * p.E + e] : 0;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          tot += v[u];
          if (bb0 + 4 * u < b) bef += v[u];
        }
      }
    }
    part[q][e] = tot;
    prior[q][e] = bef;
  }
  __syncthreads();
  if (wave == 0) {
    const int e = lane;
    const int cnt = e < p.E ? part[0][e] + part[1][e] + part[2][e] + part[3][e] : 0;
    const int padded = (cnt + p.pad - 1) / p.pad * p.pad;
    const int nt = (padded + p.tile_rows - 1) / p.tile_rows;
    const int off_inc = wave_inclusive_scan(padded), t_inc = wave_inclusive_scan(nt);
    seg[e] = off_inc - padded;
    cnt_s[e] = cnt;
    pad_s[e] = padded;
    tile0_s[e] = t_inc - nt;
    ntile_s[e] = nt;
    if (e == 63) {
      totals[0] = off_inc;
      totals[1] = t_inc;
    }
    if (b == 0 && e < p.E) {
      p.counts[e] = cnt;
      p.counts[p.E + e] = off_inc - padded;
      p.counts[2 * p.E + e] = t_inc - nt;
    }
  }
  __syncthreads();
  const int rows_used = totals[0];
  const int tiles_used = min(totals[1], p.tiles_max);
  if (b == 0) {
    // thread (q, e) writes tiles q, q + 4, ... of expert e; then the unused ones
    const int e = lane;
    if (e < p.E) {
      for (int j = wave; j < ntile_s[e]; j += 4) {
        const int ti = tile0_s[e] + j;
        if (ti < p.tiles_max) {
          int* td = p.tiles + 4 * ti;
          td[0] = e;
          td[1] = seg[e] + j * p.tile_rows;
          td[2] = seg[e] + cnt_s[e];
          td[3] = ti == 0 ? tiles_used : 0;
        }
      }
    }
    for (int ti = tiles_used + threadIdx.x; ti < p.tiles_max; ti += 256) {
      int* td = p.tiles + 4 * ti;
      td[0] = -1;
      td[1] = 0;
      td[2] = 0;
      td[3] = ti == 0 ? tiles_used : 0;
    }
  }
  {
    const int e = lane;
    if (e < p.E && e % nbl == b) {
      for (int r = seg[e] + cnt_s[e] + wave; r < seg[e] + pad_s[e]; r += 4) {
        if (r < p.rows_max) {
          p.row_token[r] = -1;
          p.row_slot[r] = -1;
          p.row_weight[r] = 0.0f;
        }
      }
    }
  }
  for (int r = rows_used + b * 256 + threadIdx.x; r < p.rows_max; r += nbl * 256) {
    p.row_token[r] = -1;
    p.row_slot[r] = -1;
    p.row_weight[r] = 0.0f;
  }

  // ---- scatter ----------------------------------------------------------------
  hist[wave][lane] = 0;
  __syncthreads();
  if (ok0) atomicAdd(&hist[wave][e0], 1);
  for (int s = s_begin + 64 + lane; s < s_end; s += 64) atomicAdd(&hist[wave][p.experts[s]], 1);
  __syncthreads();
  if (threadIdx.x < p.E) {
    const int e = threadIdx.x;
    // the block's first row for expert e, then the earlier waves' slots
    int base = seg[e] + prior[0][e] + prior[1][e] + prior[2][e] + prior[3][e];
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
    const int e = s0 == s_begin ? e0 : (ok ? p.experts[s] : 0);
    const float w = s0 == s_begin ? w0 : (ok ? p.weights[s] : 0.0f);
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
  const int nb = p.T > 0 ? ceil_div(p.T, sort_block_tokens(p.T)) : 0;  // <= kMaxSortBlocks
  if (p.x != nullptr && (p.H % 8 != 0 || p.H > kMoeRouteQuantMaxH)) return hipErrorInvalidValue;
  if (nb > 0) {
    if (p.x != nullptr)
      hipLaunchKernelGGL(k_moe_route<true>, dim3(static_cast<unsigned>(nb)), dim3(kRouteWaves * 64), 0, stream, p);
    else
      hipLaunchKernelGGL(k_moe_route<false>, dim3(static_cast<unsigned>(nb)), dim3(kRouteWaves * 64), 0, stream, p);
  }
  // one workgroup when there are no tokens: it still writes the empty plan
  hipLaunchKernelGGL(k_moe_scatter, dim3(static_cast<unsigned>(nb > 0 ? nb : 1)), dim3(256), 0, stream, p);
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
