// op1 routing on gfx950: router logits + softmax, then op3 budget routing and
// stable (expert, DFS-order) bucketing.
//
// Every floating-point operation here is written out in a fixed order with
// contraction disabled, so that the CPU restatement reproduces the outputs bit
// for bit: expert ids, gate weights, demand and every layout index.
#pragma clang fp contract(off)

#include "tm_common.h"

namespace {

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kMaxSlots = 2 * TM_MAX_TOKENS;
constexpr int kMaxChunks = kMaxSlots / 64;
constexpr int kMaxPaddedRows = 16384;

__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// One wave per token.  Lane l accumulates the 8-element chunks l, l+64, ... of
// the dot product in element order (fmaf of exact bf16 products), the 64 lane
// sums are combined by a halving tree (xor butterfly), and the sum is rounded
// to bf16 like the output of F.linear on bf16 operands
// (treemoe/kernels/op1_tree_moe.py:676).  Softmax (:677) then runs in fp32:
// max, e^(l - max), a sum in expert order, and a correctly rounded division.
__global__ void __launch_bounds__(256)
tm_router_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg,
                 float* __restrict__ gates, int T, int H, int E) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  const int nchunk = H >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)t * H);
  float my_logit = 0.0f;
  for (int e = 0; e < E; ++e) {
    const uint4* wr = reinterpret_cast<const uint4*>(wg + (size_t)e * H);
    float acc = 0.0f;
    for (int c = lane; c < nchunk; c += 64) {
      const uint4 xv = xr[c];
      const uint4 wv = wr[c];
      acc = fmaf(lo_bf16(xv.x), lo_bf16(wv.x), acc);
      acc = fmaf(hi_bf16(xv.x), hi_bf16(wv.x), acc);
      acc = fmaf(lo_bf16(xv.y), lo_bf16(wv.y), acc);
      acc = fmaf(hi_bf16(xv.y), hi_bf16(wv.y), acc);
      acc = fmaf(lo_bf16(xv.z), lo_bf16(wv.z), acc);
      acc = fmaf(hi_bf16(xv.z), hi_bf16(wv.z), acc);
      acc = fmaf(lo_bf16(xv.w), lo_bf16(wv.w), acc);
      acc = fmaf(hi_bf16(xv.w), hi_bf16(wv.w), acc);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = acc + __shfl_xor(acc, off);
    const float logit = tm_bf16_to_f32(tm_f32_to_bf16(acc));
    if (lane == e) my_logit = logit;
  }
  float m = (lane < E) ? my_logit : -INFINITY;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  const float ex = (lane < E) ? tm_expf_det(my_logit - m) : 0.0f;
  float s = 0.0f;
  for (int e = 0; e < E; ++e) s = s + __shfl(ex, e);
  if (lane < E) gates[(size_t)t * E + lane] = ex / s;
}

// Budget routing and bucketing for all T tokens in one workgroup of 16 waves.
//
//  1. demand[e] = sum_t accept[t] * gates[t, e]: lane l of the wave that owns
//     expert e sums tokens l, l+64, ... in order, then a halving tree
//     (treemoe/ref/tree_moe_ref.py:34).
//  2. keep = the `budget` experts first in the order (demand desc, e asc); for
//     the critical-path objective the order is (crit desc, demand desc, e asc)
//     with crit[e] = max accept over nodes whose unrestricted top-1, or top-2
//     when accept >= tau, is e (tree_moe_ref.py:35-49, op1_tree_moe.py:195-217).
//  3. per token: top-2 of the kept gates (ties to the lower expert id, the
//     second pick excludes the first), weights p_k / (p1 + p2), and (1, 0) when
//     accept < tau (tree_moe_ref.py:51-66).
//  4. slot s = 2t + k; stable rank inside its expert from wave ballots; the
//     reference's padded BM-row block layout (op1_tree_moe.py:111-144) and the
//     compact expert-major order with its GEMM tile list.
__global__ void __launch_bounds__(kRouteThreads)
tm_route_bucket_kernel(const float* __restrict__ gates, const float* __restrict__ accept,
                       int T, int E, int budget, float tau, int objective, int BM,
                       int max_blocks, int max_tiles, int64_t* __restrict__ topk_ids,
                       float* __restrict__ gates_flat, int64_t* __restrict__ padded_slots,
                       int64_t* __restrict__ block_expert_ids, int64_t* __restrict__ slot_to_row,
                       float* __restrict__ demand_out, int32_t* __restrict__ expert_offsets,
                       int32_t* __restrict__ sorted_slots, int32_t* __restrict__ slot_pos,
                       int32_t* __restrict__ tiles) {
  __shared__ float s_demand[TM_MAX_EXPERTS];
  __shared__ float s_crit[TM_MAX_EXPERTS];
  __shared__ int s_keep[TM_MAX_EXPERTS];
  __shared__ int s_count[TM_MAX_EXPERTS];
  __shared__ int s_block_start[TM_MAX_EXPERTS];
  __shared__ int s_nblocks[TM_MAX_EXPERTS];
  __shared__ int s_offset[TM_MAX_EXPERTS + 1];
  __shared__ uint8_t s_fe[kMaxSlots];
  __shared__ uint16_t s_cnt[kMaxChunks * TM_MAX_EXPERTS];
  __shared__ int16_t s_padded[kMaxPaddedRows];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int nslot = 2 * T;
  const int nchunk = (nslot + 63) >> 6;
  const int padded_rows = max_blocks * BM;

  // critical path needs every node's unrestricted top-2 (first occurrence).
  if (objective == TM_OBJECTIVE_CRITICAL_PATH) {
    for (int t = tid; t < T; t += kRouteThreads) {
      const float* g = gates + (size_t)t * E;
      int u1 = 0;
      float b1 = g[0];
      for (int e = 1; e < E; ++e) {
        const float v = g[e];
        if (v > b1) { b1 = v; u1 = e; }
      }
      int u2 = -1;
      float b2 = 0.0f;
      for (int e = 0; e < E; ++e) {
        if (e == u1) continue;
        const float v = g[e];
        if (u2 < 0 || v > b2) { b2 = v; u2 = e; }
      }
      s_fe[2 * t] = (uint8_t)u1;
      s_fe[2 * t + 1] = (uint8_t)u2;
    }
    __syncthreads();
  }

  // 1. demand (and criticality)
  for (int e = wave; e < E; e += kRouteWaves) {
    float acc = 0.0f;
    float crit = -INFINITY;
    for (int t = lane; t < T; t += 64) {
      const float a = accept[t];
      const float p = a * gates[(size_t)t * E + e];
      acc = acc + p;
      if (objective == TM_OBJECTIVE_CRITICAL_PATH) {
        const bool needed = (s_fe[2 * t] == e) || ((s_fe[2 * t + 1] == e) && (a >= tau));
        if (needed) crit = fmaxf(crit, a);
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      acc = acc + __shfl_xor(acc, off);
      crit = fmaxf(crit, __shfl_xor(crit, off));
    }
    if (lane == 0) {
      s_demand[e] = acc;
      s_crit[e] = crit;
      demand_out[e] = acc;
    }
  }
  __syncthreads();

  // 2. keep set: selection in lexicographic order, first occurrence on ties.
  if (tid == 0) {
    for (int e = 0; e < E; ++e) s_keep[e] = 0;
    for (int rank = 0; rank < budget; ++rank) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        if (s_keep[e]) continue;
        if (best < 0) { best = e; continue; }
        bool better;
        if (objective == TM_OBJECTIVE_CRITICAL_PATH) {
          better = (s_crit[e] > s_crit[best]) ||
                   (s_crit[e] == s_crit[best] && s_demand[e] > s_demand[best]);
        } else {
          better = s_demand[e] > s_demand[best];
        }
        if (better) best = e;
      }
      s_keep[best] = 1;
    }
  }
  __syncthreads();

  // 3. in-budget top-2, renormalisation, low-acceptance degrade
  for (int t = tid; t < T; t += kRouteThreads) {
    const float* g = gates + (size_t)t * E;
    int i1 = -1;
    float g1 = 0.0f;
    for (int e = 0; e < E; ++e) {
      const float v = s_keep[e] ? g[e] : 0.0f;
      if (i1 < 0 || v > g1) { g1 = v; i1 = e; }
    }
    int i2 = -1;
    float g2 = 0.0f;
    for (int e = 0; e < E; ++e) {
      if (e == i1) continue;
      const float v = s_keep[e] ? g[e] : 0.0f;
      if (i2 < 0 || v > g2) { g2 = v; i2 = e; }
    }
    const float s = g1 + g2;
    float tg1 = g1 / s;
    float tg2 = g2 / s;
    if (accept[t] < tau) { tg1 = 1.0f; tg2 = 0.0f; }
    topk_ids[2 * t] = i1;
    topk_ids[2 * t + 1] = i2;
    gates_flat[2 * t] = tg1;
    gates_flat[2 * t + 1] = tg2;
  }
  // s_fe may still be read by step 1 of slower waves: fence before rewriting it.
  __syncthreads();
  for (int t = tid; t < T; t += kRouteThreads) {
    s_fe[2 * t] = (uint8_t)topk_ids[2 * t];
    s_fe[2 * t + 1] = (uint8_t)topk_ids[2 * t + 1];
  }
  for (int i = tid; i < padded_rows; i += kRouteThreads) s_padded[i] = -1;
  __syncthreads();

  // 4a. per-chunk expert counts from ballots
  for (int q = wave; q < nchunk; q += kRouteWaves) {
    const int s = q * 64 + lane;
    const int fe = (s < nslot) ? (int)s_fe[s] : -1;
    for (int e = 0; e < E; ++e) {
      const unsigned long long m = __ballot(fe == e);
      if (lane == 0) s_cnt[q * TM_MAX_EXPERTS + e] = (uint16_t)__popcll(m);
    }
  }
  __syncthreads();
  // 4b. exclusive scan over chunks (slot order) for every expert
  if (tid < E) {
    int run = 0;
    for (int q = 0; q < nchunk; ++q) {
      const int c = s_cnt[q * TM_MAX_EXPERTS + tid];
      s_cnt[q * TM_MAX_EXPERTS + tid] = (uint16_t)run;
      run += c;
    }
    s_count[tid] = run;
  }
  __syncthreads();
  // 4c. block layout (reference), compact offsets and GEMM tiles
  if (tid == 0) {
    int blocks = 0;
    int off = 0;
    int j = 0;
    for (int e = 0; e < E; ++e) {
      const int c = s_count[e];
      const int nb = (c + BM - 1) / BM;
      s_block_start[e] = blocks;
      s_nblocks[e] = nb;
      blocks += nb;
      s_offset[e] = off;
      for (int r = 0; r < c; r += TM_GEMM_TILE_M) {
        if (j < max_tiles) {
          tiles[4 * j + 0] = e;
          tiles[4 * j + 1] = off + r;
          tiles[4 * j + 2] = min(TM_GEMM_TILE_M, c - r);
          tiles[4 * j + 3] = 0;
        }
        ++j;
      }
      off += c;
    }
    s_offset[E] = off;
    for (; j < max_tiles; ++j) {
      tiles[4 * j + 0] = -1;
      tiles[4 * j + 1] = 0;
      tiles[4 * j + 2] = 0;
      tiles[4 * j + 3] = 0;
    }
  }
  __syncthreads();
  if (tid <= E) expert_offsets[tid] = s_offset[tid];
  // 4d. stable in-expert rank -> destinations
  for (int q = wave; q < nchunk; q += kRouteWaves) {
    const int s = q * 64 + lane;
    const int fe = (s < nslot) ? (int)s_fe[s] : -1;
    int inrank = 0;
    for (int e = 0; e < E; ++e) {
      const unsigned long long m = __ballot(fe == e);
      if (fe == e) inrank = __popcll(m & ((1ull << lane) - 1ull));
    }
    if (s < nslot) {
      const int rank = (int)s_cnt[q * TM_MAX_EXPERTS + fe] + inrank;
      const int dest = s_block_start[fe] * BM + rank;
      const int pos = s_offset[fe] + rank;
      slot_to_row[s] = dest;
      if (dest < padded_rows) s_padded[dest] = (int16_t)s;
      sorted_slots[pos] = s;
      slot_pos[s] = pos;
    }
  }
  __syncthreads();
  for (int i = tid; i < padded_rows; i += kRouteThreads) padded_slots[i] = s_padded[i];
  for (int b = tid; b < max_blocks; b += kRouteThreads) {
    int owner = -1;
    for (int e = 0; e < E; ++e) {
      if (s_nblocks[e] > 0 && b >= s_block_start[e] && b < s_block_start[e] + s_nblocks[e]) owner = e;
    }
    block_expert_ids[b] = owner;
  }
}

}  // namespace

extern "C" int tm_op1_router_gates(const void* x, const void* wg, int64_t T, int64_t H,
                                   int64_t E, float* gates, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS || H < 8 || (H % 8) != 0)
    return TM_ERR_SHAPE;
  if (((uintptr_t)x % 16) != 0 || ((uintptr_t)wg % 16) != 0) return TM_ERR_ALIGN;
  const dim3 grid((unsigned)((T + 3) / 4));
  hipLaunchKernelGGL(tm_router_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)wg, gates, (int)T, (int)H, (int)E);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op1_route_bucket(const float* gates, const float* accept, int64_t T,
                                   int64_t E, int64_t budget, float tau, int objective,
                                   int64_t block_m, int64_t max_blocks, int64_t max_tiles,
                                   int64_t* topk_ids, float* gates_flat,
                                   int64_t* padded_slots, int64_t* block_expert_ids,
                                   int64_t* slot_to_row, float* demand,
                                   int32_t* expert_offsets, int32_t* sorted_slots,
                                   int32_t* slot_pos, int32_t* tiles, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS) return TM_ERR_SHAPE;
  if (budget < 2 || budget > E) return TM_ERR_ARG;
  if (objective != TM_OBJECTIVE_MASS && objective != TM_OBJECTIVE_CRITICAL_PATH) return TM_ERR_ARG;
  if (block_m != 16 && block_m != 32) return TM_ERR_ARG;
  if (max_blocks < 1 || max_blocks * block_m > kMaxPaddedRows || max_tiles < 1) return TM_ERR_SHAPE;
  hipLaunchKernelGGL(tm_route_bucket_kernel, dim3(1), dim3(kRouteThreads), 0,
                     (hipStream_t)stream, gates, accept, (int)T, (int)E, (int)budget, tau,
                     objective, (int)block_m, (int)max_blocks, (int)max_tiles, topk_ids,
                     gates_flat, padded_slots, block_expert_ids, slot_to_row, demand,
                     expert_offsets, sorted_slots, slot_pos, tiles);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}
