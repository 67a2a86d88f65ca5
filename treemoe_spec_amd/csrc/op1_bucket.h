// op3 budget routing and stable (expert, DFS-order) bucketing of one op1
// layer inside one workgroup, shared by the routing kernel (op1_route.hip) and
// the gate/up GEMM that routes its own jobs (op1_prefill.hip).
//
// Every floating-point operation is written out in a fixed order with
// contraction disabled, so that the CPU restatement reproduces the outputs bit
// for bit: expert ids, gate weights, demand and every layout index.  The
// phases below do not depend on the workgroup size NT (only the integer work
// is spread differently), so every instantiation computes the same bits.
#pragma once

#include "tm_common.h"

namespace tmb {

struct BucketArgs {
  const float* gates;
  const float* accept;
  int T, E, budget, objective, BM, max_blocks, max_tiles;
  float tau;
  int64_t* topk_ids;
  float* gates_flat;
  int64_t* padded_slots;
  int64_t* block_expert_ids;
  int64_t* slot_to_row;
  float* demand_out;
  int32_t* expert_offsets;
  int32_t* sorted_slots;
  int32_t* slot_pos;
  int32_t* tiles;
};

// LDS of the phases for up to MAXT tokens: the gates are staged when T * E <=
// STAGEF, and MAXBLK bounds the reference's padded blocks.
template <int MAXT, int STAGEF, int MAXBLK>
struct BucketSharedT {
  static constexpr int kMaxTokens = MAXT;
  static constexpr int kStageFloats = STAGEF;
  static constexpr int kMaxSlots = 2 * MAXT;
  static constexpr int kMaxChunks = kMaxSlots / 64;
  static constexpr int kMaxBlocks = MAXBLK;
  float gates[STAGEF];
  float accept[MAXT];
  float demand[TM_MAX_EXPERTS];
  float crit[TM_MAX_EXPERTS];
  int count[TM_MAX_EXPERTS];
  int block_start[TM_MAX_EXPERTS];
  int nblocks[TM_MAX_EXPERTS];
  int offset[TM_MAX_EXPERTS + 1];
  uint8_t fe[kMaxSlots];                 // expert of slot s
  uint8_t inrank[kMaxSlots];             // rank of slot s among its expert's slots in its chunk
  uint16_t sorted[kMaxSlots];            // compact expert-major order
  int16_t owner[MAXBLK];                 // expert of padded block b, -1 unused
  uint16_t cnt[kMaxChunks * TM_MAX_EXPERTS];
};

// Wave-wide exclusive prefix sum (lane order).
__device__ __forceinline__ int wave_exclusive_scan(int v, int lane, int* total) {
  int inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(inc, off);
    if (lane >= off) inc += u;
  }
  *total = __shfl(inc, 63);
  return inc - v;
}

// Top-2 in one pass over e = 0, 1, ...: the first pick is the first maximum;
// the second is the first maximum of the others (a later equal value never
// displaces an earlier one).
struct Top2 {
  int i1, i2;
  float g1, g2;
  __device__ __forceinline__ void offer(float v, int e) {
    if (i1 < 0 || v > g1) {
      g2 = g1;
      i2 = i1;
      g1 = v;
      i1 = e;
    } else if (i2 < 0 || v > g2) {
      g2 = v;
      i2 = e;
    }
  }
};

// Budget routing and bucketing for all T tokens in one workgroup of NT
// threads.
//
//  1. demand[e] = sum_t accept[t] * gates[t, e]: lane l of the wave that owns
//     expert e sums tokens l, l+64, ... in order, then a halving tree
//     (treemoe/ref/tree_moe_ref.py:34).
//  2. keep = the `budget` experts first in the order (demand desc, e asc); for
//     the critical-path objective the order is (crit desc, demand desc, e asc)
//     with crit[e] = max accept over nodes whose unrestricted top-1, or top-2
//     when accept >= tau, is e (tree_moe_ref.py:35-49, op1_tree_moe.py:195-217).
//     Expert e is kept when fewer than `budget` experts precede it in that
//     (strict, total) order.
//  3. per token: top-2 of the kept gates (ties to the lower expert id, the
//     second pick excludes the first), weights p_k / (p1 + p2), and (1, 0) when
//     accept < tau (tree_moe_ref.py:51-66).
//  4. slot s = 2t + k; stable rank inside its expert from wave ballots and a
//     scan over 64-slot chunks; the compact expert-major order with its GEMM
//     tile list, and the reference's padded BM-row block layout
//     (op1_tree_moe.py:111-144) read back from the compact order.
// Gates and accept are staged in LDS first and every intermediate stays in
// LDS; global memory is written only with final values, each by one thread,
// and never read back here.  So the phases are separated by LDS-only barriers:
// __syncthreads() would also wait for the phase's global stores to complete
// (its workgroup release fence), measured at 0.5-1 us per phase.
//
// WRITE = false computes the per-expert counts (sh.count), the compact
// offsets (sh.offset) and the compact order (sh.sorted) in LDS only, for a
// GEMM workgroup that needs its own rows; WRITE = true also writes every
// routing output to global memory.
template <int NT, class SH, bool WRITE>
__device__ void bucket_phases(const BucketArgs& a, SH& sh) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int T = a.T, E = a.E;
  const int nslot = 2 * T;
  const int nchunk = (nslot + 63) >> 6;
  const int padded_rows = a.max_blocks * a.BM;
  const bool critical = a.objective == TM_OBJECTIVE_CRITICAL_PATH;
  const bool staged = T * E <= SH::kStageFloats;

  // 0. stage gates and accept
  if (staged) {
    const int n = T * E;
    int done = 0;
    if ((reinterpret_cast<uintptr_t>(a.gates) & 15) == 0) {
      const int n4 = n >> 2;
      const float4* g4 = reinterpret_cast<const float4*>(a.gates);
      float4* s4 = reinterpret_cast<float4*>(sh.gates);
#pragma unroll 8
      for (int i = tid; i < n4; i += NT) s4[i] = g4[i];
      done = n4 << 2;
    }
    for (int i = done + tid; i < n; i += NT) sh.gates[i] = a.gates[i];
  }
#pragma unroll 8
  for (int t = tid; t < T; t += NT) sh.accept[t] = a.accept[t];
  if constexpr (WRITE)
    for (int b = tid; b < a.max_blocks; b += NT) sh.owner[b] = -1;
  tm_lds_barrier();
  const float* G = staged ? sh.gates : a.gates;

  if (critical) {
    for (int t = tid; t < T; t += NT) {
      const float* g = G + (size_t)t * E;
      Top2 r{-1, -1, 0.0f, 0.0f};
      for (int e = 0; e < E; ++e) r.offer(g[e], e);
      sh.fe[2 * t] = (uint8_t)r.i1;
      sh.fe[2 * t + 1] = (uint8_t)r.i2;
    }
    tm_lds_barrier();
  }

  // 1. demand (and criticality)
  for (int e = wave; e < E; e += NW) {
    float acc = 0.0f;
    float crit = -INFINITY;
    for (int t = lane; t < T; t += 64) {
      const float av = sh.accept[t];
      const float p = av * G[(size_t)t * E + e];
      acc = acc + p;
      if (critical) {
        const bool needed = (sh.fe[2 * t] == e) || ((sh.fe[2 * t + 1] == e) && (av >= a.tau));
        if (needed) crit = fmaxf(crit, av);
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      acc = acc + __shfl_xor(acc, off);
      crit = fmaxf(crit, __shfl_xor(crit, off));
    }
    if (lane == 0) {
      sh.demand[e] = acc;
      sh.crit[e] = crit;
      if constexpr (WRITE) a.demand_out[e] = acc;
    }
  }
  tm_lds_barrier();

  // 2. keep set, computed by every wave (no barrier before step 3): lane =
  //    expert, rank in the order (crit desc,) demand desc, expert asc, the
  //    other experts' values read from their lanes (readlane, uniform index).
  unsigned long long keep;
  {
    const float d = lane < E ? sh.demand[lane] : 0.0f;
    const float c = (critical && lane < E) ? sh.crit[lane] : 0.0f;
    int rank = 0;
    for (int f = 0; f < E; ++f) {
      const float df = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(d), f));
      const float cf = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), f));
      bool before;
      if (critical && cf != c) {
        before = cf > c;
      } else if (df != d) {
        before = df > d;
      } else {
        before = f < lane;
      }
      rank += before ? 1 : 0;
    }
    keep = __ballot(lane < E && rank < a.budget);
  }

  // 3. in-budget top-2, renormalisation, low-acceptance degrade; the gate row
  //    is read 4 experts at a time when its rows are 16-byte aligned
  const bool vec_rows = (E & 3) == 0 && (reinterpret_cast<uintptr_t>(G) & 15) == 0;
  for (int t = tid; t < T; t += NT) {
    const float* g = G + (size_t)t * E;
    Top2 r{-1, -1, 0.0f, 0.0f};
    if (vec_rows) {
#pragma unroll 4
      for (int e = 0; e < E; e += 4) {
        const float4 v = *reinterpret_cast<const float4*>(g + e);
        r.offer(((keep >> e) & 1ull) ? v.x : 0.0f, e);
        r.offer(((keep >> (e + 1)) & 1ull) ? v.y : 0.0f, e + 1);
        r.offer(((keep >> (e + 2)) & 1ull) ? v.z : 0.0f, e + 2);
        r.offer(((keep >> (e + 3)) & 1ull) ? v.w : 0.0f, e + 3);
      }
    } else {
      for (int e = 0; e < E; ++e) r.offer(((keep >> e) & 1ull) ? g[e] : 0.0f, e);
    }
    if constexpr (WRITE) {
      const float s = r.g1 + r.g2;
      float tg1 = r.g1 / s;
      float tg2 = r.g2 / s;
      if (sh.accept[t] < a.tau) { tg1 = 1.0f; tg2 = 0.0f; }
      a.topk_ids[2 * t] = r.i1;
      a.topk_ids[2 * t + 1] = r.i2;
      a.gates_flat[2 * t] = tg1;
      a.gates_flat[2 * t + 1] = tg2;
    }
    sh.fe[2 * t] = (uint8_t)r.i1;  // the critical-path use of fe ended at an earlier barrier
    sh.fe[2 * t + 1] = (uint8_t)r.i2;
  }
  tm_lds_barrier();

  // 4a. per-chunk expert counts and in-chunk ranks from ballots
  for (int q = wave; q < nchunk; q += NW) {
    const int s = q * 64 + lane;
    const int fe = (s < nslot) ? (int)sh.fe[s] : -1;
    int mycnt = 0, inrank = 0;
    for (int e = 0; e < E; ++e) {
      const unsigned long long m = __ballot(fe == e);
      if (lane == e) mycnt = __popcll(m);
      if (fe == e) inrank = __popcll(m & ((1ull << lane) - 1ull));
    }
    if (lane < E) sh.cnt[q * TM_MAX_EXPERTS + lane] = (uint16_t)mycnt;
    if (s < nslot) sh.inrank[s] = (uint8_t)inrank;
  }
  tm_lds_barrier();
  // 4b. exclusive scan over chunks (slot order) per expert; chunks q and q+64
  //     of one expert sit in lane q of the wave that owns the expert.
  for (int e = wave; e < E; e += NW) {
    const int v0 = (lane < nchunk) ? (int)sh.cnt[lane * TM_MAX_EXPERTS + e] : 0;
    const int v1 = (lane + 64 < nchunk) ? (int)sh.cnt[(lane + 64) * TM_MAX_EXPERTS + e] : 0;
    int tot0, tot1;
    const int x0 = wave_exclusive_scan(v0, lane, &tot0);
    const int x1 = wave_exclusive_scan(v1, lane, &tot1);
    if (lane < nchunk) sh.cnt[lane * TM_MAX_EXPERTS + e] = (uint16_t)x0;
    if (lane + 64 < nchunk) sh.cnt[(lane + 64) * TM_MAX_EXPERTS + e] = (uint16_t)(tot0 + x1);
    if (lane == 0) sh.count[e] = tot0 + tot1;
  }
  tm_lds_barrier();
  // 4c. block layout (reference), compact offsets and GEMM tiles (wave 0,
  //     lane = expert)
  if (wave == 0) {
    const int c = (lane < E) ? sh.count[lane] : 0;
    int tot_off;
    const int off = wave_exclusive_scan(c, lane, &tot_off);
    if (lane < E) sh.offset[lane] = off;
    if (lane == 0) sh.offset[E] = tot_off;
    if constexpr (WRITE) {
      const int nb = (c + a.BM - 1) / a.BM;
      const int nt = (c + TM_GEMM_TILE_M - 1) / TM_GEMM_TILE_M;
      int tot_blk, tot_tiles;
      const int bs = wave_exclusive_scan(nb, lane, &tot_blk);
      const int ts = wave_exclusive_scan(nt, lane, &tot_tiles);
      if (lane < E) {
        sh.block_start[lane] = bs;
        sh.nblocks[lane] = nb;
        a.expert_offsets[lane] = off;
        for (int b = bs; b < min(bs + nb, a.max_blocks); ++b) sh.owner[b] = (int16_t)lane;
        for (int k = 0; k < nt; ++k) {
          const int j = ts + k;
          if (j < a.max_tiles) {
            a.tiles[4 * j + 0] = lane;
            a.tiles[4 * j + 1] = off + k * TM_GEMM_TILE_M;
            a.tiles[4 * j + 2] = min(TM_GEMM_TILE_M, c - k * TM_GEMM_TILE_M);
            a.tiles[4 * j + 3] = 0;
          }
        }
      }
      if (lane == 0) a.expert_offsets[E] = tot_off;
      for (int j = tot_tiles + lane; j < a.max_tiles; j += 64) {
        a.tiles[4 * j + 0] = -1;
        a.tiles[4 * j + 1] = 0;
        a.tiles[4 * j + 2] = 0;
        a.tiles[4 * j + 3] = 0;
      }
    }
  }
  tm_lds_barrier();
  // 4d. destinations of every slot, and the owner of every padded block
  for (int s = tid; s < nslot; s += NT) {
    const int fe = sh.fe[s];
    const int rank = (int)sh.cnt[(s >> 6) * TM_MAX_EXPERTS + fe] + (int)sh.inrank[s];
    const int pos = sh.offset[fe] + rank;
    if constexpr (WRITE) {
      a.slot_to_row[s] = sh.block_start[fe] * a.BM + rank;
      a.sorted_slots[pos] = s;
      a.slot_pos[s] = pos;
    }
    sh.sorted[pos] = (uint16_t)s;
  }
  if constexpr (WRITE) {
    for (int b = tid; b < a.max_blocks; b += NT) a.block_expert_ids[b] = sh.owner[b];
  }
  tm_lds_barrier();
  // 4e. padded rows: row i of block b holds the (i - first row of the owner)-th
  //     slot of the owning expert, or -1 past its count or in an unused block.
  if constexpr (WRITE) {
    for (int i = tid; i < padded_rows; i += NT) {
      const int e = sh.owner[i / a.BM];
      int64_t slot = -1;
      if (e >= 0) {
        const int rank = i - sh.block_start[e] * a.BM;
        if (rank < sh.count[e]) slot = sh.sorted[sh.offset[e] + rank];
      }
      a.padded_slots[i] = slot;
    }
  }
}

}  // namespace tmb
