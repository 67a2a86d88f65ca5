// op1 routing on gfx950: router logits + softmax, then op3 budget routing and
// stable (expert, DFS-order) bucketing.
//
// Every floating-point operation here is written out in a fixed order with
// contraction disabled, so that the CPU restatement reproduces the outputs bit
// for bit: expert ids, gate weights, demand and every layout index.
//
// Launch shapes: the router runs one workgroup (8 waves) per token, one wave
// per expert, or from 1024 tokens one wave per token with W_g in LDS; the
// bucketing runs in one workgroup.  They are two launches:
// handing the gates to a last-finishing workgroup instead would need a
// device-scope release fence per workgroup (an L2 write-back), which measured
// slower than the kernel boundary.
#pragma clang fp contract(off)

#include "op1_bucket.h"
#include "tm_common.h"

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
// The bucketing kernel keeps every per-slot intermediate in LDS up to this
// many tokens; larger layers use tm_bucket_large_kernel.
constexpr int kLdsMaxTokens = 4096;
constexpr int kMaxPaddedRows = 16384;
// Tokens from which the row router runs: its per-workgroup W_g copy costs
// ~8 us, so below ~1024 tokens one workgroup per token is faster (T = 512:
// 6.1 against 8.6 us; T = 2048: 14.0 against 9.2 us; T = 4096: 25.4 against
// 13.1 us at H = 4096, E = 8).
constexpr int kRowsMinTokens = 1024;

// The two 16-bit elements of a 32-bit word, widened exactly to fp32 (DT is
// TM_DTYPE_BF16 or TM_DTYPE_F16).
template <int DT>
__device__ __forceinline__ float lo16(uint32_t w) {
  return DT == TM_DTYPE_F16 ? tm_f16_to_f32((uint16_t)(w & 0xffffu)) : __uint_as_float(w << 16);
}
template <int DT>
__device__ __forceinline__ float hi16(uint32_t w) {
  return DT == TM_DTYPE_F16 ? tm_f16_to_f32((uint16_t)(w >> 16))
                            : __uint_as_float(w & 0xffff0000u);
}

template <int DT>
__device__ __forceinline__ float fma8(uint4 xv, uint4 wv, float acc) {
  acc = fmaf(lo16<DT>(xv.x), lo16<DT>(wv.x), acc);
  acc = fmaf(hi16<DT>(xv.x), hi16<DT>(wv.x), acc);
  acc = fmaf(lo16<DT>(xv.y), lo16<DT>(wv.y), acc);
  acc = fmaf(hi16<DT>(xv.y), hi16<DT>(wv.y), acc);
  acc = fmaf(lo16<DT>(xv.z), lo16<DT>(wv.z), acc);
  acc = fmaf(hi16<DT>(xv.z), hi16<DT>(wv.z), acc);
  acc = fmaf(lo16<DT>(xv.w), lo16<DT>(wv.w), acc);
  acc = fmaf(hi16<DT>(xv.w), hi16<DT>(wv.w), acc);
  return acc;
}

// Softmax of one token's E logits (s_logit, bf16-rounded) by one wave: max,
// e^(l - max), a sum in expert order, a correctly rounded division.
__device__ __forceinline__ void router_softmax(const float* s_logit, float* __restrict__ gates,
                                               int t, int E, int lane) {
  const float my_logit = (lane < E) ? s_logit[lane] : 0.0f;
  float m = (lane < E) ? my_logit : -INFINITY;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  const float ex = (lane < E) ? tm_expf_det(my_logit - m) : 0.0f;
  float s = 0.0f;
  for (int e = 0; e < E; ++e) s = s + __shfl(ex, e);
  if (lane < E) gates[(size_t)t * E + lane] = ex / s;
}

// Router for token t in one workgroup.  Logit (t, e): lane l of the wave that
// owns expert e accumulates the 8-element chunks l, l+64, ... in element order
// (fmaf of exact products of the 16-bit inputs); the 64 lane sums are combined
// by a halving tree (xor butterfly) and rounded to the input type (bf16 or
// fp16), as F.linear on such operands returns (treemoe/kernels/op1_tree_moe.py:676).  Softmax (:677) in fp32: max,
// e^(l - max), a sum in expert order, a correctly rounded division.
template <int DT>
__device__ __forceinline__ void router_token(const uint16_t* __restrict__ x,
                                             const uint16_t* __restrict__ wg,
                                             float* __restrict__ gates, int t, int H, int E,
                                             float* s_logit) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int nchunk = H >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)t * H);
  for (int e = wave; e < E; e += kWaves) {
    const uint4* wr = reinterpret_cast<const uint4*>(wg + (size_t)e * H);
    float acc = 0.0f;
    int c = lane;
    for (; c + 64 * 7 < nchunk; c += 64 * 8) {
      uint4 xv[8], wv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        xv[u] = xr[c + 64 * u];
        wv[u] = wr[c + 64 * u];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = fma8<DT>(xv[u], wv[u], acc);
    }
    for (; c < nchunk; c += 64) acc = fma8<DT>(xr[c], wr[c], acc);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = acc + __shfl_xor(acc, off);
    if (lane == 0) s_logit[e] = Half16<DT>::to_f32(Half16<DT>::round(acc));
  }
  __syncthreads();
  if (wave == 0) router_softmax(s_logit, gates, t, E, lane);
}

using tmb::BucketArgs;
constexpr int kMaxBlocks = kMaxPaddedRows / 16;
// gates staged in LDS when T * E fits (64 KB)
using BucketShared = tmb::BucketSharedT<kLdsMaxTokens, 16384, kMaxBlocks>;
using tmb::Top2;
using tmb::wave_exclusive_scan;

template <int DT>
__global__ void __launch_bounds__(kThreads)
tm_router_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg,
                 float* __restrict__ gates, int T, int H, int E) {
  __shared__ float s_logit[TM_MAX_EXPERTS];
  router_token<DT>(x, wg, gates, blockIdx.x, H, E, s_logit);
}

// Router for many tokens: wave w of workgroup b takes token kWaves b + w and
// all E experts.  x stays in registers (XC 16-byte chunks per lane, H = 512
// XC) and W_g in LDS, read once per workgroup instead of once per token.  Lane
// l accumulates its chunks l, l+64, ... of each expert in the order
// router_token uses, then the same xor fold, rounding and softmax, so the
// gates are bit-identical to it.
constexpr int kRowsLdsChunks = 4096;  // W_g staged in LDS: E * H / 8 <= 4096 (64 KB)

template <int DT, int XC>
__global__ void __launch_bounds__(kThreads)
tm_router_rows_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg,
                      float* __restrict__ gates, int T, int H, int E) {
  __shared__ uint4 s_w[kRowsLdsChunks];
  __shared__ float s_logit[kWaves][TM_MAX_EXPERTS];
  const int nchunk = H >> 3;  // = 64 XC
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * kWaves + wave;
  // the token's row is requested before the W_g copy, so the two memory
  // round trips overlap instead of following each other (T = 2048: 14.9 ->
  // 14.2 us)
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)min(t, T - 1) * H);
  uint4 xv[XC];
#pragma unroll
  for (int u = 0; u < XC; ++u) xv[u] = xr[lane + 64 * u];
  const uint4* wg4 = reinterpret_cast<const uint4*>(wg);
  for (int i = threadIdx.x; i < E * nchunk; i += kThreads) s_w[i] = wg4[i];
  tm_lds_barrier();
  if (t >= T) return;
  for (int e = 0; e < E; ++e) {
    const uint4* wr = s_w + e * nchunk;
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < XC; ++u) acc = fma8<DT>(xv[u], wr[lane + 64 * u], acc);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = acc + __shfl_xor(acc, off);
    if (lane == 0) s_logit[wave][e] = Half16<DT>::to_f32(Half16<DT>::round(acc));
  }
  // s_logit[wave] is written and read by this wave only: its LDS operations
  // complete in order
  router_softmax(s_logit[wave], gates, t, E, lane);
}

// Launch the router: the row kernel when W_g fits its LDS copy, H is one of
// its register shapes and there are enough tokens to fill the chip with
// workgroups of kWaves tokens; otherwise one workgroup per token.
template <int DT>
void launch_router_dt(const uint16_t* x, const uint16_t* wg, float* gates, int T, int H, int E,
                      hipStream_t stream) {
  const bool rows_ok = T >= kRowsMinTokens && E * (H / 8) <= kRowsLdsChunks;
  const dim3 rgrid((unsigned)((T + kWaves - 1) / kWaves));
  if (rows_ok && H == 2048) {
    hipLaunchKernelGGL((tm_router_rows_kernel<DT, 4>), rgrid, dim3(kThreads), 0, stream, x, wg,
                       gates, T, H, E);
  } else if (rows_ok && H == 4096) {
    hipLaunchKernelGGL((tm_router_rows_kernel<DT, 8>), rgrid, dim3(kThreads), 0, stream, x, wg,
                       gates, T, H, E);
  } else {
    hipLaunchKernelGGL(tm_router_kernel<DT>, dim3((unsigned)T), dim3(kThreads), 0, stream, x, wg,
                       gates, T, H, E);
  }
}

void launch_router(const uint16_t* x, const uint16_t* wg, float* gates, int T, int H, int E,
                   int dtype, hipStream_t stream) {
  if (dtype == TM_DTYPE_F16)
    launch_router_dt<TM_DTYPE_F16>(x, wg, gates, T, H, E, stream);
  else
    launch_router_dt<TM_DTYPE_BF16>(x, wg, gates, T, H, E, stream);
}

__global__ void __launch_bounds__(kThreads) tm_bucket_kernel(BucketArgs args) {
  __shared__ __attribute__((aligned(16))) BucketShared sh;
  tmb::bucket_phases<kThreads, BucketShared, true>(args, sh);
}

// ------------------------------------------------------ many tokens --
// The same budget routing and bucketing for T > kLdsMaxTokens, whose per-slot
// intermediates do not fit LDS.  One workgroup of 1024 threads, the phases and
// every floating-point operation in the order of tmb::bucket_phases (so the outputs
// equal what tmb::bucket_phases would compute); the intermediates live in the output
// buffers, each overwritten by its final value after its last use:
//   expert of slot s           topk_ids[s]                  (final in phase 3)
//   rank of s in its chunk     slot_pos[s] -> its position  (final in 4d)
//   per-chunk expert counts    slot_to_row, as int32 words  (final in 4d)
//   expert of padded block b   block_expert_ids[b]          (final in 4c)
//   compact order              sorted_slots                 (final in 4d)
// Phases exchange data through global memory, so they are separated by
// __syncthreads() (its workgroup-scope release/acquire orders the stores and
// loads of the workgroup's waves).
constexpr int kLargeThreads = 1024;
constexpr int kLargeWaves = kLargeThreads / 64;

__global__ void __launch_bounds__(kLargeThreads) tm_bucket_large_kernel(BucketArgs a) {
  __shared__ float s_demand[TM_MAX_EXPERTS], s_crit[TM_MAX_EXPERTS];
  __shared__ int s_count[TM_MAX_EXPERTS], s_block_start[TM_MAX_EXPERTS + 1];
  __shared__ int s_offset[TM_MAX_EXPERTS + 1], s_tile_start[TM_MAX_EXPERTS + 1];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int T = a.T, E = a.E;
  const int nslot = 2 * T;
  const int nchunk = (nslot + 63) >> 6;
  const int padded_rows = a.max_blocks * a.BM;
  const bool critical = a.objective == TM_OBJECTIVE_CRITICAL_PATH;
  const float* G = a.gates;
  int64_t* fe = a.topk_ids;                                 // expert of slot s
  int32_t* cnt = reinterpret_cast<int32_t*>(a.slot_to_row); // [nchunk][E], 4T words

  if (critical) {  // unrestricted top-1 / top-2 of every token
    for (int t = tid; t < T; t += kLargeThreads) {
      const float* g = G + (size_t)t * E;
      Top2 r{-1, -1, 0.0f, 0.0f};
      for (int e = 0; e < E; ++e) r.offer(g[e], e);
      fe[2 * t] = r.i1;
      fe[2 * t + 1] = r.i2;
    }
    __syncthreads();
  }
  // 1. demand (and criticality): lane-strided partials in token order, xor fold
  for (int e = wave; e < E; e += kLargeWaves) {
    float acc = 0.0f;
    float crit = -INFINITY;
    for (int t = lane; t < T; t += 64) {
      const float av = a.accept[t];
      const float p = av * G[(size_t)t * E + e];
      acc = acc + p;
      if (critical) {
        const bool needed = (fe[2 * t] == e) || ((fe[2 * t + 1] == e) && (av >= a.tau));
        if (needed) crit = fmaxf(crit, av);
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
      a.demand_out[e] = acc;
    }
  }
  __syncthreads();
  // 2. keep set (every wave; as in tmb::bucket_phases)
  unsigned long long keep;
  {
    const float d = lane < E ? s_demand[lane] : 0.0f;
    const float c = (critical && lane < E) ? s_crit[lane] : 0.0f;
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
  // 3. in-budget top-2, renormalisation, degrade
  for (int t = tid; t < T; t += kLargeThreads) {
    const float* g = G + (size_t)t * E;
    Top2 r{-1, -1, 0.0f, 0.0f};
    for (int e = 0; e < E; ++e) r.offer(((keep >> e) & 1ull) ? g[e] : 0.0f, e);
    const float s = r.g1 + r.g2;
    float tg1 = r.g1 / s;
    float tg2 = r.g2 / s;
    if (a.accept[t] < a.tau) { tg1 = 1.0f; tg2 = 0.0f; }
    fe[2 * t] = r.i1;
    fe[2 * t + 1] = r.i2;
    a.gates_flat[2 * t] = tg1;
    a.gates_flat[2 * t + 1] = tg2;
  }
  __syncthreads();
  // 4a. per-chunk expert counts and in-chunk ranks from ballots
  for (int q = wave; q < nchunk; q += kLargeWaves) {
    const int sl = q * 64 + lane;
    const int f = (sl < nslot) ? (int)fe[sl] : -1;
    int mycnt = 0, inrank = 0;
    for (int e = 0; e < E; ++e) {
      const unsigned long long m = __ballot(f == e);
      if (lane == e) mycnt = __popcll(m);
      if (f == e) inrank = __popcll(m & ((1ull << lane) - 1ull));
    }
    if (lane < E) cnt[(size_t)q * E + lane] = mycnt;
    if (sl < nslot) a.slot_pos[sl] = inrank;
  }
  __syncthreads();
  // 4b. exclusive scan over chunks (slot order) per expert, 64 chunks per step
  for (int e = wave; e < E; e += kLargeWaves) {
    int carry = 0;
    for (int q0 = 0; q0 < nchunk; q0 += 64) {
      const int q = q0 + lane;
      const int v = (q < nchunk) ? cnt[(size_t)q * E + e] : 0;
      int tot;
      const int x = wave_exclusive_scan(v, lane, &tot);
      if (q < nchunk) cnt[(size_t)q * E + e] = carry + x;
      carry += tot;
    }
    if (lane == 0) s_count[e] = carry;
  }
  __syncthreads();
  // 4c. offsets, block starts and tile starts (wave 0, lane = expert)
  if (wave == 0) {
    const int c = (lane < E) ? s_count[lane] : 0;
    int tot_off, tot_blk, tot_tiles;
    const int off = wave_exclusive_scan(c, lane, &tot_off);
    const int bs = wave_exclusive_scan((c + a.BM - 1) / a.BM, lane, &tot_blk);
    const int ts = wave_exclusive_scan((c + TM_GEMM_TILE_M - 1) / TM_GEMM_TILE_M, lane, &tot_tiles);
    if (lane < E) {
      s_offset[lane] = off;
      s_block_start[lane] = bs;
      s_tile_start[lane] = ts;
      a.expert_offsets[lane] = off;
    }
    if (lane == 0) {
      s_offset[E] = tot_off;
      s_block_start[E] = tot_blk;
      s_tile_start[E] = tot_tiles;
      a.expert_offsets[E] = tot_off;
    }
  }
  __syncthreads();
  // owners of the padded blocks and the GEMM tiles, one thread per entry
  for (int b = tid; b < a.max_blocks; b += kLargeThreads) {
    int owner = -1;
    for (int e = 0; e < E; ++e)
      if (b >= s_block_start[e] && b < s_block_start[e + 1]) owner = e;
    a.block_expert_ids[b] = owner;
  }
  for (int j = tid; j < a.max_tiles; j += kLargeThreads) {
    int e = -1;
    for (int k = 0; k < E; ++k)
      if (j >= s_tile_start[k] && j < s_tile_start[k + 1]) e = k;
    int32_t* tl = a.tiles + 4 * j;
    if (e >= 0) {
      const int k = j - s_tile_start[e];
      tl[0] = e;
      tl[1] = s_offset[e] + k * TM_GEMM_TILE_M;
      tl[2] = min(TM_GEMM_TILE_M, s_count[e] - k * TM_GEMM_TILE_M);
    } else {
      tl[0] = -1;
      tl[1] = 0;
      tl[2] = 0;
    }
    tl[3] = 0;
  }
  // 4d. positions (slot_pos holds the in-chunk rank until its own thread
  //     replaces it), then the compact order and the padded rows of the slots
  for (int sl = tid; sl < nslot; sl += kLargeThreads) {
    const int f = (int)fe[sl];
    const int rank = cnt[(size_t)(sl >> 6) * E + f] + a.slot_pos[sl];
    a.slot_pos[sl] = s_offset[f] + rank;
  }
  __syncthreads();
  for (int sl = tid; sl < nslot; sl += kLargeThreads) {
    const int f = (int)fe[sl];
    const int pos = a.slot_pos[sl];
    a.slot_to_row[sl] = (int64_t)s_block_start[f] * a.BM + (pos - s_offset[f]);
    a.sorted_slots[pos] = sl;
  }
  __syncthreads();
  // 4e. padded rows
  for (int i = tid; i < padded_rows; i += kLargeThreads) {
    const int e = (int)a.block_expert_ids[i / a.BM];
    int64_t slot = -1;
    if (e >= 0) {
      const int rank = i - s_block_start[e] * a.BM;
      if (rank < s_count[e]) slot = a.sorted_slots[s_offset[e] + rank];
    }
    a.padded_slots[i] = slot;
  }
}

int check_bucket_args(int64_t T, int64_t E, int64_t budget, int objective, int64_t block_m,
                      int64_t max_blocks, int64_t max_tiles) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS) return TM_ERR_SHAPE;
  if (budget < 2 || budget > E) return TM_ERR_ARG;
  if (objective != TM_OBJECTIVE_MASS && objective != TM_OBJECTIVE_CRITICAL_PATH) return TM_ERR_ARG;
  if (block_m != 16 && block_m != 32) return TM_ERR_ARG;
  if (max_blocks < 1 || max_tiles < 1) return TM_ERR_SHAPE;
  if (T <= kLdsMaxTokens ? max_blocks * block_m > kMaxPaddedRows
                         : max_blocks * block_m > (int64_t)1 << 30)
    return TM_ERR_SHAPE;
  return TM_OK;
}

// The bucketing launch for T tokens: LDS-resident up to kLdsMaxTokens (and
// kMaxPaddedRows padded rows), else the many-token kernel.
void launch_bucket(const BucketArgs& a, hipStream_t stream) {
  if (a.T <= kLdsMaxTokens && a.max_blocks * a.BM <= kMaxPaddedRows) {
    hipLaunchKernelGGL(tm_bucket_kernel, dim3(1), dim3(kThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL(tm_bucket_large_kernel, dim3(1), dim3(kLargeThreads), 0, stream, a);
  }
}

BucketArgs make_args(const float* gates, const float* accept, int64_t T, int64_t E,
                     int64_t budget, float tau, int objective, int64_t block_m,
                     int64_t max_blocks, int64_t max_tiles, int64_t* topk_ids,
                     float* gates_flat, int64_t* padded_slots, int64_t* block_expert_ids,
                     int64_t* slot_to_row, float* demand, int32_t* expert_offsets,
                     int32_t* sorted_slots, int32_t* slot_pos, int32_t* tiles) {
  BucketArgs a;
  a.gates = gates;
  a.accept = accept;
  a.T = (int)T;
  a.E = (int)E;
  a.budget = (int)budget;
  a.objective = objective;
  a.BM = (int)block_m;
  a.max_blocks = (int)max_blocks;
  a.max_tiles = (int)max_tiles;
  a.tau = tau;
  a.topk_ids = topk_ids;
  a.gates_flat = gates_flat;
  a.padded_slots = padded_slots;
  a.block_expert_ids = block_expert_ids;
  a.slot_to_row = slot_to_row;
  a.demand_out = demand;
  a.expert_offsets = expert_offsets;
  a.sorted_slots = sorted_slots;
  a.slot_pos = slot_pos;
  a.tiles = tiles;
  return a;
}

}  // namespace

extern "C" int tm_op1_router_gates(const void* x, const void* wg, int64_t T, int64_t H,
                                   int64_t E, float* gates, int dtype, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS || H < 8 || (H % 8) != 0)
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_BF16 && dtype != TM_DTYPE_F16) return TM_ERR_ARG;
  if (((uintptr_t)x % 16) != 0 || ((uintptr_t)wg % 16) != 0) return TM_ERR_ALIGN;
  launch_router((const uint16_t*)x, (const uint16_t*)wg, gates, (int)T, (int)H, (int)E, dtype,
                (hipStream_t)stream);
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
  const int rc = check_bucket_args(T, E, budget, objective, block_m, max_blocks, max_tiles);
  if (rc != TM_OK) return rc;
  const BucketArgs a = make_args(gates, accept, T, E, budget, tau, objective, block_m, max_blocks,
                                 max_tiles, topk_ids, gates_flat, padded_slots,
                                 block_expert_ids, slot_to_row, demand, expert_offsets,
                                 sorted_slots, slot_pos, tiles);
  launch_bucket(a, (hipStream_t)stream);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op1_route(const void* x, const void* wg, const float* accept, int64_t T,
                            int64_t H, int64_t E, int64_t budget, float tau, int objective,
                            int64_t block_m, int64_t max_blocks, int64_t max_tiles,
                            float* gates, int64_t* topk_ids, float* gates_flat,
                            int64_t* padded_slots, int64_t* block_expert_ids,
                            int64_t* slot_to_row, float* demand, int32_t* expert_offsets,
                            int32_t* sorted_slots, int32_t* slot_pos, int32_t* tiles,
                            int dtype, void* stream) {
  const int rc = check_bucket_args(T, E, budget, objective, block_m, max_blocks, max_tiles);
  if (rc != TM_OK) return rc;
  if (H < 8 || (H % 8) != 0) return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_BF16 && dtype != TM_DTYPE_F16) return TM_ERR_ARG;
  if (((uintptr_t)x % 16) != 0 || ((uintptr_t)wg % 16) != 0) return TM_ERR_ALIGN;
  const BucketArgs a = make_args(gates, accept, T, E, budget, tau, objective, block_m, max_blocks,
                                 max_tiles, topk_ids, gates_flat, padded_slots,
                                 block_expert_ids, slot_to_row, demand, expert_offsets,
                                 sorted_slots, slot_pos, tiles);
  launch_router((const uint16_t*)x, (const uint16_t*)wg, gates, (int)T, (int)H, (int)E, dtype,
                (hipStream_t)stream);
  TM_HIP_CHECK_LAUNCH();
  launch_bucket(a, (hipStream_t)stream);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}
