// op4 on gfx950: first-occurrence argmax over the vocabulary for every tree
// node (row-chunked over many workgroups), the greedy accept walk from LDS in
// one workgroup, and the paged KV commit of [root] + accepted path.
#include <atomic>
#include <climits>
#include <mutex>

#include "tm_common.h"

namespace {

constexpr int kArgThreads = 256;
constexpr int kWalkThreads = 1024;
constexpr int kChunkBytes = 4096;    // bytes of one row scanned by one workgroup
constexpr int kStageNodes = 2048;    // trees up to this size are walked from LDS

// (va, ia) ranks before (vb, ib): larger value first, NaN above every number,
// equal values (and NaN vs NaN) go to the lower index.  This is the order in
// which torch.argmax / numpy.argmax pick their first maximum.
__device__ __forceinline__ bool tm_ranks_before(float va, int ia, float vb, int ib) {
  const bool na = va != va;
  const bool nb = vb != vb;
  if (na != nb) return na;
  if (!na && va != vb) return va > vb;
  return ia < ib;
}

struct Best {
  float v;
  int i;
  __device__ __forceinline__ void offer(float v2, int i2) {
    if (tm_ranks_before(v2, i2, v, i)) { v = v2; i = i2; }
  }
};

struct Partial {
  float v;
  int i;
};

__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(b.v, off);
    const int oi = __shfl_xor(b.i, off);
    b.offer(ov, oi);
  }
  return b;
}

// Elements [lo, hi) of one row.  `vec` rows are 16-byte aligned and lo is a
// multiple of the vector width, so every thread issues its (at most
// kChunkBytes / 16 / kArgThreads = 1) 16-byte load before any compare.
template <int kDtype>
__device__ __forceinline__ Best scan_range(const void* row_ptr, int lo, int hi, bool vec) {
  Best b{-INFINITY, 0x7fffffff};
  const int tid = threadIdx.x;
  if (kDtype == TM_DTYPE_F32) {
    const float* p = reinterpret_cast<const float*>(row_ptr);
    int done = lo;
    if (vec) {
      const int nv = (hi - lo) >> 2;
      const float4* p4 = reinterpret_cast<const float4*>(p + lo);
      for (int q = tid; q < nv; q += kArgThreads) {
        const float4 v = p4[q];
        const int e = lo + 4 * q;
        b.offer(v.x, e);
        b.offer(v.y, e + 1);
        b.offer(v.z, e + 2);
        b.offer(v.w, e + 3);
      }
      done = lo + (nv << 2);
    }
    for (int q = done + tid; q < hi; q += kArgThreads) b.offer(p[q], q);
  } else {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(row_ptr);
    int done = lo;
    if (vec) {
      const int nv = (hi - lo) >> 3;
      const uint4* p8 = reinterpret_cast<const uint4*>(p + lo);
      for (int q = tid; q < nv; q += kArgThreads) {
        const uint4 v = p8[q];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        const int e = lo + 8 * q;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          b.offer(__uint_as_float(w[j] << 16), e + 2 * j);
          b.offer(__uint_as_float(w[j] & 0xffff0000u), e + 2 * j + 1);
        }
      }
      done = lo + (nv << 3);
    }
    for (int q = done + tid; q < hi; q += kArgThreads) b.offer(tm_bf16_to_f32(p[q]), q);
  }
  return b;
}

// grid (parts, N): workgroup (p, row) writes the best (value, index) of
// elements [p * per_part, min(V, (p + 1) * per_part)) of `row` to
// partial[row * parts + p].  An empty range writes (-inf, INT_MAX), which
// every element ranks before.
template <int kDtype>
__global__ void __launch_bounds__(kArgThreads)
tm_argmax_part_kernel(const void* __restrict__ logits, int V, int64_t row_stride, int per_part,
                      int parts, int vec_ok, Partial* __restrict__ partial) {
  __shared__ float s_v[kArgThreads / 64];
  __shared__ int s_i[kArgThreads / 64];
  const int p = blockIdx.x;
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const size_t elem = (kDtype == TM_DTYPE_F32) ? 4 : 2;
  const char* row_ptr = reinterpret_cast<const char*>(logits) + (size_t)row * row_stride * elem;
  const int lo = min(V, p * per_part);
  const int hi = min(V, lo + per_part);
  Best b = wave_best(scan_range<kDtype>(row_ptr, lo, hi, vec_ok != 0));
  if (lane == 0) {
    s_v[wave] = b.v;
    s_i[wave] = b.i;
  }
  __syncthreads();
  if (tid == 0) {
    Best r{s_v[0], s_i[0]};
    for (int w = 1; w < kArgThreads / 64; ++w) r.offer(s_v[w], s_i[w]);
    partial[(size_t)row * parts + p] = Partial{r.v, r.i};
  }
}

// Entries of a node's child range [st, st + cnt) that lie inside the
// num_edges-entry child list (all of them for a well-formed CSR).
__device__ __forceinline__ int edge_count(int st, int cnt, int num_edges) {
  if (st < 0 || st >= num_edges || cnt <= 0) return 0;
  return min(cnt, num_edges - st);
}

struct WalkShared {
  int64_t tokens[kStageNodes];
  int argmax[kStageNodes];
  int child_start[kStageNodes];
  int child_count[kStageNodes];
  int child_list[kStageNodes];
  int next[kStageNodes];  // each node's accepted child, -1 if none
  int count;
};

// One workgroup: reduce the row partials to argmax[N], then the greedy walk
// from the root (op4_commit.py:99-131): at each level take the first child,
// in child-list order, whose token equals the node's argmax.  Trees of at
// most kStageNodes nodes are staged in LDS first and every node's accepted
// child is found in parallel (one thread per node), so the serial walk is a
// chase of one LDS read per level; larger trees are walked from global
// memory.  The walk also stops once N nodes are accepted (only a child list
// with a cycle gets there), so accepted_slots is never written past N.
__global__ void __launch_bounds__(kWalkThreads)
tm_walk_kernel(const Partial* __restrict__ partial, int parts, int N,
               const int64_t* __restrict__ tokens, const int32_t* __restrict__ child_start,
               const int32_t* __restrict__ child_count, const int32_t* __restrict__ child_list,
               int num_edges, int max_depth, int32_t* __restrict__ argmax,
               int64_t* __restrict__ accepted_slots,
               int64_t* __restrict__ accepted_tokens, int64_t* __restrict__ result) {
  __shared__ WalkShared sh;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // child_list holds num_edges entries; a node's range is clipped to it and a
  // child index outside [0, N) never matches, so no read leaves the buffers.
  const bool staged = N <= kStageNodes && num_edges <= kStageNodes;
  if (staged) {
    for (int i = tid; i < N; i += kWalkThreads) {
      sh.tokens[i] = tokens[i];
      sh.child_start[i] = child_start[i];
      sh.child_count[i] = child_count[i];
    }
    for (int i = tid; i < num_edges; i += kWalkThreads) sh.child_list[i] = child_list[i];
  }
  // Row partials: lane l of a wave takes part l % P of row r0 + l / P, with
  // P = parts rounded up to a power of two (<= 64), so one load per lane and
  // log2(P) xor steps reduce 64 / P rows at once.  The ranking is a total
  // order, so the order of the steps does not change the result.
  static_assert(TM_OP4_MAX_PARTS <= 64, "a row's partials fit one wave");
  int logp = 0;
  while ((1 << logp) < parts) ++logp;
  const int rows_per_wave = 64 >> logp;
  for (int r0 = wave * rows_per_wave; r0 < N; r0 += (kWalkThreads / 64) * rows_per_wave) {
    const int row = r0 + (lane >> logp);
    const int p = lane & ((1 << logp) - 1);
    Best b{-INFINITY, 0x7fffffff};
    if (row < N && p < parts) {
      const Partial q = partial[(size_t)row * parts + p];
      b.offer(q.v, q.i);
    }
    for (int off = (1 << logp) >> 1; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(b.v, off);
      const int oi = __shfl_xor(b.i, off);
      b.offer(ov, oi);
    }
    if (p == 0 && row < N) {
      argmax[row] = b.i;
      if (staged) sh.argmax[row] = b.i;
    }
  }
  // A staged walk reads only LDS: an LDS-only barrier, which does not wait
  // for the argmax stores.  Otherwise the walk reads argmax back from global
  // memory, which needs __syncthreads()'s release/acquire.
  if (staged) {
    tm_lds_barrier();
  } else {
    __syncthreads();
  }
  const int64_t* tok = staged ? sh.tokens : tokens;
  const int* am = staged ? sh.argmax : argmax;
  const int* cs = staged ? sh.child_start : child_start;
  const int* cc = staged ? sh.child_count : child_count;
  const int* cl = staged ? sh.child_list : child_list;
  if (staged) {
    for (int i = tid; i < N; i += kWalkThreads) {
      const int64_t target = (int64_t)sh.argmax[i];
      const int st = sh.child_start[i];
      const int cnt = edge_count(st, sh.child_count[i], num_edges);
      int acc = -1;
      for (int j = 0; j < cnt; ++j) {
        const int c = sh.child_list[st + j];
        if (c >= 0 && c < N && sh.tokens[c] == target) { acc = c; break; }
      }
      sh.next[i] = acc;
    }
    tm_lds_barrier();
  }
  if (tid == 0) {
    int node = 0;
    int count = 0;
    for (int d = 0; d < max_depth && count < N; ++d) {
      int acc = -1;
      if (staged) {
        acc = sh.next[node];
      } else {
        const int64_t target = (int64_t)am[node];
        const int st = cs[node];
        const int cnt = edge_count(st, cc[node], num_edges);
        for (int j = 0; j < cnt; ++j) {
          const int c = cl[st + j];
          if (c >= 0 && c < N && tok[c] == target) { acc = c; break; }
        }
      }
      if (acc < 0) break;
      accepted_slots[count] = acc;
      accepted_tokens[count] = tok[acc];
      ++count;
      node = acc;
    }
    sh.count = count;
    result[0] = (int64_t)am[node];
    result[1] = count;
    result[2] = node;
  }
  tm_lds_barrier();  // sh.count; the padding below writes other entries
  for (int i = sh.count + tid; i < N; i += kWalkThreads) {
    accepted_slots[i] = -1;
    accepted_tokens[i] = -1;
  }
}

// One workgroup per (layer, path position j).  Pure byte copy of one KV row of
// K and of V from the tree scratch pages to the sequence tail.
__global__ void __launch_bounds__(256)
tm_kv_commit_kernel(uint8_t* __restrict__ k, uint8_t* __restrict__ v, int64_t row_bytes,
                    int64_t stride_layer_b, int64_t stride_page_b, int64_t stride_slot_b,
                    int64_t page_size, const int64_t* __restrict__ accepted_slots,
                    const int64_t* __restrict__ result, const int32_t* __restrict__ scratch_pages,
                    int64_t n_scratch, const int32_t* __restrict__ block_table, int64_t n_table,
                    int64_t seq_len, int vec16, int64_t* __restrict__ host_count) {
  const int layer = blockIdx.x;
  const int j = blockIdx.y;
  const int64_t num = result[1];
  // the accepted count for the host: a system-scope store to its mapped word,
  // pushed out of the GPU caches at once, so the host reads it without a copy
  if (host_count != nullptr && layer == 0 && j == 0 && threadIdx.x == 0) {
    __hip_atomic_store(host_count, num, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
  }
  if (j > num) return;
  const int64_t s = (j == 0) ? 0 : accepted_slots[j - 1];
  if (s < 0 || s / page_size >= n_scratch) return;
  const int64_t q = seq_len + j;
  if (q / page_size >= n_table) return;
  const int64_t sp = scratch_pages[s / page_size];
  const int64_t dp = block_table[q / page_size];
  const int64_t src = layer * stride_layer_b + sp * stride_page_b + (s % page_size) * stride_slot_b;
  const int64_t dst = layer * stride_layer_b + dp * stride_page_b + (q % page_size) * stride_slot_b;
  if (vec16) {
    const int64_t n16 = row_bytes >> 4;
    for (int64_t i = threadIdx.x; i < n16; i += 256) {
      reinterpret_cast<uint4*>(k + dst)[i] = reinterpret_cast<const uint4*>(k + src)[i];
      reinterpret_cast<uint4*>(v + dst)[i] = reinterpret_cast<const uint4*>(v + src)[i];
    }
  } else {
    for (int64_t i = threadIdx.x; i < row_bytes; i += 256) {
      k[dst + i] = k[src + i];
      v[dst + i] = v[src + i];
    }
  }
}

// ------------------------------------------------------- rep penalty --
// In place on every node row, reference `_postprocess_softmax_kernel` pass 0
// (op4_commit.py:53-57): for each prev token t (in order),
//   x[row, t] = x > 0 ? x / penalty : x * penalty,
// so a token listed k times is penalised k times.  The same function is
// applied each time, so only the count of each token matters.  One workgroup
// counts the distinct tokens in an open-addressing table of S slots (S a
// power of two >= 2 * num_prev; keys then counts, 2 * S int32 of global
// workspace), then a grid over (row, block of slots) applies each counted
// token's penalty.  Tokens outside [0, V) are skipped.
constexpr int kPenThreads = 1024;
constexpr int kPenLdsSlots = 8192;     // tables up to this size are built in LDS
constexpr int kApplyThreads = 256;
constexpr int kApplySlots = 4;         // table slots per thread (one 16-byte load)
constexpr int kApplyBlock = kApplyThreads * kApplySlots;

__device__ __forceinline__ uint32_t pen_hash(int64_t t, int S) {
  return ((uint32_t)t * 2654435761u) & (uint32_t)(S - 1);
}

// kLds: the table lives in LDS and is copied out at the end.  Otherwise every
// access is an agent-scope atomic on the global table, coherent at L2 whatever
// the L1 holds.  Either way the barriers order init, insert and copy-out.
template <bool kLds>
__global__ void __launch_bounds__(kPenThreads)
tm_rep_count_kernel(const int64_t* __restrict__ prev, int num_prev, int V,
                    int32_t* __restrict__ table, int S) {
  __shared__ int32_t s_tab[kLds ? 2 * kPenLdsSlots : 1];
  int32_t* keys = kLds ? s_tab : table;
  int32_t* counts = kLds ? s_tab + S : table + S;
  const int tid = threadIdx.x;
  for (int i = tid; i < S; i += kPenThreads) {
    if (kLds) {
      keys[i] = -1;
      counts[i] = 0;
    } else {
      __hip_atomic_store(&keys[i], -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&counts[i], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  for (int i = tid; i < num_prev; i += kPenThreads) {
    const int64_t t = prev[i];
    if (t < 0 || t >= V) continue;
    uint32_t h = pen_hash(t, S);
    for (int probe = 0; probe < S; ++probe) {
      const int prior = atomicCAS(&keys[h], -1, (int)t);
      if (prior == -1 || prior == (int)t) {
        atomicAdd(&counts[h], 1);
        break;
      }
      h = (h + 1) & (uint32_t)(S - 1);
    }
  }
  if (kLds) {
    __syncthreads();
    for (int i = tid; i < S; i += kPenThreads) {
      table[i] = keys[i];
      table[S + i] = counts[i];
    }
  }
}

// grid (N, slot blocks): thread reads kApplySlots (key, count) pairs with one
// 16-byte load each and applies every counted token to its row.  Distinct
// slots hold distinct tokens, so no two threads touch one logit.
template <int kDtype>
__global__ void __launch_bounds__(kApplyThreads)
tm_rep_apply_kernel(void* __restrict__ logits, int64_t row_stride,
                    const int32_t* __restrict__ table, int S, float penalty) {
  const int64_t row = blockIdx.x;
  for (int base = (blockIdx.y * kApplyThreads + threadIdx.x) * kApplySlots; base < S;
       base += gridDim.y * kApplyBlock) {
    const int4 k4 = *reinterpret_cast<const int4*>(table + base);
    const int4 c4 = *reinterpret_cast<const int4*>(table + S + base);
    const int keys[4] = {k4.x, k4.y, k4.z, k4.w};
    const int counts[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
    for (int j = 0; j < kApplySlots; ++j) {
      const int k = counts[j];
      if (k == 0) continue;
      const int64_t at = row * row_stride + keys[j];
      if (kDtype == TM_DTYPE_F32) {
        float* x = reinterpret_cast<float*>(logits) + at;
        float v = *x;
        for (int r = 0; r < k; ++r) v = v > 0.0f ? v / penalty : v * penalty;
        *x = v;
      } else {
        // the reference stores (rounds to bf16) after every application
        uint16_t* x = reinterpret_cast<uint16_t*>(logits) + at;
        uint16_t b = *x;
        for (int r = 0; r < k; ++r) {
          const float v = tm_bf16_to_f32(b);
          b = tm_f32_to_bf16(v > 0.0f ? v / penalty : v * penalty);
        }
        *x = b;
      }
    }
  }
}

// ---------------------------------------------------------- sampling --
// Tree rejection sampling, reference `tree_verify_ref` sampling branch
// (treemoe/ref/verify_ref.py:60-89), in one workgroup.  At the current node:
// p = softmax(logits[node] / temperature) becomes the residual; children are
// tried in child-list order: child c (token t) is accepted when
// uniforms[c] < min(residual[t] / max(q_c[t], 1e-20), 1), q_c = draft_probs[c];
// otherwise residual = max(residual - q_c, 0) / max(sum, 1e-20).  An accepted
// child becomes the node; when every child is rejected (or at a leaf) the
// bonus token is torch.multinomial(residual, 1)'s draw for the same generator
// state: PyTorch samples one index as argmax_j residual[j] / e[j] over
// e = empty_like(residual).exponential_(1, generator) (first maximum), and the
// caller passes that e.  Every reduction is in a fixed order, so the result
// is deterministic.
constexpr int kSampThreads = 1024;
constexpr int kSampWaves = kSampThreads / 64;

// NaN as torch has it.  torch.clamp_min / clamp(max=) keep a NaN (fmaxf and
// fminf would return the bound), so NaN logits reject every child as in the
// reference (u < NaN is false) instead of accepting the first.  The softmax
// maximum propagates NaN (IEEE maximum, one v_maximum3_f32 per two entries on
// gfx950, no dearer than fmaxf): a NaN logit, a +inf one (inf - inf) or a
// row of -inf makes the row NaN, as torch.softmax's.  (A NaN test on every
// entry instead cost ~4 us per config-4 call: the walk is VALU-bound.)
__device__ __forceinline__ float clamp_min_nan(float x, float lo) {
  return x != x ? x : fmaxf(x, lo);
}
__device__ __forceinline__ float clamp_max_nan(float x, float hi) {
  return x != x ? x : fminf(x, hi);
}
__device__ __forceinline__ float max_nan(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}
// e^(x - m) for the sampling softmax, given ml = m log2(e): the hardware
// exponential v_exp_f32 of fma(x, log2(e), -ml).  The walk is VALU-bound
// (1024 threads over a vocabulary row per node) and the software tm_expf_det
// costs ~15 operations per entry; the residual's parity with the reference is
// a tolerance (torch.softmax rounds differently from either), so the cheaper
// form serves.  NaN stays NaN (also inf - inf), -inf gives 0.
constexpr float kLog2e = 1.44269504088896341f;
__device__ __forceinline__ float exp_soft(float x, float ml) {
  return __builtin_amdgcn_exp2f(fmaf(x, kLog2e, -ml));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// x / d, correctly rounded, from rcp = 1 / d (itself correctly rounded):
// Markstein's correction q + (x - q d) * rcp, whose residual x - q d one FMA
// gives exactly.  Three VALU operations instead of the IEEE division sequence;
// a non-finite quotient (a -inf logit) is returned as x * rcp.
__device__ __forceinline__ float div_by(float x, float d, float rcp) {
  const float q = x * rcp;
  const float c = fmaf(fmaf(-q, d, x), rcp, q);
  return __builtin_isfinite(q) ? c : q;
}

template <int kDtype>
__device__ __forceinline__ float logit_at(const void* logits, int64_t at) {
  if (kDtype == TM_DTYPE_F32) return reinterpret_cast<const float*>(logits)[at];
  return tm_bf16_to_f32(reinterpret_cast<const uint16_t*>(logits)[at]);
}


// ----------------------------------------------- sampling, in registers --
// For V <= kSampThreads * R: thread t owns residual entries
// [t * R, t * R + R) in registers, so a row pass issues every load of the
// thread at once instead of one dependent load per loop trip, and the bonus
// scan is a shuffle scan.  Entries at or past V hold 0 (-inf as logits).
// Reductions are in a fixed order: the thread's entries in index order, then
// a butterfly over the wave, then the 16 wave values in wave order.
struct SampRegShared {
  float red[2][kSampWaves];  // alternating buffers: one barrier per reduction
  int ridx[2][kSampWaves];   // the argmax indices beside red
  int flag;
};

// Trees up to kSampStage nodes are staged in LDS before the walk, together
// with the one draft probability each child's accept test reads,
// q[c][tokens[c]], gathered for all nodes at once; the walk's per-child reads
// are then LDS reads.  Larger trees are read from global memory.
constexpr int kSampStage = 2048;

struct SampTree {
  int tok[kSampStage];          // tokens[c], -1 outside [0, V)
  int child_start[kSampStage];
  int child_count[kSampStage];
  int child_list[kSampStage];
  float u[kSampStage];          // uniforms[c]
  float qtok[kSampStage];       // q[c][tokens[c]], 0 outside [0, V)
};

__device__ __forceinline__ void stage_tree(SampTree& s, int N, int V,
                                           const int64_t* __restrict__ tokens,
                                           const int32_t* __restrict__ child_start,
                                           const int32_t* __restrict__ child_count,
                                           const int32_t* __restrict__ child_list,
                                           int num_edges, const float* __restrict__ uniforms,
                                           const float* __restrict__ q, int64_t q_stride) {
  const int nlist = num_edges;
  for (int i = threadIdx.x; i < N; i += kSampThreads) {
    const int64_t t = tokens[i];
    const bool in = t >= 0 && t < V;
    s.tok[i] = in ? (int)t : -1;
    s.child_start[i] = child_start[i];
    s.child_count[i] = child_count[i];
    s.u[i] = uniforms[i];
    s.qtok[i] = in ? q[(int64_t)i * q_stride + t] : 0.0f;
  }
  for (int i = threadIdx.x; i < nlist; i += kSampThreads) s.child_list[i] = child_list[i];
  __syncthreads();
}

// Child list entry `at` (staged or from global memory): the child's slot c
// and its token (-1 outside [0, V)).
// A child index outside [0, N) is returned as c = -1, which is never accepted.
__device__ __forceinline__ int2 sample_child(bool staged, const SampTree& s, int at, int N, int V,
                                             const int64_t* __restrict__ tokens,
                                             const int32_t* __restrict__ child_list) {
  const int c = staged ? s.child_list[at] : child_list[at];
  if (c < 0 || c >= N) return make_int2(-1, -1);
  if (staged) return make_int2(c, s.tok[c]);
  const int64_t t = tokens[c];
  return make_int2(c, (t >= 0 && t < V) ? (int)t : -1);
}

// The accept test of child c with in-vocabulary token tok, given the
// residual's entry rv: u_c < min(rv / max(q_c[tok], 1e-20), 1).
__device__ __forceinline__ int sample_accept(bool staged, const SampTree& s, int c, int tok,
                                             float rv, const float* __restrict__ uniforms,
                                             const float* __restrict__ q, int64_t q_stride) {
  const float u = staged ? s.u[c] : uniforms[c];
  const float qt = staged ? s.qtok[c] : q[(int64_t)c * q_stride + tok];
  const float ratio = clamp_max_nan(rv / clamp_min_nan(qt, 1e-20f), 1.0f);
  return u < ratio ? 1 : 0;
}

__device__ __forceinline__ float block_reduce_fast(float v, bool is_max, SampRegShared& sh,
                                                   int& phase) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (is_max) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max_nan(v, __shfl_xor(v, off));
  } else {
    v = wave_sum(v);
  }
  float* buf = sh.red[phase];
  phase ^= 1;
  if (lane == 0) buf[wave] = v;
  __syncthreads();
  float r = buf[0];
#pragma unroll
  for (int w = 1; w < kSampWaves; ++w) r = is_max ? max_nan(r, buf[w]) : r + buf[w];
  return r;
}

// x[i] = element lo + i of a row of `kDtype` (fill beyond V); 16-byte loads
// when the row is aligned and the thread's range lies inside [0, V).
template <int kDtype, int R>
__device__ __forceinline__ void load_range(const void* row, int lo, int V, bool vec, float fill,
                                           float (&x)[R]) {
  if (vec && lo + R <= V) {
    if (kDtype == TM_DTYPE_F32) {
      const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(row) + lo);
#pragma unroll
      for (int j = 0; j < R / 4; ++j) {
        const float4 f = p[j];
        x[4 * j] = f.x;
        x[4 * j + 1] = f.y;
        x[4 * j + 2] = f.z;
        x[4 * j + 3] = f.w;
      }
    } else {
      const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(row) + lo);
#pragma unroll
      for (int j = 0; j < R / 8; ++j) {
        const uint4 u = p[j];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          x[8 * j + 2 * k] = __uint_as_float(w[k] << 16);
          x[8 * j + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i)
      x[i] = (lo + i < V) ? logit_at<kDtype>(row, lo + i) : fill;
  }
}

template <int R>
__device__ __forceinline__ void store_range(float* dst, int lo, int V, bool vec,
                                            const float (&x)[R]) {
  if (vec && lo + R <= V) {
    float4* p = reinterpret_cast<float4*>(dst + lo);
#pragma unroll
    for (int j = 0; j < R / 4; ++j)
      p[j] = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i)
      if (lo + i < V) dst[lo + i] = x[i];
  }
}

// (v, i) precedes (w, j) in torch.argmax's order: NaN above every number,
// then the larger value; among equal values (or two NaNs) the lower index.
__device__ __forceinline__ bool argmax_before(float v, int i, float w, int j) {
  const bool vn = v != v, wn = w != w;
  if (vn != wn) return vn;
  if (vn || v == w) return i < j;
  return v > w;
}

// Workgroup argmax of (v, idx) pairs in argmax_before's order (v >= 0, NaN,
// or -1 for "none").  Returns the winner to every thread.
__device__ __forceinline__ int block_argmax(float v, int idx, SampRegShared& sh, int& phase) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(idx, off);
    if (argmax_before(ov, oi, v, idx)) {
      v = ov;
      idx = oi;
    }
  }
  float* buf = sh.red[phase];
  int* ibuf = sh.ridx[phase];
  phase ^= 1;
  if (lane == 0) {
    buf[wave] = v;
    ibuf[wave] = idx;
  }
  __syncthreads();
  float bv = buf[0];
  int bi = ibuf[0];
#pragma unroll
  for (int w = 1; w < kSampWaves; ++w)
    if (argmax_before(buf[w], ibuf[w], bv, bi)) {
      bv = buf[w];
      bi = ibuf[w];
    }
  return bi;
}

// One thread's part of the exponential race over entries lo .. lo + R - 1
// (x: residual entries, e: the exponentials; entries at or past V skipped):
// the first of its largest x[i] / e[i] (IEEE division, as torch's div).  A
// NaN ratio never wins here; the residual is NaN-free or all NaN (a NaN logit
// or draft entry reaches every entry through the softmax maximum or the
// renormalising sum), and an all-NaN race finds nothing and is reported as
// index 0, torch.argmax's first NaN (bonus_token).  Only an infinite draft
// probability, not a probability, could leave a partly NaN residual, whose
// NaN entries this race skips where torch.argmax would take the first.
template <int R>
__device__ __forceinline__ void race_chunk(const float (&x)[R], const float (&e)[R], int lo,
                                           int V, float& best, int& at) {
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (lo + i < V) {
      const float t = x[i] / e[i];
      if (t > best) {  // indices ascend: ties keep the first
        best = t;
        at = lo + i;
      }
    }
  }
}

template <int kDtype, int R>
__global__ void __launch_bounds__(kSampThreads)
tm_sample_walk_reg_kernel(const void* __restrict__ logits, int N, int V, int64_t row_stride,
                          int vec_logits, const float* __restrict__ q, int64_t q_stride,
                          int vec_q, const int64_t* __restrict__ tokens,
                          const int32_t* __restrict__ child_start,
                          const int32_t* __restrict__ child_count,
                          const int32_t* __restrict__ child_list, int num_edges,
                          const float* __restrict__ uniforms,
                          const float* __restrict__ bonus_exp, int vec_e, float temperature,
                          float* __restrict__ res, int vec_res,
                          int64_t* __restrict__ accepted_slots,
                          int64_t* __restrict__ accepted_tokens, int64_t* __restrict__ result) {
  __shared__ SampRegShared sh;
  __shared__ SampTree tree;
  const int tid = threadIdx.x;
  const int lo = tid * R;
  const bool staged = N <= kSampStage && num_edges <= kSampStage;
  if (staged)
    stage_tree(tree, N, V, tokens, child_start, child_count, child_list, num_edges, uniforms, q,
               q_stride);
  int phase = 0;
  const float rtemp = 1.0f / temperature;
  const bool unit_t = temperature == 1.0f;
  int node = 0;
  int count = 0;
  float r[R];
  for (;;) {
    // r = softmax(logits[node] / temperature)
    const char* row = reinterpret_cast<const char*>(logits) +
                      (int64_t)node * row_stride * (kDtype == TM_DTYPE_F32 ? 4 : 2);
    load_range<kDtype, R>(row, lo, V, vec_logits != 0, -INFINITY, r);
    float m = -INFINITY;
    if (unit_t) {  // x / 1 = x: no division at temperature 1
#pragma unroll
      for (int i = 0; i < R; ++i) m = max_nan(m, r[i]);
    } else {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        r[i] = div_by(r[i], temperature, rtemp);
        m = max_nan(m, r[i]);
      }
    }
    m = block_reduce_fast(m, true, sh, phase);
    const float ml = m * kLog2e;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      r[i] = exp_soft(r[i], ml);
      s = s + r[i];
    }
    // the normalisations multiply by a reciprocal (within an ulp of dividing)
    const float rs = 1.0f / block_reduce_fast(s, false, sh, phase);
#pragma unroll
    for (int i = 0; i < R; ++i) r[i] = r[i] * rs;

    const int st = staged ? tree.child_start[node] : child_start[node];
    const int cnt = edge_count(st, staged ? tree.child_count[node] : child_count[node],
                               num_edges);
    int taken = -1, taken_tok = -1;
    for (int j = 0; j < cnt; ++j) {
      const int2 ct = sample_child(staged, tree, st + j, N, V, tokens, child_list);
      const int c = ct.x, tok = ct.y;
      if (c < 0) continue;
      // the owner of entry tok decides; tid 0 answers for an out-of-vocabulary token
      if (tok >= 0 ? tok / R == tid : tid == 0) {
        int ok = 0;
        if (tok >= 0) {
          float rv = 0.0f;
#pragma unroll
          for (int i = 0; i < R; ++i) rv = (lo + i == tok) ? r[i] : rv;
          ok = sample_accept(staged, tree, c, tok, rv, uniforms, q, q_stride);
        }
        sh.flag = ok;
      }
      __syncthreads();
      if (sh.flag) {
        taken = c;
        taken_tok = tok;
        break;
      }
      // rejected: r = max(r - q_c, 0) / sum (the reduction's barrier also
      // orders this read of sh.flag before the next write); q_c is read in
      // blocks of at most 16 entries, which bounds the registers live beside r
      constexpr int kQB = R < 16 ? R : 16;
      float part = 0.0f;
#pragma unroll
      for (int b = 0; b < R; b += kQB) {
        float qc[kQB];
        load_range<TM_DTYPE_F32, kQB>(q + (int64_t)c * q_stride, lo + b, V, vec_q != 0, 0.0f,
                                      qc);
#pragma unroll
        for (int i = 0; i < kQB; ++i) {
          r[b + i] = clamp_min_nan(r[b + i] - qc[i], 0.0f);
          part = part + r[b + i];
        }
      }
      const float rtot = 1.0f / clamp_min_nan(block_reduce_fast(part, false, sh, phase), 1e-20f);
#pragma unroll
      for (int i = 0; i < R; ++i) r[i] = r[i] * rtot;
    }
    if (taken >= 0 && count < N) {
      if (tid == 0) {
        accepted_slots[count] = taken;
        accepted_tokens[count] = taken_tok;
      }
      ++count;
      node = taken;
      continue;
    }
    break;
  }

  // bonus: the exponential race, argmax_j r[j] / e[j], first maximum
  float e[R];
  load_range<TM_DTYPE_F32, R>(bonus_exp, lo, V, vec_e != 0, 1.0f, e);
  float best = -1.0f;
  int at = INT_MAX;
  race_chunk<R>(r, e, lo, V, best, at);
  const int won = block_argmax(best, at, sh, phase);
  const int bonus = won == INT_MAX ? 0 : won;  // an all-NaN race: torch.argmax's index 0
  if (tid == 0) {
    result[0] = bonus;
    result[1] = count;
    result[2] = node;
  }
  store_range<R>(res, lo, V, vec_res != 0, r);
  for (int i = count + tid; i < N; i += kSampThreads) {
    accepted_slots[i] = -1;
    accepted_tokens[i] = -1;
  }
}

// ------------------------------------------------- sampling, in tiles --
// For V > kSampRegMax: the residual lives in `res` and every pass walks the
// row in tiles of kSampTile entries; thread t owns entries
// [tile * kSampTile + t * kSampTR, + kSampTR) of every tile, so it issues a
// tile's loads at once and only ever reads back residual entries it wrote
// itself.  Sums accumulate over the thread's entries tile by tile, then as in
// the register kernel; the bonus race runs over the tiles in order.
constexpr int kSampTR = 32;
constexpr int kSampTile = kSampThreads * kSampTR;
constexpr int kSampRegMax = kSampTile;          // V up to this: the register kernel
constexpr int kSampMaxTiles = 1024;             // bounds V (2^25)
constexpr int64_t kSampMaxV = (int64_t)kSampMaxTiles * kSampTile;

template <int kDtype>
__global__ void __launch_bounds__(kSampThreads)
tm_sample_walk_tiled_kernel(const void* __restrict__ logits, int N, int V, int64_t row_stride,
                            int vec_logits, const float* __restrict__ q, int64_t q_stride,
                            int vec_q, const int64_t* __restrict__ tokens,
                            const int32_t* __restrict__ child_start,
                            const int32_t* __restrict__ child_count,
                            const int32_t* __restrict__ child_list, int num_edges,
                            const float* __restrict__ uniforms,
                            const float* __restrict__ bonus_exp, int vec_e, float temperature,
                            float* __restrict__ res, int vec_res,
                            int64_t* __restrict__ accepted_slots,
                            int64_t* __restrict__ accepted_tokens,
                            int64_t* __restrict__ result) {
  __shared__ SampRegShared sh;
  __shared__ SampTree tree;
  const int tid = threadIdx.x;
  const int tiles = (V + kSampTile - 1) / kSampTile;
  const bool vl = vec_logits != 0, vq = vec_q != 0, vr = vec_res != 0;
  const bool staged = N <= kSampStage && num_edges <= kSampStage;
  if (staged)
    stage_tree(tree, N, V, tokens, child_start, child_count, child_list, num_edges, uniforms, q,
               q_stride);
  const float rtemp = 1.0f / temperature;
  const bool unit_t = temperature == 1.0f;
  int phase = 0;
  int node = 0;
  int count = 0;
  for (;;) {
    // res = softmax(logits[node] / temperature): max, sum, then the entries
    const char* row = reinterpret_cast<const char*>(logits) +
                      (int64_t)node * row_stride * (kDtype == TM_DTYPE_F32 ? 4 : 2);
    float m = -INFINITY;
    for (int tl = 0; tl < tiles; ++tl) {
      float x[kSampTR];
      load_range<kDtype, kSampTR>(row, tl * kSampTile + tid * kSampTR, V, vl, -INFINITY, x);
#pragma unroll
      for (int i = 0; i < kSampTR; ++i) m = max_nan(m, x[i]);
    }
    // max(x / T) = max(x) / T: correctly rounded division by T > 0 is monotone
    m = block_reduce_fast(m, true, sh, phase);
    if (!unit_t) m = div_by(m, temperature, rtemp);
    const float ml = m * kLog2e;
    // the exponentials go to res, then one pass scales them by 1 / sum
    float s = 0.0f;
    for (int tl = 0; tl < tiles; ++tl) {
      const int lo = tl * kSampTile + tid * kSampTR;
      float x[kSampTR];
      load_range<kDtype, kSampTR>(row, lo, V, vl, -INFINITY, x);
      if (unit_t) {
#pragma unroll
        for (int i = 0; i < kSampTR; ++i) {
          x[i] = exp_soft(x[i], ml);
          s = s + x[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < kSampTR; ++i) {
          x[i] = exp_soft(div_by(x[i], temperature, rtemp), ml);
          s = s + x[i];
        }
      }
      store_range<kSampTR>(res, lo, V, vr, x);
    }
    const float rs = 1.0f / block_reduce_fast(s, false, sh, phase);
    for (int tl = 0; tl < tiles; ++tl) {
      const int lo = tl * kSampTile + tid * kSampTR;
      float x[kSampTR];
      load_range<TM_DTYPE_F32, kSampTR>(res, lo, V, vr, 0.0f, x);
#pragma unroll
      for (int i = 0; i < kSampTR; ++i) x[i] = x[i] * rs;
      store_range<kSampTR>(res, lo, V, vr, x);
    }

    const int st = staged ? tree.child_start[node] : child_start[node];
    const int cnt = edge_count(st, staged ? tree.child_count[node] : child_count[node],
                               num_edges);
    int taken = -1, taken_tok = -1;
    for (int j = 0; j < cnt; ++j) {
      const int2 ct = sample_child(staged, tree, st + j, N, V, tokens, child_list);
      const int c = ct.x, tok = ct.y;
      if (c < 0) continue;
      // the thread that wrote res[tok] decides; tid 0 for an out-of-vocabulary token
      if (tok >= 0 ? (tok % kSampTile) / kSampTR == tid : tid == 0) {
        int ok = 0;
        if (tok >= 0) ok = sample_accept(staged, tree, c, tok, res[tok], uniforms, q, q_stride);
        sh.flag = ok;
      }
      __syncthreads();
      if (sh.flag) {
        taken = c;
        taken_tok = tok;
        break;
      }
      const float* qrow = q + (int64_t)c * q_stride;
      float part = 0.0f;
      for (int tl = 0; tl < tiles; ++tl) {
        const int lo = tl * kSampTile + tid * kSampTR;
        float x[kSampTR], qc[kSampTR];
        load_range<TM_DTYPE_F32, kSampTR>(res, lo, V, vr, 0.0f, x);
        load_range<TM_DTYPE_F32, kSampTR>(qrow, lo, V, vq, 0.0f, qc);
#pragma unroll
        for (int i = 0; i < kSampTR; ++i) {
          x[i] = clamp_min_nan(x[i] - qc[i], 0.0f);
          part = part + x[i];
        }
        store_range<kSampTR>(res, lo, V, vr, x);
      }
      const float rtot = 1.0f / clamp_min_nan(block_reduce_fast(part, false, sh, phase), 1e-20f);
      for (int tl = 0; tl < tiles; ++tl) {
        const int lo = tl * kSampTile + tid * kSampTR;
        float x[kSampTR];
        load_range<TM_DTYPE_F32, kSampTR>(res, lo, V, vr, 0.0f, x);
#pragma unroll
        for (int i = 0; i < kSampTR; ++i) x[i] = x[i] * rtot;
        store_range<kSampTR>(res, lo, V, vr, x);
      }
    }
    if (taken >= 0 && count < N) {
      if (tid == 0) {
        accepted_slots[count] = taken;
        accepted_tokens[count] = taken_tok;
      }
      ++count;
      node = taken;
      continue;
    }
    break;
  }

  // bonus: the exponential race over the tiles in order, argmax_j
  // res[j] / e[j], first maximum (each thread's entries in index order)
  float best = -1.0f;
  int at = INT_MAX;
  for (int tl = 0; tl < tiles; ++tl) {
    const int lo = tl * kSampTile + tid * kSampTR;
    float x[kSampTR], e[kSampTR];
    load_range<TM_DTYPE_F32, kSampTR>(res, lo, V, vr, 0.0f, x);
    load_range<TM_DTYPE_F32, kSampTR>(bonus_exp, lo, V, vec_e != 0, 1.0f, e);
    race_chunk<kSampTR>(x, e, lo, V, best, at);
  }
  const int won = block_argmax(best, at, sh, phase);
  const int bonus = won == INT_MAX ? 0 : won;  // an all-NaN race: torch.argmax's index 0
  if (tid == 0) {
    result[0] = bonus;
    result[1] = count;
    result[2] = node;
  }
  for (int i = count + tid; i < N; i += kSampThreads) {
    accepted_slots[i] = -1;
    accepted_tokens[i] = -1;
  }
}

// ---------------------------------------------------- softmax argmax --
// Greedy verification with a repetition penalty takes the argmax of the
// penalised rows' softmax, stored in the logits' dtype (reference
// `_postprocess_softmax_kernel` at temperature 1, then `_argmax_kernel` over
// the probabilities, op4_commit.py:207-214), not of the logits: values whose
// rounded probabilities are equal tie, and the first index wins.  With
// e_i = exp(x_i - max) and s = sum_i e_i, p_i = round(e_i / s) in fp32 (fp32
// rows) or bf16 (bf16 rows).  exp is monotone and e = 1 at the maximum, so the
// argmax is the first i with round(e_i / s) == round(1 / s).  One workgroup per
// row: the maximum; the sum (thread-strided partials in index order, a xor
// butterfly per wave, then the waves in order); the first matching index.  The
// row's (round(1 / s), index) goes to partial[row] for tm_walk_kernel (one part
// per row).  A row of -inf gives index 0.
constexpr int kSmThreads = 256;

template <int kDtype>
__device__ __forceinline__ float round_prob(float p) {
  if (kDtype == TM_DTYPE_F32) return p;
  return tm_bf16_to_f32(tm_f32_to_bf16(p));
}

template <int kDtype>
__global__ void __launch_bounds__(kSmThreads)
tm_softmax_argmax_kernel(const void* __restrict__ logits, int V, int64_t row_stride,
                         Partial* __restrict__ partial) {
  __shared__ float s_red[kSmThreads / 64];
  __shared__ int s_idx[kSmThreads / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t base = (int64_t)row * row_stride;
  float m = -INFINITY;
  for (int i = tid; i < V; i += kSmThreads) m = fmaxf(m, logit_at<kDtype>(logits, base + i));
  m = wave_max(m);
  if (lane == 0) s_red[wave] = m;
  __syncthreads();
  m = s_red[0];
#pragma unroll
  for (int w = 1; w < kSmThreads / 64; ++w) m = fmaxf(m, s_red[w]);
  __syncthreads();
  float s = 0.0f;
  for (int i = tid; i < V; i += kSmThreads)
    s = s + tm_expf_det(logit_at<kDtype>(logits, base + i) - m);
  s = wave_sum(s);
  if (lane == 0) s_red[wave] = s;
  __syncthreads();
  s = s_red[0];
#pragma unroll
  for (int w = 1; w < kSmThreads / 64; ++w) s = s + s_red[w];
  const float top = round_prob<kDtype>(1.0f / s);
  int first = INT_MAX;
  for (int i = tid; i < V; i += kSmThreads) {
    if (round_prob<kDtype>(tm_expf_det(logit_at<kDtype>(logits, base + i) - m) / s) == top) {
      first = i;
      break;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) first = min(first, __shfl_xor(first, off));
  if (lane == 0) s_idx[wave] = first;
  __syncthreads();
  if (tid == 0) {
    int f = s_idx[0];
#pragma unroll
    for (int w = 1; w < kSmThreads / 64; ++w) f = min(f, s_idx[w]);
    partial[row] = Partial{top, f == INT_MAX ? 0 : f};
  }
}

template <int kDtype>
void launch_sample_walk(const void* logits, int N, int V, int64_t row_stride, const float* q,
                        int64_t q_stride, const int64_t* tokens, const int32_t* child_start,
                        const int32_t* child_count, const int32_t* child_list, int num_edges,
                        const float* uniforms, const float* bonus_exp, float temperature,
                        float* res, int64_t* accepted_slots, int64_t* accepted_tokens,
                        int64_t* result, hipStream_t stream) {
  const int64_t elem = kDtype == TM_DTYPE_F32 ? 4 : 2;
  const int vl = ((uintptr_t)logits % 16 == 0 && (row_stride * elem) % 16 == 0) ? 1 : 0;
  const int vq = ((uintptr_t)q % 16 == 0 && q_stride % 4 == 0) ? 1 : 0;
  const int vr = ((uintptr_t)res % 16 == 0) ? 1 : 0;
  const int ve = ((uintptr_t)bonus_exp % 16 == 0) ? 1 : 0;
#define TM_SAMPLE_REG(R)                                                                       \
  hipLaunchKernelGGL((tm_sample_walk_reg_kernel<kDtype, R>), dim3(1), dim3(kSampThreads), 0,   \
                     stream, logits, N, V, row_stride, vl, q, q_stride, vq, tokens,           \
                     child_start, child_count, child_list, num_edges, uniforms, bonus_exp, ve,    \
                     temperature, res,                                                        \
                     vr, accepted_slots, accepted_tokens, result)
  if (V <= kSampThreads * 8) {
    TM_SAMPLE_REG(8);
  } else if (V <= kSampThreads * 16) {
    TM_SAMPLE_REG(16);
  } else if (V <= kSampRegMax) {
    static_assert(kSampRegMax == kSampThreads * 32, "register kernel sizes");
    TM_SAMPLE_REG(32);
  } else {
    hipLaunchKernelGGL(tm_sample_walk_tiled_kernel<kDtype>, dim3(1), dim3(kSampThreads), 0,
                       stream, logits, N, V, row_stride, vl, q, q_stride, vq, tokens,
                       child_start, child_count, child_list, num_edges, uniforms, bonus_exp, ve,
                       temperature, res, vr, accepted_slots, accepted_tokens, result);
  }
#undef TM_SAMPLE_REG
}

}  // namespace

namespace {

// Shared by tm_op4_argmax_walk (caller's workspace) and
// tm_op4_argmax_walk_noalloc (the library's static scratch).
int argmax_walk(const void* logits, int dtype, int64_t N, int64_t V, int64_t row_stride,
                const int64_t* tokens, const int32_t* child_start, const int32_t* child_count,
                const int32_t* child_list, int64_t num_edges, int64_t max_depth,
                int softmax_argmax, int32_t* argmax, int64_t* accepted_slots,
                int64_t* accepted_tokens, int64_t* result, Partial* partial,
                hipStream_t stream) {
  if (softmax_argmax) {
    if (dtype == TM_DTYPE_F32) {
      hipLaunchKernelGGL(tm_softmax_argmax_kernel<TM_DTYPE_F32>, dim3((unsigned)N),
                         dim3(kSmThreads), 0, stream, logits, (int)V, row_stride, partial);
    } else {
      hipLaunchKernelGGL(tm_softmax_argmax_kernel<TM_DTYPE_BF16>, dim3((unsigned)N),
                         dim3(kSmThreads), 0, stream, logits, (int)V, row_stride, partial);
    }
    TM_HIP_CHECK_LAUNCH();
    hipLaunchKernelGGL(tm_walk_kernel, dim3(1), dim3(kWalkThreads), 0, stream, partial, 1,
                       (int)N, tokens, child_start, child_count, child_list, (int)num_edges,
                       (int)max_depth, argmax, accepted_slots, accepted_tokens, result);
    TM_HIP_CHECK_LAUNCH();
    return TM_OK;
  }
  const int64_t elem = (dtype == TM_DTYPE_F32) ? 4 : 2;
  const int64_t width = 16 / elem;  // elements per 16-byte vector
  // rows are split into `parts` ranges of `per_part` elements (a multiple of
  // the vector width), about kChunkBytes each, at most TM_OP4_MAX_PARTS
  int64_t per_part = (kChunkBytes / elem);
  int64_t parts = (V + per_part - 1) / per_part;
  if (parts > TM_OP4_MAX_PARTS) {
    parts = TM_OP4_MAX_PARTS;
    per_part = ((V + parts - 1) / parts + width - 1) / width * width;
    parts = (V + per_part - 1) / per_part;
  }
  const int vec_ok = (((uintptr_t)logits % 16) == 0 && ((row_stride * elem) % 16) == 0) ? 1 : 0;
  const dim3 grid((unsigned)parts, (unsigned)N);
  if (dtype == TM_DTYPE_F32) {
    hipLaunchKernelGGL(tm_argmax_part_kernel<TM_DTYPE_F32>, grid, dim3(kArgThreads), 0, stream,
                       logits, (int)V, row_stride, (int)per_part, (int)parts, vec_ok, partial);
  } else {
    hipLaunchKernelGGL(tm_argmax_part_kernel<TM_DTYPE_BF16>, grid, dim3(kArgThreads), 0, stream,
                       logits, (int)V, row_stride, (int)per_part, (int)parts, vec_ok, partial);
  }
  TM_HIP_CHECK_LAUNCH();
  hipLaunchKernelGGL(tm_walk_kernel, dim3(1), dim3(kWalkThreads), 0, stream, partial,
                     (int)parts, (int)N, tokens, child_start, child_count, child_list,
                     (int)num_edges, (int)max_depth, argmax, accepted_slots, accepted_tokens,
                     result);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

int check_argmax_walk(int dtype, int64_t N, int64_t V, int64_t row_stride, int64_t num_edges,
                      int64_t max_depth, int softmax_argmax) {
  if (N < 1 || N > (1 << 20) || V < 1 || V > (1 << 30) || row_stride < V || max_depth < 0 ||
      num_edges < 0 || num_edges > (1 << 24))
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_F32 && dtype != TM_DTYPE_BF16) return TM_ERR_ARG;
  if (softmax_argmax != 0 && softmax_argmax != 1) return TM_ERR_ARG;
  return TM_OK;
}

}  // namespace

extern "C" int tm_op4_argmax_walk(const void* logits, int dtype, int64_t N, int64_t V,
                                  int64_t row_stride, const int64_t* tokens,
                                  const int32_t* child_start, const int32_t* child_count,
                                  const int32_t* child_list, int64_t num_edges,
                                  int64_t max_depth, int softmax_argmax, int32_t* argmax,
                                  int64_t* accepted_slots, int64_t* accepted_tokens,
                                  int64_t* result, void* workspace, void* stream) {
  const int rc = check_argmax_walk(dtype, N, V, row_stride, num_edges, max_depth, softmax_argmax);
  if (rc) return rc;
  if (((uintptr_t)workspace % 8) != 0) return TM_ERR_ALIGN;
  return argmax_walk(logits, dtype, N, V, row_stride, tokens, child_start, child_count,
                     child_list, num_edges, max_depth, softmax_argmax, argmax, accepted_slots,
                     accepted_tokens, result, reinterpret_cast<Partial*>(workspace),
                     (hipStream_t)stream);
}

// ------------------------------------------------- allocation-free variant --
// tm_op4_argmax_walk_noalloc keeps its row-range partials in this array
// instead of a caller's workspace: 1 MiB of device memory that every GPU the
// library runs on holds until the process ends (each device has its own copy).
// In host code the name is not a device address; the address of a device's
// copy comes from hipGetSymbolAddress, taken once per device (with that device
// current) on its first call and kept in g_scratch_addr.
static __device__ __align__(256) Partial scratch[TM_OP4_NOALLOC_MAX_NODES * TM_OP4_MAX_PARTS];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<Partial*> g_scratch_addr[kMaxDevices];

// Device address of `scratch` on the device that runs `stream` (the current
// device for the null stream).
int scratch_address(hipStream_t stream, Partial** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return TM_ERR_HIP_BASE + (int)e;
  int dev = cur;
  if (stream != nullptr) {
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) return TM_ERR_HIP_BASE + (int)e;
  }
  if (dev < 0 || dev >= kMaxDevices) return TM_ERR_ARG;
  Partial* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p != nullptr) {
    *out = p;
    return TM_OK;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_addr[dev].load(std::memory_order_relaxed);
  if (p == nullptr) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return TM_ERR_HIP_BASE + (int)e;
    void* addr = nullptr;
    e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    const hipError_t back = dev != cur ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess) return TM_ERR_HIP_BASE + (int)e;
    if (back != hipSuccess) return TM_ERR_HIP_BASE + (int)back;
    if (addr == nullptr) return TM_ERR_HIP_BASE + (int)hipErrorInvalidSymbol;
    p = static_cast<Partial*>(addr);
    g_scratch_addr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return TM_OK;
}

}  // namespace

extern "C" int tm_op4_argmax_walk_noalloc(const void* logits, int dtype, int64_t N, int64_t V,
                                          int64_t row_stride, const int64_t* tokens,
                                          const int32_t* child_start,
                                          const int32_t* child_count,
                                          const int32_t* child_list, int64_t num_edges,
                                          int64_t max_depth, int softmax_argmax,
                                          int32_t* argmax, int64_t* accepted_slots,
                                          int64_t* accepted_tokens, int64_t* result,
                                          void* stream) {
  const int rc = check_argmax_walk(dtype, N, V, row_stride, num_edges, max_depth, softmax_argmax);
  if (rc) return rc;
  if (N > TM_OP4_NOALLOC_MAX_NODES) return TM_ERR_SHAPE;
  Partial* partial = nullptr;
  const int src = scratch_address((hipStream_t)stream, &partial);
  if (src) return src;
  // every partial the walk reads is written by this call's first launch, so
  // the array needs no clearing
  return argmax_walk(logits, dtype, N, V, row_stride, tokens, child_start, child_count,
                     child_list, num_edges, max_depth, softmax_argmax, argmax, accepted_slots,
                     accepted_tokens, result, partial, (hipStream_t)stream);
}

extern "C" int tm_op4_rep_penalty(void* logits, int dtype, int64_t N, int64_t V,
                                  int64_t row_stride, const int64_t* prev_tokens,
                                  int64_t num_prev, float penalty, int32_t* table,
                                  int64_t table_size, void* stream) {
  if (N < 1 || N > (1 << 20) || V < 1 || V > (1 << 30) || row_stride < V || num_prev < 1 ||
      num_prev > (1 << 24))
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_F32 && dtype != TM_DTYPE_BF16) return TM_ERR_ARG;
  if (table_size < 2 * num_prev || table_size < kApplySlots ||
      (table_size & (table_size - 1)) != 0 || table_size > (1 << 26))
    return TM_ERR_SHAPE;
  if (!(penalty > 0.0f)) return TM_ERR_ARG;
  if (((uintptr_t)table % 16) != 0) return TM_ERR_ALIGN;
  const hipStream_t s = (hipStream_t)stream;
  const int S = (int)table_size;
  if (S <= kPenLdsSlots) {
    hipLaunchKernelGGL(tm_rep_count_kernel<true>, dim3(1), dim3(kPenThreads), 0, s, prev_tokens,
                       (int)num_prev, (int)V, table, S);
  } else {
    hipLaunchKernelGGL(tm_rep_count_kernel<false>, dim3(1), dim3(kPenThreads), 0, s, prev_tokens,
                       (int)num_prev, (int)V, table, S);
  }
  TM_HIP_CHECK_LAUNCH();
  const dim3 grid((unsigned)N, (unsigned)std::min<int64_t>((S + kApplyBlock - 1) / kApplyBlock,
                                                           4096));
  if (dtype == TM_DTYPE_F32) {
    hipLaunchKernelGGL(tm_rep_apply_kernel<TM_DTYPE_F32>, grid, dim3(kApplyThreads), 0, s,
                       logits, row_stride, table, S, penalty);
  } else {
    hipLaunchKernelGGL(tm_rep_apply_kernel<TM_DTYPE_BF16>, grid, dim3(kApplyThreads), 0, s,
                       logits, row_stride, table, S, penalty);
  }
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op4_sample_walk(const void* logits, int dtype, int64_t N, int64_t V,
                                  int64_t row_stride, const float* draft_probs, int64_t q_stride,
                                  const int64_t* tokens, const int32_t* child_start,
                                  const int32_t* child_count, const int32_t* child_list,
                                  int64_t num_edges, const float* uniforms,
                                  const float* bonus_exp, float temperature, float* residual,
                                  int64_t* accepted_slots, int64_t* accepted_tokens,
                                  int64_t* result, void* stream) {
  if (N < 1 || N > (1 << 20) || V < 1 || V > kSampMaxV || row_stride < V || q_stride < V ||
      num_edges < 0 || num_edges > (1 << 24))
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_F32 && dtype != TM_DTYPE_BF16) return TM_ERR_ARG;
  if (!(temperature > 0.0f)) return TM_ERR_ARG;
  if (dtype == TM_DTYPE_F32) {
    launch_sample_walk<TM_DTYPE_F32>(logits, (int)N, (int)V, row_stride, draft_probs, q_stride,
                                     tokens, child_start, child_count, child_list, (int)num_edges, uniforms,
                                     bonus_exp, temperature, residual, accepted_slots,
                                     accepted_tokens, result, (hipStream_t)stream);
  } else {
    launch_sample_walk<TM_DTYPE_BF16>(logits, (int)N, (int)V, row_stride, draft_probs, q_stride,
                                      tokens, child_start, child_count, child_list, (int)num_edges, uniforms,
                                      bonus_exp, temperature, residual, accepted_slots,
                                      accepted_tokens, result, (hipStream_t)stream);
  }
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op4_kv_commit(void* k, void* v, int64_t elem_bytes, int64_t L,
                                int64_t row_elems, int64_t stride_layer, int64_t stride_page,
                                int64_t stride_slot, int64_t page_size,
                                const int64_t* accepted_slots, const int64_t* result,
                                const int32_t* scratch_pages, int64_t num_scratch_pages,
                                const int32_t* block_table, int64_t num_table_pages,
                                int64_t seq_len, int64_t max_depth, int64_t* host_count,
                                void* stream) {
  if (L < 1 || L > 65535 || row_elems < 1 || page_size < 1 || max_depth < 0 ||
      max_depth > 65534 || num_scratch_pages < 1 || num_table_pages < 1 || seq_len < 0)
    return TM_ERR_SHAPE;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return TM_ERR_ARG;
  if ((seq_len + max_depth) / page_size >= num_table_pages) return TM_ERR_SHAPE;
  const int64_t row_bytes = row_elems * elem_bytes;
  const int64_t sl = stride_layer * elem_bytes, sp = stride_page * elem_bytes,
                ss = stride_slot * elem_bytes;
  const int vec16 = ((row_bytes % 16) == 0 && (sl % 16) == 0 && (sp % 16) == 0 &&
                     (ss % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0)
                        ? 1
                        : 0;
  const dim3 grid((unsigned)L, (unsigned)(max_depth + 1));
  hipLaunchKernelGGL(tm_kv_commit_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (uint8_t*)k, (uint8_t*)v, row_bytes, sl, sp, ss, page_size,
                     accepted_slots, result, scratch_pages, num_scratch_pages, block_table,
                     num_table_pages, seq_len, vec16, host_count);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}
