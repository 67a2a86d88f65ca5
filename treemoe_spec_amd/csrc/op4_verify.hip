// op4 on gfx950: first-occurrence argmax over the vocabulary for every tree
// node (row-chunked over many workgroups), the greedy accept walk from LDS in
// one workgroup, and the paged KV commit of [root] + accepted path.
#include <climits>

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

struct WalkShared {
  int64_t tokens[kStageNodes];
  int argmax[kStageNodes];
  int child_start[kStageNodes];
  int child_count[kStageNodes];
  int child_list[kStageNodes];
  int count;
};

// One workgroup: reduce the row partials to argmax[N], then the greedy walk
// from the root (op4_commit.py:99-131): at each level take the first child,
// in child-list order, whose token equals the node's argmax.  Trees of at
// most kStageNodes nodes are staged in LDS first, so the walk's dependent
// reads are LDS reads; larger trees are walked from global memory.  The walk
// also stops once N nodes are accepted (only a child list with a cycle gets
// there), so accepted_slots is never written past N.
__global__ void __launch_bounds__(kWalkThreads)
tm_walk_kernel(const Partial* __restrict__ partial, int parts, int N,
               const int64_t* __restrict__ tokens, const int32_t* __restrict__ child_start,
               const int32_t* __restrict__ child_count, const int32_t* __restrict__ child_list,
               int max_depth, int32_t* __restrict__ argmax, int64_t* __restrict__ accepted_slots,
               int64_t* __restrict__ accepted_tokens, int64_t* __restrict__ result) {
  __shared__ WalkShared sh;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const bool staged = N <= kStageNodes;
  const int nlist = N > 1 ? N - 1 : 1;
  if (staged) {
    for (int i = tid; i < N; i += kWalkThreads) {
      sh.tokens[i] = tokens[i];
      sh.child_start[i] = child_start[i];
      sh.child_count[i] = child_count[i];
    }
    for (int i = tid; i < nlist; i += kWalkThreads) sh.child_list[i] = child_list[i];
  }
  for (int row = wave; row < N; row += kWalkThreads / 64) {
    Best b{-INFINITY, 0x7fffffff};
    for (int p = lane; p < parts; p += 64) {
      const Partial q = partial[(size_t)row * parts + p];
      b.offer(q.v, q.i);
    }
    b = wave_best(b);
    if (lane == 0) {
      argmax[row] = b.i;
      if (staged) sh.argmax[row] = b.i;
    }
  }
  __syncthreads();
  const int64_t* tok = staged ? sh.tokens : tokens;
  const int* am = staged ? sh.argmax : argmax;
  const int* cs = staged ? sh.child_start : child_start;
  const int* cc = staged ? sh.child_count : child_count;
  const int* cl = staged ? sh.child_list : child_list;
  if (tid == 0) {
    int node = 0;
    int count = 0;
    for (int d = 0; d < max_depth && count < N; ++d) {
      const int64_t target = (int64_t)am[node];
      const int st = cs[node];
      const int cnt = cc[node];
      int acc = -1;
      for (int j = 0; j < cnt; ++j) {
        const int c = cl[st + j];
        if (tok[c] == target) { acc = c; break; }
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
  __syncthreads();
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
                    int64_t seq_len, int vec16) {
  const int layer = blockIdx.x;
  const int j = blockIdx.y;
  const int64_t num = result[1];
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
// applied each time, so only the count of each token matters: one workgroup
// counts the distinct tokens in an open-addressing table (global workspace,
// 2 * S int32 for S = table size, a power of two >= 2 * num_prev), then
// applies each token's count to every row.  Tokens outside [0, V) are skipped.
constexpr int kPenThreads = 1024;

template <int kDtype>
__global__ void __launch_bounds__(kPenThreads)
tm_rep_penalty_kernel(void* __restrict__ logits, int N, int V, int64_t row_stride,
                      const int64_t* __restrict__ prev, int num_prev, float penalty,
                      int32_t* __restrict__ table, int S) {
  int32_t* keys = table;
  int32_t* counts = table + S;
  const int tid = threadIdx.x;
  // every table access is an agent-scope atomic, so the table is coherent at
  // L2 whatever the L1 holds; the barriers order the three phases
  for (int i = tid; i < S; i += kPenThreads) {
    __hip_atomic_store(&keys[i], -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&counts[i], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  for (int i = tid; i < num_prev; i += kPenThreads) {
    const int64_t t = prev[i];
    if (t < 0 || t >= V) continue;
    uint32_t h = ((uint32_t)t * 2654435761u) & (uint32_t)(S - 1);
    for (int probe = 0; probe < S; ++probe) {
      const int prior = atomicCAS(&keys[h], -1, (int)t);
      if (prior == -1 || prior == (int)t) {
        atomicAdd(&counts[h], 1);
        break;
      }
      h = (h + 1) & (uint32_t)(S - 1);
    }
  }
  __syncthreads();
  const int64_t pairs = (int64_t)S * N;
  for (int64_t q = tid; q < pairs; q += kPenThreads) {
    const int slot = (int)(q % S);
    const int row = (int)(q / S);
    const int k = __hip_atomic_load(&counts[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (k == 0) continue;
    const int key = __hip_atomic_load(&keys[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int64_t at = (int64_t)row * row_stride + key;
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

// ---------------------------------------------------------- sampling --
// Tree rejection sampling, reference `tree_verify_ref` sampling branch
// (treemoe/ref/verify_ref.py:60-89), in one workgroup.  At the current node:
// p = softmax(logits[node] / temperature) becomes the residual; children are
// tried in child-list order: child c (token t) is accepted when
// uniforms[c] < min(residual[t] / max(q_c[t], 1e-20), 1), q_c = draft_probs[c];
// otherwise residual = max(residual - q_c, 0) / max(sum, 1e-20).  An accepted
// child becomes the node; when every child is rejected (or at a leaf) the
// bonus token is the inverse-CDF sample of the residual at bonus_u.  Every
// reduction is in a fixed order, so the result is deterministic.
constexpr int kSampThreads = 1024;
constexpr int kSampWaves = kSampThreads / 64;

struct SampShared {
  float red[kSampWaves];
  float bcast[2];
  int flag;
  int count;
};

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

// Workgroup sum (is_max = false) or max in a fixed order; every thread gets it.
__device__ __forceinline__ float block_reduce(float v, bool is_max, SampShared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = is_max ? wave_max(v) : wave_sum(v);
  if (lane == 0) sh.red[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = sh.red[0];
    for (int w = 1; w < kSampWaves; ++w) r = is_max ? fmaxf(r, sh.red[w]) : r + sh.red[w];
    sh.bcast[0] = r;
  }
  __syncthreads();
  const float r = sh.bcast[0];
  __syncthreads();
  return r;
}

template <int kDtype>
__device__ __forceinline__ float logit_at(const void* logits, int64_t at) {
  if (kDtype == TM_DTYPE_F32) return reinterpret_cast<const float*>(logits)[at];
  return tm_bf16_to_f32(reinterpret_cast<const uint16_t*>(logits)[at]);
}

template <int kDtype>
__global__ void __launch_bounds__(kSampThreads)
tm_sample_walk_kernel(const void* __restrict__ logits, int N, int V, int64_t row_stride,
                      const float* __restrict__ q, int64_t q_stride,
                      const int64_t* __restrict__ tokens, const int32_t* __restrict__ child_start,
                      const int32_t* __restrict__ child_count,
                      const int32_t* __restrict__ child_list, const float* __restrict__ uniforms,
                      const float* __restrict__ bonus_u, float temperature,
                      float* __restrict__ res, int64_t* __restrict__ accepted_slots,
                      int64_t* __restrict__ accepted_tokens, int64_t* __restrict__ result) {
  __shared__ SampShared sh;
  const int tid = threadIdx.x;
  int node = 0;
  int count = 0;
  for (;;) {
    // residual = softmax(logits[node] / temperature)
    const int64_t base = (int64_t)node * row_stride;
    float m = -INFINITY;
    for (int v = tid; v < V; v += kSampThreads)
      m = fmaxf(m, logit_at<kDtype>(logits, base + v) / temperature);
    m = block_reduce(m, true, sh);
    float s = 0.0f;
    for (int v = tid; v < V; v += kSampThreads)
      s = s + tm_expf_det(logit_at<kDtype>(logits, base + v) / temperature - m);
    s = block_reduce(s, false, sh);
    for (int v = tid; v < V; v += kSampThreads)
      res[v] = tm_expf_det(logit_at<kDtype>(logits, base + v) / temperature - m) / s;
    __syncthreads();

    const int st = child_start[node];
    const int cnt = child_count[node];
    int taken = -1;
    for (int j = 0; j < cnt; ++j) {
      const int c = child_list[st + j];
      if (tid == 0) {
        const int64_t tok = tokens[c];
        int ok = 0;
        if (tok >= 0 && tok < V) {
          float ratio = res[tok] / fmaxf(q[(int64_t)c * q_stride + tok], 1e-20f);
          ratio = fminf(ratio, 1.0f);
          ok = uniforms[c] < ratio ? 1 : 0;
        }
        sh.flag = ok;
      }
      __syncthreads();
      const int ok = sh.flag;
      __syncthreads();
      if (ok) {
        taken = c;
        break;
      }
      const float* qc = q + (int64_t)c * q_stride;
      float part = 0.0f;
      for (int v = tid; v < V; v += kSampThreads) {
        const float r = fmaxf(res[v] - qc[v], 0.0f);
        res[v] = r;
        part = part + r;
      }
      const float tot = fmaxf(block_reduce(part, false, sh), 1e-20f);
      for (int v = tid; v < V; v += kSampThreads) res[v] = res[v] / tot;
      __syncthreads();
    }
    if (taken >= 0 && count < N) {
      if (tid == 0) {
        accepted_slots[count] = taken;
        accepted_tokens[count] = tokens[taken];
      }
      ++count;
      node = taken;
      continue;
    }
    break;
  }

  // bonus: smallest j with res[0] + .. + res[j] > bonus_u * total, chunked
  // prefix sums (thread t owns a contiguous chunk; chunk sums scanned in
  // thread order)
  const int cs = (V + kSampThreads - 1) / kSampThreads;
  const int lo = min(V, tid * cs), hi = min(V, lo + cs);
  float csum = 0.0f;
  for (int v = lo; v < hi; ++v) csum = csum + res[v];
  // exclusive scan of chunk sums over the workgroup, in thread order
  __shared__ float s_chunk[kSampThreads];
  s_chunk[tid] = csum;
  __syncthreads();
  if (tid == 0) {
    float run = 0.0f;
    for (int t = 0; t < kSampThreads; ++t) {
      const float c = s_chunk[t];
      s_chunk[t] = run;
      run = run + c;
    }
    sh.bcast[1] = run;
    sh.flag = INT_MAX;
  }
  __syncthreads();
  const float target = bonus_u[0] * sh.bcast[1];
  float run = s_chunk[tid];
  // exactly one chunk satisfies this (the boundaries are the same rounded sums)
  if (run <= target && target < run + csum) {
    int pick = hi - 1;
    for (int v = lo; v < hi; ++v) {
      run = run + res[v];
      if (run > target) {
        pick = v;
        break;
      }
    }
    atomicMin(&sh.flag, pick);
  }
  __syncthreads();
  if (tid == 0) {
    int bonus = sh.flag;
    if (bonus == INT_MAX) {  // target at or past the total: last nonzero entry
      bonus = 0;
      for (int v = V - 1; v >= 0; --v)
        if (res[v] > 0.0f) { bonus = v; break; }
    }
    result[0] = bonus;
    result[1] = count;
    result[2] = node;
    sh.count = count;
  }
  __syncthreads();
  for (int i = sh.count + tid; i < N; i += kSampThreads) {
    accepted_slots[i] = -1;
    accepted_tokens[i] = -1;
  }
}

}  // namespace

extern "C" int tm_op4_argmax_walk(const void* logits, int dtype, int64_t N, int64_t V,
                                  int64_t row_stride, const int64_t* tokens,
                                  const int32_t* child_start, const int32_t* child_count,
                                  const int32_t* child_list, int64_t max_depth,
                                  int32_t* argmax, int64_t* accepted_slots,
                                  int64_t* accepted_tokens, int64_t* result, void* workspace,
                                  void* stream) {
  if (N < 1 || N > (1 << 20) || V < 1 || V > (1 << 30) || row_stride < V || max_depth < 0)
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_F32 && dtype != TM_DTYPE_BF16) return TM_ERR_ARG;
  if (((uintptr_t)workspace % 8) != 0) return TM_ERR_ALIGN;
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
  Partial* partial = reinterpret_cast<Partial*>(workspace);
  const dim3 grid((unsigned)parts, (unsigned)N);
  if (dtype == TM_DTYPE_F32) {
    hipLaunchKernelGGL(tm_argmax_part_kernel<TM_DTYPE_F32>, grid, dim3(kArgThreads), 0,
                       (hipStream_t)stream, logits, (int)V, row_stride, (int)per_part,
                       (int)parts, vec_ok, partial);
  } else {
    hipLaunchKernelGGL(tm_argmax_part_kernel<TM_DTYPE_BF16>, grid, dim3(kArgThreads), 0,
                       (hipStream_t)stream, logits, (int)V, row_stride, (int)per_part,
                       (int)parts, vec_ok, partial);
  }
  TM_HIP_CHECK_LAUNCH();
  hipLaunchKernelGGL(tm_walk_kernel, dim3(1), dim3(kWalkThreads), 0, (hipStream_t)stream,
                     partial, (int)parts, (int)N, tokens, child_start, child_count, child_list,
                     (int)max_depth, argmax, accepted_slots, accepted_tokens, result);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op4_rep_penalty(void* logits, int dtype, int64_t N, int64_t V,
                                  int64_t row_stride, const int64_t* prev_tokens,
                                  int64_t num_prev, float penalty, int32_t* table,
                                  int64_t table_size, void* stream) {
  if (N < 1 || N > (1 << 20) || V < 1 || V > (1 << 30) || row_stride < V || num_prev < 1 ||
      num_prev > (1 << 24))
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_F32 && dtype != TM_DTYPE_BF16) return TM_ERR_ARG;
  if (table_size < 2 * num_prev || (table_size & (table_size - 1)) != 0 || table_size > (1 << 26))
    return TM_ERR_SHAPE;
  if (!(penalty > 0.0f)) return TM_ERR_ARG;
  if (dtype == TM_DTYPE_F32) {
    hipLaunchKernelGGL(tm_rep_penalty_kernel<TM_DTYPE_F32>, dim3(1), dim3(kPenThreads), 0,
                       (hipStream_t)stream, logits, (int)N, (int)V, row_stride, prev_tokens,
                       (int)num_prev, penalty, table, (int)table_size);
  } else {
    hipLaunchKernelGGL(tm_rep_penalty_kernel<TM_DTYPE_BF16>, dim3(1), dim3(kPenThreads), 0,
                       (hipStream_t)stream, logits, (int)N, (int)V, row_stride, prev_tokens,
                       (int)num_prev, penalty, table, (int)table_size);
  }
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op4_sample_walk(const void* logits, int dtype, int64_t N, int64_t V,
                                  int64_t row_stride, const float* draft_probs, int64_t q_stride,
                                  const int64_t* tokens, const int32_t* child_start,
                                  const int32_t* child_count, const int32_t* child_list,
                                  const float* uniforms, const float* bonus_u,
                                  float temperature, float* residual,
                                  int64_t* accepted_slots, int64_t* accepted_tokens,
                                  int64_t* result, void* stream) {
  if (N < 1 || N > (1 << 20) || V < 1 || V > (1 << 30) || row_stride < V || q_stride < V)
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_F32 && dtype != TM_DTYPE_BF16) return TM_ERR_ARG;
  if (!(temperature > 0.0f)) return TM_ERR_ARG;
  if (dtype == TM_DTYPE_F32) {
    hipLaunchKernelGGL(tm_sample_walk_kernel<TM_DTYPE_F32>, dim3(1), dim3(kSampThreads), 0,
                       (hipStream_t)stream, logits, (int)N, (int)V, row_stride, draft_probs,
                       q_stride, tokens, child_start, child_count, child_list, uniforms, bonus_u,
                       temperature, residual, accepted_slots, accepted_tokens, result);
  } else {
    hipLaunchKernelGGL(tm_sample_walk_kernel<TM_DTYPE_BF16>, dim3(1), dim3(kSampThreads), 0,
                       (hipStream_t)stream, logits, (int)N, (int)V, row_stride, draft_probs,
                       q_stride, tokens, child_start, child_count, child_list, uniforms, bonus_u,
                       temperature, residual, accepted_slots, accepted_tokens, result);
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
                                int64_t seq_len, int64_t max_depth, void* stream) {
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
                     num_table_pages, seq_len, vec16);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}
