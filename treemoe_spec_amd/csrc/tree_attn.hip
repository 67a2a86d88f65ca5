// Tree attention on gfx950: every node of a draft tree attends to the whole
// committed prefix and to its own ancestors (and itself) in the tree.
//
// Keys 0 .. seq_len-1 are the prefix, read in place from the paged cache
// through the block table (no gather copy); keys seq_len .. seq_len+N-1 are
// the tree's own K/V rows.  Query head h reads KV head h / group.
//
// Work decomposition.  For one KV head the group * N query rows (rows ordered
// head-in-group major, node minor) share every K/V byte, so a workgroup takes
// 128 of those rows (4 waves x 32) against one chunk of keys; the K/V of the
// chunk is staged through LDS 64 keys at a time and each key byte is read from
// HBM once per (KV head, chunk), by the row blocks of that pair, which are
// launched on one XCD (launch indices congruent mod 8) so they share its L2.
// When the keys take several chunks, the prefix and the tree keys are chunked
// separately: the tree chunk's masked stage and its tree-row stores then run
// beside the prefix chunks instead of lengthening one of them.
//
// Per wave and 64-key stage (v_mfma_f32_32x32x16_bf16 throughout):
//   S^T = K Q^T    A = K rows from LDS, B = Q^T held in registers, two 32-key
//                  tiles; lane l gets S^T[key 32t + 8(v/4) + 4(l/32) + v%4]
//                  [query l%32] in accumulator value v;
//   online softmax in base 2, per query (= per lane column), the 2 lanes of a
//                  query combined by one xor shuffle;
//   O^T += V^T P^T B = P^T straight from the S^T registers: the MFMA's k slot j
//                  of k-step (t, m) is mapped to key 32t + 16m + 8(j/4) +
//                  4(l/32) + j%4, the lane's own value 8m + j; A = V^T read with
//                  the same key map from a transposed copy of V in LDS.
// A chunk's normalised O^T (fp16), reference maximum and sum go to a workspace
// (written through L2) and a second kernel combines the chunks in chunk order
// (deterministic); with one chunk the first kernel writes the output itself.
#include <algorithm>
#include <cmath>

#include "tm_common.h"

namespace {

constexpr int kHD = 128;                    // head dim
constexpr int kThreads = 256;               // 4 waves
constexpr int kRows = 128;                  // query rows per workgroup (4 waves x 32)
constexpr int kKeys = 64;                   // keys per LDS stage
constexpr int kKStride = kHD * 2 + 16;      // bytes per K row in LDS (272)
constexpr int kVStride = kKeys * 2 + 8;     // bytes per V^T row in LDS (136)
constexpr int kKBytes = kKeys * kKStride;   // 17,408
constexpr int kVBytes = kHD * kVStride;     // 17,408
constexpr int kStage = kKBytes + kVBytes;   // 34,816
constexpr int kMaxPages = 512;              // block-table entries staged per chunk
constexpr int kMaxNodes = 256;              // tree nodes (mask words per row <= 4)
constexpr int kCUs = 256;                   // MI355X compute units
constexpr int kMaxAutoLen = 16384;          // longest chunk the planner considers

typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

struct AttnParams {
  const uint16_t* q;          // [N, Hq, HD], node stride q_stride (elements)
  const uint16_t* k_tail;     // [N, kvh, HD], node stride tail_stride
  const uint16_t* v_tail;
  uint16_t* k_cache;          // this layer's [pages, page, kvh, HD]
  uint16_t* v_cache;
  const int32_t* block_table;
  const int32_t* scratch_pages;
  const uint64_t* mask_bits;  // [N, mask_words], bit j of row i: node j visible
  uint16_t* out;              // [N, Hq, HD], node stride out_stride
  float* part;                // chunk partials (chunks > 1)
  float* stats;
  int64_t q_stride, tail_stride, out_stride, stride_page, stride_slot;
  int page_shift, seq_len, n, hq, kvh, group, rows, row_blocks, chunks, chunk_len, pairs;
  int pre_chunks, split;      // chunks < pre_chunks tile keys [0, split), the rest [split, end)
  int mask_words, write_tree;
  float scale_log2;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats to packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Stage layout: thread t stages keys 4 * quad + r (r = 0..3) at head-dim
// elements 8 * part .. +7, with quad = (t & 3) + 4 * (t >> 6) and
// part = (t >> 2) & 15; this order keeps both the K row writes and the
// transposed V writes free of LDS bank conflicts.
struct Stage {
  u32x4_t k[4];
  u32x4_t v[4];
};

// The thread's 4 keys key0 .. key0 + 3 (key0 % 4 == 0) share one page
// (page_size >= 4), so one block-table lookup serves them.  A stage that lies
// entirely in the prefix takes the straight path; the chunk's boundary stages
// pick each key's source (cache page, tree row, or zero past the chunk).
__device__ __forceinline__ void load_stage(const AttnParams& p, const int* s_pages, int kb,
                                           int c0, int c1, int64_t head_off, int quad,
                                           Stage& st) {
  const int key0 = kb + 4 * quad;
  const int pre_end = min(c1, p.seq_len);
  const int pidx = key0 < pre_end ? (key0 >> p.page_shift) - (c0 >> p.page_shift) : 0;
  const uint32_t page = (uint32_t)s_pages[pidx];
  const int64_t cbase = (int64_t)((uint64_t)page * (uint64_t)p.stride_page) +
                        (int64_t)(key0 & ((1 << p.page_shift) - 1)) * p.stride_slot + head_off;
  if (kb + kKeys <= pre_end) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t off = cbase + r * p.stride_slot;
      st.k[r] = *reinterpret_cast<const u32x4_t*>(p.k_cache + off);
      st.v[r] = *reinterpret_cast<const u32x4_t*>(p.v_cache + off);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = key0 + r;
      const bool in_pre = key < pre_end;
      const bool in_tail = key >= p.seq_len && key < c1;
      const int node = in_tail ? key - p.seq_len : 0;  // tree row 0 stands in otherwise
      const int64_t off = in_pre ? cbase + r * p.stride_slot
                                 : (int64_t)node * p.tail_stride + head_off;
      const uint16_t* kp = in_pre ? p.k_cache : p.k_tail;
      const uint16_t* vp = in_pre ? p.v_cache : p.v_tail;
      const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(kp + off);
      const u32x4_t vv = *reinterpret_cast<const u32x4_t*>(vp + off);
      const u32x4_t zero = {0u, 0u, 0u, 0u};
      st.k[r] = (in_pre || in_tail) ? kv : zero;
      st.v[r] = (in_pre || in_tail) ? vv : zero;
    }
  }
}

__device__ __forceinline__ void store_stage(uint8_t* buf, int quad, int part, const Stage& st) {
  uint8_t* kl = buf;
  uint8_t* vl = buf + kKBytes;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    *reinterpret_cast<u32x4_t*>(kl + (4 * quad + r) * kKStride + part * 16) = st.k[r];
  // V^T[hd][key]: for head-dim element 8 * part + j, the 4 keys of this quad
  // side by side (8 bytes)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int w = j >> 1;
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    u32x2_t pk;
    pk.x = __builtin_amdgcn_perm(st.v[1][w], st.v[0][w], sel);
    pk.y = __builtin_amdgcn_perm(st.v[3][w], st.v[2][w], sel);
    *reinterpret_cast<u32x2_t*>(vl + (8 * part + j) * kVStride + quad * 8) = pk;
  }
}

// Tree rows among a staged stage's keys (keys seq_len .. c1-1) into the
// scratch pages: tree node j lives in page s_tpages[j / page] at slot j % page.
__device__ __forceinline__ void store_tree_rows(const AttnParams& p, const int* s_tpages, int kb,
                                                int c1, int quad, int64_t head_off,
                                                const Stage& st) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int key = kb + 4 * quad + r;
    if (key >= p.seq_len && key < c1) {
      const int node = key - p.seq_len;
      const int64_t dst = (int64_t)s_tpages[node >> p.page_shift] * p.stride_page +
                          (int64_t)(node & ((1 << p.page_shift) - 1)) * p.stride_slot +
                          head_off;
      *reinterpret_cast<u32x4_t*>(p.k_cache + dst) = st.k[r];
      *reinterpret_cast<u32x4_t*>(p.v_cache + dst) = st.v[r];
    }
  }
}

// Visibility of keys kb .. kb+63 for one query, bit i for key kb + i:
// prefix keys (key < seq_len) visible, tree key seq_len + j visible when bit j
// of the query's mask row mw is set, keys at or past the chunk end c1 hidden.
// d = kb - seq_len (> -64 for a stage that is not all prefix), e = c1 - kb.
__device__ __forceinline__ uint64_t stage_window(const uint64_t mw[4], int d, int e) {
  uint64_t win;
  if (d >= 0) {
    const int w = d >> 6, sh = d & 63;
    uint64_t a = mw[0], b = mw[1];
    if (w == 1) { a = mw[1]; b = mw[2]; }
    if (w == 2) { a = mw[2]; b = mw[3]; }
    if (w >= 3) { a = mw[3]; b = 0; }
    win = sh ? (a >> sh) | (b << (64 - sh)) : a;
  } else {
    const int pre = -d;
    win = pre >= 64 ? ~0ull : (mw[0] << pre) | ((1ull << pre) - 1);
  }
  if (e < 64) win &= (1ull << e) - 1;
  return win;
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

// 32x32x16 bf16 MFMA.  Lane l: A row l%32 and B column l%32, k 8(l/32) .. +7;
// accumulator value v is C[8(v/4) + 4(l/32) + v%4][l%32].
__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// One 64-key stage of one wave against its 32 queries: keys kb .. kb+63 from
// the LDS stage at kl (K rows, then V^T), scores masked on boundary stages,
// the online softmax state (m_run, l_run) and O^T (acc) updated.
__device__ __forceinline__ void attend_stage(const AttnParams& p, const uint8_t* kl, int kb,
                                             int c1, const uint64_t mw[4], int half, int c32,
                                             const u32x4_t qf[kHD / 16], f32x16_t acc[kHD / 32],
                                             float& m_run, float& l_run) {
  const uint8_t* vl = kl + kKBytes;
  // S^T = K Q^T over two 32-key tiles; lane holds keys
  // 32 kt + 8 (v/4) + 4 half + v%4 of query c32 in sc[kt][v]
  // the two key tiles' chains alternate (k-step outer), so consecutive MFMAs
  // do not wait on each other; each tile still sums its k-steps in order
  f32x16_t sc[2];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int v = 0; v < 16; ++v) sc[kt][v] = 0.0f;
#pragma unroll
  for (int ks = 0; ks < kHD / 16; ++ks) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(
          kl + (32 * kt + c32) * kKStride + ks * 32 + half * 16);
      sc[kt] = mfma32(a, qf[ks], sc[kt]);
    }
  }
  // tree and chunk-end masking (boundary stages only); integer and/or, so
  // the visibility is a plain select
  if (!(kb + kKeys <= min(c1, p.seq_len))) {
    // key kb + 32 kt + 8 (v/4) + 4 half + v%4 is bit 8 (v/4) + v%4 of
    // dword kt of the lane's window shifted by 4 half
    const uint64_t win = stage_window(mw, kb - p.seq_len, c1 - kb) >> (4 * half);
    const uint32_t wd[2] = {(uint32_t)win, (uint32_t)(win >> 32)};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t bit = (wd[kt] >> (8 * (v >> 2) + (v & 3))) & 1u;
        sc[kt][v] = bit ? sc[kt][v] : -INFINITY;
      }
    }
  }
  // running max in base 2 (scale > 0 commutes with max); the query's other
  // 32 keys of the stage sit in lane c32 ^ 32
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sc[kt][v]);
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float cand = mx * p.scale_log2;
  // The reference point moves only when the stage maximum exceeds it by more
  // than 2^8 (weights stay <= 256), so the accumulators are rescaled rarely;
  // the final division by the sum taken against the same reference makes
  // this exact in real arithmetic.
  const bool bump = cand > m_run + 8.0f;
  if (__any(bump)) {
    const float m_use = bump ? cand : m_run;
    const float alpha = bump ? exp2f(m_run - m_use) : 1.0f;
#pragma unroll
    for (int ht = 0; ht < kHD / 32; ++ht) acc[ht] *= alpha;
    l_run *= alpha;
    m_run = m_use;
  }
  const float neg_base = m_run == -INFINITY ? 0.0f : -m_run;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float e = __builtin_amdgcn_exp2f(fmaf(sc[kt][v], p.scale_log2, neg_base));
      sc[kt][v] = e;
      l_run += e;
    }
  }
  // O^T += V^T P^T: k-step (kt, m) covers keys 32 kt + 16 m + [0, 16); its
  // k slot j of lane half h is key 32 kt + 16 m + 8 (j/4) + 4 h + j%4, which
  // is the lane's own value sc[kt][8 m + j]
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      u32x4_t b;
      b.x = pack_bf16(sc[kt][8 * m + 0], sc[kt][8 * m + 1]);
      b.y = pack_bf16(sc[kt][8 * m + 2], sc[kt][8 * m + 3]);
      b.z = pack_bf16(sc[kt][8 * m + 4], sc[kt][8 * m + 5]);
      b.w = pack_bf16(sc[kt][8 * m + 6], sc[kt][8 * m + 7]);
#pragma unroll
      for (int ht = 0; ht < kHD / 32; ++ht) {
        const uint8_t* vr = vl + (32 * ht + c32) * kVStride + (32 * kt + 16 * m + 4 * half) * 2;
        const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vr);
        const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vr + 16);
        const u32x4_t a = {lo.x, lo.y, hi.x, hi.y};
        acc[ht] = mfma32(a, b, acc[ht]);
      }
    }
  }
}

// Partials of one (workgroup slot, wave): 16 groups x 64 lanes x 4 fp16 of
// the chunk's normalised O^T, and (m, l) per query (32 float2).
constexpr int kPartHalves = (kHD / 32) * 16 * 64;  // 4096 per wave slot
constexpr int kStatFloats = 64;                      // 32 queries x (m, l)

// At most 256 registers per lane, so two workgroups (2 x 70 KB of LDS) share a
// CU: 218 VGPRs without spills, against 204 VGPRs + 96 AGPRs unbounded; 5 %
// faster at 4096 cached positions, 21 % at 16384 where the grid holds two
// workgroups per CU.
__global__ void __launch_bounds__(kThreads, 2) tm_tree_attn_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t s_buf[2 * kStage];
  __shared__ int s_pages[kMaxPages];
  __shared__ int s_tpages[kMaxNodes / 4];

  const int x8 = blockIdx.x & 7, y = blockIdx.x >> 3;
  const int rb = y % p.row_blocks;
  const int pair = (y / p.row_blocks) * 8 + x8;
  if (pair >= p.pairs) return;
  const int kvhead = pair / p.chunks;
  const int chunk = pair % p.chunks;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, c32 = lane & 31;
  const int s_total = p.seq_len + p.n;
  const bool lead = chunk < p.pre_chunks;
  const int c0 = (lead ? 0 : p.split) + (lead ? chunk : chunk - p.pre_chunks) * p.chunk_len;
  const int c1 = min(c0 + p.chunk_len, lead ? p.split : s_total);
  const int quad = (tid & 3) + 4 * (tid >> 6);
  const int part = (tid >> 2) & 15;
  const int64_t head_off = (int64_t)kvhead * kHD + part * 8;

  // block-table entries of the chunk's prefix keys; the workgroups of row
  // block 0 also store the chunk's tree rows of this KV head into the scratch
  // pages, from the registers that stage them (each tree row lies in exactly
  // one chunk), so they need the scratch page list
  const int pre_end = min(c1, p.seq_len);
  const int npages = pre_end > c0 ? ((pre_end - 1) >> p.page_shift) - (c0 >> p.page_shift) + 1 : 0;
  for (int i = tid; i < npages; i += kThreads)
    s_pages[i] = p.block_table[(c0 >> p.page_shift) + i];
  const bool write_rows = p.write_tree && rb == 0 && c1 > p.seq_len;
  if (write_rows) {
    const int tpages = ((p.n - 1) >> p.page_shift) + 1;
    for (int i = tid; i < tpages; i += kThreads) s_tpages[i] = p.scratch_pages[i];
  }

  // this lane's query (column c32 of the wave's 32): Q^T fragments, mask row
  const int row = rb * kRows + wave * 32 + c32;
  const bool row_ok = row < p.rows;
  const int node = row_ok ? row % p.n : 0;
  const int head = kvhead * p.group + (row_ok ? row / p.n : 0);
  u32x4_t qf[kHD / 16];
  {
    const uint16_t* qrow = p.q + (int64_t)node * p.q_stride + (int64_t)head * kHD + 8 * half;
#pragma unroll
    for (int ks = 0; ks < kHD / 16; ++ks) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(qrow + 16 * ks);
      const u32x4_t zero = {0u, 0u, 0u, 0u};
      qf[ks] = row_ok ? v : zero;
    }
  }
  uint64_t mw[4] = {0, 0, 0, 0};
  if (c1 > p.seq_len) {
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (w < p.mask_words) mw[w] = p.mask_bits[(int64_t)node * p.mask_words + w];
  }
  __syncthreads();  // s_pages

  Stage st;
  load_stage(p, s_pages, c0, c0, c1, head_off, quad, st);
  if (write_rows && c0 + kKeys > p.seq_len)
    store_tree_rows(p, s_tpages, c0, c1, quad, head_off, st);
  store_stage(s_buf, quad, part, st);
  __syncthreads();

  f32x16_t acc[kHD / 32];
#pragma unroll
  for (int ht = 0; ht < kHD / 32; ++ht)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[ht][v] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  // stage s in LDS buffer s & 1; the next stage's loads go out before this
  // stage's MFMAs and land in the other buffer after them
  const int nstage = (c1 - c0 + kKeys - 1) / kKeys;
  for (int s = 0; s < nstage; ++s) {
    const int kb = c0 + s * kKeys, kn = kb + kKeys;
    const bool more = s + 1 < nstage;
    if (more) load_stage(p, s_pages, kn, c0, c1, head_off, quad, st);
    attend_stage(p, s_buf + (s & 1) * kStage, kb, c1, mw, half, c32, qf, acc, m_run, l_run);
    if (more) {
      if (write_rows && kn + kKeys > p.seq_len)
        store_tree_rows(p, s_tpages, kn, c1, quad, head_off, st);
      store_stage(s_buf + ((s + 1) & 1) * kStage, quad, part, st);
      __syncthreads();
    }
  }

  // the two lanes of a query hold partial sums over disjoint keys
  l_run += __shfl_xor(l_run, 32);
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;

  if (p.chunks == 1) {
    if (row_ok) {
      uint16_t* orow = p.out + (int64_t)node * p.out_stride + (int64_t)head * kHD + 4 * half;
#pragma unroll
      for (int ht = 0; ht < kHD / 32; ++ht) {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          u32x2_t o;
          o.x = pack_bf16(acc[ht][4 * gq + 0] * inv, acc[ht][4 * gq + 1] * inv);
          o.y = pack_bf16(acc[ht][4 * gq + 2] * inv, acc[ht][4 * gq + 3] * inv);
          *reinterpret_cast<u32x2_t*>(orow + 32 * ht + 8 * gq) = o;
        }
      }
    }
    return;
  }
  // chunk partial: O^T / l in fp16 (|value| <= max |v|), and (m, l), written
  // through L2 for the combine kernel
  const int64_t slot = ((int64_t)(kvhead * p.row_blocks + rb) * p.chunks + chunk) * 4 + wave;
  _Float16* pp = reinterpret_cast<_Float16*>(p.part) + slot * kPartHalves + lane * 4;
#pragma unroll
  for (int ht = 0; ht < kHD / 32; ++ht) {
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      f16x4_t h;
      h[0] = (_Float16)(acc[ht][4 * gq + 0] * inv);
      h[1] = (_Float16)(acc[ht][4 * gq + 1] * inv);
      h[2] = (_Float16)(acc[ht][4 * gq + 2] * inv);
      h[3] = (_Float16)(acc[ht][4 * gq + 3] * inv);
      tm_store_through(reinterpret_cast<f16x4_t*>(pp + (ht * 4 + gq) * 256), h);
    }
  }
  if (half == 0) {
    f32x2_t st2 = {m_run, l_run};
    tm_store_through(reinterpret_cast<f32x2_t*>(p.stats + slot * kStatFloats + c32 * 2), st2);
  }
}

// One thread per (KV head, row block, wave, 4-value group, lane): merges the
// chunks' normalised partials in chunk order with a running maximum,
//   w_c = l_c 2^(m_c - M),  O = sum_c w_c O_c / sum_c w_c,
// keeping the running sums against the running maximum.  Branch-free, so the
// loads of later chunks can issue early.
__global__ void __launch_bounds__(kThreads) tm_tree_attn_combine_kernel(AttnParams p) {
  const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int lane = (int)(u & 63);
  const int grp = (int)((u >> 6) & 15);       // (ht, gq) = (grp / 4, grp % 4)
  const int64_t kw = u >> 10;                 // (kvhead * row_blocks + rb) * 4 + wave
  const int wave = (int)(kw & 3);
  const int64_t kr = kw >> 2;
  if (kr >= (int64_t)p.kvh * p.row_blocks) return;
  const int c32 = lane & 31, half = lane >> 5;
  float m_run = -INFINITY, w_sum = 0.0f;
  f32x4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int c = 0; c < p.chunks; ++c) {
    const int64_t slot = (kr * p.chunks + c) * 4 + wave;
    const f32x2_t st = *reinterpret_cast<const f32x2_t*>(p.stats + slot * kStatFloats + c32 * 2);
    const f16x4_t hc = *reinterpret_cast<const f16x4_t*>(
        reinterpret_cast<const _Float16*>(p.part) + slot * kPartHalves + grp * 256 + lane * 4);
    const float mn = fmaxf(m_run, st.x);
    const float ref = mn == -INFINITY ? 0.0f : mn;
    const float a = exp2f(m_run - ref);       // 0 while nothing was visible
    const float b = st.y * exp2f(st.x - ref);
    w_sum = w_sum * a + b;
    o[0] = o[0] * a + (float)hc[0] * b;
    o[1] = o[1] * a + (float)hc[1] * b;
    o[2] = o[2] * a + (float)hc[2] * b;
    o[3] = o[3] * a + (float)hc[3] * b;
    m_run = mn;
  }
  const int rb = (int)(kr % p.row_blocks);
  const int kvhead = (int)(kr / p.row_blocks);
  const int row = rb * kRows + wave * 32 + c32;
  if (row >= p.rows) return;
  const int node = row % p.n;
  const int head = kvhead * p.group + row / p.n;
  const float inv = w_sum > 0.0f ? 1.0f / w_sum : 0.0f;
  u32x2_t w;
  w.x = pack_bf16(o[0] * inv, o[1] * inv);
  w.y = pack_bf16(o[2] * inv, o[3] * inv);
  const int ht = grp >> 2, gq = grp & 3;
  *reinterpret_cast<u32x2_t*>(p.out + (int64_t)node * p.out_stride + (int64_t)head * kHD +
                              32 * ht + 8 * gq + 4 * half) = w;
}

// Bit-pack a [N, N] bool mask (row stride in bytes) into [N, words] u64.
__global__ void tm_tree_mask_pack_kernel(const uint8_t* __restrict__ mask, int n,
                                         int64_t stride, int words,
                                         uint64_t* __restrict__ bits) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * words) return;
  const int row = i / words, w = i % words;
  uint64_t b = 0;
  for (int j = 0; j < 64 && w * 64 + j < n; ++j)
    b |= (uint64_t)(mask[(int64_t)row * stride + w * 64 + j] != 0) << j;
  bits[i] = b;
}

struct Plan {
  int64_t row_blocks, chunks, chunk_len, pairs, groups, part_floats, stats_floats;
  int64_t pre_chunks, split;
};

// Chunking of keys 0 .. seq_len+n-1 into chunks of at most len keys.  The
// prefix and the tree keys are chunked separately, so that the tree's masked
// stage (and its tree-row stores) runs beside the prefix chunks rather than
// lengthening one of them; the prefix chunks are evened out to whole stages.
// Work that fits one chunk stays one chunk (no combine).
struct Split {
  int64_t len, pre_chunks, split, chunks;
};

Split split_keys(int64_t seq_len, int64_t n, int64_t len) {
  const int64_t s_total = seq_len + n;
  Split sp;
  sp.len = len;
  const int64_t whole = (s_total + len - 1) / len;
  if (whole > 1 && seq_len > 0) {
    const int64_t pre = (seq_len + len - 1) / len;
    sp.len = ((seq_len + pre - 1) / pre + kKeys - 1) / kKeys * kKeys;
    sp.pre_chunks = (seq_len + sp.len - 1) / sp.len;
    sp.split = seq_len;
    sp.chunks = sp.pre_chunks + (n + sp.len - 1) / sp.len;
  } else {
    sp.pre_chunks = whole;
    sp.split = s_total;
    sp.chunks = whole;
  }
  return sp;
}

int64_t groups_of(int64_t kvh, int64_t row_blocks, int64_t chunks) {
  return (kvh * chunks + 7) / 8 * 8 * row_blocks;
}

// Planner cost of a split, in units of one 64-key stage of one workgroup:
// the longest chunk's stages plus ~2 stages of workgroup prologue and
// epilogue, times 1.6 per extra workgroup a CU has to hold (co-resident
// workgroups share its SIMDs), plus, with several chunks, ~2 stages for the
// combine kernel's launch and 0.1 per chunk it merges (its loop over the
// chunks).  Fitted to measurements on MI355X at 1024 .. 16384 cached positions
// (N = 64, 32 query and 8 KV heads), where it picks the fastest chunk length
// of those tried.
double split_cost(const Split& sp, int64_t s_total, int64_t kvh, int64_t row_blocks) {
  const int64_t keys = sp.chunks > 1 ? sp.len : s_total;
  const double stages = (double)((keys + kKeys - 1) / kKeys);
  const int64_t groups = groups_of(kvh, row_blocks, sp.chunks);
  const double stretch = groups <= kCUs ? 1.0 : 0.8 * (double)((groups + kCUs - 1) / kCUs);
  const double combine = sp.chunks > 1 ? 2.0 + 0.1 * (double)sp.chunks : 0.0;
  return (stages + 2.0) * stretch + combine;
}

int make_plan(int64_t n, int64_t hq, int64_t kvh, int64_t seq_len, int64_t page_size,
              int64_t chunk_keys, Plan* pl) {
  const int64_t s_total = seq_len + n;
  const int64_t rows = (hq / kvh) * n;
  pl->row_blocks = (rows + kRows - 1) / kRows;
  // the chunk's block-table entries must fit the LDS copy
  const int64_t max_len = (int64_t)(kMaxPages - 2) * page_size / kKeys * kKeys;
  if (max_len < kKeys) return TM_ERR_SHAPE;
  Split sp;
  if (chunk_keys > 0) {
    const int64_t len = std::min((chunk_keys + kKeys - 1) / kKeys * kKeys, max_len);
    sp = split_keys(seq_len, n, len);
  } else {
    // every distinct chunk length from the longest allowed down to one stage
    const int64_t top = std::min<int64_t>(max_len, kMaxAutoLen);
    const int64_t keys = seq_len > 0 ? seq_len : s_total;
    sp = split_keys(seq_len, n, std::min((s_total + kKeys - 1) / kKeys * kKeys, top));
    double best = split_cost(sp, s_total, kvh, pl->row_blocks);
    int64_t parts = (keys + top - 1) / top;
    for (;;) {
      const int64_t len = ((keys + parts - 1) / parts + kKeys - 1) / kKeys * kKeys;
      const Split c = split_keys(seq_len, n, len);
      const double cost = split_cost(c, s_total, kvh, pl->row_blocks);
      if (cost < best) {
        best = cost;
        sp = c;
      }
      if (len <= kKeys) break;
      parts = (keys + len - kKeys - 1) / (len - kKeys);  // first count giving a shorter len
    }
  }
  pl->chunk_len = sp.len;
  pl->pre_chunks = sp.pre_chunks;
  pl->split = sp.split;
  pl->chunks = sp.chunks;
  pl->pairs = kvh * pl->chunks;
  pl->groups = groups_of(kvh, pl->row_blocks, pl->chunks);
  const int64_t slots = pl->chunks > 1 ? kvh * pl->row_blocks * pl->chunks * 4 : 0;
  pl->part_floats = slots * kPartHalves / 2;  // fp16 partials, counted in floats
  pl->stats_floats = slots * kStatFloats;
  return TM_OK;
}

int check_shape(int64_t n, int64_t hq, int64_t kvh, int64_t hd, int64_t seq_len,
                int64_t page_size) {
  if (n < 1 || n > kMaxNodes || hd != kHD || kvh < 1 || hq < kvh || hq % kvh != 0 ||
      hq > 1024 || seq_len < 0 || seq_len > (1 << 24))
    return TM_ERR_SHAPE;
  if (page_size < 4 || page_size > (1 << 16) || (page_size & (page_size - 1)) != 0)
    return TM_ERR_SHAPE;
  return TM_OK;
}

}  // namespace

extern "C" int tm_tree_attention_plan(int64_t N, int64_t Hq, int64_t kvh, int64_t hd,
                                      int64_t seq_len, int64_t page_size, int64_t chunk_keys,
                                      int64_t* chunks, int64_t* workspace_bytes) {
  int rc = check_shape(N, Hq, kvh, hd, seq_len, page_size);
  if (rc) return rc;
  if (chunk_keys < 0) return TM_ERR_ARG;
  Plan pl;
  rc = make_plan(N, Hq, kvh, seq_len, page_size, chunk_keys, &pl);
  if (rc) return rc;
  if (chunks) *chunks = pl.chunks;
  if (workspace_bytes) *workspace_bytes = (pl.part_floats + pl.stats_floats) * 4;
  return TM_OK;
}

extern "C" int tm_tree_mask_pack(const uint8_t* mask, int64_t N, int64_t row_stride,
                                 uint64_t* bits, void* stream) {
  if (N < 1 || N > kMaxNodes || row_stride < N) return TM_ERR_SHAPE;
  if (((uintptr_t)bits % 8) != 0) return TM_ERR_ALIGN;
  const int words = (int)((N + 63) / 64);
  const int total = (int)N * words;
  hipLaunchKernelGGL(tm_tree_mask_pack_kernel, dim3((total + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, mask, (int)N, row_stride, words, bits);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_tree_attention(const void* q, int64_t q_stride, const void* k_tail,
                                 const void* v_tail, int64_t tail_stride, void* k_cache,
                                 void* v_cache, int64_t stride_page, int64_t stride_slot,
                                 int64_t page_size, const int32_t* block_table,
                                 int64_t num_table_pages, int64_t seq_len,
                                 const int32_t* scratch_pages, int64_t num_scratch_pages,
                                 int write_tree, const uint64_t* mask_bits, int64_t N,
                                 int64_t Hq, int64_t kvh, int64_t hd, float scale, void* out,
                                 int64_t out_stride, int64_t chunk_keys, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  int rc = check_shape(N, Hq, kvh, hd, seq_len, page_size);
  if (rc) return rc;
  if (chunk_keys < 0 || !(scale > 0.0f)) return TM_ERR_ARG;
  if (q_stride < Hq * hd || tail_stride < kvh * hd || out_stride < Hq * hd ||
      stride_slot < kvh * hd || stride_page < page_size * stride_slot)
    return TM_ERR_SHAPE;
  if ((seq_len + page_size - 1) / page_size > num_table_pages) return TM_ERR_SHAPE;
  if (write_tree && (N + page_size - 1) / page_size > num_scratch_pages) return TM_ERR_SHAPE;
  // 16-byte vectors everywhere: base pointers and strides in whole vectors
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k_tail | (uintptr_t)v_tail |
                          (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out;
  if ((align % 16) != 0 || (q_stride % 8) || (tail_stride % 8) || (out_stride % 8) ||
      (stride_page % 8) || (stride_slot % 8) || ((uintptr_t)mask_bits % 8) ||
      ((uintptr_t)workspace % 16))
    return TM_ERR_ALIGN;
  Plan pl;
  rc = make_plan(N, Hq, kvh, seq_len, page_size, chunk_keys, &pl);
  if (rc) return rc;
  if ((pl.part_floats + pl.stats_floats) * 4 > workspace_bytes) return TM_ERR_SHAPE;
  if (pl.groups > INT32_MAX) return TM_ERR_SHAPE;

  AttnParams p;
  p.q = (const uint16_t*)q;
  p.k_tail = (const uint16_t*)k_tail;
  p.v_tail = (const uint16_t*)v_tail;
  p.k_cache = (uint16_t*)k_cache;
  p.v_cache = (uint16_t*)v_cache;
  p.block_table = block_table;
  p.scratch_pages = scratch_pages;
  p.mask_bits = mask_bits;
  p.out = (uint16_t*)out;
  p.part = (float*)workspace;
  p.stats = (float*)workspace + pl.part_floats;
  p.q_stride = q_stride;
  p.tail_stride = tail_stride;
  p.out_stride = out_stride;
  p.stride_page = stride_page;
  p.stride_slot = stride_slot;
  int shift = 0;
  while ((int64_t(1) << shift) < page_size) ++shift;
  p.page_shift = shift;
  p.seq_len = (int)seq_len;
  p.n = (int)N;
  p.hq = (int)Hq;
  p.kvh = (int)kvh;
  p.group = (int)(Hq / kvh);
  p.rows = (int)(p.group * N);
  p.row_blocks = (int)pl.row_blocks;
  p.chunks = (int)pl.chunks;
  p.chunk_len = (int)pl.chunk_len;
  p.pre_chunks = (int)pl.pre_chunks;
  p.split = (int)pl.split;
  p.pairs = (int)pl.pairs;
  p.mask_words = (int)((N + 63) / 64);
  p.write_tree = write_tree ? 1 : 0;
  p.scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(tm_tree_attn_kernel, dim3((unsigned)pl.groups), dim3(kThreads), 0,
                     (hipStream_t)stream, p);
  TM_HIP_CHECK_LAUNCH();
  if (pl.chunks > 1) {
    // kvh * row_blocks * 4 waves * 16 groups * 64 lanes threads
    hipLaunchKernelGGL(tm_tree_attn_combine_kernel,
                       dim3((unsigned)(kvh * pl.row_blocks * 4 * 16 * 64 / kThreads)),
                       dim3(kThreads), 0, (hipStream_t)stream, p);
    TM_HIP_CHECK_LAUNCH();
  }
  return TM_OK;
}
