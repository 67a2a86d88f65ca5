/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the op1/op4 hot path.
 *
 * Plain C restatement of the reference algorithms, evaluated with a fixed
 * order of IEEE single-precision operations (built with -ffp-contract=off), so
 * that it states the exact bits the device code must produce for routing,
 * gates, demand, layouts, argmax, the greedy walk and the KV commit.  Only the
 * tests, the smoke check and the benchmark's CPU-baseline leg may load it;
 * the product library never does.
 *
 * Reference sources followed (paths relative to the reference repository):
 *   router          treemoe/kernels/op1_tree_moe.py:676-677, treemoe/ref/tree_moe_ref.py:83-84
 *   budget routing  treemoe/ref/tree_moe_ref.py:14-67, op1_tree_moe.py:189-244
 *   bucketing       treemoe/ref/tree_moe_ref.py:91-98, op1_tree_moe.py:66-149, 246-297
 *   argmax          treemoe/kernels/op4_commit.py:82-96, treemoe/ref/verify_ref.py:56
 *   greedy walk     treemoe/kernels/op4_commit.py:99-131, treemoe/ref/verify_ref.py:52-95
 *   KV commit       treemoe/kernels/op4_commit.py:134-167, 241-267,
 *                   treemoe/model/kv_cache.py:88-106
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORC_LANES 64
#define ORC_TILE_M 64

static float bf16_bits_to_f32(uint16_t b) {
  uint32_t u = ((uint32_t)b) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* round-to-nearest-even float -> bfloat16 bits (quiet NaN for NaN) */
static uint16_t f32_to_bf16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t lsb = (u >> 16) & 1u;
  u = u + 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

static float f16_bits_to_f32(uint16_t b) {
  const uint32_t sign = ((uint32_t)b & 0x8000u) << 16;
  const uint32_t ex = ((uint32_t)b >> 10) & 0x1fu;
  const uint32_t man = (uint32_t)b & 0x3ffu;
  uint32_t u;
  if (ex == 0x1fu) {
    u = sign | 0x7f800000u | (man << 13);            /* inf / NaN */
  } else if (ex != 0) {
    u = sign | ((ex + 112u) << 23) | (man << 13);    /* normal: rebias 15 -> 127 */
  } else {                                           /* zero / subnormal: man * 2^-24 */
    float f = (float)man * 5.9604644775390625e-08f;  /* exact: man < 2^10 */
    memcpy(&u, &f, 4);
    u |= sign;
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* round-to-nearest-even float -> IEEE half bits: overflow (|f| >= 65520) to
 * infinity, subnormal results kept, NaN quiet */
static uint16_t f32_to_f16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (a >= 0x38800000u) {            /* normal half: |f| >= 2^-14 */
    uint32_t m = a - 0x38000000u;    /* exponent rebias 127 -> 15 */
    m += 0xfffu + ((m >> 13) & 1u);  /* round the 13 dropped bits to nearest even */
    return (uint16_t)(sign | (m >> 13));
  }
  float af;                          /* subnormal half: round |f| / 2^-24 to an integer */
  memcpy(&af, &a, 4);
  return (uint16_t)(sign | (uint32_t)rintf(af * 16777216.0f));
}

/* fp32 -> fp16 bits for n values (the rounding the fp16 router and GEMM
 * epilogues apply) */
void orc_f32_to_f16(const float* in, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16_bits(in[i]);
}

static float half_to_f32(uint16_t b, int f16) { return f16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b); }
static uint16_t f32_to_half(float f, int f16) { return f16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f); }

static float scale_pow2(float p, int k) {
  uint32_t bits = (uint32_t)(k + 127) << 23;
  float s;
  memcpy(&s, &bits, 4);
  return p * s;
}

/*
 * e^x for x <= 0.  Cody-Waite reduction x = k ln2 + r (ln2 = 0.693145751953125
 * + 1.42860676533018704e-6), Taylor series of e^r to degree 7 by Horner's rule,
 * then multiplication by 2^k.  x <= -80 gives 0 and x > 0 is treated as 0.
 */
float orc_expf(float x) {
  if (!(x > -80.0f)) return 0.0f;
  if (x > 0.0f) x = 0.0f;
  const float k = rintf(x * 1.44269504088896341f);
  float r = fmaf(k, -0.693145751953125f, x);
  r = fmaf(k, -1.42860676533018704e-06f, r);
  static const float inv_fact[8] = {
      1.0f, 1.0f, 0.5f, 1.66666666666666667e-01f, 4.16666666666666667e-02f,
      8.33333333333333333e-03f, 1.38888888888888889e-03f, 1.98412698412698413e-04f};
  float p = inv_fact[7];
  for (int d = 6; d >= 0; --d) p = fmaf(p, r, inv_fact[d]);
  return scale_pow2(p, (int)k);
}

/* 64 partial sums folded pairwise: s[i] += s[i + w] for w = 32, 16, ..., 1 */
static float fold64(float* s) {
  for (int w = ORC_LANES / 2; w >= 1; w >>= 1)
    for (int i = 0; i < w; ++i) s[i] = s[i] + s[i + w];
  return s[0];
}

/* bits of the router logit x[t] . wg[e] in the inputs' 16-bit type (bf16, or
 * fp16 when f16): 64 lane partials over 8-element chunks (chunk c to lane
 * c % 64, fused multiply-adds in chunk order), the pairwise fold, then round
 * to the type. */
static uint16_t router_logit_bits(const uint16_t* x, const uint16_t* wg, int64_t t, int64_t e,
                                  int64_t H, int f16) {
  float part[ORC_LANES];
  for (int l = 0; l < ORC_LANES; ++l) part[l] = 0.0f;
  for (int64_t c = 0; c < H / 8; ++c) {
    const int l = (int)(c % ORC_LANES);
    for (int j = 0; j < 8; ++j) {
      const float a = half_to_f32(x[t * H + 8 * c + j], f16);
      const float b = half_to_f32(wg[e * H + 8 * c + j], f16);
      part[l] = fmaf(a, b, part[l]);
    }
  }
  return f32_to_half(fold64(part), f16);
}

/* logits[t, e] (bits of the 16-bit type) as the router computes them before
 * the softmax */
void orc_router_logits_dt(const uint16_t* x, const uint16_t* wg, int64_t T, int64_t H,
                          int64_t E, int f16, uint16_t* logits) {
  for (int64_t t = 0; t < T; ++t)
    for (int64_t e = 0; e < E; ++e) logits[t * E + e] = router_logit_bits(x, wg, t, e, H, f16);
}

void orc_router_logits(const uint16_t* x, const uint16_t* wg, int64_t T, int64_t H, int64_t E,
                       uint16_t* logits) {
  orc_router_logits_dt(x, wg, T, H, E, 0, logits);
}

/* gates[t, e] = softmax(round16(x[t] . wg[e])), round16 to bf16 or fp16 */
void orc_router_gates_dt(const uint16_t* x, const uint16_t* wg, int64_t T, int64_t H,
                         int64_t E, int f16, float* gates) {
  float logits[64];
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t e = 0; e < E; ++e)
      logits[e] = half_to_f32(router_logit_bits(x, wg, t, e, H, f16), f16);
    float m = -INFINITY;
    for (int64_t e = 0; e < E; ++e) m = fmaxf(m, logits[e]);
    float ex[64];
    float sum = 0.0f;
    for (int64_t e = 0; e < E; ++e) {
      ex[e] = orc_expf(logits[e] - m);
    }
    for (int64_t e = 0; e < E; ++e) sum = sum + ex[e];
    for (int64_t e = 0; e < E; ++e) gates[t * E + e] = ex[e] / sum;
  }
}

void orc_router_gates(const uint16_t* x, const uint16_t* wg, int64_t T, int64_t H, int64_t E,
                      float* gates) {
  orc_router_gates_dt(x, wg, T, H, E, 0, gates);
}

/*
 * Budget routing + bucketing.  Outputs as documented for tm_op1_route_bucket.
 * Returns 0, or -1 if the tile list would exceed max_tiles or a slot lands
 * outside the padded layout.
 */
int orc_route_bucket(const float* gates, const float* accept, int64_t T, int64_t E,
                     int64_t budget, float tau, int objective, int64_t BM, int64_t max_blocks,
                     int64_t max_tiles, int64_t* topk_ids, float* gates_flat,
                     int64_t* padded_slots, int64_t* block_expert_ids, int64_t* slot_to_row,
                     float* demand, int32_t* expert_offsets, int32_t* sorted_slots,
                     int32_t* slot_pos, int32_t* tiles) {
  float crit[64];
  int keep[64];
  int64_t count[64], block_start[64], nblocks[64], offset[65], seen[64];

  /* demand: accept-weighted gate mass, 64 strided partial sums then a fold */
  for (int64_t e = 0; e < E; ++e) {
    float part[ORC_LANES];
    for (int l = 0; l < ORC_LANES; ++l) part[l] = 0.0f;
    for (int64_t t = 0; t < T; ++t) {
      const float p = accept[t] * gates[t * E + e];
      part[t % ORC_LANES] = part[t % ORC_LANES] + p;
    }
    demand[e] = fold64(part);
    crit[e] = -INFINITY;
  }

  /* criticality: max accept over nodes whose unrestricted top-1 (or top-2,
   * when accept >= tau) is e */
  if (objective == 1) {
    for (int64_t t = 0; t < T; ++t) {
      const float* g = gates + t * E;
      int64_t u1 = 0;
      for (int64_t e = 1; e < E; ++e)
        if (g[e] > g[u1]) u1 = e;
      int64_t u2 = -1;
      for (int64_t e = 0; e < E; ++e) {
        if (e == u1) continue;
        if (u2 < 0 || g[e] > g[u2]) u2 = e;
      }
      crit[u1] = fmaxf(crit[u1], accept[t]);
      if (accept[t] >= tau) crit[u2] = fmaxf(crit[u2], accept[t]);
    }
  }

  /* keep set: first `budget` experts of the order (crit desc,) demand desc, e asc */
  for (int64_t e = 0; e < E; ++e) keep[e] = 0;
  for (int64_t r = 0; r < budget; ++r) {
    int64_t best = -1;
    for (int64_t e = 0; e < E; ++e) {
      if (keep[e]) continue;
      if (best < 0) {
        best = e;
      } else if (objective == 1) {
        if (crit[e] > crit[best] || (crit[e] == crit[best] && demand[e] > demand[best])) best = e;
      } else if (demand[e] > demand[best]) {
        best = e;
      }
    }
    keep[best] = 1;
  }

  /* top-2 within the kept set, p_k / (p1 + p2), degrade below tau */
  for (int64_t t = 0; t < T; ++t) {
    const float* g = gates + t * E;
    int64_t i1 = -1, i2 = -1;
    float g1 = 0.0f, g2 = 0.0f;
    for (int64_t e = 0; e < E; ++e) {
      const float v = keep[e] ? g[e] : 0.0f;
      if (i1 < 0 || v > g1) { i1 = e; g1 = v; }
    }
    for (int64_t e = 0; e < E; ++e) {
      if (e == i1) continue;
      const float v = keep[e] ? g[e] : 0.0f;
      if (i2 < 0 || v > g2) { i2 = e; g2 = v; }
    }
    const float s = g1 + g2;
    float w1 = g1 / s, w2 = g2 / s;
    if (accept[t] < tau) { w1 = 1.0f; w2 = 0.0f; }
    topk_ids[2 * t] = i1;
    topk_ids[2 * t + 1] = i2;
    gates_flat[2 * t] = w1;
    gates_flat[2 * t + 1] = w2;
  }

  /* stable (expert, slot) order */
  const int64_t S = 2 * T;
  for (int64_t e = 0; e < E; ++e) { count[e] = 0; seen[e] = 0; }
  for (int64_t s = 0; s < S; ++s) count[topk_ids[s]]++;
  int64_t blocks = 0, off = 0, ntiles = 0;
  for (int64_t e = 0; e < E; ++e) {
    nblocks[e] = (count[e] + BM - 1) / BM;
    block_start[e] = blocks;
    blocks += nblocks[e];
    offset[e] = off;
    for (int64_t r = 0; r < count[e]; r += ORC_TILE_M) {
      if (ntiles >= max_tiles) return -1;
      tiles[4 * ntiles + 0] = (int32_t)e;
      tiles[4 * ntiles + 1] = (int32_t)(off + r);
      tiles[4 * ntiles + 2] = (int32_t)((count[e] - r) < ORC_TILE_M ? (count[e] - r) : ORC_TILE_M);
      tiles[4 * ntiles + 3] = 0;
      ntiles++;
    }
    off += count[e];
  }
  offset[E] = off;
  for (int64_t j = ntiles; j < max_tiles; ++j) {
    tiles[4 * j + 0] = -1;
    tiles[4 * j + 1] = 0;
    tiles[4 * j + 2] = 0;
    tiles[4 * j + 3] = 0;
  }
  for (int64_t e = 0; e <= E; ++e) expert_offsets[e] = (int32_t)offset[e];
  for (int64_t i = 0; i < max_blocks * BM; ++i) padded_slots[i] = -1;
  for (int64_t s = 0; s < S; ++s) {
    const int64_t e = topk_ids[s];
    const int64_t rank = seen[e]++;
    const int64_t dest = block_start[e] * BM + rank;
    const int64_t pos = offset[e] + rank;
    if (dest >= max_blocks * BM) return -1;
    slot_to_row[s] = dest;
    padded_slots[dest] = s;
    sorted_slots[pos] = (int32_t)s;
    slot_pos[s] = (int32_t)pos;
  }
  for (int64_t b = 0; b < max_blocks; ++b) {
    int64_t owner = -1;
    for (int64_t e = 0; e < E; ++e)
      if (nblocks[e] > 0 && b >= block_start[e] && b < block_start[e] + nblocks[e]) owner = e;
    block_expert_ids[b] = owner;
  }
  return 0;
}

/* first-occurrence argmax with NaN ranked above every number (numpy order) */
static int ranks_before(float va, int64_t ia, float vb, int64_t ib) {
  const int na = isnan(va), nb = isnan(vb);
  if (na != nb) return na;
  if (!na && va != vb) return va > vb;
  return ia < ib;
}

void orc_argmax(const void* logits, int dtype, int64_t N, int64_t V, int64_t row_stride,
                int32_t* out) {
  for (int64_t n = 0; n < N; ++n) {
    float bv = 0.0f;
    int64_t bi = -1;
    for (int64_t v = 0; v < V; ++v) {
      const float x = (dtype == 0)
                          ? ((const float*)logits)[n * row_stride + v]
                          : bf16_bits_to_f32(((const uint16_t*)logits)[n * row_stride + v]);
      if (bi < 0 || ranks_before(x, v, bv, bi)) { bv = x; bi = v; }
    }
    out[n] = (int32_t)bi;
  }
}

/*
 * Greedy walk: from the root, at most max_depth levels; at each node the first
 * child in list order whose token equals the node's argmax is accepted.
 * result = (bonus, num_accepted, next_root).
 */
/*
 * Argmax of softmax(row) rounded to the row's dtype (the reference's greedy
 * pick after a repetition penalty: _postprocess_softmax_kernel at temperature 1
 * then _argmax_kernel over the probabilities, treemoe/kernels/op4_commit.py:
 * 207-214).  e_i = exp(x_i - max); the sum s runs in 256 index-strided partials
 * (partial j adds elements j, j+256, ... in order), each 64 partials folded
 * pairwise, the 4 folds added in order; p_i = round(e_i / s).  Returns the
 * first i with p_i equal to the row maximum's p = round(1 / s); 0 if none.
 */
void orc_softmax_argmax(const void* logits, int dtype, int64_t N, int64_t V,
                        int64_t row_stride, int32_t* out) {
  for (int64_t n = 0; n < N; ++n) {
    const float* pf = (const float*)logits + n * row_stride;
    const uint16_t* pb = (const uint16_t*)logits + n * row_stride;
#define ORC_X(i) (dtype == 0 ? pf[i] : bf16_bits_to_f32(pb[i]))
#define ORC_ROUND(p) (dtype == 0 ? (p) : bf16_bits_to_f32(f32_to_bf16_bits(p)))
    float m = -INFINITY;
    for (int64_t i = 0; i < V; ++i) m = fmaxf(m, ORC_X(i));
    float part[4 * ORC_LANES];
    for (int j = 0; j < 4 * ORC_LANES; ++j) part[j] = 0.0f;
    for (int64_t i = 0; i < V; ++i) {
      const int j = (int)(i % (4 * ORC_LANES));
      part[j] = part[j] + orc_expf(ORC_X(i) - m);
    }
    float s = fold64(part);
    for (int w = 1; w < 4; ++w) s = s + fold64(part + w * ORC_LANES);
    const float top = ORC_ROUND(1.0f / s);
    int32_t first = 0;
    for (int64_t i = 0; i < V; ++i) {
      if (ORC_ROUND(orc_expf(ORC_X(i) - m) / s) == top) {
        first = (int32_t)i;
        break;
      }
    }
    out[n] = first;
#undef ORC_X
#undef ORC_ROUND
  }
}

void orc_greedy_walk(const int32_t* argmax, const int64_t* tokens, const int32_t* child_start,
                     const int32_t* child_count, const int32_t* child_list, int64_t N,
                     int64_t max_depth, int64_t* accepted_slots, int64_t* accepted_tokens,
                     int64_t* result) {
  int64_t node = 0, count = 0;
  for (int64_t i = 0; i < N; ++i) { accepted_slots[i] = -1; accepted_tokens[i] = -1; }
  for (int64_t d = 0; d < max_depth; ++d) {
    int64_t hit = -1;
    for (int32_t j = 0; j < child_count[node]; ++j) {
      const int64_t c = child_list[child_start[node] + j];
      if (tokens[c] == (int64_t)argmax[node]) { hit = c; break; }
    }
    if (hit < 0) break;
    accepted_slots[count] = hit;
    accepted_tokens[count] = tokens[hit];
    count++;
    node = hit;
  }
  result[0] = argmax[node];
  result[1] = count;
  result[2] = node;
}

/*
 * Commit [root] + accepted path: for every layer, copy the K and V rows of
 * tree slot s (scratch page s / P, offset s % P) to sequence position
 * seq_len + j (page block_table[pos / P], offset pos % P).  Byte copy.
 */
void orc_kv_commit(uint8_t* k, uint8_t* v, int64_t elem_bytes, int64_t L, int64_t row_elems,
                   int64_t stride_layer, int64_t stride_page, int64_t stride_slot,
                   int64_t page_size, const int64_t* accepted_slots, int64_t num_accepted,
                   const int32_t* scratch_pages, const int32_t* block_table, int64_t seq_len) {
  const int64_t rb = row_elems * elem_bytes;
  for (int64_t l = 0; l < L; ++l) {
    for (int64_t j = 0; j <= num_accepted; ++j) {
      const int64_t s = (j == 0) ? 0 : accepted_slots[j - 1];
      const int64_t q = seq_len + j;
      const int64_t src = (l * stride_layer + (int64_t)scratch_pages[s / page_size] * stride_page +
                           (s % page_size) * stride_slot) * elem_bytes;
      const int64_t dst = (l * stride_layer + (int64_t)block_table[q / page_size] * stride_page +
                           (q % page_size) * stride_slot) * elem_bytes;
      memmove(k + dst, k + src, (size_t)rb);
      memmove(v + dst, v + src, (size_t)rb);
    }
  }
}
