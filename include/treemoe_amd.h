/*
 * treemoe_amd.h — C ABI of the MI355X (gfx950) verification hot path.
 *
 * One shared library, libtreemoe_amd.so, exports the entry points below.  They
 * replace the GPU work behind the reference's Python operators:
 *
 *   op1  tree_moe_forward / route_experts   treemoe/kernels/op1_tree_moe.py:641-802
 *   op4  fused_verify_commit                treemoe/kernels/op4_commit.py:170-272
 *   tree attention (verification forward)   treemoe/model/mixtral.py:208-250
 *
 * Conventions (all entry points):
 *   - plain device pointers and sizes; no torch types, no allocation inside;
 *   - every call is asynchronous on `stream` (a hipStream_t, may be NULL for the
 *     null stream) and is the last argument;
 *   - the return value is 0 (TM_OK) on success, a TM_ERR_* argument code when a
 *     size/shape check fails before any launch, or a hipError_t value (offset by
 *     TM_ERR_HIP_BASE) when a launch fails;
 *   - bf16 tensors are passed as raw 16-bit storage (`const void*`), row-major
 *     and contiguous unless a stride argument says otherwise;
 *   - calls that share workspace buffers must be serialised on one stream.
 */
#ifndef TREEMOE_AMD_H
#define TREEMOE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TM_OK 0
#define TM_ERR_SHAPE 1001      /* a size argument is out of the supported range */
#define TM_ERR_ALIGN 1002      /* a pointer or stride is not suitably aligned   */
#define TM_ERR_ARG 1003        /* an enumerated argument has an unknown value   */
#define TM_ERR_HIP_BASE 2000   /* TM_ERR_HIP_BASE + hipError_t                  */

#define TM_OBJECTIVE_MASS 0
#define TM_OBJECTIVE_CRITICAL_PATH 1

#define TM_DTYPE_F32 0
#define TM_DTYPE_BF16 1
#define TM_DTYPE_F16 2

/* Limits checked by the entry points. */
#define TM_MAX_EXPERTS 64
#define TM_MAX_TOKENS 65536     /* tokens per op1 layer (routing); the GEMMs also need their
                                    byte offsets below 2^31 */
#define TM_GEMM_TILE_M 64      /* rows of one expert processed per GEMM tile */
#define TM_OP4_MAX_PARTS 64    /* row ranges per node in the argmax workspace  */
#define TM_OP4_NOALLOC_MAX_NODES 2048  /* N limit of tm_op4_argmax_walk_noalloc */

/* ABI version (major*10000 + minor*100 + patch): 5.0.0.  Version 2 added
 * num_edges to tm_op4_argmax_walk / tm_op4_sample_walk and softmax_argmax to
 * tm_op4_argmax_walk; version 3 added host_count to tm_op4_kv_commit;
 * version 4 added `dtype` (TM_DTYPE_BF16 or TM_DTYPE_F16) to the op1 entry
 * points that read or write 16-bit activations or weights; 4.1 added
 * tm_op1_prefill_gemm1_routed; version 5 made tm_op4_sample_walk's bonus
 * argument V exponential draws (bonus_exp) instead of one uniform. */
int tm_version(void);

/* Human-readable text for a return code of any entry point. */
const char* tm_status_string(int code);

/* Device address of pinned host memory (hipHostGetDevicePointer), for
 * arguments the kernels write to host memory (tm_op4_kv_commit's host_count).
 * No reference counterpart: a utility of this ABI. */
int tm_host_device_pointer(void* host, void** device);

/* ---------------------------------------------------------------- op1 -- */

/* `dtype` of the op1 entry points is the type of x, the weights, h and the
 * output: TM_DTYPE_BF16 or TM_DTYPE_F16 (the reference kernels take either,
 * treemoe/kernels/op1_tree_moe.py:762-766); "bf16" below stands for it.
 * Arithmetic is fp32 in both cases; rounding to the type is
 * round-to-nearest-even. */

/*
 * Router: gates[t, e] = softmax_e( bf16( x[t, :] . wg[e, :] ) ), fp32.
 * Replaces `F.linear(x, W_g)` + `torch.softmax(logits.float(), -1)` at
 * treemoe/kernels/op1_tree_moe.py:676-677 (same maths as
 * treemoe/ref/tree_moe_ref.py:83-84).  x: [T, H] bf16, wg: [E, H] bf16,
 * gates: [T, E] fp32.  Requires H % 8 == 0, 1 <= T <= TM_MAX_TOKENS,
 * 2 <= E <= TM_MAX_EXPERTS.
 */
int tm_op1_router_gates(const void* x, const void* wg, int64_t T, int64_t H,
                        int64_t E, float* gates, int dtype, void* stream);

/*
 * Budget routing + stable (expert, DFS) bucketing in one workgroup.
 * Replaces `_budget_bucket_fused_kernel` (treemoe/kernels/op1_tree_moe.py:159-297)
 * and its torch fallback `route_and_bucket` (:81-149); semantics of
 * `budget_route_ref` (treemoe/ref/tree_moe_ref.py:14-67) and
 * `route_and_bucket_ref` (:70-99).
 *
 * Inputs : gates [T, E] fp32, accept [T] fp32, budget in [2, E], tau,
 *          objective (TM_OBJECTIVE_*), block_m (16 or 32) and max_blocks
 *          (= compact_block_capacity(2T, budget, block_m)) for the reference's
 *          padded layout, max_tiles (= compact_block_limit(2T, budget,
 *          TM_GEMM_TILE_M)) for the GEMM tile list.
 * Outputs (reference layout, all written every call):
 *          topk_ids [2T] i64, gates_flat [2T] f32, padded_slots
 *          [max_blocks*block_m] i64 (-1 pad), block_expert_ids [max_blocks] i64
 *          (-1 unused), slot_to_row [2T] i64, demand [E] f32;
 * Outputs (compact layout used by the GEMMs):
 *          expert_offsets [E+1] i32, sorted_slots [2T] i32 (expert-major,
 *          DFS-stable), slot_pos [2T] i32 (inverse of sorted_slots),
 *          tiles [max_tiles*4] i32 = (expert or -1, first sorted row, rows, 0).
 */
int tm_op1_route_bucket(const float* gates, const float* accept, int64_t T,
                        int64_t E, int64_t budget, float tau, int objective,
                        int64_t block_m, int64_t max_blocks, int64_t max_tiles,
                        int64_t* topk_ids, float* gates_flat,
                        int64_t* padded_slots, int64_t* block_expert_ids,
                        int64_t* slot_to_row, float* demand,
                        int32_t* expert_offsets, int32_t* sorted_slots,
                        int32_t* slot_pos, int32_t* tiles, void* stream);

/*
 * Router + budget routing + bucketing in one call (two launches on `stream`:
 * one workgroup per token computes that token's gates exactly as
 * tm_op1_router_gates, then one workgroup buckets all tokens exactly as
 * tm_op1_route_bucket).  Replaces the reference's router
 * (op1_tree_moe.py:676-677) plus `_budget_bucket_fused_kernel` (:159-297) as
 * launched by `route_experts` (:641-708).  Arguments and outputs are the union
 * of the two entry points above; gates [T, E] fp32 is written too.
 */
int tm_op1_route(const void* x, const void* wg, const float* accept, int64_t T,
                 int64_t H, int64_t E, int64_t budget, float tau, int objective,
                 int64_t block_m, int64_t max_blocks, int64_t max_tiles,
                 float* gates, int64_t* topk_ids, float* gates_flat,
                 int64_t* padded_slots, int64_t* block_expert_ids,
                 int64_t* slot_to_row, float* demand, int32_t* expert_offsets,
                 int32_t* sorted_slots, int32_t* slot_pos, int32_t* tiles,
                 int dtype, void* stream);

/*
 * Gate/up projection + SwiGLU for every routed slot.
 * Replaces `_moe_gemm1_kernel` (treemoe/kernels/op1_tree_moe.py:300-383):
 *   h[p, :] = bf16( silu(x[tok] . w1[e]^T) * (x[tok] . w3[e]^T) ), fp32 accumulate,
 * for sorted row p of expert e, tok = sorted_slots[p] / 2.
 * x: [T, H] bf16, w1/w3: [E, I, H] bf16.  h is a workspace of
 * max_tiles * TM_GEMM_TILE_M * I bf16 elements holding each tile's rows in
 * MFMA A-fragment order (tile j, 16-row sub-tile b, 32-column k-step s: 64
 * lanes x 8 elements, lane = (k/8 % 4) * 16 + row % 16), the layout
 * tm_op1_gemm2 consumes.  Requires H % 256 == 0 and I % 256 == 0.
 */
int tm_op1_gemm1(const void* x, const void* w1, const void* w3, void* h,
                 const int32_t* sorted_slots, const int32_t* tiles,
                 int64_t max_tiles, int64_t T, int64_t H, int64_t I, int64_t E,
                 int dtype, void* stream);

/*
 * Down projection, split over K = I into `split` deterministic segments.
 * Replaces `_moe_gemm2_det_kernel` (treemoe/kernels/op1_tree_moe.py:447-509):
 *   y[s, p, :] = gates_flat[slot] * ( h[p, Ks] . w2[e][:, Ks]^T ), fp32,
 * h: the tile-swizzled workspace written by tm_op1_gemm1, w2: [E, H, I] bf16,
 * y: [split, 2T, H] fp32 (workspace).
 * Requires H % 32 == 0 and (I / split) % 256 == 0.
 */
int tm_op1_gemm2(const void* h, const void* w2, float* y,
                 const float* gates_flat, const int32_t* sorted_slots,
                 const int32_t* tiles, int64_t max_tiles, int64_t split,
                 int64_t T, int64_t H, int64_t I, int64_t E, int dtype, void* stream);

/*
 * Fixed-order combine.  Replaces `_combine_kernel`
 * (treemoe/kernels/op1_tree_moe.py:512-529) and the final `.to(x.dtype)` (:798):
 *   out[t, :] = bf16( ((y[0,p0] + .. + y[S-1,p0]) + y[0,p1]) + .. + y[S-1,p1] )
 * with p_k = slot_pos[2t + k].  out: [T, H] bf16.  Requires H % 4 == 0.
 */
int tm_op1_combine(const float* y, const int32_t* slot_pos, void* out,
                   int64_t T, int64_t H, int64_t split, int dtype, void* stream);

/*
 * Gate/up projection + SwiGLU for many rows per expert (prefill / batched
 * trees), MFMA-tiled over 128 sorted rows x (128 w1 + the same 128 w3) weight
 * rows; 256 rows when 2T >= 384 E, and 64 rows x (64 + 64) weight rows when
 * 2T <= 16 max_tiles (few rows per active expert).  Same maths as
 * tm_op1_gemm1 and the reference `_moe_gemm1_kernel`
 * (treemoe/kernels/op1_tree_moe.py:300-383), but h is written ROW-MAJOR:
 *   h[p, n] = bf16( silu(x[sorted_slots[p] / 2] . w1[e, n]) * (... . w3[e, n]) )
 * for every row p of the compact expert-major order (expert e owns rows
 * expert_offsets[e] .. expert_offsets[e+1]-1).  h: [2T, I] bf16 (rows >= 2T
 * untouched).  `tiles` is the 64-row tile list of the same routing: an expert
 * whose first tile entry is masked (expert -1) is skipped.  Requires
 * H % 64 == 0 and I % 128 == 0.  Consumed by tm_op1_prefill_gemm2.
 */
int tm_op1_prefill_gemm1(const void* x, const void* w1, const void* w3, void* h,
                         const int32_t* sorted_slots, const int32_t* expert_offsets,
                         const int32_t* tiles, int64_t max_tiles, int64_t T, int64_t H,
                         int64_t I, int64_t E, int dtype, void* stream);

/*
 * tm_op1_route_bucket and tm_op1_prefill_gemm1 in ONE launch, for few tokens:
 * together with tm_op1_router_gates this replaces the routing and gate/up
 * launches of the reference's tree_moe_forward (router op1_tree_moe.py:676-677,
 * `_budget_bucket_fused_kernel` :159-297, `_moe_gemm1_kernel` :300-383, as
 * launched at :771-781).  Every GEMM wave derives its own M-tile and rows
 * from gates and accept (one token per lane, the bucketing's operations in
 * the same floating-point order); one more workgroup writes every routing
 * output of tm_op1_route_bucket (same arguments, same bits).  h is written as
 * by tm_op1_prefill_gemm1 (row-major [2T, I], no expert masked), for
 * tm_op1_prefill_gemm2 and tm_op1_combine with the routing outputs written
 * here.  Requires 1 <= T <= 64, 2 <= E <= 16, max_blocks <= 256, and the
 * shape rules of tm_op1_prefill_gemm1.
 */
int tm_op1_prefill_gemm1_routed(const void* x, const void* w1, const void* w3, void* h,
                                const float* gates, const float* accept, int64_t T, int64_t H,
                                int64_t I, int64_t E, int64_t budget, float tau, int objective,
                                int64_t block_m, int64_t max_blocks, int64_t max_tiles,
                                int64_t* topk_ids, float* gates_flat, int64_t* padded_slots,
                                int64_t* block_expert_ids, int64_t* slot_to_row, float* demand,
                                int32_t* expert_offsets, int32_t* sorted_slots,
                                int32_t* slot_pos, int32_t* tiles, int dtype, void* stream);

/*
 * Down projection for many rows per expert, MFMA-tiled over 128 rows x 256
 * output columns; the prefill counterpart of tm_op1_gemm2 (reference
 * `_moe_gemm2_det_kernel`, treemoe/kernels/op1_tree_moe.py:447-509):
 *   y[s, p, n] = gates_flat[sorted_slots[p]] * sum_{k in segment s} h[p, k] w2[e, n, k]
 * with h row-major [2T, I] from tm_op1_prefill_gemm1 and y [split, 2T, H] fp32
 * in the layout tm_op1_combine reads; masked experts (as in
 * tm_op1_prefill_gemm1) leave their rows of y untouched.  Requires
 * H % 256 == 0 and (I / split) % 64 == 0.
 */
int tm_op1_prefill_gemm2(const void* h, const void* w2, float* y, const float* gates_flat,
                         const int32_t* sorted_slots, const int32_t* expert_offsets,
                         const int32_t* tiles, int64_t max_tiles, int64_t split, int64_t T,
                         int64_t H, int64_t I, int64_t E, int dtype, void* stream);

/* ---------------------------------------------------------------- op4 -- */

/*
 * First-occurrence argmax per tree node + greedy accept walk (two launches on
 * `stream`: row ranges of ~4 KiB scanned by one workgroup each, then one
 * workgroup that reduces the ranges and walks the tree from LDS).
 * Replaces `_argmax_kernel` (treemoe/kernels/op4_commit.py:82-96) and
 * `_tree_verify_greedy_kernel` (:99-131) plus the result glue (:223-239).
 *
 * logits: [N, V] (row stride `row_stride` elements), dtype TM_DTYPE_F32 or
 * TM_DTYPE_BF16.  NaN ranks above every number (first NaN wins), as in
 * torch.argmax.  tokens [N] i64; children in CSR form: child_start [N] i32,
 * child_count [N] i32, child_list [max(1, num_edges)] i32 holding num_edges
 * entries (N - 1 for a full tree, fewer when the tree is padded with
 * edge-free slots).  Child ranges are clipped to num_edges and children
 * outside [0, N) never match.  The walk visits at most max_depth levels (and
 * accepts at most N nodes).
 * softmax_argmax = 0: argmax of the logits (reference :203-206).
 * softmax_argmax = 1: argmax of softmax(row) rounded to the logits' dtype, the
 * reference's pick when a repetition penalty was applied (:207-214): with
 * e_i = exp(x_i - max), s = sum e_i, the first i whose rounded e_i / s equals
 * the rounded 1 / s (one workgroup per row instead of the row ranges).
 * Outputs: argmax [N] i32, accepted_slots [N] i64 (-1 pad), accepted_tokens
 * [N] i64 (-1 pad), result [3] i64 = (bonus_token, num_accepted, next_root).
 * `workspace`: N * TM_OP4_MAX_PARTS * 8 bytes of device memory, 8-byte
 * aligned, no initial contents required.
 */
int tm_op4_argmax_walk(const void* logits, int dtype, int64_t N, int64_t V,
                       int64_t row_stride, const int64_t* tokens,
                       const int32_t* child_start, const int32_t* child_count,
                       const int32_t* child_list, int64_t num_edges,
                       int64_t max_depth, int softmax_argmax, int32_t* argmax,
                       int64_t* accepted_slots,
                       int64_t* accepted_tokens, int64_t* result,
                       void* workspace, void* stream);

/*
 * tm_op4_argmax_walk without the workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc): the row
 * partials live in a static device array owned by the library, 1 MiB
 * (TM_OP4_NOALLOC_MAX_NODES * TM_OP4_MAX_PARTS * 8 bytes) on every GPU the
 * library runs on, held until the process ends.  N <= TM_OP4_NOALLOC_MAX_NODES
 * (else TM_ERR_SHAPE).  Calls nothing that allocates.  All calls on one GPU
 * share that array: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller.  Arguments, outputs and
 * results as tm_op4_argmax_walk; `stream` must belong to a device this process
 * can make current.
 */
int tm_op4_argmax_walk_noalloc(const void* logits, int dtype, int64_t N, int64_t V,
                               int64_t row_stride, const int64_t* tokens,
                               const int32_t* child_start, const int32_t* child_count,
                               const int32_t* child_list, int64_t num_edges,
                               int64_t max_depth, int softmax_argmax, int32_t* argmax,
                               int64_t* accepted_slots, int64_t* accepted_tokens,
                               int64_t* result, void* stream);

/*
 * Repetition penalty, in place on every row of logits [N, V] (row stride
 * `row_stride`, TM_DTYPE_F32 or TM_DTYPE_BF16).  Replaces pass 0 of
 * `_postprocess_softmax_kernel` (treemoe/kernels/op4_commit.py:53-57) as
 * launched for greedy verification with rep_penalty != 1 (:201-214): for each
 * of the num_prev tokens in order, x = x > 0 ? x / penalty : x * penalty, so a
 * token listed k times is penalised k times (bf16 rows are rounded after each
 * application, as the reference stores them).  Tokens outside [0, V) are
 * skipped.  `table`: 2 * table_size int32 of device memory, 16-byte aligned,
 * table_size a power of two >= max(4, 2 * num_prev); no initial contents
 * required.
 */
int tm_op4_rep_penalty(void* logits, int dtype, int64_t N, int64_t V, int64_t row_stride,
                       const int64_t* prev_tokens, int64_t num_prev, float penalty,
                       int32_t* table, int64_t table_size, void* stream);

/*
 * Tree rejection sampling walk (temperature > 0), one launch.  Replaces the
 * sampling branch of `tree_verify_ref` (treemoe/ref/verify_ref.py:60-89), which
 * the reference's fused_verify_commit runs for temperature > 0
 * (treemoe/kernels/op4_commit.py:187-196).  At the current node the residual
 * is softmax(logits[node] / temperature); children are tried in child-list
 * order, child c (token t) is accepted when
 *   uniforms[c] < min(residual[t] / max(q_c[t], 1e-20), 1),  q_c = draft_probs[c],
 * and otherwise residual = max(residual - q_c, 0) / max(sum, 1e-20).  Depth is
 * unbounded (at most N accepted nodes).  When every child is rejected (or at a
 * leaf) the bonus token is the first j maximising residual[j] / bonus_exp[j]
 * (IEEE fp32 division): the reference's torch.multinomial(residual, 1,
 * generator) draws exactly that index when bonus_exp is
 * torch.empty(V).exponential_(1, generator) taken after the N uniforms, so
 * the same generator state gives the reference's bonus (PyTorch samples one
 * index by this exponential race).  draft_probs: [N, V] fp32, row stride
 * q_stride.  Children in CSR form with num_edges entries, as in
 * tm_op4_argmax_walk.  uniforms [N], bonus_exp [V] (> 0) fp32 on the device.
 * residual: V fp32 of device memory (the final residual on return).
 * V <= 2^25.  Outputs as tm_op4_argmax_walk.
 */
int tm_op4_sample_walk(const void* logits, int dtype, int64_t N, int64_t V, int64_t row_stride,
                       const float* draft_probs, int64_t q_stride, const int64_t* tokens,
                       const int32_t* child_start, const int32_t* child_count,
                       const int32_t* child_list, int64_t num_edges, const float* uniforms,
                       const float* bonus_exp, float temperature, float* residual,
                       int64_t* accepted_slots,
                       int64_t* accepted_tokens, int64_t* result, void* stream);

/*
 * Paged KV commit of [root] + accepted path.  Replaces `_kv_commit_kernel` and
 * its host glue (treemoe/kernels/op4_commit.py:134-167, 241-267); reference
 * semantics `PagedKVCache.commit_tree` (treemoe/model/kv_cache.py:88-106).
 *
 * For layer l < L and j <= num_accepted (read on device from result[1]):
 *   src slot  s = (j == 0 ? 0 : accepted_slots[j-1]),
 *             page scratch_pages[s / page_size], offset s % page_size;
 *   dest pos  q = seq_len + j, page block_table[q / page_size], offset q % page_size;
 *   k[l, dst] = k[l, src] and v[l, dst] = v[l, src], row_bytes bytes each.
 * k, v: [L, pages, page_size, kvh, hd] with strides (elements of elem_bytes):
 * stride_layer, stride_page, stride_slot.  Grid covers j <= max_depth.
 * host_count: NULL, or the device address (tm_host_device_pointer) of a pinned
 * host int64 that receives num_accepted with a system-scope store early in the
 * launch; the caller can then read the count without a device-to-host copy
 * (the reference reads it with .item(), op4_commit.py:267).
 */
int tm_op4_kv_commit(void* k, void* v, int64_t elem_bytes, int64_t L,
                     int64_t row_elems, int64_t stride_layer,
                     int64_t stride_page, int64_t stride_slot,
                     int64_t page_size, const int64_t* accepted_slots,
                     const int64_t* result, const int32_t* scratch_pages,
                     int64_t num_scratch_pages, const int32_t* block_table,
                     int64_t num_table_pages, int64_t seq_len,
                     int64_t max_depth, int64_t* host_count, void* stream);

/*
 * Tree attention: the verification forward's attention over the paged KV
 * cache.  Replaces, for the tree branch of `MixtralForward._attention`
 * (treemoe/model/mixtral.py:208-250): `PagedKVCache.write_tree`
 * (treemoe/model/kv_cache.py:80-86), `gather_with_tail` (:125-145), the mask
 * (mixtral.py:211-218) and `F.scaled_dot_product_attention(..., enable_gqa=True)`.
 *
 * Node i, query head h (kv head h / (Hq / kvh)) attends to every prefix
 * position 0 .. seq_len-1 and to tree node j when bit j of mask row i is set:
 *   out[i, h] = softmax_j(scale * q[i, h] . k_j) v_j,
 * prefix k_j/v_j read in place from the layer's cache pages: page
 * block_table[pos / page_size], slot pos % page_size; tree k_j/v_j read from
 * k_tail/v_tail [N, kvh, hd].  With write_tree the tree rows are also stored
 * in the scratch pages (node j: page scratch_pages[j / page_size], slot
 * j % page_size), as write_tree does.  A row with no visible key gives 0.
 *
 * q, out: [N, Hq, hd] bf16 (node strides q_stride, out_stride; heads
 * contiguous).  k_cache, v_cache: this layer's [pages, page_size, kvh, hd]
 * bf16 with strides stride_page, stride_slot (elements).  mask_bits: [N,
 * ceil(N/64)] u64 (tm_tree_mask_pack).  hd = 128, N <= 256, page_size a power
 * of two; 16-byte aligned pointers and strides.  chunk_keys: keys per
 * workgroup (0 = automatic); workspace: tm_tree_attention_plan's size.
 */
int tm_tree_attention(const void* q, int64_t q_stride, const void* k_tail,
                      const void* v_tail, int64_t tail_stride, void* k_cache,
                      void* v_cache, int64_t stride_page, int64_t stride_slot,
                      int64_t page_size, const int32_t* block_table,
                      int64_t num_table_pages, int64_t seq_len,
                      const int32_t* scratch_pages, int64_t num_scratch_pages,
                      int write_tree, const uint64_t* mask_bits, int64_t N,
                      int64_t Hq, int64_t kvh, int64_t hd, float scale, void* out,
                      int64_t out_stride, int64_t chunk_keys, void* workspace,
                      int64_t workspace_bytes, void* stream);

/*
 * Key chunking of tm_tree_attention for these sizes: the number of key chunks
 * and the workspace bytes it needs (0 when one chunk covers every key).  Host
 * only; no counterpart in the reference, which has no workspace.
 */
int tm_tree_attention_plan(int64_t N, int64_t Hq, int64_t kvh, int64_t hd,
                           int64_t seq_len, int64_t page_size, int64_t chunk_keys,
                           int64_t* chunks, int64_t* workspace_bytes);

/*
 * Bit-pack the tree's [N, N] bool ancestor mask (engine/tree.py:164-171
 * builds it; row stride in bytes) into [N, ceil(N/64)] u64 words, bit j of
 * word w of row i = mask[i][64 w + j].
 */
int tm_tree_mask_pack(const uint8_t* mask, int64_t N, int64_t row_stride,
                      uint64_t* bits, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TREEMOE_AMD_H */
