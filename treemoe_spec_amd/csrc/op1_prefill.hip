// op1 expert GEMMs for many rows per expert (prefill / batched trees) on gfx950.
//
// When an expert receives hundreds of rows the layer is MFMA-bound, and the
// weight-streaming kernels (which re-read an expert's weights once per 64-row
// tile) are the wrong shape.  These kernels tile both operands:
//
//   workgroup = 4 waves (2 x 2) = 128 sorted rows x 128 weight rows, K in steps
//   of 64; each wave owns 64 x 64 outputs = 2 x 2 v_mfma_f32_32x32x16_bf16
//   tiles (on gfx950 the 32x32 form sustains ~2.2 PFLOP/s, the 16x16x32 form
//   ~1.3).  A (activation rows) and B (weight rows) stage through LDS (rows
//   padded to 144 B: conflict-free fragment reads), double-buffered, with the
//   global loads of step k+2 issued before the MFMAs of step k.
//
// Gate/up: B = 64 rows of w1 and the same 64 rows of w3, so each wave holds
// the gate and up sums of the same outputs and applies SwiGLU in registers; h
// is written row-major [sorted row, I] through an LDS-staged, coalesced store.
// Down: B = 128 rows of w2 over one K segment; the gate weight multiplies the
// fp32 sums before the (LDS-staged, coalesced) store of the partial y[segment].
//
// M-tiles are BM = 128 consecutive rows of one expert in the compact
// expert-major order (expert_offsets).  Launch order: jobs (M-tile, column
// block) in 8 x 8 super-blocks, M-tile fastest.  Workgroups are dealt to the
// 8 XCDs in turn, so within a super-block each XCD takes one M-tile across 8
// column blocks (its A rows come from that XCD's L2) while the 8 XCDs share
// the same weight blocks through the Infinity Cache.  (Remapping launch
// indices so that one XCD holds a whole super-block raised the L2 hit rate
// but measured 10 % slower.)
#pragma clang fp contract(off)

#include "tm_common.h"

namespace {

constexpr int PBM = 128;                 // rows per M-tile
constexpr int PBN = 128;                 // weight rows per workgroup
constexpr int PBK = 64;                  // K per pipeline step
constexpr int PSTRIDE = PBK * 2 + 16;    // LDS row stride, bytes
constexpr int PTILE = 128 * PSTRIDE;     // one 128-row operand tile
constexpr int PSTAGE = 2 * PTILE;        // A + B
constexpr int PLDS = 2 * PSTAGE;         // double buffer (73,728 B)
constexpr uint32_t kOOR = 0x80000000u;   // out-of-range buffer offset: loads 0

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pbuf(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

template <int AUX>
__device__ __forceinline__ u32x4_t pld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// 32x32x16 bf16 MFMA.  Lane l: A row l % 32 and B column l % 32, k 8 (l / 32)
// .. +7; accumulator value v is C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32].
__device__ __forceinline__ f32x16_t pmfma(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ int acc_row(int v, int lane) {
  return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}

constexpr int SB = 8;  // super-block edge, in jobs

// Job of launch index i: M-tile slot and column job (both may be padding).
__device__ __forceinline__ void job_of(int L, int mt_max, int ncol, int* mt, int* col) {
  const int nmb = (mt_max + SB - 1) / SB;
  const int sb = L / (SB * SB), w = L - sb * (SB * SB);
  const int sbm = sb % nmb, sbc = sb / nmb;
  *mt = sbm * SB + (w % SB);
  *col = sbc * SB + (w / SB);
}

// Launch size covering every (M-tile slot, column job) pair in super-blocks.
int64_t launch_jobs(int64_t mt_max, int64_t ncol) {
  return ((mt_max + SB - 1) / SB) * ((ncol + SB - 1) / SB) * SB * SB;
}

// M-tile `idx` of the compact expert-major order: expert, first row, rows.
// An expert whose first entry in the 64-row tile list is masked (expert -1,
// as Routing.exclude_experts leaves it) is skipped, like the weight-streaming
// kernels skip its tiles.
__device__ __forceinline__ bool find_mtile(const int32_t* __restrict__ offsets,
                                           const int32_t* __restrict__ tiles, int max_tiles,
                                           int E, int idx, int* e, int* p0, int* rows) {
  int acc = 0, tile64 = 0;
  for (int k = 0; k < E; ++k) {
    const int o = offsets[k];
    const int cnt = offsets[k + 1] - o;
    const int nt = (cnt + PBM - 1) / PBM;
    if (idx < acc + nt) {
      if (tile64 >= max_tiles || tiles[4 * tile64] != k) return false;
      const int m0 = (idx - acc) * PBM;
      *e = k;
      *p0 = o + m0;
      *rows = min(PBM, cnt - m0);
      return true;
    }
    acc += nt;
    tile64 += (cnt + TM_GEMM_TILE_M - 1) / TM_GEMM_TILE_M;
  }
  return false;
}

// Global -> LDS mapping of one 128-row x 64-column bf16 operand tile: thread t
// moves 16-byte pieces c = t + 256 i (i < 4): row c / 8, bytes 16 (c % 8).
struct TileLoad {
  __amdgpu_buffer_rsrc_t rsrc[4];
  uint32_t off[4];  // byte offset of the piece at k = 0, or kOOR
};

// Operands are re-read by other workgroups from L2 and the Infinity Cache, so
// the loads use the default (temporal) cache policy.  A step past the end of K
// loads zeros out of range, without a branch: the wait counts stay exact.
__device__ __forceinline__ void load_tile(const TileLoad& t, uint32_t kb, bool valid,
                                          u32x4_t (&v)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    v[i] = pld<0>(t.rsrc[i], (valid && t.off[i] != kOOR) ? t.off[i] + kb : kOOR);
}

__device__ __forceinline__ void store_tile(uint8_t* tile, const u32x4_t (&v)[4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<u32x4_t*>(tile + ((t >> 3) + 32 * i) * PSTRIDE + (t & 7) * 16) = v[i];
}

// Fragment of 32 rows starting at `row`, k-step s (16 columns): lane l reads
// row l % 32, columns 16 s + 8 (l / 32) .. +7.
__device__ __forceinline__ u32x4_t frag(const uint8_t* tile, int row, int s, int lane) {
  return *reinterpret_cast<const u32x4_t*>(tile + (row + (lane & 31)) * PSTRIDE + s * 32 +
                                           (lane >> 5) * 16);
}

// The K loop shared by both GEMMs: acc[i][j] += A[64 wm + 32 i, :] B[brow[j], :]^T
// (32 x 32 blocks) over K = nk * 64.  The loop body has no branches (the wait
// counts stay exact): an odd nk runs one extra step of zeros.  (A third
// register set, loads three steps ahead, measured slower.)
__device__ __forceinline__ void k_loop(uint8_t* lds, const TileLoad& la, const TileLoad& lb,
                                       int nk, const int (&brow)[2], f32x16_t (&acc)[2][2]) {
  const int lane = threadIdx.x & 63;
  const int wm = (threadIdx.x >> 6) & 1;
  u32x4_t ra0[4], rb0[4], ra1[4], rb1[4];
  load_tile(la, 0, true, ra0);
  load_tile(lb, 0, true, rb0);
  load_tile(la, PBK * 2, nk > 1, ra1);
  load_tile(lb, PBK * 2, nk > 1, rb1);
  store_tile(lds, ra0);
  store_tile(lds + PTILE, rb0);
  __syncthreads();

  auto compute = [&](const uint8_t* st) {
#pragma unroll
    for (int s = 0; s < PBK / 16; ++s) {
      u32x4_t a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = frag(st, 64 * wm + 32 * i, s, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = frag(st + PTILE, brow[j], s, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = pmfma(a[i], b[j], acc[i][j]);
    }
  };
  // step k: LDS buffer k % 2 holds step k; (na, nb) hold step k + 1 in
  // flight; step k + 2 goes into (fa, fb), the set step k came in.
  auto step = [&](int k, u32x4_t (&fa)[4], u32x4_t (&fb)[4], u32x4_t (&na)[4],
                  u32x4_t (&nb)[4], uint8_t* cur, uint8_t* nxt) {
    load_tile(la, (uint32_t)(k + 2) * PBK * 2, k + 2 < nk, fa);
    load_tile(lb, (uint32_t)(k + 2) * PBK * 2, k + 2 < nk, fb);
    __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
    compute(cur);
    store_tile(nxt, na);
    store_tile(nxt + PTILE, nb);
    __syncthreads();
  };
  for (int k = 0; k < nk; k += 2) {
    step(k, ra0, rb0, ra1, rb1, lds, lds + PSTAGE);
    step(k + 1, ra1, rb1, ra0, rb0, lds + PSTAGE, lds);
  }
}

// ------------------------------------------------------------- gate/up --
// h[p, n] = bf16( silu(x[tok(p)] . w1[e, n]) * (x[tok(p)] . w3[e, n]) ) for the
// rows p of one M-tile and the 64 columns n of one column block.
__global__ void __launch_bounds__(256, 2)
tm_prefill_gemm1_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                        const uint16_t* __restrict__ w3, uint16_t* __restrict__ h,
                        const int32_t* __restrict__ sorted_slots,
                        const int32_t* __restrict__ offsets, const int32_t* __restrict__ tiles,
                        int max_tiles, int E, int H, int I, int mt_max, uint32_t x_bytes) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[PLDS];
  int mt, cb;
  job_of((int)blockIdx.x, mt_max, I / (PBN / 2), &mt, &cb);
  int e, p0, rows;
  if (mt >= mt_max || cb >= I / (PBN / 2)) return;
  if (!find_mtile(offsets, tiles, max_tiles, E, mt, &e, &p0, &rows)) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;
  const int n0 = cb * (PBN / 2);  // first h column of the block

  TileLoad la, lb;
  const __amdgpu_buffer_rsrc_t xr = pbuf(x, x_bytes);
  const size_t ebase = (size_t)e * I * H;
  const __amdgpu_buffer_rsrc_t r1 = pbuf(w1 + ebase, (uint32_t)((size_t)I * H * 2));
  const __amdgpu_buffer_rsrc_t r3 = pbuf(w3 + ebase, (uint32_t)((size_t)I * H * 2));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid >> 3) + 32 * i;
    la.rsrc[i] = xr;
    la.off[i] = r < rows ? (uint32_t)(sorted_slots[p0 + r] >> 1) * (uint32_t)H * 2u + (tid & 7) * 16u
                         : kOOR;
    lb.rsrc[i] = i < 2 ? r1 : r3;  // B rows 0..63: w1, 64..127: w3 (same n)
    lb.off[i] = (uint32_t)(n0 + (r & 63)) * (uint32_t)H * 2u + (tid & 7) * 16u;
  }
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  // accumulator column blocks: j = 0 -> w1 rows 32 wn ..; j = 1 -> the same w3 rows
  const int brow[2] = {32 * wn, 64 + 32 * wn};
  k_loop(lds, la, lb, H / PBK, brow, acc);

  // SwiGLU in registers, bf16 tile [128 rows][64 columns] in LDS, coalesced store
  uint8_t* st = lds;  // row stride PSTRIDE (= 64 bf16 + 16 B)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float a = acc[i][0][v];
      const float b = acc[i][1][v];
      const float hv = (a / (1.0f + __expf(-a))) * b;
      const int m = 64 * wm + 32 * i + acc_row(v, lane);
      const int c = 32 * wn + (lane & 31);
      *reinterpret_cast<uint16_t*>(st + m * PSTRIDE + c * 2) = tm_f32_to_bf16(hv);
    }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid >> 3) + 32 * i;
    if (r < rows) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(st + r * PSTRIDE + (tid & 7) * 16);
      *reinterpret_cast<u32x4_t*>(h + (size_t)(p0 + r) * I + n0 + (tid & 7) * 8) = v;
    }
  }
}

// ---------------------------------------------------------------- down --
// y[s, p, n] = gates_flat[slot(p)] * sum_{k in segment s} h[p, k] w2[e, n, k]
// for the rows p of one M-tile and 128 output columns n.
constexpr int YSTRIDE = PBN * 4 + 16;  // fp32 output staging row stride, bytes
static_assert(128 * YSTRIDE <= PLDS, "output staging fits in the operand buffers");

__global__ void __launch_bounds__(256, 2)
tm_prefill_gemm2_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ w2,
                        float* __restrict__ y, const float* __restrict__ gates_flat,
                        const int32_t* __restrict__ sorted_slots,
                        const int32_t* __restrict__ offsets, const int32_t* __restrict__ tiles,
                        int max_tiles, int E, int R, int H, int I, int klen, int nsplit,
                        int mt_max, uint32_t h_bytes) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[PLDS];
  int mt, job;  // job = (column block, segment)
  const int ncol = (H / PBN) * nsplit;
  job_of((int)blockIdx.x, mt_max, ncol, &mt, &job);
  if (mt >= mt_max || job >= ncol) return;
  const int cb = job / nsplit;
  const int seg = job - cb * nsplit;
  int e, p0, rows;
  if (!find_mtile(offsets, tiles, max_tiles, E, mt, &e, &p0, &rows)) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;
  const int n0 = cb * PBN;
  const uint32_t k0 = (uint32_t)seg * (uint32_t)klen * 2u;  // segment start, bytes

  TileLoad la, lb;
  const __amdgpu_buffer_rsrc_t hr = pbuf(h, h_bytes);
  const __amdgpu_buffer_rsrc_t wr = pbuf(w2 + (size_t)e * H * I, (uint32_t)((size_t)H * I * 2));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid >> 3) + 32 * i;
    la.rsrc[i] = hr;
    la.off[i] = r < rows ? (uint32_t)(p0 + r) * (uint32_t)I * 2u + k0 + (tid & 7) * 16u : kOOR;
    lb.rsrc[i] = wr;
    lb.off[i] = (uint32_t)(n0 + r) * (uint32_t)I * 2u + k0 + (tid & 7) * 16u;
  }
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  const int brow[2] = {64 * wn, 64 * wn + 32};
  k_loop(lds, la, lb, klen / PBK, brow, acc);

  // gate multiply in fp32, fp32 tile [128 rows][128 columns] in LDS, coalesced store
  uint8_t* st = lds;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = 64 * wm + 32 * i + acc_row(v, lane);
      const float gate = m < rows ? gates_flat[sorted_slots[p0 + m]] : 0.0f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = 64 * wn + 32 * j + (lane & 31);
        *reinterpret_cast<float*>(st + m * YSTRIDE + c * 4) = acc[i][j][v] * gate;
      }
    }
  __syncthreads();
  float* ys = y + (size_t)seg * R * H;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int piece = tid + 256 * i;  // 128 rows x 32 pieces of 16 B
    const int r = piece >> 5, c4 = piece & 31;
    if (r < rows) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(st + r * YSTRIDE + c4 * 16);
      *reinterpret_cast<u32x4_t*>(ys + (size_t)(p0 + r) * H + n0 + c4 * 4) = v;
    }
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

// Upper bound of the M-tiles over E experts holding `slots` rows.
int64_t mtile_bound(int64_t slots, int64_t E) { return (slots + PBM - 1) / PBM + E; }

}  // namespace

extern "C" int tm_op1_prefill_gemm1(const void* x, const void* w1, const void* w3, void* h,
                                    const int32_t* sorted_slots, const int32_t* expert_offsets,
                                    const int32_t* tiles, int64_t max_tiles, int64_t T,
                                    int64_t H, int64_t I, int64_t E, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS || max_tiles < 1)
    return TM_ERR_SHAPE;
  if (H < PBK || (H % PBK) != 0 || I < PBN / 2 || (I % (PBN / 2)) != 0) return TM_ERR_SHAPE;
  if (I * H * 2 >= (int64_t)kOOR || T * H * 2 >= (int64_t)kOOR || 2 * T * I * 2 >= (int64_t)kOOR)
    return TM_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w1) || !aligned16(w3) || !aligned16(h)) return TM_ERR_ALIGN;
  const int64_t mt_max = mtile_bound(2 * T, E);
  const int64_t jobs = launch_jobs(mt_max, I / (PBN / 2));
  if (jobs > INT32_MAX) return TM_ERR_SHAPE;
  hipLaunchKernelGGL(tm_prefill_gemm1_kernel, dim3((unsigned)jobs), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)x, (const uint16_t*)w1,
                     (const uint16_t*)w3, (uint16_t*)h, sorted_slots, expert_offsets, tiles,
                     (int)max_tiles, (int)E, (int)H, (int)I, (int)mt_max,
                     (uint32_t)(T * H * 2));
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op1_prefill_gemm2(const void* h, const void* w2, float* y,
                                    const float* gates_flat, const int32_t* sorted_slots,
                                    const int32_t* expert_offsets, const int32_t* tiles,
                                    int64_t max_tiles, int64_t split, int64_t T, int64_t H,
                                    int64_t I, int64_t E, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS || max_tiles < 1)
    return TM_ERR_SHAPE;
  if (split < 1 || (I % split) != 0) return TM_ERR_SHAPE;
  const int64_t klen = I / split;
  if (klen < PBK || (klen % PBK) != 0 || H < PBN || (H % PBN) != 0) return TM_ERR_SHAPE;
  if (H * I * 2 >= (int64_t)kOOR || 2 * T * I * 2 >= (int64_t)kOOR) return TM_ERR_SHAPE;
  if (!aligned16(h) || !aligned16(w2) || !aligned16(y)) return TM_ERR_ALIGN;
  const int64_t mt_max = mtile_bound(2 * T, E);
  const int64_t jobs = launch_jobs(mt_max, (H / PBN) * split);
  if (jobs > INT32_MAX) return TM_ERR_SHAPE;
  hipLaunchKernelGGL(tm_prefill_gemm2_kernel, dim3((unsigned)jobs), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)h, (const uint16_t*)w2, y, gates_flat,
                     sorted_slots, expert_offsets, tiles, (int)max_tiles, (int)E, (int)(2 * T),
                     (int)H, (int)I, (int)klen, (int)split, (int)mt_max,
                     (uint32_t)(2 * T * I * 2));
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}
