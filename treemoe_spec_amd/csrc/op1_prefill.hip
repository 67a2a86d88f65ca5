// op1 expert GEMMs for many rows per expert (prefill / batched trees) on gfx950.
//
// When an expert receives hundreds of rows the layer is MFMA-bound, and the
// weight-streaming kernels (which re-read an expert's weights once per 64-row
// tile) are the wrong shape.  These kernels tile both operands:
//
//   workgroup = 8 waves (2 x 4) = 128 sorted rows x 256 weight rows, K in steps
//   of 64; each wave owns 64 x 64 outputs = 2 x 2 v_mfma_f32_32x32x16_bf16
//   tiles (on gfx950 the 32x32 form sustains ~2.2 PFLOP/s, the 16x16x32 form
//   ~1.3).  Operands go from global memory straight into LDS (16-byte buffer
//   loads with the LDS flag: lane i of a load lands at byte 16 i of its 1 KB
//   block, no registers involved), three stages deep: while the MFMAs of step k
//   run, steps k+1 and k+2 are in flight.  LDS rows are 128 B with the 16-byte
//   chunks XOR-swizzled (chunk c of row r stored at c ^ ((r >> 1) & 7)), which
//   the loads arrange by choosing each lane's source chunk; 16 consecutive rows
//   read at one logical chunk then hit 16 distinct 4-bank groups.
//
// Gate/up: B = 128 rows of w1 and the same 128 rows of w3, so each wave holds
// the gate and up sums of the same outputs and applies SwiGLU in registers; h
// is written row-major [sorted row, I] through an LDS-staged, coalesced store.
// Down: B = 256 rows of w2 over one K segment; the gate weight multiplies the
// fp32 sums before the (LDS-staged, coalesced) store of the partial y[segment].
//
// M-tiles are BM = 128 consecutive rows of one expert in the compact
// expert-major order (expert_offsets).  Launch order: workgroups are dealt
// to the 8 XCDs in turn, and each XCD owns one eighth of the column jobs for
// every M-tile, walked in super-blocks of 8 M-tiles x 4 columns (job_of).
#pragma clang fp contract(off)

#include "tm_common.h"

namespace {

constexpr int PBM = 128;                 // rows per M-tile
constexpr int PBN = 256;                 // weight rows per workgroup
constexpr int PBK = 64;                  // K per pipeline step (K = 32 with two workgroups per CU measured 8 % slower)
constexpr int NT = 512;                  // threads per workgroup (8 waves)
constexpr int PROW = PBK * 2;            // LDS row, bytes (PROW / 16 swizzled chunks)
constexpr int CPR = PROW / 16;           // 16-byte chunks per row
constexpr int RPB = 256 / PROW;          // rows per 256 B (one pass over the 64 banks)
constexpr int RPK = 1024 / PROW;         // rows per 1 KB load block
constexpr int ABYTES = PBM * PROW;       // A tile of one step
constexpr int BBYTES = PBN * PROW;       // B tile of one step
constexpr int STAGE = ABYTES + BBYTES;   // three stages in LDS
constexpr int ALD = ABYTES / (NT * 16);  // 16-byte loads per thread per step: A
constexpr int BLD = BBYTES / (NT * 16);  //                                   B
constexpr int LDS_PER_STEP = ALD + BLD;
static_assert(ALD >= 1 && BLD >= 1 && CPR >= 4, "tile shape");
constexpr uint32_t kOOR = 0x80000000u;   // out-of-range buffer offset: loads 0

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pbuf(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
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

// Byte offset in a swizzled tile of logical chunk c (16 B) of row r: chunk c
// is stored at c ^ ((r / RPB) % CPR), so 16 consecutive rows read at one
// logical chunk cover 16 distinct 4-bank groups.
__device__ __forceinline__ int swz(int r, int c) {
  return r * PROW + ((c ^ ((r / RPB) & (CPR - 1))) << 4);
}

constexpr int kXcds = 8;  // workgroup i runs on XCD i % 8
constexpr int SBM = 8;    // super-block: M-tile slots (consecutive: mostly one expert) ..
constexpr int SBN = 4;    // .. x column jobs, M fastest

// Job of launch index L: M-tile slot and column job (either may be padding,
// which the kernels skip).  XCD x = L % 8 owns the column jobs
// [x * cpx, (x + 1) * cpx) for every M-tile slot, so each weight block is read
// through one XCD's L2 only, and walks them in SBM x SBN super-blocks: the
// ~32 workgroups resident on the XCD share each A tile across SBN columns and
// each weight block across the M-tiles of one expert.
__device__ __forceinline__ void job_of(int L, int mt_max, int ncol, int* mt, int* col) {
  const int x = L % kXcds, l = L / kXcds;
  const int cpx = (ncol + kXcds - 1) / kXcds;
  const int nsm = (mt_max + SBM - 1) / SBM;
  const int sb = l / (SBM * SBN), w = l - sb * (SBM * SBN);
  const int sbm = sb % nsm, sbn = sb / nsm;
  *mt = sbm * SBM + w % SBM;
  const int lc = sbn * SBN + w / SBM;  // column within the XCD's range
  *col = lc < cpx ? x * cpx + lc : ncol;
}

// Launch size: 8 XCDs x every (M-tile slot, column) pair of one XCD's range.
int64_t launch_jobs(int64_t mt_max, int64_t ncol) {
  const int64_t cpx = (ncol + kXcds - 1) / kXcds;
  return kXcds * ((mt_max + SBM - 1) / SBM) * ((cpx + SBN - 1) / SBN) * SBM * SBN;
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

// Global -> LDS: load i of a thread moves one 16-byte chunk.  Load i of wave
// w fills the 1 KB block 8 i + w of its tile (RPK rows); lane l writes byte
// 16 l of the block, i.e. row RPK (8 i + w) + l / CPR at stored chunk
// l % CPR, so it fetches the logical chunk that the swizzle stores there.
struct DmaLoad {
  __amdgpu_buffer_rsrc_t ra, rb[BLD];
  uint32_t aoff[ALD];  // byte offset of the chunk at k = 0, or kOOR
  uint32_t boff[BLD];
};

// Row of load i for this thread, and the logical chunk it fetches.
__device__ __forceinline__ int dma_row(int i) {
  return RPK * (8 * i + (threadIdx.x >> 6)) + ((threadIdx.x & 63) / CPR);
}
__device__ __forceinline__ int dma_chunk(int row) {
  return (threadIdx.x & (CPR - 1)) ^ ((row / RPB) & (CPR - 1));
}

// Load j (0 .. LDS_PER_STEP - 1: the A loads, then the B loads) of step
// `kstep` (K bytes 128 kstep ..) of both tiles into `st`; past the end of K
// the loads are out of range and store zeros.  Every step issues all
// LDS_PER_STEP loads in this order, so the wait counts below stay exact.
__device__ __forceinline__ void dma_one(const DmaLoad& d, uint8_t* st, int kstep, int nk, int j) {
  const uint32_t kb = (uint32_t)kstep * (uint32_t)PROW;
  const bool valid = kstep < nk;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // LDS base: wave-uniform
  if (j < ALD) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        d.ra, (lds_void*)(st + (8 * j + w) * 1024), 16,
        (valid && d.aoff[j] != kOOR) ? d.aoff[j] + kb : kOOR, 0, 0, 0);
  } else {
    const int i = j - ALD;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        d.rb[i], (lds_void*)(st + ABYTES + (8 * i + w) * 1024), 16,
        valid ? d.boff[i] + kb : kOOR, 0, 0, 0);
  }
}

__device__ __forceinline__ void dma_step(const DmaLoad& d, uint8_t* st, int kstep, int nk) {
#pragma unroll
  for (int j = 0; j < LDS_PER_STEP; ++j) dma_one(d, st, kstep, nk, j);
}

// Wait until at most n of this thread's vector-memory operations are
// outstanding (s_waitcnt vmcnt(n); the other counters are left alone).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Fragment of 32 rows starting at `row`, k-step s (16 columns): lane l reads
// row l % 32, logical chunk 2 s + l / 32.
__device__ __forceinline__ u32x4_t frag(const uint8_t* tile, int row, int s, int lane) {
  return *reinterpret_cast<const u32x4_t*>(tile + swz(row + (lane & 31), 2 * s + (lane >> 5)));
}

// acc[i][j] += A[64 wm + 32 i, :] B[brow[j], :]^T over one staged step.
// (Spreading the next step's loads between this step's MFMAs instead of
// issuing them before it measured no faster.)
__device__ __forceinline__ void compute_step(const uint8_t* st, const int (&brow)[2],
                                             f32x16_t (&acc)[2][2]) {
  const int lane = threadIdx.x & 63;
  const int wm = (threadIdx.x >> 6) & 1;
#pragma unroll
  for (int s = 0; s < PBK / 16; ++s) {
    u32x4_t a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) a[i] = frag(st, 64 * wm + 32 * i, s, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = frag(st + ABYTES, brow[j], s, lane);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = pmfma(a[i], b[j], acc[i][j]);
  }
}

// The K loop shared by both GEMMs over nk steps, three LDS stages (three
// distinct arrays, used in a fixed rotation, so the compiler can tell the
// stage being read from the ones being loaded).  At the top of step k, steps
// k and k+1 are in flight; the thread waits for its loads of step k, the
// barrier makes every thread's loads visible and frees the stage of step k-1,
// step k+2 goes into that stage, then step k's MFMAs run.
struct Stages {
  uint8_t* s0;
  uint8_t* s1;
  uint8_t* s2;
};

__device__ __forceinline__ void k_loop(const Stages& sb, const DmaLoad& d, int nk,
                                       const int (&brow)[2], f32x16_t (&acc)[2][2]) {
  dma_step(d, sb.s0, 0, nk);
  dma_step(d, sb.s1, 1, nk);
  // The barrier waits for this wave's LDS reads only (tm_lds_barrier), not
  // for its outstanding loads: the loads of the next steps stay in flight.
  for (int k = 0; k < nk; k += 3) {
    wait_vm<LDS_PER_STEP>();
    tm_lds_barrier();
    dma_step(d, sb.s2, k + 2, nk);
    compute_step(sb.s0, brow, acc);
    wait_vm<LDS_PER_STEP>();
    tm_lds_barrier();
    dma_step(d, sb.s0, k + 3, nk);
    if (k + 1 < nk) compute_step(sb.s1, brow, acc);
    wait_vm<LDS_PER_STEP>();
    tm_lds_barrier();
    dma_step(d, sb.s1, k + 4, nk);
    if (k + 2 < nk) compute_step(sb.s2, brow, acc);
  }
  // the last loads (zeros past the end) must land before the stages are reused
  wait_vm<0>();
  __syncthreads();
}

// ------------------------------------------------------------- gate/up --
// h[p, n] = bf16( silu(x[tok(p)] . w1[e, n]) * (x[tok(p)] . w3[e, n]) ) for the
// rows p of one M-tile and the 128 columns n of one column block.
constexpr int HSTRIDE = 128 * 2 + 16;  // bf16 output staging row stride, bytes
static_assert(PBM * HSTRIDE <= STAGE, "h staging fits in one stage");

__global__ void __launch_bounds__(NT)
tm_prefill_gemm1_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                        const uint16_t* __restrict__ w3, uint16_t* __restrict__ h,
                        const int32_t* __restrict__ sorted_slots,
                        const int32_t* __restrict__ offsets, const int32_t* __restrict__ tiles,
                        int max_tiles, int E, int H, int I, int mt_max, uint32_t x_bytes) {
  __shared__ __attribute__((aligned(16))) uint8_t s0[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s1[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s2[STAGE];
  int mt, cb;
  const int ncol = I / (PBN / 2);
  job_of((int)blockIdx.x, mt_max, ncol, &mt, &cb);
  int e, p0, rows;
  if (mt >= mt_max || cb >= ncol) return;
  if (!find_mtile(offsets, tiles, max_tiles, E, mt, &e, &p0, &rows)) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;
  const int n0 = cb * (PBN / 2);  // first h column of the block

  DmaLoad d;
  d.ra = pbuf(x, x_bytes);
  const size_t ebase = (size_t)e * I * H;
  const __amdgpu_buffer_rsrc_t r1 = pbuf(w1 + ebase, (uint32_t)((size_t)I * H * 2));
  const __amdgpu_buffer_rsrc_t r3 = pbuf(w3 + ebase, (uint32_t)((size_t)I * H * 2));
#pragma unroll
  for (int i = 0; i < ALD; ++i) {
    const int r = dma_row(i);
    d.aoff[i] = r < rows ? (uint32_t)(sorted_slots[p0 + r] >> 1) * (uint32_t)H * 2u +
                               (uint32_t)dma_chunk(r) * 16u
                         : kOOR;
  }
#pragma unroll
  for (int i = 0; i < BLD; ++i) {
    const int r = dma_row(i);  // loads 0, 1: B rows 0..127 (w1); 2, 3: 128..255 (w3, same n)
    d.rb[i] = i < BLD / 2 ? r1 : r3;
    static_assert(BLD % 2 == 0, "w1 and w3 loads split evenly");
    d.boff[i] = (uint32_t)(n0 + (r & (PBN / 2 - 1))) * (uint32_t)H * 2u + (uint32_t)dma_chunk(r) * 16u;
  }
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  // accumulator column blocks: j = 0 -> w1 rows 32 wn ..; j = 1 -> the same w3 rows
  const int brow[2] = {32 * wn, PBN / 2 + 32 * wn};
  k_loop(Stages{s0, s1, s2}, d, H / PBK, brow, acc);

  // SwiGLU in registers, bf16 tile [128 rows][128 columns] in LDS, coalesced store
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float a = acc[i][0][v];
      const float b = acc[i][1][v];
      const float hv = (a / (1.0f + __expf(-a))) * b;
      const int m = 64 * wm + 32 * i + acc_row(v, lane);
      const int c = 32 * wn + (lane & 31);
      *reinterpret_cast<uint16_t*>(s0 + m * HSTRIDE + c * 2) = tm_f32_to_bf16(hv);
    }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PBM * 16 / NT; ++j) {
    const int piece = tid + NT * j;  // 128 rows x 16 pieces of 16 B
    const int r = piece >> 4, c16 = piece & 15;
    if (r < rows) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(s0 + r * HSTRIDE + c16 * 16);
      *reinterpret_cast<u32x4_t*>(h + (size_t)(p0 + r) * I + n0 + c16 * 8) = v;
    }
  }
}

// ---------------------------------------------------------------- down --
// y[s, p, n] = gates_flat[slot(p)] * sum_{k in segment s} h[p, k] w2[e, n, k]
// for the rows p of one M-tile and 256 output columns n.  The fp32 partials
// go straight from the accumulators: for each accumulator value, 32 lanes
// store 128 contiguous bytes of one row.
__global__ void __launch_bounds__(NT)
tm_prefill_gemm2_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ w2,
                        float* __restrict__ y, const float* __restrict__ gates_flat,
                        const int32_t* __restrict__ sorted_slots,
                        const int32_t* __restrict__ offsets, const int32_t* __restrict__ tiles,
                        int max_tiles, int E, int R, int H, int I, int klen, int nsplit,
                        int mt_max, uint32_t h_bytes) {
  __shared__ __attribute__((aligned(16))) uint8_t s0[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s1[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s2[STAGE];
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

  DmaLoad d;
  d.ra = pbuf(h, h_bytes);
  const __amdgpu_buffer_rsrc_t wr = pbuf(w2 + (size_t)e * H * I, (uint32_t)((size_t)H * I * 2));
#pragma unroll
  for (int i = 0; i < ALD; ++i) {
    const int r = dma_row(i);
    d.aoff[i] = r < rows ? (uint32_t)(p0 + r) * (uint32_t)I * 2u + k0 + (uint32_t)dma_chunk(r) * 16u
                         : kOOR;
  }
#pragma unroll
  for (int i = 0; i < BLD; ++i) {
    const int r = dma_row(i);
    d.rb[i] = wr;
    d.boff[i] = (uint32_t)(n0 + r) * (uint32_t)I * 2u + k0 + (uint32_t)dma_chunk(r) * 16u;
  }
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  const int brow[2] = {64 * wn, 64 * wn + 32};
  k_loop(Stages{s0, s1, s2}, d, klen / PBK, brow, acc);

  float* ys = y + (size_t)seg * R * H;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = 64 * wm + 32 * i + acc_row(v, lane);
      if (m < rows) {
        const float gate = gates_flat[sorted_slots[p0 + m]];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int c = 64 * wn + 32 * j + (lane & 31);
          ys[(size_t)(p0 + m) * H + n0 + c] = acc[i][j][v] * gate;
        }
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
  hipLaunchKernelGGL(tm_prefill_gemm1_kernel, dim3((unsigned)jobs), dim3(NT), 0,
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
  hipLaunchKernelGGL(tm_prefill_gemm2_kernel, dim3((unsigned)jobs), dim3(NT), 0,
                     (hipStream_t)stream, (const uint16_t*)h, (const uint16_t*)w2, y, gates_flat,
                     sorted_slots, expert_offsets, tiles, (int)max_tiles, (int)E, (int)(2 * T),
                     (int)H, (int)I, (int)klen, (int)split, (int)mt_max,
                     (uint32_t)(2 * T * I * 2));
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}
