// op1 expert GEMMs for many rows per expert (prefill / batched trees) on gfx950.
//
// When an expert receives tens to thousands of rows the weight-streaming
// kernels (which re-read an expert's weights once per 64-row tile) are the
// wrong shape.  These kernels tile both operands:
//
//   workgroup = NW waves (2 row halves x NW / 2 column groups) = BM sorted rows
//   x 32 NW weight rows; each wave owns BM/2 x 64 outputs = (BM/64) x 2
//   v_mfma_f32_32x32x16_bf16 tiles (on gfx950 the 32x32 form sustains ~2.2
//   PFLOP/s, the 16x16x32 form ~1.3).
//   Operands go from global memory straight into LDS (16-byte buffer loads
//   with the LDS flag: lane i of a load lands at byte 16 i of its 1 KB block,
//   no registers involved), NS stages deep: while the MFMAs of step k run,
//   steps k+1 .. k+NS-1 are in flight.  LDS rows hold one K step (2 BK bytes)
//   with the 16-byte chunks XOR-swizzled (swz), which the loads arrange by
//   choosing each lane's source chunk; 16 consecutive rows read at one
//   logical chunk then hit 16 distinct 4-bank groups.
//
// Three tile configurations, all 8 waves x 256 weight rows but the last:
// BM = 128 with K steps of 64 and three 48 KB stages; BM = 256 with K steps
// of 32 and four 32 KB stages (fewer operand bytes per flop, larger jobs);
// BM = 64 with K steps of 64 against 128 weight rows on 4 waves, three 24 KB
// stages, so two workgroups share a CU.  Down always uses the first; gate/up
// uses the second when the experts average 384 rows or more and the third
// when the tile list leaves at most 16 rows per entry.  A tile whose M-tile
// holds fewer than BM real rows runs the MFMAs of the 64-row parts that hold
// them only.  Where the MFMAs bound the kernel (the 256-row gate/up tile, and
// the down GEMM when the experts average 384 rows or more) the two 4-wave
// halves of a workgroup run the K loop half a step apart (k_loop_pp), so one
// wave per SIMD issues MFMAs while the other reads its fragments (config 5,
// same box: gate/up 1045 -> 990 us, down 576 -> 558 us, bit-identical).
//
// Gate/up: B = 128 rows of w1 and the same 128 rows of w3 (64 and 64 in the
// 4-wave tile), so each wave holds the gate and up sums of the same outputs
// and applies SwiGLU in registers; h is written row-major [sorted row, I]
// through an LDS-staged, coalesced store.
// Down: B = 256 rows of w2 over one K segment; the gate weight multiplies the
// fp32 sums before the store of the partial y[segment].
//
// M-tiles are BM consecutive rows of one expert in the compact expert-major
// order (expert_offsets).  Launch order: workgroups are dealt to the 8 XCDs
// in turn, and each XCD owns one eighth of the column jobs for every M-tile,
// walked expert by expert, M fastest, when the experts average two M-tiles
// or more, else in super-blocks of 8 M-tiles x 4 columns (expert_job; the
// self-routed decode gate/up always takes the super-blocks, job_of).
#pragma clang fp contract(off)

#include <algorithm>

#include "op1_bucket.h"
#include "tm_common.h"

namespace {

constexpr uint32_t kOOR = 0x80000000u;   // out-of-range buffer offset: loads 0

// Tile configuration: BM sorted rows per M-tile, K steps of BK, NS stages,
// BN weight rows per workgroup, NTH threads (NTH / 64 waves as 2 row halves x
// NTH / 128 column groups of 32 outputs, so BN = 32 x waves).
template <int BM, int BK, int NS, int BN = 256, int NTH = 512, bool PINGPONG = false>
struct Tile {
  // the two wave halves run the K loop half a step apart (k_loop_pp)
  static constexpr bool PP = PINGPONG;
  static constexpr int PBM = BM;
  static constexpr int PBK = BK;
  static constexpr int NSTAGE = NS;
  static constexpr int PBN = BN;                  // weight rows per workgroup
  static constexpr int NT = NTH;                  // threads per workgroup
  static constexpr int NW = NTH / 64;             // waves
  static constexpr int PROW = PBK * 2;            // LDS row, bytes (PROW / 16 swizzled chunks)
  static constexpr int CPR = PROW / 16;           // 16-byte chunks per row
  static constexpr int RPB = 256 / PROW;          // rows per 256 B (one pass over the 64 banks)
  static constexpr int RPK = 1024 / PROW;         // rows per 1 KB load block
  static constexpr int ABYTES = PBM * PROW;       // A tile of one step
  static constexpr int BBYTES = PBN * PROW;       // B tile of one step
  static constexpr int STAGE = ABYTES + BBYTES;   // one stage in LDS
  static constexpr int ALD = ABYTES / (NT * 16);  // 16-byte loads per thread per step: A
  static constexpr int BLD = BBYTES / (NT * 16);  //                                   B
  static constexpr int LDS_PER_STEP = ALD + BLD;
  static constexpr int MT = PBM / 64;             // 32-row accumulator tiles per wave
  // weight loads of an expert with a single M-tile go non-temporal (below)
  // for tiles of at most 128 rows; the 256-row gate/up tile runs where most
  // experts take several M-tiles, and there the policy measured slower
  static constexpr bool NT_WEIGHTS = BM <= 128;
  // bf16 h staging: rows of PBN / 2 columns, padded by 16 bytes; rows per
  // stage: the whole tile in one stage when it fits
  static constexpr int HSTRIDE = PBN + 16;
  static constexpr int HROWS = PBM * HSTRIDE <= STAGE ? PBM : PBM / NSTAGE;
  static_assert(ALD >= 1 && BLD >= 1 && BLD % 2 == 0 && CPR >= 4, "tile shape");
  static_assert(PBN == 32 * NW && (NW == 4 || NW == 8), "wave layout");
  static_assert(NS == 3 || NS == 4, "stage rotation");
  static_assert(HROWS * HSTRIDE <= STAGE && (PBM + HROWS - 1) / HROWS <= NS, "h staging");
  static_assert(NS * STAGE <= 160 * 1024, "LDS");
  static_assert(!PINGPONG || NTH == 512, "ping-pong: two halves of four waves");
};
using Tile128 = Tile<128, 64, 3>;
using Tile256 = Tile<256, 32, 4, 256, 512, true>;
// The down GEMM's tile where the experts average many rows (MFMA-bound).
using Tile128PP = Tile<128, 64, 3, 256, 512, true>;
// Few rows per expert: 64-row M-tiles against 128 weight rows with 4 waves,
// 72 KB of LDS, so two workgroups share a CU.  Same per-output K order as
// Tile128, so the same bits.
using TileDec = Tile<64, 64, 3, 128, 256>;

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pbuf(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// 32x32x16 bf16 MFMA.  Lane l: A row l % 32 and B column l % 32, k 8 (l / 32)
// .. +7; accumulator value v is C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32].
// (DT: TM_DTYPE_BF16 or TM_DTYPE_F16 operands, same lane layout.)
template <int DT>
__device__ __forceinline__ f32x16_t pmfma(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (DT == TM_DTYPE_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ int acc_row(int v, int lane) {
  return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}

// Byte offset in a swizzled tile of logical chunk c (16 B) of row r: chunk c
// is stored at c ^ ((r / RPB) % CPR), so 16 consecutive rows read at one
// logical chunk cover 16 distinct 4-bank groups.
template <class C>
__device__ __forceinline__ int swz(int r, int c) {
  return r * C::PROW + ((c ^ ((r / C::RPB) & (C::CPR - 1))) << 4);
}

constexpr int kXcds = 8;  // workgroup i runs on XCD i % 8
constexpr int SBM = 8;    // super-block: M-tile slots (consecutive: mostly one expert) ..
constexpr int SBN = 4;    // .. x column jobs, M fastest

// Job of launch index L over the layer's real M-tiles (n_mt of them) in the
// super-block order (the self-routed decode gate/up, whose waves compute it
// in registers, and expert_job when most experts take one M-tile): M-tile
// and column job, or false for a launch index past the real jobs (those are
// the launch's last indices, so the real jobs all start in the first round).
// XCD x = L % 8 owns the column jobs [x * cpx, (x + 1) * cpx) for every
// M-tile, so each weight block is read through one XCD's L2 only, and walks
// them in strips of SBN columns, each strip in groups of SBM M-tiles, M
// fastest (the last strip and group may be narrower): the ~32 workgroups
// resident on the XCD share each A tile across SBN columns and each weight
// block across the M-tiles of one expert.
__device__ __forceinline__ bool job_of(int L, int n_mt, int ncol, int* mt, int* col) {
  const int x = L % kXcds, l = L / kXcds;
  const int cpx = (ncol + kXcds - 1) / kXcds;
  if (l >= n_mt * cpx) return false;
  const int s = l / (n_mt * SBN);                // column strip
  const int ws = min(SBN, cpx - s * SBN);         // its width
  const int j = l - s * n_mt * SBN;
  const int g = j / (SBM * ws);                  // M-tile group within the strip
  const int mg = min(SBM, n_mt - g * SBM);       // its size
  const int jj = j - g * SBM * ws;
  *mt = g * SBM + jj % mg;
  *col = x * cpx + s * SBN + jj / mg;
  return *col < ncol;
}

// Job of launch index L for the prefill GEMMs: M-tile (in the compact
// expert-major order) and column job, or false for a launch index past the
// real jobs (those are the launch's last indices).  The first wave scans
// ceil(rows_e / BM) over the experts (E <= 64 loads).  When the active
// experts average two M-tiles or more, XCD x = L % 8 walks its column jobs
// [x * cpx, (x + 1) * cpx) of every M-tile one expert at a time, the
// expert's M-tiles fastest, then its columns: the ~32 workgroups resident on
// an XCD then run the jobs of one expert or of a few adjacent ones, so all
// the M-tiles that read a weight block run together and share it in that
// L2, and each A tile is shared by the expert's nearby columns.  With fewer
// M-tiles it takes the super-block order (job_of), whose resident jobs read
// several experts' weights at once.  (Same box, bit-identical, expert order
// against super-blocks: config 5 1787 against 1801 us, T = 2048 uniform 1719
// against 1771, T = 4096 3111 against 3202, T = 1536 1374 against 1411; but
// T = 128 535 against 501, T = 256 542 against 513, T = 512 720 against 705,
// where most experts take one M-tile.)
template <class C>
__device__ __forceinline__ bool expert_job(int L, const int32_t* __restrict__ offsets, int E,
                                           int mt_max, int ncol, int* mt, int* col) {
  // every wave computes the job itself (no LDS, no barrier)
  const int x = L % kXcds, l = L / kXcds;
  const int cpx = (ncol + kXcds - 1) / kXcds;
  const int lane = threadIdx.x & 63;
  int n = 0;
  if (lane < E) {
    const int cnt = offsets[lane + 1] - offsets[lane];
    n = (cnt + C::PBM - 1) / C::PBM;
  }
  int incl = n;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  const int first = incl - n;  // M-tiles of the experts before this lane's
  const int total = __shfl(incl, 63);
  const int active = __popcll(__ballot(n > 0));
  int m = -1, c = 0;
  if (total < 2 * active) {
    // Mostly one M-tile per expert: the super-block order, whose jobs
    // resident together read different experts' weights.
    int jm = -1, jc = 0;
    const bool ok = job_of(L, min(total, mt_max), ncol, &jm, &jc);
    m = ok ? jm : -1;
    c = jc;
  } else {
    // the expert (lane) whose column range of this XCD holds l
    const bool mine = n > 0 && l >= first * cpx && l < incl * cpx;
    const unsigned long long owner = __ballot(mine);
    if (owner != 0ull) {
      const int src = __ffsll((long long)owner) - 1;
      const int j = l - first * cpx;
      m = __shfl(first + (n > 0 ? j % n : 0), src);
      c = __shfl(x * cpx + (n > 0 ? j / n : 0), src);
    }
  }
  *mt = __builtin_amdgcn_readfirstlane(m);
  *col = __builtin_amdgcn_readfirstlane(c);
  return *mt >= 0 && *mt < mt_max && *col < ncol;
}

// Launch size: 8 XCDs x (M-tile bound) x the columns of one XCD's range.
int64_t launch_jobs(int64_t mt_max, int64_t ncol) {
  return kXcds * mt_max * ((ncol + kXcds - 1) / kXcds);
}

// M-tile `idx` of the compact expert-major order: expert, first row, rows.
// An expert whose first entry in the 64-row tile list is masked (expert -1,
// as Routing.exclude_experts leaves it) is skipped, like the weight-streaming
// kernels skip its tiles.
template <class C>
__device__ __forceinline__ bool find_mtile(const int32_t* __restrict__ offsets,
                                           const int32_t* __restrict__ tiles, int max_tiles,
                                           int E, int idx, int* e, int* p0, int* rows,
                                           bool* single) {
  int acc = 0, tile64 = 0;
  for (int k = 0; k < E; ++k) {
    const int o = offsets[k];
    const int cnt = offsets[k + 1] - o;
    const int nt = (cnt + C::PBM - 1) / C::PBM;
    if (idx < acc + nt) {
      if (tile64 >= max_tiles || tiles[4 * tile64] != k) return false;
      const int m0 = (idx - acc) * C::PBM;
      *e = k;
      *p0 = o + m0;
      *rows = min(C::PBM, cnt - m0);
      *single = nt == 1;
      return true;
    }
    acc += nt;
    tile64 += (cnt + TM_GEMM_TILE_M - 1) / TM_GEMM_TILE_M;
  }
  return false;
}

// Upper bound of the M-tiles over E experts holding `slots` rows.
template <class C>
int64_t mtile_bound(int64_t slots, int64_t E) {
  return (slots + C::PBM - 1) / C::PBM + E;
}

// Global -> LDS: load i of a thread moves one 16-byte chunk.  Load i of wave
// w fills the 1 KB block 8 i + w of its tile (RPK rows); lane l writes byte
// 16 l of the block, i.e. row RPK (8 i + w) + l / CPR at stored chunk
// l % CPR, so it fetches the logical chunk that the swizzle stores there.
template <class C>
struct DmaLoad {
  __amdgpu_buffer_rsrc_t ra;        // A
  __amdgpu_buffer_rsrc_t rb0, rb1;  // B: the first and the second half of its loads
  uint32_t aoff[C::ALD];  // byte offset of the chunk at k = 0, or kOOR
  uint32_t boff[C::BLD];
};

// Row of load i for this thread, and the logical chunk it fetches.
template <class C>
__device__ __forceinline__ int dma_row(int i) {
  return C::RPK * (C::NW * i + (threadIdx.x >> 6)) + ((threadIdx.x & 63) / C::CPR);
}
template <class C>
__device__ __forceinline__ int dma_chunk(int row) {
  return (threadIdx.x & (C::CPR - 1)) ^ ((row / C::RPB) & (C::CPR - 1));
}

// Step `kstep` (K bytes PROW kstep ..) of both tiles into `st`: the A loads,
// then the B loads; past the end of K the loads are out of range and store
// zeros.  Every step issues all LDS_PER_STEP loads in this order, so the wait
// counts below stay exact.  (Spreading a step's loads between the previous
// step's MFMAs instead measured no faster.)
// One 16-byte buffer load per lane into LDS at `lds` + 16 lane (lds
// wave-uniform).  A plain function: the host compilation pass rejects the
// builtin inside some instantiations of the templates below.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint8_t* lds,
                                           uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voffset, 0, 0, 0);
}
// The same with the non-temporal cache policy (weights streamed through).
__device__ __forceinline__ void lds_load16_nt(__amdgpu_buffer_rsrc_t r, uint8_t* lds,
                                              uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voffset, 0, 0, 2);
}

template <class C, bool NTB>
__device__ __forceinline__ void dma_step(const DmaLoad<C>& d, uint8_t* st, int kstep, int nk) {
  const uint32_t kb = (uint32_t)kstep * (uint32_t)C::PROW;
  const bool valid = kstep < nk;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // LDS base: wave-uniform
#pragma unroll
  for (int i = 0; i < C::ALD; ++i)
    lds_load16(d.ra, st + (C::NW * i + w) * 1024,
               (valid && d.aoff[i] != kOOR) ? d.aoff[i] + kb : kOOR);
#pragma unroll
  for (int i = 0; i < C::BLD; ++i)
    if constexpr (NTB)
      lds_load16_nt(i < C::BLD / 2 ? d.rb0 : d.rb1, st + C::ABYTES + (C::NW * i + w) * 1024,
                    valid ? d.boff[i] + kb : kOOR);
    else
      lds_load16(i < C::BLD / 2 ? d.rb0 : d.rb1, st + C::ABYTES + (C::NW * i + w) * 1024,
                 valid ? d.boff[i] + kb : kOOR);
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
template <class C>
__device__ __forceinline__ u32x4_t frag(const uint8_t* tile, int row, int s, int lane) {
  return *reinterpret_cast<const u32x4_t*>(tile + swz<C>(row + (lane & 31), 2 * s + (lane >> 5)));
}

// acc[i][j] += A[32 M wm + 32 i, :] B[brow[j], :]^T over one staged step.  M
// (<= MT) is the accumulator tiles per wave along the rows: M = MT covers the
// whole M-tile, a smaller M its first 64 M rows (a tile with at most 64 M real
// rows, whose other rows are zeros).
template <class C, int M, int DT>
__device__ __forceinline__ void compute_step(const uint8_t* st, const int (&brow)[2],
                                             f32x16_t (&acc)[M][2]) {
  const int lane = threadIdx.x & 63;
  const int wm = (threadIdx.x >> 6) & 1;
  constexpr int S = C::PBK / 16;
  if constexpr (S >= 4) {
    // K steps of 64: the fragments of k-step s + 1 are read between the
    // MFMAs of k-step s (one MFMA, then one LDS read, while reads remain), so
    // each MFMA waits only for reads issued a k-step earlier.  Same MFMAs in
    // the same order.  (Config 5 down GEMM 588 -> 569 us same-box; on the
    // 256-row gate/up tile, whose steps have two k-steps, it measured slower,
    // 1043 -> 1068 us, so that tile keeps the loop below.)
    u32x4_t a[2][M], b[2][2];
#pragma unroll
    for (int i = 0; i < M; ++i) a[0][i] = frag<C>(st, 32 * M * wm + 32 * i, 0, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j) b[0][j] = frag<C>(st + C::ABYTES, brow[j], 0, lane);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      __builtin_amdgcn_sched_barrier(0);
      if (s + 1 < S) {
#pragma unroll
        for (int i = 0; i < M; ++i) a[nxt][i] = frag<C>(st, 32 * M * wm + 32 * i, s + 1, lane);
#pragma unroll
        for (int j = 0; j < 2; ++j) b[nxt][j] = frag<C>(st + C::ABYTES, brow[j], s + 1, lane);
      }
#pragma unroll
      for (int i = 0; i < M; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = pmfma<DT>(a[cur][i], b[cur][j], acc[i][j]);
      if (s + 1 < S) {
#pragma unroll
        for (int k = 0; k < M + 2 && k < 2 * M; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
        if constexpr (2 * M > M + 2)
          __builtin_amdgcn_sched_group_barrier(0x008, 2 * M - (M + 2), 0);
      }
    }
    // keep the next step's wait, barrier and loads after these MFMAs
    __builtin_amdgcn_sched_barrier(0);
  } else {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      u32x4_t a[M], b[2];
#pragma unroll
      for (int i = 0; i < M; ++i) a[i] = frag<C>(st, 32 * M * wm + 32 * i, s, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = frag<C>(st + C::ABYTES, brow[j], s, lane);
#pragma unroll
      for (int i = 0; i < M; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = pmfma<DT>(a[i], b[j], acc[i][j]);
    }
  }
}

// The LDS stages: distinct arrays used in a fixed rotation, so the compiler
// can tell the stage being read from the ones being loaded (s3 is unused with
// three stages).
struct Stages {
  uint8_t* s0;
  uint8_t* s1;
  uint8_t* s2;
  uint8_t* s3;
};

// A workgroup barrier (after this wave's LDS operations) that the compiler
// schedules nothing across.
__device__ __forceinline__ void pp_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  tm_lds_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// All fragments of one staged step (S = BK / 16 k-steps) into registers.
template <class C, int M>
__device__ __forceinline__ void read_step(const uint8_t* st, const int (&brow)[2],
                                          u32x4_t (&a)[C::PBK / 16][M],
                                          u32x4_t (&b)[C::PBK / 16][2]) {
  const int lane = threadIdx.x & 63;
  const int wm = (threadIdx.x >> 6) & 1;
#pragma unroll
  for (int s = 0; s < C::PBK / 16; ++s) {
#pragma unroll
    for (int i = 0; i < M; ++i) a[s][i] = frag<C>(st, 32 * M * wm + 32 * i, s, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j) b[s][j] = frag<C>(st + C::ABYTES, brow[j], s, lane);
  }
}

// The MFMAs of one staged step from registers, in compute_step's order.
template <class C, int M, int DT>
__device__ __forceinline__ void mfma_step(const u32x4_t (&a)[C::PBK / 16][M],
                                          const u32x4_t (&b)[C::PBK / 16][2],
                                          f32x16_t (&acc)[M][2]) {
#pragma unroll
  for (int s = 0; s < C::PBK / 16; ++s)
#pragma unroll
    for (int i = 0; i < M; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = pmfma<DT>(a[s][i], b[s][j], acc[i][j]);
}

// Ping-pong K loop (8 waves).  Waves 0-3 (half 0, one per SIMD) and waves
// 4-7 (half 1) alternate between a memory phase (issue the loads of a future
// step, read all fragments of the current step into registers) and an MFMA
// phase, half a step apart, so on every SIMD one wave's MFMAs run while the
// other wave reads its fragments; in the plain loop both waves of a SIMD
// leave each step's barrier together and wait for their first fragments
// together.  Barriers b(0), b(1), ... separate the phases:
//   half 0, step k:  b(2k)  [memory k]  b(2k+1)  [MFMA k, wait loads of k+1]
//   half 1, step k:  b(2k+1) [memory k, wait loads of k+1]  b(2k+2)  [MFMA k]
// Step k's loads are complete in every thread before b(2k), so both halves
// read it after that barrier; both have read step k-1 before b(2k), so the
// loads of step k+NS-1 go into its stage after it.  Each half issues every
// step's loads once, so the wait counts are those of k_loop; half 1 starts
// with two barriers and half 0 ends with two, so both pass the same number.
// Same MFMAs in the same order per output as k_loop.  (A workgroup's waves
// go to the CU's four SIMDs in turn, so waves w and w + 4 share a SIMD; the
// ordering argument above holds for any placement, only the overlap needs
// it.)
template <class C, int M, int DT, bool NTB>
__device__ __forceinline__ void k_loop_pp(const Stages& sb, const DmaLoad<C>& d, int nk,
                                          const int (&brow)[2], f32x16_t (&acc)[M][2]) {
  constexpr int NS = C::NSTAGE;
  constexpr int S = C::PBK / 16;
  constexpr int W = (NS - 2) * C::LDS_PER_STEP;
  uint8_t* const st[4] = {sb.s0, sb.s1, sb.s2, sb.s3};
  const bool half1 = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8)) != 0;
#pragma unroll
  for (int u = 0; u < NS - 1; ++u) dma_step<C, NTB>(d, st[u], u, nk);
  wait_vm<W>();
  u32x4_t a[S][M], b[S][2];
  if (!half1) {
    for (int k = 0; k < nk; k += NS) {
#pragma unroll
      for (int u = 0; u < NS; ++u) {
        if (u == 0 || k + u < nk) {
          pp_barrier();                                                  // b(2k)
          dma_step<C, NTB>(d, st[(u + NS - 1) % NS], k + u + NS - 1, nk);
          read_step<C, M>(st[u], brow, a, b);
          pp_barrier();                                                  // b(2k+1)
          mfma_step<C, M, DT>(a, b, acc);
          wait_vm<W>();
        }
      }
    }
    pp_barrier();
    pp_barrier();
  } else {
    pp_barrier();
    pp_barrier();
    for (int k = 0; k < nk; k += NS) {
#pragma unroll
      for (int u = 0; u < NS; ++u) {
        if (u == 0 || k + u < nk) {
          dma_step<C, NTB>(d, st[(u + NS - 1) % NS], k + u + NS - 1, nk);
          read_step<C, M>(st[u], brow, a, b);
          wait_vm<W>();
          pp_barrier();                                                  // b(2k+2)
          mfma_step<C, M, DT>(a, b, acc);
          pp_barrier();                                                  // b(2k+3)
        }
      }
    }
  }
  // the last loads (zeros past the end) must land before the stages are reused
  wait_vm<0>();
  __syncthreads();
}

// The K loop shared by both GEMMs over nk steps.  At the top of step k, steps
// k .. k+NS-2 are in flight; the thread waits for its loads of step k, the
// barrier makes every thread's loads visible and frees the stage of step k-1,
// step k+NS-1 goes into that stage, then step k's MFMAs run.  The barrier
// waits for this wave's LDS reads only (tm_lds_barrier), not for its
// outstanding loads: the loads of the next steps stay in flight.
template <class C, int M, int DT, bool NTB>
__device__ __forceinline__ void k_loop(const Stages& sb, const DmaLoad<C>& d, int nk,
                                       const int (&brow)[2], f32x16_t (&acc)[M][2]) {
  if constexpr (C::PP) {
    k_loop_pp<C, M, DT, NTB>(sb, d, nk, brow, acc);
    return;
  }
  constexpr int NS = C::NSTAGE;
  uint8_t* const st[4] = {sb.s0, sb.s1, sb.s2, sb.s3};
#pragma unroll
  for (int u = 0; u < NS - 1; ++u) dma_step<C, NTB>(d, st[u], u, nk);
  for (int k = 0; k < nk; k += NS) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      wait_vm<(NS - 2) * C::LDS_PER_STEP>();
      tm_lds_barrier();
      dma_step<C, NTB>(d, st[(u + NS - 1) % NS], k + u + NS - 1, nk);
      if (u == 0 || k + u < nk) compute_step<C, M, DT>(st[u], brow, acc);
    }
  }
  // the last loads (zeros past the end) must land before the stages are reused
  wait_vm<0>();
  __syncthreads();
}

// ------------------------------------------------------------- gate/up --
// h[p, n] = bf16( silu(x[tok(p)] . w1[e, n]) * (x[tok(p)] . w3[e, n]) ) for the
// rows p of one M-tile and the 128 columns n of one column block.
template <class C>
__device__ __forceinline__ uint8_t* h_stage(const Stages& sb, int m) {
  const int s = m / C::HROWS;
  uint8_t* base = s == 0 ? sb.s0 : s == 1 ? sb.s1 : s == 2 ? sb.s2 : sb.s3;
  return base + (m % C::HROWS) * C::HSTRIDE;
}

// The MFMAs and the epilogue of one gate/up tile with M accumulator tiles
// per wave (see compute_step): SwiGLU in registers, the bf16 tile staged in
// LDS, then a coalesced store of its `rows` rows.
template <class C, int M, int DT, bool NTB>
__device__ __forceinline__ void gemm1_tile(const Stages& sb, const DmaLoad<C>& d, int nk,
                                           int rows, int p0, int n0, int I,
                                           uint16_t* __restrict__ h) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;
  f32x16_t acc[M][2];
#pragma unroll
  for (int i = 0; i < M; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  // accumulator column blocks: j = 0 -> w1 rows 32 wn ..; j = 1 -> the same w3 rows
  const int brow[2] = {32 * wn, C::PBN / 2 + 32 * wn};
  k_loop<C, M, DT, NTB>(sb, d, nk, brow, acc);
#pragma unroll
  for (int i = 0; i < M; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float a = acc[i][0][v];
      const float b = acc[i][1][v];
      const float hv = (a / (1.0f + __expf(-a))) * b;
      const int m = 32 * M * wm + 32 * i + acc_row(v, lane);
      const int c = 32 * wn + (lane & 31);
      *reinterpret_cast<uint16_t*>(h_stage<C>(sb, m) + c * 2) = Half16<DT>::round(hv);
    }
  __syncthreads();
  constexpr int PPR = C::PBN / 16;  // 16-byte pieces of an h row (PBN / 2 columns)
#pragma unroll
  for (int j = 0; j < 64 * M * PPR / C::NT; ++j) {
    const int piece = tid + C::NT * j;  // 64 M rows x PPR pieces
    const int r = piece / PPR, c16 = piece % PPR;
    if (r < rows) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(h_stage<C>(sb, r) + c16 * 16);
      *reinterpret_cast<u32x4_t*>(h + (size_t)(p0 + r) * I + n0 + c16 * 8) = v;
    }
  }
}

// gemm1_tile with the fewest accumulator tiles M <= MM per wave whose 64 M
// rows (two waves of 32 M) cover `rows`.  Each output keeps the same K order
// whatever M is, so the bits do not depend on it.
template <class C, int MM, int DT, bool NTB>
__device__ __forceinline__ void gemm1_rows(const Stages& sb, const DmaLoad<C>& d, int nk,
                                           int rows, int p0, int n0, int I,
                                           uint16_t* __restrict__ h) {
  if constexpr (MM > 1) {
    if (rows <= 64 * (MM - 1)) {
      gemm1_rows<C, MM - 1, DT, NTB>(sb, d, nk, rows, p0, n0, I, h);
      return;
    }
  }
  gemm1_tile<C, MM, DT, NTB>(sb, d, nk, rows, p0, n0, I, h);
}

// One gate/up job: M-tile (expert e, sorted rows p0 .. p0 + rows) against
// column block cb; d.ra and d.aoff (the A rows) are set by the caller.
template <class C, int DT>
__device__ __forceinline__ void gemm1_job(const Stages& sb, DmaLoad<C>& d,
                                          const uint16_t* __restrict__ w1,
                                          const uint16_t* __restrict__ w3,
                                          uint16_t* __restrict__ h, int e, int p0, int rows,
                                          bool single, int cb, int H, int I) {
  const int n0 = cb * (C::PBN / 2);  // first h column of the block
  const size_t ebase = (size_t)e * I * H;
  d.rb0 = pbuf(w1 + ebase, (uint32_t)((size_t)I * H * 2));
  d.rb1 = pbuf(w3 + ebase, (uint32_t)((size_t)I * H * 2));
#pragma unroll
  for (int i = 0; i < C::BLD; ++i) {
    const int r = dma_row<C>(i);  // first half of the loads: w1 rows; second: the same w3 rows
    d.boff[i] = (uint32_t)(n0 + (r & (C::PBN / 2 - 1))) * (uint32_t)H * 2u +
                (uint32_t)dma_chunk<C>(r) * 16u;
  }
  // A tile with fewer than BM real rows (an expert's last) runs the MFMAs of
  // its first ceil(rows / 64) 64-row quarters only; its A rows past `rows`
  // are loaded as zeros without memory traffic.  An expert that takes one
  // M-tile has its weights read by this job alone: they stream through with
  // the non-temporal policy (a load-only probe streams 7.1 TB/s with it, 6.2
  // without).  With several M-tiles the other jobs of the expert find them in
  // L2, so those loads stay cached.
  if (C::NT_WEIGHTS && single)
    gemm1_rows<C, C::MT, DT, C::NT_WEIGHTS>(sb, d, H / C::PBK, rows, p0, n0, I, h);
  else gemm1_rows<C, C::MT, DT, false>(sb, d, H / C::PBK, rows, p0, n0, I, h);
}

template <class C, int DT>
__global__ void __launch_bounds__(C::NT)
tm_prefill_gemm1_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                        const uint16_t* __restrict__ w3, uint16_t* __restrict__ h,
                        const int32_t* __restrict__ sorted_slots,
                        const int32_t* __restrict__ offsets, const int32_t* __restrict__ tiles,
                        int max_tiles, int E, int H, int I, int mt_max, uint32_t x_bytes) {
  __shared__ __attribute__((aligned(16))) uint8_t s0[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s1[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s2[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s3[C::NSTAGE > 3 ? C::STAGE : 16];
  const Stages sb{s0, s1, s2, s3};
  int mt, cb;
  const int ncol = I / (C::PBN / 2);
  if (!expert_job<C>((int)blockIdx.x, offsets, E, mt_max, ncol, &mt, &cb)) return;
  int e, p0, rows;
  bool single;
  if (!find_mtile<C>(offsets, tiles, max_tiles, E, mt, &e, &p0, &rows, &single)) return;
  DmaLoad<C> d;
  d.ra = pbuf(x, x_bytes);
#pragma unroll
  for (int i = 0; i < C::ALD; ++i) {
    const int r = dma_row<C>(i);
    d.aoff[i] = r < rows ? (uint32_t)(sorted_slots[p0 + r] >> 1) * (uint32_t)H * 2u +
                               (uint32_t)dma_chunk<C>(r) * 16u
                         : kOOR;
  }
  gemm1_job<C, DT>(sb, d, w1, w3, h, e, p0, rows, single, cb, H, I);
}

// ------------------------------------------------ gate/up, self-routed --
// At few tokens the budget routing and bucketing run inside the gate/up
// launch instead of in a launch of their own.  Launch index 0 runs the
// routing phases of the routing kernel (tmb::bucket_phases, same code and
// floating-point order) and writes every routing output (topk_ids,
// gates_flat, the layouts, demand) for the down GEMM, the combine and the
// Routing handle; indices 1 .. 7 exit, so GEMM job j = index - 8 keeps XCD
// j % 8 (job_of).  Every wave of a GEMM workgroup derives its job from the
// router gates by itself, one token per lane, with cross-lane operations only
// (rr_job): no LDS and no barrier, one round of global loads (the gates), and
// the same operations in the same order as the phases, so the same experts,
// counts and rows.  Measured on MI355X against the routing launch, same box,
// whole layer: config 2 440 against 445 us, config 3 (B = 4) 247 against
// 252.5 us, the TP-2 and TP-4 shares 5 us faster each.  Tried first: every
// GEMM workgroup running the LDS phases themselves (their barriers cost it
// as much as the routing launch saved), and a per-wave view with one
// reduction chain per expert in turn (~9 us per job instead of ~5).
constexpr int kRrMaxTokens = 64;       // one token per lane
constexpr int kRrMaxExperts = 16;      // gates of a token held in registers
constexpr int kRvMaxBlocks = 256;      // reference padded blocks (the writer's LDS)
constexpr int kRvLeaders = 8;          // launch indices before the GEMM jobs
using RvShared = tmb::BucketSharedT<kRrMaxTokens, kRrMaxTokens * kRrMaxExperts, kRvMaxBlocks>;

// Position of the j-th set bit (j from 0) of m, which has more than j.
__device__ __forceinline__ int nth_set_bit(unsigned long long m, int j) {
  int pos = 0;
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const unsigned long long low = m & ((1ull << w) - 1ull);
    const int c = __popcll(low);
    if (j >= c) {
      j -= c;
      pos += w;
      m >>= w;
    }
  }
  return pos;
}

// The kept experts (bit e) from the demand and criticality of every token
// held in its lane (g: the lane's gates, zero past E or T; a_ld: the lane's
// accept probability, loaded with the gates), as the phases compute them.
template <int EM>
__device__ __forceinline__ unsigned long long keep_set(const tmb::BucketArgs& a,
                                                       const float (&g)[EM], float a_ld,
                                                       bool tok, int lane) {
  const int E = a.E;
  const float av = tok ? a_ld : 0.0f;
  const bool critical = a.objective == TM_OBJECTIVE_CRITICAL_PATH;
  // demand: the EM halving trees, level by level
  float acc[EM];
#pragma unroll
  for (int e = 0; e < EM; ++e) {
    float z = 0.0f;
    const float p = av * g[e];
    acc[e] = tok ? z + p : z;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
    for (int e = 0; e < EM; ++e) acc[e] = acc[e] + __shfl_xor(acc[e], off);
  float d_mine = 0.0f;
#pragma unroll
  for (int e = 0; e < EM; ++e) d_mine = lane == e ? acc[e] : d_mine;
  float c_mine = 0.0f;
  if (critical) {
    tmb::Top2 u{-1, -1, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < EM; ++e)
      if (e < E) u.offer(g[e], e);
    float crit[EM];
#pragma unroll
    for (int e = 0; e < EM; ++e) {
      const bool needed = tok && ((u.i1 == e) || ((u.i2 == e) && (av >= a.tau)));
      crit[e] = needed ? fmaxf(-INFINITY, av) : -INFINITY;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
      for (int e = 0; e < EM; ++e) crit[e] = fmaxf(crit[e], __shfl_xor(crit[e], off));
#pragma unroll
    for (int e = 0; e < EM; ++e) c_mine = lane == e ? crit[e] : c_mine;
  }
  // keep set: lane = expert, as in the phases
  {
    const float d = lane < E ? d_mine : 0.0f;
    const float c = (critical && lane < E) ? c_mine : 0.0f;
    int rank = 0;
#pragma unroll
    for (int f = 0; f < EM; ++f) {
      if (f < E) {
        const float df = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(
                                                       __builtin_bit_cast(int, acc[f])));
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
    }
    return __ballot(lane < E && rank < a.budget);
  }
}

// The job of GEMM launch index l (M-tile of BM rows of one expert x column
// block, job_of over the layer's real M-tiles) from the router gates, in one
// wave: lane t holds token t's gates, EM >= E registers of them.  The expert
// of each routed slot, each expert's count and compact offset, and the
// M-tiles follow tmb::bucket_phases step by step:
//   demand[e] = 0 + accept[t] gates[t, e] in lane t (0 past T), then the xor
//   halving tree; crit[e] likewise with fmaxf (critical-path objective only);
//   keep = ranks in the order (crit desc,) demand desc, e asc;
//   masked top-2 per token, offered in expert order;
//   the slots of expert e in slot order are the tokens whose top-2 holds e
//   (the two picks differ), so each expert's rows are the set bits of one
//   64-bit ballot, in token order, and its count that ballot's popcount.
// The EM halving trees run interleaved and everything after them on wave-
// uniform (scalar) values: a wave spends about a microsecond here beyond the
// gates' load.  Returns false when l has no job.  `mask` is the expert's
// token ballot and m0 the rank of the M-tile's first row among its rows.
template <class C, int EM>
__device__ __forceinline__ bool rr_job(const tmb::BucketArgs& a, int l, int ncol, int mt_max,
                                       int* e_out, int* p0_out, int* rows_out, int* m0_out,
                                       bool* single_out, int* cb_out,
                                       unsigned long long* mask_out) {
  const int lane = threadIdx.x & 63;
  const int T = a.T, E = a.E;
  const bool tok = lane < T;
  // the accept probability is read with the gates (one memory round trip:
  // loaded after the gates had arrived it cost a second one, ~2 us per job)
  const float a_ld = a.accept[tok ? lane : 0];
  float g[EM];
  if ((E & 3) == 0 && (reinterpret_cast<uintptr_t>(a.gates) & 15) == 0) {
#pragma unroll
    for (int q = 0; q < EM / 4; ++q) {
      const bool ok = tok && 4 * q < E;
      const float4 v = *reinterpret_cast<const float4*>(a.gates + (ok ? lane * E + 4 * q : 0));
      g[4 * q] = ok ? v.x : 0.0f;
      g[4 * q + 1] = ok ? v.y : 0.0f;
      g[4 * q + 2] = ok ? v.z : 0.0f;
      g[4 * q + 3] = ok ? v.w : 0.0f;
    }
  } else {
#pragma unroll
    for (int e = 0; e < EM; ++e) {
      const bool ok = tok && e < E;
      const float v = a.gates[ok ? lane * E + e : 0];
      g[e] = ok ? v : 0.0f;
    }
  }
  // with a budget of every expert, all are kept whatever the demand
  unsigned long long keep = (1ull << E) - 1ull;
  if (a.budget < E) keep = keep_set<EM>(a, g, a_ld, tok, lane);
  // masked top-2 of this lane's token
  tmb::Top2 r{-1, -1, 0.0f, 0.0f};
#pragma unroll
  for (int e = 0; e < EM; ++e)
    if (e < E) r.offer(((keep >> e) & 1ull) ? g[e] : 0.0f, e);
  const int i1 = tok ? r.i1 : -1;
  const int i2 = tok ? r.i2 : -1;
  // per-expert counts, compact offsets and M-tiles on scalars
  int cnt[EM], off_e[EM], ps[EM];
  int run_off = 0, run_mt = 0;
#pragma unroll
  for (int e = 0; e < EM; ++e) {
    cnt[e] = __popcll(__ballot(i1 == e || i2 == e));
    off_e[e] = run_off;
    ps[e] = run_mt;
    run_off += cnt[e];
    run_mt += (cnt[e] + C::PBM - 1) / C::PBM;
  }
  const int n_mt = min(run_mt, mt_max);
  int mt, cb;
  if (!job_of(l, n_mt, ncol, &mt, &cb)) return false;
  int e = -1;
#pragma unroll
  for (int k = 0; k < EM; ++k)
    if (e < 0 && mt < ps[k] + (cnt[k] + C::PBM - 1) / C::PBM) e = k;
  if (e < 0) return false;
  int cnt_e = 0, off_sel = 0, ps_sel = 0;
#pragma unroll
  for (int k = 0; k < EM; ++k)
    if (k == e) {
      cnt_e = cnt[k];
      off_sel = off_e[k];
      ps_sel = ps[k];
    }
  const int m0 = (mt - ps_sel) * C::PBM;
  *e_out = e;
  *m0_out = m0;
  *p0_out = off_sel + m0;
  *rows_out = min(C::PBM, cnt_e - m0);
  *single_out = (cnt_e + C::PBM - 1) / C::PBM == 1;
  *cb_out = cb;
  *mask_out = __ballot(i1 == e || i2 == e);
  return true;
}

template <class C, int DT, int EM>
__global__ void __launch_bounds__(C::NT)
tm_prefill_gemm1_routed_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                               const uint16_t* __restrict__ w3, uint16_t* __restrict__ h,
                               tmb::BucketArgs ra, int H, int I, int mt_max, uint32_t x_bytes) {
  __shared__ __attribute__((aligned(16))) uint8_t s0[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s1[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s2[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s3[C::NSTAGE > 3 ? C::STAGE : 16];
  static_assert(sizeof(RvShared) <= C::STAGE, "the routing writer uses the first stage");
  const int L = (int)blockIdx.x;
  if (L < kRvLeaders) {
    if (L == 0) tmb::bucket_phases<C::NT, RvShared, true>(ra, *reinterpret_cast<RvShared*>(s0));
    return;
  }
  int e, p0, rows, m0, cb;
  bool single;
  unsigned long long mask;
  if (!rr_job<C, EM>(ra, L - kRvLeaders, I / (C::PBN / 2), mt_max, &e, &p0, &rows, &m0,
                     &single, &cb, &mask))
    return;
  DmaLoad<C> d;
  d.ra = pbuf(x, x_bytes);
#pragma unroll
  for (int i = 0; i < C::ALD; ++i) {
    const int r = dma_row<C>(i);
    d.aoff[i] = r < rows ? (uint32_t)nth_set_bit(mask, m0 + r) * (uint32_t)H * 2u +
                               (uint32_t)dma_chunk<C>(r) * 16u
                         : kOOR;
  }
  const Stages sb{s0, s1, s2, s3};
  gemm1_job<C, DT>(sb, d, w1, w3, h, e, p0, rows, single, cb, H, I);
}

// ---------------------------------------------------------------- down --
// y[s, p, n] = gates_flat[slot(p)] * sum_{k in segment s} h[p, k] w2[e, n, k]
// for the rows p of one M-tile and 256 output columns n.  The fp32 partials
// go straight from the accumulators: for each accumulator value, 32 lanes
// store 128 contiguous bytes of one row.
template <class C, int M, int DT, bool NTB>
__device__ __forceinline__ void gemm2_tile(const Stages& sb, const DmaLoad<C>& d, int nk,
                                           int rows, int p0, int H,
                                           const float* __restrict__ gates_flat,
                                           const int32_t* __restrict__ sorted_slots,
                                           float* __restrict__ ys) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave & 1, wn = wave >> 1;
  f32x16_t acc[M][2];
#pragma unroll
  for (int i = 0; i < M; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  const int brow[2] = {64 * wn, 64 * wn + 32};
  k_loop<C, M, DT, NTB>(sb, d, nk, brow, acc);
#pragma unroll
  for (int i = 0; i < M; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = 32 * M * wm + 32 * i + acc_row(v, lane);
      if (m < rows) {
        const float gate = gates_flat[sorted_slots[p0 + m]];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int c = 64 * wn + 32 * j + (lane & 31);
          ys[(size_t)(p0 + m) * H + c] = acc[i][j][v] * gate;
        }
      }
    }
}

template <class C, int DT>
__global__ void __launch_bounds__(C::NT)
tm_prefill_gemm2_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ w2,
                        float* __restrict__ y, const float* __restrict__ gates_flat,
                        const int32_t* __restrict__ sorted_slots,
                        const int32_t* __restrict__ offsets, const int32_t* __restrict__ tiles,
                        int max_tiles, int E, int R, int H, int I, int klen, int nsplit,
                        int mt_max, uint32_t h_bytes) {
  __shared__ __attribute__((aligned(16))) uint8_t s0[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s1[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s2[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s3[C::NSTAGE > 3 ? C::STAGE : 16];
  static_assert(C::NW == 8, "down GEMM: 8 waves, 64 output columns per column group");
  int mt, job;  // job = (segment, column block), segment-major
  const int ncb = H / C::PBN;
  const int ncol = ncb * nsplit;
  if (!expert_job<C>((int)blockIdx.x, offsets, E, mt_max, ncol, &mt, &job)) return;
  // Each XCD owns a contiguous range of these jobs, so segment-major puts
  // one K segment on each XCD (2 segments over 8 XCDs: 4 each) and an XCD
  // reads the h rows of its segment only, instead of all of h.
  const int seg = job / ncb;
  const int cb = job - seg * ncb;
  int e, p0, rows;
  bool single;
  if (!find_mtile<C>(offsets, tiles, max_tiles, E, mt, &e, &p0, &rows, &single)) return;
  const int n0 = cb * C::PBN;
  const uint32_t k0 = (uint32_t)seg * (uint32_t)klen * 2u;  // segment start, bytes

  DmaLoad<C> d;
  d.ra = pbuf(h, h_bytes);
  d.rb0 = d.rb1 = pbuf(w2 + (size_t)e * H * I, (uint32_t)((size_t)H * I * 2));
#pragma unroll
  for (int i = 0; i < C::ALD; ++i) {
    const int r = dma_row<C>(i);
    d.aoff[i] = r < rows ? (uint32_t)(p0 + r) * (uint32_t)I * 2u + k0 +
                               (uint32_t)dma_chunk<C>(r) * 16u
                         : kOOR;
  }
#pragma unroll
  for (int i = 0; i < C::BLD; ++i) {
    const int r = dma_row<C>(i);
    d.boff[i] = (uint32_t)(n0 + r) * (uint32_t)I * 2u + k0 + (uint32_t)dma_chunk<C>(r) * 16u;
  }
  const Stages sb{s0, s1, s2, s3};
  float* ys = y + (size_t)seg * R * H + n0;
  if constexpr (C::MT > 1) {
    if (rows <= C::PBM / 2) {  // as in gate/up
      if (C::NT_WEIGHTS && single)
        gemm2_tile<C, C::MT / 2, DT, C::NT_WEIGHTS>(sb, d, klen / C::PBK, rows, p0, H, gates_flat,
                                           sorted_slots, ys);
      else
        gemm2_tile<C, C::MT / 2, DT, false>(sb, d, klen / C::PBK, rows, p0, H, gates_flat,
                                            sorted_slots, ys);
      return;
    }
  }
  if (C::NT_WEIGHTS && single)
    gemm2_tile<C, C::MT, DT, C::NT_WEIGHTS>(sb, d, klen / C::PBK, rows, p0, H, gates_flat, sorted_slots,
                                   ys);
  else
    gemm2_tile<C, C::MT, DT, false>(sb, d, klen / C::PBK, rows, p0, H, gates_flat, sorted_slots,
                                    ys);
}

bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

// The gate/up launch with tile C: jobs for the M-tile bound (the tile list's
// length, capped by what 2T rows in E experts can take).
template <class C, int DT>
int launch_gemm1(const void* x, const void* w1, const void* w3, void* h,
                 const int32_t* sorted_slots, const int32_t* expert_offsets,
                 const int32_t* tiles, int64_t max_tiles, int64_t T, int64_t H, int64_t I,
                 int64_t E, hipStream_t stream) {
  const int64_t mt_max = std::min<int64_t>(max_tiles, mtile_bound<C>(2 * T, E));
  const int64_t jobs = launch_jobs(mt_max, I / (C::PBN / 2));
  if (jobs > INT32_MAX) return TM_ERR_SHAPE;
  hipLaunchKernelGGL((tm_prefill_gemm1_kernel<C, DT>), dim3((unsigned)jobs), dim3(C::NT), 0, stream,
                     (const uint16_t*)x, (const uint16_t*)w1, (const uint16_t*)w3,
                     (uint16_t*)h, sorted_slots, expert_offsets, tiles, (int)max_tiles,
                     (int)E, (int)H, (int)I, (int)mt_max, (uint32_t)(T * H * 2));
  return TM_OK;
}

// The self-routed gate/up launch with tile C.
template <class C, int DT>
int launch_gemm1_routed(const void* x, const void* w1, const void* w3, void* h,
                        const tmb::BucketArgs& ra, int64_t T, int64_t H, int64_t I,
                        hipStream_t stream) {
  const int64_t mt_max = std::min<int64_t>(ra.max_tiles, mtile_bound<C>(2 * T, ra.E));
  const int64_t jobs = launch_jobs(mt_max, I / (C::PBN / 2)) + kRvLeaders;
  if (jobs > INT32_MAX) return TM_ERR_SHAPE;
  if (ra.E <= 8)
    hipLaunchKernelGGL((tm_prefill_gemm1_routed_kernel<C, DT, 8>), dim3((unsigned)jobs),
                       dim3(C::NT), 0, stream, (const uint16_t*)x, (const uint16_t*)w1,
                       (const uint16_t*)w3, (uint16_t*)h, ra, (int)H, (int)I, (int)mt_max,
                       (uint32_t)(T * H * 2));
  else
    hipLaunchKernelGGL((tm_prefill_gemm1_routed_kernel<C, DT, kRrMaxExperts>),
                       dim3((unsigned)jobs), dim3(C::NT), 0, stream, (const uint16_t*)x,
                       (const uint16_t*)w1, (const uint16_t*)w3, (uint16_t*)h, ra, (int)H,
                       (int)I, (int)mt_max, (uint32_t)(T * H * 2));
  return TM_OK;
}

}  // namespace

extern "C" int tm_op1_prefill_gemm1(const void* x, const void* w1, const void* w3, void* h,
                                    const int32_t* sorted_slots, const int32_t* expert_offsets,
                                    const int32_t* tiles, int64_t max_tiles, int64_t T,
                                    int64_t H, int64_t I, int64_t E, int dtype, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS || max_tiles < 1)
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_BF16 && dtype != TM_DTYPE_F16) return TM_ERR_ARG;
  if (H < Tile128::PBK || (H % Tile128::PBK) != 0 || I < Tile128::PBN / 2 ||
      (I % (Tile128::PBN / 2)) != 0)
    return TM_ERR_SHAPE;
  if (I * H * 2 >= (int64_t)kOOR || T * H * 2 >= (int64_t)kOOR || 2 * T * I * 2 >= (int64_t)kOOR)
    return TM_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w1) || !aligned16(w3) || !aligned16(h)) return TM_ERR_ALIGN;
  // 256-row tiles when the experts average 384 rows or more: they read fewer
  // operand bytes per flop, but below that their coarser jobs and padding
  // cost more than that saves (measured at the Mixtral shape).  TileDec when
  // the tile list leaves at most 16 rows per entry (2T <= 16 max_tiles: few
  // rows per active expert, e.g. 64 tree tokens over 8 experts): half the
  // weight rows per workgroup and two workgroups per CU stream the weights
  // faster there (config 2 gate/up 302 -> 289 us same-box).
  const bool big = 2 * T >= 384 * E;
  const bool dec = !big && 2 * T <= 16 * max_tiles;
  const hipStream_t st = (hipStream_t)stream;
  const bool f16 = dtype == TM_DTYPE_F16;
  int rc;
  if (big) {
    rc = f16 ? launch_gemm1<Tile256, TM_DTYPE_F16>(x, w1, w3, h, sorted_slots, expert_offsets,
                                                   tiles, max_tiles, T, H, I, E, st)
             : launch_gemm1<Tile256, TM_DTYPE_BF16>(x, w1, w3, h, sorted_slots, expert_offsets,
                                                    tiles, max_tiles, T, H, I, E, st);
  } else if (dec) {
    rc = f16 ? launch_gemm1<TileDec, TM_DTYPE_F16>(x, w1, w3, h, sorted_slots, expert_offsets,
                                                   tiles, max_tiles, T, H, I, E, st)
             : launch_gemm1<TileDec, TM_DTYPE_BF16>(x, w1, w3, h, sorted_slots, expert_offsets,
                                                    tiles, max_tiles, T, H, I, E, st);
  } else {
    rc = f16 ? launch_gemm1<Tile128, TM_DTYPE_F16>(x, w1, w3, h, sorted_slots, expert_offsets,
                                                   tiles, max_tiles, T, H, I, E, st)
             : launch_gemm1<Tile128, TM_DTYPE_BF16>(x, w1, w3, h, sorted_slots, expert_offsets,
                                                    tiles, max_tiles, T, H, I, E, st);
  }
  if (rc) return rc;
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op1_prefill_gemm1_routed(
    const void* x, const void* w1, const void* w3, void* h, const float* gates,
    const float* accept, int64_t T, int64_t H, int64_t I, int64_t E, int64_t budget, float tau,
    int objective, int64_t block_m, int64_t max_blocks, int64_t max_tiles, int64_t* topk_ids,
    float* gates_flat, int64_t* padded_slots, int64_t* block_expert_ids, int64_t* slot_to_row,
    float* demand, int32_t* expert_offsets, int32_t* sorted_slots, int32_t* slot_pos,
    int32_t* tiles, int dtype, void* stream) {
  if (T < 1 || T > kRrMaxTokens || E < 2 || E > kRrMaxExperts) return TM_ERR_SHAPE;
  if (budget < 2 || budget > E) return TM_ERR_ARG;
  if (objective != TM_OBJECTIVE_MASS && objective != TM_OBJECTIVE_CRITICAL_PATH) return TM_ERR_ARG;
  if (block_m != 16 && block_m != 32) return TM_ERR_ARG;
  if (max_blocks < 1 || max_blocks > kRvMaxBlocks || max_tiles < 1) return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_BF16 && dtype != TM_DTYPE_F16) return TM_ERR_ARG;
  if (H < Tile128::PBK || (H % Tile128::PBK) != 0 || I < Tile128::PBN / 2 ||
      (I % (Tile128::PBN / 2)) != 0)
    return TM_ERR_SHAPE;
  if (I * H * 2 >= (int64_t)kOOR || T * H * 2 >= (int64_t)kOOR || 2 * T * I * 2 >= (int64_t)kOOR)
    return TM_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w1) || !aligned16(w3) || !aligned16(h)) return TM_ERR_ALIGN;
  tmb::BucketArgs ra;
  ra.gates = gates;
  ra.accept = accept;
  ra.T = (int)T;
  ra.E = (int)E;
  ra.budget = (int)budget;
  ra.objective = objective;
  ra.BM = (int)block_m;
  ra.max_blocks = (int)max_blocks;
  ra.max_tiles = (int)max_tiles;
  ra.tau = tau;
  ra.topk_ids = topk_ids;
  ra.gates_flat = gates_flat;
  ra.padded_slots = padded_slots;
  ra.block_expert_ids = block_expert_ids;
  ra.slot_to_row = slot_to_row;
  ra.demand_out = demand;
  ra.expert_offsets = expert_offsets;
  ra.sorted_slots = sorted_slots;
  ra.slot_pos = slot_pos;
  ra.tiles = tiles;
  // the tile rule of tm_op1_prefill_gemm1 (2T < 384 E here, so never the
  // 256-row tile)
  const bool dec = 2 * T <= 16 * max_tiles;
  const hipStream_t st = (hipStream_t)stream;
  const bool f16 = dtype == TM_DTYPE_F16;
  int rc;
  if (dec) {
    rc = f16 ? launch_gemm1_routed<TileDec, TM_DTYPE_F16>(x, w1, w3, h, ra, T, H, I, st)
             : launch_gemm1_routed<TileDec, TM_DTYPE_BF16>(x, w1, w3, h, ra, T, H, I, st);
  } else {
    rc = f16 ? launch_gemm1_routed<Tile128, TM_DTYPE_F16>(x, w1, w3, h, ra, T, H, I, st)
             : launch_gemm1_routed<Tile128, TM_DTYPE_BF16>(x, w1, w3, h, ra, T, H, I, st);
  }
  if (rc) return rc;
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

namespace {

// The down launch with tile C.
template <class C>
int launch_gemm2(const void* h, const void* w2, float* y, const float* gates_flat,
                 const int32_t* sorted_slots, const int32_t* expert_offsets,
                 const int32_t* tiles, int64_t max_tiles, int64_t split, int64_t T, int64_t H,
                 int64_t I, int64_t E, int dtype, hipStream_t stream) {
  const int64_t klen = I / split;
  const int64_t mt_max = std::min<int64_t>(max_tiles, mtile_bound<C>(2 * T, E));
  const int64_t jobs = launch_jobs(mt_max, (H / C::PBN) * split);
  if (jobs > INT32_MAX) return TM_ERR_SHAPE;
  hipLaunchKernelGGL((dtype == TM_DTYPE_F16 ? tm_prefill_gemm2_kernel<C, TM_DTYPE_F16>
                                            : tm_prefill_gemm2_kernel<C, TM_DTYPE_BF16>),
                     dim3((unsigned)jobs), dim3(C::NT), 0, stream, (const uint16_t*)h,
                     (const uint16_t*)w2, y, gates_flat, sorted_slots, expert_offsets, tiles,
                     (int)max_tiles, (int)E, (int)(2 * T), (int)H, (int)I, (int)klen,
                     (int)split, (int)mt_max, (uint32_t)(2 * T * I * 2));
  return TM_OK;
}

}  // namespace

extern "C" int tm_op1_prefill_gemm2(const void* h, const void* w2, float* y,
                                    const float* gates_flat, const int32_t* sorted_slots,
                                    const int32_t* expert_offsets, const int32_t* tiles,
                                    int64_t max_tiles, int64_t split, int64_t T, int64_t H,
                                    int64_t I, int64_t E, int dtype, void* stream) {
  using C = Tile128;
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS || max_tiles < 1)
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_BF16 && dtype != TM_DTYPE_F16) return TM_ERR_ARG;
  if (split < 1 || (I % split) != 0) return TM_ERR_SHAPE;
  const int64_t klen = I / split;
  if (klen < C::PBK || (klen % C::PBK) != 0 || H < C::PBN || (H % C::PBN) != 0) return TM_ERR_SHAPE;
  if (H * I * 2 >= (int64_t)kOOR || 2 * T * I * 2 >= (int64_t)kOOR) return TM_ERR_SHAPE;
  if (!aligned16(h) || !aligned16(w2) || !aligned16(y)) return TM_ERR_ALIGN;
  // where the experts average 384 rows or more (the gate/up rule for its
  // 256-row tile) the MFMAs bound the kernel and the ping-pong loop runs
  const bool big = 2 * T >= 384 * E;
  const int rc = big ? launch_gemm2<Tile128PP>(h, w2, y, gates_flat, sorted_slots,
                                               expert_offsets, tiles, max_tiles, split, T, H,
                                               I, E, dtype, (hipStream_t)stream)
                     : launch_gemm2<Tile128>(h, w2, y, gates_flat, sorted_slots, expert_offsets,
                                             tiles, max_tiles, split, T, H, I, E, dtype,
                                             (hipStream_t)stream);
  if (rc) return rc;
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}
