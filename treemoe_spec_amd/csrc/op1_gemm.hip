// op1 expert GEMMs on gfx950: gate/up + SwiGLU, down projection with a
// deterministic K split, and the fixed-order combine.
//
// Work item = one workgroup = 2 x 16 weight rows of one expert (the same rows of
// w1 and w3, or two adjacent row blocks of w2) x one GEMM tile
// (<= 64 sorted rows of that expert, NSUB = ceil(rows/16) 16-row sub-tiles,
// a template parameter chosen per tile).  The 4 waves of the workgroup split
// the reduction dimension: wave w takes K chunks w, w+4, w+8, ...; their
// partial sums are added in LDS in the fixed order (wave 0 + 1 + 2 + 3), so
// results are bitwise reproducible.  Small items keep the drain at the end of
// each launch short.
//
// Weights stream HBM -> VGPR with coalesced 16-byte non-temporal buffer loads
// (one instruction = 8 rows x 128 contiguous bytes), one chunk ahead of use,
// and are turned into v_mfma_f32_16x16x32_bf16 B operands (lane l: row l%16,
// k-group l/16) through a per-wave LDS scratch whose rows are padded by 16
// bytes (conflict-free fragment reads).  Activations are read straight into A
// operands: x rows gathered by token for the gate/up GEMM; for the down GEMM,
// h, which the gate/up GEMM writes in A-fragment order ("swizzled": one 16-row
// sub-tile x 32-column k-step = 64 lanes x 16 contiguous bytes), so every h
// load is one contiguous 1 KB per wave.
#include "tm_common.h"

namespace {

constexpr int WAVES = 4;
constexpr int ROWS = 16;           // weight rows per workgroup
constexpr int MT = TM_GEMM_TILE_M; // rows per GEMM tile (<= 4 sub-tiles)
constexpr uint32_t kOutOfRange = 0x80000000u;
constexpr int kNt = 2;             // buffer cache policy: non-temporal
constexpr int kScratchBytes = 69632;  // >= 4 waves x 2 matrices x 16 rows x 528 B


template <int NSUB>
struct Cfg {
  static constexpr int KC = NSUB <= 1 ? 256 : (NSUB == 2 ? 128 : 64);  // K elements per chunk
  static constexpr int NSTEP = KC / 32;             // MFMA k-steps per chunk
  static constexpr int WLD = KC / 32;               // 1 KB weight loads per matrix per chunk
  static constexpr int SROW = KC * 2 + 16;          // scratch row stride, bytes
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tm_buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

template <int AUX>
__device__ __forceinline__ u32x4_t ld_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
}

// 16x16x32 MFMA on bf16 or fp16 operands held as 32-bit integer vectors.
template <int DT>
__device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (DT == TM_DTYPE_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Keep the machine scheduler from sinking the next chunk's loads below the
// current chunk's MFMAs.
__device__ __forceinline__ void tm_sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// 16 weight rows of one matrix, coalesced: load q (0 <= q < WLD) covers rows
// 8*(q&1) + lane/8 and bytes 128*(q>>1) + 16*(lane%8) of the chunk.
template <int NSUB>
struct WeightRows {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t base;     // byte offset of (first row + lane/8, 16*(lane%8)) at k = 0
  uint32_t half;     // byte distance of 8 rows
  int lds_w;         // scratch byte offset written by this lane for q = 0

  __device__ __forceinline__ void load(u32x4_t (&v)[Cfg<NSUB>::WLD], uint32_t kbyte,
                                       bool valid) const {
#pragma unroll
    for (int q = 0; q < Cfg<NSUB>::WLD; ++q) {
      const uint32_t off = base + kbyte + (q & 1) * half + (q >> 1) * 128u;
      v[q] = ld_b128<kNt>(rsrc, valid ? off : kOutOfRange);
    }
  }
  __device__ __forceinline__ void stage(uint8_t* scratch,
                                        const u32x4_t (&v)[Cfg<NSUB>::WLD]) const {
#pragma unroll
    for (int q = 0; q < Cfg<NSUB>::WLD; ++q)
      *reinterpret_cast<u32x4_t*>(scratch + lds_w + (q & 1) * 8 * Cfg<NSUB>::SROW + (q >> 1) * 128) =
          v[q];
  }
};

// B fragment of k-step s from the scratch: lane l reads row l%16, k-group l/16.
template <int NSUB>
__device__ __forceinline__ u32x4_t b_frag(const uint8_t* scratch, int lane, int s) {
  return *reinterpret_cast<const u32x4_t*>(scratch + (lane & 15) * Cfg<NSUB>::SROW + s * 64 +
                                           (lane >> 4) * 16);
}

// Fixed-order sum of the 4 waves' partial accumulators (wave 0 + 1 + 2 + 3)
// through LDS; returns the total for sub-tile `sub` of matrix `mat` in the
// wave that calls it (one wave per sub-tile).
__device__ __forceinline__ f32x4_t reduce_partials(const f32x4_t* red, int nsub, int sub, int mat,
                                                   int nmat, int lane) {
  f32x4_t s = red[((0 * nsub + sub) * nmat + mat) * 64 + lane];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) {
    const f32x4_t p = red[((w * nsub + sub) * nmat + mat) * 64 + lane];
    s[0] = s[0] + p[0];
    s[1] = s[1] + p[1];
    s[2] = s[2] + p[2];
    s[3] = s[3] + p[3];
  }
  return s;
}

// ----------------------------------------------------------------- GEMM1 --
// h[p, n] = bf16( silu(sum_k x[tok(p), k] w1[e, n, k]) * sum_k x[tok(p), k] w3[e, n, k] )
template <int NSUB, int DT>
__device__ __forceinline__ void gemm1_item(uint8_t* lds, const uint16_t* x, const uint16_t* w1,
                                           const uint16_t* w3, uint16_t* __restrict__ hsw,
                                           const int32_t* __restrict__ sorted_slots, int tile,
                                           int ng, int e, int row0, int rows, int H, int I,
                                           uint32_t x_bytes) {
  using C = Cfg<NSUB>;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  uint8_t* scratch = lds + wave * 2 * ROWS * C::SROW;

  WeightRows<NSUB> wr1, wr3;
  const size_t ebase = (size_t)e * I * H;
  wr1.rsrc = tm_buffer(w1 + ebase, (uint32_t)((size_t)I * H * 2));
  wr3.rsrc = tm_buffer(w3 + ebase, (uint32_t)((size_t)I * H * 2));
  wr1.base = wr3.base = (uint32_t)(ng * ROWS + (lane >> 3)) * (uint32_t)H * 2u + (lane & 7) * 16u;
  wr1.half = wr3.half = 8u * (uint32_t)H * 2u;
  wr1.lds_w = (lane >> 3) * C::SROW + (lane & 7) * 16;
  wr3.lds_w = wr1.lds_w + ROWS * C::SROW;

  const __amdgpu_buffer_rsrc_t xr = tm_buffer(x, x_bytes);
  uint32_t xrow[NSUB];
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) {
    const int m = sub * 16 + (lane & 15);
    xrow[sub] = (m < rows)
                    ? 2u * (uint32_t)((sorted_slots[row0 + m] >> 1) * H + (lane >> 4) * 8)
                    : kOutOfRange;
  }

  f32x4_t acc1[NSUB], acc3[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    acc1[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    acc3[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  u32x4_t a1[C::WLD], a3[C::WLD], b1[C::WLD], b3[C::WLD];
  u32x4_t ax[C::NSTEP * NSUB], bx[C::NSTEP * NSUB];

  auto load = [&](u32x4_t (&w1r)[C::WLD], u32x4_t (&w3r)[C::WLD],
                  u32x4_t (&xf)[C::NSTEP * NSUB], int c, bool valid) {
    const uint32_t kb = (uint32_t)c * C::KC * 2u;
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s)
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
        xf[s * NSUB + sub] = ld_b128<0>(xr, valid ? xrow[sub] + kb + s * 64u : kOutOfRange);
    wr1.load(w1r, kb, valid);
    wr3.load(w3r, kb, valid);
  };
  auto process = [&](const u32x4_t (&w1r)[C::WLD], const u32x4_t (&w3r)[C::WLD],
                     const u32x4_t (&xf)[C::NSTEP * NSUB]) {
    wr1.stage(scratch, w1r);
    wr3.stage(scratch, w3r);
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s) {
      const u32x4_t f1 = b_frag<NSUB>(scratch, lane, s);
      const u32x4_t f3 = b_frag<NSUB>(scratch + ROWS * C::SROW, lane, s);
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        acc1[sub] = mfma16<DT>(xf[s * NSUB + sub], f1, acc1[sub]);
        acc3[sub] = mfma16<DT>(xf[s * NSUB + sub], f3, acc3[sub]);
      }
    }
  };

  const int nch = H / C::KC;
  load(a1, a3, ax, wave, wave < nch);
  // One basic block per trip (no early exit), so no load is sunk below the
  // MFMAs it should overlap.  A chunk past the end loads zeros out of range
  // and its MFMAs add exact zeros.
  for (int c = wave; c < nch; c += 2 * WAVES) {
    const int c1 = c + WAVES;
    load(b1, b3, bx, c1, c1 < nch);
    tm_sched_fence();
    process(a1, a3, ax);
    const int c2 = c1 + WAVES;
    load(a1, a3, ax, c2, c2 < nch);
    tm_sched_fence();
    process(b1, b3, bx);
  }

  // cross-wave reduction in the (now free) scratch, then the SwiGLU epilogue
  __syncthreads();
  f32x4_t* red = reinterpret_cast<f32x4_t*>(lds);
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) {
    red[((wave * NSUB + sub) * 2 + 0) * 64 + lane] = acc1[sub];
    red[((wave * NSUB + sub) * 2 + 1) * 64 + lane] = acc3[sub];
  }
  __syncthreads();
  if (wave < NSUB) {
    const int sub = wave;
    const f32x4_t s1 = reduce_partials(red, NSUB, sub, 0, 2, lane);
    const f32x4_t s3 = reduce_partials(red, NSUB, sub, 1, 2, lane);
    const int r = lane & 15, g = lane >> 4;
    const int n = ng * ROWS + r;
    const int kk = n & 31;
    const size_t frag = ((size_t)(tile * 4 + sub) * (I / 32) + (n >> 5)) * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int mm = g * 4 + i;  // row within the sub-tile
      if (sub * 16 + mm < rows) {
        const float a = s1[i];
        const float b = s3[i];
        const float hv = (a / (1.0f + __expf(-a))) * b;
        hsw[(frag + (kk >> 3) * 16 + mm) * 8 + (kk & 7)] = Half16<DT>::round(hv);
      }
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(256, 2)
tm_gemm1_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                const uint16_t* __restrict__ w3, uint16_t* __restrict__ hsw,
                const int32_t* __restrict__ sorted_slots, const int32_t* __restrict__ tiles,
                int max_tiles, int H, int I, uint32_t x_bytes, int group_major) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kScratchBytes];
  // Job order.  Group-major (weight group ng major, tile minor): consecutive
  // workgroups stream the same rows of different experts' weights, measured
  // 4-5 % faster at T = 64 (one tile per expert).  Tile-major when experts
  // have many tiles: consecutive workgroups then share one tile's x rows.
  const int gpt = I / ROWS;
  int ng, tile;
  if (group_major) {
    ng = (int)blockIdx.x / max_tiles;
    tile = (int)blockIdx.x - ng * max_tiles;
  } else {
    tile = (int)blockIdx.x / gpt;
    ng = (int)blockIdx.x - tile * gpt;
  }
  const int e = tiles[4 * tile];
  if (e < 0) return;
  const int row0 = tiles[4 * tile + 1];
  const int rows = tiles[4 * tile + 2];
  switch ((rows + 15) >> 4) {
    case 1: gemm1_item<1, DT>(lds, x, w1, w3, hsw, sorted_slots, tile, ng, e, row0, rows, H, I, x_bytes); break;
    case 2: gemm1_item<2, DT>(lds, x, w1, w3, hsw, sorted_slots, tile, ng, e, row0, rows, H, I, x_bytes); break;
    case 3: gemm1_item<3, DT>(lds, x, w1, w3, hsw, sorted_slots, tile, ng, e, row0, rows, H, I, x_bytes); break;
    default: gemm1_item<4, DT>(lds, x, w1, w3, hsw, sorted_slots, tile, ng, e, row0, rows, H, I, x_bytes); break;
  }
}

// ----------------------------------------------------------------- GEMM2 --
// y[s, p, n] = gates_flat[slot(p)] * sum_{k in segment s} h[p, k] w2[e, n, k]
// A workgroup streams two 16-row blocks of w2 (32 output columns) that share
// the h fragments, so each wave keeps as many weight bytes in flight as in
// the gate/up GEMM.
template <int NSUB, int DT>
__device__ __forceinline__ void gemm2_item(uint8_t* lds, const uint16_t* hsw, const uint16_t* w2,
                                           float* __restrict__ y,
                                           const float* __restrict__ gates_flat,
                                           const int32_t* __restrict__ sorted_slots, int tile,
                                           int e, int row0, int rows, int R, int H, int I,
                                           int klen, uint32_t h_bytes) {
  using C = Cfg<NSUB>;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int ng = blockIdx.x;  // 32 output columns
  const int split = blockIdx.y;
  const int kbase = split * klen;
  uint8_t* scratch = lds + wave * 2 * ROWS * C::SROW;

  WeightRows<NSUB> wr0, wr1;
  wr0.rsrc = wr1.rsrc = tm_buffer(w2 + (size_t)e * H * I, (uint32_t)((size_t)H * I * 2));
  wr0.base = (uint32_t)(ng * 2 * ROWS + (lane >> 3)) * (uint32_t)I * 2u + (uint32_t)kbase * 2u +
             (lane & 7) * 16u;
  wr1.base = wr0.base + (uint32_t)ROWS * (uint32_t)I * 2u;
  wr0.half = wr1.half = 8u * (uint32_t)I * 2u;
  wr0.lds_w = (lane >> 3) * C::SROW + (lane & 7) * 16;
  wr1.lds_w = wr0.lds_w + ROWS * C::SROW;

  // h fragments: sub-tile `sub`, global k-step ks -> 64 lanes x 16 contiguous bytes
  const __amdgpu_buffer_rsrc_t hr = tm_buffer(hsw, h_bytes);
  const uint32_t ksteps = (uint32_t)I / 32u;
  const uint32_t hbase = ((uint32_t)tile * 4u * ksteps + (uint32_t)kbase / 32u) * 1024u + lane * 16u;

  f32x4_t acc0[NSUB], acc1[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    acc0[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    acc1[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  u32x4_t a0[C::WLD], a1[C::WLD], b0[C::WLD], b1[C::WLD];
  u32x4_t ah[C::NSTEP * NSUB], bh[C::NSTEP * NSUB];

  auto load = [&](u32x4_t (&w0r)[C::WLD], u32x4_t (&w1r)[C::WLD],
                  u32x4_t (&hf)[C::NSTEP * NSUB], int c, bool valid) {
    const uint32_t kstep0 = (uint32_t)c * C::NSTEP;
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s)
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
        hf[s * NSUB + sub] = ld_b128<0>(
            hr, valid ? hbase + ((uint32_t)sub * ksteps + kstep0 + s) * 1024u : kOutOfRange);
    const uint32_t kb = (uint32_t)c * C::KC * 2u;
    wr0.load(w0r, kb, valid);
    wr1.load(w1r, kb, valid);
  };
  auto process = [&](const u32x4_t (&w0r)[C::WLD], const u32x4_t (&w1r)[C::WLD],
                     const u32x4_t (&hf)[C::NSTEP * NSUB]) {
    wr0.stage(scratch, w0r);
    wr1.stage(scratch, w1r);
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s) {
      const u32x4_t f0 = b_frag<NSUB>(scratch, lane, s);
      const u32x4_t f1 = b_frag<NSUB>(scratch + ROWS * C::SROW, lane, s);
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        acc0[sub] = mfma16<DT>(hf[s * NSUB + sub], f0, acc0[sub]);
        acc1[sub] = mfma16<DT>(hf[s * NSUB + sub], f1, acc1[sub]);
      }
    }
  };

  const int nch = klen / C::KC;
  load(a0, a1, ah, wave, wave < nch);
  for (int c = wave; c < nch; c += 2 * WAVES) {
    const int c1 = c + WAVES;
    load(b0, b1, bh, c1, c1 < nch);
    tm_sched_fence();
    process(a0, a1, ah);
    const int c2 = c1 + WAVES;
    load(a0, a1, ah, c2, c2 < nch);
    tm_sched_fence();
    process(b0, b1, bh);
  }

  __syncthreads();
  f32x4_t* red = reinterpret_cast<f32x4_t*>(lds);
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) {
    red[((wave * NSUB + sub) * 2 + 0) * 64 + lane] = acc0[sub];
    red[((wave * NSUB + sub) * 2 + 1) * 64 + lane] = acc1[sub];
  }
  __syncthreads();
  if (wave < NSUB) {
    const int sub = wave;
    const f32x4_t s0 = reduce_partials(red, NSUB, sub, 0, 2, lane);
    const f32x4_t s1 = reduce_partials(red, NSUB, sub, 1, 2, lane);
    const int r = lane & 15, g = lane >> 4;
    const int n = ng * 2 * ROWS + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = sub * 16 + g * 4 + i;
      if (m < rows) {
        const int p = row0 + m;
        const float gate = gates_flat[sorted_slots[p]];
        float* yr = y + ((size_t)split * R + p) * H;
        yr[n] = s0[i] * gate;
        yr[n + ROWS] = s1[i] * gate;
      }
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(256, 2)
tm_gemm2_kernel(const uint16_t* __restrict__ hsw, const uint16_t* __restrict__ w2,
                float* __restrict__ y, const float* __restrict__ gates_flat,
                const int32_t* __restrict__ sorted_slots, const int32_t* __restrict__ tiles,
                int R, int H, int I, int klen, uint32_t h_bytes) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kScratchBytes];
  const int tile = blockIdx.z;
  const int e = tiles[4 * tile];
  if (e < 0) return;
  const int row0 = tiles[4 * tile + 1];
  const int rows = tiles[4 * tile + 2];
  switch ((rows + 15) >> 4) {
    case 1: gemm2_item<1, DT>(lds, hsw, w2, y, gates_flat, sorted_slots, tile, e, row0, rows, R, H, I, klen, h_bytes); break;
    case 2: gemm2_item<2, DT>(lds, hsw, w2, y, gates_flat, sorted_slots, tile, e, row0, rows, R, H, I, klen, h_bytes); break;
    case 3: gemm2_item<3, DT>(lds, hsw, w2, y, gates_flat, sorted_slots, tile, e, row0, rows, R, H, I, klen, h_bytes); break;
    default: gemm2_item<4, DT>(lds, hsw, w2, y, gates_flat, sorted_slots, tile, e, row0, rows, R, H, I, klen, h_bytes); break;
  }
}

static_assert(kScratchBytes >= WAVES * 2 * ROWS * Cfg<1>::SROW, "gemm1 scratch");
static_assert(kScratchBytes >= WAVES * 4 * 2 * 64 * 16, "gemm1 reduction");

// --------------------------------------------------------------- combine --
// out[t, n] = bf16( sum over (k = 0, 1) of sum over split s of y[s, pos(2t+k), n] ),
// accumulated in exactly that order from 0.  SC > 0 is the split count known
// at compile time: all 2 SC loads are issued before the first add, so the
// thread waits for one memory round trip instead of one per partial (with a
// run-time count the loop waits for each load before the next is issued).
template <int DT, int SC>
__global__ void __launch_bounds__(256)
tm_combine_kernel(const float* __restrict__ y, const int32_t* __restrict__ slot_pos,
                  uint16_t* __restrict__ out, int T, int H, int S, int R) {
  const int t = blockIdx.x;
  const int n = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (n >= H) return;
  const int p0 = slot_pos[2 * t];
  const int p1 = slot_pos[2 * t + 1];
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  if constexpr (SC > 0) {
    float4 v[2 * SC];
#pragma unroll
    for (int s = 0; s < SC; ++s) {
      v[s] = *reinterpret_cast<const float4*>(y + ((size_t)s * R + p0) * H + n);
      v[SC + s] = *reinterpret_cast<const float4*>(y + ((size_t)s * R + p1) * H + n);
    }
#pragma unroll
    for (int i = 0; i < 2 * SC; ++i) {
      a0 = a0 + v[i].x; a1 = a1 + v[i].y; a2 = a2 + v[i].z; a3 = a3 + v[i].w;
    }
  } else {
    for (int s = 0; s < S; ++s) {
      const float4 v = *reinterpret_cast<const float4*>(y + ((size_t)s * R + p0) * H + n);
      a0 = a0 + v.x; a1 = a1 + v.y; a2 = a2 + v.z; a3 = a3 + v.w;
    }
    for (int s = 0; s < S; ++s) {
      const float4 v = *reinterpret_cast<const float4*>(y + ((size_t)s * R + p1) * H + n);
      a0 = a0 + v.x; a1 = a1 + v.y; a2 = a2 + v.z; a3 = a3 + v.w;
    }
  }
  u16x4_t o;
  o[0] = Half16<DT>::round(a0);
  o[1] = Half16<DT>::round(a1);
  o[2] = Half16<DT>::round(a2);
  o[3] = Half16<DT>::round(a3);
  *reinterpret_cast<u16x4_t*>(out + (size_t)t * H + n) = o;
}

bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

}  // namespace

extern "C" int tm_op1_gemm1(const void* x, const void* w1, const void* w3, void* h,
                            const int32_t* sorted_slots, const int32_t* tiles,
                            int64_t max_tiles, int64_t T, int64_t H, int64_t I, int64_t E,
                            int dtype, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS) return TM_ERR_SHAPE;
  if (H < 256 || (H % 256) != 0 || I < 256 || (I % 256) != 0 || max_tiles < 1)
    return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_BF16 && dtype != TM_DTYPE_F16) return TM_ERR_ARG;
  if (I * H * 2 >= (int64_t)kOutOfRange || T * H * 2 >= (int64_t)kOutOfRange ||
      max_tiles * MT * I * 2 >= (int64_t)kOutOfRange)
    return TM_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w1) || !aligned16(w3) || !aligned16(h)) return TM_ERR_ALIGN;
  if ((I / ROWS) * max_tiles > INT32_MAX) return TM_ERR_SHAPE;
  const dim3 grid((unsigned)((I / ROWS) * max_tiles));
  hipLaunchKernelGGL(dtype == TM_DTYPE_F16 ? tm_gemm1_kernel<TM_DTYPE_F16>
                                           : tm_gemm1_kernel<TM_DTYPE_BF16>,
                     grid, dim3(64 * WAVES), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)w1, (const uint16_t*)w3,
                     (uint16_t*)h, sorted_slots, tiles, (int)max_tiles, (int)H, (int)I,
                     (uint32_t)(T * H * 2), max_tiles <= 2 * E ? 1 : 0);
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op1_gemm2(const void* h, const void* w2, float* y,
                            const float* gates_flat, const int32_t* sorted_slots,
                            const int32_t* tiles, int64_t max_tiles, int64_t split,
                            int64_t T, int64_t H, int64_t I, int64_t E, int dtype,
                            void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS) return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_BF16 && dtype != TM_DTYPE_F16) return TM_ERR_ARG;
  if (split < 1 || (I % split) != 0) return TM_ERR_SHAPE;
  const int64_t klen = I / split;
  if (klen < 256 || (klen % 256) != 0 || H < 2 * ROWS || (H % (2 * ROWS)) != 0 ||
      max_tiles < 1)
    return TM_ERR_SHAPE;
  if (H * I * 2 >= (int64_t)kOutOfRange || max_tiles * MT * I * 2 >= (int64_t)kOutOfRange)
    return TM_ERR_SHAPE;
  if (!aligned16(h) || !aligned16(w2)) return TM_ERR_ALIGN;
  const dim3 grid((unsigned)(H / (2 * ROWS)), (unsigned)split, (unsigned)max_tiles);
  hipLaunchKernelGGL(dtype == TM_DTYPE_F16 ? tm_gemm2_kernel<TM_DTYPE_F16>
                                           : tm_gemm2_kernel<TM_DTYPE_BF16>,
                     grid, dim3(64 * WAVES), 0, (hipStream_t)stream,
                     (const uint16_t*)h, (const uint16_t*)w2, y, gates_flat, sorted_slots,
                     tiles, (int)(2 * T), (int)H, (int)I, (int)klen,
                     (uint32_t)(max_tiles * MT * I * 2));
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op1_combine(const float* y, const int32_t* slot_pos, void* out, int64_t T,
                              int64_t H, int64_t split, int dtype, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || H < 4 || (H % 4) != 0 || split < 1) return TM_ERR_SHAPE;
  if (dtype != TM_DTYPE_BF16 && dtype != TM_DTYPE_F16) return TM_ERR_ARG;
  if (!aligned16(y) || ((uintptr_t)out % 8) != 0) return TM_ERR_ALIGN;
  const dim3 grid((unsigned)T, (unsigned)((H + 1023) / 1024));
  const bool f16 = dtype == TM_DTYPE_F16;
  void (*kern)(const float*, const int32_t*, uint16_t*, int, int, int, int);
  switch (split) {  // the split counts the forward uses
    case 1: kern = f16 ? tm_combine_kernel<TM_DTYPE_F16, 1> : tm_combine_kernel<TM_DTYPE_BF16, 1>; break;
    case 2: kern = f16 ? tm_combine_kernel<TM_DTYPE_F16, 2> : tm_combine_kernel<TM_DTYPE_BF16, 2>; break;
    case 4: kern = f16 ? tm_combine_kernel<TM_DTYPE_F16, 4> : tm_combine_kernel<TM_DTYPE_BF16, 4>; break;
    default: kern = f16 ? tm_combine_kernel<TM_DTYPE_F16, 0> : tm_combine_kernel<TM_DTYPE_BF16, 0>;
  }
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, (hipStream_t)stream, y, slot_pos,
                     (uint16_t*)out, (int)T, (int)H, (int)split, (int)(2 * T));
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}
