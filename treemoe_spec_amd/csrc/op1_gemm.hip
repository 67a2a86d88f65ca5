// op1 expert GEMMs on gfx950: gate/up + SwiGLU, down projection with a
// deterministic K split, and the fixed-order combine.
//
// Work unit = (GEMM tile of <= 64 sorted rows of one expert) x (64 weight rows).
// A workgroup is 4 waves; wave w owns 16 weight rows and all 16-row sub-tiles
// of the tile (NSUB = 1..4, a template parameter chosen per tile), so every
// weight byte is read from HBM once per tile.  Weights go global -> VGPR with
// 16-byte non-temporal buffer loads laid out as the B operand of
// v_mfma_f32_16x16x32_bf16 (lane l: weight row l%16, k-group l/16), one
// 256-element K chunk ahead of the MFMAs.  Activation rows (x gathered by
// token, or h) are staged through a double-buffered LDS tile; a chunk's
// activation loads are issued before its weight loads, so storing them to LDS
// waits only for older loads and the next chunk's weights stay in flight
// across the workgroup barrier.  The loop has no data-dependent branches: the
// prefetch past the last chunk uses an out-of-range buffer offset, which
// returns zeros without touching memory.
#include "tm_common.h"

namespace {

constexpr int KC = 256;            // K elements per staged chunk
constexpr int LDS_LD = KC + 8;     // padded LDS row, elements (528 B, 16 B aligned)
constexpr int NSTEP = KC / 32;     // MFMA k-steps per chunk
constexpr int MT = TM_GEMM_TILE_M; // rows per tile
constexpr int NWAVE = 4;
constexpr int BN = 16 * NWAVE;     // weight rows per workgroup
constexpr uint32_t kOutOfRange = 0x80000000u;
constexpr int kNt = 2;             // buffer cache policy: non-temporal

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tm_buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Operands travel as 32-bit integer vectors and become bf16x8 only at the MFMA
// (bf16 vectors built from integer loads would be repacked element-wise).
template <int AUX>
__device__ __forceinline__ u32x4_t ld_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
}

__device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Activation tile rows staged for NSUB sub-tiles: thread tid stages pieces
// p = tid + 256*i (i < 2*NSUB): tile row (tid >> 5) + 8*i, columns
// (tid & 31)*8 .. +8.  off[i] is the byte offset of that row segment at k = 0,
// or kOutOfRange for rows past the tile (zeros).
template <int NSUB>
struct Acts {
  static constexpr int XP = 2 * NSUB;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off[XP];
  int lds_off;  // element offset of this thread's first piece in a stage

  __device__ __forceinline__ void load(u32x4_t (&v)[XP], uint32_t kbyte, bool valid) const {
#pragma unroll
    for (int i = 0; i < XP; ++i) v[i] = ld_b128<0>(rsrc, valid ? off[i] + kbyte : kOutOfRange);
  }
  __device__ __forceinline__ void store(uint16_t* stage, const u32x4_t (&v)[XP]) const {
#pragma unroll
    for (int i = 0; i < XP; ++i)
      *reinterpret_cast<u32x4_t*>(stage + lds_off + 8 * i * LDS_LD) = v[i];
  }
};

// Weight rows of one matrix for this lane: row n (within the expert), k-group g.
struct Weights {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off;  // byte offset of (n, 8g) at the first chunk

  __device__ __forceinline__ void load(u32x4_t (&w)[NSTEP], uint32_t kbyte, bool valid) const {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s)
      w[s] = ld_b128<kNt>(rsrc, valid ? off + kbyte + 64u * s : kOutOfRange);
  }
};

// Keep the machine scheduler from sinking the next chunk's loads below the
// current chunk's MFMAs (which would shrink the bytes in flight to a few KB).
__device__ __forceinline__ void tm_sched_fence() { __builtin_amdgcn_sched_barrier(0); }

__device__ __forceinline__ u32x4_t lds_frag(const uint16_t* stage, int row, int s, int g) {
  return *reinterpret_cast<const u32x4_t*>(stage + row * LDS_LD + s * 32 + g * 8);
}

// ----------------------------------------------------------------- GEMM1 --
// h[p, n] = bf16( silu(sum_k x[tok(p), k] w1[e, n, k]) * sum_k x[tok(p), k] w3[e, n, k] )
template <int NSUB>
__device__ __forceinline__ void gemm1_body(uint16_t* __restrict__ lds, const uint16_t* x,
                                           const uint16_t* w1, const uint16_t* w3,
                                           uint16_t* __restrict__ h,
                                           const int32_t* __restrict__ sorted_slots, int e,
                                           int row0, int rows, int H, int I, uint32_t x_bytes) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int n = blockIdx.x * BN + wave * 16 + r;
  const size_t ebase = (size_t)e * I * H;

  Acts<NSUB> act;
  act.rsrc = tm_buffer(x, x_bytes);
  act.lds_off = (tid >> 5) * LDS_LD + (tid & 31) * 8;
#pragma unroll
  for (int i = 0; i < Acts<NSUB>::XP; ++i) {
    const int m = (tid >> 5) + 8 * i;
    act.off[i] = (m < rows) ? 2u * (uint32_t)((sorted_slots[row0 + m] >> 1) * H + (tid & 31) * 8)
                            : kOutOfRange;
  }
  Weights wt1, wt3;
  wt1.rsrc = tm_buffer(w1 + ebase, (uint32_t)((size_t)I * H * 2));
  wt3.rsrc = tm_buffer(w3 + ebase, (uint32_t)((size_t)I * H * 2));
  wt1.off = wt3.off = 2u * (uint32_t)(n * H + g * 8);

  f32x4_t acc1[NSUB], acc3[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    acc1[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    acc3[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  u32x4_t a1[NSTEP], a3[NSTEP], b1[NSTEP], b3[NSTEP];
  u32x4_t xr[Acts<NSUB>::XP];
  uint16_t* L0 = lds;
  uint16_t* L1 = lds + MT * LDS_LD;

  auto compute = [&](const uint16_t* stage, const u32x4_t (&w1r)[NSTEP],
                     const u32x4_t (&w3r)[NSTEP]) {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const u32x4_t a = lds_frag(stage, sub * 16 + r, s, g);
        acc1[sub] = mfma16(a, w1r[s], acc1[sub]);
        acc3[sub] = mfma16(a, w3r[s], acc3[sub]);
      }
    }
  };

  const int nch = H / KC;
  act.load(xr, 0, true);
  wt1.load(a1, 0, true);
  wt3.load(a3, 0, true);
  act.store(L0, xr);
  tm_lds_barrier();
  for (int c = 0; c + 1 < nch; c += 2) {
    const uint32_t k1 = (uint32_t)(c + 1) * KC * 2;
    act.load(xr, k1, true);
    wt1.load(b1, k1, true);
    wt3.load(b3, k1, true);
    tm_sched_fence();
    compute(L0, a1, a3);
    act.store(L1, xr);
    tm_lds_barrier();
    const bool more = (c + 2) < nch;
    const uint32_t k2 = (uint32_t)(c + 2) * KC * 2;
    act.load(xr, k2, more);
    wt1.load(a1, k2, more);
    wt3.load(a3, k2, more);
    tm_sched_fence();
    compute(L1, b1, b3);
    act.store(L0, xr);
    tm_lds_barrier();
  }
  if (nch & 1) compute(L0, a1, a3);

  // epilogue: lane holds C[m = 4g + i][n] of each sub-tile
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = sub * 16 + g * 4 + i;
      if (m < rows) {
        const float a = acc1[sub][i];
        const float b = acc3[sub][i];
        const float hv = (a / (1.0f + __expf(-a))) * b;
        h[(size_t)(row0 + m) * I + n] = tm_f32_to_bf16(hv);
      }
    }
  }
}

__global__ void __launch_bounds__(256, 2)
tm_gemm1_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                const uint16_t* __restrict__ w3, uint16_t* __restrict__ h,
                const int32_t* __restrict__ sorted_slots, const int32_t* __restrict__ tiles,
                int H, int I, uint32_t x_bytes) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * MT * LDS_LD];
  const int tile = blockIdx.y;
  const int e = tiles[4 * tile];
  if (e < 0) return;
  const int row0 = tiles[4 * tile + 1];
  const int rows = tiles[4 * tile + 2];
  switch ((rows + 15) >> 4) {
    case 1: gemm1_body<1>(lds, x, w1, w3, h, sorted_slots, e, row0, rows, H, I, x_bytes); break;
    case 2: gemm1_body<2>(lds, x, w1, w3, h, sorted_slots, e, row0, rows, H, I, x_bytes); break;
    case 3: gemm1_body<3>(lds, x, w1, w3, h, sorted_slots, e, row0, rows, H, I, x_bytes); break;
    default: gemm1_body<4>(lds, x, w1, w3, h, sorted_slots, e, row0, rows, H, I, x_bytes); break;
  }
}

// ----------------------------------------------------------------- GEMM2 --
// y[s, p, n] = gates_flat[slot(p)] * sum_{k in segment s} h[p, k] w2[e, n, k]
template <int NSUB>
__device__ __forceinline__ void gemm2_body(uint16_t* __restrict__ lds, const uint16_t* h,
                                           const uint16_t* w2, float* __restrict__ y,
                                           const float* __restrict__ gates_flat,
                                           const int32_t* __restrict__ sorted_slots, int e,
                                           int row0, int rows, int R, int H, int I, int klen,
                                           uint32_t h_bytes) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int n = blockIdx.x * BN + wave * 16 + r;
  const int split = blockIdx.y;
  const int kbase = split * klen;

  Acts<NSUB> act;
  act.rsrc = tm_buffer(h, h_bytes);
  act.lds_off = (tid >> 5) * LDS_LD + (tid & 31) * 8;
#pragma unroll
  for (int i = 0; i < Acts<NSUB>::XP; ++i) {
    const int m = (tid >> 5) + 8 * i;
    act.off[i] = (m < rows) ? 2u * (uint32_t)((row0 + m) * I + kbase + (tid & 31) * 8)
                            : kOutOfRange;
  }
  Weights wt;
  wt.rsrc = tm_buffer(w2 + (size_t)e * H * I, (uint32_t)((size_t)H * I * 2));
  wt.off = 2u * (uint32_t)(n * I + kbase + g * 8);

  f32x4_t acc[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) acc[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  u32x4_t wa[NSTEP], wb[NSTEP];
  u32x4_t xr[Acts<NSUB>::XP];
  uint16_t* L0 = lds;
  uint16_t* L1 = lds + MT * LDS_LD;

  auto compute = [&](const uint16_t* stage, const u32x4_t (&wr)[NSTEP]) {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
        acc[sub] = mfma16(lds_frag(stage, sub * 16 + r, s, g), wr[s], acc[sub]);
    }
  };

  const int nch = klen / KC;
  act.load(xr, 0, true);
  wt.load(wa, 0, true);
  act.store(L0, xr);
  tm_lds_barrier();
  for (int c = 0; c + 1 < nch; c += 2) {
    const uint32_t k1 = (uint32_t)(c + 1) * KC * 2;
    act.load(xr, k1, true);
    wt.load(wb, k1, true);
    tm_sched_fence();
    compute(L0, wa);
    act.store(L1, xr);
    tm_lds_barrier();
    const bool more = (c + 2) < nch;
    const uint32_t k2 = (uint32_t)(c + 2) * KC * 2;
    act.load(xr, k2, more);
    wt.load(wa, k2, more);
    tm_sched_fence();
    compute(L1, wb);
    act.store(L0, xr);
    tm_lds_barrier();
  }
  if (nch & 1) compute(L0, wa);

#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = sub * 16 + g * 4 + i;
      if (m < rows) {
        const int p = row0 + m;
        const float gate = gates_flat[sorted_slots[p]];
        y[((size_t)split * R + p) * H + n] = acc[sub][i] * gate;
      }
    }
  }
}

__global__ void __launch_bounds__(256, 2)
tm_gemm2_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ w2,
                float* __restrict__ y, const float* __restrict__ gates_flat,
                const int32_t* __restrict__ sorted_slots, const int32_t* __restrict__ tiles,
                int R, int H, int I, int klen, uint32_t h_bytes) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * MT * LDS_LD];
  const int tile = blockIdx.z;
  const int e = tiles[4 * tile];
  if (e < 0) return;
  const int row0 = tiles[4 * tile + 1];
  const int rows = tiles[4 * tile + 2];
  switch ((rows + 15) >> 4) {
    case 1: gemm2_body<1>(lds, h, w2, y, gates_flat, sorted_slots, e, row0, rows, R, H, I, klen, h_bytes); break;
    case 2: gemm2_body<2>(lds, h, w2, y, gates_flat, sorted_slots, e, row0, rows, R, H, I, klen, h_bytes); break;
    case 3: gemm2_body<3>(lds, h, w2, y, gates_flat, sorted_slots, e, row0, rows, R, H, I, klen, h_bytes); break;
    default: gemm2_body<4>(lds, h, w2, y, gates_flat, sorted_slots, e, row0, rows, R, H, I, klen, h_bytes); break;
  }
}

// --------------------------------------------------------------- combine --
// out[t, n] = bf16( sum over (k = 0, 1) of sum over split s of y[s, pos(2t+k), n] ),
// accumulated in exactly that order from 0.
__global__ void __launch_bounds__(256)
tm_combine_kernel(const float* __restrict__ y, const int32_t* __restrict__ slot_pos,
                  uint16_t* __restrict__ out, int T, int H, int S, int R) {
  const int t = blockIdx.x;
  const int n = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (n >= H) return;
  const int p0 = slot_pos[2 * t];
  const int p1 = slot_pos[2 * t + 1];
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int s = 0; s < S; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(y + ((size_t)s * R + p0) * H + n);
    a0 = a0 + v.x; a1 = a1 + v.y; a2 = a2 + v.z; a3 = a3 + v.w;
  }
  for (int s = 0; s < S; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(y + ((size_t)s * R + p1) * H + n);
    a0 = a0 + v.x; a1 = a1 + v.y; a2 = a2 + v.z; a3 = a3 + v.w;
  }
  u16x4_t o;
  o[0] = tm_f32_to_bf16(a0);
  o[1] = tm_f32_to_bf16(a1);
  o[2] = tm_f32_to_bf16(a2);
  o[3] = tm_f32_to_bf16(a3);
  *reinterpret_cast<u16x4_t*>(out + (size_t)t * H + n) = o;
}

bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

}  // namespace

extern "C" int tm_op1_gemm1(const void* x, const void* w1, const void* w3, void* h,
                            const int32_t* sorted_slots, const int32_t* tiles,
                            int64_t max_tiles, int64_t T, int64_t H, int64_t I, int64_t E,
                            void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS) return TM_ERR_SHAPE;
  if (H < KC || (H % KC) != 0 || I < BN || (I % BN) != 0 || max_tiles < 1) return TM_ERR_SHAPE;
  if (I * H * 2 >= (int64_t)kOutOfRange || T * H * 2 >= (int64_t)kOutOfRange)
    return TM_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w1) || !aligned16(w3)) return TM_ERR_ALIGN;
  const dim3 grid((unsigned)(I / BN), (unsigned)max_tiles);
  hipLaunchKernelGGL(tm_gemm1_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)w1, (const uint16_t*)w3,
                     (uint16_t*)h, sorted_slots, tiles, (int)H, (int)I,
                     (uint32_t)(T * H * 2));
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op1_gemm2(const void* h, const void* w2, float* y,
                            const float* gates_flat, const int32_t* sorted_slots,
                            const int32_t* tiles, int64_t max_tiles, int64_t split,
                            int64_t T, int64_t H, int64_t I, int64_t E, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || E < 2 || E > TM_MAX_EXPERTS) return TM_ERR_SHAPE;
  if (split < 1 || (I % split) != 0) return TM_ERR_SHAPE;
  const int64_t klen = I / split;
  if (klen < KC || (klen % KC) != 0 || H < BN || (H % BN) != 0 || max_tiles < 1) return TM_ERR_SHAPE;
  if (H * I * 2 >= (int64_t)kOutOfRange || 2 * T * I * 2 >= (int64_t)kOutOfRange)
    return TM_ERR_SHAPE;
  if (!aligned16(h) || !aligned16(w2)) return TM_ERR_ALIGN;
  const dim3 grid((unsigned)(H / BN), (unsigned)split, (unsigned)max_tiles);
  hipLaunchKernelGGL(tm_gemm2_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)h, (const uint16_t*)w2, y, gates_flat, sorted_slots,
                     tiles, (int)(2 * T), (int)H, (int)I, (int)klen,
                     (uint32_t)(2 * T * I * 2));
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}

extern "C" int tm_op1_combine(const float* y, const int32_t* slot_pos, void* out, int64_t T,
                              int64_t H, int64_t split, void* stream) {
  if (T < 1 || T > TM_MAX_TOKENS || H < 4 || (H % 4) != 0 || split < 1) return TM_ERR_SHAPE;
  if (!aligned16(y) || ((uintptr_t)out % 8) != 0) return TM_ERR_ALIGN;
  const dim3 grid((unsigned)T, (unsigned)((H + 1023) / 1024));
  hipLaunchKernelGGL(tm_combine_kernel, grid, dim3(256), 0, (hipStream_t)stream, y, slot_pos,
                     (uint16_t*)out, (int)T, (int)H, (int)split, (int)(2 * T));
  TM_HIP_CHECK_LAUNCH();
  return TM_OK;
}
