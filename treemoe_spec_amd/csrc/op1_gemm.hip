// op1 expert GEMMs on gfx950: gate/up + SwiGLU, down projection with a
// deterministic K split, and the fixed-order combine.
//
// Work unit = (GEMM tile of <= 64 sorted rows of one expert) x (64 weight rows).
// A workgroup is 4 waves; wave w owns 16 weight rows and all (<= 4) 16-row
// sub-tiles of the tile, so every weight byte is read from HBM exactly once per
// tile.  Weights go global -> VGPR with 16-byte non-temporal loads laid out as
// the B operand of v_mfma_f32_16x16x32_bf16 (lane l: weight row l%16, k-group
// l/16), one 256-element K chunk ahead of the MFMAs.  The activation rows
// (x gathered by token, or h) are staged through a double-buffered LDS tile.
#include "tm_common.h"

namespace {

constexpr int KC = 256;            // K elements per staged chunk
constexpr int LDS_LD = KC + 8;     // padded LDS row, elements (528 B, 16 B aligned)
constexpr int NSTEP = KC / 32;     // MFMA k-steps per chunk
constexpr int MT = TM_GEMM_TILE_M; // rows per tile
constexpr int NWAVE = 4;
constexpr int BN = 16 * NWAVE;     // weight rows per workgroup
constexpr int XPIECES = (MT * KC / 8) / (64 * NWAVE);  // 16-byte pieces per thread per chunk

static_assert(XPIECES == 8, "staging map assumes 8 pieces per thread");

__device__ __forceinline__ bf16x8_t ld_weight(const bf16x8_t* p) {
  return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Row sources of the LDS activation tile.  Thread tid stages pieces
// p = tid + 256*i: tile row (tid >> 5) + 8*i, columns (tid & 31)*8 .. +8.
struct RowStage {
  const uint16_t* src[XPIECES];  // nullptr: row outside the tile -> zeros
  int col;
  int row0;

  __device__ __forceinline__ void load(uint4 (&v)[XPIECES], int k0) const {
#pragma unroll
    for (int i = 0; i < XPIECES; ++i) {
      if (src[i] != nullptr) {
        v[i] = *reinterpret_cast<const uint4*>(src[i] + k0);
      } else {
        v[i] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* lds, const uint4 (&v)[XPIECES], int nrows) const {
#pragma unroll
    for (int i = 0; i < XPIECES; ++i) {
      const int m = row0 + 8 * i;
      if (m < nrows) *reinterpret_cast<uint4*>(lds + m * LDS_LD + col) = v[i];
    }
  }
};

// ----------------------------------------------------------------- GEMM1 --
// h[p, n] = bf16( silu(sum_k x[tok(p), k] w1[e, n, k]) * sum_k x[tok(p), k] w3[e, n, k] )
__global__ void __launch_bounds__(256, 2)
tm_gemm1_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                const uint16_t* __restrict__ w3, uint16_t* __restrict__ h,
                const int32_t* __restrict__ sorted_slots, const int32_t* __restrict__ tiles,
                int H, int I) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][MT * LDS_LD];
  const int tile = blockIdx.y;
  const int e = tiles[4 * tile];
  if (e < 0) return;
  const int row0 = tiles[4 * tile + 1];
  const int rows = tiles[4 * tile + 2];
  const int nsub = (rows + 15) >> 4;
  const int srows = nsub * 16;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int n = blockIdx.x * BN + wave * 16 + r;
  const size_t wrow = ((size_t)e * I + n) * (size_t)H;
  const bf16x8_t* w1p = reinterpret_cast<const bf16x8_t*>(w1 + wrow) + g;
  const bf16x8_t* w3p = reinterpret_cast<const bf16x8_t*>(w3 + wrow) + g;

  RowStage st;
  st.row0 = tid >> 5;
  st.col = (tid & 31) * 8;
#pragma unroll
  for (int i = 0; i < XPIECES; ++i) {
    const int m = st.row0 + 8 * i;
    st.src[i] = (m < rows) ? x + (size_t)(sorted_slots[row0 + m] >> 1) * H + st.col : nullptr;
  }

  f32x4_t acc1[4], acc3[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    acc1[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    acc3[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  bf16x8_t wa1[NSTEP], wa3[NSTEP], wb1[NSTEP], wb3[NSTEP];
  uint4 xv[XPIECES];

  auto load_w = [&](bf16x8_t (&d1)[NSTEP], bf16x8_t (&d3)[NSTEP], int c) {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
      d1[s] = ld_weight(w1p + c * (KC / 8) + s * 4);
      d3[s] = ld_weight(w3p + c * (KC / 8) + s * 4);
    }
  };
  auto compute = [&](const uint16_t* lds, const bf16x8_t (&b1)[NSTEP], const bf16x8_t (&b3)[NSTEP]) {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        if (sub < nsub) {
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(lds + (sub * 16 + r) * LDS_LD + s * 32 + g * 8);
          acc1[sub] = mfma16(a, b1[s], acc1[sub]);
          acc3[sub] = mfma16(a, b3[s], acc3[sub]);
        }
      }
    }
  };

  const int nch = H / KC;
  load_w(wa1, wa3, 0);
  st.load(xv, 0);
  st.store(xs[0], xv, srows);
  tm_lds_barrier();
  for (int c = 0; c < nch; c += 2) {
    const bool has1 = (c + 1) < nch;
    if (has1) {
      load_w(wb1, wb3, c + 1);
      st.load(xv, (c + 1) * KC);
    }
    compute(xs[0], wa1, wa3);
    if (!has1) break;
    st.store(xs[1], xv, srows);
    tm_lds_barrier();
    const bool has2 = (c + 2) < nch;
    if (has2) {
      load_w(wa1, wa3, c + 2);
      st.load(xv, (c + 2) * KC);
    }
    compute(xs[1], wb1, wb3);
    if (has2) {
      st.store(xs[0], xv, srows);
      tm_lds_barrier();
    }
  }

  // epilogue: lane holds C[m = 4g + i][n] of each sub-tile
#pragma unroll
  for (int sub = 0; sub < 4; ++sub) {
    if (sub < nsub) {
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
}

// ----------------------------------------------------------------- GEMM2 --
// y[s, p, n] = gates_flat[slot(p)] * sum_{k in segment s} h[p, k] w2[e, n, k]
__global__ void __launch_bounds__(256, 2)
tm_gemm2_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ w2,
                float* __restrict__ y, const float* __restrict__ gates_flat,
                const int32_t* __restrict__ sorted_slots, const int32_t* __restrict__ tiles,
                int R, int H, int I, int klen) {
  __shared__ __attribute__((aligned(16))) uint16_t hs[2][MT * LDS_LD];
  const int tile = blockIdx.z;
  const int e = tiles[4 * tile];
  if (e < 0) return;
  const int row0 = tiles[4 * tile + 1];
  const int rows = tiles[4 * tile + 2];
  const int nsub = (rows + 15) >> 4;
  const int srows = nsub * 16;
  const int split = blockIdx.y;
  const int kbase = split * klen;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int n = blockIdx.x * BN + wave * 16 + r;
  const bf16x8_t* w2p =
      reinterpret_cast<const bf16x8_t*>(w2 + ((size_t)e * H + n) * (size_t)I + kbase) + g;

  RowStage st;
  st.row0 = tid >> 5;
  st.col = (tid & 31) * 8;
#pragma unroll
  for (int i = 0; i < XPIECES; ++i) {
    const int m = st.row0 + 8 * i;
    st.src[i] = (m < rows) ? h + (size_t)(row0 + m) * I + kbase + st.col : nullptr;
  }

  f32x4_t acc[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) acc[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  bf16x8_t wa[NSTEP], wb[NSTEP];
  uint4 xv[XPIECES];

  auto load_w = [&](bf16x8_t (&d)[NSTEP], int c) {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) d[s] = ld_weight(w2p + c * (KC / 8) + s * 4);
  };
  auto compute = [&](const uint16_t* lds, const bf16x8_t (&b)[NSTEP]) {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        if (sub < nsub) {
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(lds + (sub * 16 + r) * LDS_LD + s * 32 + g * 8);
          acc[sub] = mfma16(a, b[s], acc[sub]);
        }
      }
    }
  };

  const int nch = klen / KC;
  load_w(wa, 0);
  st.load(xv, 0);
  st.store(hs[0], xv, srows);
  tm_lds_barrier();
  for (int c = 0; c < nch; c += 2) {
    const bool has1 = (c + 1) < nch;
    if (has1) {
      load_w(wb, c + 1);
      st.load(xv, (c + 1) * KC);
    }
    compute(hs[0], wa);
    if (!has1) break;
    st.store(hs[1], xv, srows);
    tm_lds_barrier();
    const bool has2 = (c + 2) < nch;
    if (has2) {
      load_w(wa, c + 2);
      st.load(xv, (c + 2) * KC);
    }
    compute(hs[1], wb);
    if (has2) {
      st.store(hs[0], xv, srows);
      tm_lds_barrier();
    }
  }

#pragma unroll
  for (int sub = 0; sub < 4; ++sub) {
    if (sub < nsub) {
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
  if ((int64_t)E * I * H > (int64_t)1 << 40) return TM_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w1) || !aligned16(w3)) return TM_ERR_ALIGN;
  const dim3 grid((unsigned)(I / BN), (unsigned)max_tiles);
  hipLaunchKernelGGL(tm_gemm1_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)w1, (const uint16_t*)w3,
                     (uint16_t*)h, sorted_slots, tiles, (int)H, (int)I);
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
  if ((int64_t)E * I * H > (int64_t)1 << 40) return TM_ERR_SHAPE;
  if (!aligned16(h) || !aligned16(w2)) return TM_ERR_ALIGN;
  const dim3 grid((unsigned)(H / BN), (unsigned)split, (unsigned)max_tiles);
  hipLaunchKernelGGL(tm_gemm2_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)h, (const uint16_t*)w2, y, gates_flat, sorted_slots,
                     tiles, (int)(2 * T), (int)H, (int)I, (int)klen);
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
