// Shared pieces of the log-linear Mamba-2 kernels (forward and backward):
// constants, the segment size, chunk staging through buffer loads, and the
// per-segment summary kernel Sum(q) = sum_t exp(G_end(q) - G_t) k_t v_t^T.
#pragma once

#include <cstddef>

#include "common.h"

namespace hattn {

constexpr int kBT = 64;       // chunk length (the reference's only chunk size)
constexpr int kKD = 64;       // head dim of q / k
constexpr int kMaxLoc = 4;    // local levels held in registers (S <= 16 chunks)
constexpr int kMaxTop = 8;    // top levels (LDS-resident, T <= 64 * 2^12)
constexpr int kMaxLU = 7 + kMaxLoc + kMaxTop;  // lambda columns read (levels 0 .. 6 + nlev)
constexpr int kLd = 72;       // LDS row stride (bf16) of 64-wide tiles

// Chunks per segment: 16 (2^kMaxLoc), or the whole sequence when shorter.
__host__ __device__ inline int seg_log2(int NT) {
  int nlev = 0;
  while ((1 << nlev) < NT) ++nlev;
  return nlev < kMaxLoc ? nlev : kMaxLoc;
}

// ---------------------------------------------------------------------------
// chunk staging shared by both kernels
// ---------------------------------------------------------------------------
// Row-major 64 x 64 bf16 tile of a [.., T, heads, 64-block] tensor: 512 units
// of 16 bytes, two per thread.
__device__ __forceinline__ void load_tile_bf16(uint4 (&r)[2], const __bf16* __restrict__ base,
                                               int row_stride) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int u = tid + 256 * rr;
    r[rr] = *(const uint4*)(base + (u >> 3) * row_stride + 8 * (u & 7));
  }
}

__device__ __forceinline__ void store_tile_bf16(const uint4 (&r)[2], __bf16* s) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int u = tid + 256 * rr;
    *(uint4*)(s + (u >> 3) * kLd + 8 * (u & 7)) = r[rr];
  }
}

template <typename TV>
struct VTile {
  static constexpr int N = sizeof(TV) == 2 ? 2 : 4;
  uint4 r[N];
};

template <typename TV>
__device__ __forceinline__ void load_vtile(VTile<TV>& t, const TV* __restrict__ base,
                                           int row_stride) {
  const int tid = threadIdx.x;
  if constexpr (sizeof(TV) == 2) {
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int u = tid + 256 * rr;
      t.r[rr] = *(const uint4*)(base + (u >> 3) * row_stride + 8 * (u & 7));
    }
  } else {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int u = tid + 256 * rr;
      t.r[rr] = *(const uint4*)(base + (u >> 4) * row_stride + 4 * (u & 15));
    }
  }
}

template <typename TV>
__device__ __forceinline__ void store_vtile(const VTile<TV>& t, __bf16* s) {
  const int tid = threadIdx.x;
  if constexpr (sizeof(TV) == 2) {
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int u = tid + 256 * rr;
      *(uint4*)(s + (u >> 3) * kLd + 8 * (u & 7)) = t.r[rr];
    }
  } else {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int u = tid + 256 * rr;
      const float* e = (const float*)&t.r[rr];
      *(bf16x4*)(s + (u >> 4) * kLd + 4 * (u & 15)) = bf16x4{(__bf16)e[0], (__bf16)e[1],
                                                             (__bf16)e[2], (__bf16)e[3]};
    }
  }
}

// Inclusive cumsum of g over the 64 tokens of a chunk (fla chunk_local_cumsum,
// chunkwise.py:1175); lane l holds g[t = l] on entry and Gc[l] on exit.
__device__ __forceinline__ float chunk_cumsum(float x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  return x;
}

// ---------------------------------------------------------------------------
// Per-segment summaries Sum(q) and total log-decay D_q
// ---------------------------------------------------------------------------
// One workgroup per (row, segment, 64-column block of V).  Wave w owns summary
// rows k = 16w .. 16w + 15, all 64 columns (4 MFMA tiles).
struct SumSmem {
  __bf16 k[2][kBT * kLd];
  __bf16 v[2][kBT * kLd];
  float wt[2][kBT];   // exp(Gc_last - Gc_t)
  float cl[2];        // chunk total Gc_last
};

// GCUM: g already holds the chunk-local inclusive cumsum (the backward's input,
// chunkwise.py:1286-1299) instead of per-step log-decays.
template <typename TV, bool GCUM>
__global__ __launch_bounds__(256) void mamba2_seg_sum_kernel(
    const __bf16* __restrict__ k, const TV* __restrict__ v, const float* __restrict__ g,
    float* __restrict__ sums, float* __restrict__ segd, int T, int G, int H, int V, int NT,
    int S, int NSEG, int nvb64) {
  __shared__ __attribute__((aligned(16))) SumSmem sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int vblk = blockIdx.x % nvb64;
  const int rest = blockIdx.x / nvb64;
  const int h = rest % H, p = (rest / H) % NSEG, b = rest / (H * NSEG);
  const int row = b * H + h, gq = h / (H / G);
  const int c0 = p * S;
  const int nch = min(S, NT - c0);
  const int vcol0 = vblk * 64;
  const int kstr = G * kKD, vstr = H * V;
  const rsrc_t rk = make_rsrc(k + ((size_t)b * T * G + gq) * kKD, (size_t)T * kstr * 2);
  const rsrc_t rv = make_rsrc(v + ((size_t)b * T * H + h) * V + vcol0, (size_t)T * vstr * sizeof(TV));
  const rsrc_t rgg = make_rsrc(g + (size_t)b * T * H + h, (size_t)T * H * 4);
  const unsigned int vo_k = ((tid >> 3) * kstr + 8 * (tid & 7)) * 2;
  unsigned int vo_v, so_v2;
  if constexpr (sizeof(TV) == 2) {
    vo_v = ((tid >> 3) * vstr + 8 * (tid & 7)) * 2;
    so_v2 = 32 * vstr * 2;
  } else {
    vo_v = ((tid >> 4) * vstr + 4 * (tid & 15)) * 4;
    so_v2 = 16 * vstr * 4;
  }
  const unsigned int vo_g = lane * H * 4;

  floatx4 acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) acc[n] = zero4();
  float dsum = 0.f;

  uint4 k0, k1;
  VTile<TV> vr;
  float gr = 0.f;
#define SEG_LOAD(jj)                                                                   \
  {                                                                                    \
    const unsigned int row0 = (unsigned int)(c0 + (jj)) * kBT;                         \
    k0 = buf_load16(rk, vo_k, row0 * kstr * 2);                                        \
    k1 = buf_load16(rk, vo_k, (row0 + 32) * kstr * 2);                                 \
    _Pragma("unroll") for (int rr = 0; rr < VTile<TV>::N; ++rr)                        \
        vr.r[rr] = buf_load16(rv, vo_v, row0 * vstr * sizeof(TV) + rr * so_v2);        \
    if (w == 0) gr = buf_load<float>(rgg, vo_g, row0 * H * 4);                         \
  }
#define SEG_STORE(buf)                                                                 \
  {                                                                                    \
    *(uint4*)(sm.k[buf] + (tid >> 3) * kLd + 8 * (tid & 7)) = k0;                      \
    *(uint4*)(sm.k[buf] + ((tid >> 3) + 32) * kLd + 8 * (tid & 7)) = k1;               \
    store_vtile(vr, sm.v[buf]);                                                        \
    if (w == 0) {                                                                      \
      const float x = GCUM ? gr : chunk_cumsum(gr);                                    \
      const float last = __shfl(x, 63, 64);                                            \
      sm.wt[buf][lane] = fexp(last - x);                                               \
      if (lane == 0) sm.cl[buf] = last;                                                \
    }                                                                                  \
  }
  SEG_LOAD(0);
  SEG_STORE(0);
  if (nch > 1) SEG_LOAD(1);
  __syncthreads();
  for (int j = 0; j < nch; ++j) {
    const int buf = j & 1;
    const float clast = sm.cl[buf];
    const float dl = fexp(clast);
    dsum += clast;
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[n][i] *= dl;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const bf16x8 a = tr_frag(sm.k[buf], kLd, 32 * c, 16 * w);   // K^T[k][t]
      const floatx4 w0 = *(const floatx4*)(&sm.wt[buf][32 * c + 8 * lq]);
      const floatx4 w1 = *(const floatx4*)(&sm.wt[buf][32 * c + 8 * lq + 4]);
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const bf16x8 vv = tr_frag(sm.v[buf], kLd, 32 * c, 16 * n);  // V[t][v]
        bf16x8 bv;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          bv[jj] = (__bf16)((float)vv[jj] * w0[jj]);
          bv[4 + jj] = (__bf16)((float)vv[4 + jj] * w1[jj]);
        }
        acc[n] = mfma16x16x32(a, bv, acc[n]);
      }
    }
    if (j + 1 < nch) {
      SEG_STORE(buf ^ 1);
      if (j + 2 < nch) SEG_LOAD(j + 2);
    }
    __syncthreads();
  }
#undef SEG_LOAD
#undef SEG_STORE
  float* out = sums + ((size_t)row * NSEG + p) * kKD * V + vcol0;
#pragma unroll
  for (int n = 0; n < 4; ++n)
#pragma unroll
    for (int i = 0; i < 4; ++i) out[(size_t)(16 * w + 4 * lq + i) * V + 16 * n + ln] = acc[n][i];
  if (tid == 0 && vblk == 0) segd[(size_t)row * NSEG + p] = dsum;
}

}  // namespace hattn
