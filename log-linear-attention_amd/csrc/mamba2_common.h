// Shared pieces of the log-linear Mamba-2 kernels (forward and backward):
// constants, the segment size, chunk staging through buffer loads, and the
// per-segment summary kernel Sum(q) = sum_t exp(G_end(q) - G_t) k_t v_t^T.
#pragma once

#include <cstddef>

#include "common.h"

namespace hattn {

constexpr int kBT = 64;       // chunk length (the reference's only chunk size)
constexpr int kKD = 64;       // head dim of q / k
constexpr int kMaxLoc = 4;    // local levels held in registers, bf16 kernels (S <= 16 chunks)
constexpr int kMaxLocX3 = 6;  // same, bf16x3 kernels (S <= 64 chunks: fewer LDS-resident top levels)
constexpr int kMaxTop = 8;    // top levels (LDS-resident, T <= 64 * 2^12 in bf16 mode)
constexpr int kMaxLU = 7 + kMaxLoc + kMaxTop;  // lambda columns read by the bf16 kernels
constexpr int kLd = 72;       // LDS row stride (bf16) of 64-wide tiles

// Chunks per segment: 2^maxloc, or the whole sequence when shorter.
__host__ __device__ inline int seg_log2(int NT, int maxloc = kMaxLoc) {
  int nlev = 0;
  while ((1 << nlev) < NT) ++nlev;
  return nlev < maxloc ? nlev : maxloc;
}

// ---------------------------------------------------------------------------
// chunk staging shared by the kernels
// ---------------------------------------------------------------------------
// Row-major 64 x 64 tile of a [.., T, heads, 64-block] tensor in 16-byte units,
// 256 threads: bf16 512 units (row u >> 3, col 8 (u & 7)), fp32 1024 units
// (row u >> 4, col 4 (u & 15)), unit u = tid + 256 r.
template <typename T>
struct Tile64 {
  static constexpr int N = sizeof(T) == 2 ? 2 : 4;
  static constexpr int RSTEP = sizeof(T) == 2 ? 32 : 16;   // rows between a thread's units
  uint4 r[N];
};

template <typename T>
__device__ __forceinline__ unsigned int tile64_voff(int row_stride_elems) {
  const int tid = threadIdx.x;
  if constexpr (sizeof(T) == 2) return ((tid >> 3) * row_stride_elems + 8 * (tid & 7)) * 2;
  else return ((tid >> 4) * row_stride_elems + 4 * (tid & 15)) * 4;
}

template <typename T>
__device__ __forceinline__ void load_tile64(Tile64<T>& t, rsrc_t rs, unsigned int voff,
                                            unsigned int soff, int row_stride_elems) {
#pragma unroll
  for (int rr = 0; rr < Tile64<T>::N; ++rr)
    t.r[rr] = buf_load16(rs, voff, soff + rr * Tile64<T>::RSTEP * row_stride_elems * sizeof(T));
}

// Store a staged tile as NP bf16 planes (plane 1: the bf16x3 low part of fp32 data).
template <int NP, typename T>
__device__ __forceinline__ void store_tile64(const Tile64<T>& t, __bf16* p0, __bf16* p1) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int rr = 0; rr < Tile64<T>::N; ++rr) {
    if constexpr (sizeof(T) == 2) {
      const int off = ((tid >> 3) + 32 * rr) * kLd + 8 * (tid & 7);
      *(uint4*)(p0 + off) = t.r[rr];
    } else {
      const int off = ((tid >> 4) + 16 * rr) * kLd + 4 * (tid & 15);
      const float* e = (const float*)&t.r[rr];
      bf16x4 hi, lo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hi[j] = (__bf16)e[j];
        lo[j] = bf16_lo(e[j], hi[j]);
      }
      *(bf16x4*)(p0 + off) = hi;
      if constexpr (NP == 2) *(bf16x4*)(p1 + off) = lo;
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
// rows k = 16w .. 16w + 15, all 64 columns (4 MFMA tiles).  NP = 2 keeps the
// bf16x3 low planes of fp32 k and v and multiplies with three MFMAs.
template <int NP>
struct SumSmem {
  __bf16 k[2][NP][kBT * kLd];
  __bf16 v[2][NP][kBT * kLd];
  float wt[2][kBT];   // exp(Gc_last - Gc_t)
  float cl[2];        // chunk total Gc_last
};

// GCUM: g already holds the chunk-local inclusive cumsum (the backward's input,
// chunkwise.py:1286-1299) instead of per-step log-decays.
template <typename TK, typename TV, bool GCUM, int NP>
__global__ __launch_bounds__(256) void mamba2_seg_sum_kernel(
    const TK* __restrict__ k, const TV* __restrict__ v, const float* __restrict__ g,
    float* __restrict__ sums, float* __restrict__ segd, int T, int G, int H, int V, int NT,
    int S, int NSEG, int nvb64) {
  __shared__ __attribute__((aligned(16))) SumSmem<NP> sm;
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
  const rsrc_t rk = make_rsrc(k + ((size_t)b * T * G + gq) * kKD, (size_t)T * kstr * sizeof(TK));
  const rsrc_t rv = make_rsrc(v + ((size_t)b * T * H + h) * V + vcol0, (size_t)T * vstr * sizeof(TV));
  const rsrc_t rgg = make_rsrc(g + (size_t)b * T * H + h, (size_t)T * H * 4);
  const unsigned int vo_k = tile64_voff<TK>(kstr), vo_v = tile64_voff<TV>(vstr);
  const unsigned int vo_g = lane * H * 4;

  floatx4 acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) acc[n] = zero4();
  float dsum = 0.f;

  Tile64<TK> kr;
  Tile64<TV> vr;
  float gr = 0.f;
#define SEG_LOAD(jj)                                                                   \
  {                                                                                    \
    const unsigned int row0 = (unsigned int)(c0 + (jj)) * kBT;                         \
    load_tile64(kr, rk, vo_k, row0 * kstr * sizeof(TK), kstr);                         \
    load_tile64(vr, rv, vo_v, row0 * vstr * sizeof(TV), vstr);                        \
    if (w == 0) gr = buf_load<float>(rgg, vo_g, row0 * H * 4);                         \
  }
#define SEG_STORE(buf)                                                                 \
  {                                                                                    \
    store_tile64<NP>(kr, sm.k[buf][0], sm.k[buf][NP - 1]);                             \
    store_tile64<NP>(vr, sm.v[buf][0], sm.v[buf][NP - 1]);                             \
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
      bf16x8 a[NP];   // K^T[k][t]
#pragma unroll
      for (int pl = 0; pl < NP; ++pl) a[pl] = tr_frag(sm.k[buf][pl], kLd, 32 * c, 16 * w);
      const floatx4 w0 = *(const floatx4*)(&sm.wt[buf][32 * c + 8 * lq]);
      const floatx4 w1 = *(const floatx4*)(&sm.wt[buf][32 * c + 8 * lq + 4]);
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        float wv[8];   // w o V[t][v], fp32
        {
          const bf16x8 vh = tr_frag(sm.v[buf][0], kLd, 32 * c, 16 * n);
          bf16x8 vl{};
          if constexpr (NP == 2) vl = tr_frag(sm.v[buf][1], kLd, 32 * c, 16 * n);
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            const float x = NP == 2 ? (float)vh[jj] + (float)vl[jj] : (float)vh[jj];
            wv[jj] = x * (jj < 4 ? w0[jj] : w1[jj - 4]);
          }
        }
        bf16x8 bv[NP];
        split8<NP>(wv, bv);
        acc[n] = mma<NP>(a, bv, acc[n]);
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
