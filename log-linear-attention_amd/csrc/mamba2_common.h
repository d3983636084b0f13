// Shared pieces of the log-linear Mamba-2 kernels (forward and backward):
// constants, the segment size, chunk staging through buffer loads, and the
// per-segment summary kernel Sum(q) = sum_t exp(G_end(q) - G_t) k_t v_t^T.
#pragma once

#include <cstddef>

#include "common.h"
#include "layer_math.h"

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
template <int NP, typename T, typename E = __bf16>
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
        hi[j] = to16<E>(e[j]);
        if constexpr (NP == 2) lo[j] = bf16_lo(e[j], hi[j]);
      }
      *(bf16x4*)(p0 + off) = hi;
      if constexpr (NP == 2) *(bf16x4*)(p1 + off) = lo;
    }
  }
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
//
// The decay weights w_s = exp(G_end - G_s) are applied to the wave's own K^T
// fragment (16 k rows), so the V fragments enter the MFMA as staged.  Two
// chunks wait in registers while one is multiplied from LDS, so every load has
// two chunk iterations to land.
// Cache-policy bits of the buffer accesses that other workgroups of the same
// launch read or write (the fused forward's segment summaries and flags):
// sc1 makes the access coherent across the XCDs' L2 caches, sc0 also skips
// the CU's L1.  Every such access carries them, so no cache write-back or
// invalidate is needed.
constexpr int kCohLoad = 17;   // sc0 | sc1
constexpr int kCohStore = 16;  // sc1

// Body of the summary pass over segment p of one (row, 64-column block of V):
// writes Sum(p) into out (row-major [K][V] with row stride V, this block's 64
// columns) and returns D_p (on every thread).  COH: the stores carry kCohStore.
// LAYER: v is the layer's x and g comes from dt (v = x dt', g = A dt', see
// layer_math.h); bf16 x only.  NSLOT: chunks held in registers ahead of the
// one being multiplied (the loads in flight per workgroup).  Element (k, v) of
// the summary goes to out[(k V + v) ostride], multiplied by oscale.
// E: the 16-bit MFMA format of K and V (bf16, or fp16 for fp16 inputs; NP = 1).
template <typename TK, typename TV, bool GCUM, int NP, bool COH, bool LAYER = false, int NSLOT = 2,
          typename E = __bf16>
__device__ __forceinline__ float seg_sum_body(SumSmem<NP>& sm, const TK* __restrict__ k,
                                              const TV* __restrict__ v,
                                              const float* __restrict__ g, float* __restrict__ out,
                                              int b, int h, int p, int vblk, int T, int G, int H,
                                              int V, int NT, int S,
                                              const LayerArgs& la = LayerArgs{},
                                              int ostride = 1, float oscale = 1.f) {
  static_assert(!LAYER || (sizeof(TV) == 2 && NP == 1 && !GCUM), "layer mode: bf16 x");
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int gq = h / (H / G);
  const int c0 = p * S;
  const int nch = min(S, NT - c0);
  const int vcol0 = vblk * 64;
  const int kstr = G * kKD, vstr = H * V;
  const rsrc_t rk = make_rsrc(k + ((size_t)b * T * G + gq) * kKD, (size_t)T * kstr * sizeof(TK));
  const rsrc_t rv = make_rsrc(v + ((size_t)b * T * H + h) * V + vcol0, (size_t)T * vstr * sizeof(TV));
  // g (or, in layer mode, its dt words) is used by wave 0 only: the other waves
  // issue the same load through an empty range, which returns zeros without a
  // memory request.  Every load of the pass is unconditional, so the compiler
  // can count the loads in flight and wait for one chunk's data only.
  const rsrc_t rgg = make_rsrc(g + (size_t)b * T * H + h, w == 0 ? (size_t)T * H * 4 : 0);
  const unsigned int vo_k = tile64_voff<TK>(kstr), vo_v = tile64_voff<TV>(vstr);
  const unsigned int vo_g = lane * H * 4;
  // layer mode: dt words of the wave-0 lane's row (g) and of the thread's two
  // V tile rows (tid >> 3, + 32)
  const int desz = la.dt_f32 ? 4 : 2;
  const rsrc_t rdt = make_rsrc(LAYER ? (const char*)la.dt + (size_t)b * T * H * desz : (const char*)g,
                               LAYER ? (size_t)T * H * desz : 0);
  const rsrc_t rdt0 = make_rsrc(LAYER ? (const char*)la.dt + (size_t)b * T * H * desz : (const char*)g,
                                LAYER && w == 0 ? (size_t)T * H * desz : 0);
  const float Ah = LAYER ? la.A[h] : 0.f, bh = LAYER && la.bias ? la.bias[h] : 0.f;
  const unsigned int el_g = (unsigned int)(lane * H + h), el_v = (unsigned int)((tid >> 3) * H + h);

  floatx4 acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) acc[n] = zero4();
  float dsum = 0.f;

  static_assert(NSLOT == 2 || NSLOT == 4, "register slots");
  Tile64<TK> kr[NSLOT];
  Tile64<TV> vr[NSLOT];
  float gr[NSLOT];
  unsigned int dw[NSLOT][2];   // layer: dt words of the V rows
#pragma unroll
  for (int s = 0; s < NSLOT; ++s) gr[s] = 0.f, dw[s][0] = dw[s][1] = 0u;
  auto seg_load = [&](int jj, int slot) {   // chunk jj of the segment -> register slot
    // past the segment's end the last chunk is loaded again (unused)
    const unsigned int row0 = (unsigned int)(c0 + min(jj, nch - 1)) * kBT;
#pragma unroll
    for (int s = 0; s < NSLOT; ++s)
      if (s == slot) {
        load_tile64(kr[s], rk, vo_k, row0 * kstr * sizeof(TK), kstr);
        load_tile64(vr[s], rv, vo_v, row0 * vstr * sizeof(TV), vstr);
        if constexpr (LAYER) {
          const unsigned int e0 = row0 * H;   // even: the bf16 half of an element is its own parity
          gr[s] = buf_load<float>(rdt0, ((e0 + el_g) * desz) & ~3u, 0);
#pragma unroll
          for (int r = 0; r < 2; ++r)
            dw[s][r] = __builtin_bit_cast(unsigned int, buf_load<float>(
                rdt, ((e0 + el_v + 32u * r * H) * desz) & ~3u, 0));
        } else {
          gr[s] = buf_load<float>(rgg, vo_g, row0 * H * 4);
        }
      }
  };
  auto seg_store = [&](int slot, int buf) {   // register slot -> LDS buffer
#pragma unroll
    for (int s = 0; s < NSLOT; ++s)
      if (s == slot) {
        store_tile64<NP, TK, E>(kr[s], sm.k[buf][0], sm.k[buf][NP - 1]);
        if constexpr (LAYER) {
          // v = x dt' on the thread's two rows (tid >> 3 and + 32), rounded to bf16
          Tile64<TV> vs = vr[s];
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const float d = layer_dtp(layer_dt_word(dw[s][r], el_v + 32u * r * H, la.dt_f32),
                                      bh, la.softplus);
            bf16x8 xv = __builtin_bit_cast(bf16x8, vs.r[r]);
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = (__bf16)((float)xv[i] * d);
            vs.r[r] = __builtin_bit_cast(uint4, xv);
          }
          store_tile64<NP>(vs, sm.v[buf][0], sm.v[buf][NP - 1]);
        } else {
          store_tile64<NP, TV, E>(vr[s], sm.v[buf][0], sm.v[buf][NP - 1]);
        }
        if (w == 0) {
          float gv = gr[s];
          if constexpr (LAYER)
            gv = layer_g(Ah, layer_dtp(layer_dt_word(__builtin_bit_cast(unsigned int, gr[s]), el_g,
                                                   la.dt_f32), bh, la.softplus));
          const float x = GCUM ? gv : chunk_cumsum(gv);
          const float last = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
          sm.wt[buf][lane] = fexp(last - x);
          if (lane == 0) sm.cl[buf] = last;
        }
      }
  };
  // chunk j is multiplied from LDS buffer j & 1; chunks j + 1 .. j + NSLOT
  // wait in register slot (chunk index) % NSLOT
#pragma unroll
  for (int s = 0; s < NSLOT; ++s) seg_load(s, s);
  seg_store(0, 0);
  seg_load(NSLOT, 0);
  __syncthreads();
  auto step = [&](int j, int buf, int slot_next) {
    if (j < nch) {
      const float clast = sm.cl[buf];
      const float dl = fexp(clast);
      dsum += clast;
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[n][i] *= dl;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        // A: (K^T diag(w))[k = 16w + ln][s = 32c + 8lq + jj], NP planes
        const floatx4 w0 = *(const floatx4*)(&sm.wt[buf][32 * c + 8 * lq]);
        const floatx4 w1 = *(const floatx4*)(&sm.wt[buf][32 * c + 8 * lq + 4]);
        float ka[8];
        {
          const bf16x8 kh = tr_frag(sm.k[buf][0], kLd, 32 * c, 16 * w);
          bf16x8 kl{};
          if constexpr (NP == 2) kl = tr_frag(sm.k[buf][1], kLd, 32 * c, 16 * w);
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            const float x = NP == 2 ? (float)kh[jj] + (float)kl[jj] : from16<E>(kh[jj]);
            ka[jj] = x * (jj < 4 ? w0[jj] : w1[jj - 4]);
          }
        }
        bf16x8 a[NP];
        split8<NP, E>(ka, a);
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          bf16x8 bv[NP];   // V[s][v = 16n + ln]
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) bv[pl] = tr_frag(sm.v[buf][pl], kLd, 32 * c, 16 * n);
          acc[n] = mma<NP, E>(a, bv, acc[n]);
        }
      }
    }
    // the next chunk -> LDS and a later one -> registers, also past the
    // segment's end (then unused), so the loads do not depend on a branch
    seg_store(slot_next, buf ^ 1);
    seg_load(j + 1 + NSLOT, slot_next);
    __syncthreads();
  };
  for (int j = 0; j < nch; j += NSLOT) {
    step(j, 0, 1);
    step(j + 1, 1, 2 % NSLOT);
    if (NSLOT == 4) {
      step(j + 2, 0, 3);
      step(j + 3, 1, 0);
    }
  }
  if constexpr (COH) {
    // relaxed device-scope atomic stores: plain stores with the sc1 bit.  (The
    // raw-buffer-store builtin fed acc[n][i] here compiled to four stores of
    // acc[n][0] with hipcc 7.2 inside the fused forward kernel.)
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __hip_atomic_store(out + ((size_t)(16 * w + 4 * lq + i) * V + 16 * n + ln) * ostride,
                           acc[n][i] * oscale,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        out[((size_t)(16 * w + 4 * lq + i) * V + 16 * n + ln) * ostride] = acc[n][i] * oscale;
  }
  return dsum;
}

template <typename TK, typename TV, bool GCUM, int NP, typename E = __bf16>
__global__ __launch_bounds__(256) void mamba2_seg_sum_kernel(
    const TK* __restrict__ k, const TV* __restrict__ v, const float* __restrict__ g,
    float* __restrict__ sums, float* __restrict__ segd, int B, int T, int G, int H, int V,
    int NT, int S, int NSEG, int nvb64) {
  __shared__ __attribute__((aligned(16))) SumSmem<NP> sm;
  // grid: xcd_head_grid(B * NSEG, H, nvb64); the heads of one (batch, segment) share an XCD
  const XcdHeadMap xm = xcd_head_map(blockIdx.x, H, nvb64);
  if (xm.grp >= B * NSEG) return;
  const int vblk = xm.slice, h = xm.h, p = xm.grp % NSEG, b = xm.grp / NSEG;
  const int row = b * H + h;
  float* out = sums + ((size_t)row * NSEG + p) * kKD * V + vblk * 64;
  const float dsum = seg_sum_body<TK, TV, GCUM, NP, false, false, 2, E>(sm, k, v, g, out, b, h, p, vblk, T, G,
                                                          H, V, NT, S);
  if (threadIdx.x == 0 && vblk == 0) segd[(size_t)row * NSEG + p] = dsum;
}

// ---------------------------------------------------------------------------
// Top-level states every segment reads (from the segment summaries)
// ---------------------------------------------------------------------------
// A scan over the segments of one row: per top level e2 (inter-chunk level
// s + e2, blocks of 2^(e2 + 1) segments) the state
//   h <- (p ends its aligned block ? 0 : exp(D_p) h) + (bit e2 of p clear ? Sum(p) : 0)
// is read (before the update) by the segments with bit e2 set, which is
// Htop_e2(p).  One workgroup per (row, 64-column block of V, quarter of the
// 64 x 64 tile); each thread owns 4 consecutive elements and streams the
// row's summaries.  Output: NP bf16 planes [row][p][e2][vblk][plane][64][64],
// written only where segment p reads level e2.
template <int NP, typename E = __bf16>
__global__ __launch_bounds__(256) void mamba2_htop_kernel(const float* __restrict__ sums,
                                                          const float* __restrict__ segd,
                                                          __bf16* __restrict__ htop, int V,
                                                          int NSEG, int ntop, int nvb64) {
  const int quarter = blockIdx.x & 3;
  const int vblk = (blockIdx.x >> 2) % nvb64;
  const int row = (blockIdx.x >> 2) / nvb64;
  const int el = quarter * 1024 + 4 * threadIdx.x;
  const int kk = el >> 6, c = el & 63;
  const float* src = sums + ((size_t)row * NSEG * kKD + kk) * V + vblk * 64 + c;
  const size_t sstride = (size_t)kKD * V;
  __bf16* dst = htop + (size_t)row * NSEG * ntop * nvb64 * NP * (kKD * 64) + (size_t)vblk * NP * (kKD * 64) + el;
  const size_t pstride = (size_t)ntop * nvb64 * NP * (kKD * 64), estride = (size_t)nvb64 * NP * (kKD * 64);
  const float* dp = segd + (size_t)row * NSEG;
  floatx4 h[kMaxTop];
#pragma unroll
  for (int e2 = 0; e2 < kMaxTop; ++e2) h[e2] = zero4();
  constexpr int kBatch = 8;   // summaries loaded per round, all in flight together
  for (int p0 = 0; p0 < NSEG; p0 += kBatch) {
    floatx4 xs[kBatch];
    float ds[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int pj = p0 + j < NSEG ? p0 + j : NSEG - 1;
      xs[j] = *(const floatx4*)(src + (size_t)pj * sstride);
      ds[j] = dp[pj];
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
    const int p = p0 + j;
    if (p >= NSEG) break;
    const floatx4 x = xs[j];
    const float dec = fexp(ds[j]);
#pragma unroll
    for (int e2 = 0; e2 < kMaxTop; ++e2) {
      if (e2 < ntop) {
        const bool rd = (p >> e2) & 1;
        if (rd) {
          bf16x4 hi, lo;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            hi[jj] = to16<E>(h[e2][jj]);
            if constexpr (NP == 2) lo[jj] = bf16_lo(h[e2][jj], hi[jj]);
          }
          __bf16* o = dst + (size_t)p * pstride + (size_t)e2 * estride;
          *(bf16x4*)o = hi;
          if constexpr (NP == 2) *(bf16x4*)(o + kKD * 64) = lo;
        }
        const int per = 2 << e2;
        if ((p & (per - 1)) == per - 1) {
          h[e2] = zero4();
        } else {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) h[e2][jj] = h[e2][jj] * dec + (rd ? 0.f : x[jj]);
        }
      }
    }
    }
  }
}

}  // namespace hattn
