// Log-linear Mamba-2 chunkwise backward for gfx950, segment-parallel.
//
// Replaces chunkwise_bwd (chunkwise.py:1286-1597): the reference launches
// chunk_bwd_kernel_dqkwg and chunk_bwd_kernel_dv for the intra-chunk part and,
// per inter-chunk level, a forward state recompute (chunk_fwd_kernel_h), a
// reverse state scan (chunk_bwd_kernel_dh) and the dqkwg / dv kernels again,
// with dlambda scattered by atomics and fp32 h / dh round-tripping HBM.
//
// With o_t = sum_{s<=t} M[t,s] (q_t . k_s) v_s and M[t,s] = lambda[t, lev(t,s)]
// exp(G_t - G_s):
//   dq_t = sum_s M[t,s] (do_t . v_s) k_s           (past tokens: forward scan)
//   dk_s = sum_t M[t,s] (do_t . v_s) q_t           (future tokens: reverse scan)
//   dv_s = sum_t M[t,s] (q_t . k_s) do_t           (future tokens: reverse scan)
//   dlambda[t, l] = sum_{s: lev(t,s) = l} exp(G_t - G_s) (q_t . k_s)(do_t . v_s)
//   dG_t = q_t . dq_t - k_t . dk_t,  dg_u = sum_{t >= u} dG_t
// (the last identity is what the reference's reverse chunk-local cumsum of its
// dg accumulator computes, chunkwise.py:1596).
//
// Segments of S = 16 chunks as in the forward.  Inter-chunk level e is a
// source for chunk j when bit e of j is clear and is read when it is set.
//   * mamba2_seg_sum_kernel<.., GCUM, ..>: forward summaries Sum(q), D_q (shared with
//     the forward).
//   * mamba2_bwd_rsum_kernel: reverse summaries of the top levels,
//     R_e(q) = sum_{t in q} lambda[t, 7 + e] exp(G_t - G_start(q)) q_t do_t^T.
//   * mamba2_bwd_dq_kernel: walks a segment forwards; forward level states
//     h_e (local in registers, top built from Sum) give dq and the inter-chunk
//     dlambda; the intra-chunk tile gives dq and dlambda[.., 0..6].
//   * mamba2_bwd_dkv_kernel: walks a segment backwards with the reverse level
//     states DH_e (local, registers) plus one combined top-level state built
//     from R_e; waves 0-3 produce dk, waves 4-7 dv (each role keeps the states
//     in the MFMA layout its contraction needs).  It also forms dG and its
//     within-segment reverse cumsum.
//   * mamba2_bwd_dg_kernel: adds the later segments' totals to dg.
#include "mamba2_common.h"

namespace hattn {

// ---------------------------------------------------------------------------
// staging
// ---------------------------------------------------------------------------
// NP bf16 planes per tile: 1 (bf16 q, k, dO: plain bf16 MFMA) or 2 (fp32 q, k,
// v, dO as bf16x3 hi / lo planes, three MFMAs per product; every intermediate
// that feeds another product is split the same way).
template <int NP>
struct BwdStage {
  __bf16 q[NP][kBT * kLd];
  __bf16 k[NP][kBT * kLd];
  __bf16 v[NP][kBT * kLd];
  __bf16 d[NP][kBT * kLd];  // dO
  float gc[kBT];            // chunk-local cumsum Gc (the input g)
  float wt[kBT];            // exp(Gc_last - Gc_t)
  float eg[kBT];            // exp(Gc_t)
  float lam[kMaxLU * kBT];  // lambda^T [level][t]; levels >= 7 pre-multiplied by exp(Gc_t)
};

// Registers of one chunk in flight (NTHR threads share a 64 x 64 tile).  TK:
// element type of q, k and dO; TV of v.
template <int NTHR, typename TK, typename TV, typename TL>
struct BwdRegs {
  static constexpr int NU = 512 / NTHR;  // 16-byte units of a bf16 tile per thread
  static constexpr int NK = sizeof(TK) == 2 ? NU : 2 * NU;
  static constexpr int NV = sizeof(TV) == 2 ? NU : 2 * NU;
  static constexpr int NL = (kMaxLU + NTHR / 64 - 1) / (NTHR / 64);
  uint4 q[NK], k[NK], d[NK], v[NV];
  float g;
  TL lam[NL];
};

// One 16-byte unit of a staged tile: bf16 data as is, fp32 data as NP bf16
// planes of four elements (row r, column c of a kLd-strided tile).
template <int NP, typename T, typename E = __bf16>
__device__ __forceinline__ void stage_unit(const uint4& u, __bf16 (*dst)[kBT * kLd], int off) {
  if constexpr (sizeof(T) == 2) {
    *(uint4*)(dst[0] + off) = u;
  } else {
    const float* e = (const float*)&u;
    bf16x4 hi, lo;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      hi[j] = to16<E>(e[j]);
      if constexpr (NP == 2) lo[j] = bf16_lo(e[j], hi[j]);
    }
    *(bf16x4*)(dst[0] + off) = hi;
    if constexpr (NP == 2) *(bf16x4*)(dst[NP - 1] + off) = lo;
  }
}

// Per-row descriptors and per-lane offsets of the chunk loads.
template <int NTHR, typename TK, typename TV, typename TL>
struct BwdLoader {
  rsrc_t rq, rk, rv, rd, rg, rl;
  unsigned int vo_qk, vo_v, vo_d, vo_g, vo_l;
  unsigned int qrow, vrow, drow, lrowb;  // bytes per token row
  int lrow, lcol, lu;

  __device__ void init(const TK* q, const TK* k, const TV* v, const TK* dO, const float* g,
                       const TL* l, int b, int h, int T, int H, int V, int L, int lu_) {
    const int tid = threadIdx.x, lane = tid & 63;
    const size_t rq0 = ((size_t)b * T * H + h);
    qrow = H * kKD * sizeof(TK);
    vrow = H * V * sizeof(TV);
    drow = H * V * sizeof(TK);
    lrowb = H * L * sizeof(TL);
    rq = make_rsrc(q + rq0 * kKD, (size_t)T * qrow);
    rk = make_rsrc(k + rq0 * kKD, (size_t)T * qrow);
    rv = make_rsrc(v + rq0 * V, (size_t)T * vrow);
    rd = make_rsrc(dO + rq0 * V, (size_t)T * drow);
    rg = make_rsrc(g + rq0, (size_t)T * H * 4);
    rl = make_rsrc(l + rq0 * L, (size_t)T * lrowb);
    if constexpr (sizeof(TK) == 2) {
      vo_qk = (tid >> 3) * qrow + 16 * (tid & 7);
      vo_d = (tid >> 3) * drow + 16 * (tid & 7);
    } else {
      vo_qk = (tid >> 4) * qrow + 16 * (tid & 15);
      vo_d = (tid >> 4) * drow + 16 * (tid & 15);
    }
    if constexpr (sizeof(TV) == 2) vo_v = (tid >> 3) * vrow + 16 * (tid & 7);
    else vo_v = (tid >> 4) * vrow + 16 * (tid & 15);
    vo_g = lane * H * 4;
    constexpr int TPR = NTHR / 64;          // threads per lambda row
    lrow = tid / TPR;
    lcol = tid % TPR;
    vo_l = lrow * lrowb + lcol * sizeof(TL);
    lu = lu_;
  }

  __device__ void load(BwdRegs<NTHR, TK, TV, TL>& r, int chunk) const {
    using R = BwdRegs<NTHR, TK, TV, TL>;
    const unsigned int t0 = (unsigned int)chunk * kBT;
    constexpr int RK = sizeof(TK) == 2 ? NTHR / 8 : NTHR / 16;   // rows per q / k / dO load
#pragma unroll
    for (int u = 0; u < R::NK; ++u) {
      const unsigned int row = t0 + u * RK;
      r.q[u] = buf_load16(rq, vo_qk, row * qrow);
      r.k[u] = buf_load16(rk, vo_qk, row * qrow);
      r.d[u] = buf_load16(rd, vo_d, row * drow);
    }
#pragma unroll
    for (int u = 0; u < R::NV; ++u) {
      const unsigned int row = t0 + u * (sizeof(TV) == 2 ? NTHR / 8 : NTHR / 16);
      r.v[u] = buf_load16(rv, vo_v, row * vrow);
    }
    r.g = buf_load<float>(rg, vo_g, t0 * H_of(qrow) * 4);
    // every lane loads (columns past the row's levels repeat the last one and are
    // not staged): a load behind a per-lane branch makes the compiler wait for
    // every outstanding memory operation wherever it waits for this one
    // (the column index is made opaque here, so the clamped offsets are
    // recomputed per chunk rather than held in registers across the walk)
    int lc;
    asm volatile("v_mov_b32 %0, %1" : "=v"(lc) : "v"(lcol));
    const unsigned int vo_row = vo_l - lcol * sizeof(TL);
#pragma unroll
    for (int c = 0; c < R::NL; ++c) {
      const int col = min(lc + c * (NTHR / 64), lu - 1);
      r.lam[c] = buf_load<TL>(rl, vo_row + col * sizeof(TL), t0 * lrowb);
    }
  }

  // heads per token row, from the q row bytes
  __device__ static unsigned int H_of(unsigned int qrow_bytes) {
    return qrow_bytes / (kKD * sizeof(TK));
  }

  // Returns exp(Gc) of this thread's lambda row (token lrow of the chunk).
  template <int NP, typename E = __bf16>
  __device__ float store(const BwdRegs<NTHR, TK, TV, TL>& r, BwdStage<NP>& s) const {
    using R = BwdRegs<NTHR, TK, TV, TL>;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
#pragma unroll
    for (int u = 0; u < R::NK; ++u) {
      const int off = sizeof(TK) == 2 ? ((tid >> 3) + u * (NTHR / 8)) * kLd + 8 * (tid & 7)
                                      : ((tid >> 4) + u * (NTHR / 16)) * kLd + 4 * (tid & 15);
      stage_unit<NP, TK, E>(r.q[u], s.q, off);
      stage_unit<NP, TK, E>(r.k[u], s.k, off);
      stage_unit<NP, TK, E>(r.d[u], s.d, off);
    }
#pragma unroll
    for (int u = 0; u < R::NV; ++u) {
      const int off = sizeof(TV) == 2 ? ((tid >> 3) + u * (NTHR / 8)) * kLd + 8 * (tid & 7)
                                      : ((tid >> 4) + u * (NTHR / 16)) * kLd + 4 * (tid & 15);
      stage_unit<NP, TV, E>(r.v[u], s.v, off);
    }
    const float x = r.g;                       // already the chunk-local cumsum
    const float last = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
    if (w == 0) {
      s.gc[lane] = x;
      s.wt[lane] = fexp(last - x);
      s.eg[lane] = fexp(x);
    }
    const float eg = fexp(__shfl(x, lrow, 64));
#pragma unroll
    for (int c = 0; c < R::NL; ++c) {
      const int col = lcol + c * (NTHR / 64);
      if (col < lu) {
        float val = to_f32<TL>(r.lam[c]);
        if (col >= 7) val *= eg;
        s.lam[col * kBT + lrow] = val;
      }
    }
    return eg;
  }
};

// Phase-1 tiles (t-tile mt, s-tile jt) of the 64 x 64 intra-chunk matrices:
// the 10 causal tiles plus the zero tiles (0,1) and (2,3) that the 32-wide
// contraction steps read.  code = mt * 4 + jt, +16 marks a zero tile, -1 none.
// 4 waves, 3 each: one diagonal tile per wave, the six sub-diagonal tiles two
// on each of waves 0, 1 and one on each of 2, 3 (with a zero tile)
__device__ __forceinline__ int p1_tile4(int w, int n) {
  constexpr int tab[4][3] = {{0, 4, 8}, {5, 9, 12}, {10, 13, 16 + 1}, {15, 14, 16 + 11}};
  return tab[w][n];
}
// 8 waves, 2 each: every diagonal tile on a wave of its own, the six
// sub-diagonal tiles two on each of waves 4, 5 and one on each of 6, 7 (with a
// zero tile)
__device__ __forceinline__ int p1_tile8(int w, int n) {
  constexpr int tab[8][2] = {{0, -1}, {5, -1}, {10, -1}, {15, -1}, {4, 8}, {9, 12},
                             {13, 16 + 1}, {14, 16 + 11}};
  return tab[w][n];
}

// Fragment planes of a staged tile at one element offset.
template <int NP>
__device__ __forceinline__ void frag8(const __bf16 (*X)[kBT * kLd], int off, bf16x8* f) {
#pragma unroll
  for (int pl = 0; pl < NP; ++pl) f[pl] = *(const bf16x8*)(X[pl] + off);
}
template <int NP>
__device__ __forceinline__ void trfrag(const __bf16 (*X)[kBT * kLd], int r0, int c0, bf16x8* f) {
#pragma unroll
  for (int pl = 0; pl < NP; ++pl) f[pl] = tr_frag(X[pl], kLd, r0, c0);
}

// S^T and dP^T tile (s rows 16jt.., t columns 16mt..): D[m = s][n = t].
template <int NP, typename E = __bf16>
__device__ __forceinline__ void st_dpt_tile(const BwdStage<NP>& s, int mt, int jt, floatx4& S,
                                            floatx4& P) {
  const int lane = threadIdx.x & 63, lq = lane >> 4, ln = lane & 15;
  S = zero4();
  P = zero4();
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int ra = (16 * jt + ln) * kLd + 32 * c + 8 * lq;
    const int rb = (16 * mt + ln) * kLd + 32 * c + 8 * lq;
    bf16x8 a[NP], bq[NP];
    frag8<NP>(s.k, ra, a);
    frag8<NP>(s.q, rb, bq);
    S = mma<NP, E>(a, bq, S);
    frag8<NP>(s.v, ra, a);
    frag8<NP>(s.d, rb, bq);
    P = mma<NP, E>(a, bq, P);
  }
}

// fp32 value of staged element planes
template <int NP, typename E = __bf16>
__device__ __forceinline__ float plane_val(const __bf16 (*X)[kBT * kLd], int off) {
  return NP == 2 ? (float)X[0][off] + (float)X[NP - 1][off] : from16<E>(X[0][off]);
}

// Four fp32 values stored as NP bf16 planes of an intermediate tile.
template <int NP, typename E = __bf16>
__device__ __forceinline__ void store_planes4(__bf16 (*X)[kBT * kLd], int off, const float* x) {
  bf16x4 hi, lo;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hi[i] = to16<E>(x[i]);
    if constexpr (NP == 2) lo[i] = bf16_lo(x[i], hi[i]);
  }
  *(bf16x4*)(X[0] + off) = hi;
  if constexpr (NP == 2) *(bf16x4*)(X[NP - 1] + off) = lo;
}

// S^T and dP^T of two tiles (as st_dpt_tile): every LDS read of a 32-wide
// contraction step is issued before its four MFMAs.
template <typename E = __bf16>
__device__ __forceinline__ void st_dpt_tiles2(const BwdStage<1>& s, const int (&mt)[2],
                                              const int (&jt)[2], floatx4 (&S)[2],
                                              floatx4 (&P)[2]) {
  const int lane = threadIdx.x & 63, lq = lane >> 4, ln = lane & 15;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    bf16x8 ka[2], qb[2], va[2], db[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int ra = (16 * jt[n] + ln) * kLd + 32 * c + 8 * lq;
      const int rb = (16 * mt[n] + ln) * kLd + 32 * c + 8 * lq;
      ka[n] = *(const bf16x8*)(s.k[0] + ra);
      qb[n] = *(const bf16x8*)(s.q[0] + rb);
      va[n] = *(const bf16x8*)(s.v[0] + ra);
      db[n] = *(const bf16x8*)(s.d[0] + rb);
    }
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      S[n] = mfma16<E>(ka[n], qb[n], c ? S[n] : zero4());
      P[n] = mfma16<E>(va[n], db[n], c ? P[n] : zero4());
    }
  }
}

// exp(Gc_t - Gc_s) * [s <= t] and the level of each element of a phase-1 tile.
struct TileMask {
  float dec[4];
  int lev[4];    // level of the pair (0..6)
};
template <int NP>
__device__ __forceinline__ TileMask tile_mask(const BwdStage<NP>& s, int mt, int jt) {
  const int lane = threadIdx.x & 63, lq = lane >> 4, ln = lane & 15;
  TileMask m;
  const int t = 16 * mt + ln;
  const float gct = s.gc[t];
  const floatx4 gs = *(const floatx4*)(s.gc + 16 * jt + 4 * lq);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int sl = 4 * lq + i;
    if (jt < mt) {
      m.lev[i] = 4 + intra_level(mt, jt);
      m.dec[i] = fexp(gct - gs[i]);
    } else {
      m.lev[i] = intra_level(ln, sl);
      m.dec[i] = sl <= ln ? fexp(gct - gs[i]) : 0.f;
    }
  }
  return m;
}

// tile_mask without branches on the tile (mt, jt are wave-uniform but not
// compile-time): dec is zero for every element when the tile is not causal
template <int NP>
__device__ __forceinline__ TileMask tile_mask_sel(const BwdStage<NP>& s, int mt, int jt,
                                                  bool causal) {
  const int lane = threadIdx.x & 63, lq = lane >> 4, ln = lane & 15;
  TileMask m;
  const float gct = s.gc[16 * mt + ln];
  const floatx4 gs = *(const floatx4*)(s.gc + 16 * jt + 4 * lq);
  const bool off = jt < mt;
  const int lev_off = 4 + intra_level(mt, jt);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int sl = 4 * lq + i;
    m.lev[i] = off ? lev_off : intra_level(ln, sl);
    const float d = fexp(gct - gs[i]);
    m.dec[i] = causal && (off || sl <= ln) ? d : 0.f;
  }
  return m;
}

// 8-byte LDS read pair in the D-fragment row order: X[row][c0 + 4lq + i] and
// X[row][c0 + 16 + 4lq + i], i = 0..3.
__device__ __forceinline__ bf16x8 row_pair(const __bf16* X, int row, int c0) {
  const int lq = (threadIdx.x & 63) >> 4;
  const __bf16* p = X + row * kLd + c0 + 4 * lq;
  const bf16x4 lo = *(const bf16x4*)p;
  const bf16x4 hi = *(const bf16x4*)(p + 16);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
template <int NP>
__device__ __forceinline__ void row_pairs(const __bf16 (*X)[kBT * kLd], int row, int c0,
                                          bf16x8* f) {
#pragma unroll
  for (int pl = 0; pl < NP; ++pl) f[pl] = row_pair(X[pl], row, c0);
}

template <typename E = __bf16>
__device__ __forceinline__ bf16x8 scale8(bf16x8 x, floatx4 a, floatx4 b) {
  bf16x8 y;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[i] = to16<E>(from16<E>(x[i]) * a[i]);
    y[4 + i] = to16<E>(from16<E>(x[4 + i]) * b[i]);
  }
  return y;
}
// planes x (value hi + lo) scaled elementwise by (a, b), re-split into planes
template <int NP, typename E = __bf16>
__device__ __forceinline__ void scale8s(const bf16x8* x, floatx4 a, floatx4 b, bf16x8* y) {
  if constexpr (NP == 1) {
    y[0] = scale8<E>(x[0], a, b);
  } else {
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = ((float)x[0][i] + (float)x[1][i]) * a[i];
      f[4 + i] = ((float)x[0][4 + i] + (float)x[1][4 + i]) * b[i];
    }
    split8<NP>(f, y);
  }
}

// ---------------------------------------------------------------------------
// Reverse summaries of the top levels
// ---------------------------------------------------------------------------
// One workgroup per (row, segment, group of 4 top levels); wave w owns rows
// k = 16w.. of R_e.  sig[e][t] = lambda[t, 7 + e] exp(E_i + Gc_t).
template <int NP>
struct RsumSmem {
  __bf16 q[NP][kBT * kLd];
  __bf16 d[NP][kBT * kLd];
  float sig[4][kBT];
};

template <int NP, typename TK, typename TL, typename E = __bf16>
__global__ __launch_bounds__(256) void mamba2_bwd_rsum_kernel(
    const TK* __restrict__ q, const TK* __restrict__ dO, const float* __restrict__ gcin,
    const TL* __restrict__ l, float* __restrict__ rsum, int B, int T, int H, int L, int NT,
    int slog, int NSEG, int nloc, int ntop, int ngrp) {
  __shared__ __attribute__((aligned(16))) RsumSmem<NP> sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  // grid: xcd_head_grid(B * NSEG, H, ngrp): the heads of one (batch, segment)
  // share an XCD, so the lambda and g lines that interleave them are fetched once
  const XcdHeadMap xm = xcd_head_map(blockIdx.x, H, ngrp);
  if (xm.grp >= B * NSEG) return;
  const int grp = xm.slice;
  const int h = xm.h, p = xm.grp % NSEG, b = xm.grp / NSEG;
  const int row = b * H + h;
  const int c0 = p << slog, cend = min(c0 + (1 << slog), NT);
  const int e0 = 4 * grp;
  const int ne = min(4, ntop - e0);
  const size_t rq0 = (size_t)b * T * H + h;
  const unsigned int qrow = H * kKD * sizeof(TK), lrowb = H * L * sizeof(TL);
  const rsrc_t rq = make_rsrc(q + rq0 * kKD, (size_t)T * qrow);
  const rsrc_t rd = make_rsrc(dO + rq0 * kKD, (size_t)T * qrow);
  const rsrc_t rg = make_rsrc(gcin + rq0, (size_t)T * H * 4);
  const rsrc_t rl = make_rsrc(l + rq0 * L, (size_t)T * lrowb);
  constexpr int NK = sizeof(TK) == 2 ? 2 : 4;   // 16-byte units of a tile per thread
  constexpr int RK = 64 / NK;                    // rows between them
  const unsigned int vo = sizeof(TK) == 2 ? (tid >> 3) * qrow + 16 * (tid & 7)
                                          : (tid >> 4) * qrow + 16 * (tid & 15);
  const int soff = sizeof(TK) == 2 ? (tid >> 3) * kLd + 8 * (tid & 7)
                                   : (tid >> 4) * kLd + 4 * (tid & 15);
  const int lt = tid >> 2, le = tid & 3;   // sigma entry of this thread

  floatx4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[a][n] = zero4();
  // chunk ic + 2 is loaded into the register slot that chunk ic leaves when it
  // is stored to LDS, so two chunks' loads are in flight behind each chunk's
  // MFMAs (the loop is unrolled by two so the slots are static registers).
  // Every lane issues the same loads: the lambda column is clamped to a valid
  // one and zeroed at the store, so no load sits behind a divergent branch.
  struct ChunkRegs {
    uint4 q[NK], d[NK];
    float gct, glast, lv;
  };
  const unsigned int lcol = (unsigned int)(7 + nloc + e0 + min(le, ne - 1));
  ChunkRegs rr[2];
  auto load = [&](int ic, int slot) {
    if (ic >= cend) return;
    const unsigned int t0 = (unsigned int)ic * kBT;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
      if (sl == slot) {
#pragma unroll
        for (int u = 0; u < NK; ++u) {
          rr[sl].q[u] = buf_load16(rq, vo, (t0 + RK * u) * qrow);
          rr[sl].d[u] = buf_load16(rd, vo, (t0 + RK * u) * qrow);
        }
        rr[sl].gct = buf_load<float>(rg, lt * H * 4, t0 * H * 4);
        rr[sl].glast = buf_load<float>(rg, 63 * H * 4, t0 * H * 4);
        rr[sl].lv = to_f32<TL>(buf_load<TL>(rl, (lt * H * L + lcol) * sizeof(TL), t0 * lrowb));
      }
  };
  float Ecum = 0.f;
  auto step = [&](int ic, int slot) {
    __syncthreads();   // previous chunk's reads of sm are done
    float glast = 0.f;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
      if (sl == slot) {
#pragma unroll
        for (int u = 0; u < NK; ++u) {
          stage_unit<NP, TK, E>(rr[sl].q[u], sm.q, soff + RK * u * kLd);
          stage_unit<NP, TK, E>(rr[sl].d[u], sm.d, soff + RK * u * kLd);
        }
        sm.sig[le][lt] = le < ne ? rr[sl].lv * fexp(Ecum + rr[sl].gct) : 0.f;
        glast = rr[sl].glast;
      }
    load(ic + 2, slot);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      bf16x8 qa[NP];   // Q[t][k = 16w + ln]
      trfrag<NP>(sm.q, 32 * c, 16 * w, qa);
      bf16x8 db[4][NP];
#pragma unroll
      for (int n = 0; n < 4; ++n) trfrag<NP>(sm.d, 32 * c, 16 * n, db[n]);
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        if (a < ne) {
          const float* sg = sm.sig[a] + 32 * c + 8 * lq;
          bf16x8 qs[NP];
          scale8s<NP, E>(qa, *(const floatx4*)sg, *(const floatx4*)(sg + 4), qs);
#pragma unroll
          for (int n = 0; n < 4; ++n) acc[a][n] = mma<NP, E>(qs, db[n], acc[a][n]);
        }
      }
    }
    Ecum += glast;
  };
  load(c0, 0);
  load(c0 + 1, 1);
  for (int ic = c0; ic < cend; ic += 2) {
    step(ic, 0);
    if (ic + 1 < cend) step(ic + 1, 1);
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    if (a < ne) {
      float* out = rsum + (((size_t)row * NSEG + p) * ntop + e0 + a) * kKD * kKD;
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) out[(16 * w + 4 * lq + i) * kKD + 16 * n + ln] = acc[a][n][i];
    }
  }
}

// ---------------------------------------------------------------------------
// dq and dlambda: forward walk over one segment
// ---------------------------------------------------------------------------
// LDS of the dq kernel (about 73 KB, so two workgroups share a CU); the
// top-level states stay in HBM / L2 (see htop below).
template <int NP>
struct DqSmem {
  BwdStage<NP> st;
  __bf16 a[NP][kBT * kLd];                  // (M o dP)[t][s], NP bf16 planes
  float dl_off[kBT][4][4];                  // off-diagonal tile partials [t][jt][lq]
  float dl_diag[kBT][5][4];                 // diagonal tile partials [t][level][lq]
  float dl_int[kBT][kMaxLoc + kMaxTop][4];  // inter-level partials [t][e][wave]
  float eg_own[256];                        // exp(Gc_t), t = tid >> 2, one slot per thread
};

// htop: the top-level states Htop_e2(p) of every (row, segment) in bf16 [k][v]
// tiles, written by mamba2_htop_kernel<1> from the segment summaries (layout
// [row][p][e2][64][64]).  Every chunk of a segment reads the same tiles, so
// after the first chunk their MFMA fragments come from L2; the fragments of
// the segment's first top level are loaded once, before the walk, the others
// one level ahead of their use.
template <int NP, typename TK, typename TV, typename TL, typename E = __bf16>
__global__ __launch_bounds__(256, NP == 1 ? 2 : 1) void mamba2_bwd_dq_kernel(
    const TK* __restrict__ q, const TK* __restrict__ k, const TV* __restrict__ v,
    const TK* __restrict__ dO, const float* __restrict__ gcin, const TL* __restrict__ l,
    const __bf16* __restrict__ htop, TK* __restrict__ dq, float* __restrict__ dl,
    float* __restrict__ dgq, int B, int T, int H, int V, int L, int nlev, int slog, int NSEG) {
  __shared__ __attribute__((aligned(16))) DqSmem<NP> sm;
  BwdStage<NP>& s = sm.st;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq0 = lane >> 4, ln0 = lane & 15;
  // grid: xcd_head_grid(B * NSEG, H, 1): the heads of one (batch, segment) share an XCD
  const XcdHeadMap xm = xcd_head_map(blockIdx.x, H, 1);
  if (xm.grp >= B * NSEG) return;
  const int h = xm.h, p = xm.grp % NSEG, b = xm.grp / NSEG;
  const int row = b * H + h;
  const int NT = T / kBT;
  const int c0 = p << slog, cend = min(c0 + (1 << slog), NT);
  const int lu = 7 + nlev;
  const int nloc = min(slog, nlev), ntop = nlev - nloc;
  const int topmask = ntop > 0 ? (p & ((1 << ntop) - 1)) : 0;   // top levels this segment reads

  // A operand of a top level: h[k = 16w + ln][v = c0 + 4lq + i, c0 + 16 + 4lq + i]
  // (htop: [row][p][e2][plane][64][64])
  const rsrc_t rt = make_rsrc(ntop > 0 ? (const void*)(htop + ((size_t)row * NSEG + p) * ntop * NP * kKD * kKD)
                                       : (const void*)htop,
                              ntop > 0 ? (size_t)ntop * NP * kKD * kKD * 2 : 0);
  const unsigned int vo_t = ((16 * w + ln0) * kKD + 4 * lq0) * 2;
  auto top_frag = [&](int e2, int cc, bf16x8* f) {
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
      const unsigned int so = (unsigned int)((e2 * NP + pl) * kKD * kKD + cc) * 2;
      const uint2 lo = buf_load8(rt, vo_t, so), hi = buf_load8(rt, vo_t, so + 32);
      f[pl] = __builtin_bit_cast(bf16x8, uint4{lo.x, lo.y, hi.x, hi.y});
    }
  };
  bf16x8 tf0[NP] = {}, tf1[NP] = {};   // the segment's first top level (loaded once)
  if (topmask) {
    const int e0 = __builtin_ctz(topmask);
    top_frag(e0, 0, tf0);
    top_frag(e0, 32, tf1);
  }

  BwdLoader<256, TK, TV, TL> ld;
  ld.init(q, k, v, dO, gcin, l, b, h, T, H, V, L, lu);
  const size_t rq0 = (size_t)b * T * H + h;
  const rsrc_t rdq = make_rsrc(dq + rq0 * kKD, (size_t)T * H * kKD * sizeof(TK));
  const rsrc_t rdl = make_rsrc(dl + rq0 * L, (size_t)T * H * L * 4);
  const rsrc_t rgq = make_rsrc(dgq + rq0, (size_t)T * H * 4);
  const unsigned int vo_dq = (ln0 * H * kKD + 16 * w + 4 * lq0) * sizeof(TK);

  // forward states h_e^T [v][k]: lane holds v = 16m + 4lq + i, k = 16w + ln
  floatx4 hT[kMaxLoc][4];
#pragma unroll
  for (int e = 0; e < kMaxLoc; ++e)
#pragma unroll
    for (int m = 0; m < 4; ++m) hT[e][m] = zero4();

  BwdRegs<256, TK, TV, TL> rg;
  ld.load(rg, c0);
  __builtin_amdgcn_sched_barrier(0);
  {
    // Four dq-shaped stores through an empty range (no request is made): on the
    // back edge the chunk's four dq stores follow the next chunk's loads, so
    // the loop header sees the same memory-operation order on both incoming
    // paths and the staging wait leaves those stores in flight.
    const rsrc_t rnone = make_rsrc(dq, 0);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      buf_store4<TK>(zero4(), rnone, vo_dq, 16u * mt * H * kKD * sizeof(TK));
  }
  float Eseg = 0.f;
  // cend > c0: a do-while, so the preheader runs straight into the body; the
  // next chunk's loads are unconditional (the last chunk reloaded at the end)
  int ic = c0;
  do {
    // exp(Gc_t) of token t = tid >> 2 (the lambda row this thread stages) goes to
    // the thread's own slot: the dlambda section reads it after the chunk's last
    // barrier, and the next chunk's staging rewrites the shared stage before its
    // first barrier
    sm.eg_own[tid] = ld.template store<NP, E>(rg, s);
    __syncthreads();
    // lane indices made opaque per chunk, so the LDS addresses of the phases are
    // recomputed (a few VALU ops) instead of held in VGPRs across the walk
    int lq, ln;
    asm volatile("v_mov_b32 %0, %1" : "=v"(lq) : "v"(lq0));
    asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(ln0));

    // ---- phase 1: (M o dP) tiles and the intra-chunk dlambda partials ----------
    // bf16 (bf16 v: with fp32 v the staging registers leave no room): the
    // wave's diagonal tile (its first) and its first sub-diagonal tile together
    // (LDS reads, MFMAs, masks, then the partials), the third tile (a
    // sub-diagonal one on waves 0 and 1, a zero tile on 2 and 3) after them
    constexpr bool kP1Pair = NP == 1 && sizeof(TV) == 2;
    if constexpr (kP1Pair) {
      const int c1 = p1_tile4(w, 1);
      int tmt[2] = {w, (c1 & 15) >> 2}, tjt[2] = {w, c1 & 3};
      floatx4 S[2], P[2];
      st_dpt_tiles2<E>(s, tmt, tjt, S, P);
      float out[2][4], x[2][4];
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const TileMask mk = tile_mask_sel(s, tmt[n], tjt[n], true);
        const int t = 16 * tmt[n] + ln;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pd = mk.dec[i] * P[n][i];
          out[n][i] = pd * s.lam[mk.lev[i] * kBT + t];
          x[n][i] = pd * S[n][i];
        }
        if (n == 0) {
#pragma unroll
          for (int lv = 0; lv < 5; ++lv) {
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) a += mk.lev[i] == lv ? x[0][i] : 0.f;
            sm.dl_diag[t][lv][lq] = a;
          }
        } else {
          sm.dl_off[t][tjt[1]][lq] = x[1][0] + x[1][1] + x[1][2] + x[1][3];
        }
        store_planes4<NP, E>(sm.a, t * kLd + 16 * tjt[n] + 4 * lq, out[n]);
      }
    }
#pragma unroll
    for (int n = kP1Pair ? 2 : 0; n < 3; ++n) {
      const int code = p1_tile4(w, n);
      const int mt = (code & 15) >> 2, jt = code & 3;
      const int t = 16 * mt + ln;
      float out[4] = {0.f, 0.f, 0.f, 0.f};
      if (code < 16) {
        floatx4 S, P;
        st_dpt_tile<NP, E>(s, mt, jt, S, P);
        const TileMask mk = tile_mask(s, mt, jt);
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pd = mk.dec[i] * P[i];
          out[i] = pd * s.lam[mk.lev[i] * kBT + t];
          x[i] = pd * S[i];
        }
        if (jt < mt) {
          sm.dl_off[t][jt][lq] = x[0] + x[1] + x[2] + x[3];
        } else {
#pragma unroll
          for (int lv = 0; lv < 5; ++lv) {
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) a += mk.lev[i] == lv ? x[i] : 0.f;
            sm.dl_diag[t][lv][lq] = a;
          }
        }
      }
      store_planes4<NP, E>(sm.a, t * kLd + 16 * jt + 4 * lq, out);
    }
    __syncthreads();
    // the next chunk's loads, issued after phase 1 rather than at the chunk start,
    // right behind the previous chunk's dq / dlambda stores, where their issue
    // waits for those stores to drain
    ld.load(rg, min(ic + 1, cend - 1));

    // ---- phase 2: dq^T[k-tile w][t] ----------------------------------------------
    floatx4 dqT[4];
    {
      bf16x8 kt0[NP], kt1[NP];
      trfrag<NP>(s.k, 0, 16 * w, kt0);
      trfrag<NP>(s.k, 32, 16 * w, kt1);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int ar = (16 * mt + ln) * kLd + 8 * lq;
        bf16x8 af[NP];
        frag8<NP>(sm.a, ar, af);
        dqT[mt] = mma<NP, E>(kt0, af, zero4());
        if (mt >= 2) {
          frag8<NP>(sm.a, ar + 32, af);
          dqT[mt] = mma<NP, E>(kt1, af, dqT[mt]);
        }
      }
    }
    // q[t][k] for this lane's (t = 16mt + ln, k = 16w + 4lq + i)
    floatx4 qk[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int off = (16 * mt + ln) * kLd + 16 * w + 4 * lq;
      const bf16x4 x = *(const bf16x4*)(s.q[0] + off);
      qk[mt] = floatx4{from16<E>(x[0]), from16<E>(x[1]), from16<E>(x[2]), from16<E>(x[3])};
      if constexpr (NP == 2) {
        const bf16x4 y = *(const bf16x4*)(s.q[1] + off);
        qk[mt] += floatx4{(float)y[0], (float)y[1], (float)y[2], (float)y[3]};
      }
    }
    if (nlev > 0) {
      bf16x8 da[4][2][NP];   // dO[t][v] in the states' v order
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int c = 0; c < 2; ++c) row_pairs<NP>(s.d, 16 * mt + ln, 32 * c, da[mt][c]);
      // Y^T[k][t] = sum_v h[k][v] dO[t][v] for two t-tiles at a time (their LDS
      // reads, then their MFMAs, then the dq and q . Y terms), then one
      // transposed cross-row sum of the four tiles' q . Y: lane (lq, ln) stores
      // the dlambda partial of token 16 lq + ln
      auto level = [&](const bf16x8* a0, const bf16x8* a1, int e, int col, float scale) {
        float r[4];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          float sg[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) sg[u] = s.lam[col * kBT + 16 * (2 * hf + u) + ln] * scale;
          floatx4 y[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            y[u] = mma<NP, E>(a0, da[2 * hf + u][0], zero4());
            y[u] = mma<NP, E>(a1, da[2 * hf + u][1], y[u]);
          }
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int mt = 2 * hf + u;
            float rr = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              dqT[mt][i] += y[u][i] * sg[u];
              rr += qk[mt][i] * y[u][i];
            }
            r[mt] = rr;
          }
        }
        sm.dl_int[16 * lq + ln][e][w] = sum_lq_t(r, lq) * scale;   // dlambda / exp(Gc_t)
      };
      if (nloc > 0) {
        // only the levels the chunk reads (bit e of the chunk index, uniform) are
        // multiplied; the others contribute zero to dq and dlambda
#pragma unroll
        for (int e = 0; e < kMaxLoc; ++e) {
          if (e < nloc) {
            if (ic > c0 && ((ic >> e) & 1)) {
              bf16x8 h0[NP], h1[NP];
              cat8s<NP, E>(hT[e][0], hT[e][1], h0);
              cat8s<NP, E>(hT[e][2], hT[e][3], h1);
              level(h0, h1, e, 7 + e, 1.f);
            } else {
              sm.dl_int[16 * lq + ln][e][w] = 0.f;
            }
          }
        }
      }
      if (topmask) {
        const float ee = fexp(Eseg);
        int m = topmask, e2 = __builtin_ctz(topmask);
        bf16x8 a0[NP], a1[NP];
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) {
          a0[pl] = tf0[pl];
          a1[pl] = tf1[pl];
        }
        while (true) {
          m &= m - 1;
          bf16x8 n0[NP], n1[NP];
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) {
            n0[pl] = a0[pl];
            n1[pl] = a1[pl];
          }
          if (m) {   // the next read level's fragments, in flight during this level
            top_frag(__builtin_ctz(m), 0, n0);
            top_frag(__builtin_ctz(m), 32, n1);
          }
          level(a0, a1, nloc + e2, 7 + nloc + e2, ee);
          if (!m) break;
          e2 = __builtin_ctz(m);
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) {
            a0[pl] = n0[pl];
            a1[pl] = n1[pl];
          }
        }
      }
      for (int e2 = 0; e2 < ntop; ++e2)
        if (!((p >> e2) & 1)) sm.dl_int[16 * lq + ln][nloc + e2][w] = 0.f;
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      buf_store4<TK>(dqT[mt], rdq, vo_dq, ((unsigned int)ic * kBT + 16 * mt) * H * kKD * sizeof(TK));

    // ---- phase 3: forward state update h^T_e[v][k] += (w o V)^T K ---------------
    const float glr = s.gc[kBT - 1];
    if (nloc > 0) {
      floatx4 kv[4];
      {
        bf16x8 kt[NP], kb0[NP], kb1[NP];
        trfrag<NP>(s.k, 0, 16 * w, kt);
        scale8s<NP, E>(kt, *(const floatx4*)(s.wt + 8 * lq), *(const floatx4*)(s.wt + 8 * lq + 4),
                    kb0);
        trfrag<NP>(s.k, 32, 16 * w, kt);
        scale8s<NP, E>(kt, *(const floatx4*)(s.wt + 32 + 8 * lq),
                    *(const floatx4*)(s.wt + 36 + 8 * lq), kb1);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          bf16x8 vf[NP];
          trfrag<NP>(s.v, 0, 16 * m, vf);
          kv[m] = mma<NP, E>(vf, kb0, zero4());
          trfrag<NP>(s.v, 32, 16 * m, vf);
          kv[m] = mma<NP, E>(vf, kb1, kv[m]);
        }
      }
      const float gl = fexp(glr);
#pragma unroll
      for (int e = 0; e < kMaxLoc; ++e) {
        if (e < nloc) {
          const int per = 2 << e;
          const bool reset = (ic & (per - 1)) == per - 1;
          const bool wr = !((ic >> e) & 1);
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            if (reset) {
              hT[e][m] = wr ? kv[m] : zero4();
            } else if (wr) {
#pragma unroll
              for (int i = 0; i < 4; ++i) hT[e][m][i] = hT[e][m][i] * gl + kv[m][i];
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) hT[e][m][i] *= gl;
            }
          }
        }
      }
    }
    Eseg += glr;
    __syncthreads();

    // ---- dlambda row of every token, and q . dq = sum_l lambda_l dlambda_l ----------
    // (the identity holds term by term: row t of (M o S o dP) summed by level; it
    // uses the fp32 tile products instead of the bf16-rounded (M o dP) behind dq)
    {
      const int t = tid >> 2, part = tid & 3;
      const int mt = t >> 4;
      // per-lane part of the offsets in the VGPR operand, the chunk's in the SGPR
      // one (a lane-dependent scalar offset makes the compiler loop over lanes)
      const unsigned int vo = (unsigned int)t * H * L * 4, so = (unsigned int)ic * kBT * H * L * 4;
      float qdq = 0.f;
      for (int col = part; col < L; col += 4) {
        float val = 0.f;
        if (col <= 4) {
          val = sm.dl_diag[t][col][0] + sm.dl_diag[t][col][1] + sm.dl_diag[t][col][2] +
                sm.dl_diag[t][col][3];
        } else if (col <= 6) {
          for (int jt = 0; jt < mt; ++jt)
            if (4 + intra_level(mt, jt) == col)
              val += sm.dl_off[t][jt][0] + sm.dl_off[t][jt][1] + sm.dl_off[t][jt][2] +
                     sm.dl_off[t][jt][3];
        } else if (col < lu) {
          const int e = col - 7;
          const float raw =
              sm.dl_int[t][e][0] + sm.dl_int[t][e][1] + sm.dl_int[t][e][2] + sm.dl_int[t][e][3];
          qdq += raw * s.lam[col * kBT + t];   // lambda exp(Gc_t) * dlambda / exp(Gc_t)
          val = raw * sm.eg_own[tid];
        }
        if (col <= 6) qdq += val * s.lam[col * kBT + t];
        buf_store<float>(val, rdl, vo + col * 4, so);
      }
      qdq = quad_sum(qdq);
      if (part == 0) buf_store<float>(qdq, rgq, (unsigned int)t * H * 4, (unsigned int)ic * kBT * H * 4);
    }
  } while (++ic < cend);
}

// ---------------------------------------------------------------------------
// dk, dv and dG: reverse walk over one segment, 8 waves
// ---------------------------------------------------------------------------
template <int NP>
struct DkvSmem {
  BwdStage<NP> st;
  __bf16 as[NP][kBT * kLd];  // (M o S)[t][s]
  __bf16 ap[NP][kBT * kLd];  // (M o dP)[t][s]
  float dgk[kBT][4];        // k . dk inter-chunk partials [s][wave]
  float kdk[kBT][4];        // k . dk intra-chunk column sums [s][t-tile]
};

template <int NP, typename TK, typename TV, typename TL, typename E = __bf16>
__global__ __launch_bounds__(512, 1) void mamba2_bwd_dkv_kernel(
    const TK* __restrict__ q, const TK* __restrict__ k, const TV* __restrict__ v,
    const TK* __restrict__ dO, const float* __restrict__ gcin, const TL* __restrict__ l,
    const float* __restrict__ rsum, const float* __restrict__ segd,
    const float* __restrict__ dgq, TK* __restrict__ dk, TV* __restrict__ dv,
    float* __restrict__ dg, float* __restrict__ segtot, int B, int T, int H, int V, int L,
    int nlev, int slog, int NSEG) {
  __shared__ __attribute__((aligned(16))) DkvSmem<NP> sm;
  BwdStage<NP>& s = sm.st;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int role = w >> 2, wr = w & 3;     // role 0: dk (k-tile wr), role 1: dv (v-tile wr)
  const int I = blockIdx.x;
  const int h = I % H, p = (I / H) % NSEG, b = I / (H * NSEG);
  const int row = b * H + h;
  const int NT = T / kBT;
  const int c0 = p << slog, cend = min(c0 + (1 << slog), NT);
  const int lu = 7 + nlev;
  const int nloc = min(slog, nlev), ntop = nlev - nloc;

  // Reverse states in the role's layout, lane (lq, ln), m = 0..3, i = 0..3:
  //   role 0: DH^T[v = 16m + 4lq + i][k = 16wr + ln]
  //   role 1: DH  [k = 16m + 4lq + i][v = 16wr + ln]
  floatx4 dh[kMaxLoc][4];
#pragma unroll
  for (int e = 0; e < kMaxLoc; ++e)
#pragma unroll
    for (int m = 0; m < 4; ++m) dh[e][m] = zero4();
  // combined top-level state: sum over top levels whose bit in p is clear of
  // the reading block's summaries decayed to the end of segment p
  floatx4 tp[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) tp[m] = zero4();
  if (ntop > 0) {
    const float* dp = segd + (size_t)row * NSEG;
    // element (a, c) of this lane's part of a summary: role 0 reads R[c][a], role 1 R[a][c]
    const int c = 16 * wr + ln;
    for (int e2 = 0; e2 < ntop; ++e2) {
      if ((p >> e2) & 1) continue;
      const int lo = ((p >> e2) | 1) << e2;
      const int hi = min(lo + (1 << e2), NSEG);
      float dlog = 0.f;
      for (int r = p + 1; r < lo; ++r) dlog += dp[r];
      // two summaries per step, all their loads issued before the sums
      for (int q0 = lo; q0 < hi; q0 += 2) {
        float x[2][16], sc[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int qs = min(q0 + u, hi - 1);
          const float* src = rsum + (((size_t)row * NSEG + qs) * ntop + e2) * kKD * kKD;
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int a = 16 * m + 4 * lq + i;
              x[u][4 * m + i] = role == 0 ? src[c * kKD + a] : src[a * kKD + c];
            }
        }
        sc[0] = fexp(dlog);
        dlog += dp[q0];
        sc[1] = q0 + 1 < hi ? fexp(dlog) : 0.f;
        if (q0 + 1 < hi) dlog += dp[q0 + 1];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) tp[m][i] += sc[u] * x[u][4 * m + i];
      }
    }
  }

  BwdLoader<512, TK, TV, TL> ld;
  ld.init(q, k, v, dO, gcin, l, b, h, T, H, V, L, lu);
  const size_t rq0 = (size_t)b * T * H + h;
  const rsrc_t rdk = make_rsrc(dk + rq0 * kKD, (size_t)T * H * kKD * sizeof(TK));
  const rsrc_t rdv = make_rsrc(dv + rq0 * V, (size_t)T * H * V * sizeof(TV));
  // dg and q . dq are wave 0's: the other waves issue the same load and store
  // through empty ranges, so every wave has one memory-operation sequence
  const rsrc_t rdg = make_rsrc(dg + rq0, w == 0 ? (size_t)T * H * 4 : 0);
  const rsrc_t rgq = make_rsrc(dgq + rq0, w == 0 ? (size_t)T * H * 4 : 0);
  const unsigned int vo_dk = (ln * H * kKD + 16 * wr + 4 * lq) * sizeof(TK);
  const unsigned int vo_dv = (ln * H * V + 16 * wr + 4 * lq) * sizeof(TV);

  BwdRegs<512, TK, TV, TL> rg;
  ld.load(rg, cend - 1);
  __builtin_amdgcn_sched_barrier(0);
  {
    // As many stores through an empty range as the loop issues after the next
    // chunk's loads (the q . dq load, four dk / dv stores and the dg store
    // follow them on the back edge): the loop header then sees the same
    // memory-operation order on both incoming paths, and the staging wait
    // leaves those operations in flight.
    const rsrc_t rnone = make_rsrc(dk, 0);
#pragma unroll
    for (int m = 0; m < 6; ++m)
      buf_store4<TK>(zero4(), rnone, vo_dk, 16u * m * H * kKD * sizeof(TK));
  }
  float carry = 0.f;   // sum of dG over the later chunks of this segment
  // cend > c0: a do-while, so the preheader runs straight into the body; the
  // previous chunk's loads are unconditional (the first chunk reloaded at the end)
  int ic = cend - 1;
  do {
    ld.template store<NP, E>(rg, s);
    // q . dq of this chunk's tokens (written by the dq kernel), needed by wave 0 at
    // the end of the chunk: loaded now so the load has the whole chunk to land
    const unsigned int vo_g = (unsigned int)lane * H * 4, so_g = (unsigned int)ic * kBT * H * 4;
    const float qdq = buf_load<float>(rgq, vo_g, so_g);
    __syncthreads();

    // ---- phase 1: (M o S) and (M o dP) tiles ---------------------------------------
    if constexpr (NP == 1) {
      // the wave's two tiles together (LDS reads, MFMAs, masks, then the eight
      // independent row sums); a missing second tile computes tile (0, 0) and
      // stores nothing, a zero tile stores zeros
      int tmt[2], tjt[2];
      bool live[2], causal[2];
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const int code = p1_tile8(w, n);
        live[n] = code >= 0;
        causal[n] = code >= 0 && code < 16;
        const int cc = code >= 0 ? code : 0;
        tmt[n] = (cc & 15) >> 2;
        tjt[n] = cc & 3;
      }
      floatx4 S[2], P[2];
      st_dpt_tiles2<E>(s, tmt, tjt, S, P);
      float os[2][4], op[2][4], c[2][4];
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const TileMask mk = tile_mask_sel(s, tmt[n], tjt[n], causal[n]);
        const int t = 16 * tmt[n] + ln;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float m = mk.dec[i] * s.lam[mk.lev[i] * kBT + t];
          os[n][i] = m * S[n][i];
          op[n][i] = m * P[n][i];
          c[n][i] = m * S[n][i] * P[n][i];
        }
      }
      // k_s . dk_s (intra part) = column sum over t of (M o S o dP), in fp32
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) c[n][i] = row_sum16(c[n][i]);
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        if (causal[n] && ln == 0)
#pragma unroll
          for (int i = 0; i < 4; ++i) sm.kdk[16 * tjt[n] + 4 * lq + i][tmt[n]] = c[n][i];
        if (live[n]) {
          const int off = (16 * tmt[n] + ln) * kLd + 16 * tjt[n] + 4 * lq;
          store_planes4<NP, E>(sm.as, off, os[n]);
          store_planes4<NP, E>(sm.ap, off, op[n]);
        }
      }
    } else
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int code = p1_tile8(w, n);
      if (code >= 0) {
        const int mt = (code & 15) >> 2, jt = code & 3;
        const int t = 16 * mt + ln;
        float os[4] = {0.f, 0.f, 0.f, 0.f}, op[4] = {0.f, 0.f, 0.f, 0.f};
        if (code < 16) {
          floatx4 S, P;
          st_dpt_tile<NP, E>(s, mt, jt, S, P);
          const TileMask mk = tile_mask(s, mt, jt);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float m = mk.dec[i] * s.lam[mk.lev[i] * kBT + t];
            os[i] = m * S[i];
            op[i] = m * P[i];
            // k_s . dk_s (intra part) = column sum over t of (M o S o dP), in fp32
            const float c = row_sum16(m * S[i] * P[i]);
            if (ln == 0) sm.kdk[16 * jt + 4 * lq + i][mt] = c;
          }
        }
        store_planes4<NP, E>(sm.as, t * kLd + 16 * jt + 4 * lq, os);
        store_planes4<NP, E>(sm.ap, t * kLd + 16 * jt + 4 * lq, op);
      }
    }
    __syncthreads();
    // the previous chunk's loads, issued after phase 1 rather than at the chunk
    // start, right behind the dk / dv / dg stores of the chunk before
    ld.load(rg, max(ic - 1, c0));

    // ---- phase 2: dk^T (role 0) / dv^T (role 1) for the chunk's tokens s -------------
    typedef const __bf16 (*Planes)[kBT * kLd];
    Planes xa = role == 0 ? s.q : s.d;      // A of the intra product: Q^T / dO^T
    Planes xb = role == 0 ? sm.ap : sm.as;  // B: (M o dP) / (M o S)
    Planes xs = role == 0 ? s.v : s.k;      // B of the inter product: V / K rows s
    floatx4 out[4];
    {
      bf16x8 a1[NP], a0[NP];
      trfrag<NP>(xa, 32, 16 * wr, a1);
      trfrag<NP>(xa, 0, 16 * wr, a0);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        // t-steps covering t >= s: both for s-tiles 0, 1; the second for 2, 3
        bf16x8 bx[NP];
        trfrag<NP>(xb, 32, 16 * mt, bx);
        out[mt] = mma<NP, E>(a1, bx, zero4());
        if (mt < 2) {
          trfrag<NP>(xb, 0, 16 * mt, bx);
          out[mt] = mma<NP, E>(a0, bx, out[mt]);
        }
      }
    }
    {
      // DHsum = sum of the local levels this chunk is a source of, plus the top part
      floatx4 dsum[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) dsum[m] = tp[m];
#pragma unroll
      for (int e = 0; e < kMaxLoc; ++e) {
        if (e < nloc && !((ic >> e) & 1)) {
#pragma unroll
          for (int m = 0; m < 4; ++m) dsum[m] += dh[e][m];
        }
      }
      bf16x8 a0[NP], a1[NP];
      cat8s<NP, E>(dsum[0], dsum[1], a0);
      cat8s<NP, E>(dsum[2], dsum[3], a1);
      // two s-tiles at a time: their LDS reads, then their MFMAs, then the FMAs;
      // k_s . dk_s (inter-chunk part) by one transposed cross-row sum at the end
      float r[4];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        bf16x8 rp[2][2][NP];
        float ws[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          row_pairs<NP>(xs, 16 * (2 * hf + u) + ln, 0, rp[u][0]);
          row_pairs<NP>(xs, 16 * (2 * hf + u) + ln, 32, rp[u][1]);
          ws[u] = s.wt[16 * (2 * hf + u) + ln];
        }
        floatx4 y[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          y[u] = mma<NP, E>(a0, rp[u][0], zero4());
          y[u] = mma<NP, E>(a1, rp[u][1], y[u]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int mt = 2 * hf + u;
#pragma unroll
          for (int i = 0; i < 4; ++i) out[mt][i] += y[u][i] * ws[u];
          if (role == 0) {
            const int koff = (16 * mt + ln) * kLd + 16 * wr + 4 * lq;
            const bf16x4 kx = *(const bf16x4*)(s.k[0] + koff);
            float rr = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) rr += from16<E>(kx[i]) * y[u][i];
            if constexpr (NP == 2) {
              const bf16x4 kl = *(const bf16x4*)(s.k[1] + koff);
#pragma unroll
              for (int i = 0; i < 4; ++i) rr += (float)kl[i] * y[u][i];
            }
            r[mt] = rr;
          }
        }
      }
      if (role == 0) sm.dgk[16 * lq + ln][wr] = sum_lq_t(r, lq) * s.wt[16 * lq + ln];
    }
    if (role == 0) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        buf_store4<TK>(out[mt], rdk, vo_dk, ((unsigned int)ic * kBT + 16 * mt) * H * kKD * sizeof(TK));
    } else {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        buf_store4<TV>(out[mt], rdv, vo_dv, ((unsigned int)ic * kBT + 16 * mt) * H * V * sizeof(TV));
    }

    // ---- phase 3: reverse states to the boundary before this chunk ----------------------
    const float cl = s.gc[kBT - 1];
    const float gl = fexp(cl);
    if (nloc > 0) {
      Planes ya = role == 0 ? s.d : s.q;   // A: dO^T / Q^T (rows of the state)
      Planes yb = role == 0 ? s.q : s.d;   // B: sigma o Q / sigma o dO
      // bf16 inputs: the A fragments and the unscaled B fragments are the same for
      // every level the chunk reads (only the lambda scaling of B differs), so they
      // are loaded once per chunk, before the level loop, when any level reads
      constexpr int NA = NP == 1 ? 4 : 1;
      bf16x8 af[NA][2][NP], yt0[NP], yt1[NP];
      if constexpr (NP == 1) {
        if (ic & ((1 << nloc) - 1)) {
          trfrag<NP>(yb, 0, 16 * wr, yt0);
          trfrag<NP>(yb, 32, 16 * wr, yt1);
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            trfrag<NP>(ya, 0, 16 * m, af[m][0]);
            trfrag<NP>(ya, 32, 16 * m, af[m][1]);
          }
        }
      }
#pragma unroll
      for (int e = 0; e < kMaxLoc; ++e) {
        if (e < nloc) {
          const int per = 2 << e;
          const bool reset = (ic & (per - 1)) == 0;
          const bool rd = (ic >> e) & 1;
          if (reset) {
#pragma unroll
            for (int m = 0; m < 4; ++m) dh[e][m] = zero4();
          } else {
#pragma unroll
            for (int m = 0; m < 4; ++m) dh[e][m] *= gl;
            if (rd) {
              const float* sg = s.lam + (7 + e) * kBT;
              bf16x8 b0[NP], b1[NP];
              if constexpr (NP == 1) {
                scale8s<NP, E>(yt0, *(const floatx4*)(sg + 8 * lq), *(const floatx4*)(sg + 8 * lq + 4),
                            b0);
                scale8s<NP, E>(yt1, *(const floatx4*)(sg + 32 + 8 * lq),
                            *(const floatx4*)(sg + 36 + 8 * lq), b1);
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                  dh[e][m] = mma<NP, E>(af[m][0], b0, dh[e][m]);
                  dh[e][m] = mma<NP, E>(af[m][1], b1, dh[e][m]);
                }
              } else {
                bf16x8 yt[NP];
                trfrag<NP>(yb, 0, 16 * wr, yt);
                scale8s<NP, E>(yt, *(const floatx4*)(sg + 8 * lq), *(const floatx4*)(sg + 8 * lq + 4),
                            b0);
                trfrag<NP>(yb, 32, 16 * wr, yt);
                scale8s<NP, E>(yt, *(const floatx4*)(sg + 32 + 8 * lq),
                            *(const floatx4*)(sg + 36 + 8 * lq), b1);
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                  trfrag<NP>(ya, 0, 16 * m, af[0][0]);
                  dh[e][m] = mma<NP, E>(af[0][0], b0, dh[e][m]);
                  trfrag<NP>(ya, 32, 16 * m, af[0][1]);
                  dh[e][m] = mma<NP, E>(af[0][1], b1, dh[e][m]);
                }
              }
            }
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) tp[m] *= gl;
    __syncthreads();

    // ---- dG = q . dq - k . dk and its reverse cumsum inside the segment --------------
    float xg = 0.f;
    if (w == 0) {
      // column sums over the t-tiles at or after this s-tile (the others are zero)
      float kdk = sm.dgk[lane][0] + sm.dgk[lane][1] + sm.dgk[lane][2] + sm.dgk[lane][3];
      for (int mt = lane >> 4; mt < 4; ++mt) kdk += sm.kdk[lane][mt];
      const float dG = qdq - kdk;
      const float x = chunk_rsum(dG);   // inclusive suffix sum over the chunk
      xg = x + carry;
      carry += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 0));
    }
    buf_store<float>(xg, rdg, vo_g, so_g);
  } while (--ic >= c0);
  if (tid == 0) segtot[(size_t)row * NSEG + p] = carry;
}

// dg of segment p += sum of the totals of the segments after p.
__global__ __launch_bounds__(256) void mamba2_bwd_dg_kernel(float* __restrict__ dg,
                                                            const float* __restrict__ segtot,
                                                            int T, int H, int slog, int NSEG) {
  const int I = blockIdx.x;
  const int h = I % H, p = (I / H) % NSEG, b = I / (H * NSEG);
  const int row = b * H + h;
  float off = 0.f;
  for (int r = p + 1; r < NSEG; ++r) off += segtot[(size_t)row * NSEG + r];
  const int t0 = (p << slog) * kBT, t1 = min(((p + 1) << slog) * kBT, T);
  float* d = dg + (size_t)b * T * H + h;
  for (int t = t0 + (int)threadIdx.x; t < t1; t += 256) d[(size_t)t * H] += off;
}

// ---------------------------------------------------------------------------
// host launcher
// ---------------------------------------------------------------------------
struct BwdWs {
  float *segd, *sums, *rsum, *dgq, *segtot;
  __bf16* htop;
  size_t bytes;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

inline BwdWs bwd_ws_layout(void* base, int B, int T, int H, int V, int nlev) {
  const int NT = T / kBT;
  const int slog = seg_log2(NT);
  const int NSEG = (NT + (1 << slog) - 1) >> slog;
  const int ntop = nlev - min(slog, nlev);
  const size_t rows = (size_t)B * H;
  BwdWs w;
  size_t off = 0;
  char* p = (char*)base;
  w.segd = (float*)(p + off);   off += align256(rows * NSEG * 4);
  w.segtot = (float*)(p + off); off += align256(rows * NSEG * 4);
  w.dgq = (float*)(p + off);    off += align256((size_t)B * T * H * 4);
  w.sums = (float*)(p + off);   off += align256(NSEG > 1 ? rows * NSEG * kKD * V * 4 : 0);
  w.rsum = (float*)(p + off);   off += align256(rows * NSEG * ntop * kKD * kKD * 4);
  // room for two bf16 planes (the bf16x3 backward)
  w.htop = (__bf16*)(p + off);  off += align256(rows * NSEG * ntop * kKD * kKD * 2 * 2);
  w.bytes = off;
  return w;
}

// fsums / fsegd (or null): the forward's segment summaries and log-decays of
// these inputs (its workspace, same segmentation and layout), which then
// replace the summary pass.
// E: the 16-bit MFMA format (NP = 1): bf16, or fp16 for fp16 q / k / v / dO.
template <int NP, typename TK, typename TV, typename TL, typename E = __bf16>
static hipError_t bwd_launch_t(const void* q, const void* k, const void* v, const float* gc,
                               const void* l, const void* dO, void* dq, void* dk, void* dv,
                               float* dg, float* dl, void* ws, const float* fsums,
                               const float* fsegd, int B, int T, int H, int V, int L, int nlev,
                               hipStream_t stream) {
  const int NT = T / kBT;
  const int slog = seg_log2(NT);
  const int NSEG = (NT + (1 << slog) - 1) >> slog;
  const int nloc = min(slog, nlev), ntop = nlev - nloc;
  const int rows = B * H;
  const BwdWs w = bwd_ws_layout(ws, B, T, H, V, nlev);
  const bool reuse = fsums != nullptr && fsegd != nullptr;
  const float* sums = reuse ? fsums : w.sums;
  const float* segd = reuse ? fsegd : w.segd;
  hipError_t e;
  if (NSEG > 1 && !reuse) {
    auto sk = mamba2_seg_sum_kernel<TK, TV, true, NP, E>;
    hipLaunchKernelGGL(sk, dim3(xcd_head_grid(B * NSEG, H, 1)), dim3(256), 0, stream,
                       (const TK*)k, (const TV*)v, gc, w.sums, w.segd, B, T, H, H, V, NT,
                       1 << slog, NSEG, 1);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (ntop > 0) {
    // top-level states of every segment for the dq kernel
    auto hk = mamba2_htop_kernel<NP, E>;
    hipLaunchKernelGGL(hk, dim3(rows * 4), dim3(256), 0, stream, sums, segd, w.htop, V, NSEG,
                       ntop, 1);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int ngrp = (ntop + 3) / 4;
    auto rk = mamba2_bwd_rsum_kernel<NP, TK, TL, E>;
    hipLaunchKernelGGL(rk, dim3(xcd_head_grid(B * NSEG, H, ngrp)), dim3(256), 0, stream,
                       (const TK*)q, (const TK*)dO, gc, (const TL*)l, w.rsum, B, T, H, L, NT,
                       slog, NSEG, nloc, ntop, ngrp);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    auto kq = mamba2_bwd_dq_kernel<NP, TK, TV, TL, E>;
    hipLaunchKernelGGL(kq, dim3(xcd_head_grid(B * NSEG, H, 1)), dim3(256), 0, stream,
                       (const TK*)q, (const TK*)k, (const TV*)v, (const TK*)dO, gc,
                       (const TL*)l, w.htop, (TK*)dq, dl, w.dgq, B, T, H, V, L, nlev, slog,
                       NSEG);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    auto kk = mamba2_bwd_dkv_kernel<NP, TK, TV, TL, E>;
    hipLaunchKernelGGL(kk, dim3(rows * NSEG), dim3(512), 0, stream, (const TK*)q,
                       (const TK*)k, (const TV*)v, (const TK*)dO, gc, (const TL*)l,
                       w.rsum, segd, w.dgq, (TK*)dk, (TV*)dv, dg, w.segtot, B, T, H, V, L,
                       nlev, slog, NSEG);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (NSEG > 1) {
    hipLaunchKernelGGL(mamba2_bwd_dg_kernel, dim3(rows * NSEG), dim3(256), 0, stream, dg,
                       w.segtot, T, H, slog, NSEG);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace hattn

size_t hattn_mamba2_bwd_ws_bytes(int B, int T, int H, int V, int nlev) {
  return hattn::bwd_ws_layout(nullptr, B, T, H, V, nlev).bytes;
}

// dt_qk (= the dtype of dO): bf16 selects the bf16 kernels (v and lambda bf16 or
// fp32); fp32 the bf16x3 kernels, which take fp32 v and lambda and write fp32
// dq, dk, dv.
hipError_t hattn_mamba2_bwd_launch(const void* q, const void* k, const void* v, const float* gc,
                                   const void* l, const void* dO, void* dq, void* dk, void* dv,
                                   float* dg, float* dl, void* ws, const float* fsums,
                                   const float* fsegd, int B, int T, int H, int V, int L,
                                   int nlev, int dt_qk, int dt_v, int dt_l, hipStream_t stream,
                                   int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  if (dt_qk == 2) {
    if (dt_v == 2 && dt_l == 2)
      return bwd_launch_t<2, float, float, float>(q, k, v, gc, l, dO, dq, dk, dv, dg, dl, ws, fsums,
                                                  fsegd, B, T, H, V, L, nlev, stream);
    *unsupported = 1;
    return hipSuccess;
  }
  if (dt_qk == 1) {
    // fp16 q / k / dO on fp16 MFMA (fp32 lambda; v fp16 or fp32)
    if (dt_l == 2 && dt_v == 1)
      return bwd_launch_t<1, _Float16, _Float16, float, _Float16>(
          q, k, v, gc, l, dO, dq, dk, dv, dg, dl, ws, fsums, fsegd, B, T, H, V, L, nlev, stream);
    if (dt_l == 2 && dt_v == 2)
      return bwd_launch_t<1, _Float16, float, float, _Float16>(
          q, k, v, gc, l, dO, dq, dk, dv, dg, dl, ws, fsums, fsegd, B, T, H, V, L, nlev, stream);
    *unsupported = 1;
    return hipSuccess;
  }
  if (dt_qk != 0) {
    *unsupported = 1;
    return hipSuccess;
  }
  if (dt_v == 0 && dt_l == 0)
    return bwd_launch_t<1, __bf16, __bf16, __bf16>(q, k, v, gc, l, dO, dq, dk, dv, dg, dl, ws, fsums, fsegd, B, T, H, V, L, nlev, stream);
  if (dt_v == 0 && dt_l == 2)
    return bwd_launch_t<1, __bf16, __bf16, float>(q, k, v, gc, l, dO, dq, dk, dv, dg, dl, ws, fsums, fsegd, B, T, H, V, L, nlev, stream);
  if (dt_v == 2 && dt_l == 0)
    return bwd_launch_t<1, __bf16, float, __bf16>(q, k, v, gc, l, dO, dq, dk, dv, dg, dl, ws, fsums, fsegd, B, T, H, V, L, nlev, stream);
  if (dt_v == 2 && dt_l == 2)
    return bwd_launch_t<1, __bf16, float, float>(q, k, v, gc, l, dO, dq, dk, dv, dg, dl, ws, fsums, fsegd, B, T, H, V, L, nlev, stream);
  *unsupported = 1;
  return hipSuccess;
}
