// Log-linear Mamba-2 chunkwise backward for the strong hierarchy (HType.STRONG)
// on gfx950.
//
// Replaces chunkwise.chunkwise_bwd with htype == STRONG (chunkwise.py:1286-1597):
// the reference runs the intra-chunk dqkwg / dv kernels with USE_A2 (the
// sub-diagonal tiles) and, per inter-chunk level from 1, a state recompute and
// a reverse state scan with four phase states per level (USE_H2,
// MODE_H2 = 3, chunkwise.py:1377-1384, 1460-1580).
//
// The forward (mamba2_strong.hip) writes
//   o_t = sum_{s in chunk n}     lam[t, intra(a, b)] e^{G_t - G_s} (q_t.k_s) v_s
//       + sum_{s in chunk n - 1} lam[t, sub(a, b)]   e^{G_t - G_s} (q_t.k_s) v_s
//       + sum_{j >= 2} lam[t, 6 + j] e^{Gc_t} q_t . S_j(n),
// S_j(n) level j of the chunk-level strong state (one insertion per chunk,
// value kv_n = K_n^T diag(e^{Gc_last - Gc}) V_n, gate e^{Gc_last}), read after
// the cascade of step n.  Its gradients:
//   * far, forward in time (mamba2_strong_bwd_walk_kernel, forward half):
//       dq_t += sum_j lam[t, 6 + j] e^{Gc_t} S_j(n) do_t
//       dlam[t, 6 + j] = e^{Gc_t} q_t . S_j(n) do_t
//   * far, backward in time (the same kernel, reverse half): the adjoint A of
//     the state runs the transposed steps in reverse order (A_0 -> d kv_n,
//     A_0 = 0, A *= e^{Gc_last}, A_j += Q_n^T diag(lam[., 6 + j] e^{Gc}) dO_n,
//     then the transposed cascade: levels 0 .. m-1 take levels 1 .. m, m the
//     merge level of the forward cascade at step n), and d kv_n gives
//       dk_s += e^{Gc_last - Gc_s} d kv_n v_s,  dv_s += e^{Gc_last - Gc_s} d kv_n^T k_s
//   * the diagonal and sub-diagonal blocks, one workgroup per chunk
//     (mamba2_strong_bwd_dq_kernel: target chunk n -> dq, dlam[., 0 .. 7] from
//     the per-(target, level) source ranges, the far parts added;
//     mamba2_strong_bwd_dkv_kernel: source chunk n -> dk, dv);
//   * dG_t = q_t . dq_t - k_t . dk_t and dg_u = sum_{t >= u} dG_t (the
//     reference's reverse chunk-local cumsum of its dg accumulator,
//     chunkwise.py:1596, with the inter-chunk terms inside dq and dk):
//     chunk-local in the dkv kernel, the later chunks' totals added by
//     mamba2_strong_bwd_dg_kernel.
// The walks hold one 16-row slice of K of every level (16 x 64 fp32 per level
// in registers); the four slices of a row reduce dlam through a workspace in a
// fixed order.  bf16 q, k, v, dO (bf16 MFMA, fp32 accumulation), K = V = 64.
#include "mamba2_strong.h"

namespace hattn {

__device__ constexpr StrongTables kStrongB{};
__device__ constexpr StrongRanges kStrongR{};

constexpr int kWLd = 72;                 // row stride of 64-wide bf16 tiles
constexpr int kWLs = 24;                 // row stride of 16-wide bf16 tiles
constexpr int kNFar = kSMaxLev - 2;      // far levels j = 2 .. 9
constexpr int kSMaxChunks = 1 << (kSMaxLev - 1);
constexpr int kMLd = 2 * kSC + 4;        // row stride of the staged dlambda terms

struct StrongBwdWs {
  float* dqf;     // [row][T][64] far part of dq
  float* dlf;     // [4][row][T][nf] far dlambda, one partial per 16-row K slice
  __bf16* adj;    // [row][NT][64 k][64 v] adjoint of each chunk's insertion
  float* qdq;     // [row][T] q . dq
  float* dgt;     // [row][NT] chunk totals of dG
  size_t bytes;
};

inline size_t align256s(size_t x) { return (x + 255) & ~(size_t)255; }

inline StrongBwdWs strong_bwd_ws_layout(void* base, int B, int T, int H, int nf) {
  const size_t rows = (size_t)B * H, NT = T / kSC;
  const size_t nf1 = nf > 0 ? nf : 1;
  StrongBwdWs w;
  char* p = (char*)base;
  size_t off = 0;
  w.dqf = (float*)(p + off);  off += align256s(rows * T * 64 * 4);
  w.dlf = (float*)(p + off);  off += align256s(4 * rows * T * nf1 * 4);
  w.adj = (__bf16*)(p + off); off += align256s(rows * NT * 64 * 64 * 2);
  w.qdq = (float*)(p + off);  off += align256s(rows * T * 4);
  w.dgt = (float*)(p + off);  off += align256s(rows * NT * 4);
  w.bytes = off;
  return w;
}

// ---------------------------------------------------------------------------
// chunk walks (far levels)
// ---------------------------------------------------------------------------
constexpr int kWThreads = 512;   // eight waves per walk workgroup

struct WalkSmem {
  __bf16 d[kSC * kWLd];               // dO [t][v]
  __bf16 v[kSC * kWLd];               // V [t][v] (forward walk)
  __bf16 q[2][kSC * kWLs];            // q [t][16-row K slice]: the forward walk's slice
                                      // (first), or the reverse walk's two slices
  __bf16 k[kSC * kWLs];               // k [t][16-row K slice] (forward walk)
  __bf16 hs[kSMaxLev][16 * kWLd];     // forward walk: levels >= 2 as bf16 [k][v]
  float gc[kSC];
  float f[kNFar][kSC];                // lam[t, 8 + jj] e^{Gc_t}
  unsigned char mlev[kSMaxChunks];    // reverse walk: merge level of each step
};

struct WalkArgs {
  const __bf16 *q, *k, *v, *dO;
  const float* gc;
  const void* l;
  StrongBwdWs ws;
  int rows, T, H, L, nf;
};

// The chunk's dO (and for the forward walk V), the q (and k) columns of the
// workgroup's K slices, Gc and the far lambda weights, loaded into registers
// one chunk ahead (walk_load) and written to LDS at the chunk start
// (walk_store).  One 16-byte unit of each per thread.
template <typename TL>
struct WalkPre {
  u32x4 d, v, q, k;
  float g;
  TL lf;
  float gf;
};

// k0: the first K column of the workgroup's slices (16 forward, 32 reverse)
template <typename TL, bool FWD>
__device__ __forceinline__ void walk_load(WalkPre<TL>& p, const WalkArgs& a, size_t tok0, int h,
                                          int k0) {
  const int tid = threadIdx.x, lane = tid & 63;
  const size_t hd = (size_t)a.H * 64;
  {
    const int r = tid >> 3, c8 = 8 * (tid & 7);
    const size_t off = (tok0 + r) * hd + (size_t)h * 64 + c8;
    p.d = *(const u32x4*)(a.dO + off);
    if constexpr (FWD) p.v = *(const u32x4*)(a.v + off);
  }
  if constexpr (FWD) {
    const int r = (tid & 127) >> 1, c8 = 8 * (tid & 1);
    const size_t off = (tok0 + r) * hd + (size_t)h * 64 + k0 + c8;
    p.q = *(const u32x4*)(a.q + off);
    p.k = *(const u32x4*)(a.k + off);
  } else {
    const int r = (tid & 255) >> 2, c8 = 8 * (tid & 3);
    p.q = *(const u32x4*)(a.q + (tok0 + r) * hd + (size_t)h * 64 + k0 + c8);
  }
  p.g = a.gc[(tok0 + lane) * a.H + h];
  const TL* l = (const TL*)a.l;
  const int nf1 = a.nf > 0 ? a.nf : 1;
  const int i = min(tid, nf1 * kSC - 1);
  const size_t tk = (tok0 + i / nf1) * a.H + h;
  p.lf = l[tk * a.L + min(8 + i % nf1, a.L - 1)];   // column clamped for nf == 0
  p.gf = a.gc[tk];
}

template <typename TL, bool FWD>
__device__ __forceinline__ void walk_store(WalkSmem& s, const WalkPre<TL>& p, const WalkArgs& a) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  {
    const int r = tid >> 3, c8 = 8 * (tid & 7);
    *(u32x4*)(s.d + r * kWLd + c8) = p.d;
    if constexpr (FWD) *(u32x4*)(s.v + r * kWLd + c8) = p.v;
  }
  if constexpr (FWD) {
    if (tid < 128) {
      const int r = tid >> 1, c8 = 8 * (tid & 1);
      *(u32x4*)(s.q[0] + r * kWLs + c8) = p.q;
      *(u32x4*)(s.k + r * kWLs + c8) = p.k;
    }
  } else {
    if (tid < 256) {
      const int r = tid >> 2, c8 = 8 * (tid & 3);
      *(u32x4*)(s.q[c8 >> 4] + r * kWLs + (c8 & 15)) = p.q;
    }
  }
  if (w == 0) s.gc[lane] = p.g;
  if (tid < a.nf * kSC) s.f[tid % a.nf][tid / a.nf] = to_f32<TL>(p.lf) * fexp(p.gf);
}

// Forward walk: far dq of the slice (complete) and the slice's partial far
// dlambda.  Near waves 0-3 own the strong state (S_j[k = k0 + 4 lq + i][v =
// 16 w + ln]): the cascade, the bf16 staging of the levels >= 2 and, after the
// far products are issued, the decay and insertion of the chunk; far waves
// 4-7 run the products of the levels >= 2 for the tokens 16 (w - 4) .. + 15.
template <typename TL>
__device__ __forceinline__ void strong_walk_fwd(WalkSmem& s, const WalkArgs& a, int row, int kap) {
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const bool near = w < 4;
  const int wq = w & 3;
  const int b = row / a.H, h = row % a.H, NT = a.T / kSC, k0 = 16 * kap;
  const int t_me = 16 * wq + ln;
  floatx4 st[kSMaxLev];   // near: S_j[k = k0 + 4 lq + i][v = 16 w + ln]
  int cnt[kSMaxLev];
#pragma unroll
  for (int j = 0; j < kSMaxLev; ++j) {
    st[j] = zero4();
    cnt[j] = 0;
  }
  WalkPre<TL> pre;
  walk_load<TL, true>(pre, a, (size_t)b * a.T, h, k0);
  for (int ic = 0; ic < NT; ++ic) {
    // cascade (recurrent.py:56-74) over the chunk-level states
    if (near) {
      floatx4 carry = zero4();
      int cc = 0;
#pragma unroll
      for (int j = 0; j < kSMaxLev; ++j) {
        const int cap = 1 << (j > 0 ? j - 1 : 0);
        const bool swap = j == 0 || cnt[j] + cc > cap;
        const floatx4 old = st[j];
        const int oc = cnt[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          st[j][i] = swap ? carry[i] : old[i] + carry[i];
          carry[i] = swap ? old[i] : 0.f;
        }
        cnt[j] = swap ? cc : oc + cc;
        cc = swap ? oc : 0;
      }
    }
    walk_store<TL, true>(s, pre, a);
    if (near) {
#pragma unroll
      for (int j = 2; j < kSMaxLev; ++j)
        if (j - 2 < a.nf)
#pragma unroll
          for (int i = 0; i < 4; ++i) s.hs[j][(4 * lq + i) * kWLd + 16 * w + ln] = (__bf16)st[j][i];
    }
    __syncthreads();
    if (ic + 1 < NT) walk_load<TL, true>(pre, a, (size_t)b * a.T + (size_t)(ic + 1) * kSC, h, k0);

    if (!near) {
      // Y^T[k][t] = S_j[k][v] dO^T[v][t] for the lane's token t_me, k = k0 + 4 lq + i
      const bf16x8 bd0 = *(const bf16x8*)(s.d + t_me * kWLd + 8 * lq);
      const bf16x8 bd1 = *(const bf16x8*)(s.d + t_me * kWLd + 32 + 8 * lq);
      const bf16x4 q4 = *(const bf16x4*)(s.q[0] + t_me * kWLs + 4 * lq);
      const float eg = fexp(s.gc[t_me]);
      floatx4 dq = zero4();
      float* dlrow = a.ws.dlf + (((size_t)kap * a.rows + row) * a.T + (size_t)ic * kSC + t_me) * a.nf;
#pragma unroll
      for (int j = 2; j < kSMaxLev; ++j) {
        if (j - 2 < a.nf) {
          floatx4 y = mfma16x16x32(*(const bf16x8*)(s.hs[j] + ln * kWLd + 8 * lq), bd0, zero4());
          y = mfma16x16x32(*(const bf16x8*)(s.hs[j] + ln * kWLd + 32 + 8 * lq), bd1, y);
          const float f = s.f[j - 2][t_me];
          float p = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            dq[i] += f * y[i];
            p += (float)q4[i] * y[i];
          }
          p += __shfl_xor(p, 16, 64);
          p += __shfl_xor(p, 32, 64);
          if (lq == ((j - 2) & 3)) dlrow[j - 2] = p * eg;
        }
      }
      *(floatx4*)(a.ws.dqf + ((size_t)row * a.T + (size_t)ic * kSC + t_me) * 64 + k0 + 4 * lq) = dq;
    } else {
      // decay, then S_0 = K^T diag(e^{Gc_last - Gc}) V
      const float glast = s.gc[kSC - 1];
      const float gd = fexp(glast);
#pragma unroll
      for (int j = 1; j < kSMaxLev; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[j][i] *= gd;
      floatx4 sum = zero4();
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        bf16x8 ka = tr_frag(s.k, kWLs, 32 * c, 0);   // K[t = 32 c + 8 lq + jj][k0 + ln]
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          ka[jj] = (__bf16)((float)ka[jj] * fexp(glast - s.gc[32 * c + 8 * lq + jj]));
        sum = mfma16x16x32(ka, tr_frag(s.v, kWLd, 32 * c, 16 * w), sum);
      }
      st[0] = sum;
      cnt[0] += 1;
    }
    __syncthreads();
  }
}

// Reverse walk: the adjoint of every chunk's insertion, d kv_n, for two 16-row
// slices of K (slices 2 kp and 2 kp + 1): waves 4 sl .. 4 sl + 3 run slice
// 2 kp + sl, wave w & 3 owning the columns v = 16 (w & 3) .. + 15.
template <typename TL>
__device__ __forceinline__ void strong_walk_rev(WalkSmem& s, const WalkArgs& a, int row, int kp) {
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int wv = w & 3, sl = w >> 2;
  const int b = row / a.H, h = row % a.H, NT = a.T / kSC, k0 = 16 * (2 * kp + sl);
  // merge level of the forward cascade at each step: the first level >= 1
  // that keeps (or takes into an empty slot) the carry; kSMaxLev = dropped
  if (tid == 0) {
    int cnt[kSMaxLev];
#pragma unroll
    for (int j = 0; j < kSMaxLev; ++j) cnt[j] = 0;
    for (int n = 0; n < NT; ++n) {
      int cc = 0, m = kSMaxLev;
#pragma unroll
      for (int j = 0; j < kSMaxLev; ++j) {
        const int cap = 1 << (j > 0 ? j - 1 : 0);
        const bool swap = j == 0 || cnt[j] + cc > cap;
        const int oc = cnt[j];
        cnt[j] = swap ? cc : oc + cc;
        cc = swap ? oc : 0;
        if (j >= 1 && m == kSMaxLev && (!swap || oc == 0)) m = j;
      }
      s.mlev[n] = (unsigned char)m;
      cnt[0] += 1;
    }
  }
  floatx4 st[kSMaxLev];   // A_j[k = k0 + 4 lq + i][v = 16 wv + ln]
#pragma unroll
  for (int j = 0; j < kSMaxLev; ++j) st[j] = zero4();
  WalkPre<TL> pre;
  walk_load<TL, false>(pre, a, (size_t)b * a.T + (size_t)(NT - 1) * kSC, h, 32 * kp);
  for (int ic = NT - 1; ic >= 0; --ic) {
    walk_store<TL, false>(s, pre, a);
    {
      __bf16* ap = a.ws.adj + (((size_t)row * NT + ic) * 64 + k0 + 4 * lq) * 64 + 16 * wv + ln;
#pragma unroll
      for (int i = 0; i < 4; ++i) ap[i * 64] = (__bf16)st[0][i];
    }
    st[0] = zero4();
    __syncthreads();
    if (ic > 0) walk_load<TL, false>(pre, a, (size_t)b * a.T + (size_t)(ic - 1) * kSC, h, 32 * kp);
    const float gd = fexp(s.gc[kSC - 1]);
#pragma unroll
    for (int j = 1; j < kSMaxLev; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) st[j][i] *= gd;
    // A_j[k][v] += sum_t Q[t][k] f_j[t] dO[t][v], t = 32 c + 8 lq + jj
    const bf16x8 bd0 = tr_frag(s.d, kWLd, 0, 16 * wv), bd1 = tr_frag(s.d, kWLd, 32, 16 * wv);
    const bf16x8 qa0 = tr_frag(s.q[sl], kWLs, 0, 0), qa1 = tr_frag(s.q[sl], kWLs, 32, 0);
#pragma unroll
    for (int j = 2; j < kSMaxLev; ++j) {
      if (j - 2 < a.nf) {
        const floatx4 f0 = *(const floatx4*)(&s.f[j - 2][8 * lq]);
        const floatx4 f1 = *(const floatx4*)(&s.f[j - 2][8 * lq + 4]);
        const floatx4 f2 = *(const floatx4*)(&s.f[j - 2][32 + 8 * lq]);
        const floatx4 f3 = *(const floatx4*)(&s.f[j - 2][32 + 8 * lq + 4]);
        bf16x8 a0, a1;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          a0[jj] = (__bf16)((float)qa0[jj] * f0[jj]);
          a0[4 + jj] = (__bf16)((float)qa0[4 + jj] * f1[jj]);
          a1[jj] = (__bf16)((float)qa1[jj] * f2[jj]);
          a1[4 + jj] = (__bf16)((float)qa1[4 + jj] * f3[jj]);
        }
        st[j] = mfma16x16x32(a0, bd0, st[j]);
        st[j] = mfma16x16x32(a1, bd1, st[j]);
      }
    }
    // transposed cascade: levels 0 .. m-1 take levels 1 .. m (the top takes zero)
    const int m = __builtin_amdgcn_readfirstlane((int)s.mlev[ic]);
#pragma unroll
    for (int e = 0; e < kSMaxLev; ++e) {
      const floatx4 nx = e + 1 < kSMaxLev ? st[e + 1 < kSMaxLev ? e + 1 : e] : zero4();
      if (e < m) st[e] = nx;
    }
    __syncthreads();
  }
}

// Blocks [0, half): forward walks, one per (row, 16-row K slice); blocks
// [half, ..): reverse walks, one per (row, pair of K slices).
template <typename TL>
__global__ __launch_bounds__(kWThreads) void mamba2_strong_bwd_walk_kernel(WalkArgs a, int half) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  WalkSmem& s = *(WalkSmem*)smem_raw;
  int wg = blockIdx.x;
  const bool rev = wg >= half;
  if (rev) wg -= half;
  const XcdMap mp = xcd_map(wg, rev ? 2 : 4);
  if (mp.row >= a.rows) return;
  if (rev) strong_walk_rev<TL>(s, a, mp.row, mp.slice);
  else strong_walk_fwd<TL>(s, a, mp.row, mp.slice);
}

// ---------------------------------------------------------------------------
// diagonal / sub-diagonal blocks: dq and dlambda (target chunk n)
// ---------------------------------------------------------------------------
struct LocQSmem {
  __bf16 k[2][kSC * kWLd];     // K of chunks n - 1 (0) and n (1) [s][k]
  __bf16 v[2][kSC * kWLd];     // V of chunks n - 1, n [s][v]
  float m[kSC * kMLd];         // e^{G_t - G_s} (q_t.k_s)(do_t.v_s) [t][i], i = sub b / 64 + intra b
  float gc[2][kSC];
  float lam[kSC][kSLocLev];    // lambda[t, 0 .. 7] of chunk n
};

// One workgroup per (row, target chunk n).  Wave w owns the targets t = 16 w ..
// +15; transposed products (lane: one target, four consecutive sources / keys):
//   S^T = K Q^T, D^T = V dO^T over the sources of chunk n (s <= t) and n - 1,
//   dq^T[k][t] = sum_s K^T[k][s] (W o D)^T[s][t].
template <typename TL>
__global__ __launch_bounds__(256, 2) void mamba2_strong_bwd_dq_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const __bf16* __restrict__ dO, const float* __restrict__ gc, const TL* __restrict__ l,
    __bf16* __restrict__ dq, float* __restrict__ dl, StrongBwdWs ws, int rows, int T, int H,
    int L, int nf) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  LocQSmem& s = *(LocQSmem*)smem_raw;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int NT = T / kSC;
  const XcdMap mp = xcd_map(blockIdx.x, NT);
  if (mp.row >= rows) return;
  const int row = mp.row, n = mp.slice;
  const int b = row / H, h = row % H;
  const size_t tok0 = (size_t)b * T + (size_t)n * kSC;
  const size_t hd = (size_t)H * 64, hoff = (size_t)h * 64;
  const int t_me = 16 * w + ln;

  {
    const int r = tid >> 2, c16 = 16 * (tid & 3);
#pragma unroll
    for (int cur = 0; cur < 2; ++cur) {
      if (cur == 0 && n == 0) continue;
      const size_t off = (tok0 - (cur ? 0 : kSC) + r) * hd + hoff + c16;
      const u32x4 k0 = *(const u32x4*)(k + off), k1 = *(const u32x4*)(k + off + 8);
      const u32x4 v0 = *(const u32x4*)(v + off), v1 = *(const u32x4*)(v + off + 8);
      *(u32x4*)(s.k[cur] + r * kWLd + c16) = k0;
      *(u32x4*)(s.k[cur] + r * kWLd + c16 + 8) = k1;
      *(u32x4*)(s.v[cur] + r * kWLd + c16) = v0;
      *(u32x4*)(s.v[cur] + r * kWLd + c16 + 8) = v1;
    }
    if (w == 0) {
      s.gc[1][lane] = gc[(tok0 + lane) * H + h];
      if (n > 0) s.gc[0][lane] = gc[(tok0 - kSC + lane) * H + h];
    }
    for (int i = tid; i < kSC * kSLocLev; i += 256) {
      const int t = i / kSLocLev, e = i % kSLocLev;
      s.lam[t][e] = e < L ? to_f32<TL>(l[((tok0 + t) * H + h) * L + e]) : 0.f;
    }
  }
  // B operands of this wave's targets: Q^T[k][t_me], dO^T[v][t_me]
  const size_t rme = (tok0 + t_me) * hd + hoff;
  const bf16x8 bq0 = *(const bf16x8*)(q + rme + 8 * lq), bq1 = *(const bf16x8*)(q + rme + 32 + 8 * lq);
  const bf16x8 bd0 = *(const bf16x8*)(dO + rme + 8 * lq), bd1 = *(const bf16x8*)(dO + rme + 32 + 8 * lq);
  // every later global read, issued now: the level-table words of the lane's
  // source tiles, the far dq and q (q . dq), the far dlambda partials
  unsigned lvw[2][4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    lvw[0][st] = *(const unsigned*)(kStrongB.sub + t_me * kSC + 16 * st + 4 * lq);
    lvw[1][st] = *(const unsigned*)(kStrongB.intra + t_me * kSC + 16 * st + 4 * lq);
  }
  floatx4 fq[4];
  bf16x4 qk4[4];
  {
    const float* fp = ws.dqf + ((size_t)row * T + (size_t)n * kSC + t_me) * 64 + 4 * lq;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      fq[kt] = *(const floatx4*)(fp + 16 * kt);
      qk4[kt] = *(const bf16x4*)(q + rme + 16 * kt + 4 * lq);
    }
  }
  const int t_dl = tid >> 2, l0 = tid & 3;
  float dlp[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int jj = min(l0 + 4 * u, nf > 0 ? nf - 1 : 0);
#pragma unroll
    for (int kap = 0; kap < 4; ++kap)
      dlp[u][kap] = nf > 0 ? ws.dlf[(((size_t)kap * rows + row) * T + (size_t)n * kSC + t_dl) * nf + jj]
                           : 0.f;
  }
  __syncthreads();

  const float gct = s.gc[1][t_me];
  floatx4 acc[4];   // dq^T[k = 16 kt + 4 lq + i][t_me]
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) acc[kt] = zero4();
  float* mrow = s.m + t_me * kMLd;
#pragma unroll
  for (int cur = 0; cur < 2; ++cur) {
    if (cur == 0 && n == 0) {
#pragma unroll
      for (int st = 0; st < 4; ++st) *(floatx4*)(mrow + 16 * st + 4 * lq) = zero4();
      continue;
    }
    const float base = cur ? 0.f : s.gc[0][kSC - 1];
    const int npair = cur ? (w >> 1) + 1 : 2;
    for (int p = 0; p < npair; ++p) {
      bf16x8 pb;   // (W o D)^T[s = 32 p + {4 lq + i, 16 + 4 lq + i}][t_me]
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int st = 2 * p + half;
        const __bf16* kr = s.k[cur] + (16 * st + ln) * kWLd + 8 * lq;
        const __bf16* vr = s.v[cur] + (16 * st + ln) * kWLd + 8 * lq;
        floatx4 sc = mfma16x16x32(*(const bf16x8*)kr, bq0, zero4());
        sc = mfma16x16x32(*(const bf16x8*)(kr + 32), bq1, sc);
        floatx4 dd = mfma16x16x32(*(const bf16x8*)vr, bd0, zero4());
        dd = mfma16x16x32(*(const bf16x8*)(vr + 32), bd1, dd);
        const unsigned lv4 = lvw[cur][st];
        floatx4 mv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int sp = 16 * st + 4 * lq + i;
          float e = 0.f, wt = 0.f;
          if (!cur || sp <= t_me) {
            e = fexp(gct + base - s.gc[cur][sp]);
            wt = e * s.lam[t_me][(lv4 >> (8 * i)) & 0xff];
          }
          pb[4 * half + i] = (__bf16)(wt * dd[i]);
          mv[i] = e * sc[i] * dd[i];
        }
        *(floatx4*)(mrow + 64 * cur + 16 * st + 4 * lq) = mv;
      }
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        acc[kt] = mfma16x16x32(tr_frag_d(s.k[cur], kWLd, 32 * p, 16 * kt), pb, acc[kt]);
    }
  }

  // dq: far part, q . dq, store
  {
    float qd = 0.f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[kt][i] += fq[kt][i];
        qd += (float)qk4[kt][i] * acc[kt][i];
      }
      *(bf16x4*)(dq + rme + 16 * kt + 4 * lq) = cvt4(acc[kt]);
    }
    qd += __shfl_xor(qd, 16, 64);
    qd += __shfl_xor(qd, 32, 64);
    if (lq == 0) ws.qdq[(size_t)row * T + (size_t)n * kSC + t_me] = qd;
  }
  __syncthreads();

  // dlambda row of every target: levels 0 .. 7 from their source ranges, far
  // levels from the four slice partials, zero above
  {
    const int t = t_dl;
    float* dlrow = dl + ((tok0 + t) * H + h) * L;
    const float* mr = s.m + t * kMLd;
#pragma unroll
    for (int l = l0; l < kSLocLev; l += 4) {
      const int lo = kStrongR.lo[t][l], hi = kStrongR.hi[t][l];
      float x = 0.f;
#pragma unroll 8
      for (int i = lo; i < hi; ++i) x += mr[i];
      if (l < L) dlrow[l] = x;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (l0 + 4 * u < nf) dlrow[kSLocLev + l0 + 4 * u] = dlp[u][0] + dlp[u][1] + dlp[u][2] + dlp[u][3];
    for (int c = kSLocLev + nf + l0; c < L; c += 4) dlrow[c] = 0.f;
  }
}

// ---------------------------------------------------------------------------
// diagonal / sub-diagonal blocks: dk, dv and dg (source chunk n)
// ---------------------------------------------------------------------------
struct LocKVSmem {
  __bf16 q[2][kSC * kWLd];     // Q of chunks n (0) and n + 1 (1) [t][k]
  __bf16 d[2][kSC * kWLd];     // dO of chunks n, n + 1 [t][v]
  __bf16 adj[kSC * kWLd];      // d kv_n [k][v]
  float gc[2][kSC];
  float lam[2][kSC][kSLocLev];
  unsigned char tab[2][kSC * kSC];
  float dG[kSC];
};

// One workgroup per (row, source chunk n).  Wave w owns the sources s = 16 w ..
// +15; products with the lane on one source:
//   S = Q K^T, D = dO V^T over the targets of chunk n (t >= s) and n + 1,
//   dk^T[k][s] = sum_t Q^T[k][t] (W o D)[t][s], dv^T[v][s] = sum_t dO^T[v][t] (W o S)[t][s],
//   plus e^{Gc_last - Gc_s} (d kv_n v_s, d kv_n^T k_s).
template <typename TL>
__global__ __launch_bounds__(256, 2) void mamba2_strong_bwd_dkv_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const __bf16* __restrict__ dO, const float* __restrict__ gc, const TL* __restrict__ l,
    __bf16* __restrict__ dk, __bf16* __restrict__ dv, float* __restrict__ dg, StrongBwdWs ws,
    int rows, int T, int H, int L) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  LocKVSmem& s = *(LocKVSmem*)smem_raw;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int NT = T / kSC;
  const XcdMap mp = xcd_map(blockIdx.x, NT);
  if (mp.row >= rows) return;
  const int row = mp.row, n = mp.slice;
  const int b = row / H, h = row % H;
  const size_t tok0 = (size_t)b * T + (size_t)n * kSC;
  const size_t hd = (size_t)H * 64, hoff = (size_t)h * 64;
  const int s_me = 16 * w + ln;
  const bool has_next = n + 1 < NT;

  {
    const int r = tid >> 2, c16 = 16 * (tid & 3);
#pragma unroll
    for (int cur = 0; cur < 2; ++cur) {
      if (cur == 1 && !has_next) continue;
      const size_t off = (tok0 + (cur ? kSC : 0) + r) * hd + hoff + c16;
      const u32x4 q0 = *(const u32x4*)(q + off), q1 = *(const u32x4*)(q + off + 8);
      const u32x4 d0 = *(const u32x4*)(dO + off), d1 = *(const u32x4*)(dO + off + 8);
      *(u32x4*)(s.q[cur] + r * kWLd + c16) = q0;
      *(u32x4*)(s.q[cur] + r * kWLd + c16 + 8) = q1;
      *(u32x4*)(s.d[cur] + r * kWLd + c16) = d0;
      *(u32x4*)(s.d[cur] + r * kWLd + c16 + 8) = d1;
    }
    const __bf16* ap = ws.adj + ((size_t)row * NT + n) * 64 * 64 + r * 64 + c16;
    *(u32x4*)(s.adj + r * kWLd + c16) = *(const u32x4*)ap;
    *(u32x4*)(s.adj + r * kWLd + c16 + 8) = *(const u32x4*)(ap + 8);
    if (w == 0) {
      s.gc[0][lane] = gc[(tok0 + lane) * H + h];
      if (has_next) s.gc[1][lane] = gc[(tok0 + kSC + lane) * H + h];
    }
    for (int i = tid; i < 2 * kSC * kSLocLev; i += 256) {
      const int cur = i / (kSC * kSLocLev), t = (i / kSLocLev) % kSC, e = i % kSLocLev;
      if (cur == 1 && !has_next) continue;
      s.lam[cur][t][e] =
          e < L ? to_f32<TL>(l[((tok0 + (cur ? kSC : 0) + t) * H + h) * L + e]) : 0.f;
    }
    for (int i = tid; i < kSC * kSC / 4; i += 256) {
      ((unsigned*)s.tab[0])[i] = ((const unsigned*)kStrongB.intra)[i];
      ((unsigned*)s.tab[1])[i] = ((const unsigned*)kStrongB.sub)[i];
    }
  }
  // B operands of this wave's sources: K^T[k][s_me], V^T[v][s_me]
  const size_t rme = (tok0 + s_me) * hd + hoff;
  const bf16x8 bk0 = *(const bf16x8*)(k + rme + 8 * lq), bk1 = *(const bf16x8*)(k + rme + 32 + 8 * lq);
  const bf16x8 bv0 = *(const bf16x8*)(v + rme + 8 * lq), bv1 = *(const bf16x8*)(v + rme + 32 + 8 * lq);
  bf16x4 kk4[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) kk4[kt] = *(const bf16x4*)(k + rme + 16 * kt + 4 * lq);
  const float qdq_me = ws.qdq[(size_t)row * T + (size_t)n * kSC + s_me];
  __syncthreads();

  const float gcs = s.gc[0][s_me];
  floatx4 ak[4], av[4];   // dk^T[k = 16 kt + 4 lq + i][s_me], dv^T[v][s_me]
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) ak[kt] = av[kt] = zero4();
#pragma unroll
  for (int cur = 0; cur < 2; ++cur) {
    if (cur == 1 && !has_next) continue;
    const float base = cur ? s.gc[0][kSC - 1] : 0.f;
    const unsigned char* tab = s.tab[cur];
    // target tiles: chunk n from this wave's tile on (t >= s), chunk n + 1 all
    const int p0 = cur ? 0 : (w >> 1);
    for (int p = p0; p < 2; ++p) {
      bf16x8 pp, pd;   // (W o S)[t][s_me], (W o D)[t][s_me], t = 32 p + {4 lq + i, 16 + 4 lq + i}
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int tt = 2 * p + half;
        const __bf16* qr = s.q[cur] + (16 * tt + ln) * kWLd + 8 * lq;
        const __bf16* dr = s.d[cur] + (16 * tt + ln) * kWLd + 8 * lq;
        floatx4 sc = mfma16x16x32(*(const bf16x8*)qr, bk0, zero4());
        sc = mfma16x16x32(*(const bf16x8*)(qr + 32), bk1, sc);
        floatx4 dd = mfma16x16x32(*(const bf16x8*)dr, bv0, zero4());
        dd = mfma16x16x32(*(const bf16x8*)(dr + 32), bv1, dd);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tp = 16 * tt + 4 * lq + i;
          float wt = 0.f;
          if (cur || tp >= s_me)
            wt = fexp(s.gc[cur][tp] + base - gcs) * s.lam[cur][tp][tab[tp * kSC + s_me]];
          pp[4 * half + i] = (__bf16)(wt * sc[i]);
          pd[4 * half + i] = (__bf16)(wt * dd[i]);
        }
      }
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        ak[kt] = mfma16x16x32(tr_frag_d(s.q[cur], kWLd, 32 * p, 16 * kt), pd, ak[kt]);
        av[kt] = mfma16x16x32(tr_frag_d(s.d[cur], kWLd, 32 * p, 16 * kt), pp, av[kt]);
      }
    }
  }
  // far: e^{Gc_last - Gc_s} (d kv_n v_s, d kv_n^T k_s)
  {
    const float ws_ = fexp(s.gc[0][kSC - 1] - gcs);
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const __bf16* ar = s.adj + (16 * kt + ln) * kWLd + 8 * lq;
      floatx4 fk = mfma16x16x32(*(const bf16x8*)ar, bv0, zero4());
      fk = mfma16x16x32(*(const bf16x8*)(ar + 32), bv1, fk);
      floatx4 fv = mfma16x16x32(tr_frag(s.adj, kWLd, 0, 16 * kt), bk0, zero4());
      fv = mfma16x16x32(tr_frag(s.adj, kWLd, 32, 16 * kt), bk1, fv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ak[kt][i] += ws_ * fk[i];
        av[kt][i] += ws_ * fv[i];
      }
    }
  }
  // stores, k . dk, dG = q . dq - k . dk, chunk-local reverse cumsum
  {
    float kd = 0.f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) kd += (float)kk4[kt][i] * ak[kt][i];
      *(bf16x4*)(dk + rme + 16 * kt + 4 * lq) = cvt4(ak[kt]);
      *(bf16x4*)(dv + rme + 16 * kt + 4 * lq) = cvt4(av[kt]);
    }
    kd += __shfl_xor(kd, 16, 64);
    kd += __shfl_xor(kd, 32, 64);
    if (lq == 0) s.dG[s_me] = qdq_me - kd;
  }
  __syncthreads();
  if (w == 0) {
    float x = s.dG[lane];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float y = __shfl_down(x, d, 64);
      if (lane + d < 64) x += y;
    }
    dg[(tok0 + lane) * H + h] = x;
    if (lane == 0) ws.dgt[(size_t)row * NT + n] = x;
  }
}

// dg of chunk n += sum of the later chunks' dG totals (fixed-order sum).
__global__ __launch_bounds__(64) void mamba2_strong_bwd_dg_kernel(float* __restrict__ dg,
                                                                  const float* __restrict__ dgt,
                                                                  int rows, int T, int H) {
  const int lane = threadIdx.x;
  const int NT = T / kSC;
  const XcdMap mp = xcd_map(blockIdx.x, NT);
  if (mp.row >= rows) return;
  const int row = mp.row, n = mp.slice;
  const int b = row / H, h = row % H;
  float x = 0.f;
  for (int c = n + 1 + lane; c < NT; c += 64) x += dgt[(size_t)row * NT + c];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) x += __shfl_xor(x, d, 64);
  dg[((size_t)b * T + (size_t)n * kSC + lane) * H + h] += x;
}

template <typename TL>
static hipError_t strong_bwd_launch_t(const void* q, const void* k, const void* v,
                                      const float* gc, const void* l, const void* dO, void* dq,
                                      void* dk, void* dv, float* dg, float* dl, void* wsp, int B,
                                      int T, int H, int L, int nlev, hipStream_t stream) {
  const int rows = B * H, NT = T / kSC;
  const int nf = nlev > 1 ? nlev - 1 : 0;
  const StrongBwdWs ws = strong_bwd_ws_layout(wsp, B, T, H, nf);
  const int rpad = (rows + 7) / 8 * 8;
  hipError_t e;
  {
    auto kf = mamba2_strong_bwd_walk_kernel<TL>;
    const int smem = (int)sizeof(WalkSmem);
    if ((e = hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 smem)) != hipSuccess)
      return e;
    WalkArgs a{(const __bf16*)q, (const __bf16*)k, (const __bf16*)v, (const __bf16*)dO, gc, l,
               ws, rows, T, H, L, nf};
    const int half = rpad * 4;   // forward walks; then rpad * 2 reverse walks
    hipLaunchKernelGGL(kf, dim3(half + rpad * 2), dim3(kWThreads), smem, stream, a, half);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    auto kf = mamba2_strong_bwd_dq_kernel<TL>;
    const int smem = (int)sizeof(LocQSmem);
    if ((e = hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 smem)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(kf, dim3(rpad * NT), dim3(256), smem, stream, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, (const __bf16*)dO, gc, (const TL*)l,
                       (__bf16*)dq, dl, ws, rows, T, H, L, nf);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    auto kf = mamba2_strong_bwd_dkv_kernel<TL>;
    const int smem = (int)sizeof(LocKVSmem);
    if ((e = hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 smem)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(kf, dim3(rpad * NT), dim3(256), smem, stream, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, (const __bf16*)dO, gc, (const TL*)l,
                       (__bf16*)dk, (__bf16*)dv, dg, ws, rows, T, H, L);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (NT > 1) {
    hipLaunchKernelGGL(mamba2_strong_bwd_dg_kernel, dim3(rpad * NT), dim3(64), 0, stream, dg,
                       (const float*)ws.dgt, rows, T, H);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace hattn

size_t hattn_mamba2_strong_bwd_ws_bytes(int B, int T, int H, int nlev) {
  return hattn::strong_bwd_ws_layout(nullptr, B, T, H, nlev > 1 ? nlev - 1 : 0).bytes;
}

// bf16 q, k, v, dO (dq, dk, dv written in bf16); lambda bf16 or fp32; K = V = 64.
hipError_t hattn_mamba2_strong_bwd_launch(const void* q, const void* k, const void* v,
                                          const float* gc, const void* l, const void* dO,
                                          void* dq, void* dk, void* dv, float* dg, float* dl,
                                          void* ws, int B, int T, int H, int L, int nlev,
                                          int dt_l, hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  if (dt_l == 0)
    return strong_bwd_launch_t<__bf16>(q, k, v, gc, l, dO, dq, dk, dv, dg, dl, ws, B, T, H, L,
                                       nlev, stream);
  if (dt_l == 2)
    return strong_bwd_launch_t<float>(q, k, v, gc, l, dO, dq, dk, dv, dg, dl, ws, B, T, H, L,
                                      nlev, stream);
  *unsupported = 1;
  return hipSuccess;
}
