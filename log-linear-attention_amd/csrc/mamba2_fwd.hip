// Log-linear Mamba-2 chunkwise forward for gfx950, segment-parallel.
//
// Replaces the reference's 1 + 2 * nlev Triton launches (chunkwise.py:1118-1275:
// chunk_fwd_kernel_o with USE_A, then per inter-chunk level chunk_fwd_kernel_h
// and chunk_fwd_kernel_o) with two launches; the main one reads q, k, v, g and
// lambda once and writes o once.
//
// The sequence of NT 64-token chunks is cut into aligned segments of S = 2^s
// chunks, so a Fenwick block of 2^(e+1) <= S chunks never straddles a segment.
// Inter-chunk level e (absolute level 7 + e) is
//   * local (e < s): its blocks live inside one segment; the main kernel keeps
//     the state in fp32 registers while it walks the segment's chunks;
//   * top (e >= s): every chunk of segment p reads the same block of whole
//     earlier segments (bit e - s of p set), decayed to the chunk.  With scalar
//     per-token decay that state is exp(E_i) * Htop_e(p), where E_i is the
//     log-decay from the segment start to chunk i and
//         Htop_e(p) = sum_{q in block} exp(sum_{r=q+1}^{p-1} D_r) Sum(q),
//         Sum(q)    = sum_{t in q} exp(G_end(q) - G_t) k_t v_t^T,
//     with D_r the total log-decay of segment r.
//
// Kernel 1 (seg_sum) streams K, V, g and writes Sum(q) (fp32 [K, V]) and D_q
// per segment.  Kernel 2 (main) builds Htop for its segment from those
// summaries, then walks the segment's chunks.  One workgroup (4 waves) owns
// one (batch, head) row, one segment and one 64-wide block of V:
//   phase 1  the ten causal 16x16 tiles of S^T = K Q^T (three per wave, balanced)
//            on MFMA, scaled by exp(Gc_t - Gc_s) and lambda[t, bit_length(t ^ s)]
//            in registers, written as A = (S o M) in bf16 to LDS;
//   phase 2  wave w owns V columns 16w..16w+15 for all 64 tokens: o = A V plus,
//            for every level the chunk reads, lambda[t, 7 + e] exp(Gc_t) q_t h_e;
//   phase 3  wave w updates the local-level states for its V columns with the
//            chunk's decayed K^T V, computed once for all levels (the reference
//            recomputes it once per level, chunkwise.py:256-266).
// The level states stay in registers in the MFMA D layout; read as B operands
// they pair row k = 32c + 4lq + i / 32c + 16 + 4lq + i with the same k order in
// the Q fragments (any bijection of the contraction index works if both
// operands use it).  K^T and V fragments of the contractions over t come from
// row-major LDS tiles through the transposing LDS read.
#include <atomic>
#include <mutex>

#include "mamba2_common.h"

namespace hattn {

// ---------------------------------------------------------------------------
// Kernel 2: main pass over one segment, one 64-wide block of V
// ---------------------------------------------------------------------------
// NP bf16 planes per operand: 1 (bf16 inputs, bf16 MFMA) or 2 (fp32 inputs as
// bf16x3 hi / lo planes, three MFMAs per product).  MAXLOC local levels live in
// registers.  LDS: one chunk stage (single-buffered; the next chunk waits in
// registers), the A tile, and the top-level states ([level][plane][k][v]).
template <int NP, int MAXLOC>
struct Stage {
  static constexpr int LU = 7 + MAXLOC + kMaxTop;  // lambda columns (levels 0 .. 6 + nlev)
  __bf16 q[NP][kBT * kLd];
  __bf16 k[NP][kBT * kLd];
  __bf16 v[NP][kBT * kLd];
  float gc[kBT];            // chunk-local inclusive cumsum of g
  float wt[kBT];            // exp(Gc_last - Gc_t)
  float lam[LU * kBT];      // lambda^T [level][t]; levels >= 7 pre-multiplied by exp(Gc_t)
};

template <int NP, int MAXLOC>
struct MainSmem {
  Stage<NP, MAXLOC> st;
  __bf16 a[NP][kBT * kLd];  // A[t][s] = (S o M)[t][s] of the current chunk
  __bf16 top[1];            // [ntop][NP][kKD][kLd] top-level states (dynamic size)
};

template <int NP, int MAXLOC>
inline int main_smem_bytes(int ntop) {
  using Smem = MainSmem<NP, MAXLOC>;
  return (int)offsetof(Smem, top) + ntop * NP * kKD * kLd * 2;
}

template <typename TK, typename TV, typename TL, int LR>
struct MainRegs {
  Tile64<TK> q, k;
  Tile64<TV> v;
  float g;
  TL lam[LR];
};

// Phase-1 tile schedule: the 10 causal 16x16 tiles (t-tile mt, s-tile j <= mt)
// and the two zero tiles the 32-wide s steps of A V read above the diagonal
// ((0,1), (2,3)), three per wave: code = mt * 4 + j, +16 marks a zero tile.
__device__ __forceinline__ int p1_tile(int w, int n) {
  constexpr int tab[4][3] = {{0, 10, 14}, {5, 12, 16 + 1}, {4, 8, 15}, {9, 13, 16 + 11}};
  return tab[w][n];
}

template <typename TK, typename TV, typename TL, typename TO, int NP, int MAXLOC>
__global__ __launch_bounds__(256, NP == 1 ? 2 : 1) void mamba2_fwd_main_kernel(
    const TK* __restrict__ q, const TK* __restrict__ k, const TV* __restrict__ v,
    const float* __restrict__ g, const TL* __restrict__ l, TO* __restrict__ o,
    float* __restrict__ gcum, float* __restrict__ ht, const float* __restrict__ sums,
    const float* __restrict__ segd, const __bf16* __restrict__ htop, int B, int T, int G, int H,
    int V, int L, int nlev, int nvb64, int slog, int NSEG, int final_state) {
  using Smem = MainSmem<NP, MAXLOC>;
  constexpr int kPl = kKD * kLd;                         // one bf16 plane of a 64 x 64 tile
  constexpr int kLR = (Stage<NP, MAXLOC>::LU + 3) / 4;   // lambda registers per thread
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Smem& sm = *(Smem*)smem_raw;
  Stage<NP, MAXLOC>& s = sm.st;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  // grid: xcd_head_grid(B * NSEG, H, nvb64): the heads (and V slices) of one
  // (batch, segment) run together on one XCD and share its L2
  const XcdHeadMap xm = xcd_head_map(blockIdx.x, H, nvb64);
  if (xm.grp >= B * NSEG) return;
  const int h = xm.h, p = xm.grp % NSEG, b = xm.grp / NSEG;
  const int row = b * H + h, vblk = xm.slice;
  const int gq = h / (H / G);
  const int NT = T / kBT;
  const int c0 = p << slog;
  const int cend = min(c0 + (1 << slog), NT);
  const int lu = 7 + nlev;
  const int nloc = min(slog, nlev);
  const int ntop = nlev - nloc;
  const int vcol0 = vblk * 64;
  const int vc = vcol0 + 16 * w + ln;   // this lane's V column in phases 2 and 3
  const bool is_final_seg = final_state && ht != nullptr && p == NSEG - 1;
  float* htb = ht ? ht + ((size_t)b * H + h) * kKD * V * L : nullptr;

  // ---- top levels: Htop_e(p) (from the scan kernel) -> LDS ---------------------
  if (ntop > 0) {
    const __bf16* hsrc = htop + (((size_t)row * NSEG + p) * ntop * nvb64 + vblk) * NP * (kKD * 64);
    for (int e2 = 0; e2 < ntop; ++e2) {
      if (!((p >> e2) & 1)) continue;
#pragma unroll
      for (int pl = 0; pl < NP; ++pl) {
        const __bf16* src = hsrc + ((size_t)e2 * nvb64 * NP + pl) * (kKD * 64);
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          const int u = tid + 256 * rr, r = u >> 3, c = 8 * (u & 7);
          *(uint4*)(sm.top + (e2 * NP + pl) * kPl + r * kLd + c) = *(const uint4*)(src + r * 64 + c);
        }
      }
    }
  }
  if (ntop > 0 && is_final_seg) {
    // final states of the top levels (chunkwise.py:229-279): a level the last
    // chunk reads holds its block decayed over segment p; one it writes holds
    // segments [lo, p] decayed to the end of p.  P[q] = sum_{r < q} D_r in LDS
    // (the A tile is free until the first chunk).
    float* pre = (float*)sm.a[0];
    const float* dp = segd + (size_t)row * NSEG;
    if (w == 0) {
      float carry = 0.f;
      for (int base = 0; base <= p + 1; base += 64) {
        const int q = base + lane;
        const float x = q <= p ? dp[q] : 0.f;
        float y = x;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const float z = __shfl_up(y, d, 64);
          if (lane >= d) y += z;
        }
        if (q <= p + 1) pre[q] = carry + y - x;
        carry += __shfl(y, 63, 64);
      }
    }
    __syncthreads();
    const float* sp = sums + (size_t)row * NSEG * kKD * V + vc;
    const size_t qstride = (size_t)kKD * V;
    for (int e2 = 0; e2 < ntop; ++e2) {
      const bool reads = (p >> e2) & 1;
      const int lo = reads ? (p >> (e2 + 1)) << (e2 + 1) : (p >> e2) << e2;
      const int hi = reads ? lo + (1 << e2) : p + 1;
      floatx4 hacc[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) hacc[m] = zero4();
      for (int qs = lo; qs < hi; ++qs) {
        const float sc = fexp(pre[p + 1] - pre[qs + 1]);
        const float* src = sp + qs * qstride;
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i) hacc[m][i] += sc * src[(size_t)(16 * m + 4 * lq + i) * V];
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          htb[((size_t)(16 * m + 4 * lq + i) * V + vc) * L + 7 + nloc + e2] = hacc[m][i];
    }
  }

  // ---- per-row buffer descriptors and per-lane offsets ---------------------------
  // Chunk j of the segment starts (c0 + j) * 64 rows into the row's span; that
  // offset is uniform (SGPR), the lane's part of each access pattern is fixed.
  const int qstr = G * kKD, vstr = H * V, lstr = H * L;
  const rsrc_t rq = make_rsrc(q + ((size_t)b * T * G + gq) * kKD, (size_t)T * qstr * sizeof(TK));
  const rsrc_t rk = make_rsrc(k + ((size_t)b * T * G + gq) * kKD, (size_t)T * qstr * sizeof(TK));
  const rsrc_t rv = make_rsrc(v + ((size_t)b * T * H + h) * V + vcol0, (size_t)T * vstr * sizeof(TV));
  const rsrc_t rg_ = make_rsrc(g + (size_t)b * T * H + h, (size_t)T * H * 4);
  const rsrc_t rl = make_rsrc(l + ((size_t)b * T * H + h) * L, (size_t)T * lstr * sizeof(TL));
  const rsrc_t ro = make_rsrc(o + ((size_t)b * T * H + h) * V + vcol0, (size_t)T * vstr * sizeof(TO));
  const bool write_gcum = gcum != nullptr && vblk == 0;
  const rsrc_t rgc = make_rsrc(write_gcum ? (const void*)(gcum + (size_t)b * T * H + h) : (const void*)g,
                               write_gcum ? (size_t)T * H * 4 : 0);
  const unsigned int vo_qk = tile64_voff<TK>(qstr), vo_v = tile64_voff<TV>(vstr);
  const unsigned int vo_g = lane * H * 4;
  // lambda tile: thread -> row tid >> 2, columns (tid & 3) + 4r
  const int lrow = tid >> 2, lcol = tid & 3;
  const unsigned int vo_l = (lrow * lstr + lcol) * sizeof(TL);
  const unsigned int vo_o = (4 * lq * vstr + 16 * w + ln) * sizeof(TO);

  MainRegs<TK, TV, TL, kLR> rg;
  auto load = [&](int j) {  // j: chunk index within the segment
    const unsigned int row0 = (unsigned int)(c0 + j) * kBT;
    load_tile64(rg.q, rq, vo_qk, row0 * qstr * sizeof(TK), qstr);
    load_tile64(rg.k, rk, vo_qk, row0 * qstr * sizeof(TK), qstr);
    load_tile64(rg.v, rv, vo_v, row0 * vstr * sizeof(TV), vstr);
    rg.g = buf_load<float>(rg_, vo_g, row0 * H * 4);
    const unsigned int so_l = row0 * lstr * sizeof(TL);
#pragma unroll
    for (int r = 0; r < kLR; ++r)
      if (lcol + 4 * r < lu) rg.lam[r] = buf_load<TL>(rl, vo_l, so_l + 4 * r * sizeof(TL));
  };
  auto store = [&](int j) {
    store_tile64<NP>(rg.q, s.q[0], s.q[NP - 1]);
    store_tile64<NP>(rg.k, s.k[0], s.k[NP - 1]);
    store_tile64<NP>(rg.v, s.v[0], s.v[NP - 1]);
    const float x = chunk_cumsum(rg.g);   // every wave scans the chunk's g
    const float last = __shfl(x, 63, 64);
    if (w == 0) {
      s.gc[lane] = x;
      s.wt[lane] = fexp(last - x);
      if (write_gcum) buf_store<float>(x, rgc, vo_g, (unsigned int)(c0 + j) * kBT * H * 4);
    }
    const float eg = fexp(__shfl(x, lrow, 64));
#pragma unroll
    for (int r = 0; r < kLR; ++r) {
      const int col = lcol + 4 * r;
      if (col < lu) {
        float val = to_f32<TL>(rg.lam[r]);
        if (col >= 7) val *= eg;
        s.lam[col * kBT + lrow] = val;
      }
    }
  };

  floatx4 st[MAXLOC][4];
#pragma unroll
  for (int e = 0; e < MAXLOC; ++e)
#pragma unroll
    for (int m = 0; m < 4; ++m) st[e][m] = zero4();

  const int nch = cend - c0;
  load(0);
  float Eseg = 0.f;  // log-decay from the segment start to the current chunk start
  for (int j = 0; j < nch; ++j) {
    const int ic = c0 + j;
    store(j);
    if (j + 1 < nch) load(j + 1);
    __syncthreads();

    // ---- phase 1: three tiles of A[t][s] per wave ------------------------------
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      const int code = p1_tile(w, n);
      const int mt = (code & 15) >> 2, jt = code & 3;
      const int t = 16 * mt + ln;
      float out[4] = {0.f, 0.f, 0.f, 0.f};
      if (code < 16) {
        floatx4 acc = zero4();
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          bf16x8 a[NP], bq[NP];
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) {
            a[pl] = *(const bf16x8*)(s.k[pl] + (16 * jt + ln) * kLd + 32 * c + 8 * lq);
            bq[pl] = *(const bf16x8*)(s.q[pl] + t * kLd + 32 * c + 8 * lq);
          }
          acc = mma<NP>(a, bq, acc);  // S^T[s = 16jt + 4lq + i][t]
        }
        const float gct = s.gc[t];
        const floatx4 gs = *(const floatx4*)(s.gc + 16 * jt + 4 * lq);
        if (jt < mt) {
          // off-diagonal tile: level 4 + bit_length(mt ^ jt) for every pair
          const float lam = s.lam[(4 + intra_level(mt, jt)) * kBT + t];
#pragma unroll
          for (int i = 0; i < 4; ++i) out[i] = acc[i] * fexp(gct - gs[i]) * lam;
        } else {
          // diagonal tile: level bit_length(ln ^ (4lq + i)), causal s <= t
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int sl = 4 * lq + i;
            const float val = acc[i] * fexp(gct - gs[i]) * s.lam[intra_level(ln, sl) * kBT + t];
            out[i] = sl <= ln ? val : 0.f;
          }
        }
      }
      bf16x4 ohi, olo;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ohi[i] = (__bf16)out[i];
        if constexpr (NP == 2) olo[i] = bf16_lo(out[i], ohi[i]);
      }
      *(bf16x4*)(sm.a[0] + t * kLd + 16 * jt + 4 * lq) = ohi;
      if constexpr (NP == 2) *(bf16x4*)(sm.a[1] + t * kLd + 16 * jt + 4 * lq) = olo;
    }
    __syncthreads();

    // ---- phase 2: o[all t][V columns 16w..] ------------------------------------
    floatx4 acc[4];
    {
      bf16x8 vf0[NP], vf1[NP];   // V[s][v], s = 0..31 / 32..63
#pragma unroll
      for (int pl = 0; pl < NP; ++pl) {
        vf0[pl] = tr_frag(s.v[pl], kLd, 0, 16 * w);
        vf1[pl] = tr_frag(s.v[pl], kLd, 32, 16 * w);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        bf16x8 af[NP];
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) af[pl] = *(const bf16x8*)(sm.a[pl] + (16 * mt + ln) * kLd + 8 * lq);
        acc[mt] = mma<NP>(af, vf0, zero4());
        if (mt >= 2) {
#pragma unroll
          for (int pl = 0; pl < NP; ++pl)
            af[pl] = *(const bf16x8*)(sm.a[pl] + (16 * mt + ln) * kLd + 32 + 8 * lq);
          acc[mt] = mma<NP>(af, vf1, acc[mt]);
        }
      }
    }
    const bool any_loc = nloc > 0 && j > 0;
    const bool any_top = ntop > 0 && p > 0;
    if (any_loc || any_top) {
      const float ee = fexp(Eseg);
      // Q fragments in the states' row order: k = 32c + 4lq + i, 32c + 16 + 4lq + i
      bf16x8 qa[4][2][NP];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) {
            const __bf16* qp = s.q[pl] + (16 * mt + ln) * kLd + 32 * c + 4 * lq;
            const bf16x4 lo = *(const bf16x4*)qp;
            const bf16x4 hi = *(const bf16x4*)(qp + 16);
            qa[mt][c][pl] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          }
      const float* lamt = s.lam + 4 * lq;
      // only the local levels the chunk reads (bit e of the chunk index; a
      // uniform branch): with three MFMAs per product the skipped half of the
      // level products is the larger cost, not the lost interleaving
#pragma unroll
      for (int e = 0; e < MAXLOC; ++e) {
        if (any_loc && e < nloc && ((ic >> e) & 1)) {
          bf16x8 b0[NP], b1[NP];
          cat8s<NP>(st[e][0], st[e][1], b0);
          cat8s<NP>(st[e][2], st[e][3], b1);
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            floatx4 tmp = mma<NP>(qa[mt][0], b0, zero4());
            tmp = mma<NP>(qa[mt][1], b1, tmp);
            const floatx4 lam = *(const floatx4*)(lamt + (7 + e) * kBT + 16 * mt);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mt][i] += tmp[i] * lam[i];
          }
        }
      }
      if (any_top) {
        for (int e2 = 0; e2 < ntop; ++e2) {
          if ((p >> e2) & 1) {
            const __bf16* tp = sm.top + e2 * NP * kPl;
            bf16x8 b0[NP], b1[NP];
#pragma unroll
            for (int pl = 0; pl < NP; ++pl) {
              b0[pl] = tr_frag_d(tp + pl * kPl, kLd, 0, 16 * w);
              b1[pl] = tr_frag_d(tp + pl * kPl, kLd, 32, 16 * w);
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
              floatx4 tmp = mma<NP>(qa[mt][0], b0, zero4());
              tmp = mma<NP>(qa[mt][1], b1, tmp);
              const floatx4 lam = *(const floatx4*)(lamt + (7 + nloc + e2) * kBT + 16 * mt);
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[mt][i] += tmp[i] * (lam[i] * ee);
            }
          }
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        buf_store<TO>(from_f32<TO>(acc[mt][i]), ro, vo_o,
                      ((unsigned int)ic * kBT + 16 * mt + i) * vstr * sizeof(TO));

    // ---- phase 3: local state update for V columns 16w.. -----------------------
    const float glr = s.gc[kBT - 1];
    if (nloc > 0) {
      const floatx4 w0a = *(const floatx4*)(s.wt + 8 * lq);
      const floatx4 w0b = *(const floatx4*)(s.wt + 8 * lq + 4);
      const floatx4 w1a = *(const floatx4*)(s.wt + 32 + 8 * lq);
      const floatx4 w1b = *(const floatx4*)(s.wt + 32 + 8 * lq + 4);
      // (w o V)[s][v] for s = 0..31 / 32..63
      const bf16x8 vh0 = tr_frag(s.v[0], kLd, 0, 16 * w), vh1 = tr_frag(s.v[0], kLd, 32, 16 * w);
      bf16x8 vl0{}, vl1{};
      if constexpr (NP == 2) {
        vl0 = tr_frag(s.v[1], kLd, 0, 16 * w);
        vl1 = tr_frag(s.v[1], kLd, 32, 16 * w);
      }
      float x0[8], x1[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x0[i] = ((float)vh0[i] + (float)vl0[i]) * w0a[i];
        x0[4 + i] = ((float)vh0[4 + i] + (float)vl0[4 + i]) * w0b[i];
        x1[i] = ((float)vh1[i] + (float)vl1[i]) * w1a[i];
        x1[4 + i] = ((float)vh1[4 + i] + (float)vl1[4 + i]) * w1b[i];
      }
      bf16x8 wv0[NP], wv1[NP];
      split8<NP>(x0, wv0);
      split8<NP>(x1, wv1);
      floatx4 kv[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        bf16x8 kf[NP];
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) kf[pl] = tr_frag(s.k[pl], kLd, 0, 16 * m);
        kv[m] = mma<NP>(kf, wv0, zero4());
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) kf[pl] = tr_frag(s.k[pl], kLd, 32, 16 * m);
        kv[m] = mma<NP>(kf, wv1, kv[m]);
      }
      const float gl = fexp(glr);
      const bool last = (ic == NT - 1);
#pragma unroll
      for (int e = 0; e < MAXLOC; ++e) {
        if (e < nloc) {
          const int per = 2 << e;
          const bool reset = ((ic & (per - 1)) == per - 1) && !(last && final_state);
          const bool write_kv = !((ic >> e) & 1);
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            if (reset) {
              st[e][m] = write_kv ? kv[m] : zero4();
            } else if (write_kv) {
#pragma unroll
              for (int i = 0; i < 4; ++i) st[e][m][i] = st[e][m][i] * gl + kv[m][i];
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) st[e][m][i] *= gl;
            }
          }
        }
      }
      if (last && is_final_seg) {
        // ht[b, h, k, v, 7 + e] (chunkwise.py:1179, 277-279)
#pragma unroll
        for (int e = 0; e < MAXLOC; ++e)
          if (e < nloc)
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                htb[((size_t)(16 * m + 4 * lq + i) * V + vc) * L + 7 + e] = st[e][m][i];
      }
    }
    Eseg += glr;
    __syncthreads();   // every wave is done with the stage before it is refilled
  }
}

// ---------------------------------------------------------------------------
// Kernel 2 (bf16 inputs): main pass, output computed transposed
// ---------------------------------------------------------------------------
// Same segment walk and the same three phases as mamba2_fwd_main_kernel, laid
// out so that a wave issues as few instructions per chunk as possible:
//   * every product of phase 2 is computed as o^T (rows v, columns t), so the
//     lambda weight of a level is one scalar per lane and tile, and a lane
//     stores 4 consecutive v of one token (one 8-byte store per t-tile);
//   * the Q fragments are read from LDS once per chunk and serve both as the
//     B operand of S^T = K Q^T (phase 1) and of o^T += h^T Q^T (phase 2);
//   * the level states are produced by phase 3 with the contraction index in
//     natural order (k = 32c + 8lq + j), by pointing the transposing LDS reads
//     of K^T at column blocks 32c + 8(lane & 3) + 4h; so states, Q and the
//     top-level states (stored [v][k]) all pair by plain 16-byte fragments;
//   * only the levels a chunk reads are computed (uniform branches);
//   * a local state carries a pending log-decay instead of being rescaled
//     every chunk: h_e = st_e * 2^dl_e, rescaled only when it is written.
// LDS holds the chunk stage (single-buffered; the next chunk waits in
// registers), the A tile, lambda and decay vectors and the top-level states.
//
// The four 64 x 64 bf16 tiles have unpadded 128-byte rows whose 16-byte units
// are permuted per row: element (r, c) sits in unit (c >> 3) ^ f(r), with one
// XOR map f per tile chosen for that tile's accesses (gfx950 LDS: 64 banks for
// reads, serving 16-byte reads 16 lanes (two 8-lane row groups) at a time and
// 8-byte transposing reads 32 lanes at a time; 32 banks for writes):
//   Q, K  f = bits 1, 2 of r, and bit 3 onto unit bit 2: row-fragment reads
//         (16 rows x 2 units per 16 lanes) and the transposing K^T reads (rows
//         r0 + 8lq + (ln >> 2)) each take the minimum number of LDS cycles;
//   V     f = bit 1 of r, and bit 3 onto unit bit 2: conflict-free transposing reads;
//   A     f = bits 1, 2 of r, and bit 3 onto unit bit 0: conflict-free
//         row-fragment reads; the 8-byte writes of the MFMA D layout two-way.
// Staging writes (one row of 8 units per 8 lanes) are conflict-free for all.
// lambda columns a staging wave may write per token row: three 16-byte bf16
// pieces (or six fp32 pieces) cover 24 columns, plus one for a misaligned row
constexpr int kLamCols = 25;
static_assert(kMaxLU + 1 < kLamCols, "lambda pieces cover every level");

// LT: element type of the staged lambda values: fp32, or for bf16 lambda
// inputs bf16 (exact; half the LDS of the double-buffered staging), used where
// that lets two workgroups share a CU (five top levels, T >= 32768).
template <typename LT>
struct Bf16Smem {
  __bf16 q[kBT * 64];         // Q[t][k]
  __bf16 k[kBT * 64];         // K[s][k]
  __bf16 v[kBT * 64];         // V[s][v] (this workgroup's 64 columns)
  __bf16 a[kBT * 64];         // A[t][s] = (S o M)[t][s]
  float gc[kBT];              // log2(e) * chunk-local inclusive cumsum of g
  float wt[kBT];              // exp(Gc_last - Gc_s)
  // lambda[t = 16nt + ln][lev] at row lev + 1, column 4ln + nt, and exp(Gc_t)
  // at [4ln + nt], double-buffered: chunk j + 1's are staged while chunk j's
  // are read.  A staging lane writes all the values of its 16-byte lambda
  // pieces, columns -1 .. kLamCols - 2 of its token row (the row's misalignment
  // shifts them by one), to rows 0 .. kLamCols - 1: a value's row is a
  // compile-time offset from a per-lane base, and the rows outside 1 .. lu hold
  // values nobody reads (the neighbouring head's lambda or zeros)
  LT lam[2][kLamCols * kBT];
  float eg[2][kBT];
  float lpar[32];             // layer mode: L[h, 0 .. L - 1] (lambda parameters of the head)
  __bf16 top[1];              // [ntop][v][64] top-level states, transposed, swizzled
};

template <typename LT>
inline int bf16_smem_bytes(int ntop) {
  return (int)offsetof(Bf16Smem<LT>, top) + ntop * kKD * 64 * 2;
}

// LDS of one CU (two workgroups of the bf16 kernel per CU need at most half each)
constexpr int kLdsPerCu = 160 * 1024;

// four consecutive staged lambda values as fp32
__device__ __forceinline__ floatx4 lam4(const float* p) { return *(const floatx4*)p; }
__device__ __forceinline__ floatx4 lam4(const __bf16* p) {
  const bf16x4 x = *(const bf16x4*)p;
  return floatx4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
}

// Top-level state element (v, k) in a 64 x 64 bf16 tile without padding: the
// 16-byte unit k >> 3 of row v is stored at unit (k >> 3) ^ (v & 7), so the
// 16-byte fragment reads of eight consecutive rows hit eight different units.
__device__ __forceinline__ int top_idx(int v, int k) {
  return v * 64 + ((((k >> 3) ^ v) & 7) << 3) + (k & 7);
}

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int swz_qk(int r) { return (r & 6) ^ ((r >> 1) & 4); }
__device__ __forceinline__ int swz_v(int r) { return (r & 2) ^ ((r >> 1) & 4); }
__device__ __forceinline__ int swz_a(int r) { return (r & 6) ^ ((r >> 3) & 1); }
// element offset of (r, c) in a swizzled tile
template <int (*F)(int)>
__device__ __forceinline__ int sidx(int r, int c) {
  return r * 64 + ((((c >> 3) ^ F(r)) & 7) << 3) + (c & 7);
}

// Stage a 64 x 64 tile held in registers (Tile64 layout) into a swizzled
// bf16 tile: bf16 data as 16-byte units, fp32 data converted to 8-byte halves.
template <int (*F)(int), typename T, typename E = __bf16>
__device__ __forceinline__ void store_tile_swz(const Tile64<T>& t, __bf16* dst) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int rr = 0; rr < Tile64<T>::N; ++rr) {
    if constexpr (sizeof(T) == 2) {
      const int r = (tid >> 3) + 32 * rr;
      *(uint4*)(dst + sidx<F>(r, 8 * (tid & 7))) = t.r[rr];
    } else {
      const int r = (tid >> 4) + 16 * rr;
      const float* e = (const float*)&t.r[rr];
      *(bf16x4*)(dst + sidx<F>(r, 4 * (tid & 15))) =
          cvt4e<E>(floatx4{e[0], e[1], e[2], e[3]});
    }
  }
}

constexpr float kLog2e = 1.4426950408889634f;

// K^T fragment with the contraction over s: lane (lq, ln) receives
// K[s = r0 + 8lq + j][k = 32c + 8(ln >> 2) + 4h + (ln & 3)], j = 0..7, so the D
// rows 4lq + i of the product are k = 32c + 8lq + 4h + i.
// Per-lane element offsets of one chunk's swizzled LDS accesses.  The XOR term
// of every pattern depends on the lane only (tile and row-block steps change
// row bits that no swizzle map reads), so each pattern needs one or two
// per-lane bases and its steps become immediate offsets.
struct LdsBase {
  int rq0, rq1;   // Q / K rows 16m + ln, columns 8lq (+0 / +32); +1024 per 16-row tile
  int ra0, ra1;   // A rows 16m + ln, columns 8lq (+0 / +32)
  int aw, awu;    // A writes: row ln, half lq & 1; unit (2jt + (lq >> 1)) ^ f = awu ^ 2jt
  int kt0, kt1;   // K^T reads (rows 8lq + (ln >> 2)): k-half 0 / 1; rows + 4 swap the bases
  int vt;         // V reads (rows 8lq + (ln >> 2)), this wave's 16 columns
};

__device__ __forceinline__ LdsBase lds_base(int lq, int ln, int w) {
  LdsBase b;
  const int uq = lq ^ swz_qk(ln);
  b.rq0 = ln * 64 + (uq << 3);
  b.rq1 = ln * 64 + ((uq ^ 4) << 3);
  const int fa = swz_a(ln);
  const int ua = lq ^ fa;
  b.ra0 = ln * 64 + (ua << 3);
  b.ra1 = ln * 64 + ((ua ^ 4) << 3);
  b.awu = (lq >> 1) ^ fa;
  b.aw = ln * 64 + 4 * (lq & 1);
  const int rk = 8 * lq + (ln >> 2);
  const int uk = (ln & 3) ^ swz_qk(rk);
  b.kt0 = rk * 64 + (uk << 3);
  b.kt1 = rk * 64 + ((uk ^ 4) << 3);
  b.vt = rk * 64 + (((((ln & 3) >> 1) ^ swz_v(rk)) ^ (2 * w)) << 3) + 4 * (ln & 1);
  return b;
}

// K^T fragment: lane (lq, ln) receives K[s = r0 + 8lq + j][k = 32c + 8(ln >> 2) + 4h + (ln & 3)]
// (row r + 4 flips unit bit 2 under swz_qk, which swaps the two k-half bases).
__device__ __forceinline__ bf16x8 ktr_frag(const __bf16* X, const LdsBase& b, int r0, int c, int h) {
  const int lo_off = (c ? b.kt1 : b.kt0) + r0 * 64 + 4 * h;
  const int hi_off = (c ? b.kt0 : b.kt1) + (r0 + 4) * 64 + 4 * h;
  const bf16x4 lo = ds_read_tr(X + lo_off);
  const bf16x4 hi = ds_read_tr(X + hi_off);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// V fragment with the contraction over s: lane (lq, ln) receives
// V[s = r0 + 8lq + j][v = 16w + ln], j = 0..7.
__device__ __forceinline__ bf16x8 vtr_frag(const __bf16* X, const LdsBase& b, int r0) {
  const bf16x4 lo = ds_read_tr(X + b.vt + r0 * 64);
  const bf16x4 hi = ds_read_tr(X + b.vt + (r0 + 4) * 64);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Phase-1 schedule: the 10 causal tiles plus the two zero tiles the 32-wide s
// steps of A V read above the diagonal ((0,1), (2,3)), three per wave; tile n
// of wave W is (P1T<W>::mt[n], P1T<W>::jt[n]).  A diagonal tile (a lambda
// column per element) costs about twice an off-diagonal one (one lambda per
// row), so every wave takes one diagonal tile: waves 0, 1 two off-diagonal
// tiles, waves 2, 3 one (and a zero tile, skipped).
template <int W> struct P1T;
template <> struct P1T<0> { static constexpr int mt[3] = {0, 1, 2}, jt[3] = {0, 0, 0}; };
template <> struct P1T<1> { static constexpr int mt[3] = {1, 2, 3}, jt[3] = {1, 1, 0}; };
template <> struct P1T<2> { static constexpr int mt[3] = {2, 3, 0}, jt[3] = {2, 1, 1}; };
template <> struct P1T<3> { static constexpr int mt[3] = {3, 3, 2}, jt[3] = {3, 2, 3}; };

// Phase 1 of one wave plus the chunk's K^T diag(w) V for its V columns (which
// needs no level state, so it is computed here, where its LDS reads and MFMAs
// interleave with the tile work): every LDS read is issued first, then the
// MFMAs, then the scaling of the A tiles.
//   A tile (mt, jt): S^T[s = 16jt + 4lq + i][t = 16mt + ln] o exp(Gc_t - Gc_s)
//                    o lambda[t, level(t, s)] (causal) -> bf16 A[t][s] in LDS.
//   kv[2c + h]: D rows k = 32c + 8lq + 4h + i, column v = 16w + ln.
template <int W, typename LT, typename E = __bf16>
__device__ __forceinline__ void bf16_p1(Bf16Smem<LT>& sm, const LdsBase& lb, const LT* li,
                                        const bf16x8 (&qa)[4][2], const bf16x8& vt0,
                                        const bf16x8& vt1, floatx4 (&kv)[4], int lq, int ln) {
  using S = P1T<W>;
  // ---- LDS reads ----
  bf16x8 kf[3][2];
  float gt[3];
  floatx4 gs[3];
  float lam[3][4];
#pragma unroll
  for (int n = 0; n < 3; ++n) {
    const int mt = S::mt[n], jt = S::jt[n];
    if (jt > mt) continue;
    const int t = 16 * mt + ln;
#pragma unroll
    for (int c = 0; c < 2; ++c) kf[n][c] = *(const bf16x8*)(sm.k + (c ? lb.rq1 : lb.rq0) + 1024 * jt);
    gt[n] = sm.gc[t];
    gs[n] = *(const floatx4*)(sm.gc + 16 * jt + 4 * lq);
    if (jt < mt) {
      const int lev = 4 + (32 - __builtin_clz(mt ^ jt));
      lam[n][0] = (float)li[lev * kBT + 4 * ln + mt];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) lam[n][i] = (float)li[intra_level(ln, 4 * lq + i) * kBT + 4 * ln + mt];
    }
  }
  bf16x8 kt[2][2];   // [h][s-half], first for k-half c = 0
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    kt[hh][0] = ktr_frag(sm.k, lb, 0, 0, hh);
    kt[hh][1] = ktr_frag(sm.k, lb, 32, 0, hh);
  }
  const floatx4 w0a = *(const floatx4*)(sm.wt + 8 * lq);
  const floatx4 w0b = *(const floatx4*)(sm.wt + 8 * lq + 4);
  const floatx4 w1a = *(const floatx4*)(sm.wt + 32 + 8 * lq);
  const floatx4 w1b = *(const floatx4*)(sm.wt + 32 + 8 * lq + 4);
  __builtin_amdgcn_sched_barrier(0);
  // ---- MFMAs ----
  floatx4 acc[3];
#pragma unroll
  for (int n = 0; n < 3; ++n) {
    const int mt = S::mt[n], jt = S::jt[n];
    if (jt > mt) continue;
    acc[n] = mfma16<E>(kf[n][0], qa[mt][0], zero4());
    acc[n] = mfma16<E>(kf[n][1], qa[mt][1], acc[n]);
  }
  bf16x8 wv0, wv1;   // (w o V)[s][v = 16w + ln], s = 8lq + j / 32 + 8lq + j
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wv0[i] = to16<E>(from16<E>(vt0[i]) * w0a[i]);
    wv0[4 + i] = to16<E>(from16<E>(vt0[4 + i]) * w0b[i]);
    wv1[i] = to16<E>(from16<E>(vt1[i]) * w1a[i]);
    wv1[4 + i] = to16<E>(from16<E>(vt1[4 + i]) * w1b[i]);
  }
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    kv[hh] = mfma16<E>(kt[hh][0], wv0, zero4());
    kv[hh] = mfma16<E>(kt[hh][1], wv1, kv[hh]);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    kt[hh][0] = ktr_frag(sm.k, lb, 0, 1, hh);
    kt[hh][1] = ktr_frag(sm.k, lb, 32, 1, hh);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    kv[2 + hh] = mfma16<E>(kt[hh][0], wv0, zero4());
    kv[2 + hh] = mfma16<E>(kt[hh][1], wv1, kv[2 + hh]);
  }
  // ---- scaling, A tiles -> LDS ----
#pragma unroll
  for (int n = 0; n < 3; ++n) {
    const int mt = S::mt[n], jt = S::jt[n];
    if (jt > mt) continue;   // the zero tiles are written once, before the walk
    const int t = 16 * mt + ln;
    bf16x4 out;
    if (jt < mt) {
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) val[i] = acc[n][i] * fexp2(gt[n] - gs[n][i]) * lam[n][0];
      out = cvt4e<E>(floatx4{val[0], val[1], val[2], val[3]});
    } else {
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = acc[n][i] * fexp2(gt[n] - gs[n][i]) * lam[n][i];
        val[i] = 4 * lq + i <= ln ? x : 0.f;
      }
      out = cvt4e<E>(floatx4{val[0], val[1], val[2], val[3]});
    }
    *(bf16x4*)(sm.a + lb.aw + 1024 * mt + ((lb.awu ^ (2 * jt)) << 3)) = out;
  }
}

// FUSED: one launch computes everything (single pass).  Work items (segment,
// batch, head, V block) are handed out by eight ticket counters, one per XCD
// (workgroup blockIdx.x goes to XCD blockIdx.x % 8): the groups g = p B + b
// (segment p of batch b) g = x, x + 8, x + 16, .. go to XCD x, in that order,
// each with all its heads and V blocks, so the cache lines of lambda and g
// that interleave the heads of a token row are fetched into one L2.  A
// workgroup only ever waits for a smaller group (an earlier segment of its
// batch); each XCD claims its groups in increasing order,
// so the smallest unfinished group is always claimed by running workgroups
// whose waits are all satisfied, and the launch cannot deadlock.
// Phase A streams the segment's K, V, g and publishes Sum(p) and D_p
// (coherent stores, then a flag); the workgroup then waits for the flags of
// the earlier segments of its row and builds its top-level states from their
// summaries (coherent loads).  The walk re-reads K and V shortly after phase A,
// from the L2 / memory-side cache.  Not FUSED: the summaries come from
// mamba2_seg_sum_kernel (or there is a single segment and none are needed).
//
// sync (zeroed by mamba2_fwd_sync_init_kernel before the launch): the ticket
// counter of XCD x at [16 x], the status word at [kSyncStatus], one flag per
// (row, V block, segment) from [kSyncHdr].  The look-back wait is bounded
// (spin_limit polls, ~1 s by default): a wait that gives up sets bit 0 of the
// status word and the workgroup writes NaN over its outputs (o, g_cumsum, its
// part of ht) instead of computing them, so a lost flag (or a call that
// overlaps another on the same workspace) shows as NaN, never as a hang or as
// plausible wrong numbers.
constexpr int kSpinLimit = 1 << 24;
constexpr int kSyncStatus = 128;
constexpr int kSyncHdr = 144;
constexpr unsigned int kStatusLookbackTimeout = 1u;

// Look-back controls: spin_limit polls before a wait gives up, and publish = 0
// suppresses the flags of phase A (every later wait then gives up): the test
// hook hattn_debug_lookback sets both to exercise the timeout path.
struct LookbackCtl {
  int spin_limit;
  int publish;
};

__global__ void mamba2_fwd_sync_init_kernel(unsigned int* __restrict__ sync, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) sync[i] = 0u;
}

// LAYER: the layer pre- / post-processing of hmamba_chunk_scan_combined
// (mamba_apis.py:346-403) folded into the loads and stores: v is the layer's x
// (v = x dt' as it is staged), l is dl (lambda = compute_lambda(L[h], dl) as it
// is staged), g comes from dt (g = A dt'), and the output is bf16(o) + x D[h]
// (see layer_math.h); bf16 x only.
template <typename TV, typename TL, typename TO, bool FUSED, bool LAYER = false, bool LAM16 = false,
          typename E = __bf16>
__global__ __launch_bounds__(256, 2) void mamba2_fwd_bf16_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const TV* __restrict__ v,
    const float* __restrict__ g, const TL* __restrict__ l, TO* __restrict__ o,
    float* __restrict__ gcum, float* __restrict__ ht, float* __restrict__ sums,
    float* __restrict__ segd, unsigned int* __restrict__ sync, int B, int T, int G, int H,
    int V, int L, int nlev, int nvb64, int slog, int NSEG, int final_state, LayerArgs la,
    LookbackCtl lbc) {
  static_assert(!LAYER || (sizeof(TV) == 2 && __is_same(E, __bf16)), "layer mode: bf16 x");
  constexpr int kPl = kKD * 64;                           // one top-level state tile
  constexpr int kLPS = (kMaxLoc + kMaxTop) * kBT;          // one lambda' buffer
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  static_assert(!LAM16 || (sizeof(TL) == 2 && !LAYER), "bf16 staging of bf16 lambda inputs");
  using LT = typename std::conditional<LAM16, __bf16, float>::type;
  Bf16Smem<LT>& sm = *(Bf16Smem<LT>*)smem_raw;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq0 = lane >> 4, ln0 = lane & 15;
  int h, p, b, vblk;
  __shared__ int lb_fail;   // a look-back wait of this workgroup gave up
  if constexpr (FUSED) {
    __shared__ int ticket;
    const int xcd = blockIdx.x & 7;
    if (tid == 0) {
      ticket = (int)__hip_atomic_fetch_add(sync + 16 * xcd, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
      lb_fail = 0;
    }
    __syncthreads();
    // ticket -> (group xcd + 8 i, head, V block), V block fastest; the grid has
    // as many workgroups per XCD as the XCD with the most groups has items.
    // Groups are segment-major (g = p B + b): every batch's segment p is
    // claimed before any segment p + 1, so the look-backs find their summaries
    // early and the last items claimed are last segments, which have no
    // summary pass (p = NSEG - 1 waits only for smaller groups either way).
    const int per = H * nvb64;
    const int grp = xcd + 8 * (ticket / per);
    if (grp >= B * NSEG) return;
    const int r = ticket % per;
    vblk = r % nvb64;
    h = r / nvb64;
    p = grp / B;
    b = grp % B;
  } else {
    // grid: xcd_head_grid(B * NSEG, H, nvb64)
    const XcdHeadMap xm = xcd_head_map(blockIdx.x, H, nvb64);
    if (xm.grp >= B * NSEG) return;
    h = xm.h;
    p = xm.grp % NSEG;
    b = xm.grp / NSEG;
    vblk = xm.slice;
  }
  const int row = b * H + h;
  const int gq = h / (H / G);
  const int NT = T / kBT;
  const int c0 = p << slog;
  const int nch = min(c0 + (1 << slog), NT) - c0;
  const int lu = 7 + nlev;
  const int nloc = min(slog, nlev);
  const int ntop = nlev - nloc;
  const int vcol0 = vblk * 64;
  const bool is_final_seg = final_state && ht != nullptr && p == NSEG - 1;
  float* htb = ht ? ht + ((size_t)b * H + h) * kKD * V * L : nullptr;
  // this row's summaries ([segment][K][V], fp32) and segment log-decays
  const float* srow = sums + (size_t)row * NSEG * kKD * V;
  const float* drow = FUSED ? segd + ((size_t)row * nvb64 + vblk) * NSEG : segd + (size_t)row * NSEG;
  const rsrc_t rsum = make_rsrc(srow, (size_t)NSEG * kKD * V * 4);
  const rsrc_t rsd = make_rsrc(drow, (size_t)NSEG * 4);
  // summary reads: coherent when another workgroup of this launch wrote them
  auto sum4 = [&](size_t el) -> floatx4 {
    if constexpr (FUSED)
      return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rsum, (unsigned int)(el * 4), 0, kCohLoad));
    else
      return *(const floatx4*)(srow + el);
  };
  auto sum1 = [&](size_t el) -> float {
    if constexpr (FUSED)
      return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsum, (unsigned int)(el * 4), 0, kCohLoad));
    else
      return srow[el];
  };
  auto segd1 = [&](int qq) -> float {
    if constexpr (FUSED)
      return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsd, (unsigned int)qq * 4, 0, kCohLoad));
    else
      return drow[qq];
  };

  if constexpr (FUSED) {
    // ---- phase A: Sum(p), D_p for the later segments (and this one's final states) ----
    if (p < NSEG - 1 || is_final_seg) {
      SumSmem<1>& ss = *(SumSmem<1>*)smem_raw;
      float* out = sums + ((size_t)row * NSEG + p) * kKD * V + vcol0;
      const float dsum = seg_sum_body<__bf16, TV, false, 1, true, LAYER, 4, E>(
          ss, k, v, g, out, b, h, p, vblk, T, G, H, V, NT, 1 << slog, la);
      if (tid == 0)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, dsum), rsd,
                                              (unsigned int)p * 4, 0, kCohStore);
      __builtin_amdgcn_s_waitcnt(0);   // this thread's summary stores are complete
      __syncthreads();
      if (tid == 0 && lbc.publish)
        __hip_atomic_store(sync + kSyncHdr + ((size_t)row * nvb64 + vblk) * NSEG + p, 1u,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (tid == 0) {
      // no later segment reads the last one's summary; its log-decay slot is
      // zeroed so the workspace (which the backward may reuse) holds no stale value
      __builtin_amdgcn_raw_buffer_store_b32(0u, rsd, (unsigned int)p * 4, 0, kCohStore);
    }
  }

  // ---- per-row buffer descriptors and per-lane offsets ---------------------------
  const int qstr = G * kKD, vstr = H * V, lstr = H * L;
  const rsrc_t rq = make_rsrc(q + ((size_t)b * T * G + gq) * kKD, (size_t)T * qstr * 2);
  const rsrc_t rk = make_rsrc(k + ((size_t)b * T * G + gq) * kKD, (size_t)T * qstr * 2);
  const rsrc_t rv = make_rsrc(v + ((size_t)b * T * H + h) * V + vcol0, (size_t)T * vstr * sizeof(TV));
  // g is read by wave 0 only: the other waves issue the same load through an
  // empty range, which returns zeros without a memory request
  const rsrc_t rg_ = make_rsrc(g + (size_t)b * T * H + h, w == 0 ? (size_t)T * H * 4 : 0);
  const rsrc_t ro = make_rsrc(o + ((size_t)b * T * H + h) * V + vcol0, (size_t)T * vstr * sizeof(TO));
  const bool write_gcum = gcum != nullptr && vblk == 0;
  // wave 0 computes Gc; the other waves issue the same store through an empty
  // range, so every wave has the same memory-operation sequence per chunk
  const rsrc_t rgc = make_rsrc(write_gcum ? (const void*)(gcum + (size_t)b * T * H + h) : (const void*)g,
                               write_gcum && w == 0 ? (size_t)T * H * 4 : 0);
  const unsigned int vo_qk = tile64_voff<__bf16>(qstr), vo_v = tile64_voff<TV>(vstr);
  const unsigned int vo_g = lane * H * 4;
  const unsigned int vo_o = (ln0 * vstr + 16 * w + 4 * lq0) * sizeof(TO);
  // g and lambda are read with one lane per token row (lane = t) and as few
  // instructions as possible: each of their rows is a separate cache line, so
  // the cost is per instruction and row, not per byte.  Wave 0 reads g (4 B per
  // row) and owns the chunk's decay vectors; waves 1 .. 3 read lambda in 16-byte
  // pieces of the row, aligned down to 4 bytes: piece r of a bf16 row holds
  // columns 8r - m .. 8r - m + 7 (m = the row's misalignment in elements), of an
  // fp32 row columns 4r .. 4r + 3.  Wave w reads pieces w - 1 and w + 2.
  constexpr bool kL16 = sizeof(TL) == 2;
  constexpr int kPE = kL16 ? 8 : 4;   // lambda columns per 16-byte piece
  const char* lbase = (const char*)(l + (size_t)b * T * H * L);
  const unsigned int lbmis = (unsigned int)((uintptr_t)lbase & 3);   // descriptor base aligned down
  // lambda is read by waves 1 .. 3 only (wave 0's range is empty, as for g);
  // bf16 rows of at most 15 used columns fit in pieces 0 and 1 whatever their
  // misalignment, so then wave 3 (piece 2) reads nothing either
  const bool lam_reader = w > 0 && !(kL16 && w == 3 && lu + 1 <= 2 * kPE);
  const rsrc_t rlb = make_rsrc(lbase - lbmis, lam_reader ? (size_t)T * H * L * sizeof(TL) + lbmis : 0);
  const unsigned int lrow_b = lbmis + (unsigned int)((lane * H + h) * L) * sizeof(TL);
  const int lmis = kL16 ? (int)((lrow_b >> 1) & 1) : 0;
  const unsigned int vo_l = lrow_b & ~3u;

  MainRegs<__bf16, TV, TL, 1> rg;
  constexpr int kLP = kL16 ? 1 : 2;   // pieces per wave (bf16 rows: lu <= 19 needs <= 3 pieces)
  const int lpw0 = w > 0 ? w - 1 : 0;   // first lambda piece of this wave
  // layer mode: dt words (wave 0: the lane's token row, for g; every thread: its
  // two V tile rows tid >> 3 and + 32, for v = x dt'), the head's A, bias, D and
  // the L[h] entries of the lambda columns this lane stages
  const int desz = la.dt_f32 ? 4 : 2;
  const char* dtb = LAYER ? (const char*)la.dt + (size_t)b * T * H * desz : (const char*)g;
  const rsrc_t rdt = make_rsrc(dtb, LAYER ? (size_t)T * H * desz : 0);
  const rsrc_t rdt0 = make_rsrc(dtb, LAYER && w == 0 ? (size_t)T * H * desz : 0);
  const float lay_A = LAYER ? la.A[h] : 0.f, lay_b = LAYER && la.bias ? la.bias[h] : 0.f;
  const float lay_D = LAYER && la.D ? la.D[h] : 0.f;
  const unsigned int el_g = (unsigned int)(lane * H + h), el_v = (unsigned int)((tid >> 3) * H + h);
  unsigned int dwv[2] = {0u, 0u};
  if (LAYER && tid < L) sm.lpar[tid] = la.Lp[h * L + tid];   // read after the first barrier
  uint4 lamr[kLP];
  const int lslot = 4 * (lane & 15) + (lane >> 4);   // this lane's token row t, permuted
  // value i of piece r goes to column kPE (w - 1 + 3 r) + i - lmis, staged at
  // row column + 1: element offset lam_lane + (3 kPE r + i) kBT of the buffer
  const int lam_lane = lslot + (1 - lmis + kPE * (w - 1)) * kBT;
  // part < 0: everything; parts 0, 1, 2: q / k / v, g and lambda (the loads of
  // chunk j + 2 are spread over phase 2 of chunk j, between its MFMA groups)
  auto load = [&](int j, int part) {
    const unsigned int row0 = (unsigned int)(c0 + j) * kBT;
    if (part <= 0) {
      // g and lambda first: they are one cache line per token row each, so they
      // take the longest to arrive, and their staging work is the first to use them.
      // Every wave issues the same loads (wave 0 uses only g, waves 1 .. 3 only
      // their lambda pieces; a piece past the row reads bytes of the next row, or
      // zeros past the buffer end, and is not used): a load assigned on some waves
      // only makes the compiler merge registers after the branch with copies that
      // wait for the load, i.e. a full memory round trip per chunk.  The unused
      // load of a wave goes through an empty range, so it makes no request.
      if constexpr (LAYER) rg.g = buf_load<float>(rdt0, ((row0 * H + el_g) * desz) & ~3u, 0);
      else rg.g = buf_load<float>(rg_, vo_g, row0 * H * 4);
      const unsigned int so_l = row0 * lstr * sizeof(TL);
#pragma unroll
      for (int r = 0; r < kLP; ++r) lamr[r] = buf_load16(rlb, vo_l, so_l + 16 * (lpw0 + 3 * r));
      load_tile64(rg.q, rq, vo_qk, row0 * qstr * 2, qstr);
    }
    if (part < 0 || part == 1) load_tile64(rg.k, rk, vo_qk, row0 * qstr * 2, qstr);
    if (part == 0 || part == 1) return;
    load_tile64(rg.v, rv, vo_v, row0 * vstr * sizeof(TV), vstr);
    if constexpr (LAYER) {
#pragma unroll
      for (int r = 0; r < 2; ++r)
        dwv[r] = __builtin_bit_cast(unsigned int, buf_load<float>(
            rdt, ((row0 * H + el_v + 32u * r * H) * desz) & ~3u, 0));
    }
  };
  // chunk j's registers -> LDS; par: the lambda / exp(Gc) buffer it goes to
  auto store = [&](int j, int par) {
    float gx = 0.f;
    store_tile_swz<swz_qk, __bf16, E>(rg.q, sm.q);
    store_tile_swz<swz_qk, __bf16, E>(rg.k, sm.k);
    if constexpr (LAYER) {
      // v = x dt' on the thread's two rows (dwv holds their dt', see dt_xform),
      // rounded to bf16 as the layer's v
      auto xs = rg.v;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const float d = __builtin_bit_cast(float, dwv[r]);
        bf16x8 xv = __builtin_bit_cast(bf16x8, xs.r[r]);
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = (__bf16)((float)xv[i] * d);
        xs.r[r] = __builtin_bit_cast(uint4, xv);
      }
      store_tile_swz<swz_v>(xs, sm.v);
    } else {
      store_tile_swz<swz_v, TV, E>(rg.v, sm.v);
    }
    if (w == 0) {
      const float x = chunk_cumsum(rg.g);   // lane t holds Gc_t (layer mode: g from dt_xform)
      const float last = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
      sm.gc[lane] = x * kLog2e;
      sm.wt[lane] = fexp(last - x);
      sm.eg[par][4 * ln0 + lq0] = fexp(x);
      gx = x;
    } else {
      // every value of the lane's pieces is stored, at a compile-time offset
      // from one per-lane base (no compares, no divergent branches)
      LT* lamw = sm.lam[par] + lam_lane;
#pragma unroll
      for (int r = 0; r < kLP; ++r) {
        const unsigned int* u = (const unsigned int*)&lamr[r];
#pragma unroll
        for (int i = 0; i < kPE; ++i) {
          if constexpr (sizeof(LT) == 2) {
            lamw[(3 * kPE * r + i) * kBT] = __builtin_bit_cast(bf16x8, lamr[r])[i];
          } else {
            float val;
            if constexpr (kL16) val = __builtin_bit_cast(float, (i & 1) ? (u[i >> 1] & 0xffff0000u) : (u[i >> 1] << 16));
            else val = __builtin_bit_cast(float, u[i]);
            lamw[(3 * kPE * r + i) * kBT] = val;
          }
        }
      }
    }
    buf_store<float>(gx, rgc, vo_g, (unsigned int)(c0 + j) * kBT * H * 4);
  };

  // layer mode: the dt words of the chunk in the prefetch registers become dt'
  // (V rows) and g = A dt' (wave 0) once they have landed, at the end of a
  // chunk rather than in the register-heavy middle where store() runs
  auto dt_xform = [&]() {
    if constexpr (LAYER) {
#pragma unroll
      for (int r = 0; r < 2; ++r)
        dwv[r] = __builtin_bit_cast(unsigned int,
                                    layer_dtp(layer_dt_word(dwv[r], el_v + 32u * r * H, la.dt_f32),
                                              lay_b, la.softplus));
      if (w == 0)
        rg.g = layer_g(lay_A, layer_dtp(layer_dt_word(__builtin_bit_cast(unsigned int, rg.g), el_g,
                                                      la.dt_f32), lay_b, la.softplus));
    }
  };
  // layer mode: lambda = compute_lambda(L[h], dl) applied in place to the dl
  // values this lane staged for chunk jj (its own entries only; the next
  // barrier publishes them), away from the register-heavy middle of a chunk
  auto lam_xform = [&](int jj) {
    if constexpr (LAYER) {
      if (w > 0) {
        float* lamw = sm.lam[jj & 1] + lam_lane;
#pragma unroll
        for (int r = 0; r < kLP; ++r) {
          const int col0 = kPE * (w - 1 + 3 * r) - lmis;
#pragma unroll
          for (int i = 0; i < kPE; ++i) {
            const int col = col0 + i;
            if ((unsigned int)col < (unsigned int)lu) {
              const int off = (3 * kPE * r + i) * kBT;
              float val = lambda_of(sm.lpar[col], lamw[off], la.mode);
              if (la.lam_bf16) val = (float)(__bf16)val;
              lamw[off] = val;
            }
          }
        }
      }
    }
  };

  floatx4 st[kMaxLoc][4];     // local states: tile 2c + h holds k = 32c + 8lq + 4h + i, v = ln
  float dl[kMaxLoc];          // pending log2-decay of each local state
#pragma unroll
  for (int e = 0; e < kMaxLoc; ++e) {
    dl[e] = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) st[e][m] = zero4();
  }

  // Pipeline: chunk j + 1 is staged in LDS right after phase 1 of chunk j (from
  // then on chunk j's stage is dead except lambda', which is double-buffered),
  // and chunk j + 2's loads are issued at the same point, so they have a whole
  // chunk period to land and a chunk needs two barriers instead of three.
  // the first chunk's loads go out before the look-back and the top-level
  // build, so their latency hides behind the wait for the earlier segments
  load(0, -1);
  if (LAYER) __syncthreads();   // L[h] staged in LDS
  dt_xform();
  if constexpr (FUSED) {
    // ---- look-back: the earlier segments of this row have published ----
    if (p > 0) {
      if (tid < p) {
        const unsigned int* f = sync + kSyncHdr + ((size_t)row * nvb64 + vblk) * NSEG + tid;
        unsigned int fv = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int spins = 0; fv == 0u && spins < lbc.spin_limit; ++spins) {
          __builtin_amdgcn_s_sleep(2);
          fv = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (fv == 0u) lb_fail = 1;
      }
      __syncthreads();
      if (lb_fail) {
        // the wait gave up: report it and poison this item's outputs
        if (tid == 0)
          __hip_atomic_fetch_or(sync + kSyncStatus, kStatusLookbackTimeout, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
        const float qnan = __builtin_nanf("");
        // o (layer mode: y): 64 rows x 64 columns per chunk, 8 columns per thread and row
        for (int jj = 0; jj < nch; ++jj)
          for (int u = tid; u < kBT * 8; u += 256) {
            const unsigned int t = (unsigned int)(c0 + jj) * kBT + (u >> 3);
#pragma unroll
            for (int c = 0; c < 8; ++c)
              buf_store<TO>(from_f32<TO>(qnan), ro,
                            (t * vstr + 8 * (u & 7) + c) * (unsigned int)sizeof(TO), 0);
          }
        for (int t = lane; t < nch * kBT; t += 64)   // wave 0 (the others' range is empty)
          buf_store<float>(qnan, rgc, 0, (((unsigned int)c0 * kBT + t) * H) * 4);
        if (is_final_seg)
          for (int u = tid; u < kKD * 64; u += 256)
            for (int e = 0; e < nlev; ++e)
              htb[((size_t)(u >> 6) * V + vcol0 + (u & 63)) * L + 7 + e] = qnan;
        return;
      }
    }
  }

  // ---- top levels: Htop_e(p) for the levels segment p reads -> LDS (bf16, [v][k]) ----
  // Htop_e(p) = sum_{q in block} exp(P[p] - P[q + 1]) Sum(q), block = the 2^e
  // segments before p's half of its aligned 2^(e+1) block, P[x] = sum_{r < x} D_r
  // (the top-level scan of chunkwise.py:199-247 over whole segments; the blocks
  // of the levels p reads partition [0, p)).  The summaries were just written
  // by the segment-summary kernel and are read from L2 / MALL.
  if (ntop > 0 && (p > 0 || is_final_seg)) {
    float* pre = (float*)sm.a;   // P[0 .. p + 1]; the A tile is free until the first chunk
    if (w == 0) {
      float carry = 0.f;
      for (int base = 0; base <= p + 1; base += 64) {
        const int qq = base + lane;
        const float x = qq <= p ? segd1(qq) : 0.f;
        const float y = chunk_cumsum(x);
        if (qq <= p + 1) pre[qq] = carry + y - x;
        carry += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, y), 63));
      }
    }
    __syncthreads();
    // thread: V columns 4 (tid & 15) .. + 3, k rows (tid >> 4) + 16 i
    const int v4 = 4 * (tid & 15), kr = tid >> 4;
    const size_t sp = (size_t)kr * V + vcol0 + v4;   // element offset in the row's summaries
    const size_t qstride = (size_t)kKD * V;
    const float pp = pre[p];
    for (int e2 = 0; e2 < ntop && p > 0; ++e2) {
      if (!((p >> e2) & 1)) continue;
      const int lo = (p >> (e2 + 1)) << (e2 + 1);
      floatx4 hacc[4] = {zero4(), zero4(), zero4(), zero4()};
      for (int q0 = lo; q0 < lo + (1 << e2); q0 += 4) {
        floatx4 xs[4][4];
        float sc[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int qs = min(q0 + u, lo + (1 << e2) - 1);
          sc[u] = q0 + u < lo + (1 << e2) ? fexp(pp - pre[qs + 1]) : 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) xs[u][i] = sum4(sp + qs * qstride + (size_t)16 * i * V);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) hacc[i][c] += sc[u] * xs[u][i][c];
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.top[e2 * kPl + top_idx(v4 + c, kr + 16 * i)] = to16<E>(hacc[i][c]);
    }
    if (is_final_seg) {
      // final states of the top levels (chunkwise.py:229-279): a level the last
      // chunk reads holds its block decayed over segment p; one it writes holds
      // segments [lo, p] decayed to the end of p
      const int vc = vcol0 + 16 * w + ln0;
      for (int e2 = 0; e2 < ntop; ++e2) {
        const bool reads = (p >> e2) & 1;
        const int lo = reads ? (p >> (e2 + 1)) << (e2 + 1) : (p >> e2) << e2;
        const int hi = reads ? lo + (1 << e2) : p + 1;
        floatx4 hacc[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) hacc[m] = zero4();
        for (int qs = lo; qs < hi; ++qs) {
          const float sc = fexp(pre[p + 1] - pre[qs + 1]);
          const size_t src = qs * qstride + vc;
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) hacc[m][i] += sc * sum1(src + (size_t)(16 * m + 4 * lq0 + i) * V);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            htb[((size_t)(16 * m + 4 * lq0 + i) * V + vc) * L + 7 + nloc + e2] = hacc[m][i];
      }
    }
  }

  // the two A tiles above the diagonal that the 32-wide s steps of A V read
  // ((t-tile 0, s-tile 1) and (2, 3)) stay zero for the whole walk
  __syncthreads();   // the A tile may have served as scratch for the top-level build
  {
    const int r = tid >> 3, c = 4 * (tid & 3), tile = (tid >> 2) & 1;
    *(bf16x4*)(sm.a + sidx<swz_a>(32 * tile + (r & 15), 16 + 32 * tile + c)) = bf16x4{};
  }
  store(0, 0);
  lam_xform(0);
  // The loads and LDS staging of chunks 1, j + 1, j + 2 are unconditional (the
  // chunk index clamped to the last chunk, the staging of a chunk past the end
  // repeating the last one into buffers nothing reads): a memory operation
  // behind a branch makes the compiler's wait counts ignore the operations
  // after it, i.e. wait for more than the chunk being staged.
  load(min(1, nch - 1), -1);
  dt_xform();
  __builtin_amdgcn_sched_barrier(0);
  {
    // Four o-shaped stores through an empty range (no request is made): on the
    // back edge the loop's four o stores follow the next chunk's loads, so with
    // these the loop header sees the same memory-operation order on both
    // incoming paths, and the staging waits of chunk j + 1 leave the previous
    // chunk's o stores in flight instead of waiting for every operation.
    const rsrc_t rnone = make_rsrc(o, 0);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) buf_store4<TO>(zero4(), rnone, vo_o, 16u * nt * vstr * sizeof(TO));
  }
  float Eseg = 0.f;   // log2-decay from the segment start to the current chunk start
  const int topmask = ntop > 0 ? (p & ((1 << ntop) - 1)) : 0;   // top levels this segment reads
  // nch >= 1: a do-while, so the preheader runs straight into the body (a loop
  // guard would let the compiler sink chunk 1's loads below the stores above)
  int j = 0;
  do {
    const int ic = c0 + j;
    __syncthreads();   // chunk j staged; every wave is done with chunk j - 1
    // Lane indices made opaque per chunk, so the compiler recomputes the LDS
    // addresses of the phases (a few VALU ops) instead of keeping dozens of
    // loop-invariant addresses in VGPRs across the whole walk.
    int lq, ln;
    asm volatile("v_mov_b32 %0, %1" : "=v"(lq) : "v"(lq0));
    asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(ln0));
    const LdsBase lb = lds_base(lq, ln, w);

    // Q fragments Q[t = 16mt + ln][k = 32c + 8lq + j]; V fragments
    // V[s = 32c + 8lq + j][v = 16w + ln] (A operand of o^T = V^T A^T, and with
    // the decay weights the B operand of K^T diag(w) V)
    bf16x8 qa[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int c = 0; c < 2; ++c) qa[mt][c] = *(const bf16x8*)(sm.q + (c ? lb.rq1 : lb.rq0) + 1024 * mt);
    const bf16x8 vt0 = vtr_frag(sm.v, lb, 0);
    const bf16x8 vt1 = vtr_frag(sm.v, lb, 32);

    // ---- phase 1: A = S o M, and the chunk's K^T diag(w) V -------------------------
    floatx4 kv[4];
    switch (w) {
      case 0: bf16_p1<0, LT, E>(sm, lb, sm.lam[j & 1] + kBT, qa, vt0, vt1, kv, lq, ln); break;
      case 1: bf16_p1<1, LT, E>(sm, lb, sm.lam[j & 1] + kBT, qa, vt0, vt1, kv, lq, ln); break;
      case 2: bf16_p1<2, LT, E>(sm, lb, sm.lam[j & 1] + kBT, qa, vt0, vt1, kv, lq, ln); break;
      default: bf16_p1<3, LT, E>(sm, lb, sm.lam[j & 1] + kBT, qa, vt0, vt1, kv, lq, ln); break;
    }
    const float glr = sm.gc[kBT - 1];   // chunk log2-decay
    __syncthreads();   // A visible; chunk j's stage (but lambda') no longer read
    store(min(j + 1, nch - 1), (j + 1) & 1);
    const int jn = min(j + 2, nch - 1);
    load(jn, 0);
    const LT* lpr = sm.lam[j & 1] + 8 * kBT;   // level 7 (row 8)
    const floatx4 egr = *(const floatx4*)(sm.eg[j & 1] + 4 * ln);   // exp(Gc_t), t = 16nt + ln

    // ---- phase 2: o^T[v = 16w + 4lq + i][t = 16nt + ln] ------------------------------
    floatx4 acc[4];
    {
      bf16x8 af[6];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) af[nt] = *(const bf16x8*)(sm.a + lb.ra0 + 1024 * nt);
      af[4] = *(const bf16x8*)(sm.a + lb.ra1 + 1024 * 2);
      af[5] = *(const bf16x8*)(sm.a + lb.ra1 + 1024 * 3);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[nt] = mfma16<E>(vt0, af[nt], zero4());
      acc[2] = mfma16<E>(vt1, af[4], acc[2]);
      acc[3] = mfma16<E>(vt1, af[5], acc[3]);
    }
    load(jn, 1);
    // local levels the chunk reads (bit e of the chunk index): all eight MFMAs of
    // a level are issued before its lambda-weighted accumulation
#pragma unroll
    for (int e = 0; e < kMaxLoc; ++e) {
      if (e < nloc && ((ic >> e) & 1)) {
        const floatx4 lam = lam4(lpr + e * kBT + 4 * ln);
        const bf16x8 h0 = cat8e<E>(st[e][0], st[e][1]);
        const bf16x8 h1 = cat8e<E>(st[e][2], st[e][3]);
        floatx4 tmp[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) tmp[nt] = mfma16<E>(h0, qa[nt][0], zero4());
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) tmp[nt] = mfma16<E>(h1, qa[nt][1], tmp[nt]);
        const float sc = fexp2(dl[e]);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const float cf = lam[nt] * egr[nt] * sc;
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[nt][i] += tmp[nt][i] * cf;
        }
      }
    }
    load(jn, 2);
    // top levels (bits of the segment index), the next level's fragments
    // prefetched while the current one multiplies
    if (topmask && j >= 0) {
      const float ee = fexp2(Eseg);
      int m = topmask;
      int e2 = __builtin_ctz(m);
      // A operand h^T[v = 16w + ln][k = 32c + 8lq + j]: 16-byte units lq, 4 + lq of row v
      const int vrow = 16 * w + ln;
      const __bf16* tb = sm.top + vrow * 64;
      const int u0 = ((lq ^ vrow) & 7) << 3, u1 = (((4 + lq) ^ vrow) & 7) << 3;
      bf16x8 h0 = *(const bf16x8*)(tb + e2 * kPl + u0);
      bf16x8 h1 = *(const bf16x8*)(tb + e2 * kPl + u1);
      floatx4 lam = lam4(lpr + (nloc + e2) * kBT + 4 * ln);
      while (true) {
        m &= m - 1;
        bf16x8 n0 = h0, n1 = h1;
        floatx4 nl = lam;
        if (m) {
          const int e2n = __builtin_ctz(m);
          n0 = *(const bf16x8*)(tb + e2n * kPl + u0);
          n1 = *(const bf16x8*)(tb + e2n * kPl + u1);
          nl = lam4(lpr + (nloc + e2n) * kBT + 4 * ln);
        }
        floatx4 tmp[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) tmp[nt] = mfma16<E>(h0, qa[nt][0], zero4());
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) tmp[nt] = mfma16<E>(h1, qa[nt][1], tmp[nt]);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const float cf = lam[nt] * egr[nt] * ee;
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[nt][i] += tmp[nt][i] * cf;
        }
        if (!m) break;
        h0 = n0;
        h1 = n1;
        lam = nl;
      }
    }
    if (LAYER && la.D != nullptr) {
      // y = bf16(o) + x D[h]: x[t = 16 nt + ln][v = 16 w + 4 lq .. + 3]
      // one x row group at a time, fenced so the loads are not hoisted into the
      // register-heavy part of the chunk
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        __builtin_amdgcn_sched_barrier(0);
        const bf16x4 x4 = __builtin_bit_cast(
            bf16x4, buf_load8(rv, (ln0 * vstr + 16 * w + 4 * lq0) * 2,
                              ((unsigned int)ic * kBT + 16 * nt) * vstr * 2));
        floatx4 y;
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = layer_out((float)(__bf16)acc[nt][i], (float)x4[i], lay_D);
        buf_store4<TO>(y, ro, vo_o, ((unsigned int)ic * kBT + 16 * nt) * vstr * sizeof(TO));
      }
      __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        buf_store4<TO>(acc[nt], ro, vo_o, ((unsigned int)ic * kBT + 16 * nt) * vstr * sizeof(TO));
    }

    // ---- local state update with the chunk's K^T diag(w) V ---------------------------
    if (nloc > 0) {
      const bool keep_last = (ic == NT - 1) && final_state;
#pragma unroll
      for (int e = 0; e < kMaxLoc; ++e) {
        if (e < nloc) {
          const int per = 2 << e;
          if (((ic & (per - 1)) == per - 1) && !keep_last) {
            dl[e] = 0.f;   // block ends: the next chunk starts a fresh state
#pragma unroll
            for (int m = 0; m < 4; ++m) st[e][m] = zero4();
          } else if (!((ic >> e) & 1)) {
            const float s = fexp2(dl[e] + glr);
            dl[e] = 0.f;
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
              for (int i = 0; i < 4; ++i) st[e][m][i] = st[e][m][i] * s + kv[m][i];
          } else {
            dl[e] += glr;
          }
        }
      }
      if (keep_last && is_final_seg) {
        // ht[b, h, k, v, 7 + e] (chunkwise.py:1179, 277-279)
        const int vc = vcol0 + 16 * w + ln;
#pragma unroll
        for (int e = 0; e < kMaxLoc; ++e)
          if (e < nloc) {
            const float s = fexp2(dl[e]);
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                htb[((size_t)(32 * (m >> 1) + 8 * lq + 4 * (m & 1) + i) * V + vc) * L + 7 + e] =
                    st[e][m][i] * s;
          }
      }
    }
    if (j + 1 < nch) lam_xform(j + 1);
    dt_xform();   // chunk j + 2's dt words (the last chunk's again past the end)
    Eseg += glr;
  } while (++j < nch);
}

}  // namespace hattn

// dtype codes shared with the C-ABI (include/hattn.h)
enum { DT_BF16 = 0, DT_FP16 = 1, DT_FP32 = 2 };

namespace {
size_t segd_bytes(size_t rows, int NSEG) {
  return (rows * NSEG * sizeof(float) + 255) & ~(size_t)255;
}
int max_loc(int x3) { return x3 ? hattn::kMaxLocX3 : hattn::kMaxLoc; }

// x3: fp32 q / k / v / lambda computed as bf16x3 (more local levels per segment).
// Workspace: segment log-decays, segment summaries (fp32 [row][seg][K][V]) and
// the top-level states (bf16 planes [row][seg][level][vblk][plane][64][64]).
struct FwdWs {
  float* segd;
  float* sums;
  __bf16* htop;
  unsigned int* sync;   // fused bf16 forward: ticket counters, status word, one flag per (row, V block, segment)
  int nsync;
  size_t bytes;
};

// x3 (bf16x3 kernels): segment log-decays per row, summaries, staged top-level
// states.  bf16 (fused single pass): log-decays per (row, V block), summaries,
// the ticket counter and flags.
FwdWs fwd_ws_layout(void* base, int B, int T, int H, int V, int x3) {
  const int NT = T / hattn::kBT;
  const int slog = hattn::seg_log2(NT, max_loc(x3));
  const int NSEG = (NT + (1 << slog) - 1) >> slog;
  int nlev = 0;
  while ((1 << nlev) < NT) ++nlev;
  const int ntop = nlev - (slog < nlev ? slog : nlev);
  FwdWs w{nullptr, nullptr, nullptr, nullptr, 0, 0};
  if (NSEG <= 1) return w;
  const size_t rows = (size_t)B * H;
  const int nvb = V / 64;
  char* p = (char*)base;
  const size_t a = segd_bytes(x3 ? rows : rows * nvb, NSEG);
  const size_t b = (rows * NSEG * hattn::kKD * V * sizeof(float) + 255) & ~(size_t)255;
  // top-level states are staged by the scan kernel only for the bf16x3 kernels;
  // the bf16 main kernel builds them from the summaries itself
  const size_t c = x3 ? rows * NSEG * ntop * (size_t)(V / 64) * 2 * hattn::kKD * 64 * 2 : 0;
  w.segd = (float*)p;
  w.sums = (float*)(p + a);
  w.htop = (__bf16*)(p + a + b);
  w.bytes = a + b + c;
  if (!x3) {
    w.nsync = hattn::kSyncHdr + (int)(rows * nvb * NSEG);
    w.sync = (unsigned int*)(p + a + b);
    w.bytes = a + b + (((size_t)w.nsync * 4 + 255) & ~(size_t)255);
  }
  return w;
}
}  // namespace

size_t hattn_mamba2_fwd_ws_bytes(int B, int T, int H, int V, int x3) {
  return fwd_ws_layout(nullptr, B, T, H, V, x3).bytes;
}

// Where a bf16 forward's workspace holds its segment summaries (fp32
// [row][segment][K][V]) and segment log-decays ([row][V block][segment]); both
// null when the sizes have a single segment (no summaries).
void hattn_mamba2_fwd_ws_summaries(void* ws, int B, int T, int H, int V, const float** sums,
                                   const float** segd) {
  const FwdWs w = fwd_ws_layout(ws, B, T, H, V, 0);
  *sums = w.sums;
  *segd = w.segd;
}

// ---------------------------------------------------------------------------
// Static scratch of the no-allocation forward entry point
// ---------------------------------------------------------------------------
// A file-scope device array that replaces the caller's workspace for callers
// that cannot allocate.  Each GPU holds its own copy (at its own address) until
// the process ends; every call on a GPU shares it, so calls that overlap on one
// GPU race.  Host code never uses the array's name as an address: the device
// address comes from hipGetSymbolAddress, looked up once per device.
namespace {
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

size_t hattn_mamba2_fwd_static_scratch_bytes() { return kStaticScratchBytes; }

// Device address of the current device's static scratch (looked up on the
// first call on that device, with the device current).
hipError_t hattn_mamba2_fwd_static_scratch(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

// Largest inter-chunk level count: register-resident local levels plus the
// top levels whose states fit in LDS.
int hattn_mamba2_fwd_max_levels(int x3) {
  using namespace hattn;
  if (!x3) return kMaxLoc + kMaxTop;
  constexpr int kLdsBytes = 160 * 1024;
  const int base = main_smem_bytes<2, kMaxLocX3>(0), per = main_smem_bytes<2, kMaxLocX3>(1) - base;
  const int ntop = (kLdsBytes - base) / per;
  return kMaxLocX3 + (ntop < kMaxTop ? ntop : kMaxTop);
}

// Look-back controls of the fused forward launches (test hook; the defaults
// are the production values).
namespace {
std::atomic<int> g_spin_limit{hattn::kSpinLimit};
std::atomic<int> g_publish{1};
}  // namespace

void hattn_mamba2_fwd_set_lookback(int spin_limit, int publish) {
  g_spin_limit.store(spin_limit > 0 ? spin_limit : hattn::kSpinLimit);
  g_publish.store(publish ? 1 : 0);
}

// Where the fused forward's status word sits in its workspace (null when the
// sizes have a single segment and the forward has no look-back).
const unsigned int* hattn_mamba2_fwd_status_word(const void* ws, int B, int T, int H, int V) {
  const FwdWs w = fwd_ws_layout(const_cast<void*>(ws), B, T, H, V, 0);
  return w.sync ? w.sync + hattn::kSyncStatus : nullptr;
}

namespace hattn {

inline LookbackCtl lookback_ctl() { return LookbackCtl{g_spin_limit.load(), g_publish.load()}; }

// E: the 16-bit MFMA format of the fused single pass (NP = 1): bf16, or fp16
// for fp16 q / k / v.
template <typename TK, typename TV, typename TL, typename TO, int NP, int MAXLOC,
          typename E = __bf16>
static hipError_t launch_t(const void* q, const void* k, const void* v, const float* g,
                           const void* l, void* o, float* gcum, float* ht, void* ws, int B,
                           int T, int G, int H, int V, int L, int nlev, hipStream_t stream) {
  const int NT = T / kBT;
  const int slog = seg_log2(NT, MAXLOC);
  const int S = 1 << slog;
  const int NSEG = (NT + S - 1) / S;
  const int rows = B * H;
  const int nvb64 = V / 64;
  const FwdWs w = fwd_ws_layout(ws, B, T, H, V, NP == 2);
  const int ntop = nlev - min(slog, nlev);
  if constexpr (NP == 1) {
    // bf16: one fused single-pass launch (plus the flag reset) when there is
    // more than one segment, else the plain walk
    // bf16 lambda staged as bf16 where only that fits two workgroups per CU
    const bool lam16 = sizeof(TL) == 2 && 2 * bf16_smem_bytes<float>(ntop) > kLdsPerCu &&
                       2 * bf16_smem_bytes<__bf16>(ntop) <= kLdsPerCu;
    const int smem = lam16 ? bf16_smem_bytes<__bf16>(ntop) : bf16_smem_bytes<float>(ntop);
    hipError_t e;
    if (NSEG > 1) {
      hipLaunchKernelGGL(mamba2_fwd_sync_init_kernel, dim3((w.nsync + 255) / 256), dim3(256), 0,
                         stream, w.sync, w.nsync);
      if ((e = hipGetLastError()) != hipSuccess) return e;
      auto kern = mamba2_fwd_bf16_kernel<TV, TL, TO, true, false, false, E>;
      if constexpr (sizeof(TL) == 2)
        if (lam16) kern = mamba2_fwd_bf16_kernel<TV, TL, TO, true, false, true, E>;
      e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(kern, dim3(xcd_head_grid(B * NSEG, H, nvb64)), dim3(256), smem, stream,
                         (const __bf16*)q, (const __bf16*)k, (const TV*)v, g, (const TL*)l, (TO*)o,
                         gcum, ht, w.sums, w.segd, w.sync, B, T, G, H, V, L, nlev, nvb64, slog,
                         NSEG, ht != nullptr ? 1 : 0, LayerArgs{}, lookback_ctl());
      return hipGetLastError();
    }
    auto kern = mamba2_fwd_bf16_kernel<TV, TL, TO, false, false, false, E>;
    e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(xcd_head_grid(B * NSEG, H, nvb64)), dim3(256), smem, stream,
                       (const __bf16*)q, (const __bf16*)k, (const TV*)v, g, (const TL*)l, (TO*)o,
                       gcum, ht, w.sums, w.segd, w.sync, B, T, G, H, V, L, nlev, nvb64, slog, NSEG,
                       ht != nullptr ? 1 : 0, LayerArgs{}, lookback_ctl());
    return hipGetLastError();
  } else {
  // bf16x3 (NP = 2): segment summaries, staged top-level states, then the walk
  if (NSEG > 1) {
    auto sk = mamba2_seg_sum_kernel<TK, TV, false, NP>;
    hipLaunchKernelGGL(sk, dim3(xcd_head_grid(B * NSEG, H, nvb64)), dim3(256), 0, stream,
                       (const TK*)k, (const TV*)v, g, w.sums, w.segd, B, T, G, H, V, NT, S, NSEG,
                       nvb64);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ntop > 0 && NP == 2) {
      auto hk = mamba2_htop_kernel<NP>;
      hipLaunchKernelGGL(hk, dim3(rows * nvb64 * 4), dim3(256), 0, stream, w.sums, w.segd,
                         w.htop, V, NSEG, ntop, nvb64);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  const int grid = xcd_head_grid(B * NSEG, H, nvb64);
  const int smem = main_smem_bytes<NP, MAXLOC>(ntop);
  auto kern = mamba2_fwd_main_kernel<TK, TV, TL, TO, NP, MAXLOC>;
  hipError_t e =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), smem, stream, (const TK*)q, (const TK*)k,
                     (const TV*)v, g, (const TL*)l, (TO*)o, gcum, ht, w.sums, w.segd,
                     (const __bf16*)w.htop, B, T, G, H, V, L, nlev, nvb64, slog, NSEG,
                     ht != nullptr ? 1 : 0);
  return hipGetLastError();
  }
}

// The layer scan of hmamba_chunk_scan_combined with its pre- and
// post-processing folded into the fused bf16 forward: x and dl are read in
// place of v and lambda, dt in place of g; o receives bf16(scan) + x D[h] (or
// the scan output when D is null).
template <typename TL, typename TO>
static hipError_t layer_launch_t(const void* q, const void* k, const void* x, const void* dl,
                                 void* o, float* gcum, void* ws, const LayerArgs& la, int B, int T,
                                 int G, int H, int V, int L, int nlev, hipStream_t stream) {
  const int NT = T / kBT;
  const int slog = seg_log2(NT, kMaxLoc);
  const int NSEG = (NT + (1 << slog) - 1) >> slog;
  const int nvb64 = V / 64;
  const FwdWs w = fwd_ws_layout(ws, B, T, H, V, 0);
  const int ntop = nlev - min(slog, nlev);
  const int smem = bf16_smem_bytes<float>(ntop);
  hipError_t e;
  if (NSEG > 1) {
    hipLaunchKernelGGL(mamba2_fwd_sync_init_kernel, dim3((w.nsync + 255) / 256), dim3(256), 0,
                       stream, w.sync, w.nsync);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    auto kern = mamba2_fwd_bf16_kernel<__bf16, TL, TO, true, true>;
    e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(xcd_head_grid(B * NSEG, H, nvb64)), dim3(256), smem, stream,
                       (const __bf16*)q, (const __bf16*)k, (const __bf16*)x, (const float*)nullptr,
                       (const TL*)dl, (TO*)o, gcum, (float*)nullptr, w.sums, w.segd, w.sync, B, T,
                       G, H, V, L, nlev, nvb64, slog, NSEG, 0, la, lookback_ctl());
    return hipGetLastError();
  }
  auto kern = mamba2_fwd_bf16_kernel<__bf16, TL, TO, false, true>;
  e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(xcd_head_grid(B * NSEG, H, nvb64)), dim3(256), smem, stream,
                     (const __bf16*)q, (const __bf16*)k, (const __bf16*)x, (const float*)nullptr,
                     (const TL*)dl, (TO*)o, gcum, (float*)nullptr, w.sums, w.segd, w.sync, B, T, G,
                     H, V, L, nlev, nvb64, slog, NSEG, 0, la, lookback_ctl());
  return hipGetLastError();
}

}  // namespace hattn

// dt_qk == DT_FP32 selects the bf16x3 kernels, which take fp32 q, k, v, lambda
// and write fp32 o.
hipError_t hattn_mamba2_fwd_launch(const void* q, const void* k, const void* v, const float* g,
                                   const void* l, void* o, float* gcum, float* ht, void* ws,
                                   int B, int T, int G, int H, int V, int L, int nlev, int dt_qk,
                                   int dt_v, int dt_l, int dt_o, hipStream_t stream,
                                   int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  if (dt_qk == DT_FP32) {
    if (dt_v == DT_FP32 && dt_l == DT_FP32 && dt_o == DT_FP32)
      return launch_t<float, float, float, float, 2, kMaxLocX3>(q, k, v, g, l, o, gcum, ht, ws,
                                                                B, T, G, H, V, L, nlev, stream);
    *unsupported = 1;
    return hipSuccess;
  }
  if (dt_qk == DT_FP16) {
    // fp16 q / k / v on fp16 MFMA (fp32 lambda; v and o fp16 or fp32)
#define HATTN_DISPATCH_H(TV_, TO_)                                                               \
  return launch_t<_Float16, TV_, float, TO_, 1, kMaxLoc, _Float16>(q, k, v, g, l, o, gcum, ht, ws, \
                                                                  B, T, G, H, V, L, nlev, stream);
    if (dt_l == DT_FP32) {
      if (dt_v == DT_FP16 && dt_o == DT_FP16) { HATTN_DISPATCH_H(_Float16, _Float16) }
      if (dt_v == DT_FP16 && dt_o == DT_FP32) { HATTN_DISPATCH_H(_Float16, float) }
      if (dt_v == DT_FP32 && dt_o == DT_FP16) { HATTN_DISPATCH_H(float, _Float16) }
      if (dt_v == DT_FP32 && dt_o == DT_FP32) { HATTN_DISPATCH_H(float, float) }
    }
#undef HATTN_DISPATCH_H
    *unsupported = 1;
    return hipSuccess;
  }
  if (dt_qk != DT_BF16) {
    *unsupported = 1;
    return hipSuccess;
  }
#define HATTN_DISPATCH_O(TV_, TL_)                                                             \
  if (dt_o == DT_BF16)                                                                       \
    return launch_t<__bf16, TV_, TL_, __bf16, 1, kMaxLoc>(q, k, v, g, l, o, gcum, ht, ws, B, T, \
                                                          G, H, V, L, nlev, stream);           \
  if (dt_o == DT_FP32)                                                                       \
    return launch_t<__bf16, TV_, TL_, float, 1, kMaxLoc>(q, k, v, g, l, o, gcum, ht, ws, B, T,  \
                                                         G, H, V, L, nlev, stream);
  if (dt_v == DT_BF16 && dt_l == DT_BF16) { HATTN_DISPATCH_O(__bf16, __bf16) }
  if (dt_v == DT_BF16 && dt_l == DT_FP32) { HATTN_DISPATCH_O(__bf16, float) }
  if (dt_v == DT_FP32 && dt_l == DT_BF16) { HATTN_DISPATCH_O(float, __bf16) }
  if (dt_v == DT_FP32 && dt_l == DT_FP32) { HATTN_DISPATCH_O(float, float) }
#undef HATTN_DISPATCH_O
  *unsupported = 1;
  return hipSuccess;
}

// Layer scan with the pre- / post-processing folded in: bf16 q (= C), k (= B),
// x; dl bf16 or fp32; o (y) bf16 or fp32; dt bf16 or fp32 (la.dt_f32).
hipError_t hattn_mamba2_layer_fwd_launch(const void* q, const void* k, const void* x,
                                         const void* dl, void* o, float* gcum, void* ws,
                                         const void* dt, const float* A, const float* dt_bias,
                                         const float* Lp, const float* D, int dt_f32,
                                         int softplus, int mode, int lam_bf16, int B, int T,
                                         int G, int H, int V, int L, int nlev, int dt_l,
                                         int dt_o, hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  const LayerArgs la{dt, A, dt_bias, Lp, D, dt_f32, softplus, mode, lam_bf16};
  if (dt_l == DT_BF16 && dt_o == DT_BF16)
    return layer_launch_t<__bf16, __bf16>(q, k, x, dl, o, gcum, ws, la, B, T, G, H, V, L, nlev, stream);
  if (dt_l == DT_BF16 && dt_o == DT_FP32)
    return layer_launch_t<__bf16, float>(q, k, x, dl, o, gcum, ws, la, B, T, G, H, V, L, nlev, stream);
  if (dt_l == DT_FP32 && dt_o == DT_BF16)
    return layer_launch_t<float, __bf16>(q, k, x, dl, o, gcum, ws, la, B, T, G, H, V, L, nlev, stream);
  if (dt_l == DT_FP32 && dt_o == DT_FP32)
    return layer_launch_t<float, float>(q, k, x, dl, o, gcum, ws, la, B, T, G, H, V, L, nlev, stream);
  *unsupported = 1;
  return hipSuccess;
}
