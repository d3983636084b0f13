// Log-linear Gated DeltaNet chunkwise forward for gfx950.
//
// Replaces chunkwise_hgdn.chunkwise_fwd (chunkwise_hgdn.py:566-788): the
// reference materialises gamma = exp(segsum(g)) in torch, then launches
// chunk_scaled_dot_kkt, two solve_tril passes, recompute_w_u, preprocess_qkw,
// a torch einsum for q_new, the intra-chunk output kernel and, per inter-chunk
// level, torch masked copies of u / w / g plus the delta-rule state kernel and
// the output kernel.
//
// Per (b, h) row, chunk of C = 64 tokens, chunk-local cumsum Gc, with
// A = strict-tril(diag(beta) K K^T), Aw = (I + A)^-1, gamma[t,s] =
// exp(Gc_t - Gc_s) (s <= t), Au = Aw o gamma, M = tril(Q K^T):
//   W = Aw (beta K),  U = Au (beta V),  K_new = exp(Gc_last - Gc) K,
//   W_new = exp(Gc) W,  q_new = exp(Gc) (Q - M W),
//   P = (M Aw) o gamma o beta_s o lambda[t, lev(t, s)],  o_intra = P V,
// and every inter-chunk level e runs the delta-rule recurrence over chunks
//   h_e <- (reset ? 0 : exp(Gc_last) h_e) + K_new^T ((write ? U : 0) - (reset ? 0 : W_new h_e))
// (write: bit e of the chunk index clear; reset after the last chunk of an
// aligned 2^(e+1) block), read by the chunks with bit e set:
//   o += lambda[t, 7 + e] q_new h_e.
//
// Kernel 1 (gdn_prep_kernel): persistent workgroups of eight waves walk the
// chunks; the next chunk's Q / K / V tiles are loaded into registers while the
// current one computes.  Per chunk: K K^T and Q K^T on MFMA, the fp32
// unit-lower-triangular inverse (on fp32 MFMA), then W, q_new, U and P as transposed MFMA
// products (each lane ends with four consecutive columns of one row, stored
// as one 8-byte write).  K is handled in 64-column blocks and V in 64-column
// blocks, so K up to 256 and any V fit the LDS.  Outputs: q_new, W_new (token
// major), K_new transposed per chunk ([row][chunk][k][t], the scan's MFMA
// operand layout), U, and P (bf16, [row][chunk][t][s]); the backward's
// recompute also writes K_new token-major.
// Kernel 2 (gdn_scan_kernel): one workgroup per (row, BV columns of V), eight
// waves in two level groups.  Every level's [K x BV] state lives in fp32
// registers (a group's levels, the wave's k-quarter).  Per chunk the states
// are staged in LDS as bf16, each wave forms W_new h_e (-> V_new_e, LDS) and
// q_new h_e (-> the level reads) of its group's levels for its 16-row t-tile,
// group 0 adds o_intra = P V and writes o, and every wave updates its state
// tiles with K_new^T V_new_e.  The next chunk's operands are loaded while the
// current one computes.  The slices of one row run on one XCD, so the chunk
// tiles they share are fetched into one L2.
#include "gdn_common.h"

namespace hattn {

// ---------------------------------------------------------------------------
// chunk-local preparation
// ---------------------------------------------------------------------------
template <int KD>
struct GdnPrepSmem {
  static constexpr int LK = KD + 8;
  __bf16 q[kGC * LK];
  __bf16 k[kGC * LK];
  float ax[2 * kGC * kLM];        // A | X = (I + A)^-1, fp32
  __bf16 aw[kGC * kLd64];         // Aw (bf16)
  __bf16 au[kGC * kLd64];         // Au = Aw o gamma (bf16)
  __bf16 mq[kGC * kLd64];         // M = tril(Q K^T) (bf16)
  union {
    __bf16 w[kGC * kLd64];        // one 64-column block of W (bf16)
    float inv[kInvScratchFloats]; // scratch of the inverse
  } wt;
  __bf16 v[kGC * kLd64];          // one 64-column block of V
  float gc[kGC];
  float beta[kGC];
  float lam[7][kGC];              // intra-chunk lambda columns 0..6
};

constexpr int kPrepThreads = 512;
// MODE kPrepFwd: g is the per-step log decay (its chunk-local cumsum is
// written to gcum); outputs Aw, Au, q_new, W_new, K_new^T, U, P.
// MODE kPrepRecompute (the backward): g already holds the chunk-local cumsum
// (chunkwise_hgdn.py:799-817); outputs q_new, W_new, K_new (token-major and
// transposed) and U.
enum { kPrepFwd = 0, kPrepRecompute = 1 };

template <int KD, typename TB, typename TL, int MODE>
__global__ __launch_bounds__(kPrepThreads) void gdn_prep_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const TB* __restrict__ beta, const float* __restrict__ g, const TL* __restrict__ l,
    float* __restrict__ gcum, __bf16* __restrict__ aw_out, __bf16* __restrict__ au_out,
    __bf16* __restrict__ qn, __bf16* __restrict__ wn, __bf16* __restrict__ kn,
    __bf16* __restrict__ knT, __bf16* __restrict__ un, __bf16* __restrict__ pm, int nchunks,
    int T, int H, int V, int L, int norm_qk, float qk_scale) {
  using Sm = GdnPrepSmem<KD>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Sm& s = *(Sm*)smem_raw;
  constexpr int LK = Sm::LK;
  constexpr int NTH = kPrepThreads;
  constexpr int QU = KD / 64;     // 16-byte units of a Q (K) tile per thread
  constexpr int UPR = KD / 8;     // 16-byte units per row
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int tt = w & 3, wh = w >> 2;   // output t-tile, half of the 64-column block
  const int NT = T / kGC;
  const int NVB = V / 64;
  const size_t hk = (size_t)H * KD, hv = (size_t)H * V;
  float* A = s.ax;                // [64][kLM]
  float* X = s.ax + kGC * kLM;    // [64][kLM]

  int ci = blockIdx.x;
  if (ci >= nchunks) return;

  // ---- register prefetch of one chunk ----------------------------------------------
  // Every load is issued unconditionally (clamped to a valid address where the
  // value is not used), so the compiler does not wait for it at a branch merge.
  u32x4 pq[QU], pk[QU], pv[2];
  float pg, pb, pl;
  auto tok_of = [&](int c) __attribute__((always_inline)) {
    const int row = c / NT;
    return (size_t)(row / H) * T + (size_t)(c % NT) * kGC;
  };
  auto fetch_qk = [&](int c) __attribute__((always_inline)) {
    const size_t t0 = tok_of(c);
    const int h = (c / NT) % H;
#pragma unroll
    for (int i = 0; i < QU; ++i) {
      const int u = tid + NTH * i, r = u / UPR, cc = 8 * (u % UPR);
      const size_t off = (t0 + r) * hk + (size_t)h * KD + cc;
      pq[i] = *(const u32x4*)(q + off);
      pk[i] = *(const u32x4*)(k + off);
    }
    const int e = min(tid, 7 * kGC - 1);
    pg = g[(t0 + lane) * H + h];
    pb = to_f32<TB>(beta[(t0 + lane) * H + h]);
    pl = to_f32<TL>(l[((t0 + e / 7) * H + h) * L + e % 7]);
  };
  auto fetch_v = [&](int c, int vb, u32x4& dst) __attribute__((always_inline)) {
    const size_t t0 = tok_of(c);
    const int h = (c / NT) % H;
    const int vbc = min(vb, NVB - 1);
    dst = *(const u32x4*)(v + (t0 + (tid >> 3)) * hv + (size_t)h * V + 64 * vbc + 8 * (tid & 7));
  };
  fetch_qk(ci);
  fetch_v(ci, 0, pv[0]);
  fetch_v(ci, 1, pv[1]);

  for (; ci < nchunks; ci += gridDim.x) {
    const int row = ci / NT, ic = ci % NT;
    const int h = row % H;
    const size_t tok0 = tok_of(ci);
    const int nxt = min(ci + (int)gridDim.x, nchunks - 1);

    // ---- stage the chunk -------------------------------------------------------------
#pragma unroll
    for (int i = 0; i < QU; ++i) {
      const int u = tid + NTH * i, r = u / UPR, cc = 8 * (u % UPR);
      *(u32x4*)(s.q + r * LK + cc) = pq[i];
      *(u32x4*)(s.k + r * LK + cc) = pk[i];
    }
    if (w == 0) {
      float x = pg;
      if constexpr (MODE == kPrepFwd) {
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const float y = __shfl_up(x, d, 64);
          if (lane >= d) x += y;
        }
        gcum[(tok0 + lane) * H + h] = x;
      }
      s.gc[lane] = x;
    } else if (w == 1) {
      s.beta[lane] = pb;
    }
    if (tid < 7 * kGC) s.lam[tid % 7][tid / 7] = pl;
    __syncthreads();
    fetch_qk(nxt);
    if (norm_qk) {
      // use_qk_l2norm_in_kernel (kernel.py:110-111): k / ||k|| and q scale / ||q||
      if (tid < 256) l2norm_rows<KD, LK>(s.k, 1.f, nullptr);
      else l2norm_rows<KD, LK, 256>(s.q, qk_scale, nullptr);
      __syncthreads();
    }

    // ---- K K^T (-> A, fp32) and Q K^T (-> M, bf16): wave w owns rows t-tile tt,
    // column tiles 2wh, 2wh + 1 -------------------------------------------------------
    {
      floatx4 kk[2], qk[2];
#pragma unroll
      for (int n = 0; n < 2; ++n) kk[n] = qk[n] = zero4();
#pragma unroll
      for (int c = 0; c < KD / 32; ++c) {
        const bf16x8 ak = *(const bf16x8*)(s.k + (16 * tt + ln) * LK + 32 * c + 8 * lq);
        const bf16x8 aq = *(const bf16x8*)(s.q + (16 * tt + ln) * LK + 32 * c + 8 * lq);
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const int nt = 2 * wh + n;
          const bf16x8 bk = *(const bf16x8*)(s.k + (16 * nt + ln) * LK + 32 * c + 8 * lq);
          kk[n] = mfma16x16x32(ak, bk, kk[n]);
          qk[n] = mfma16x16x32(aq, bk, qk[n]);
        }
      }
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * tt + 4 * lq + i, sc = 16 * (2 * wh + n) + ln;
          A[t * kLM + sc] = sc < t ? s.beta[t] * kk[n][i] : 0.f;
          s.mq[t * kLd64 + sc] = (__bf16)(sc <= t ? qk[n][i] : 0.f);
        }
    }
    __syncthreads();

    // ---- X = (I + A)^-1, fp32 ------------------------------------------------------
    tri_inv64_mfma<NTH>(A, X, s.wt.inv);

    // ---- Aw, Au (bf16) to LDS and to the outputs --------------------------------------
    {
      const int t = tid >> 3, s0 = 8 * (tid & 7);
      bf16x8 a, au;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int sc = s0 + j;
        const float x = sc <= t ? X[t * kLM + sc] : 0.f;
        a[j] = (__bf16)x;
        au[j] = (__bf16)(sc <= t ? x * fexp(s.gc[t] - s.gc[sc]) : 0.f);
      }
      *(bf16x8*)(s.aw + t * kLd64 + s0) = a;
      *(bf16x8*)(s.au + t * kLd64 + s0) = au;
      if constexpr (MODE == kPrepFwd) {
        *(bf16x8*)(aw_out + ((tok0 + t) * H + h) * kGC + s0) = a;
        *(bf16x8*)(au_out + ((tok0 + t) * H + h) * kGC + s0) = au;
      }
    }
    __syncthreads();

    // Transposed products: D^T = B^T A^T, so lane (lq, ln) of a 16 x 16 tile ends
    // with row t = 16 tt + ln, columns 4 lq .. 4 lq + 3 of the product.  The B
    // operand is always a row block of a 64 x 64 bf16 matrix X[t][s] (rows of
    // t-tile tt, contraction over s).
    auto rows_frag = [&](const __bf16* Xm, int c) __attribute__((always_inline)) {
      return *(const bf16x8*)(Xm + (16 * tt + ln) * kLd64 + 32 * c + 8 * lq);
    };
    const int t = 16 * tt + ln;
    const float egt = fexp(s.gc[t]);

    // ---- P = (M Aw) o gamma o beta_s o lambda[t, lev(t, s)] (bf16 output) -------------
    if constexpr (MODE == kPrepFwd) {
      const bf16x8 bm0 = rows_frag(s.mq, 0), bm1 = rows_frag(s.mq, 1);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int st = 2 * wh + j;
        floatx4 d = mfma16x16x32(tr_frag(s.aw, kLd64, 0, 16 * st), bm0, zero4());
        d = mfma16x16x32(tr_frag(s.aw, kLd64, 32, 16 * st), bm1, d);
        bf16x4 pb4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int sc = 16 * st + 4 * lq + i;
          float x = 0.f;
          if (sc <= t)
            x = d[i] * fexp(s.gc[t] - s.gc[sc]) * s.beta[sc] * s.lam[intra_level(t, sc)][t];
          pb4[i] = (__bf16)x;
        }
        *(bf16x4*)(pm + (((size_t)row * NT + ic) * kGC + t) * kGC + 16 * st + 4 * lq) = pb4;
      }
    }

    // ---- per 64-column block of K: W -> W_new, q_new, K_new -------------------------
    const bf16x8 ba0 = rows_frag(s.aw, 0), ba1 = rows_frag(s.aw, 1);
    const bf16x8 bq0 = rows_frag(s.mq, 0), bq1 = rows_frag(s.mq, 1);
    const float egl = s.gc[kGC - 1];
#pragma unroll 1
    for (int cb = 0; cb < KD / 64; ++cb) {
      // W^T tile (column tile ct, t-tile tt): A[m = col][s] = beta_s K[s][col]
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ct = 2 * wh + j;
        floatx4 d = zero4();
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          bf16x8 a = tr_frag(s.k, LK, 32 * c, 64 * cb + 16 * ct);
          const floatx4 b0 = *(const floatx4*)(s.beta + 32 * c + 8 * lq);
          const floatx4 b1 = *(const floatx4*)(s.beta + 32 * c + 8 * lq + 4);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            a[jj] = (__bf16)((float)a[jj] * b0[jj]);
            a[4 + jj] = (__bf16)((float)a[4 + jj] * b1[jj]);
          }
          d = mfma16x16x32(a, c ? ba1 : ba0, d);
        }
        const int col = 16 * ct + 4 * lq;
        *(bf16x4*)(s.wt.w + t * kLd64 + col) = cvt4(d);
        floatx4 dw = d;
#pragma unroll
        for (int i = 0; i < 4; ++i) dw[i] *= egt;
        *(bf16x4*)(wn + ((tok0 + t) * H + h) * KD + 64 * cb + col) = cvt4(dw);
      }
      // K_new = exp(Gc_last - Gc_t) K: transposed per chunk (thread: column tid >> 3,
      // tokens 8 (tid & 7) .. +7), and token-major for the backward
      {
        const int col = tid >> 3, t8 = 8 * (tid & 7);
        bf16x8 x;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          x[j] = (__bf16)((float)s.k[(t8 + j) * LK + 64 * cb + col] * fexp(egl - s.gc[t8 + j]));
        *(bf16x8*)(knT + (((size_t)row * NT + ic) * KD + 64 * cb + col) * kGC + t8) = x;
        if constexpr (MODE == kPrepRecompute) {
          const int tr = tid >> 3, c8 = 8 * (tid & 7);
          const float ek = fexp(egl - s.gc[tr]);
          const bf16x8 kx = *(const bf16x8*)(s.k + tr * LK + 64 * cb + c8);
          bf16x8 kb;
#pragma unroll
          for (int j = 0; j < 8; ++j) kb[j] = (__bf16)((float)kx[j] * ek);
          *(bf16x8*)(kn + ((tok0 + tr) * H + h) * KD + 64 * cb + c8) = kb;
        }
      }
      __syncthreads();
      // q_new^T tile: A[m = col][s] = W[s][col]
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ct = 2 * wh + j;
        floatx4 d = mfma16x16x32(tr_frag(s.wt.w, kLd64, 0, 16 * ct), bq0, zero4());
        d = mfma16x16x32(tr_frag(s.wt.w, kLd64, 32, 16 * ct), bq1, d);
        const int col = 16 * ct + 4 * lq;
        const bf16x4 qx = *(const bf16x4*)(s.q + t * LK + 64 * cb + col);
        floatx4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = egt * ((float)qx[i] - d[i]);
        *(bf16x4*)(qn + ((tok0 + t) * H + h) * KD + 64 * cb + col) = cvt4(r);
      }
      __syncthreads();
    }

    // ---- per 64-column block of V: U = Au (beta V) ------------------------------------
    const bf16x8 bu0 = rows_frag(s.au, 0), bu1 = rows_frag(s.au, 1);
#pragma unroll 1
    for (int vb = 0; vb < NVB; ++vb) {
      u32x4 x;
      if (vb < 2) {
        x = pv[vb & 1];
      } else {
        fetch_v(ci, vb, x);
      }
      *(u32x4*)(s.v + (tid >> 3) * kLd64 + 8 * (tid & 7)) = x;
      if (vb < 2) fetch_v(nxt, vb, pv[vb & 1]);
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ct = 2 * wh + j;
        floatx4 d = zero4();
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          bf16x8 a = tr_frag(s.v, kLd64, 32 * c, 16 * ct);
          const floatx4 b0 = *(const floatx4*)(s.beta + 32 * c + 8 * lq);
          const floatx4 b1 = *(const floatx4*)(s.beta + 32 * c + 8 * lq + 4);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            a[jj] = (__bf16)((float)a[jj] * b0[jj]);
            a[4 + jj] = (__bf16)((float)a[4 + jj] * b1[jj]);
          }
          d = mfma16x16x32(a, c ? bu1 : bu0, d);
        }
        *(bf16x4*)(un + ((tok0 + t) * H + h) * V + 64 * vb + 16 * ct + 4 * lq) = cvt4(d);
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// level scan
// ---------------------------------------------------------------------------
template <int KD, int BV>
struct GdnScanCfg {
  static constexpr int NVT = BV / 16;                 // 16-column v-tiles
  static constexpr int MT = KD / 64;                  // 16-row k-tiles of one k-quarter
  static constexpr int NC = KD / 32;                  // MFMA steps of a contraction over K
  static constexpr int LPG = kGMaxLev / 2;            // levels per level group
  static constexpr int LK = KD + 8;                   // row stride of the staged states
  static constexpr int LVS = BV + 8;                  // row stride of the staged V and U slices
  static constexpr int KU = KD / 64;                  // 16-byte units of K_new^T per thread
};

template <int KD, int BV>
struct GdnScanSmem {
  using C = GdnScanCfg<KD, BV>;
  __bf16 hs[kGMaxLev][BV * C::LK];    // states, bf16 [v][k]
  __bf16 vn[kGMaxLev][BV * kLd64];    // V_new, bf16 [v][t]
  __bf16 kb[KD * kGC];                // the chunk's K_new^T [k][t] (swz64)
  __bf16 pm[kGC * kGC];               // the chunk's P [t][s] (swz64)
  __bf16 vs[kGC * C::LVS];            // the chunk's V slice [t][v] (o_intra)
  __bf16 us[kGC * C::LVS];            // the chunk's U slice [t][v] (V_new)
  float lam[kGMaxLev][kGC];           // lambda[t, 7 + e], zero for e >= nlev
  floatx4 xacc[4][C::NVT][64];        // level group 1's reads, summed into group 0's
};

// Element offset of 16-byte unit u of row r in a [rows][64] bf16 tile whose
// units are XOR-permuted by the row: the 16-byte row-fragment reads of the
// MFMA operands (16 rows, one unit each) hit distinct banks.
__device__ __forceinline__ int swz64(int r, int u) { return r * 64 + ((u ^ r) & 7) * 8; }

// Eight waves in two level groups: wave w runs levels 4 (w >> 2) .. +3 with
// q = w & 3 as its t-tile (the products W_new h_e and q_new h_e, which share
// each B fragment) and as its k-quarter (the state rows it holds and updates).
// All levels of a group run every chunk without a branch per level, so the
// compiler interleaves their LDS reads and MFMA chains; a level e >= nlev
// never writes (its V_new is zero, so its state stays zero) and is never read
// (lambda is zero for it, bit e of the chunk index is clear).
// Operand pipeline: the loads of chunk ic + 1 are issued right after the
// level products of chunk ic, small operands first, and land in LDS at the
// start of chunk ic + 1 (K_new^T, read only by the state update, right after
// the first barrier), so no wave waits for memory inside a chunk.  The K_new^T,
// P, V and U tiles are loaded once per workgroup (one 16-byte unit per thread
// and tile) instead of once per wave.
// HSAVE (the backward's recompute): every level's state at every chunk start
// is written to hsave, bf16 [row][chunk][level][v][k]; then o may be null and
// pm any valid pointer.  A separate instantiation, so the forward carries no
// registers for it.
template <int KD, int BV, typename TL, typename TO, bool HSAVE>
__global__ __launch_bounds__(512) void gdn_scan_kernel(
    const __bf16* __restrict__ qn, const __bf16* __restrict__ wn, const __bf16* __restrict__ knT,
    const __bf16* __restrict__ un, const __bf16* __restrict__ pm, const __bf16* __restrict__ vin,
    const float* __restrict__ gcum, const TL* __restrict__ l, TO* __restrict__ o,
    float* __restrict__ ht, __bf16* __restrict__ hsave, int nrows, int T, int H, int V, int L,
    int nlev, int final_state) {
  using C = GdnScanCfg<KD, BV>;
  using Sm = GdnScanSmem<KD, BV>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Sm& s = *(Sm*)smem_raw;
  constexpr int LK = C::LK, LVS = C::LVS, NVT = C::NVT, MT = C::MT, NC = C::NC, LPG = C::LPG;
  constexpr int KU = C::KU;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int nvb = V / BV;
  const XcdMap mp = xcd_map(blockIdx.x, nvb);
  if (mp.row >= nrows) return;
  const int row = mp.row, v0 = mp.slice * BV;
  const int b = row / H, h = row % H;
  const int NT = T / kGC;
  const size_t rowtok = (size_t)b * T * H + h;   // (token 0 of the row) * H + h
  const int lg = w >> 2, q = w & 3, e0 = LPG * lg;

  // states: level e0 + le, rows k = 16 (MT q + m) + 4 lq + i, columns v = 16 n + ln
  floatx4 st[LPG][MT][NVT];
#pragma unroll
  for (int le = 0; le < LPG; ++le)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < NVT; ++n) st[le][m][n] = zero4();
  for (int i = tid; i < kGMaxLev * kGC; i += 512) s.lam[i / kGC][i % kGC] = 0.f;

  // Operand loads: a uniform per-row base plus a 32-bit lane offset, advanced
  // by a uniform per-chunk offset.  Every load is unconditional, so the
  // compiler does not wait for it at a branch.
  const unsigned HV = (unsigned)H * V, HK = (unsigned)H * KD, HL = (unsigned)H * L;
  const __bf16* qrow = qn + rowtok * KD;
  const __bf16* wrow = wn + rowtok * KD;
  const unsigned a_off = (16 * q + ln) * HK + 8 * lq;
  const __bf16* knrow = knT + (size_t)row * NT * KD * kGC;
  const __bf16* pmrow = pm + (size_t)row * NT * kGC * kGC;
  const unsigned u_off = (16 * q + 4 * lq) * HV + ln;   // o[t = 16q + 4lq + i][v = 16n + ln]
  // V slice (threads 0 .. 8 BV - 1) and U slice (8 BV .. 16 BV - 1): one
  // 16-byte unit of the [64 x BV] tile each; threads past 16 BV repeat the
  // last unit and do not store it
  const bool s_store = tid < 16 * BV;
  const int su = s_store ? tid : 16 * BV - 1;
  const bool is_u = su >= 8 * BV;
  const int vu = is_u ? su - 8 * BV : su;
  const __bf16* sbase = (is_u ? un : vin) + rowtok * V + v0;
  const unsigned s_off = (vu / (BV / 8)) * HV + 8 * (vu % (BV / 8));
  __bf16* sdst = (is_u ? s.us : s.vs) + (vu / (BV / 8)) * LVS + 8 * (vu % (BV / 8));
  const int nl1 = nlev > 0 ? nlev : 1;   // T = 64 has no inter-chunk level
  const int e2 = min(tid, nl1 * kGC - 1);
  const TL* lrow = l + rowtok * L;
  const unsigned l_off = (e2 / nl1) * HL + min(7 + e2 % nl1, L - 1);
  // Gc_last through a buffer (vector-memory) load: a scalar load would share the
  // LDS wait counter and stall every LDS wait until it returns
  const rsrc_t grs = make_rsrc(gcum + rowtok + (size_t)(kGC - 1) * H, (size_t)T * H * 4);
  __bf16* hrow = HSAVE ? hsave + (size_t)row * NT * nlev * V * KD + (size_t)v0 * KD : nullptr;
  const unsigned h_off = ln * KD + 16 * MT * q + 4 * lq;

  u32x4 aq[NC], aw[NC], kfn[KU], pvu, pp1;
  TL plr;
  float pgl;
  auto load_a = [&](int jc) __attribute__((always_inline)) {
    const size_t off = (size_t)jc * kGC * HK;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      aq[c] = *(const u32x4*)(qrow + off + a_off + 32 * c);
      aw[c] = *(const u32x4*)(wrow + off + a_off + 32 * c);
    }
  };
  auto load_k = [&](int jc) __attribute__((always_inline)) {
    const __bf16* base = knrow + (size_t)jc * KD * kGC;
#pragma unroll
    for (int r = 0; r < KU; ++r) kfn[r] = *(const u32x4*)(base + 8 * (tid + 512 * r));
  };
  auto fetch_small = [&](int jc) __attribute__((always_inline)) {
    const size_t tokoff = (size_t)jc * kGC * H;   // chunk jc's first token, times H
    pvu = *(const u32x4*)(sbase + tokoff * V + s_off);
    if constexpr (!HSAVE) pp1 = *(const u32x4*)(pmrow + (size_t)jc * kGC * kGC + 8 * tid);
    plr = lrow[tokoff * L + l_off];
    pgl = buf_load<float>(grs, 0, (unsigned)(tokoff * 4));
  };
  fetch_small(0);
  load_k(0);
  load_a(0);

  for (int ic = 0; ic < NT; ++ic) {
    const int icn = min(ic + 1, NT - 1);
    const float glast = pgl;
    // states -> LDS (bf16 [v][k]) and, with hsave, to hsave[row][chunk][level][v][k]
#pragma unroll
    for (int le = 0; le < LPG; ++le)
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < NVT; ++n) {
          const bf16x4 h4 = cvt4(st[le][m][n]);
          const int kk = 16 * (MT * q + m) + 4 * lq, vv = 16 * n + ln;
          *(bf16x4*)(s.hs[e0 + le] + vv * LK + kk) = h4;
          if (HSAVE && e0 + le < nlev)
            *(bf16x4*)(hrow + ((size_t)ic * nlev + e0 + le) * V * KD + h_off + (16 * n * KD + 16 * m)) = h4;
        }
    // the chunk's lambda, V and U slices and P -> LDS
    if (tid < nlev * kGC) s.lam[tid % nlev][tid / nlev] = to_f32<TL>(plr);
    if (s_store) *(u32x4*)sdst = pvu;
    if constexpr (!HSAVE) *(u32x4*)(s.pm + swz64(tid >> 3, tid & 7)) = pp1;
    __syncthreads();
    // the chunk's K_new^T -> LDS: every wave is past the previous chunk's state
    // update, and the second barrier orders these stores before this chunk's
#pragma unroll
    for (int r = 0; r < KU; ++r) {
      const int u = tid + 512 * r;
      *(u32x4*)(s.kb + swz64(u >> 3, u & 7)) = kfn[r];
    }

    // ---- V_new_e = (write ? U : 0) - (reset ? 0 : W_new h_e) -> LDS, and the reads
    //      lambda_e o (q_new h_e) of the levels with bit e of ic set.  The level's
    //      flags enter as 0 / 1 factors.
    const bool last = ic == NT - 1;
    float uu[NVT][4];
#pragma unroll
    for (int n = 0; n < NVT; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) uu[n][i] = (float)s.us[(16 * q + 4 * lq + i) * LVS + 16 * n + ln];
    floatx4 acc[NVT];
#pragma unroll
    for (int n = 0; n < NVT; ++n) acc[n] = zero4();
#pragma unroll
    for (int le = 0; le < LPG; ++le) {
      const int e = e0 + le;
      const int per = 2 << e;
      const bool rd = (ic >> e) & 1;
      const float frd = rd ? 1.f : 0.f;
      const float fwr = (e < nlev && !rd) ? 1.f : 0.f;
      const float fkeep = (((ic & (per - 1)) == per - 1) && !(last && final_state)) ? 0.f : 1.f;
      const floatx4 lam4 = *(const floatx4*)(&s.lam[e][16 * q + 4 * lq]);
#pragma unroll
      for (int n = 0; n < NVT; ++n) {
        floatx4 y = zero4(), z = zero4();
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const bf16x8 bh = *(const bf16x8*)(s.hs[e] + (16 * n + ln) * LK + 32 * c + 8 * lq);
          y = mfma16x16x32(__builtin_bit_cast(bf16x8, aw[c]), bh, y);
          z = mfma16x16x32(__builtin_bit_cast(bf16x8, aq[c]), bh, z);
        }
        bf16x4 vb4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          vb4[i] = (__bf16)(fwr * uu[n][i] - fkeep * y[i]);
          acc[n][i] += frd * lam4[i] * z[i];
        }
        *(bf16x4*)(s.vn[e] + (16 * n + ln) * kLd64 + 16 * q + 4 * lq) = vb4;
      }
      // bound the scheduler's hoisting of the next level's LDS reads (register
      // pressure)
      __builtin_amdgcn_sched_barrier(0);
    }
    // chunk ic + 1's operands: the ones needed first are issued first (the
    // wait counter is in order)
    fetch_small(icn);
    load_k(icn);
    load_a(icn);
    if (lg == 1) {
#pragma unroll
      for (int n = 0; n < NVT; ++n) s.xacc[q][n][lane] = acc[n];
    } else if (o != nullptr) {
      // o_intra = P V
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const bf16x8 pf = *(const bf16x8*)(s.pm + swz64(16 * q + ln, lq + 4 * c));
#pragma unroll
        for (int n = 0; n < NVT; ++n)
          acc[n] = mfma16x16x32(pf, tr_frag(s.vs, LVS, 32 * c, 16 * n), acc[n]);
      }
    }
    __syncthreads();

    // ---- group 0: o = o_intra + reads of both groups --------------------------------
    if (lg == 0 && o != nullptr) {
      TO* ob = o + (rowtok + (size_t)ic * kGC * H) * V + v0;
#pragma unroll
      for (int n = 0; n < NVT; ++n) {
        const floatx4 x = acc[n] + s.xacc[q][n][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) ob[u_off + i * HV + 16 * n] = from_f32<TO>(x[i]);
      }
    }

    // ---- h_e = (reset ? 0 : exp(Gc_last) h_e) + K_new^T V_new_e -----------------------
    const float gl = fexp(glast);
    bf16x8 kf[MT][2];   // K_new^T[k = 16 (MT q + m) + ln][t = 32 c + 8 lq ..]
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        kf[m][c] = *(const bf16x8*)(s.kb + swz64(16 * (MT * q + m) + ln, lq + 4 * c));
#pragma unroll
    for (int le = 0; le < LPG; ++le) {
      const int e = e0 + le;
      const int per = 2 << e;
      const bool reset = ((ic & (per - 1)) == per - 1) && !(last && final_state);
      const float gk = reset ? 0.f : gl;
#pragma unroll
      for (int n = 0; n < NVT; ++n) {
        const bf16x8 b0 = *(const bf16x8*)(s.vn[e] + (16 * n + ln) * kLd64 + 8 * lq);
        const bf16x8 b1 = *(const bf16x8*)(s.vn[e] + (16 * n + ln) * kLd64 + 32 + 8 * lq);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          floatx4 x = st[le][m][n];
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] *= gk;
          x = mfma16x16x32(kf[m][0], b0, x);
          x = mfma16x16x32(kf[m][1], b1, x);
          st[le][m][n] = x;
        }
      }
      if (le & 1) __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (final_state && ht != nullptr) {
    // ht[b, h, k, v, 7 + e] (chunkwise_hgdn.py:786-787)
    float* hb = ht + (size_t)row * KD * V * L + v0 * L + 7 + e0;
    const unsigned VL = (unsigned)V * L;
    const unsigned t_off = (16 * MT * q + 4 * lq) * VL + ln * L;
#pragma unroll
    for (int le = 0; le < LPG; ++le)
      if (e0 + le < nlev)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int n = 0; n < NVT; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              hb[t_off + (16 * m + i) * VL + 16 * n * L + le] = st[le][m][n][i];
  }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
struct GdnWs {
  __bf16 *qn, *wn, *knT, *un, *pm;
  size_t bytes;
};

inline size_t galign(size_t x) { return (x + 255) & ~(size_t)255; }

inline GdnWs gdn_ws_layout(void* base, int B, int T, int H, int K, int V) {
  GdnWs w;
  char* p = (char*)base;
  size_t off = 0;
  const size_t n = (size_t)B * T * H;
  w.qn = (__bf16*)(p + off); off += galign(n * K * 2);
  w.wn = (__bf16*)(p + off); off += galign(n * K * 2);
  w.knT = (__bf16*)(p + off); off += galign(n * K * 2);
  w.un = (__bf16*)(p + off); off += galign(n * V * 2);
  w.pm = (__bf16*)(p + off); off += galign(n * kGC * 2);
  w.bytes = off;
  return w;
}

// V columns per scan workgroup (K >= 192: 16, so that the states of four levels of a
// k-quarter and the A operands fit the registers of two waves per SIMD).
template <int KD> struct ScanBV { static constexpr int value = KD >= 192 ? 16 : 32; };

inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

template <int KD, typename TB, typename TL, int MODE>
static hipError_t gdn_prep_launch_t(const void* q, const void* k, const void* v, const void* beta,
                                    const float* g, const void* l, float* gcum, void* aw, void* au,
                                    __bf16* qn, __bf16* wn, __bf16* kn, __bf16* knT, __bf16* un,
                                    __bf16* pm, int B, int T, int H, int V, int L, int norm_qk,
                                    float scale, hipStream_t stream) {
  auto kp = gdn_prep_kernel<KD, TB, TL, MODE>;
  const int smem = (int)sizeof(GdnPrepSmem<KD>);
  hipError_t e;
  if ((e = hipFuncSetAttribute((const void*)kp, hipFuncAttributeMaxDynamicSharedMemorySize,
                               smem)) != hipSuccess)
    return e;
  const int nchunks = B * H * (T / kGC);
  const int per_cu = max(1, (160 * 1024) / smem);
  const int grid = min(nchunks, device_cus() * per_cu);
  hipLaunchKernelGGL(kp, dim3(grid), dim3(kPrepThreads), smem, stream, (const __bf16*)q,
                     (const __bf16*)k, (const __bf16*)v, (const TB*)beta, g, (const TL*)l, gcum,
                     (__bf16*)aw, (__bf16*)au, qn, wn, kn, knT, un, pm, nchunks, T, H, V, L,
                     norm_qk, scale);
  return hipGetLastError();
}

template <int KD, typename TL, typename TO>
static hipError_t gdn_scan_launch_t(const GdnWs& w, const void* v, const float* gcum,
                                    const void* l, void* o, float* ht, __bf16* hsave, int B,
                                    int T, int H, int V, int L, int nlev, int final_state,
                                    hipStream_t stream) {
  constexpr int BV = ScanBV<KD>::value;
  auto ks = hsave ? gdn_scan_kernel<KD, BV, TL, TO, true> : gdn_scan_kernel<KD, BV, TL, TO, false>;
  const int smem = (int)sizeof(GdnScanSmem<KD, BV>);
  hipError_t e;
  if ((e = hipFuncSetAttribute((const void*)ks, hipFuncAttributeMaxDynamicSharedMemorySize,
                               smem)) != hipSuccess)
    return e;
  const int rows = B * H;
  const int grid = (rows + 7) / 8 * 8 * (V / BV);
  hipLaunchKernelGGL(ks, dim3(grid), dim3(512), smem, stream, w.qn, w.wn, w.knT, w.un, w.pm,
                     (const __bf16*)v, gcum, (const TL*)l, (TO*)o, ht, hsave, rows, T, H, V, L,
                     nlev, final_state);
  return hipGetLastError();
}

template <int KD, typename TB, typename TL, typename TO>
static hipError_t gdn_launch_t(const void* q, const void* k, const void* v, const void* beta,
                               const float* g, const void* l, void* o, float* gcum, void* aw,
                               void* au, float* ht, void* ws, int B, int T, int H, int V, int L,
                               int nlev, int norm_qk, float scale, hipStream_t stream) {
  const GdnWs w = gdn_ws_layout(ws, B, T, H, KD, V);
  hipError_t e = gdn_prep_launch_t<KD, TB, TL, kPrepFwd>(
      q, k, v, beta, g, l, gcum, aw, au, w.qn, w.wn, nullptr, w.knT, w.un, w.pm, B, T, H, V, L,
      norm_qk, scale, stream);
  if (e != hipSuccess) return e;
  return gdn_scan_launch_t<KD, TL, TO>(w, v, gcum, l, o, ht, nullptr, B, T, H, V, L, nlev,
                                       ht != nullptr ? 1 : 0, stream);
}

}  // namespace hattn

size_t hattn_gdn_fwd_ws_bytes(int B, int T, int H, int K, int V) {
  return hattn::gdn_ws_layout(nullptr, B, T, H, K, V).bytes;
}

int hattn_gdn_fwd_max_levels() { return hattn::kGMaxLev; }

// K values with a forward instantiation (V: any multiple of 64).
int hattn_gdn_fwd_supports_k(int K) { return K == 64 || K == 128 || K == 192 || K == 256; }

hipError_t hattn_gdn_fwd_launch(const void* q, const void* k, const void* v, const void* beta,
                                const float* g, const void* l, void* o, float* gcum, void* aw,
                                void* au, float* ht, void* ws, int B, int T, int H, int K, int V,
                                int L, int nlev, int dt_b, int dt_l, int dt_o, int norm_qk,
                                float scale, hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
#define HATTN_GDN_DT(KD_, TB_, TL_)                                                             \
  return gdn_launch_t<KD_, TB_, TL_, __bf16>(q, k, v, beta, g, l, o, gcum, aw, au, ht, ws, B, T, \
                                             H, V, L, nlev, norm_qk, scale, stream);
#define HATTN_GDN(KD_)                                                                          \
  if (K == KD_ && dt_o == 0) {                                                                  \
    if (dt_b == 0 && dt_l == 0) HATTN_GDN_DT(KD_, __bf16, __bf16)                               \
    if (dt_b == 2 && dt_l == 2) HATTN_GDN_DT(KD_, float, float)                                 \
    if (dt_b == 0 && dt_l == 2) HATTN_GDN_DT(KD_, __bf16, float)                                \
    if (dt_b == 2 && dt_l == 0) HATTN_GDN_DT(KD_, float, __bf16)                                \
  }
  HATTN_GDN(64)
  HATTN_GDN(128)
  HATTN_GDN(192)
  HATTN_GDN(256)
#undef HATTN_GDN
#undef HATTN_GDN_DT
  *unsupported = 1;
  return hipSuccess;
}

// Forward recompute for the backward: q_new, K_new (token-major and per-chunk
// transposed), W_new, U from the chunk-local cumsum (prep kernel) and every
// level's per-chunk starting state, bf16 [row][chunk][level][v][k] (scan
// kernel, no output).
hipError_t hattn_gdn_recompute_launch(const void* q, const void* k, const void* v,
                                      const void* beta, const float* gcum, const void* l,
                                      __bf16* qn, __bf16* kn, __bf16* knT, __bf16* wn, __bf16* un,
                                      __bf16* hsave, int B, int T, int H, int K, int V, int L,
                                      int nlev, int dt_b, int dt_l, int norm_qk, float scale,
                                      hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  GdnWs w;
  w.qn = qn;
  w.wn = wn;
  w.knT = knT;
  w.un = un;
  w.pm = qn;   // read but unused without an output
#define HATTN_GDN_RC(KD_, TB_, TL_)                                                               \
  {                                                                                               \
    hipError_t e = gdn_prep_launch_t<KD_, TB_, TL_, kPrepRecompute>(                              \
        q, k, v, beta, gcum, l, nullptr, nullptr, nullptr, qn, wn, kn, knT, un, nullptr, B, T, H, \
        V, L, norm_qk, scale, stream);                                                            \
    if (e != hipSuccess) return e;                                                                \
    return gdn_scan_launch_t<KD_, TL_, __bf16>(w, v, gcum, l, nullptr, nullptr, hsave, B, T, H, V, \
                                               L, nlev, 0, stream);                               \
  }
#define HATTN_GDN_RC_D(KD_)                                                                      \
  if (K == KD_) {                                                                                \
    if (dt_b == 0 && dt_l == 0) HATTN_GDN_RC(KD_, __bf16, __bf16)                                \
    if (dt_b == 2 && dt_l == 2) HATTN_GDN_RC(KD_, float, float)                                  \
    if (dt_b == 0 && dt_l == 2) HATTN_GDN_RC(KD_, __bf16, float)                                 \
    if (dt_b == 2 && dt_l == 0) HATTN_GDN_RC(KD_, float, __bf16)                                 \
  }
  HATTN_GDN_RC_D(64)
  HATTN_GDN_RC_D(128)
  HATTN_GDN_RC_D(192)
#undef HATTN_GDN_RC_D
#undef HATTN_GDN_RC
  *unsupported = 1;
  return hipSuccess;
}
