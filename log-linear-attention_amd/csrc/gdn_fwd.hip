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
// Kernel 2 (gdn_scan_kernel): one workgroup per (row, BV columns of V), one
// wave per inter-chunk level.  Each wave keeps its level's [K x BV] state in
// fp32 registers and runs the level's recurrence on its own (the products take
// the state and V_new as B operands straight from the accumulators, with the
// A operands' contraction index permuted to match), so the waves meet only to
// share the chunk's operands (staged in LDS from registers loaded during the
// previous chunk) and to sum the level reads into o.  The slices of one row
// run on one XCD, so the chunk tiles they share are fetched into one L2.
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
// MODE kPrepFwdKeep: the same, plus the token-major K_new, so that the
// backward can take q_new, W_new, K_new and U from the forward.
// MODE kPrepRecompute (the backward): g already holds the chunk-local cumsum
// (chunkwise_hgdn.py:799-817); outputs q_new, W_new, K_new (token-major and
// transposed) and U.
enum { kPrepFwd = 0, kPrepRecompute = 1, kPrepFwdKeep = 2 };

// STRONG: the P tile takes lambda at the strong level of each pair (the
// reference's HType.STRONG, chunkwise_hgdn.py:630); only P depends on it.
// E: the 16-bit format of q, k, v and of every stored intermediate (bf16, or
// fp16 for fp16 inputs: fp16 MFMA, as the reference's fp16 dots).
template <int KD, typename TB, typename TL, int MODE, bool STRONG = false, typename E = __bf16>
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
  // the chunk-local cumsum of g is written by wave 0; the other waves store
  // through an empty range, so the store (like every load) is unconditional and
  // the compiler can count the memory operations in flight
  constexpr bool kFwd = MODE != kPrepRecompute;
  const rsrc_t rgc = make_rsrc(gcum, kFwd && w == 0 ? (size_t)nchunks * kGC * 4 : 0);

  // ---- stage a chunk: Q, K (l2-normalised on request), the cumsum of g, beta,
  //      lambda -> LDS.  Called before the walk and at the end of each chunk.
  //      The next chunk's loads are issued after the K K^T barrier of the
  //      current one: issued here, right behind the previous chunk's output
  //      stores, they queue in the CU's memory pipeline until those drain.
  auto stage = [&](int c) __attribute__((always_inline)) {
    const int hs = (c / NT) % H;
    const size_t t0 = tok_of(c);
#pragma unroll
    for (int i = 0; i < QU; ++i) {
      const int u = tid + NTH * i, r = u / UPR, cc = 8 * (u % UPR);
      *(u32x4*)(s.q + r * LK + cc) = pq[i];
      *(u32x4*)(s.k + r * LK + cc) = pk[i];
    }
    float x = pg;
    if constexpr (kFwd) {
      x = chunk_cumsum(x);
      buf_store<float>(x, rgc, (unsigned int)(lane * H * 4), (unsigned int)((t0 * H + hs) * 4));
    }
    if (w == 0) s.gc[lane] = x;
    if (w == 1) s.beta[lane] = pb;
    if (tid < 7 * kGC) s.lam[tid % 7][tid / 7] = pl;
    __syncthreads();
    if (norm_qk) {
      // use_qk_l2norm_in_kernel (kernel.py:110-111): k / ||k|| and q scale / ||q||
      if (tid < 256) l2norm_rows<KD, LK, 0, E>(s.k, 1.f, nullptr);
      else l2norm_rows<KD, LK, 256, E>(s.q, qk_scale, nullptr);
      __syncthreads();
    }
  };
  stage(ci);

  for (;;) {
    const int row = ci / NT, ic = ci % NT;
    const int h = row % H;
    const size_t tok0 = tok_of(ci);
    const int nxt = min(ci + (int)gridDim.x, nchunks - 1);

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
          kk[n] = mfma16<E>(ak, bk, kk[n]);
          qk[n] = mfma16<E>(aq, bk, qk[n]);
        }
      }
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * tt + 4 * lq + i, sc = 16 * (2 * wh + n) + ln;
          A[t * kLM + sc] = sc < t ? s.beta[t] * kk[n][i] : 0.f;
          s.mq[t * kLd64 + sc] = to16<E>(sc <= t ? qk[n][i] : 0.f);
        }
    }
    __syncthreads();
    fetch_qk(nxt);   // the next chunk's Q, K, g, beta, lambda (staged at the end)

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
        a[j] = to16<E>(x);
        au[j] = to16<E>(sc <= t ? x * fexp(s.gc[t] - s.gc[sc]) : 0.f);
      }
      *(bf16x8*)(s.aw + t * kLd64 + s0) = a;
      *(bf16x8*)(s.au + t * kLd64 + s0) = au;
      if constexpr (kFwd) {
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
    if constexpr (kFwd) {
      const bf16x8 bm0 = rows_frag(s.mq, 0), bm1 = rows_frag(s.mq, 1);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int st = 2 * wh + j;
        floatx4 d = mfma16<E>(tr_frag(s.aw, kLd64, 0, 16 * st), bm0, zero4());
        d = mfma16<E>(tr_frag(s.aw, kLd64, 32, 16 * st), bm1, d);
        bf16x4 pb4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int sc = 16 * st + 4 * lq + i;
          float x = 0.f;
          if (sc <= t)
            x = d[i] * fexp(s.gc[t] - s.gc[sc]) * s.beta[sc] * s.lam[gdn_intra_level<STRONG>(t, sc)][t];
          pb4[i] = to16<E>(x);
        }
        *(bf16x4*)(pm + (((size_t)row * NT + ic) * kGC + t) * kGC + 16 * st + 4 * lq) = pb4;
      }
    }

    // ---- per 64-column block of K: W -> W_new, q_new, K_new -------------------------
    const bf16x8 ba0 = rows_frag(s.aw, 0), ba1 = rows_frag(s.aw, 1);
    const bf16x8 bq0 = rows_frag(s.mq, 0), bq1 = rows_frag(s.mq, 1);
    const float egl = s.gc[kGC - 1];
#pragma unroll
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
            a[jj] = to16<E>(from16<E>(a[jj]) * b0[jj]);
            a[4 + jj] = to16<E>(from16<E>(a[4 + jj]) * b1[jj]);
          }
          d = mfma16<E>(a, c ? ba1 : ba0, d);
        }
        const int col = 16 * ct + 4 * lq;
        *(bf16x4*)(s.wt.w + t * kLd64 + col) = cvt4e<E>(d);
        floatx4 dw = d;
#pragma unroll
        for (int i = 0; i < 4; ++i) dw[i] *= egt;
        *(bf16x4*)(wn + ((tok0 + t) * H + h) * KD + 64 * cb + col) = cvt4e<E>(dw);
      }
      // K_new = exp(Gc_last - Gc_t) K: transposed per chunk (thread: column tid >> 3,
      // tokens 8 (tid & 7) .. +7), and token-major for the backward
      {
        const int col = tid >> 3, t8 = 8 * (tid & 7);
        bf16x8 x;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          x[j] = to16<E>(from16<E>(s.k[(t8 + j) * LK + 64 * cb + col]) * fexp(egl - s.gc[t8 + j]));
        *(bf16x8*)(knT + (((size_t)row * NT + ic) * KD + 64 * cb + col) * kGC + t8) = x;
        if constexpr (MODE != kPrepFwd) {
          const int tr = tid >> 3, c8 = 8 * (tid & 7);
          const float ek = fexp(egl - s.gc[tr]);
          const bf16x8 kx = *(const bf16x8*)(s.k + tr * LK + 64 * cb + c8);
          bf16x8 kb;
#pragma unroll
          for (int j = 0; j < 8; ++j) kb[j] = to16<E>(from16<E>(kx[j]) * ek);
          *(bf16x8*)(kn + ((tok0 + tr) * H + h) * KD + 64 * cb + c8) = kb;
        }
      }
      __syncthreads();
      // q_new^T tile: A[m = col][s] = W[s][col]
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ct = 2 * wh + j;
        floatx4 d = mfma16<E>(tr_frag(s.wt.w, kLd64, 0, 16 * ct), bq0, zero4());
        d = mfma16<E>(tr_frag(s.wt.w, kLd64, 32, 16 * ct), bq1, d);
        const int col = 16 * ct + 4 * lq;
        const bf16x4 qx = *(const bf16x4*)(s.q + t * LK + 64 * cb + col);
        floatx4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = egt * (from16<E>(qx[i]) - d[i]);
        *(bf16x4*)(qn + ((tok0 + t) * H + h) * KD + 64 * cb + col) = cvt4e<E>(r);
      }
      __syncthreads();
    }

    // ---- per 64-column block of V: U = Au (beta V) ------------------------------------
    // blocks 0 and 1 come from the prefetch registers (their next-chunk loads are
    // issued unconditionally; with one block the second reloads block 0), later
    // blocks are loaded here
    const bf16x8 bu0 = rows_frag(s.au, 0), bu1 = rows_frag(s.au, 1);
    auto u_block = [&](int vb, const u32x4& x) __attribute__((always_inline)) {
      *(u32x4*)(s.v + (tid >> 3) * kLd64 + 8 * (tid & 7)) = x;
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
            a[jj] = to16<E>(from16<E>(a[jj]) * b0[jj]);
            a[4 + jj] = to16<E>(from16<E>(a[4 + jj]) * b1[jj]);
          }
          d = mfma16<E>(a, c ? bu1 : bu0, d);
        }
        *(bf16x4*)(un + ((tok0 + t) * H + h) * V + 64 * vb + 16 * ct + 4 * lq) = cvt4e<E>(d);
      }
      __syncthreads();
    };
    {
      const u32x4 x0 = pv[0], x1 = pv[1];
      fetch_v(nxt, 0, pv[0]);
      fetch_v(nxt, 1, pv[1]);
      u_block(0, x0);
      if (NVB > 1) u_block(1, x1);
    }
    for (int vb = 2; vb < NVB; ++vb) {
      u32x4 x;
      fetch_v(ci, vb, x);
      u_block(vb, x);
    }
    ci += gridDim.x;
    if (ci >= nchunks) break;
    stage(ci);
  }
}

// ---------------------------------------------------------------------------
// level scan
// ---------------------------------------------------------------------------
template <int KD, int BV>
struct GdnScanCfg {
  static constexpr int NVT = BV / 16;   // 16-column v-tiles
  static constexpr int NKT = KD / 16;   // 16-row k-tiles of the state
  static constexpr int NC = KD / 32;    // MFMA steps of a contraction over K
  static constexpr int LK = KD + 8;     // row stride of the staged W_new / q_new tiles
  static constexpr int LT = kGC + 8;    // row stride of the staged K_new^T, U^T and P tiles
  static constexpr int LVS = BV + 8;    // row stride of the staged V slice
  // row stride (floats) of the level-read partials (unpadded at K = 256, which
  // needs the LDS for its operand tiles)
  static constexpr int LP = KD >= 256 ? BV : BV + 4;
  static constexpr int KU = KD / 64;    // 16-byte units per thread of a [64 x KD] or [KD x 64] tile
};

template <int KD, int BV>
struct GdnScanSmem {
  using C = GdnScanCfg<KD, BV>;
  __bf16 wq[2][kGC * C::LK];             // the chunk's W_new, q_new [t][k]
  __bf16 kt[KD * C::LT];                 // K_new^T [k][t]
  __bf16 ut[BV * C::LT];                 // U slice, transposed [v][t]
  __bf16 pm[kGC * C::LT];                // P [t][s]
  __bf16 vs[kGC * C::LVS];               // V slice [t][v]
  float lam[kGMaxLev][kGC];              // lambda[t, 7 + e]
  float part[kGMaxLev + 1][kGC * C::LP]; // lambda_e o (q_new h_e) per level, o_intra last; [t][v]
};

// A-operand fragment whose contraction index runs in the row order of two
// stacked D tiles: lane (lq, ln) receives row r's elements c .. c + 3 and
// c + 16 .. c + 19 (c = 32 step + 4 lq).  Paired with a B fragment built from
// two D-layout accumulator quads (cat8), so states and V_new feed the next
// product straight from registers.
__device__ __forceinline__ bf16x8 frag_k2(const __bf16* X, int ld, int r, int c) {
  const bf16x4 lo = *(const bf16x4*)(X + r * ld + c);
  const bf16x4 hi = *(const bf16x4*)(X + r * ld + c + 16);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// One wave per inter-chunk level: wave e holds level e's whole [K x BV] state
// in fp32 registers (tile (kt, nt) holds rows 16 kt + 4 lq + i, columns
// 16 nt + ln) and runs its recurrence on its own,
//   R   = q_new h_e                         (chunks with bit e set: the level read)
//   V_new = (write ? U : 0) - W_new h_e     (not on the chunk that resets the level)
//   h_e = (reset ? 0 : exp(Gc_last) h_e) + K_new^T V_new,
// skipping the products of a zero state (the first chunk of a block) and of a
// chunk whose result the reset discards; a level e >= nlev does nothing.
// Wave 0 also forms o_intra = P V.  Per chunk the waves meet twice: the first
// barrier publishes the chunk's operands (staged in LDS from registers loaded
// during the previous chunk), the second the level reads, which every thread
// then sums for four outputs and stores.
// SMODE kScanOut: the forward (o).  kScanSave (the backward's recompute): every
// level's state at every chunk start is written to hsave, bf16
// [row][chunk][level][v][k]; no output (o, q_new, P and the V slice are not
// read).  kScanOutSave: both, for a forward whose backward takes the states
// from it.  Separate instantiations, so the plain forward carries no
// registers for the states' stores.
enum { kScanOut = 0, kScanSave = 1, kScanOutSave = 2 };
template <int KD, int BV, typename TL, typename TO, int SMODE, typename E = __bf16>
__global__ __launch_bounds__(512) void gdn_scan_kernel(
    const __bf16* __restrict__ qn, const __bf16* __restrict__ wn, const __bf16* __restrict__ knT,
    const __bf16* __restrict__ un, const __bf16* __restrict__ pm, const __bf16* __restrict__ vin,
    const float* __restrict__ gcum, const TL* __restrict__ l, TO* __restrict__ o,
    float* __restrict__ ht, __bf16* __restrict__ hsave, int nrows, int T, int H, int V, int L,
    int nlev, int final_state, int strong) {
  using C = GdnScanCfg<KD, BV>;
  using Sm = GdnScanSmem<KD, BV>;
  constexpr bool kSave = SMODE != kScanOut, kOut = SMODE != kScanSave;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Sm& s = *(Sm*)smem_raw;
  constexpr int NVT = C::NVT, NKT = C::NKT, NC = C::NC, LK = C::LK, LT = C::LT, LVS = C::LVS;
  constexpr int LP = C::LP, KU = C::KU;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int nvb = V / BV;
  const XcdMap mp = xcd_map(blockIdx.x, nvb);
  if (mp.row >= nrows) return;
  const int row = mp.row, v0 = mp.slice * BV;
  const int b = row / H, h = row % H;
  const int NT = T / kGC;
  const size_t rowtok = (size_t)b * T * H + h;   // (token 0 of the row) * H + h
  const int e = w;                               // this wave's level
  const bool act = e < nlev;

  floatx4 st[NKT][NVT];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int nt = 0; nt < NVT; ++nt) st[kt][nt] = zero4();
  for (int i = tid; i < kGMaxLev * kGC; i += 512) s.lam[i / kGC][i % kGC] = 0.f;

  // ---- staging loads: one 16-byte unit per thread and tile row piece; every
  //      load is unconditional (threads past a tile repeat its last unit and
  //      do not store it), so the compiler can count the loads in flight
  const unsigned HV = (unsigned)H * V, HK = (unsigned)H * KD, HL = (unsigned)H * L;
  const __bf16* wrow = wn + rowtok * KD;
  const __bf16* qrow = qn + rowtok * KD;
  const __bf16* knrow = knT + (size_t)row * NT * KD * kGC;
  const __bf16* pmrow = pm + (size_t)row * NT * kGC * kGC;
  unsigned wq_off[KU];   // element offset of unit tid + 512 r of a [64 x KD] token-major tile
  int wq_lds[KU];
#pragma unroll
  for (int r = 0; r < KU; ++r) {
    const int u = tid + 512 * r, t = u / (KD / 8), ku = u % (KD / 8);
    wq_off[r] = t * HK + 8 * ku;
    wq_lds[r] = t * LK + 8 * ku;
  }
  // V and U slices: thread tid < 16 BV stages 4 elements of each (token s_t,
  // columns s_v .. s_v + 3), so the transposing U writes are spread over every
  // wave (the others repeat the last unit and do not store it)
  const bool s_store = tid < 16 * BV;
  const int su = s_store ? tid : 16 * BV - 1;
  const int s_t = su / (BV / 4), s_v = 4 * (su % (BV / 4));
  const __bf16* vbase = vin + rowtok * V + v0;
  const __bf16* ubase = un + rowtok * V + v0;
  const unsigned s_off = s_t * HV + s_v;
  const int nl1 = nlev > 0 ? nlev : 1;   // T = 64 has no inter-chunk level
  const int e2 = min(tid, nl1 * kGC - 1);
  const TL* lrow = l + rowtok * L;
  const unsigned l_off = (e2 / nl1) * HL + min(7 + e2 % nl1, L - 1);
  // Gc_last through a buffer (vector-memory) load: a scalar load would share the
  // LDS wait counter and stall every LDS wait until it returns
  const rsrc_t grs = make_rsrc(gcum + rowtok + (size_t)(kGC - 1) * H, (size_t)T * H * 4);

  u32x4 rw[KU], rq[KU], rk[KU], rp;
  uint2 rsv, rsu;
  TL rl;
  float rg;
  auto stage_load = [&](int jc) __attribute__((always_inline)) {
    const size_t tokoff = (size_t)jc * kGC * H;   // chunk jc's first token, times H
    rsv = *(const uint2*)(vbase + tokoff * V + s_off);
    rsu = *(const uint2*)(ubase + tokoff * V + s_off);
    rl = lrow[tokoff * L + l_off];
    rg = buf_load<float>(grs, 0, (unsigned)(tokoff * 4));
#pragma unroll
    for (int r = 0; r < KU; ++r)
      rk[r] = *(const u32x4*)(knrow + (size_t)jc * KD * kGC + 8 * (tid + 512 * r));
#pragma unroll
    for (int r = 0; r < KU; ++r) rw[r] = *(const u32x4*)(wrow + tokoff * KD + wq_off[r]);
    if constexpr (kOut) {
      rp = *(const u32x4*)(pmrow + (size_t)jc * kGC * kGC + 8 * tid);
#pragma unroll
      for (int r = 0; r < KU; ++r) rq[r] = *(const u32x4*)(qrow + tokoff * KD + wq_off[r]);
    }
  };
  auto stage_store = [&]() __attribute__((always_inline)) {
    if (tid < nlev * kGC) s.lam[tid % nlev][tid / nlev] = to_f32<TL>(rl);
    if (s_store) {
      *(uint2*)(s.vs + s_t * LVS + s_v) = rsv;
      const bf16x4 x = __builtin_bit_cast(bf16x4, rsu);
#pragma unroll
      for (int j = 0; j < 4; ++j) s.ut[(s_v + j) * LT + s_t] = x[j];
    }
#pragma unroll
    for (int r = 0; r < KU; ++r) {
      const int u = tid + 512 * r;
      *(u32x4*)(s.kt + (u >> 3) * LT + 8 * (u & 7)) = rk[r];
      *(u32x4*)(s.wq[0] + wq_lds[r]) = rw[r];
    }
    if constexpr (kOut) {
      *(u32x4*)(s.pm + (tid >> 3) * LT + 8 * (tid & 7)) = rp;
#pragma unroll
      for (int r = 0; r < KU; ++r) *(u32x4*)(s.wq[1] + wq_lds[r]) = rq[r];
    }
  };

  // outputs: thread -> token row ot of the chunk and columns ov .. ov + 3 of the
  // slice (threads past the 64 x BV tile store through an empty range)
  constexpr int VG = BV / 4;
  const int ot = tid / VG, ov = 4 * (tid % VG);
  // ot < kGC <=> tid < 64 VG <=> w < VG: a wave-uniform test, so the output
  // descriptor is scalar (a per-lane one makes the store a loop over lanes)
  const bool o_ok = kOut && o != nullptr && w < VG;
  const rsrc_t ro = make_rsrc(o_ok ? (const void*)(o + rowtok * V + v0) : (const void*)gcum,
                              o_ok ? (size_t)T * H * V * sizeof(TO) : 0);
  const unsigned o_voff = ((o_ok ? ot : 0) * HV + ov) * sizeof(TO);
  // hsave: this level's planes (an empty range for the waves without a level)
  const rsrc_t rh = make_rsrc(kSave ? (const void*)(hsave + (size_t)row * NT * nlev * V * KD +
                                                    (size_t)(act ? e : 0) * V * KD + (size_t)v0 * KD)
                                    : (const void*)gcum,
                              kSave && act ? (size_t)NT * nlev * V * KD * 2 : 0);

  stage_load(0);
  stage_store();
  __syncthreads();

  for (int ic = 0; ic < NT; ++ic) {
    const float gl = fexp(rg);   // exp(Gc_last) of chunk ic
    const bool last = ic == NT - 1;

    const int per = 2 << e, pos = ic & (per - 1);
    const bool bit = (ic >> e) & 1;
    // the level read: chunks with bit e set; with strong every chunk reads every
    // level >= 1 (and level 0 is read by none), the states are the same
    const bool rd = act && (strong ? e >= 1 : bit);
    const bool first = act && pos == 0;
    const bool reset = act && pos == per - 1 && !(last && final_state);
    const bool wr = act && !bit;
    const bool needy = act && !first && !reset;

    if constexpr (kSave) {
      // level e's state at the chunk start -> hsave[row][ic][e][v][k]
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int nt = 0; nt < NVT; ++nt)
          buf_store8(__builtin_bit_cast(uint2, cvt4e<E>(st[kt][nt])), rh,
                     (unsigned)(((16 * nt + ln) * KD + 16 * kt + 4 * lq) * 2),
                     (unsigned)((size_t)ic * nlev * V * KD * 2));
    }
    if constexpr (kOut) {
      if (rd) {
        // the level read lambda[t, 7 + e] (q_new h_e)[t][v] -> part[e]
        floatx4 racc[4][NVT];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int nt = 0; nt < NVT; ++nt) racc[tt][nt] = zero4();
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          bf16x8 bh[NVT];
#pragma unroll
          for (int nt = 0; nt < NVT; ++nt) bh[nt] = cat8e<E>(st[2 * c][nt], st[2 * c + 1][nt]);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            const bf16x8 a = frag_k2(s.wq[1], LK, 16 * tt + ln, 32 * c + 4 * lq);
#pragma unroll
            for (int nt = 0; nt < NVT; ++nt) racc[tt][nt] = mfma16<E>(a, bh[nt], racc[tt][nt]);
          }
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const floatx4 lam4 = *(const floatx4*)(&s.lam[e][16 * tt + 4 * lq]);
#pragma unroll
          for (int nt = 0; nt < NVT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              s.part[e][(16 * tt + 4 * lq + i) * LP + 16 * nt + ln] = racc[tt][nt][i] * lam4[i];
        }
      }
      if (w == 0) {
        // o_intra = P V -> part[kGMaxLev]
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          floatx4 x[NVT];
#pragma unroll
          for (int nt = 0; nt < NVT; ++nt) x[nt] = zero4();
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const bf16x8 a = *(const bf16x8*)(s.pm + (16 * tt + ln) * LT + 32 * c + 8 * lq);
#pragma unroll
            for (int nt = 0; nt < NVT; ++nt)
              x[nt] = mfma16<E>(a, tr_frag(s.vs, LVS, 32 * c, 16 * nt), x[nt]);
          }
#pragma unroll
          for (int nt = 0; nt < NVT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) s.part[kGMaxLev][(16 * tt + 4 * lq + i) * LP + 16 * nt + ln] = x[nt][i];
        }
      }
    }
    // chunk ic + 1's operands, into registers while this chunk's state update runs
    stage_load(min(ic + 1, NT - 1));

    if (reset) {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int nt = 0; nt < NVT; ++nt) st[kt][nt] = zero4();
    } else if (act) {
      // V_new[t = 16 tt + 4 lq + i][v = 16 nt + ln] = (write ? U : 0) - W_new h_e
      floatx4 vn[4][NVT];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int nt = 0; nt < NVT; ++nt) vn[tt][nt] = zero4();
      if (needy) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          bf16x8 bh[NVT];
#pragma unroll
          for (int nt = 0; nt < NVT; ++nt) bh[nt] = cat8e<E>(st[2 * c][nt], st[2 * c + 1][nt]);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            const bf16x8 a = frag_k2(s.wq[0], LK, 16 * tt + ln, 32 * c + 4 * lq);
#pragma unroll
            for (int nt = 0; nt < NVT; ++nt) vn[tt][nt] = mfma16<E>(a, bh[nt], vn[tt][nt]);
          }
        }
      }
      if (wr) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int nt = 0; nt < NVT; ++nt) {
            const bf16x4 u4 = *(const bf16x4*)(s.ut + (16 * nt + ln) * LT + 16 * tt + 4 * lq);
#pragma unroll
            for (int i = 0; i < 4; ++i) vn[tt][nt][i] = from16<E>(u4[i]) - vn[tt][nt][i];
          }
      } else {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int nt = 0; nt < NVT; ++nt) vn[tt][nt] = -vn[tt][nt];
      }
      // h_e = exp(Gc_last) h_e + K_new^T V_new (the state is zero on a block's first chunk)
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int nt = 0; nt < NVT; ++nt) st[kt][nt] *= gl;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        bf16x8 bv[NVT];
#pragma unroll
        for (int nt = 0; nt < NVT; ++nt) bv[nt] = cat8e<E>(vn[2 * c][nt], vn[2 * c + 1][nt]);
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
          const bf16x8 a = frag_k2(s.kt, LT, 16 * kt + ln, 32 * c + 4 * lq);
#pragma unroll
          for (int nt = 0; nt < NVT; ++nt) st[kt][nt] = mfma16<E>(a, bv[nt], st[kt][nt]);
        }
      }
    }
    __syncthreads();   // the chunk's operands are consumed, its level reads written

    stage_store();     // chunk ic + 1
    if constexpr (kOut) {
      // o = o_intra + the reads of the levels with bit e of ic set (strong: of
      // every level >= 1)
      const int po = (ot & (kGC - 1)) * LP + ov;
      floatx4 x = *(const floatx4*)(&s.part[kGMaxLev][po]);
      for (int le = 0; le < nlev; ++le)
        if (strong ? le >= 1 : ((ic >> le) & 1)) x += *(const floatx4*)(&s.part[le][po]);
      buf_store4<TO>(x, ro, o_voff, (unsigned)((size_t)ic * kGC * HV * sizeof(TO)));
    }
    __syncthreads();   // chunk ic + 1 staged; the level reads are summed
  }
  if (final_state && ht != nullptr && act && !(strong && e == 0)) {
    // ht[b, h, k, v, 7 + e] (chunkwise_hgdn.py:786-787; strong: levels >= 1,
    // level 7 stays as the caller zeroed it, :724-728)
    float* hb = ht + (size_t)row * KD * V * L + (size_t)v0 * L + 7 + e;
    const size_t VL = (size_t)V * L;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int nt = 0; nt < NVT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          hb[(size_t)(16 * kt + 4 * lq + i) * VL + (16 * nt + ln) * L] = st[kt][nt][i];
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

// The forward that keeps, for the backward, what its recompute would produce:
// the forward's buffers, then the token-major K_new and every level's state at
// every chunk start (bf16 [row][chunk][level][v][k], the backward's layout).
struct GdnKeepWs {
  GdnWs f;
  __bf16 *kn, *hs;
  size_t bytes;
};

inline GdnKeepWs gdn_keep_ws_layout(void* base, int B, int T, int H, int K, int V, int nlev) {
  GdnKeepWs w;
  w.f = gdn_ws_layout(base, B, T, H, K, V);
  char* p = (char*)base;
  size_t off = w.f.bytes;
  const size_t n = (size_t)B * T * H, NT = (size_t)T / kGC, nl = nlev > 0 ? (size_t)nlev : 1;
  w.kn = (__bf16*)(p + off); off += galign(n * K * 2);
  w.hs = (__bf16*)(p + off); off += galign((size_t)B * H * NT * nl * V * K * 2);
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

template <int KD, typename TB, typename TL, int MODE, bool STRONG = false, typename E = __bf16>
static hipError_t gdn_prep_launch_t(const void* q, const void* k, const void* v, const void* beta,
                                    const float* g, const void* l, float* gcum, void* aw, void* au,
                                    __bf16* qn, __bf16* wn, __bf16* kn, __bf16* knT, __bf16* un,
                                    __bf16* pm, int B, int T, int H, int V, int L, int norm_qk,
                                    float scale, hipStream_t stream) {
  auto kp = gdn_prep_kernel<KD, TB, TL, MODE, STRONG, E>;
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

template <int KD, typename TL, typename TO, typename E = __bf16>
static hipError_t gdn_scan_launch_t(const GdnWs& w, const void* v, const float* gcum,
                                    const void* l, void* o, float* ht, __bf16* hsave, int B,
                                    int T, int H, int V, int L, int nlev, int final_state,
                                    int strong, hipStream_t stream) {
  constexpr int BV = ScanBV<KD>::value;
  // hsave without o: the recompute; both: a forward that keeps the states
  auto ks = !hsave ? gdn_scan_kernel<KD, BV, TL, TO, kScanOut, E>
            : o ? gdn_scan_kernel<KD, BV, TL, TO, kScanOutSave, E>
                : gdn_scan_kernel<KD, BV, TL, TO, kScanSave, E>;
  const int smem = (int)sizeof(GdnScanSmem<KD, BV>);
  hipError_t e;
  if ((e = hipFuncSetAttribute((const void*)ks, hipFuncAttributeMaxDynamicSharedMemorySize,
                               smem)) != hipSuccess)
    return e;
  const int rows = B * H;
  const int grid = (rows + 7) / 8 * 8 * (V / BV);
  hipLaunchKernelGGL(ks, dim3(grid), dim3(512), smem, stream, w.qn, w.wn, w.knT, w.un, w.pm,
                     (const __bf16*)v, gcum, (const TL*)l, (TO*)o, ht, hsave, rows, T, H, V, L,
                     nlev, final_state, strong);
  return hipGetLastError();
}

template <int KD, typename TB, typename TL, typename TO, bool STRONG, typename E = __bf16>
static hipError_t gdn_launch_t(const void* q, const void* k, const void* v, const void* beta,
                               const float* g, const void* l, void* o, float* gcum, void* aw,
                               void* au, float* ht, void* ws, int B, int T, int H, int V, int L,
                               int nlev, int norm_qk, float scale, hipStream_t stream) {
  const GdnWs w = gdn_ws_layout(ws, B, T, H, KD, V);
  hipError_t e = gdn_prep_launch_t<KD, TB, TL, kPrepFwd, STRONG, E>(
      q, k, v, beta, g, l, gcum, aw, au, w.qn, w.wn, nullptr, w.knT, w.un, w.pm, B, T, H, V, L,
      norm_qk, scale, stream);
  if (e != hipSuccess) return e;
  return gdn_scan_launch_t<KD, TL, TO, E>(w, v, gcum, l, o, ht, nullptr, B, T, H, V, L, nlev,
                                       ht != nullptr ? 1 : 0, STRONG ? 1 : 0, stream);
}

template <int KD, typename TB, typename TL, typename TO, bool STRONG, typename E = __bf16>
static hipError_t gdn_launch_keep_t(const void* q, const void* k, const void* v, const void* beta,
                                    const float* g, const void* l, void* o, float* gcum, void* aw,
                                    void* au, float* ht, void* ws, int B, int T, int H, int V,
                                    int L, int nlev, int norm_qk, float scale, hipStream_t stream) {
  const GdnKeepWs w = gdn_keep_ws_layout(ws, B, T, H, KD, V, nlev);
  hipError_t e = gdn_prep_launch_t<KD, TB, TL, kPrepFwdKeep, STRONG, E>(
      q, k, v, beta, g, l, gcum, aw, au, w.f.qn, w.f.wn, w.kn, w.f.knT, w.f.un, w.f.pm, B, T, H,
      V, L, norm_qk, scale, stream);
  if (e != hipSuccess) return e;
  return gdn_scan_launch_t<KD, TL, TO, E>(w.f, v, gcum, l, o, ht, w.hs, B, T, H, V, L, nlev,
                                       ht != nullptr ? 1 : 0, STRONG ? 1 : 0, stream);
}

}  // namespace hattn

size_t hattn_gdn_fwd_keep_ws_bytes(int B, int T, int H, int K, int V, int nlev) {
  return hattn::gdn_keep_ws_layout(nullptr, B, T, H, K, V, nlev).bytes;
}

void hattn_gdn_fwd_keep_buffers(const void* ws, int B, int T, int H, int K, int V, int nlev,
                                const __bf16** qn, const __bf16** wn, const __bf16** kn,
                                const __bf16** un, const __bf16** hs) {
  const hattn::GdnKeepWs w = hattn::gdn_keep_ws_layout(const_cast<void*>(ws), B, T, H, K, V, nlev);
  *qn = w.f.qn;
  *wn = w.f.wn;
  *kn = w.kn;
  *un = w.f.un;
  *hs = w.hs;
}

// The forward plus, in the workspace, the backward's recompute results
// (q_new, W_new, K_new, U, every level's state at every chunk start).
hipError_t hattn_gdn_fwd_keep_launch(const void* q, const void* k, const void* v,
                                     const void* beta, const float* g, const void* l, void* o,
                                     float* gcum, void* aw, void* au, float* ht, void* ws, int B,
                                     int T, int H, int K, int V, int L, int nlev, int dt_b,
                                     int dt_l, int dt_o, int norm_qk, float scale, int strong,
                                     int h16, hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  if (h16) {
    // fp16 q / k / v and o on fp16 MFMA (HType.WEAK, fp32 beta and lambda)
#define HATTN_GDN_KH(KD_)                                                                       \
  if (K == KD_)                                                                                 \
    return gdn_launch_keep_t<KD_, float, float, _Float16, false, _Float16>(                     \
        q, k, v, beta, g, l, o, gcum, aw, au, ht, ws, B, T, H, V, L, nlev, norm_qk, scale, stream);
    if (!strong && dt_b == 2 && dt_l == 2 && dt_o == 1) {
      HATTN_GDN_KH(64)
      HATTN_GDN_KH(128)
      HATTN_GDN_KH(192)
      HATTN_GDN_KH(256)
    }
#undef HATTN_GDN_KH
    *unsupported = 1;
    return hipSuccess;
  }
#define HATTN_GDN_KDT(KD_, TB_, TL_)                                                            \
  return strong ? gdn_launch_keep_t<KD_, TB_, TL_, __bf16, true>(                                 \
                      q, k, v, beta, g, l, o, gcum, aw, au, ht, ws, B, T, H, V, L, nlev, norm_qk,  \
                      scale, stream)                                                              \
                : gdn_launch_keep_t<KD_, TB_, TL_, __bf16, false>(                                \
                      q, k, v, beta, g, l, o, gcum, aw, au, ht, ws, B, T, H, V, L, nlev, norm_qk,  \
                      scale, stream);
#define HATTN_GDN_K(KD_)                                                                        \
  if (K == KD_ && dt_o == 0) {                                                                  \
    if (dt_b == 0 && dt_l == 0) HATTN_GDN_KDT(KD_, __bf16, __bf16)                              \
    if (dt_b == 2 && dt_l == 2) HATTN_GDN_KDT(KD_, float, float)                                \
    if (dt_b == 0 && dt_l == 2) HATTN_GDN_KDT(KD_, __bf16, float)                               \
    if (dt_b == 2 && dt_l == 0) HATTN_GDN_KDT(KD_, float, __bf16)                               \
  }
  HATTN_GDN_K(64)
  HATTN_GDN_K(128)
  HATTN_GDN_K(192)
  HATTN_GDN_K(256)
#undef HATTN_GDN_K
#undef HATTN_GDN_KDT
  *unsupported = 1;
  return hipSuccess;
}

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
                                float scale, int strong, int h16, hipStream_t stream,
                                int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  if (h16) {
    // fp16 q / k / v and o on fp16 MFMA (HType.WEAK, fp32 beta and lambda)
#define HATTN_GDN_H(KD_)                                                                        \
  if (K == KD_)                                                                                 \
    return gdn_launch_t<KD_, float, float, _Float16, false, _Float16>(                          \
        q, k, v, beta, g, l, o, gcum, aw, au, ht, ws, B, T, H, V, L, nlev, norm_qk, scale, stream);
    if (!strong && dt_b == 2 && dt_l == 2 && dt_o == 1) {
      HATTN_GDN_H(64)
      HATTN_GDN_H(128)
      HATTN_GDN_H(192)
      HATTN_GDN_H(256)
    }
#undef HATTN_GDN_H
    *unsupported = 1;
    return hipSuccess;
  }
#define HATTN_GDN_DT(KD_, TB_, TL_)                                                             \
  return strong ? gdn_launch_t<KD_, TB_, TL_, __bf16, true>(q, k, v, beta, g, l, o, gcum, aw, au, \
                                                            ht, ws, B, T, H, V, L, nlev, norm_qk,  \
                                                            scale, stream)                        \
                : gdn_launch_t<KD_, TB_, TL_, __bf16, false>(q, k, v, beta, g, l, o, gcum, aw,    \
                                                             au, ht, ws, B, T, H, V, L, nlev,     \
                                                             norm_qk, scale, stream);
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
                                      int h16, hipStream_t stream, int* unsupported) {
  // the recompute writes the level states only, which do not depend on the
  // hierarchy type (strong changes the reads), so it has no strong flag
  using namespace hattn;
  *unsupported = 0;
  GdnWs w;
  w.qn = qn;
  w.wn = wn;
  w.knT = knT;
  w.un = un;
  w.pm = qn;   // read but unused without an output
#define HATTN_GDN_RCE(KD_, TB_, TL_, E_)                                                          \
  {                                                                                               \
    hipError_t e = gdn_prep_launch_t<KD_, TB_, TL_, kPrepRecompute, false, E_>(                   \
        q, k, v, beta, gcum, l, nullptr, nullptr, nullptr, qn, wn, kn, knT, un, nullptr, B, T, H, \
        V, L, norm_qk, scale, stream);                                                            \
    if (e != hipSuccess) return e;                                                                \
    return gdn_scan_launch_t<KD_, TL_, __bf16, E_>(w, v, gcum, l, nullptr, nullptr, hsave, B, T, \
                                                   H, V, L, nlev, 0, 0, stream);                  \
  }
#define HATTN_GDN_RC(KD_, TB_, TL_) HATTN_GDN_RCE(KD_, TB_, TL_, __bf16)
  if (h16) {
    if (dt_b == 2 && dt_l == 2) {
      if (K == 64) HATTN_GDN_RCE(64, float, float, _Float16)
      if (K == 128) HATTN_GDN_RCE(128, float, float, _Float16)
      if (K == 192) HATTN_GDN_RCE(192, float, float, _Float16)
      if (K == 256) HATTN_GDN_RCE(256, float, float, _Float16)
    }
    *unsupported = 1;
    return hipSuccess;
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
  HATTN_GDN_RC_D(256)
#undef HATTN_GDN_RC_D
#undef HATTN_GDN_RC
#undef HATTN_GDN_RCE
  *unsupported = 1;
  return hipSuccess;
}
