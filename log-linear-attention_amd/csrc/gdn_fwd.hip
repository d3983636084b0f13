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
// exp(Gc_t - Gc_s) (s <= t), Au = Aw o gamma:
//   W = Aw (beta K),  U = Au (beta V),  K_new = exp(Gc_last - Gc) K,
//   W_new = exp(Gc) W,  q_new = exp(Gc) (Q - tril(Q K^T) W),
//   o_intra = ((tril(Q K^T) Aw) o gamma o beta_s o lambda[t, lev(t, s)]) V
// and every inter-chunk level e runs the delta-rule recurrence over chunks
//   h_e <- (reset ? 0 : exp(Gc_last) h_e) + K_new^T ((write ? U : 0) - (reset ? 0 : W_new h_e))
// (write: bit e of the chunk index clear; reset after the last chunk of an
// aligned 2^(e+1) block), read by the chunks with bit e set:
//   o += lambda[t, 7 + e] q_new h_e.
//
// Kernel 1 (gdn_prep_kernel): one workgroup per chunk computes everything
// that is local to the chunk: the two 64 x 64 products K K^T and Q K^T on
// MFMA, the fp32 unit-lower-triangular inverse (16 x 16 diagonal blocks by
// substitution, off-diagonal blocks by block substitution), W, U, q_new,
// K_new, W_new and o_intra, plus the Aw / Au the reference returns.  Its LDS
// holds one workgroup per CU, so it runs eight waves (two per SIMD): wave w
// owns output rows t-tile w & 3 and half w >> 2 of the column tiles.
// Kernel 2 (gdn_scan_kernel): one workgroup per (row, 32 columns of V) walks
// the chunks in order with every level's [K x 32] state in fp32 registers
// (wave w owns K / 4 state rows); per chunk it stages the states in LDS
// as bf16, forms W_new h_e and q_new h_e for all levels, then
// h_e += K_new^T V_new_e, and writes o = o_intra + sum of the level reads.
#include "gdn_common.h"

namespace hattn {

template <int KD, int VD>
struct GdnPrepSmem {
  static constexpr int LK = KD + 8, LV = VD + 8, LF = (KD > VD ? KD : VD) + 4;
  static constexpr int NF = kGC * LF > 2 * kGC * 65 ? kGC * LF : 2 * kGC * 65;
  __bf16 k[kGC * LK];
  __bf16 q[kGC * LK];
  __bf16 v[kGC * LV];
  float f[NF];                    // A / X (two 64 x 65 fp32 blocks), later fp32 staging
  float t1[4][16 * 17];           // per-wave block-substitution scratch
  __bf16 aw[kGC * kLd64];         // Aw (bf16)
  __bf16 au[kGC * kLd64];         // Au = Aw o gamma (bf16)
  __bf16 qk[kGC * kLd64];         // tril(Q K^T) (bf16)
  __bf16 pm[kGC * kLd64];         // (tril(Q K^T) Aw) o gamma o beta o lambda (bf16)
  __bf16 w[kGC * LK];             // W (bf16)
  float gc[kGC];
  float beta[kGC];
  float lam[7][kGC];              // intra-chunk lambda columns 0..6
};

// GCUM: g already holds the chunk-local cumsum (the backward's input,
// chunkwise_hgdn.py:799-817) and gcum is not written.  aw_out, au_out and oi
// may be null (the backward recomputes only q_new, K_new, W_new and U).
constexpr int kPrepThreads = 512;

template <int KD, int VD, typename TB, typename TL, bool GCUM = false>
__global__ __launch_bounds__(kPrepThreads, 1) void gdn_prep_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const TB* __restrict__ beta, const float* __restrict__ g, const TL* __restrict__ l,
    float* __restrict__ gcum, __bf16* __restrict__ aw_out, __bf16* __restrict__ au_out,
    __bf16* __restrict__ qn, __bf16* __restrict__ kn, __bf16* __restrict__ wn,
    __bf16* __restrict__ un, float* __restrict__ oi, int T, int H, int L, int norm_qk,
    float qk_scale) {
  using Sm = GdnPrepSmem<KD, VD>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Sm& s = *(Sm*)smem_raw;
  constexpr int LK = Sm::LK, LV = Sm::LV, LF = Sm::LF;
  constexpr int NTH = kPrepThreads;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int wt = w & 3, wh = w >> 2;   // output row tile, column-tile half
  const int NT = T / kGC;
  const int ic = blockIdx.x % NT;
  const int row = blockIdx.x / NT;
  const int b = row / H, h = row % H;
  const size_t tok0 = (size_t)b * T + (size_t)ic * kGC;   // first token of the chunk
  const size_t hk = (size_t)H * KD, hv = (size_t)H * VD;
  float* A = s.f;                 // [64][kLM]
  float* X = s.f + kGC * kLM;     // [64][65]

  // ---- load the chunk ---------------------------------------------------------
  // threads 0..255 stage K and V rows 0..31, threads 256..511 Q and V rows 32..63
  if (tid < 256) {
    g2s_tile<KD>(k + tok0 * hk + (size_t)h * KD, hk, s.k, LK);
    g2s_tile<VD, kGC / 2>(v + tok0 * hv + (size_t)h * VD, hv, s.v, LV);
  } else {
    g2s_tile<KD, kGC, 256>(q + tok0 * hk + (size_t)h * KD, hk, s.q, LK);
    g2s_tile<VD, kGC / 2, 256>(v + (tok0 + kGC / 2) * hv + (size_t)h * VD, hv,
                               s.v + (kGC / 2) * LV, LV);
  }
  if (w == 0) {
    float x = g[(tok0 + lane) * H + h];
    if constexpr (!GCUM) {
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
      }
      gcum[(tok0 + lane) * H + h] = x;
    }
    s.gc[lane] = x;
    s.beta[lane] = to_f32<TB>(beta[(tok0 + lane) * H + h]);
  }
  {
    static_assert(NTH >= 7 * kGC, "one lambda entry per thread");
    const int e = min(tid, 7 * kGC - 1);
    const float lv = to_f32<TL>(l[((tok0 + e / 7) * H + h) * L + e % 7]);
    if (tid < 7 * kGC) s.lam[e % 7][e / 7] = lv;
  }
  __syncthreads();
  if (norm_qk) {
    // use_qk_l2norm_in_kernel (kernel.py:110-111): k / ||k|| and q scale / ||q||
    if (tid < 256) l2norm_rows<KD, LK>(s.k, 1.f, nullptr);
    else l2norm_rows<KD, LK, 256>(s.q, qk_scale, nullptr);
    __syncthreads();
  }

  // ---- K K^T (-> A, fp32) and Q K^T (-> tril, bf16): wave w owns rows t-tile wt,
  // column tiles 2wh, 2wh + 1 ------------------------------------------------------
  {
    floatx4 kk[2], qk[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) kk[n] = qk[n] = zero4();
#pragma unroll
    for (int c = 0; c < KD / 32; ++c) {
      const bf16x8 ak = *(const bf16x8*)(s.k + (16 * wt + ln) * LK + 32 * c + 8 * lq);
      const bf16x8 aq = *(const bf16x8*)(s.q + (16 * wt + ln) * LK + 32 * c + 8 * lq);
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
        const int t = 16 * wt + 4 * lq + i, sc = 16 * (2 * wh + n) + ln;
        A[t * kLM + sc] = sc < t ? s.beta[t] * kk[n][i] : 0.f;
        s.qk[t * kLd64 + sc] = (__bf16)(sc <= t ? qk[n][i] : 0.f);
      }
  }
  __syncthreads();

  // ---- X = (I + A)^-1, fp32 ----------------------------------------------------
  tri_inv64<NTH>(A, X, s.t1);

  // ---- Aw, Au (bf16) to LDS and to the outputs ----------------------------------------
  for (int u = tid; u < kGC * 8; u += NTH) {
    const int t = u >> 3, s0 = 8 * (u & 7);
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
    if (aw_out) *(bf16x8*)(aw_out + ((tok0 + t) * H + h) * kGC + s0) = a;
    if (au_out) *(bf16x8*)(au_out + ((tok0 + t) * H + h) * kGC + s0) = au;
  }
  __syncthreads();

  // X[t][s] (bf16 LDS) times (beta o Y)[s][n] (bf16 LDS, row-major [s][n]):
  // wave w computes output rows t-tile wt, its half of the N/16 column tiles,
  // into the fp32 staging.
  auto gemm_rows = [&](const __bf16* xa, const __bf16* yb, int ldb, int ntile, bool scale_beta) {
    const bf16x8 a0 = *(const bf16x8*)(xa + (16 * wt + ln) * kLd64 + 8 * lq);
    const bf16x8 a1 = *(const bf16x8*)(xa + (16 * wt + ln) * kLd64 + 32 + 8 * lq);
    const floatx4 b0a = *(const floatx4*)(s.beta + 8 * lq), b0b = *(const floatx4*)(s.beta + 8 * lq + 4);
    const floatx4 b1a = *(const floatx4*)(s.beta + 32 + 8 * lq),
                  b1b = *(const floatx4*)(s.beta + 36 + 8 * lq);
    const int nh = ntile / 2;
    for (int nt = wh * nh; nt < (wh + 1) * nh; ++nt) {
      bf16x8 y0 = tr_frag(yb, ldb, 0, 16 * nt), y1 = tr_frag(yb, ldb, 32, 16 * nt);
      if (scale_beta) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          y0[j] = (__bf16)((float)y0[j] * b0a[j]);
          y0[4 + j] = (__bf16)((float)y0[4 + j] * b0b[j]);
          y1[j] = (__bf16)((float)y1[j] * b1a[j]);
          y1[4 + j] = (__bf16)((float)y1[4 + j] * b1b[j]);
        }
      }
      floatx4 acc = mfma16x16x32(a0, y0, zero4());
      acc = mfma16x16x32(a1, y1, acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) s.f[(16 * wt + 4 * lq + i) * LF + 16 * nt + ln] = acc[i];
    }
  };

  // ---- W = Aw (beta K) -> W (bf16 LDS), W_new = exp(Gc) W (output) ---------------
  gemm_rows(s.aw, s.k, LK, KD / 16, true);
  __syncthreads();
  for (int u = tid; u < kGC * KD / 8; u += NTH) {
    const int t = u / (KD / 8), c0 = 8 * (u % (KD / 8));
    const float eg = fexp(s.gc[t]);
    bf16x8 wb, wnb;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = s.f[t * LF + c0 + j];
      wb[j] = (__bf16)x;
      wnb[j] = (__bf16)(x * eg);
    }
    *(bf16x8*)(s.w + t * LK + c0) = wb;
    *(bf16x8*)(wn + (tok0 + t) * hk + (size_t)h * KD + c0) = wnb;
    // K_new = exp(Gc_last - Gc_t) K
    const float ek = fexp(s.gc[kGC - 1] - s.gc[t]);
    const bf16x8 kx = *(const bf16x8*)(s.k + t * LK + c0);
    bf16x8 knb;
#pragma unroll
    for (int j = 0; j < 8; ++j) knb[j] = (__bf16)((float)kx[j] * ek);
    *(bf16x8*)(kn + (tok0 + t) * hk + (size_t)h * KD + c0) = knb;
  }
  __syncthreads();

  // ---- U = Au (beta V) (output) ------------------------------------------------------
  gemm_rows(s.au, s.v, LV, VD / 16, true);
  __syncthreads();
  for (int u = tid; u < kGC * VD / 8; u += NTH) {
    const int t = u / (VD / 8), c0 = 8 * (u % (VD / 8));
    bf16x8 ub;
#pragma unroll
    for (int j = 0; j < 8; ++j) ub[j] = (__bf16)s.f[t * LF + c0 + j];
    *(bf16x8*)(un + (tok0 + t) * hv + (size_t)h * VD + c0) = ub;
  }
  __syncthreads();

  // ---- q_new = exp(Gc) (Q - tril(Q K^T) W) (output) ---------------------------------
  gemm_rows(s.qk, s.w, LK, KD / 16, false);
  __syncthreads();
  for (int u = tid; u < kGC * KD / 8; u += NTH) {
    const int t = u / (KD / 8), c0 = 8 * (u % (KD / 8));
    const float eg = fexp(s.gc[t]);
    const bf16x8 qx = *(const bf16x8*)(s.q + t * LK + c0);
    bf16x8 qb;
#pragma unroll
    for (int j = 0; j < 8; ++j) qb[j] = (__bf16)(eg * ((float)qx[j] - s.f[t * LF + c0 + j]));
    *(bf16x8*)(qn + (tok0 + t) * hk + (size_t)h * KD + c0) = qb;
  }
  __syncthreads();

  if (oi == nullptr) return;

  // ---- P = (tril(Q K^T) Aw) o gamma o beta_s o lambda[t, lev] (bf16 LDS) -----------
  gemm_rows(s.qk, s.aw, kLd64, 4, false);
  __syncthreads();
  for (int u = tid; u < kGC * 8; u += NTH) {
    const int t = u >> 3, s0 = 8 * (u & 7);
    bf16x8 pb;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int sc = s0 + j;
      float x = 0.f;
      if (sc <= t)
        x = s.f[t * LF + sc] * fexp(s.gc[t] - s.gc[sc]) * s.beta[sc] *
            s.lam[intra_level(t, sc)][t];
      pb[j] = (__bf16)x;
    }
    *(bf16x8*)(s.pm + t * kLd64 + s0) = pb;
  }
  __syncthreads();

  // ---- o_intra = P V (fp32 output) ---------------------------------------------------
  gemm_rows(s.pm, s.v, LV, VD / 16, false);
  __syncthreads();
  for (int u = tid; u < kGC * VD / 4; u += NTH) {
    const int t = u / (VD / 4), c0 = 4 * (u % (VD / 4));
    *(floatx4*)(oi + (tok0 + t) * hv + (size_t)h * VD + c0) = *(const floatx4*)(s.f + t * LF + c0);
  }
}

// ---------------------------------------------------------------------------
// level scan
// ---------------------------------------------------------------------------
template <int KD>
struct GdnScanSmem {
  static constexpr int LK = KD + 8;
  __bf16 qn[kGC * LK];
  __bf16 wn[kGC * LK];
  __bf16 kn[kGC * LK];
  __bf16 u[kGC * (kBVs + 8)];                 // U[t][v] slice
  float lam[kGMaxLev][kGC];                   // lambda[t, 7 + e]
  __bf16 hs[kGMaxLev][kBVs * LK];             // states, bf16 [v][k]
  __bf16 vn[kGMaxLev][kBVs * kLd64];          // V_new, bf16 [v][t]
};

template <int KD, typename TL, typename TO>
__global__ __launch_bounds__(256, 1) void gdn_scan_kernel(
    const __bf16* __restrict__ qn, const __bf16* __restrict__ wn, const __bf16* __restrict__ kn,
    const __bf16* __restrict__ un, const float* __restrict__ oi, const float* __restrict__ gcum,
    const TL* __restrict__ l, TO* __restrict__ o, float* __restrict__ ht,
    __bf16* __restrict__ hsave, int T, int H, int V, int L, int nlev, int final_state) {
  using Sm = GdnScanSmem<KD>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Sm& s = *(Sm*)smem_raw;
  constexpr int LK = Sm::LK;
  constexpr int LU = kBVs + 8;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int nvb = V / kBVs;
  const int vb = blockIdx.x % nvb;
  const int row = blockIdx.x / nvb;
  const int b = row / H, h = row % H;
  const int NT = T / kGC;
  const size_t hk = (size_t)H * KD, hv = (size_t)H * V;
  const int v0 = vb * kBVs;

  // states: wave w owns rows k = RW w + 16m + 4lq + i (RW = K / 4 rows, MT = RW / 16
  // tiles), columns v = 16n + ln
  constexpr int MT = KD / 64, RW = KD / 4;
  floatx4 st[kGMaxLev][MT][2];
#pragma unroll
  for (int e = 0; e < kGMaxLev; ++e)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n) st[e][m][n] = zero4();

  // Chunk ic + 1's q_new / W_new / K_new / U tiles, lambda columns and last
  // decay are loaded into registers while chunk ic computes, and chunk ic + 1's
  // o_intra after chunk ic's output is written; each chunk starts by moving them
  // to LDS.  Thread tid owns 16-byte units tid + 256 i of each tile.  Every
  // load is issued unconditionally (clamped to a valid address where its value
  // is not used): a load under a condition would make the compiler merge its
  // registers after the branch, which waits for the load right away.
  constexpr int UPR = KD / 8, QU = kGC * UPR / 256;   // units per row / per thread
  static_assert(kGC * kBVs / 8 == 256, "one U unit per thread");
  u32x4 pq[QU], pw[QU], pk[QU], pu;
  float plam[2], pgl = 0.f, poi[2][4];
  auto fetch_tiles = [&](int jc) __attribute__((always_inline)) {
    const size_t t0 = (size_t)b * T + (size_t)jc * kGC;
#pragma unroll
    for (int i = 0; i < QU; ++i) {
      const int u = tid + 256 * i, r = u / UPR, c = 8 * (u % UPR);
      const size_t off = (t0 + r) * hk + (size_t)h * KD + c;
      pq[i] = *(const u32x4*)(qn + off);
      pw[i] = *(const u32x4*)(wn + off);
      pk[i] = *(const u32x4*)(kn + off);
    }
    pu = *(const u32x4*)(un + (t0 + (tid >> 2)) * hv + (size_t)h * V + v0 + 8 * (tid & 3));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e2 = min(tid + 256 * i, nlev * kGC - 1);
      plam[i] = to_f32<TL>(l[((t0 + e2 / nlev) * H + h) * L + 7 + e2 % nlev]);
    }
    pgl = gcum[(t0 + kGC - 1) * H + h];
  };
  // without an output (the backward's recompute) the o_intra loads read gcum
  // row 0 instead, and their values are not used
  const float* oisrc = o ? oi : gcum;
  auto fetch_oi = [&](int jc) __attribute__((always_inline)) {
    const size_t t0 = (size_t)b * T + (size_t)jc * kGC;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        poi[n][i] = oisrc[o ? (t0 + 16 * w + 4 * lq + i) * hv + (size_t)h * V + v0 + 16 * n + ln : 0];
  };
  fetch_tiles(0);
  fetch_oi(0);

  for (int ic = 0; ic < NT; ++ic) {
    const size_t tok0 = (size_t)b * T + (size_t)ic * kGC;
#pragma unroll
    for (int i = 0; i < QU; ++i) {
      const int u = tid + 256 * i, r = u / UPR, c = 8 * (u % UPR);
      *(u32x4*)(s.qn + r * LK + c) = pq[i];
      *(u32x4*)(s.wn + r * LK + c) = pw[i];
      *(u32x4*)(s.kn + r * LK + c) = pk[i];
    }
    *(u32x4*)(s.u + (tid >> 2) * LU + 8 * (tid & 3)) = pu;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e2 = tid + 256 * i;
      if (e2 < nlev * kGC) s.lam[e2 % nlev][e2 / nlev] = plam[i];
    }
    const float glast = pgl;
    // states -> LDS, bf16 [v][k] (4 consecutive k per lane); with hsave also to
    // hsave[row][chunk][level][v][k] (the state each chunk starts from)
#pragma unroll
    for (int e = 0; e < kGMaxLev; ++e) {
      if (e < nlev) {
        __bf16* hg = hsave ? hsave + (((size_t)row * NT + ic) * nlev + e) * (size_t)V * KD +
                                 (size_t)v0 * KD
                           : nullptr;
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int n = 0; n < 2; ++n) {
            const bf16x4 hv4 = cvt4(st[e][m][n]);
            const int kk = RW * w + 16 * m + 4 * lq;
            *(bf16x4*)(s.hs[e] + (16 * n + ln) * LK + kk) = hv4;
            if (hg) *(bf16x4*)(hg + (size_t)(16 * n + ln) * KD + kk) = hv4;
          }
      }
    }
    __syncthreads();
    fetch_tiles(min(ic + 1, NT - 1));

    // ---- reads (q_new h_e) and V_new_e = (write ? U : 0) - (reset ? 0 : W_new h_e) ----
    // Branch-free per level: both products are always formed and the level's
    // read / write / reset flags enter as 0 / 1 factors, so the LDS reads and
    // MFMAs of a level issue back to back instead of one wait per product.
    const bool last = ic == NT - 1;
    floatx4 acc[2] = {zero4(), zero4()};
    {
      bf16x8 aw[KD / 32], aq[KD / 32];
#pragma unroll
      for (int c = 0; c < KD / 32; ++c) {
        aw[c] = *(const bf16x8*)(s.wn + (16 * w + ln) * LK + 32 * c + 8 * lq);
        aq[c] = *(const bf16x8*)(s.qn + (16 * w + ln) * LK + 32 * c + 8 * lq);
      }
      float uv[2][4];   // U[t = 16w + 4lq + i][16n + ln]
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) uv[n][i] = (float)s.u[(16 * w + 4 * lq + i) * LU + 16 * n + ln];
#pragma unroll
      for (int e = 0; e < kGMaxLev; ++e) {
        if (e < nlev) {
          const int per = 2 << e;
          const float frd = ((ic >> e) & 1) ? 1.f : 0.f;
          const float fkeep = (((ic & (per - 1)) == per - 1) && !(last && final_state)) ? 0.f : 1.f;
          const floatx4 lam4 = *(const floatx4*)(&s.lam[e][16 * w + 4 * lq]);
          bf16x8 bh[2][KD / 32];
#pragma unroll
          for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int c = 0; c < KD / 32; ++c)
              bh[n][c] = *(const bf16x8*)(s.hs[e] + (16 * n + ln) * LK + 32 * c + 8 * lq);
#pragma unroll
          for (int n = 0; n < 2; ++n) {
            floatx4 y = zero4(), z = zero4();
#pragma unroll
            for (int c = 0; c < KD / 32; ++c) {
              y = mfma16x16x32(aw[c], bh[n][c], y);
              z = mfma16x16x32(aq[c], bh[n][c], z);
            }
            bf16x4 vb4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[n][i] += frd * lam4[i] * z[i];
              vb4[i] = (__bf16)((1.f - frd) * uv[n][i] - fkeep * y[i]);
            }
            *(bf16x4*)(s.vn[e] + (16 * n + ln) * kLd64 + 16 * w + 4 * lq) = vb4;
          }
        }
      }
    }
    // ---- o = o_intra + reads ----------------------------------------------------------
    if (o) {
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const size_t idx = (tok0 + 16 * w + 4 * lq + i) * hv + (size_t)h * V + v0 + 16 * n + ln;
          o[idx] = from_f32<TO>(poi[n][i] + acc[n][i]);
        }
    }
    fetch_oi(min(ic + 1, NT - 1));
    __syncthreads();

    // ---- h_e = (reset ? 0 : exp(Gc_last) h_e) + K_new^T V_new_e -----------------------
    {
      bf16x8 ak[MT][2];
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int c = 0; c < 2; ++c) ak[m][c] = tr_frag(s.kn, LK, 32 * c, RW * w + 16 * m);
      const float gl = fexp(glast);
#pragma unroll
      for (int e = 0; e < kGMaxLev; ++e) {
        if (e < nlev) {
          const int per = 2 << e;
          const bool reset = ((ic & (per - 1)) == per - 1) && !(last && final_state);
          const float gk = reset ? 0.f : gl;
          bf16x8 b0[2], b1[2];
#pragma unroll
          for (int n = 0; n < 2; ++n) {
            b0[n] = *(const bf16x8*)(s.vn[e] + (16 * n + ln) * kLd64 + 8 * lq);
            b1[n] = *(const bf16x8*)(s.vn[e] + (16 * n + ln) * kLd64 + 32 + 8 * lq);
          }
#pragma unroll
          for (int n = 0; n < 2; ++n) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
              floatx4 x = st[e][m][n];
#pragma unroll
              for (int i = 0; i < 4; ++i) x[i] *= gk;
              x = mfma16x16x32(ak[m][0], b0[n], x);
              x = mfma16x16x32(ak[m][1], b1[n], x);
              st[e][m][n] = x;
            }
          }
        }
      }
    }
    if (last && final_state && ht != nullptr) {
      // ht[b, h, k, v, 7 + e] (chunkwise_hgdn.py:786-787)
#pragma unroll
      for (int e = 0; e < kGMaxLev; ++e)
        if (e < nlev)
#pragma unroll
          for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < 2; ++n)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int kk = RW * w + 16 * m + 4 * lq + i, vv = v0 + 16 * n + ln;
                ht[((((size_t)b * H + h) * KD + kk) * V + vv) * L + 7 + e] = st[e][m][n][i];
              }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// host launcher
// ---------------------------------------------------------------------------
struct GdnWs {
  __bf16 *qn, *kn, *wn, *un;
  float* oi;
  size_t bytes;
};

inline size_t galign(size_t x) { return (x + 255) & ~(size_t)255; }

inline GdnWs gdn_ws_layout(void* base, int B, int T, int H, int K, int V) {
  GdnWs w;
  char* p = (char*)base;
  size_t off = 0;
  const size_t n = (size_t)B * T * H;
  w.qn = (__bf16*)(p + off); off += galign(n * K * 2);
  w.kn = (__bf16*)(p + off); off += galign(n * K * 2);
  w.wn = (__bf16*)(p + off); off += galign(n * K * 2);
  w.un = (__bf16*)(p + off); off += galign(n * V * 2);
  w.oi = (float*)(p + off);  off += galign(n * V * 4);
  w.bytes = off;
  return w;
}

template <int KD, int VD, typename TB, typename TL, typename TO>
static hipError_t gdn_launch_t(const void* q, const void* k, const void* v, const void* beta,
                               const float* g, const void* l, void* o, float* gcum, void* aw,
                               void* au, float* ht, void* ws, int B, int T, int H, int L,
                               int nlev, int norm_qk, float scale, hipStream_t stream) {
  const GdnWs w = gdn_ws_layout(ws, B, T, H, KD, VD);
  const int NT = T / kGC;
  hipError_t e;
  {
    auto kp = gdn_prep_kernel<KD, VD, TB, TL>;
    const int smem = (int)sizeof(GdnPrepSmem<KD, VD>);
    if ((e = hipFuncSetAttribute((const void*)kp, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 smem)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(kp, dim3(B * H * NT), dim3(kPrepThreads), smem, stream, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, (const TB*)beta, g, (const TL*)l, gcum,
                       (__bf16*)aw, (__bf16*)au, w.qn, w.kn, w.wn, w.un, w.oi, T, H, L, norm_qk,
                       scale);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    auto ks = gdn_scan_kernel<KD, TL, TO>;
    const int smem = (int)sizeof(GdnScanSmem<KD>);
    if ((e = hipFuncSetAttribute((const void*)ks, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 smem)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(ks, dim3(B * H * (VD / kBVs)), dim3(256), smem, stream, w.qn, w.wn, w.kn,
                       w.un, w.oi, gcum, (const TL*)l, (TO*)o, ht, (__bf16*)nullptr, T, H, VD, L,
                       nlev, ht != nullptr ? 1 : 0);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace hattn

size_t hattn_gdn_fwd_ws_bytes(int B, int T, int H, int K, int V) {
  return hattn::gdn_ws_layout(nullptr, B, T, H, K, V).bytes;
}

int hattn_gdn_fwd_max_levels() { return hattn::kGMaxLev; }

hipError_t hattn_gdn_fwd_launch(const void* q, const void* k, const void* v, const void* beta,
                                const float* g, const void* l, void* o, float* gcum, void* aw,
                                void* au, float* ht, void* ws, int B, int T, int H, int K, int V,
                                int L, int nlev, int dt_b, int dt_l, int dt_o, int norm_qk,
                                float scale, hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
#define HATTN_GDN(KD_, VD_)                                                                     \
  if (K == KD_ && V == VD_) {                                                                   \
    if (dt_b == 0 && dt_l == 0 && dt_o == 0)                                                    \
      return gdn_launch_t<KD_, VD_, __bf16, __bf16, __bf16>(q, k, v, beta, g, l, o, gcum, aw, au, \
                                                            ht, ws, B, T, H, L, nlev, norm_qk, scale, stream);  \
    if (dt_b == 2 && dt_l == 2 && dt_o == 0)                                                    \
      return gdn_launch_t<KD_, VD_, float, float, __bf16>(q, k, v, beta, g, l, o, gcum, aw, au, \
                                                          ht, ws, B, T, H, L, nlev, norm_qk, scale, stream);    \
    if (dt_b == 0 && dt_l == 2 && dt_o == 0)                                                    \
      return gdn_launch_t<KD_, VD_, __bf16, float, __bf16>(q, k, v, beta, g, l, o, gcum, aw, au, \
                                                           ht, ws, B, T, H, L, nlev, norm_qk, scale, stream);   \
    if (dt_b == 2 && dt_l == 0 && dt_o == 0)                                                    \
      return gdn_launch_t<KD_, VD_, float, __bf16, __bf16>(q, k, v, beta, g, l, o, gcum, aw, au, \
                                                           ht, ws, B, T, H, L, nlev, norm_qk, scale, stream);   \
  }
  HATTN_GDN(128, 128)
  HATTN_GDN(64, 64)
#undef HATTN_GDN
  *unsupported = 1;
  return hipSuccess;
}

// Forward recompute for the backward: q_new, K_new, W_new, U from the
// chunk-local cumsum (prep kernel) and every level's per-chunk starting state,
// bf16 [row][chunk][level][v][k] (scan kernel, no output).
hipError_t hattn_gdn_recompute_launch(const void* q, const void* k, const void* v,
                                      const void* beta, const float* gcum, const void* l,
                                      __bf16* qn, __bf16* kn, __bf16* wn, __bf16* un,
                                      __bf16* hsave, int B, int T, int H, int K, int V, int L,
                                      int nlev, int dt_b, int dt_l, int norm_qk, float scale,
                                      hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  const int NT = T / kGC;
  hipError_t e;
#define HATTN_GDN_RC(KD_, VD_, TB_, TL_)                                                           \
  {                                                                                              \
    auto kp = gdn_prep_kernel<KD_, VD_, TB_, TL_, true>;                                         \
    const int smem = (int)sizeof(GdnPrepSmem<KD_, VD_>);                                         \
    if ((e = hipFuncSetAttribute((const void*)kp, hipFuncAttributeMaxDynamicSharedMemorySize,   \
                                 smem)) != hipSuccess)                                           \
      return e;                                                                                  \
    hipLaunchKernelGGL(kp, dim3(B * H * NT), dim3(kPrepThreads), smem, stream, (const __bf16*)q, \
                       (const __bf16*)k, (const __bf16*)v, (const TB_*)beta, gcum,               \
                       (const TL_*)l, (float*)nullptr, (__bf16*)nullptr, (__bf16*)nullptr, qn,   \
                       kn, wn, un, (float*)nullptr, T, H, L, norm_qk, scale);                    \
    if ((e = hipGetLastError()) != hipSuccess) return e;                                         \
    auto ks = gdn_scan_kernel<KD_, TL_, __bf16>;                                                 \
    const int smem2 = (int)sizeof(GdnScanSmem<KD_>);                                             \
    if ((e = hipFuncSetAttribute((const void*)ks, hipFuncAttributeMaxDynamicSharedMemorySize,   \
                                 smem2)) != hipSuccess)                                          \
      return e;                                                                                  \
    hipLaunchKernelGGL(ks, dim3(B * H * (VD_ / kBVs)), dim3(256), smem2, stream, qn, wn, kn, un, \
                       (const float*)nullptr, gcum, (const TL_*)l, (__bf16*)nullptr,             \
                       (float*)nullptr, hsave, T, H, VD_, L, nlev, 0);                           \
    return hipGetLastError();                                                                    \
  }
#define HATTN_GDN_RC_D(KD_, VD_)                                                                 \
  if (K == KD_ && V == VD_) {                                                                    \
    if (dt_b == 0 && dt_l == 0) HATTN_GDN_RC(KD_, VD_, __bf16, __bf16)                           \
    if (dt_b == 2 && dt_l == 2) HATTN_GDN_RC(KD_, VD_, float, float)                             \
    if (dt_b == 0 && dt_l == 2) HATTN_GDN_RC(KD_, VD_, __bf16, float)                            \
    if (dt_b == 2 && dt_l == 0) HATTN_GDN_RC(KD_, VD_, float, __bf16)                            \
  }
  HATTN_GDN_RC_D(128, 128)
  HATTN_GDN_RC_D(64, 64)
#undef HATTN_GDN_RC_D
#undef HATTN_GDN_RC
  *unsupported = 1;
  return hipSuccess;
}
