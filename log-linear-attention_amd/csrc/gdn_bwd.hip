// Log-linear Gated DeltaNet chunkwise backward for gfx950.
//
// Replaces chunkwise_hgdn.chunkwise_bwd (chunkwise_hgdn.py:791-1222): the
// reference runs two intra-chunk kernels, then per inter-chunk level a state
// recompute, the delta-rule dh scan, torch products and three gradient kernels,
// then the WY / UT-transform backward (fla_future/wy_fast.py:15-132).
//
// Forward quantities of one chunk (C = 64 tokens, chunk-local cumsum Gc,
// e = exp(Gc), r = exp(Gc_last - Gc), Gamma[t,s] = exp(Gc_t - Gc_s) for s <= t):
//   A = strict-tril(diag(beta) K K^T), Aw = (I + A)^-1, M = tril(Q K^T),
//   P = M Aw, W = Aw diag(beta) K, U = (Aw o Gamma) diag(beta) V,
//   q_new = e o (Q - M W), W_new = e o W, K_new = r o K,
//   o_intra = (P o Gamma o Lambda o beta_s) V,
// and per level e, over the chunks c:
//   o_c += lambda_e o (q_new_c h_c),
//   V_new_c = wr U_c - nr W_new_c h_c,
//   h_{c+1} = nr exp(Gc_last) h_c + K_new_c^T V_new_c
// (rd / wr: bit e of c set / clear; nr: c is not the last chunk of an aligned
// 2^(e+1) block).
//
// Four launches:
//   1. prep recompute (gdn_fwd.hip, from g_cumsum): q_new, K_new, W_new, U;
//   2. forward scan recompute: every level's state at every chunk start, bf16;
//   3. gdn_bwd_scan_kernel, one workgroup per (row, 32 columns of V), walks the
//      chunks backwards with every level's dh [K x 32] in fp32 registers:
//        dV_new = K_new dh_{c+1},   dU += wr dV_new,
//        dq_new += rd lambda_e o (dO h_c^T),  dlambda_e = rd rowsum(dO o q_new h_c),
//        dW_new -= nr dV_new h_c^T,  dK_new += V_new dh_{c+1}^T,
//        d exp(Gc_last) += nr <h_c, dh_{c+1}>,
//        dh_c = nr (exp(Gc_last) dh_{c+1} - W_new^T dV_new) + rd q_new^T (lambda_e o dO);
//      the contractions over V give per-slice partials (bf16), summed in fp32 by kernel 4;
//   4. gdn_bwd_chunk_kernel, one workgroup per chunk, backpropagates through
//      the chunk-local algebra.  With X = e o dq_new and E = dP - (X K^T) o beta_s,
//        dM = tril(E Aw^T),  dAw = M^T E + ((e o dW_new) K^T + (dU V^T) o Gamma) o beta_s,
//        dA = -strict-tril(Aw^T dAw Aw^T),
//        dQ = X + dM K,
//        dK = dM^T Q + dA^T (beta o K) + beta o (-P^T X + Aw^T (e o dW_new) + dA K) + r o dK_new,
//        dV = beta o (Au^T dU + (P o Gamma o Lambda)^T dO),
//      dbeta from the same row products, dGc from every e / r / Gamma factor, then
//      dg = reverse chunk-local cumsum of dGc (chunkwise_hgdn.py:1219).  The
//      64 x 64 products with fp32 operands run as bf16x3 (three MFMAs); the
//      inverse is recomputed in fp32, so the Aw / Au of the forward are not read.
#include "gdn_common.h"

hipError_t hattn_gdn_recompute_launch(const void* q, const void* k, const void* v,
                                      const void* beta, const float* gcum, const void* l,
                                      __bf16* qn, __bf16* kn, __bf16* knT, __bf16* wn, __bf16* un,
                                      __bf16* hsave, int B, int T, int H, int K, int V, int L,
                                      int nlev, int dt_b, int dt_l, int norm_qk, float scale,
                                      int h16, hipStream_t stream, int* unsupported);

namespace hattn {

// ---------------------------------------------------------------------------
// Kernel 3: reverse level scan
// ---------------------------------------------------------------------------
template <int KD>
struct GdnBscanSmem {
  static constexpr int LK = KD + 8, LVS = kBVs + 8;
  __bf16 qn[kGC * LK];
  __bf16 wn[kGC * LK];
  __bf16 kn[kGC * LK];
  __bf16 u[kGC * LVS];       // U[t][v] slice
  __bf16 dO[kGC * LVS];      // dO[t][v] slice
  __bf16 ldo[kGC * LVS];     // lambda[t, 7 + e] dO[t][v] of the current level e
  __bf16 hs[kBVs * LK];      // h_e at the chunk start, [v][k]
  __bf16 dhs[kBVs * LK];     // dh_e after the chunk, [v][k]
  __bf16 dvn[kBVs * kLd64];  // dV_new_e, [v][t]
  __bf16 vn[kBVs * kLd64];   // V_new_e, [v][t]
  float lam[kGBwdMaxLev][kGC];  // lambda[t, 7 + e]
  float dlr[2][kGC];         // dlambda row sums of the two 16-column halves
  float red[8];
};

// NW = 8 waves (the wave-count parameter keeps the tile map general).  With
// VTW = 8 / NW, wave w owns: dh tiles (k-tile, v-tile) = ((w TPW + j) >> 1,
// (w TPW + j) & 1), TPW = VTW K / 64; the [64 x 32] products of step (i) at
// (t-tile w & 3, v-tile (w >> 2) VTW + x), x < VTW; the [64 x K] accumulators at
// t-tile w & 3, k-tiles ((w >> 2) VTW + x) APW + j, APW = K / 32.  At K = 192
// every level's dh (96 registers) and the three accumulators (72) leave too
// few registers for the products and some values spill.
template <int KD>
constexpr int gdn_bscan_waves() { return 8; }

// E: the 16-bit format of q_new, W_new, K_new, U, dO and the saved states (bf16,
// or fp16 for fp16 inputs; fp16 MFMA).  The per-V-slice partial gradients are
// bf16 either way (summed in fp32 by the chunk kernel).
template <int KD, typename TL, typename E = __bf16>
__global__ __launch_bounds__(64 * gdn_bscan_waves<KD>(), 1) void gdn_bwd_scan_kernel(
    const __bf16* __restrict__ qn, const __bf16* __restrict__ wn, const __bf16* __restrict__ kn,
    const __bf16* __restrict__ un, const __bf16* __restrict__ dO, const float* __restrict__ gcum,
    const TL* __restrict__ l, const __bf16* __restrict__ hsave, __bf16* __restrict__ dq_p,
    __bf16* __restrict__ dw_p, __bf16* __restrict__ dk_p, float* __restrict__ du,
    float* __restrict__ dl_p, float* __restrict__ del_p, int B, int T, int H, int V, int L,
    int nlev, int strong) {
  using Sm = GdnBscanSmem<KD>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Sm& s = *(Sm*)smem_raw;
  constexpr int NW = gdn_bscan_waves<KD>(), NTH = 64 * NW, VTW = 8 / NW;
  constexpr int LK = Sm::LK, LVS = Sm::LVS, TPW = VTW * KD / 64, APW = KD / 32;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int tt = w & 3, vt0 = (w >> 2) * VTW;   // step (i) tiles; tt is also the accumulators' t-tile
  const int nvb = V / kBVs;
  const int vb = blockIdx.x % nvb;
  const int row = blockIdx.x / nvb;
  const int b = row / H, h = row % H;
  const int NT = T / kGC;
  const size_t hk = (size_t)H * KD, hv = (size_t)H * V;
  const size_t BTH = (size_t)B * T * H;
  const int v0 = vb * kBVs;

  floatx4 dh[kGBwdMaxLev][TPW];
#pragma unroll
  for (int e = 0; e < kGBwdMaxLev; ++e)
#pragma unroll
    for (int j = 0; j < TPW; ++j) dh[e][j] = zero4();

  // Register prefetch: the saved state of the next (chunk, level) pair is
  // loaded while the current level computes (thread tid owns 16-byte unit tid
  // of the [32 x K] slice), and the next chunk's q_new / W_new / K_new / U / dO
  // tiles, lambda columns and last decay while the current chunk computes
  // (K = 64 only: with K = 128 those registers would spill, and the tiles are
  // loaded at the chunk start).  Every load is issued unconditionally, clamped
  // to a valid address where its value is not used: a load under a condition
  // makes the compiler merge its registers after the branch, which waits for
  // the load right away.
  constexpr bool kPrefTiles = KD <= 64;
  constexpr int UPR = KD / 8, QU = kGC * UPR / NTH;   // units per row / per thread
  constexpr int HU = (kBVs * UPR + NTH - 1) / NTH;     // units of the saved state per thread
  static_assert(kGC * UPR % NTH == 0 && kGC * kBVs / 8 <= NTH, "units per thread");
  const __bf16* hsrow = hsave + (size_t)row * NT * nlev * V * KD + (size_t)v0 * KD;
  u32x4 ph[HU];
  auto fetch_h = [&](int jc, int e) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < HU; ++i) {
      const int u = (tid + NTH * i) % (kBVs * UPR);
      ph[i] = *(const u32x4*)(hsrow + ((size_t)jc * nlev + e) * V * KD + (size_t)(u / UPR) * KD +
                              8 * (u % UPR));
    }
  };
  u32x4 pq[QU], pw[QU], pk[QU], pu, pdo;
  float plam, peL;
  auto fetch_tiles = [&](int jc) __attribute__((always_inline)) {
    const size_t t0 = (size_t)b * T + (size_t)jc * kGC;
#pragma unroll
    for (int i = 0; i < QU; ++i) {
      const int u = tid + NTH * i, r = u / UPR, c = 8 * (u % UPR);
      const size_t off = (t0 + r) * hk + (size_t)h * KD + c;
      pq[i] = *(const u32x4*)(qn + off);
      pw[i] = *(const u32x4*)(wn + off);
      pk[i] = *(const u32x4*)(kn + off);
    }
    {
      const int u = tid % (kGC * kBVs / 8);
      const size_t off = (t0 + (u >> 2)) * hv + (size_t)h * V + v0 + 8 * (u & 3);
      pu = *(const u32x4*)(un + off);
      pdo = *(const u32x4*)(dO + off);
    }
    const int nl1 = nlev > 0 ? nlev : 1;   // T = 64 has no inter-chunk level
    const int le = min(tid, nl1 * kGC - 1);
    plam = to_f32<TL>(l[((t0 + le / nl1) * H + h) * L + min(7 + le % nl1, L - 1)]);
    peL = gcum[(t0 + kGC - 1) * H + h];
  };
  if (kPrefTiles) fetch_tiles(NT - 1);
  fetch_h(NT - 1, 0);
  const rsrc_t rdl = make_rsrc(dl_p + ((size_t)vb * BTH + h) * nlev,
                               w == 0 ? (size_t)B * T * H * nlev * 4 : 0);

  for (int ic = NT - 1; ic >= 0; --ic) {
    const size_t tok0 = (size_t)b * T + (size_t)ic * kGC;
    if (!kPrefTiles) fetch_tiles(ic);
#pragma unroll
    for (int i = 0; i < QU; ++i) {
      const int u = tid + NTH * i, r = u / UPR, c = 8 * (u % UPR);
      *(u32x4*)(s.qn + r * LK + c) = pq[i];
      *(u32x4*)(s.wn + r * LK + c) = pw[i];
      *(u32x4*)(s.kn + r * LK + c) = pk[i];
    }
    if (tid < kGC * kBVs / 8) {
      *(u32x4*)(s.u + (tid >> 2) * LVS + 8 * (tid & 3)) = pu;
      *(u32x4*)(s.dO + (tid >> 2) * LVS + 8 * (tid & 3)) = pdo;
    }
    if (tid < nlev * kGC) s.lam[tid % nlev][tid / nlev] = plam;
    const float eL = fexp(peL);
    // the first level's barrier publishes the tiles; the prefetch registers are
    // reloaded after it

    floatx4 adq[VTW * APW], adw[VTW * APW], adk[VTW * APW], adu[VTW];
#pragma unroll
    for (int j = 0; j < VTW * APW; ++j) adq[j] = adw[j] = adk[j] = zero4();
#pragma unroll
    for (int x = 0; x < VTW; ++x) adu[x] = zero4();
    float del = 0.f;

    // the level loop stays rolled (an unrolled one holds every level's fragments
    // at once); slot 0 of the dh array is the current level and the array
    // rotates by one level per iteration (kGBwdMaxLev iterations, the levels
    // >= nlev only rotating), so it is only indexed by constants.  The level's
    // read / write / no-reset flags enter the products as 0 / 1 factors or
    // operand selects, so that its LDS reads and MFMAs issue without a branch
    // per product.
#pragma unroll 1
    for (int e = 0; e < kGBwdMaxLev; ++e) {
      floatx4 cur[TPW];
#pragma unroll
      for (int j = 0; j < TPW; ++j) cur[j] = dh[0][j];
      if (e < nlev) {
        const int per = 2 << e;
        const bool bit = (ic >> e) & 1;
        // the forward's level read: bit e set; strong: every chunk reads every
        // level >= 1 and none reads level 0 (the writes keep the weak masks)
        const bool rd = strong ? e >= 1 : bit;
        const bool nr = (ic & (per - 1)) != per - 1;
        const float frd = rd ? 1.f : 0.f, fwr = bit ? 0.f : 1.f, fnr = nr ? 1.f : 0.f;
#pragma unroll
        for (int i = 0; i < HU; ++i) {
          const int u = tid + NTH * i;
          if (u < kBVs * UPR) *(u32x4*)(s.hs + (u / UPR) * LK + 8 * (u % UPR)) = ph[i];
        }
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
          const int kt = (w * TPW + j) >> 1, vv = (w * TPW + j) & 1;
          *(bf16x4*)(s.dhs + (16 * vv + ln) * LK + 16 * kt + 4 * lq) = cvt4e<E>(cur[j]);
        }
        __syncthreads();
        {
          const bool nxt = e + 1 < nlev;
          fetch_h(nxt ? ic : max(ic - 1, 0), nxt ? e + 1 : 0);
        }
        if (kPrefTiles && e == 0) fetch_tiles(max(ic - 1, 0));
        // lambda_e o dO, once per level for the products of steps (ii), (iii): written
        // after the barrier that publishes the chunk's dO and lambda (and that
        // orders it after the previous level's readers), read after the next one
        for (int u = tid; u < kGC * kBVs / 4; u += NTH) {
          const int t = u / (kBVs / 4), c = 4 * (u % (kBVs / 4));
          const float la = s.lam[e][t];
          const bf16x4 x = *(const bf16x4*)(s.dO + t * LVS + c);
          *(bf16x4*)(s.ldo + t * LVS + c) =
              bf16x4{to16<E>(from16<E>(x[0]) * la), to16<E>(from16<E>(x[1]) * la),
                     to16<E>(from16<E>(x[2]) * la), to16<E>(from16<E>(x[3]) * la)};
        }

        // (i) dV_new = K_new dh, V_new = wr U - nr W_new h, q_new h (for dlambda)
#pragma unroll
        for (int x = 0; x < VTW; ++x) {
          const int vt = vt0 + x;
          floatx4 dv = zero4(), y = zero4(), z = zero4();
#pragma unroll
          for (int c = 0; c < KD / 32; ++c) {
            // bound the operand loads in flight (registers) for the wide K
            if (KD > 128) __builtin_amdgcn_sched_barrier(0);
            const bf16x8 bd = *(const bf16x8*)(s.dhs + (16 * vt + ln) * LK + 32 * c + 8 * lq);
            const bf16x8 bh = *(const bf16x8*)(s.hs + (16 * vt + ln) * LK + 32 * c + 8 * lq);
            dv = mfma16<E>(*(const bf16x8*)(s.kn + (16 * tt + ln) * LK + 32 * c + 8 * lq), bd, dv);
            y = mfma16<E>(*(const bf16x8*)(s.wn + (16 * tt + ln) * LK + 32 * c + 8 * lq), bh, y);
            z = mfma16<E>(*(const bf16x8*)(s.qn + (16 * tt + ln) * LK + 32 * c + 8 * lq), bh, z);
          }
          bf16x4 dvb, vnb;
          float dlr[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = 16 * tt + 4 * lq + i;
            vnb[i] = to16<E>(fwr * from16<E>(s.u[t * LVS + 16 * vt + ln]) - fnr * y[i]);
            dvb[i] = to16<E>(dv[i]);
            adu[x][i] += fwr * dv[i];
            dlr[i] = frd * from16<E>(s.dO[t * LVS + 16 * vt + ln]) * z[i];
          }
          *(bf16x4*)(s.dvn + (16 * vt + ln) * kLd64 + 16 * tt + 4 * lq) = dvb;
          *(bf16x4*)(s.vn + (16 * vt + ln) * kLd64 + 16 * tt + 4 * lq) = vnb;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float xs = row_sum16(dlr[i]);
            if (ln == 0) s.dlr[vt][16 * tt + 4 * lq + i] = xs;
          }
        }
        __syncthreads();
        // wave 0's lanes store the level's dlambda row sums; the other waves store
        // through an empty range, so the store is unconditional and the memory
        // waits of the walk count exactly
        buf_store<float>(s.dlr[0][lane] + s.dlr[1][lane], rdl,
                         (unsigned int)((lane * H) * nlev + e) * 4, (unsigned int)(tok0 * H * nlev * 4));

        // (ii) contractions over this slice's 32 columns of V
        {
          // A operands with the level's factors in their rows (t = 16 tt + ln): the
          // staged lambda_e o dO, and the read / no-reset flags as selects, so the
          // three accumulators take plain MFMA accumulation
          const bf16x8 ldo8 = *(const bf16x8*)(s.ldo + (16 * tt + ln) * LVS + 8 * lq);
          const bf16x8 dvn8 = tr_frag(s.dvn, kLd64, 0, 16 * tt);   // dV_new[t][v]
          const bf16x8 adO = rd ? ldo8 : bf16x8{};
          const bf16x8 advn = nr ? dvn8 : bf16x8{};
          const bf16x8 avn = tr_frag(s.vn, kLd64, 0, 16 * tt);     // V_new[t][v]
#pragma unroll
          for (int j = 0; j < VTW * APW; ++j) {
            if (KD > 128 && (j & 1) == 0) __builtin_amdgcn_sched_barrier(0);
            const int kt = vt0 * APW + j;
            const bf16x8 bh = tr_frag(s.hs, LK, 0, 16 * kt);    // h^T[v][k]
            const bf16x8 bd = tr_frag(s.dhs, LK, 0, 16 * kt);   // dh^T[v][k]
            adq[j] = mfma16<E>(adO, bh, adq[j]);
            adw[j] = mfma16<E>(advn, bh, adw[j]);
            adk[j] = mfma16<E>(avn, bd, adk[j]);
          }
          float dd = 0.f;
#pragma unroll
          for (int j = 0; j < TPW; ++j) {
            const int kt = (w * TPW + j) >> 1, vv = (w * TPW + j) & 1;
            const bf16x4 hv4 = *(const bf16x4*)(s.hs + (16 * vv + ln) * LK + 16 * kt + 4 * lq);
#pragma unroll
            for (int i = 0; i < 4; ++i) dd += from16<E>(hv4[i]) * cur[j][i];
          }
          del += fnr * dd;
        }

        // (iii) dh_e <- nr (eL dh_e - W_new^T dV_new) + rd q_new^T (lambda_e o dO)
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
          if (KD > 128) __builtin_amdgcn_sched_barrier(0);
          const int kt = (w * TPW + j) >> 1, vv = (w * TPW + j) & 1;
          floatx4 tw = zero4(), tq = zero4();
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const bf16x8 bdv = *(const bf16x8*)(s.dvn + (16 * vv + ln) * kLd64 + 32 * c + 8 * lq);
            tw = mfma16<E>(tr_frag(s.wn, LK, 32 * c, 16 * kt), bdv, tw);
            const bf16x8 x = tr_frag(s.ldo, LVS, 32 * c, 16 * vv);   // (lambda_e o dO)[t][v]
            tq = mfma16<E>(tr_frag(s.qn, LK, 32 * c, 16 * kt), x, tq);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) cur[j][i] = fnr * (eL * cur[j][i] - tw[i]) + frd * tq[i];
        }
        __syncthreads();
      }
      // rotate: level e + 1 moves to slot 0; after all kGBwdMaxLev steps every
      // level is back in its own slot
#pragma unroll
      for (int l = 0; l + 1 < kGBwdMaxLev; ++l)
#pragma unroll
        for (int j = 0; j < TPW; ++j) dh[l][j] = dh[l + 1][j];
#pragma unroll
      for (int j = 0; j < TPW; ++j) dh[kGBwdMaxLev - 1][j] = cur[j];
    }

    // ---- the chunk's outputs -----------------------------------------------------
#pragma unroll
    for (int j = 0; j < VTW * APW; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const size_t o = ((size_t)vb * BTH + (tok0 + 16 * tt + 4 * lq + i) * H + h) * KD +
                         16 * (vt0 * APW + j) + ln;
        dq_p[o] = (__bf16)adq[j][i];
        dw_p[o] = (__bf16)-adw[j][i];
        dk_p[o] = (__bf16)adk[j][i];
      }
#pragma unroll
    for (int x = 0; x < VTW; ++x)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        du[((tok0 + 16 * tt + 4 * lq + i) * H + h) * V + v0 + 16 * (vt0 + x) + ln] = adu[x][i];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) del += __shfl_xor(del, off, 64);
    if (lane == 0) s.red[w] = del;
    __syncthreads();
    if (tid == 0) {
      float x = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) x += s.red[w2];
      del_p[(size_t)vb * B * H * NT + (size_t)row * NT + ic] = x;
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 4: chunk-local backward
// ---------------------------------------------------------------------------
// QG (K > 192): q is not staged in LDS (the tile would not fit next to the
// fp32 matrices); its fragments come from global memory (L2) and each
// 64-column block is staged beside the fp32 staging tile when a step needs it.
template <int KD, int VD>
struct GdnBchunkSmem {
  static constexpr bool QG = KD > 192;
  static constexpr int LK = KD + 8;
  static constexpr int LS = 64 + 4;     // fp32 staging row stride (64-column blocks)
  static constexpr int LDB = 64 + 8;    // bf16 staging row stride
  static constexpr int NR = 2 * kGC * kLM;
  static_assert(kGC * LS + kGC * LDB / 2 <= NR, "step 14 staging fits the S4 | S5 region");
  __bf16 q[QG ? 8 : kGC * LK];
  __bf16 k[kGC * LK];
  float m[4][kGC * kLM];   // S0 .. S3: 64 x 64 fp32 matrices
  float rg[NR];            // S4 | S5, or the fp32 (and bf16) staging tiles, or the inverse scratch
  float gc[kGC], e[kGC], r[kGC], beta[kGC];
  float lam[7][kGC];       // lambda[t, 0..6]
  float dlam[7][kGC];      // intra-chunk dlambda
  float dgr[kGC];          // dGc: contributions of each row's owner
  float dgcol[4][kGC];     // dGc: column-sum contributions, per wave
  float dbr[kGC];          // dbeta
  float lastc[kGC];        // contributions to dGc_last
  float rq[kGC], rk[kGC];  // 1 / ||q_t||, 1 / ||k_t|| (in-kernel l2 normalisation)
};

// fp32 fragments of a 16 x 32 MFMA operand held in a row-major fp32 matrix:
// element j of lane (lq, ln) is the operand's (non-contracted ln, contracted
// 8lq + j) entry.  frn: stored [non-contracted][contracted]; frt: stored
// [contracted][non-contracted].
template <int LD>
__device__ __forceinline__ void frn(const float* X, int r0, int c0, float* f) {
  const int lane = threadIdx.x & 63;
  const float* p = X + (r0 + (lane & 15)) * LD + c0 + 8 * (lane >> 4);
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = p[j];
}
template <int LD>
__device__ __forceinline__ void frt(const float* X, int r0, int c0, float* f) {
  const int lane = threadIdx.x & 63;
  const float* p = X + (c0 + 8 * (lane >> 4)) * LD + r0 + (lane & 15);
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = p[j * LD];
}
// Four consecutive elements of bf16 or fp32 memory as fp32.
template <typename T>
__device__ __forceinline__ floatx4 ld4f(const T* p) {
  if constexpr (sizeof(T) == 4) {
    return *(const floatx4*)p;
  } else {
    const bf16x4 x = *(const bf16x4*)p;
    return floatx4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
  }
}
// An fp32 fragment of a 16 x 32 MFMA operand from global rows of stride rs,
// sc * the sum over NP partials pstride apart (element j of lane (lq, ln): row
// r0 + ln, column c0 + 8 lq + j), in two halves: frg_load issues the loads
// (raw values in registers), frg_done sums and scales, so the loads can be
// issued a step before the fragment is used.
template <int NP, typename T>
struct FrgPf {
  using V4 = typename std::conditional<sizeof(T) == 4, floatx4, bf16x4>::type;
  V4 a[NP], b[NP];
};
template <int NP, typename T>
__device__ __forceinline__ void frg_load(FrgPf<NP, T>& f, const T* X, size_t rs, size_t pstride,
                                         int r0, int c0) {
  const int lane = threadIdx.x & 63;
  const T* p = X + (size_t)(r0 + (lane & 15)) * rs + c0 + 8 * (lane >> 4);
#pragma unroll
  for (int pp = 0; pp < NP; ++pp) {
    f.a[pp] = *(const typename FrgPf<NP, T>::V4*)(p + pp * pstride);
    f.b[pp] = *(const typename FrgPf<NP, T>::V4*)(p + pp * pstride + 4);
  }
}
template <int NP, typename T>
__device__ __forceinline__ void frg_done(const FrgPf<NP, T>& f, float sc, float* out) {
  floatx4 a = zero4(), b = zero4();
#pragma unroll
  for (int pp = 0; pp < NP; ++pp) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[j] += (float)f.a[pp][j];
      b[j] += (float)f.b[pp][j];
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out[j] = sc * a[j];
    out[4 + j] = sc * b[j];
  }
}
// bf16x3 products: both operands fp32 (three MFMAs), or fp32 x bf16 (two).
__device__ __forceinline__ floatx4 mma_ff(const float* a, const float* b, floatx4 c) {
  bf16x8 A[2], Bf[2];
  split8<2>(a, A);
  split8<2>(b, Bf);
  return mma<2>(A, Bf, c);
}
// E = fp16: the fp16 operand is exact as bf16 hi + lo (8 + 8 bits of mantissa,
// a wider exponent range), so the product is the bf16x3 one (three MFMAs).
template <typename E = __bf16>
__device__ __forceinline__ floatx4 mma_fb(const float* a, bf16x8 b, floatx4 c) {
  bf16x8 A[2];
  split8<2>(a, A);
  if constexpr (__is_same(E, _Float16)) {
    float bf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) bf[j] = from16<E>(b[j]);
    bf16x8 Bp[2];
    split8<2>(bf, Bp);
    return mma<2>(A, Bp, c);
  } else {
    c = mfma16x16x32(A[1], b, c);
    return mfma16x16x32(A[0], b, c);
  }
}
// ST[t][c] = (scale ? scale[t] : 1) * sum over NP partials of X[t][c], 64 rows of N.
// Two units per step with all their partial loads issued together.
template <int N, int LS, int NP, typename T>
__device__ __forceinline__ void stage_rows(float* ST, const T* X, size_t rs, size_t pstride,
                                           const float* scale) {
  constexpr int IT = kGC * N / 4 / 256;
  static_assert(IT % 2 == 0, "units per thread");
#pragma unroll 1
  for (int i0 = 0; i0 < IT; i0 += 2) {
    floatx4 pv[2][NP];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const int u = threadIdx.x + 256 * (i0 + d);
      const int t = u / (N / 4), c = 4 * (u % (N / 4));
#pragma unroll
      for (int pp = 0; pp < NP; ++pp) pv[d][pp] = ld4f(X + (size_t)t * rs + c + pp * pstride);
    }
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const int u = threadIdx.x + 256 * (i0 + d);
      const int t = u / (N / 4), c = 4 * (u % (N / 4));
      floatx4 a = pv[d][0];
#pragma unroll
      for (int pp = 1; pp < NP; ++pp) a += pv[d][pp];
      if (scale) a *= scale[t];
      *(floatx4*)(ST + t * LS + c) = a;
    }
  }
}

// stage_rows of 64 bf16 partial rows of 64 columns in two halves: rows_load
// issues every load of the block (4 units per thread, NP partials each) into
// registers, rows_store sums, scales and writes them to ST later, so the loads
// of a block fly while an earlier step computes.
template <int NP>
struct RowsPf {
  bf16x4 x[4][NP];
};
template <int NP>
__device__ __forceinline__ void rows_load(RowsPf<NP>& pf, const __bf16* X, size_t rs,
                                          size_t pstride) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int u = threadIdx.x + 256 * d, t = u >> 4, c = 4 * (u & 15);
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) pf.x[d][pp] = *(const bf16x4*)(X + (size_t)t * rs + c + pp * pstride);
  }
}
template <int LS, int NP>
__device__ __forceinline__ void rows_store(float* ST, const RowsPf<NP>& pf, const float* scale) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int u = threadIdx.x + 256 * d, t = u >> 4, c = 4 * (u & 15);
    floatx4 a = zero4();
#pragma unroll
    for (int pp = 0; pp < NP; ++pp)
      a += floatx4{(float)pf.x[d][pp][0], (float)pf.x[d][pp][1], (float)pf.x[d][pp][2],
                   (float)pf.x[d][pp][3]};
    if (scale) a *= scale[t];
    *(floatx4*)(ST + t * LS + c) = a;
  }
}

// Store a 64 x (16 NKT) gradient held in the MFMA D layout (x[nt][i] is row
// t16 + 4lq + i, column 16 nt + ln) as bf16 rows of stride ld.  With norm set,
// the rows are the gradient w.r.t. y = x r s (r = 1 / ||x||, staged y in Y)
// and the stored gradient is w.r.t. x: r s (x - y' (y' . x)), y' = y / s.
// yat(t, c): the staged (normalised, scaled) value of row t, column c.
template <int NKT, typename E, typename YAt>
__device__ __forceinline__ void store_l2norm_grad(float (&x)[NKT][4], YAt yat,
                                                  const float* rinv, float inv_s, float s,
                                                  int norm, __bf16* out, size_t ld, int t16) {
  const int lane = threadIdx.x & 63, lq = lane >> 4, ln = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t16 + 4 * lq + i;
    float f = 1.f, dot = 0.f;
    if (norm) {
#pragma unroll
      for (int nt = 0; nt < NKT; ++nt) dot += yat(t, 16 * nt + ln) * inv_s * x[nt][i];
      dot = row_sum16(dot);
      f = rinv[t] * s;
    }
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt) {
      const float y = norm ? yat(t, 16 * nt + ln) * inv_s : 0.f;
      out[t * ld + 16 * nt + ln] = to16<E>(f * (x[nt][i] - y * dot));
    }
  }
}

// STRONG: lambda of an intra-chunk pair at its strong level (the forward's P).
// E: the 16-bit format of q, k, v, dO, dq, dk, dv (bf16, or fp16 for fp16 inputs).
template <int KD, int VD, typename TB, typename TL, bool STRONG = false, typename E = __bf16>
__global__ __launch_bounds__(256, 1) void gdn_bwd_chunk_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const TB* __restrict__ beta, const float* __restrict__ gcum, const TL* __restrict__ l,
    const __bf16* __restrict__ dO, const __bf16* __restrict__ dq_p, const __bf16* __restrict__ dw_p,
    const __bf16* __restrict__ dk_p, const float* __restrict__ du, const float* __restrict__ dl_p,
    const float* __restrict__ del_p, __bf16* __restrict__ dq, __bf16* __restrict__ dk,
    __bf16* __restrict__ dv, TB* __restrict__ db, float* __restrict__ dg, float* __restrict__ dl,
    int B, int T, int H, int L, int nlev, int norm_qk, float qk_scale) {
  using Sm = GdnBchunkSmem<KD, VD>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Sm& s = *(Sm*)smem_raw;
  constexpr int LK = Sm::LK, LS = Sm::LS, LDB = Sm::LDB, NKT = KD / 16;
  constexpr int NPV = VD / kBVs;   // V slices of the level scan = partials per entry
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int NT = T / kGC;
  const int ic = blockIdx.x % NT, row = blockIdx.x / NT;
  const int b = row / H, h = row % H;
  const size_t tok0 = (size_t)b * T + (size_t)ic * kGC;
  const size_t hk = (size_t)H * KD, hv = (size_t)H * VD;
  const size_t BTH = (size_t)B * T * H;
  const size_t rowk = (tok0 * H + h) * KD, rowv = (tok0 * H + h) * VD;
  float* S0 = s.m[0];
  float* S1 = s.m[1];
  float* S2 = s.m[2];
  float* S3 = s.m[3];
  float* S4 = s.rg;
  float* S5 = s.rg + kGC * kLM;
  float* ST = s.rg;
  const int t16 = 16 * w;   // this wave's 16-row tile

  // ---- load ------------------------------------------------------------------
  constexpr bool QG = Sm::QG;
  g2s_tile<KD>(k + rowk, hk, s.k, LK);
  if constexpr (!QG) g2s_tile<KD>(q + rowk, hk, s.q, LK);
  if (norm_qk) {
    // use_qk_l2norm_in_kernel: the gradients below are w.r.t. q scale / ||q|| and
    // k / ||k||; the chain rule back to q and k is applied where dq, dk are stored
    if constexpr (QG) l2norm_rinv_global<KD, E>(q + rowk, hk, s.rq);
    __syncthreads();
    if constexpr (!QG) l2norm_rows<KD, LK, 0, E>(s.q, qk_scale, s.rq);
    l2norm_rows<KD, LK, 0, E>(s.k, 1.f, s.rk);
  }
  // the staged value of q[t][c] (QG: from global memory, normalised as staged)
  auto q_at = [&](int t, int c) -> float {
    if constexpr (QG) {
      const float x = from16<E>(q[rowk + (size_t)t * hk + c]);
      return norm_qk ? from16<E>(to16<E>(from16<E>(to16<E>(x * s.rq[t])) * qk_scale)) : x;
    } else {
      return from16<E>(s.q[t * LK + c]);
    }
  };
  if (w == 0) {
    const float x = gcum[(tok0 + lane) * H + h];
    const float gl = __shfl(x, kGC - 1, 64);
    s.gc[lane] = x;
    s.e[lane] = fexp(x);
    s.r[lane] = fexp(gl - x);
    s.beta[lane] = to_f32<TB>(beta[(tok0 + lane) * H + h]);
  }
  {
    float lv[2];   // both loads issued before either store
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int u = min(tid + 256 * i, 7 * kGC - 1);
      lv[i] = to_f32<TL>(l[((tok0 + u / 7) * H + h) * L + u % 7]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int u = tid + 256 * i;
      if (u < 7 * kGC) {
        s.lam[u % 7][u / 7] = lv[i];
        s.dlam[u % 7][u / 7] = 0.f;
      }
    }
  }
  if (tid < kGC) {
    s.dgr[tid] = s.dbr[tid] = s.lastc[tid] = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) s.dgcol[w2][tid] = 0.f;
  }
  __syncthreads();

  // ---- 1: A = strict-tril(beta_t K K^T) -> S0, M = tril(Q K^T) -> S1 ---------------
  {
    floatx4 kk[4], qk[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) kk[nt] = qk[nt] = zero4();
#pragma unroll
    for (int c = 0; c < KD / 32; ++c) {
      const bf16x8 ak = *(const bf16x8*)(s.k + (t16 + ln) * LK + 32 * c + 8 * lq);
      bf16x8 aq;
      if constexpr (QG) {
        aq = *(const bf16x8*)(q + rowk + (size_t)(t16 + ln) * hk + 32 * c + 8 * lq);
        if (norm_qk) aq = l2norm_scale8<E>(aq, s.rq[t16 + ln], qk_scale);
      } else {
        aq = *(const bf16x8*)(s.q + (t16 + ln) * LK + 32 * c + 8 * lq);
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const bf16x8 bk = *(const bf16x8*)(s.k + (16 * nt + ln) * LK + 32 * c + 8 * lq);
        kk[nt] = mfma16<E>(ak, bk, kk[nt]);
        qk[nt] = mfma16<E>(aq, bk, qk[nt]);
      }
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t16 + 4 * lq + i, sc = 16 * nt + ln;
        S0[t * kLM + sc] = sc < t ? s.beta[t] * kk[nt][i] : 0.f;
        S1[t * kLM + sc] = sc <= t ? qk[nt][i] : 0.f;
      }
  }
  __syncthreads();

  // ---- 2: Aw = (I + A)^-1 -> S2 (fp32 MFMA, the forward's inverse) --------------------
  static_assert(kGC * kLM >= kInvScratchFloats, "inverse scratch fits S5");
  tri_inv64_mfma<256>(S0, S2, S5);

  // ---- 3: P = M Aw -> S3 ------------------------------------------------------------
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    floatx4 acc = zero4();
    if (nt <= w) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float a[8], bb[8];
        frn<kLM>(S1, t16, 32 * c, a);
        frt<kLM>(S2, 16 * nt, 32 * c, bb);
        acc = mma_ff(a, bb, acc);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) S3[(t16 + 4 * lq + i) * kLM + 16 * nt + ln] = acc[i];
  }
  __syncthreads();

  // step 5's fragments of X = e o dq_new (partials) are loaded while step 4 computes
  FrgPf<NPV, __bf16> pfx[KD / 32];
#pragma unroll
  for (int c = 0; c < KD / 32; ++c) frg_load(pfx[c], dq_p + rowk, hk, BTH * KD, t16, 32 * c);

  // ---- 4: Z = dO V^T; Z o P o Gamma -> S0, dP = Z o Gamma o Lambda o beta_s -> S4 -----
  {
    bf16x8 ad[VD / 32];
#pragma unroll
    for (int c = 0; c < VD / 32; ++c) ad[c] = *(const bf16x8*)(dO + rowv + (size_t)(t16 + ln) * hv + 32 * c + 8 * lq);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      floatx4 z = zero4();
      if (nt <= w) {
#pragma unroll
        for (int c = 0; c < VD / 32; ++c)
          z = mfma16<E>(ad[c], *(const bf16x8*)(v + rowv + (size_t)(16 * nt + ln) * hv + 32 * c + 8 * lq), z);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t16 + 4 * lq + i, sc = 16 * nt + ln;
        float zp = 0.f, dp = 0.f;
        if (sc <= t) {
          const float gam = fexp(s.gc[t] - s.gc[sc]);
          zp = z[i] * S3[t * kLM + sc] * gam;
          dp = z[i] * gam * s.lam[gdn_intra_level<STRONG>(t, sc)][t] * s.beta[sc];
        }
        S0[t * kLM + sc] = zp;
        S4[t * kLM + sc] = dp;
      }
    }
  }
  __syncthreads();

  // ---- 4b: intra-chunk dlambda; Gamma term of o_intra in dGc --------------------------
  // four threads per row t (consecutive lanes), each over 16 columns s, then
  // four per column s over 16 rows t; the partial sums meet by lane shuffles
  {
    const int r = tid >> 2, part = tid & 3, c0 = 16 * part;
    float dlv[7] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float rs = 0.f;
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int sc = c0 + x;
      if (sc <= r) {
        const int lv = gdn_intra_level<STRONG>(r, sc);
        const float val = S0[r * kLM + sc] * s.beta[sc];
#pragma unroll
        for (int l = 0; l < 7; ++l) dlv[l] += l == lv ? val : 0.f;
        rs += val * s.lam[lv][r];
      }
    }
    float cs = 0.f;
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int t = c0 + x;
      if (t >= r) cs += S0[t * kLM + r] * s.lam[gdn_intra_level<STRONG>(t, r)][t];
    }
#pragma unroll
    for (int l = 0; l < 7; ++l) {
      dlv[l] += __shfl_xor(dlv[l], 1, 64);
      dlv[l] += __shfl_xor(dlv[l], 2, 64);
    }
    rs += __shfl_xor(rs, 1, 64);
    rs += __shfl_xor(rs, 2, 64);
    cs += __shfl_xor(cs, 1, 64);
    cs += __shfl_xor(cs, 2, 64);
    if (part == 0) {
#pragma unroll
      for (int l = 0; l < 7; ++l) s.dlam[l][r] += dlv[l];
      s.dgr[r] += rs;
      s.dgcol[1][r] -= cs * s.beta[r];
    }
  }
  __syncthreads();

  // ---- 5: F1 = X K^T (X = e o dq_new); E = dP - F1 o beta_s -> S4; F1 o beta_s -> S0 ---
  {
    float ax[KD / 32][8];
#pragma unroll
    for (int c = 0; c < KD / 32; ++c) frg_done(pfx[c], s.e[t16 + ln], ax[c]);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      floatx4 f = zero4();
#pragma unroll
      for (int c = 0; c < KD / 32; ++c)
        f = mma_fb<E>(ax[c], *(const bf16x8*)(s.k + (16 * nt + ln) * LK + 32 * c + 8 * lq), f);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t16 + 4 * lq + i, sc = 16 * nt + ln;
        const float fb = f[i] * s.beta[sc];
        S4[t * kLM + sc] -= fb;
        S0[t * kLM + sc] = fb;
      }
    }
  }
  __syncthreads();

  // step 7's fragments of e o dW_new (partials) and dU are loaded while step 6 computes
  FrgPf<NPV, __bf16> pfw[KD / 32];
  FrgPf<1, float> pfu[VD / 32];
#pragma unroll
  for (int c = 0; c < KD / 32; ++c) frg_load(pfw[c], dw_p + rowk, hk, BTH * KD, t16, 32 * c);
#pragma unroll
  for (int c = 0; c < VD / 32; ++c) frg_load(pfu[c], du + rowv, hv, 0, t16, 32 * c);

  // ---- 6: H = (F1 beta) Aw^T, D = E Aw^T; dGc_t -= rowsum(M o H); dM = tril(D) -> S0 --
  {
    floatx4 hacc[4], dacc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) hacc[nt] = dacc[nt] = zero4();
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float ah[8], ae[8];
      frn<kLM>(S0, t16, 32 * c, ah);
      frn<kLM>(S4, t16, 32 * c, ae);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        float bw[8];
        frn<kLM>(S2, 16 * nt, 32 * c, bw);
        hacc[nt] = mma_ff(ah, bw, hacc[nt]);
        dacc[nt] = mma_ff(ae, bw, dacc[nt]);
      }
    }
    float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) rs[i] += S1[(t16 + 4 * lq + i) * kLM + 16 * nt + ln] * hacc[nt][i];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = row_sum16(rs[i]);
      if (ln == 0) s.dgr[t16 + 4 * lq + i] -= x;
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t16 + 4 * lq + i, sc = 16 * nt + ln;
        S0[t * kLM + sc] = sc <= t ? dacc[nt][i] : 0.f;
      }
  }
  __syncthreads();

  // ---- 7: F2 = (e o dW_new) K^T, F3 = dU V^T; (F2 + F3 o Gamma) o beta_s -> S5;
  //         dGc from the W_new factor e and the Gamma of Au --------------------------
  {
    float a2[KD / 32][8], a3[VD / 32][8];
#pragma unroll
    for (int c = 0; c < KD / 32; ++c) frg_done(pfw[c], s.e[t16 + ln], a2[c]);
#pragma unroll
    for (int c = 0; c < VD / 32; ++c) frg_done(pfu[c], 1.f, a3[c]);
    float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      floatx4 f2 = zero4(), f3 = zero4();
#pragma unroll
      for (int c = 0; c < KD / 32; ++c)
        f2 = mma_fb<E>(a2[c], *(const bf16x8*)(s.k + (16 * nt + ln) * LK + 32 * c + 8 * lq), f2);
#pragma unroll
      for (int c = 0; c < VD / 32; ++c)
        f3 = mma_fb<E>(a3[c], *(const bf16x8*)(v + rowv + (size_t)(16 * nt + ln) * hv + 32 * c + 8 * lq), f3);
      float cs = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t16 + 4 * lq + i, sc = 16 * nt + ln;
        const float aw = S2[t * kLM + sc], bs = s.beta[sc];
        const float gam = sc <= t ? fexp(s.gc[t] - s.gc[sc]) : 0.f;
        const float t2 = f3[i] * bs * aw * gam;
        rs[i] += aw * f2[i] * bs + t2;
        cs += t2;
        S5[t * kLM + sc] = (f2[i] + f3[i] * gam) * bs;
      }
      cs = sum_lq(cs);
      if (lq == 0) s.dgcol[w][16 * nt + ln] -= cs;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = row_sum16(rs[i]);
      if (ln == 0) s.dgr[t16 + 4 * lq + i] += x;
    }
  }
  __syncthreads();

  // ---- 8: dAw = S5 + M^T E -> S5 ------------------------------------------------------
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    floatx4 acc = zero4();
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float a[8], bb[8];
      frt<kLM>(S1, t16, 32 * c, a);
      frt<kLM>(S4, 16 * nt, 32 * c, bb);
      acc = mma_ff(a, bb, acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) S5[(t16 + 4 * lq + i) * kLM + 16 * nt + ln] += acc[i];
  }
  __syncthreads();

  // the kb loop's first partial block (X) is loaded while steps 9 compute
  constexpr bool PF = KD <= 128;   // partial blocks prefetched into registers
  RowsPf<NPV> pf;
  if constexpr (PF) rows_load<NPV>(pf, dq_p + rowk, hk, BTH * KD);

  // ---- 9: Y = dAw Aw^T -> S1; dA = -strict-tril(Aw^T Y) -> S1 --------------------------
  {
    floatx4 acc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      acc[nt] = zero4();
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float a[8], bb[8];
        frn<kLM>(S5, t16, 32 * c, a);
        frn<kLM>(S2, 16 * nt, 32 * c, bb);
        acc[nt] = mma_ff(a, bb, acc[nt]);
      }
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) S1[(t16 + 4 * lq + i) * kLM + 16 * nt + ln] = acc[nt][i];
  }
  __syncthreads();
  {
    floatx4 acc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      acc[nt] = zero4();
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float a[8], bb[8];
        frt<kLM>(S2, t16, 32 * c, a);
        frt<kLM>(S1, 16 * nt, 32 * c, bb);
        acc[nt] = mma_ff(a, bb, acc[nt]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ii = t16 + 4 * lq + i, jj = 16 * nt + ln;
        S1[ii * kLM + jj] = jj < ii ? -acc[nt][i] : 0.f;
      }
  }
  __syncthreads();

  // live: S0 = dM, S1 = dA, S2 = Aw, S3 = P; the staging region is free.
  // Steps 10 - 13 run per 64-column block kb of K (the staged blocks of X,
  // e o dW_new and dK_new fit the staging region for every K); dq and dk stay
  // in registers until the l2norm chain rule, which needs whole rows.
  float dqh[NKT][4], dkh[NKT][4];
  float qx = 0.f;                                   // rowdot(X, Q), thread (t = tid >> 2, part)
  float rb[4] = {0.f, 0.f, 0.f, 0.f}, kd[4] = {0.f, 0.f, 0.f, 0.f};
  // QG: the block of q the steps below read, [t][k] bf16 beside the staging tile
  __bf16* SQ = (__bf16*)(s.rg + kGC * LS);
  const __bf16* QB = QG ? SQ : s.q;    // Q block base and row stride for steps 10, 12
  constexpr int LQB = QG ? LDB : LK;
#pragma unroll
  for (int kb = 0; kb < KD / 64; ++kb) {
    const int k0 = 64 * kb;
    const int kq = QG ? 0 : k0;        // column of the block in QB
    if constexpr (QG) {
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int u = tid + 256 * rr, t = u >> 3, c = 8 * (u & 7);
        bf16x8 x = *(const bf16x8*)(q + rowk + (size_t)t * hk + k0 + c);
        if (norm_qk) x = l2norm_scale8<E>(x, s.rq[t], qk_scale);
        *(bf16x8*)(SQ + t * LDB + c) = x;
      }
    }
    // ---- 10: X -> ST; dQ = X + dM K; U2 = -P^T X; dGc += rowdot(X, Q) ----------------
    // (PF: each block's partial loads are issued one step before it is staged)
    if constexpr (PF) {
      rows_store<LS, NPV>(ST, pf, s.e);
      rows_load<NPV>(pf, dw_p + rowk + k0, hk, BTH * KD);
    } else {
      stage_rows<64, LS, NPV>(ST, dq_p + rowk + k0, hk, BTH * KD, s.e);
    }
    __syncthreads();
    floatx4 u2[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      floatx4 acc = zero4(), a2 = zero4();
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float am[8], ap[8], bx[8];
        frn<kLM>(S0, t16, 32 * c, am);
        acc = mma_fb<E>(am, tr_frag(s.k, LK, 32 * c, k0 + 16 * nt), acc);
        frt<kLM>(S3, t16, 32 * c, ap);
        frt<LS>(ST, 16 * nt, 32 * c, bx);
        a2 = mma_ff(ap, bx, a2);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) dqh[4 * kb + nt][i] = ST[(t16 + 4 * lq + i) * LS + 16 * nt + ln] + acc[i];
      u2[nt] = -a2;
    }
    {
      const int t = tid >> 2, part = tid & 3;
#pragma unroll
      for (int kk = 16 * part; kk < 16 * part + 16; ++kk)
        qx += ST[t * LS + kk] * from16<E>(QB[t * LQB + kq + kk]);
    }
    __syncthreads();

    // ---- 11: e o dW_new -> ST; U2 += Aw^T ST ---------------------------------------------
    if constexpr (PF) {
      rows_store<LS, NPV>(ST, pf, s.e);
      rows_load<NPV>(pf, dk_p + rowk + k0, hk, BTH * KD);
    } else {
      stage_rows<64, LS, NPV>(ST, dw_p + rowk + k0, hk, BTH * KD, s.e);
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float a[8], bb[8];
        frt<kLM>(S2, t16, 32 * c, a);
        frt<LS>(ST, 16 * nt, 32 * c, bb);
        u2[nt] = mma_ff(a, bb, u2[nt]);
      }
    __syncthreads();

    // ---- 12: U2 += dA K; U1 = dM^T Q + dA^T (beta o K) ----------------------------------
    floatx4 u1[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      floatx4 a1 = zero4();
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const bf16x8 bk = tr_frag(s.k, LK, 32 * c, k0 + 16 * nt);
        const bf16x8 bq = tr_frag(QB, LQB, 32 * c, kq + 16 * nt);
        float ad[8], am[8], at[8];
        frn<kLM>(S1, t16, 32 * c, ad);
        u2[nt] = mma_fb<E>(ad, bk, u2[nt]);
        frt<kLM>(S0, t16, 32 * c, am);
        a1 = mma_fb<E>(am, bq, a1);
        frt<kLM>(S1, t16, 32 * c, at);
#pragma unroll
        for (int j = 0; j < 8; ++j) at[j] *= s.beta[32 * c + 8 * lq + j];
        a1 = mma_fb<E>(at, bk, a1);
      }
      u1[nt] = a1;
    }

    // ---- 13: dK_new -> ST; dK = U1 + beta o U2 + r o dK_new; dbeta, dGc of K_new -------
    if constexpr (PF) {
      rows_store<LS, NPV>(ST, pf, nullptr);
      if (kb + 1 < KD / 64) rows_load<NPV>(pf, dq_p + rowk + k0 + 64, hk, BTH * KD);
    } else {
      stage_rows<64, LS, NPV>(ST, dk_p + rowk + k0, hk, BTH * KD, nullptr);
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int sr = t16 + 4 * lq + i, kk = 16 * nt + ln;
        const float kv = from16<E>(s.k[sr * LK + k0 + kk]), dkn = ST[sr * LS + kk];
        dkh[4 * kb + nt][i] = u1[nt][i] + s.beta[sr] * u2[nt][i] + s.r[sr] * dkn;
        rb[i] += kv * u2[nt][i];
        kd[i] += dkn * kv;
      }
    __syncthreads();
  }
  // dq = dq_hat, or with the in-kernel normalisation x -> y = x r (r = 1 / ||x||)
  // scaled by s: dq = r s (dq_hat - y (y . dq_hat)) (fla l2norm_bwd, kernel.py:24-29)
  store_l2norm_grad<NKT, E>(dqh, q_at, s.rq, norm_qk ? 1.f / qk_scale : 1.f, qk_scale, norm_qk,
                         dq + rowk, hk, t16);
  store_l2norm_grad<NKT, E>(dkh, [&](int t, int c) { return from16<E>(s.k[t * LK + c]); }, s.rk, 1.f,
                         1.f, norm_qk, dk + rowk, hk, t16);
  {
    qx += __shfl_xor(qx, 1, 64);
    qx += __shfl_xor(qx, 2, 64);
    if ((tid & 3) == 0) s.dgr[tid >> 2] += qx;
  }
  __syncthreads();   // the next updates of dGc come from other threads
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x = row_sum16(rb[i]), y = row_sum16(kd[i]);
    if (ln == 0) {
      const int sr = t16 + 4 * lq + i;
      s.dbr[sr] += x;
      s.dgr[sr] -= s.r[sr] * y;
      s.lastc[sr] = s.r[sr] * y;
    }
  }
  __syncthreads();

  // ---- 14: per 64-column block of V: dU, dO -> staging; GV = Au^T dU +
  //          (P o Gamma o Lambda)^T dO; dV = beta o GV -------------------------------------
  {
    __bf16* SD = (__bf16*)(s.rg + kGC * LS);   // dO block [t][v]
    float au[2][8], ar[2][8];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      frt<kLM>(S2, t16, 32 * c, au[c]);
      frt<kLM>(S3, t16, 32 * c, ar[c]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int t = 32 * c + 8 * lq + j, sc = t16 + ln;
        const float gam = t >= sc ? fexp(s.gc[t] - s.gc[sc]) : 0.f;
        au[c][j] *= gam;
        ar[c][j] *= gam * s.lam[gdn_intra_level<STRONG>(t, sc)][t];
      }
    }
    float rbv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int vb = 0; vb < VD / 64; ++vb) {
      const int v0 = 64 * vb;
      stage_rows<64, LS, 1>(ST, du + rowv + v0, hv, 0, nullptr);
      g2s_tile<64>(dO + rowv + v0, hv, SD, LDB);
      __syncthreads();
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        floatx4 acc = zero4();
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          float bu[8];
          frt<LS>(ST, 16 * nt, 32 * c, bu);
          acc = mma_ff(au[c], bu, acc);
          acc = mma_fb<E>(ar[c], tr_frag(SD, LDB, 32 * c, 16 * nt), acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int sr = t16 + 4 * lq + i, vv = v0 + 16 * nt + ln;
          dv[rowv + sr * hv + vv] = to16<E>(s.beta[sr] * acc[i]);
          rbv[i] += from16<E>(v[rowv + sr * hv + vv]) * acc[i];
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = row_sum16(rbv[i]);
      if (ln == 0) s.dbr[t16 + 4 * lq + i] += x;
    }
  }
  __syncthreads();

  // ---- 15: per token: dg = reverse chunk-local cumsum of dGc, dbeta, dlambda ---------
  if (w == 0) {
    const int t = lane;
    float x = s.dgr[t] + s.dgcol[0][t] + s.dgcol[1][t] + s.dgcol[2][t] + s.dgcol[3][t];
    if (t == kGC - 1) {
      float lc = 0.f, de = 0.f;
      for (int u = 0; u < kGC; ++u) lc += s.lastc[u];
#pragma unroll
      for (int p = 0; p < NPV; ++p) de += del_p[(size_t)p * B * H * NT + (size_t)row * NT + ic];
      x += lc + s.e[kGC - 1] * de;
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float y = __shfl_down(x, d, 64);
      if (t + d < 64) x += y;
    }
    dg[(tok0 + t) * H + h] = x;
    db[(tok0 + t) * H + h] = from_f32<TB>(s.dbr[t]);
  }
  // four elements per thread and round: the partial loads of every slice and
  // element of a round issue together (inter-chunk columns; clamped to column
  // 7 elsewhere and to the last element past the end, and not used there;
  // with no inter-chunk level (T = 64) the partial buffer is empty and nothing
  // is loaded)
  for (int u0 = 0; u0 < kGC * L; u0 += 4 * 256) {
    float pl[4][NPV];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int u = min(u0 + tid + 256 * q, kGC * L - 1);
      const int t = u / L, c = u % L;
      const int ce = min(max(c, 7), 6 + nlev) - 7;
#pragma unroll
      for (int p = 0; p < NPV; ++p)
        pl[q][p] = nlev > 0 ? dl_p[((size_t)p * BTH + (tok0 + t) * H + h) * nlev + ce] : 0.f;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int u = u0 + tid + 256 * q;
      if (u < kGC * L) {
        const int t = u / L, c = u % L;
        float x = 0.f;
        if (c < 7) {
          x = s.dlam[c][t];
        } else if (c < 7 + nlev) {
#pragma unroll
          for (int p = 0; p < NPV; ++p) x += pl[q][p];
        }
        dl[((tok0 + t) * H + h) * L + c] = x;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host launcher
// ---------------------------------------------------------------------------
struct GdnBwdWs {
  __bf16 *qn, *kn, *knT, *wn, *un, *hs;
  __bf16 *dq_p, *dw_p, *dk_p;   // per-V-slice partials, bf16 (summed in fp32 by the chunk kernel)
  float *du, *dl_p, *del_p;
  size_t bytes;
};

inline size_t balign(size_t x) { return (x + 255) & ~(size_t)255; }

// recompute = false: no recompute regions (the caller brings q_new, K_new,
// W_new, U and the level states from a forward that kept them).
inline GdnBwdWs gdn_bwd_ws_layout(void* base, int B, int T, int H, int K, int V, int nlev,
                                  bool recompute = true) {
  GdnBwdWs w;
  char* p = (char*)base;
  size_t off = 0;
  const size_t n = (size_t)B * T * H;
  const size_t NT = (size_t)T / kGC, nvs = (size_t)V / kBVs;
  const size_t nl = nlev > 0 ? (size_t)nlev : 1;
  w.qn = w.kn = w.knT = w.wn = w.un = w.hs = nullptr;
  if (recompute) {
    w.qn = (__bf16*)(p + off); off += balign(n * K * 2);
    w.kn = (__bf16*)(p + off); off += balign(n * K * 2);
    w.knT = (__bf16*)(p + off); off += balign(n * K * 2);
    w.wn = (__bf16*)(p + off); off += balign(n * K * 2);
    w.un = (__bf16*)(p + off); off += balign(n * V * 2);
    w.hs = (__bf16*)(p + off); off += balign((size_t)B * H * NT * nl * V * K * 2);
  }
  w.dq_p = (__bf16*)(p + off); off += balign(nvs * n * K * 2);
  w.dw_p = (__bf16*)(p + off); off += balign(nvs * n * K * 2);
  w.dk_p = (__bf16*)(p + off); off += balign(nvs * n * K * 2);
  w.du = (float*)(p + off); off += balign(n * V * 4);
  w.dl_p = (float*)(p + off); off += balign(nvs * n * nl * 4);
  w.del_p = (float*)(p + off); off += balign(nvs * B * H * NT * 4);
  w.bytes = off;
  return w;
}

template <int KD, int VD, typename TB, typename TL, bool STRONG, typename E = __bf16>
static hipError_t gdn_bwd_t(const void* q, const void* k, const void* v, const void* beta,
                            const float* gcum, const void* l, const void* dO, void* dq, void* dk,
                            void* dv, void* db, float* dg, float* dl, const GdnBwdWs& w, int B,
                            int T, int H, int L, int nlev, int norm_qk, float scale,
                            hipStream_t stream) {
  const int NT = T / kGC;
  hipError_t e;
  {
    auto ks = gdn_bwd_scan_kernel<KD, TL, E>;
    const int smem = (int)sizeof(GdnBscanSmem<KD>);
    if ((e = hipFuncSetAttribute((const void*)ks, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 smem)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(ks, dim3(B * H * (VD / kBVs)), dim3(64 * gdn_bscan_waves<KD>()), smem,
                       stream, w.qn, w.wn, w.kn,
                       w.un, (const __bf16*)dO, gcum, (const TL*)l, w.hs, w.dq_p, w.dw_p, w.dk_p,
                       w.du, w.dl_p, w.del_p, B, T, H, VD, L, nlev, STRONG ? 1 : 0);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    auto kc = gdn_bwd_chunk_kernel<KD, VD, TB, TL, STRONG, E>;
    const int smem = (int)sizeof(GdnBchunkSmem<KD, VD>);
    if ((e = hipFuncSetAttribute((const void*)kc, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 smem)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(kc, dim3(B * H * NT), dim3(256), smem, stream, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, (const TB*)beta, gcum, (const TL*)l,
                       (const __bf16*)dO, w.dq_p, w.dw_p, w.dk_p, w.du, w.dl_p, w.del_p,
                       (__bf16*)dq, (__bf16*)dk, (__bf16*)dv, (TB*)db, dg, dl, B, T,
                       H, L, nlev, norm_qk, scale);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace hattn

int hattn_gdn_bwd_max_levels() { return hattn::kGBwdMaxLev; }

size_t hattn_gdn_bwd_ws_bytes(int B, int T, int H, int K, int V, int nlev) {
  return hattn::gdn_bwd_ws_layout(nullptr, B, T, H, K, V, nlev).bytes;
}

namespace {
// The level scan and the chunk kernel on the recompute results in w.
hipError_t gdn_bwd_dispatch(const void* q, const void* k, const void* v, const void* beta,
                            const float* gcum, const void* l, const void* dO, void* dq, void* dk,
                            void* dv, void* db, float* dg, float* dl, const hattn::GdnBwdWs& w,
                            int B, int T, int H, int K, int V, int L, int nlev, int dt_b, int dt_l,
                            int norm_qk, float scale, int strong, int h16, hipStream_t stream,
                            int* unsupported) {
  using namespace hattn;
#define HATTN_GDN_BT(KD_, VD_, TB_, TL_)                                                        \
  return strong ? gdn_bwd_t<KD_, VD_, TB_, TL_, true>(q, k, v, beta, gcum, l, dO, dq, dk, dv, db,  \
                                                      dg, dl, w, B, T, H, L, nlev, norm_qk, scale, \
                                                      stream)                                      \
                : gdn_bwd_t<KD_, VD_, TB_, TL_, false>(q, k, v, beta, gcum, l, dO, dq, dk, dv, db, \
                                                       dg, dl, w, B, T, H, L, nlev, norm_qk,       \
                                                       scale, stream);
// fp16 q/k/v: the weak hierarchy with fp32 beta / lambda only.
#define HATTN_GDN_B(KD_, VD_)                                                                   \
  if (K == KD_ && V == VD_) {                                                                   \
    if (h16) {                                                                                  \
      if (!strong && dt_b == 2 && dt_l == 2)                                                    \
        return gdn_bwd_t<KD_, VD_, float, float, false, _Float16>(                              \
            q, k, v, beta, gcum, l, dO, dq, dk, dv, db, dg, dl, w, B, T, H, L, nlev, norm_qk,   \
            scale, stream);                                                                     \
      *unsupported = 1;                                                                         \
      return hipSuccess;                                                                        \
    }                                                                                           \
    if (dt_b == 0 && dt_l == 0) HATTN_GDN_BT(KD_, VD_, __bf16, __bf16)                          \
    if (dt_b == 2 && dt_l == 2) HATTN_GDN_BT(KD_, VD_, float, float)                            \
    if (dt_b == 0 && dt_l == 2) HATTN_GDN_BT(KD_, VD_, __bf16, float)                           \
    if (dt_b == 2 && dt_l == 0) HATTN_GDN_BT(KD_, VD_, float, __bf16)                           \
  }
  HATTN_GDN_B(256, 128)
  HATTN_GDN_B(256, 64)
  HATTN_GDN_B(192, 128)
  HATTN_GDN_B(192, 64)
  HATTN_GDN_B(128, 128)
  HATTN_GDN_B(128, 64)
  HATTN_GDN_B(64, 128)
  HATTN_GDN_B(64, 64)
#undef HATTN_GDN_B
#undef HATTN_GDN_BT
  *unsupported = 1;
  return hipSuccess;
}
}  // namespace

hipError_t hattn_gdn_bwd_launch(const void* q, const void* k, const void* v, const void* beta,
                                const float* gcum, const void* l, const void* dO, void* dq,
                                void* dk, void* dv, void* db, float* dg, float* dl, void* ws,
                                int B, int T, int H, int K, int V, int L, int nlev, int dt_b,
                                int dt_l, int norm_qk, float scale, int strong, int h16,
                                hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  const GdnBwdWs w = gdn_bwd_ws_layout(ws, B, T, H, K, V, nlev);
  hipError_t e = hattn_gdn_recompute_launch(q, k, v, beta, gcum, l, w.qn, w.kn, w.knT, w.wn, w.un, w.hs,
                                            B, T, H, K, V, L, nlev, dt_b, dt_l, norm_qk, scale,
                                            h16, stream, unsupported);
  if (e != hipSuccess || *unsupported) return e;
  return gdn_bwd_dispatch(q, k, v, beta, gcum, l, dO, dq, dk, dv, db, dg, dl, w, B, T, H, K, V,
                          L, nlev, dt_b, dt_l, norm_qk, scale, strong, h16, stream, unsupported);
}

size_t hattn_gdn_bwd_kept_ws_bytes(int B, int T, int H, int K, int V, int nlev) {
  return hattn::gdn_bwd_ws_layout(nullptr, B, T, H, K, V, nlev, false).bytes;
}

// The backward with q_new, W_new, K_new, U and the level states from a forward
// that kept them (hattn_gdn_fwd_keep_launch): no recompute.
hipError_t hattn_gdn_bwd_kept_launch(const void* q, const void* k, const void* v,
                                     const void* beta, const float* gcum, const void* l,
                                     const void* dO, void* dq, void* dk, void* dv, void* db,
                                     float* dg, float* dl, const __bf16* qn, const __bf16* wn,
                                     const __bf16* kn, const __bf16* un, const __bf16* hs,
                                     void* ws, int B, int T, int H, int K, int V, int L, int nlev,
                                     int dt_b, int dt_l, int norm_qk, float scale, int strong,
                                     int h16, hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  GdnBwdWs w = gdn_bwd_ws_layout(ws, B, T, H, K, V, nlev, false);
  w.qn = const_cast<__bf16*>(qn);
  w.wn = const_cast<__bf16*>(wn);
  w.kn = const_cast<__bf16*>(kn);
  w.un = const_cast<__bf16*>(un);
  w.hs = const_cast<__bf16*>(hs);
  return gdn_bwd_dispatch(q, k, v, beta, gcum, l, dO, dq, dk, dv, db, dg, dl, w, B, T, H, K, V,
                          L, nlev, dt_b, dt_l, norm_qk, scale, strong, h16, stream, unsupported);
}
