// Log-linear Mamba-2 chunkwise forward for the strong hierarchy (HType.STRONG)
// on gfx950.
//
// Replaces chunkwise.chunkwise_fwd with htype == STRONG (chunkwise.py:1118-1275):
// the reference runs the intra-chunk kernel with USE_A2 (the sub-diagonal
// tiles, chunkwise.py:587-641) and, per inter-chunk level from 1, the state
// kernel with four phase states per level (USE_H2, chunkwise.py:199-276) and
// the output kernel.
//
// The strong level function (base.py:49-62) at a chunk of 64 tokens: every
// diagonal 64 x 64 block holds one level table (kStrong.intra), every
// sub-diagonal block (source chunk = target chunk - 1) one other table
// (kStrong.sub), and a pair of chunks further apart has the single level
// 6 + strong(c_t, c_s) (the strong function of the chunk indices).  So
//   o_t = sum_{s in chunk c}     lam[t, intra(a, b)] e^{G_t - G_s} (q_t.k_s) v_s
//       + sum_{s in chunk c - 1} lam[t, sub(a, b)]   e^{G_t - G_s} (q_t.k_s) v_s
//       + sum_{j >= 2} lam[t, 6 + j] e^{Gc_t} q_t . S_j(c),
// where S_j(c) is level j of a chunk-level strong state: the cascade of
// HState.cascade_strong (recurrent.py:56-74) with one insertion per chunk
// (value sum_s e^{Gc_last - Gc_s} k_s v_s^T, gate e^{Gc_last}), read after
// the cascade and before the chunk's own decay and insertion.
//
// One workgroup (eight waves) per (batch, head, 32 columns of V; 16 for the
// serial walks below) walks the chunks in order; the walk is a chain of
// dependent steps, so the chunk's work is split over two sets of waves that
// run side by side.  Near wave w (0-3) owns the state rows k = 16 w .. +15 of
// every chunk-level level (one 16 x 16 fp32 tile per 16 columns and level in
// registers); wave w and far wave w + 4 both
// own the output rows t = 16 w .. +15.  Per chunk: the cascade (near, uniform
// selects over the levels), the levels >= 2 staged in LDS as bf16, then with
// transposed products (lane: one token t, four consecutive v)
//   near: o^T  = V^T (P o W)^T over the chunk and its predecessor (P = Q K^T,
//               W the decay and lambda weights, from the two level tables in
//               LDS), handed to the far wave through LDS
//   far:  o^T += sum_j S_j^T (lam_j e^{Gc} Q)^T, and the store of o
// and, after the hand-over, S_0 = K^T diag(e^{Gc_last - Gc}) V after the decay
// (near).
//
// Segment-parallel walks.  The chunks are cut into segments of S = 2^s chunks
// (s = kSLog).  Right after the cascade at the first chunk c0 = S p of a
// segment p >= 1 the state holds, at level s + 1 - m (m = 0 .. s), the previous
// segment's chunks [S - S / 2^m, S - S / 2^(m+1)) (for S = 16: chunks 0-7 at
// level 5, 8-11 at 4, 12-13 at 3, 14 at 2, 15 at 1), and at a level j >= s + 2
// the whole segments q <= p - 2 with s + strong(p, q) = j (the strong function
// of the segment indices: strong(S p + i, S q + x) = s + strong(p, q) for every
// i, x), each level the sum of its chunks' insertions decayed to c0, with its
// chunk count; within the segment the cascade never carries into a level
// >= s + 2.  So the walk of segment p starts there: a first kernel writes, per
// segment, those s + 1 block sums and the whole segment's
// (fp32 [K][V], decayed to the segment end) and the segment's total log-decay;
// the walk of segment p loads the previous segment's s + 1 blocks, adds the
// earlier segments at their levels, decayed over the segments between, and
// walks its S chunks.  Without a workspace for the block sums one walk per
// row covers every chunk.
#include "mamba2_strong.h"

namespace hattn {

// NV 16-column tiles of V per workgroup: 2 for the segment-parallel walks,
// 1 for the serial walks (twice the workgroups where every row is one chain).
constexpr int kSLK = 64 + 8;      // row stride of the bf16 q / k tiles
// Row strides of the per-token LDS rows that each lane of a 16-lane group reads
// for a different token: 33 words (lambda) and 17 words (level tables) put
// the 16 rows on 16 different banks.
constexpr int kSLam = 33;
constexpr int kSTab = 17;

__device__ constexpr StrongTables kStrong{};

template <int NV>
struct StrongSmem {
  static constexpr int kSLV = 16 * NV + 8;   // row stride of the bf16 v tiles
  __bf16 q[kSC * kSLK];
  __bf16 k[2][kSC * kSLK];           // this chunk and the previous one (by parity)
  __bf16 v[2][kSC * kSLV];
  __bf16 hs[kSMaxLev][16 * NV * kSLK];  // chunk-level states, bf16 [v][k]
  float gc[2][kSC];                  // chunk-local inclusive cumsum of g
  float lam[kSC][kSLam];             // lambda[t, 0 .. L-1] of this chunk (L <= 32)
  unsigned tab[2][kSC * kSTab];      // intra / sub level tables, four levels a word
  floatx4 onear[kSC][4 * NV];      // o^T of the near blocks, [t][v / 4]
};

constexpr int kSThreads = 512;
constexpr int kSLog = 5;              // segments of 2^kSLog chunks
constexpr int kSSeg = 1 << kSLog;     // chunks per segment of the segment-parallel walks
constexpr int kSBlk = kSLog + 2;      // block sums per segment: kSLog + 1 blocks, the whole

// ---------------------------------------------------------------------------
// Block sums of a segment (the starting state of the next segments' walks)
// ---------------------------------------------------------------------------
// One workgroup (four waves) per (row, segment p <= NSEG - 2, 64 columns of V):
// per chunk X = K^T diag(e^{Gc_last - Gc}) V on MFMA (wave w: rows k = 16 w ..
// +15), and kSBlk running sums, every one decayed by the chunk's total decay
// before the chunk's X joins its block and the whole segment.
//   blk [row][p][kSBlk][K = 64][V] fp32,  segd [row][NSEG] (p <= NSEG - 2 written)
struct SegBlkSmem {
  __bf16 k[kSC * kSLK];   // [t][k]
  __bf16 v[kSC * kSLK];   // [t][v], 64 columns
  float gc[kSC];          // chunk-local inclusive cumsum of g
};

__global__ __launch_bounds__(256) void mamba2_strong_segblk_kernel(
    const __bf16* __restrict__ k, const __bf16* __restrict__ v, const float* __restrict__ g,
    float* __restrict__ blk, float* __restrict__ segd, int nrows, int T, int G, int H, int V,
    int NSEG) {
  __shared__ __attribute__((aligned(16))) SegBlkSmem s;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const int nvb = V / 64;
  const XcdMap mp = xcd_map(blockIdx.x, (NSEG - 1) * nvb);
  if (mp.row >= nrows) return;
  const int row = mp.row, p = mp.slice / nvb, v0 = (mp.slice % nvb) * 64;
  const int b = row / H, h = row % H, gq = h / (H / G);
  const size_t hk = (size_t)G * 64, hv = (size_t)H * V;
  // two 16-byte units of k and of v per thread: rows r_ld and r_ld + 32
  const int r_ld = tid >> 3, c_ld = 8 * (tid & 7);
  u32x4 pk[2], pv[2];
  float pg;
  auto prefetch = [&](int jc) __attribute__((always_inline)) {
    const size_t t0 = (size_t)b * T + (size_t)jc * kSC;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const size_t tr = t0 + r_ld + 32 * u;
      pk[u] = *(const u32x4*)(k + tr * hk + (size_t)gq * 64 + c_ld);
      pv[u] = *(const u32x4*)(v + tr * hv + (size_t)h * V + v0 + c_ld);
    }
    pg = g[(t0 + lane) * H + h];
  };
  floatx4 acc[kSBlk][4];
#pragma unroll
  for (int m = 0; m < kSBlk; ++m)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[m][nt] = zero4();
  float dseg = 0.f;
  const int c0 = p * kSSeg;
  prefetch(c0);
  for (int i = 0; i < kSSeg; ++i) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      *(u32x4*)(s.k + (r_ld + 32 * u) * kSLK + c_ld) = pk[u];
      *(u32x4*)(s.v + (r_ld + 32 * u) * kSLK + c_ld) = pv[u];
    }
    if (w == 0) {
      float x = pg;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
      }
      s.gc[lane] = x;
    }
    __syncthreads();
    if (i + 1 < kSSeg) prefetch(c0 + i + 1);
    const float glast = s.gc[kSC - 1];
    const float gd = fexp(glast);
    dseg += glast;
    // x[nt][e] = X[k = 16 w + 4 lq + e][v = 16 nt + ln]
    floatx4 x[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) x[nt] = zero4();
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      bf16x8 a = tr_frag(s.k, kSLK, 32 * c, 16 * w);   // K[s][k = 16 w + ln]
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
        a[jj] = (__bf16)((float)a[jj] * fexp(glast - s.gc[32 * c + 8 * lq + jj]));
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        x[nt] = mfma16x16x32(a, tr_frag(s.v, kSLK, 32 * c, 16 * nt), x[nt]);
    }
    // block m = 0 .. kSLog: chunks [S - S / 2^m, S - S / 2^(m+1)) (the last: chunk S - 1)
    int bi = 0;
#pragma unroll
    for (int m = 1; m <= kSLog; ++m)
      if (i >= kSSeg - (kSSeg >> m)) bi = m;
#pragma unroll
    for (int m = 0; m < kSBlk; ++m) {
      const float on = (m == bi || m == kSBlk - 1) ? 1.f : 0.f;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[m][nt][e] = acc[m][nt][e] * gd + on * x[nt][e];
    }
    __syncthreads();   // the next chunk's staging overwrites k, v, gc
  }
  float* out = blk + (size_t)(row * (NSEG - 1) + p) * kSBlk * 64 * V + v0 + ln;
#pragma unroll
  for (int m = 0; m < kSBlk; ++m)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        out[((size_t)m * 64 + 16 * w + 4 * lq + e) * V + 16 * nt] = acc[m][nt][e];
  if (v0 == 0 && tid == 0) segd[row * NSEG + p] = dseg;
}

template <typename TL, typename TO, int NV>
__global__ __launch_bounds__(kSThreads) void mamba2_strong_fwd_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const float* __restrict__ g, const TL* __restrict__ l, TO* __restrict__ o,
    float* __restrict__ gcum, const float* __restrict__ blk, const float* __restrict__ segd,
    int nrows, int T, int G, int H, int V, int L, int NSEG) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  StrongSmem<NV>& s = *(StrongSmem<NV>*)smem_raw;
  constexpr int kSBV = 16 * NV, kSNV = NV, kSVU = 2 * NV, kSLV = StrongSmem<NV>::kSLV;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  // waves 0-3 (near): the cascade and the chunk-level states (rows k = 16 w ..),
  // the diagonal and sub-diagonal blocks, the insertion; waves 4-7 (far): the
  // levels >= 2 and the output stores.  Wave w & 3 owns the tokens 16 (w & 3) ..
  const bool near = w < 4;
  const int wq = w & 3;
  const int nvb = V / kSBV;
  // NSEG > 1: segment seg's chunks c0 .. cend - 1 from the state at c0 (the
  // block sums blk, segd); NSEG == 1: every chunk from the empty state
  const XcdMap mp = xcd_map(blockIdx.x, nvb * NSEG);
  if (mp.row >= nrows) return;
  const int row = mp.row, seg = mp.slice / nvb, v0 = (mp.slice % nvb) * kSBV;
  const int b = row / H, h = row % H, gq = h / (H / G);
  const int NT = T / kSC;
  const int c0 = seg * kSSeg;
  const int cend = NSEG > 1 ? min(c0 + kSSeg, NT) : NT;
  const size_t hk = (size_t)G * 64, hv = (size_t)H * V;
  const int t_me = 16 * wq + ln;   // this lane's token in the transposed products

  for (int i = tid; i < kSC * kSC / 4; i += kSThreads) {
    s.tab[0][(i >> 4) * kSTab + (i & 15)] = ((const unsigned*)kStrong.intra)[i];
    s.tab[1][(i >> 4) * kSTab + (i & 15)] = ((const unsigned*)kStrong.sub)[i];
  }

  // Level-j state (near waves): one 16 x 16 fp32 tile, rows k = 16 w + 4 lq + i,
  // column v = ln (the MFMA D layout), and the number of chunks it holds.
  floatx4 st[kSMaxLev][kSNV];
#pragma unroll
  for (int j = 0; j < kSMaxLev; ++j)
#pragma unroll
    for (int nt = 0; nt < kSNV; ++nt) st[j][nt] = zero4();
  int cnt[kSMaxLev];
#pragma unroll
  for (int j = 0; j < kSMaxLev; ++j) cnt[j] = 0;

  // Inputs of one chunk in registers, loaded one chunk ahead so their latency
  // hides behind the previous chunk's products: one 16-byte unit of q and of
  // k per thread, a v unit (threads < 128), g (wave 0) and up to four lambda
  // entries per thread (64 x L <= 2048).
  const int r_ld = tid >> 3, c_ld = 8 * (tid & 7);
  const int rv_ld = tid / kSVU, cv_ld = 8 * (tid % kSVU);
  const bool v_ld = tid < kSC * kSVU;
  int lrel[4], llds[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = min(tid + kSThreads * u, kSC * L - 1);
    lrel[u] = (i / L) * H * L + i % L;
    llds[u] = (i / L) * kSLam + i % L;
  }
  u32x4 pq, pk, pv;
  float pg;
  TL pl[4];
  auto prefetch = [&](int jc) __attribute__((always_inline)) {
    const size_t t0 = (size_t)b * T + (size_t)jc * kSC;
    const size_t rq = (t0 + r_ld) * hk + (size_t)gq * 64 + c_ld;
    pq = *(const u32x4*)(q + rq);
    pk = *(const u32x4*)(k + rq);
    pv = *(const u32x4*)(v + (t0 + (v_ld ? rv_ld : 0)) * hv + (size_t)h * V + v0 + cv_ld);
    pg = g[(t0 + lane) * H + h];
    const TL* lb = l + (t0 * H + h) * L;
#pragma unroll
    for (int u = 0; u < 4; ++u) pl[u] = lb[lrel[u]];
  };

  if (c0 > 0) {
    if (near) {
      // the previous segment's blocks m = 0 .. kSLog -> levels kSLog + 1 - m
      // (S / 2, S / 4, .., 1, 1 chunks)
      const int kr = 16 * w + 4 * lq;
      const float* pb = blk + (size_t)(row * (NSEG - 1) + seg - 1) * kSBlk * 64 * V + v0 + ln;
#pragma unroll
      for (int m = 0; m <= kSLog; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int nt = 0; nt < kSNV; ++nt)
            st[kSLog + 1 - m][nt][i] = pb[((size_t)m * 64 + kr + i) * V + 16 * nt];
        cnt[kSLog + 1 - m] = m < kSLog ? kSSeg >> (m + 1) : 1;
      }
      // the whole segments q <= seg - 2 at level kSLog + strong(seg, q), decayed
      // over the segments q + 1 .. seg - 1
      float dec = 0.f;
      for (int q = seg - 2; q >= 0; --q) {
        dec += segd[row * NSEG + q + 1];
        const float f = fexp(dec);
        const int lev = kSLog + strong_level_ce(seg, q);
        const float* ps = blk + ((size_t)(row * (NSEG - 1) + q) * kSBlk + kSBlk - 1) * 64 * V + v0 + ln;
        float y[kSNV][4];
#pragma unroll
        for (int nt = 0; nt < kSNV; ++nt)
#pragma unroll
          for (int i = 0; i < 4; ++i) y[nt][i] = f * ps[(size_t)(kr + i) * V + 16 * nt];
#pragma unroll
        for (int j = kSLog + 2; j < kSMaxLev; ++j)
          if (lev == j) {
#pragma unroll
            for (int nt = 0; nt < kSNV; ++nt)
#pragma unroll
              for (int i = 0; i < 4; ++i) st[j][nt][i] += y[nt][i];
            cnt[j] += kSSeg;
          }
      }
    }
    // chunk c0 - 1 (k, v, g cumsum) for the first sub-diagonal block; the
    // loop's first barrier orders these writes before their reads
    prefetch(c0 - 1);
    const int pp = (c0 - 1) & 1;
    *(u32x4*)(s.k[pp] + r_ld * kSLK + c_ld) = pk;
    if (v_ld) *(u32x4*)(s.v[pp] + rv_ld * kSLV + cv_ld) = pv;
    if (w == 0) {
      float x = pg;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
      }
      s.gc[pp][lane] = x;
    }
  }
  prefetch(c0);

  for (int ic = c0; ic < cend; ++ic) {
    const int par = ic & 1;
    const size_t tok0 = (size_t)b * T + (size_t)ic * kSC;
    // ---- cascade (recurrent.py:56-74) over the chunk-level states ------------------
    // (a segment's walk starts from the state after the cascade at c0)
    if (near && (ic > c0 || c0 == 0)) {
      floatx4 carry[kSNV];
#pragma unroll
      for (int nt = 0; nt < kSNV; ++nt) carry[nt] = zero4();
      int cc = 0;
#pragma unroll
      for (int j = 0; j < kSMaxLev; ++j) {
        const int cap = 1 << (j > 0 ? j - 1 : 0);
        const bool swap = j == 0 || cnt[j] + cc > cap;
        const int oc = cnt[j];
#pragma unroll
        for (int nt = 0; nt < kSNV; ++nt) {
          const floatx4 old = st[j][nt];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            st[j][nt][i] = swap ? carry[nt][i] : old[i] + carry[nt][i];
            carry[nt][i] = swap ? old[i] : 0.f;
          }
        }
        cnt[j] = swap ? cc : oc + cc;
        cc = swap ? oc : 0;
      }
    }
    // ---- stage: q, k, v tiles, g cumsum, lambda, levels >= 2 -------------------------
    {
      *(u32x4*)(s.q + r_ld * kSLK + c_ld) = pq;
      *(u32x4*)(s.k[par] + r_ld * kSLK + c_ld) = pk;
      if (v_ld) *(u32x4*)(s.v[par] + rv_ld * kSLV + cv_ld) = pv;
      if (w == 0) {
        float x = pg;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const float y = __shfl_up(x, d, 64);
          if (lane >= d) x += y;
        }
        s.gc[par][lane] = x;
        if (v0 == 0) gcum[(tok0 + lane) * H + h] = x;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (tid + kSThreads * u < kSC * L) (&s.lam[0][0])[llds[u]] = to_f32<TL>(pl[u]);
      if (near) {
#pragma unroll
        for (int j = 2; j < kSMaxLev; ++j)
#pragma unroll
          for (int nt = 0; nt < kSNV; ++nt)
            *(bf16x4*)(s.hs[j] + (16 * nt + ln) * kSLK + 16 * w + 4 * lq) = cvt4(st[j][nt]);
      }
    }
    __syncthreads();
    if (ic + 1 < cend) prefetch(ic + 1);

    floatx4 acc[kSNV];   // o^T[v = 16 nt + 4 lq + i][t = t_me]
#pragma unroll
    for (int nt = 0; nt < kSNV; ++nt) acc[nt] = zero4();
    const float gct = s.gc[par][t_me];
    // B operand of the q . k products: Q[t_me][32 c + 8 lq ..]
    const bf16x8 bq0 = *(const bf16x8*)(s.q + t_me * kSLK + 8 * lq);
    const bf16x8 bq1 = *(const bf16x8*)(s.q + t_me * kSLK + 32 + 8 * lq);
    if (near) {
      // ---- diagonal (cur = 1) and sub-diagonal (cur = 0) blocks -------------------------
#pragma unroll
      for (int cur = 1; cur >= 0; --cur) {
        if (!cur && ic == 0) break;
        const int pk2 = cur ? par : par ^ 1;
        const unsigned* tab = s.tab[cur ? 0 : 1] + t_me * kSTab;
        const float* lrow = s.lam[t_me];
        // the source tiles of the block: the diagonal stops at this wave's tile
        const int npair = cur ? (w >> 1) + 1 : 2;
        const float base = cur ? 0.f : s.gc[pk2][kSC - 1];
        for (int pp = 0; pp < npair; ++pp) {
          bf16x8 pb;
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int n = 2 * pp + half;   // source tile
            floatx4 sc = zero4();
            sc = mfma16x16x32(*(const bf16x8*)(s.k[pk2] + (16 * n + ln) * kSLK + 8 * lq), bq0, sc);
            sc = mfma16x16x32(*(const bf16x8*)(s.k[pk2] + (16 * n + ln) * kSLK + 32 + 8 * lq), bq1, sc);
            // sc[i] = q_t . k_s, s = 16 n + 4 lq + i, t = t_me
            const unsigned lv4 = tab[4 * n + lq];   // levels of the lane's four sources
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int sp = 16 * n + 4 * lq + i;
              float x = 0.f;
              if (!cur || sp <= t_me) {
                const int lev = (lv4 >> (8 * i)) & 0xff;
                x = sc[i] * fexp(gct + base - s.gc[pk2][sp]) * lrow[lev];
              }
              pb[4 * half + i] = (__bf16)x;
            }
          }
          // o^T[v][t] += V[s][v] P^T[s][t] over the 32 sources of the pair
#pragma unroll
          for (int nt = 0; nt < kSNV; ++nt)
            acc[nt] = mfma16x16x32(tr_frag_d(s.v[pk2], kSLV, 32 * pp, 16 * nt), pb, acc[nt]);
        }
      }
#pragma unroll
      for (int nt = 0; nt < kSNV; ++nt) s.onear[t_me][4 * nt + lq] = acc[nt];
    } else {
      // ---- far levels: o^T[v][t] += S_j^T[v][k] (lam[t, 6 + j] e^{Gc_t} q_t[k]) ----------
      // a lane's four values share its token t_me: the level weight is one
      // scalar per lane, applied to the product (q stays the exact bf16 input)
      const float eg = fexp(gct);
#pragma unroll
      for (int j = 2; j < kSMaxLev; ++j) {
        if (6 + j < L) {
          const float f = s.lam[t_me][6 + j] * eg;
#pragma unroll
          for (int nt = 0; nt < kSNV; ++nt) {
            const __bf16* hr = s.hs[j] + (16 * nt + ln) * kSLK + 8 * lq;
            floatx4 y = mfma16x16x32(*(const bf16x8*)hr, bq0, zero4());
            y = mfma16x16x32(*(const bf16x8*)(hr + 32), bq1, y);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[nt][i] += f * y[i];
          }
        }
      }
    }
    __syncthreads();   // the near blocks' o^T in LDS

    if (near) {
      // ---- decay the levels, insert S_0 = K^T diag(e^{Gc_last - Gc}) V ----------------
      const float glast = s.gc[par][kSC - 1];
      const float gd = fexp(glast);
#pragma unroll
      for (int j = 1; j < kSMaxLev; ++j)
#pragma unroll
        for (int nt = 0; nt < kSNV; ++nt)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[j][nt][i] *= gd;
      floatx4 sum[kSNV];
#pragma unroll
      for (int nt = 0; nt < kSNV; ++nt) sum[nt] = zero4();
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        bf16x8 a = tr_frag(s.k[par], kSLK, 32 * c, 16 * w);   // K[s][k = 16 w + ln]
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          a[jj] = (__bf16)((float)a[jj] * fexp(glast - s.gc[par][32 * c + 8 * lq + jj]));
#pragma unroll
        for (int nt = 0; nt < kSNV; ++nt)
          sum[nt] = mfma16x16x32(a, tr_frag(s.v[par], kSLV, 32 * c, 16 * nt), sum[nt]);
      }
#pragma unroll
      for (int nt = 0; nt < kSNV; ++nt) st[0][nt] = sum[nt];
      cnt[0] += 1;
    } else {
      // ---- o[t_me][v0 + 16 nt + 4 lq .. +3] = far + near ----------------------------
#pragma unroll
      for (int nt = 0; nt < kSNV; ++nt) {
        const floatx4 an = s.onear[t_me][4 * nt + lq];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[nt][i] += an[i];
        TO* op = o + (tok0 + t_me) * hv + (size_t)h * V + v0 + 16 * nt + 4 * lq;
        if constexpr (sizeof(TO) == 2) {
          *(bf16x4*)op = cvt4(acc[nt]);
        } else {
          *(floatx4*)op = acc[nt];
        }
      }
    }
    // No barrier here: the next chunk's staging writes q, lambda, the level
    // states and the other parity's k / v / g cumsum, which this chunk read
    // before the barrier above; the insertion reads this parity's, and the
    // near waves stage the level states after it (program order).
  }
}

// Workspace of the segment-parallel walks (0: one segment, no workspace).
struct StrongFwdWs {
  float* blk;
  float* segd;
  int nseg;
  size_t bytes;
};
inline StrongFwdWs strong_fwd_ws_layout(void* ws, int B, int T, int H, int V) {
  StrongFwdWs w{nullptr, nullptr, 1, 0};
  const int NT = T / kSC;
  if (NT <= kSSeg) return w;
  w.nseg = (NT + kSSeg - 1) / kSSeg;
  const size_t rows = (size_t)B * H;
  const size_t nb = (rows * (w.nseg - 1) * kSBlk * 64 * V * 4 + 255) / 256 * 256;
  w.bytes = nb + rows * w.nseg * 4;
  unsigned char* p = (unsigned char*)ws;
  if (p != nullptr) {
    w.blk = (float*)p;
    w.segd = (float*)(p + nb);
  }
  return w;
}

template <typename TL, typename TO>
static hipError_t strong_launch_t(const void* q, const void* k, const void* v, const float* g,
                                  const void* l, void* o, float* gcum, void* ws, size_t ws_bytes,
                                  int B, int T, int G, int H, int V, int L, hipStream_t stream) {
  const int rows = B * H;
  StrongFwdWs w = strong_fwd_ws_layout(ws, B, T, H, V);
  if (ws == nullptr || ws_bytes < w.bytes) w = StrongFwdWs{nullptr, nullptr, 1, 0};
  hipError_t e;
  if (w.nseg > 1) {
    const int gridb = (rows + 7) / 8 * 8 * (w.nseg - 1) * (V / 64);
    hipLaunchKernelGGL(mamba2_strong_segblk_kernel, dim3(gridb), dim3(256), 0, stream,
                       (const __bf16*)k, (const __bf16*)v, g, w.blk, w.segd, rows, T, G, H, V,
                       w.nseg);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  auto walk = [&](auto kf, int smem, int bv) {
    hipError_t r = hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       smem);
    if (r != hipSuccess) return r;
    const int grid = (rows + 7) / 8 * 8 * (V / bv) * w.nseg;
    hipLaunchKernelGGL(kf, dim3(grid), dim3(kSThreads), smem, stream, (const __bf16*)q,
                       (const __bf16*)k, (const __bf16*)v, g, (const TL*)l, (TO*)o, gcum,
                       (const float*)w.blk, (const float*)w.segd, rows, T, G, H, V, L, w.nseg);
    return hipGetLastError();
  };
  if (w.nseg > 1)
    return walk(mamba2_strong_fwd_kernel<TL, TO, 2>, (int)sizeof(StrongSmem<2>), 32);
  return walk(mamba2_strong_fwd_kernel<TL, TO, 1>, (int)sizeof(StrongSmem<1>), 16);
}

// ---------------------------------------------------------------------------
// Final states (output_final_state) of the strong hierarchy
// ---------------------------------------------------------------------------
// The reference stores, for each inter-chunk level ell = 1 .. nlev - 1 of the
// strong loop (ell_init = 1, chunkwise.py:1215-1219), the raw phase-0 state b_h
// of chunk_fwd_kernel_h with USE_H2 after its last chunk (chunkwise.py:179-279):
// per chunk i, b_h is reset when i % 2^(ell+1) == 2^(ell+1) - 1 (skip_g, except
// at the last chunk, which decays) or else decayed by exp(Gc_last(i)), then
// gains the chunk's e^{Gc_last - Gc}-weighted k^T v when get_phase_index(i, ell)
// is 0, i.e. i % 2^(ell+1) < 2^(ell-1).  After the last reset (the chunk before
// base = 2^(ell+1) floor((NT - 1) / 2^(ell+1))) those chunks are
// base .. base + 2^(ell-1) - 1, so
//   ht[.., 7 + ell] = exp(G_T - G_end) Sum(base .. end),  end = min(base + 2^(ell-1), NT),
// the range's summary (mamba2_common.h) decayed over the tokens after it.
// Levels 0 .. 7 stay as the caller initialised them (zero, like the reference).
// One workgroup per (row, ell, 64-column block of V).
__global__ __launch_bounds__(256) void mamba2_strong_ht_kernel(
    const __bf16* __restrict__ k, const __bf16* __restrict__ v, const float* __restrict__ g,
    float* __restrict__ ht, int B, int T, int G, int H, int V, int L, int nlev) {
  __shared__ __attribute__((aligned(16))) SumSmem<1> sm;
  __shared__ float red[16];
  const int nvb = V / 64;
  const int vblk = blockIdx.x % nvb, ell = 1 + (blockIdx.x / nvb) % (nlev - 1);
  const int row = blockIdx.x / (nvb * (nlev - 1));
  if (row >= B * H) return;
  const int b = row / H, h = row % H;
  const int NT = T / kBT;
  const int P = 2 << ell, S = 1 << (ell - 1);
  const int base = (NT - 1) / P * P;
  const int tend = min(base + S, NT) * kBT;   // first token after the range
  // log-decay of the tokens after the range: sum of g over t >= tend
  const float* gr = g + (size_t)b * T * H + h;
  float x = 0.f;
  for (int t = tend + (int)threadIdx.x; t < T; t += 256) x += gr[(size_t)t * H];
  x = row_sum16(x);   // every lane of a 16-lane row holds the row's sum
  if ((threadIdx.x & 15) == 0) red[threadIdx.x >> 4] = x;
  __syncthreads();
  float tail = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) tail += red[i];
  float* out = ht + (size_t)row * kKD * V * L + 7 + ell + (size_t)vblk * 64 * L;
  seg_sum_body<__bf16, __bf16, false, 1, false>(sm, k, v, g, out, b, h, base / S, vblk, T, G, H,
                                                 V, NT, S, LayerArgs{}, L, fexp(tail));
}

}  // namespace hattn

int hattn_mamba2_strong_max_levels() { return hattn::kSMaxLev - 1; }

// Workspace bytes for the segment-parallel strong forward (0: the sizes have one
// segment); with less, the forward walks every row serially.
size_t hattn_mamba2_strong_fwd_ws_bytes(int B, int T, int H, int V) {
  return hattn::strong_fwd_ws_layout(nullptr, B, T, H, V).bytes;
}

// bf16 q / k / v; lambda bf16 or fp32; o bf16 or fp32; K = 64; V a multiple of 16;
// L <= 32.
hipError_t hattn_mamba2_strong_fwd_launch(const void* q, const void* k, const void* v,
                                          const float* g, const void* l, void* o, float* gcum,
                                          void* ws, size_t ws_bytes, int B, int T, int G, int H,
                                          int V, int L, int dt_l, int dt_o, hipStream_t stream,
                                          int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
  if (dt_l == 0 && dt_o == 0)
    return strong_launch_t<__bf16, __bf16>(q, k, v, g, l, o, gcum, ws, ws_bytes, B, T, G, H, V, L,
                                         stream);
  if (dt_l == 2 && dt_o == 0)
    return strong_launch_t<float, __bf16>(q, k, v, g, l, o, gcum, ws, ws_bytes, B, T, G, H, V, L,
                                         stream);
  if (dt_l == 0 && dt_o == 2)
    return strong_launch_t<__bf16, float>(q, k, v, g, l, o, gcum, ws, ws_bytes, B, T, G, H, V, L,
                                         stream);
  if (dt_l == 2 && dt_o == 2)
    return strong_launch_t<float, float>(q, k, v, g, l, o, gcum, ws, ws_bytes, B, T, G, H, V, L,
                                         stream);
  *unsupported = 1;
  return hipSuccess;
}

// Final states of the strong hierarchy (levels 8 .. 6 + nlev of ht, the
// others left as the caller initialised them); after the strong forward on the
// same stream.  bf16 k, v; fp32 g (per-step log-decay).
hipError_t hattn_mamba2_strong_ht_launch(const void* k, const void* v, const float* g, float* ht,
                                         int B, int T, int G, int H, int V, int L,
                                         hipStream_t stream) {
  using namespace hattn;
  int nlev = 0;
  while ((1 << nlev) < T / kBT) ++nlev;
  if (nlev < 2) return hipSuccess;   // only level 7 exists, and the reference leaves it zero
  const int grid = B * H * (nlev - 1) * (V / 64);
  hipLaunchKernelGGL(mamba2_strong_ht_kernel, dim3(grid), dim3(256), 0, stream, (const __bf16*)k,
                     (const __bf16*)v, g, ht, B, T, G, H, V, L, nlev);
  return hipGetLastError();
}
