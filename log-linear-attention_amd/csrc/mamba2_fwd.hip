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
#include "mamba2_common.h"

namespace hattn {

// ---------------------------------------------------------------------------
// Kernel 2: main pass over one segment, one 64-wide block of V
// ---------------------------------------------------------------------------
// LDS: one chunk stage (single-buffered; the next chunk waits in registers),
// the A tile, and the top-level states (bf16, [level][k][v]).
struct Stage {
  __bf16 q[kBT * kLd];
  __bf16 k[kBT * kLd];
  __bf16 v[kBT * kLd];
  float gc[kBT];            // chunk-local inclusive cumsum of g
  float wt[kBT];            // exp(Gc_last - Gc_t)
  float lam[kMaxLU * kBT];  // lambda^T [level][t]; levels >= 7 pre-multiplied by exp(Gc_t)
};

struct MainSmem {
  Stage st;
  __bf16 a[kBT * kLd];      // A[t][s] = (S o M)[t][s] of the current chunk, bf16
  __bf16 top[1];            // [ntop][kKD][kLd] top-level states (dynamic size)
};

inline int main_smem_bytes(int ntop) {
  return (int)offsetof(MainSmem, top) + ntop * kKD * kLd * 2;
}

template <typename TV, typename TL>
struct MainRegs {
  uint4 q[2], k[2];
  VTile<TV> v;
  float g;
  TL lam[kMaxLU / 4 + 1];
};

// Phase-1 tile schedule: the 10 causal 16x16 tiles (t-tile mt, s-tile j <= mt)
// and the two zero tiles the 32-wide s steps of A V read above the diagonal
// ((0,1), (2,3)), three per wave: code = mt * 4 + j, +16 marks a zero tile.
__device__ __forceinline__ int p1_tile(int w, int n) {
  constexpr int tab[4][3] = {{0, 10, 14}, {5, 12, 16 + 1}, {4, 8, 15}, {9, 13, 16 + 11}};
  return tab[w][n];
}

template <typename TV, typename TL, typename TO>
__global__ __launch_bounds__(256, 2) void mamba2_fwd_main_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const TV* __restrict__ v,
    const float* __restrict__ g, const TL* __restrict__ l, TO* __restrict__ o,
    float* __restrict__ gcum, float* __restrict__ ht, const float* __restrict__ sums,
    const float* __restrict__ segd, int B, int T, int G, int H, int V, int L, int nlev,
    int nvb64, int slog, int NSEG, int final_state) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  MainSmem& sm = *(MainSmem*)smem_raw;
  Stage& s = sm.st;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const XcdMap xm = xcd_map(blockIdx.x, nvb64);
  if (xm.row >= B * H * NSEG) return;
  // heads fastest: the workgroups reading the same rows of q / k / v run together
  const int h = xm.row % H, p = (xm.row / H) % NSEG, b = xm.row / (H * NSEG);
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

  // ---- top levels: Htop_e(p) from the segment summaries -> LDS (bf16) ----------
  if (ntop > 0) {
    const float* sp = sums + (size_t)row * NSEG * kKD * V + vc;
    const float* dp = segd + (size_t)row * NSEG;
    const size_t qstride = (size_t)kKD * V;
    for (int e2 = 0; e2 < ntop; ++e2) {
      const bool reads = (p >> e2) & 1;
      if (!reads && !is_final_seg) continue;
      // reads: block [lo, lo + 2^e2) decayed to the start of p;
      // final state of a level the last chunk writes: segments [lo, p] decayed to the end
      const int lo = reads ? (p >> (e2 + 1)) << (e2 + 1) : (p >> e2) << e2;
      const int hi = reads ? lo + (1 << e2) : p + 1;
      float dlog = 0.f;
      for (int r = hi; r < p; ++r) dlog += dp[r];
      floatx4 hacc[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) hacc[m] = zero4();
      for (int qs = hi - 1; qs >= lo; --qs) {
        const float sc = fexp(dlog);
        const float* src = sp + qs * qstride;
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i) hacc[m][i] += sc * src[(size_t)(16 * m + 4 * lq + i) * V];
        dlog += dp[qs];
      }
      if (reads) {
        __bf16* tp = sm.top + e2 * kKD * kLd + 16 * w + ln;
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i) tp[(16 * m + 4 * lq + i) * kLd] = (__bf16)hacc[m][i];
      }
      if (is_final_seg) {
        // final state (chunkwise.py:229-279): a level the last chunk reads holds
        // its block decayed over segment p; one it writes holds [lo, p]
        const float sc = reads ? fexp(dp[p]) : 1.f;
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            htb[((size_t)(16 * m + 4 * lq + i) * V + vc) * L + 7 + nloc + e2] = hacc[m][i] * sc;
      }
    }
  }

  // ---- per-row buffer descriptors and per-lane offsets ---------------------------
  // Chunk j of the segment starts (c0 + j) * 64 rows into the row's span; that
  // offset is uniform (SGPR), the lane's part of each access pattern is fixed.
  const int qstr = G * kKD, vstr = H * V, lstr = H * L;
  const rsrc_t rq = make_rsrc(q + ((size_t)b * T * G + gq) * kKD, (size_t)T * qstr * 2);
  const rsrc_t rk = make_rsrc(k + ((size_t)b * T * G + gq) * kKD, (size_t)T * qstr * 2);
  const rsrc_t rv = make_rsrc(v + ((size_t)b * T * H + h) * V + vcol0, (size_t)T * vstr * sizeof(TV));
  const rsrc_t rg_ = make_rsrc(g + (size_t)b * T * H + h, (size_t)T * H * 4);
  const rsrc_t rl = make_rsrc(l + ((size_t)b * T * H + h) * L, (size_t)T * lstr * sizeof(TL));
  const rsrc_t ro = make_rsrc(o + ((size_t)b * T * H + h) * V + vcol0, (size_t)T * vstr * sizeof(TO));
  const bool write_gcum = gcum != nullptr && vblk == 0;
  const rsrc_t rgc = make_rsrc(write_gcum ? (const void*)(gcum + (size_t)b * T * H + h) : (const void*)g,
                               write_gcum ? (size_t)T * H * 4 : 0);
  // 16-byte units of a 64 x 64 tile: u = tid (+256): row u >> 3, col 8 (u & 7)
  const unsigned int vo_qk = ((tid >> 3) * qstr + 8 * (tid & 7)) * 2;
  const unsigned int so_qk2 = 32 * qstr * 2;                     // second unit: +32 rows
  unsigned int vo_v, so_v2;
  if constexpr (sizeof(TV) == 2) {
    vo_v = ((tid >> 3) * vstr + 8 * (tid & 7)) * 2;
    so_v2 = 32 * vstr * 2;
  } else {
    vo_v = ((tid >> 4) * vstr + 4 * (tid & 15)) * 4;                // 4 units, +16 rows each
    so_v2 = 16 * vstr * 4;
  }
  const unsigned int vo_g = lane * H * 4;
  // lambda tile: thread -> row tid >> 2, columns (tid & 3) + 4r
  const int lrow = tid >> 2, lcol = tid & 3;
  const unsigned int vo_l = (lrow * lstr + lcol) * sizeof(TL);
  const unsigned int vo_o = (4 * lq * vstr + 16 * w + ln) * sizeof(TO);
  constexpr int kLR = kMaxLU / 4 + 1;

  MainRegs<TV, TL> rg;
  auto load = [&](int j) {  // j: chunk index within the segment
    const unsigned int row0 = (unsigned int)(c0 + j) * kBT;
    const unsigned int so_qk = row0 * qstr * 2;
    rg.q[0] = buf_load16(rq, vo_qk, so_qk);
    rg.q[1] = buf_load16(rq, vo_qk, so_qk + so_qk2);
    rg.k[0] = buf_load16(rk, vo_qk, so_qk);
    rg.k[1] = buf_load16(rk, vo_qk, so_qk + so_qk2);
    const unsigned int so_v = row0 * vstr * sizeof(TV);
#pragma unroll
    for (int rr = 0; rr < VTile<TV>::N; ++rr) rg.v.r[rr] = buf_load16(rv, vo_v, so_v + rr * so_v2);
    rg.g = buf_load<float>(rg_, vo_g, row0 * H * 4);
    const unsigned int so_l = row0 * lstr * sizeof(TL);
#pragma unroll
    for (int r = 0; r < kLR; ++r)
      if (lcol + 4 * r < lu) rg.lam[r] = buf_load<TL>(rl, vo_l, so_l + 4 * r * sizeof(TL));
  };
  auto store = [&](int j) {
    store_tile_bf16(rg.q, s.q);
    store_tile_bf16(rg.k, s.k);
    store_vtile(rg.v, s.v);
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

  floatx4 st[kMaxLoc][4];
#pragma unroll
  for (int e = 0; e < kMaxLoc; ++e)
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
      bf16x4 out = bf16x4{};
      if (code < 16) {
        floatx4 acc = zero4();
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const bf16x8 a = *(const bf16x8*)(s.k + (16 * jt + ln) * kLd + 32 * c + 8 * lq);
          const bf16x8 bq = *(const bf16x8*)(s.q + t * kLd + 32 * c + 8 * lq);
          acc = mfma16x16x32(a, bq, acc);  // S^T[s = 16jt + 4lq + i][t]
        }
        const float gct = s.gc[t];
        const floatx4 gs = *(const floatx4*)(s.gc + 16 * jt + 4 * lq);
        if (jt < mt) {
          // off-diagonal tile: level 4 + bit_length(mt ^ jt) for every pair
          const float lam = s.lam[(4 + intra_level(mt, jt)) * kBT + t];
#pragma unroll
          for (int i = 0; i < 4; ++i) out[i] = (__bf16)(acc[i] * fexp(gct - gs[i]) * lam);
        } else {
          // diagonal tile: level bit_length(ln ^ (4lq + i)), causal s <= t
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int sl = 4 * lq + i;
            const float val = acc[i] * fexp(gct - gs[i]) * s.lam[intra_level(ln, sl) * kBT + t];
            out[i] = (__bf16)(sl <= ln ? val : 0.f);
          }
        }
      }
      *(bf16x4*)(sm.a + t * kLd + 16 * jt + 4 * lq) = out;
    }
    __syncthreads();

    // ---- phase 2: o[all t][V columns 16w..] ------------------------------------
    floatx4 acc[4];
    {
      const bf16x8 vf0 = tr_frag(s.v, kLd, 0, 16 * w);    // V[s][v], s = 0..31
      const bf16x8 vf1 = tr_frag(s.v, kLd, 32, 16 * w);   // s = 32..63
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const __bf16* ar = sm.a + (16 * mt + ln) * kLd + 8 * lq;
        acc[mt] = mfma16x16x32(*(const bf16x8*)ar, vf0, zero4());
        if (mt >= 2) acc[mt] = mfma16x16x32(*(const bf16x8*)(ar + 32), vf1, acc[mt]);
      }
    }
    const bool any_loc = nloc > 0 && j > 0;
    const bool any_top = ntop > 0 && p > 0;
    if (any_loc || any_top) {
      const float ee = fexp(Eseg);
      // Q fragments in the states' row order: k = 32c + 4lq + i, 32c + 16 + 4lq + i
      bf16x8 qa[4][2];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const __bf16* qp = s.q + (16 * mt + ln) * kLd + 32 * c + 4 * lq;
          const bf16x4 lo = *(const bf16x4*)qp;
          const bf16x4 hi = *(const bf16x4*)(qp + 16);
          qa[mt][c] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      const float* lamt = s.lam + 4 * lq;
      // local levels without branches (a level the chunk does not read gets a
      // zero B operand), so the MFMA chains of all levels interleave
#pragma unroll
      for (int e = 0; e < kMaxLoc; ++e) {
        const bool rd = any_loc && e < nloc && ((ic >> e) & 1);
        const float z = rd ? 1.f : 0.f;
        const bf16x8 b0 = cat8(st[e][0] * z, st[e][1] * z), b1 = cat8(st[e][2] * z, st[e][3] * z);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          floatx4 tmp = mfma16x16x32(qa[mt][0], b0, zero4());
          tmp = mfma16x16x32(qa[mt][1], b1, tmp);
          const floatx4 lam = *(const floatx4*)(lamt + (7 + e) * kBT + 16 * mt);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mt][i] += tmp[i] * lam[i];
        }
      }
      if (any_top) {
        for (int e2 = 0; e2 < ntop; ++e2) {
          if ((p >> e2) & 1) {
            const __bf16* tp = sm.top + e2 * kKD * kLd;
            const bf16x8 b0 = tr_frag_d(tp, kLd, 0, 16 * w), b1 = tr_frag_d(tp, kLd, 32, 16 * w);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
              floatx4 tmp = mfma16x16x32(qa[mt][0], b0, zero4());
              tmp = mfma16x16x32(qa[mt][1], b1, tmp);
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
      const bf16x8 vf0 = tr_frag(s.v, kLd, 0, 16 * w), vf1 = tr_frag(s.v, kLd, 32, 16 * w);
      bf16x8 wv0, wv1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wv0[i] = (__bf16)((float)vf0[i] * w0a[i]);
        wv0[4 + i] = (__bf16)((float)vf0[4 + i] * w0b[i]);
        wv1[i] = (__bf16)((float)vf1[i] * w1a[i]);
        wv1[4 + i] = (__bf16)((float)vf1[4 + i] * w1b[i]);
      }
      floatx4 kv[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        kv[m] = mfma16x16x32(tr_frag(s.k, kLd, 0, 16 * m), wv0, zero4());
        kv[m] = mfma16x16x32(tr_frag(s.k, kLd, 32, 16 * m), wv1, kv[m]);
      }
      const float gl = fexp(glr);
      const bool last = (ic == NT - 1);
#pragma unroll
      for (int e = 0; e < kMaxLoc; ++e) {
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
        for (int e = 0; e < kMaxLoc; ++e)
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

}  // namespace hattn

// dtype codes shared with the C-ABI (include/hattn.h)
enum { DT_BF16 = 0, DT_FP16 = 1, DT_FP32 = 2 };

namespace {
size_t segd_bytes(size_t rows, int NSEG) {
  return (rows * NSEG * sizeof(float) + 255) & ~(size_t)255;
}
}  // namespace

size_t hattn_mamba2_fwd_ws_bytes(int B, int T, int H, int V) {
  const int NT = T / hattn::kBT;
  const int slog = hattn::seg_log2(NT);
  const int NSEG = (NT + (1 << slog) - 1) >> slog;
  if (NSEG <= 1) return 0;
  const size_t rows = (size_t)B * H;
  return segd_bytes(rows, NSEG) + rows * NSEG * hattn::kKD * V * sizeof(float);
}

// Largest inter-chunk level count the register-resident states support.
int hattn_mamba2_fwd_max_levels() { return hattn::kMaxLoc + hattn::kMaxTop; }

namespace hattn {

template <typename TV, typename TL, typename TO>
static hipError_t launch_t(const void* q, const void* k, const void* v, const float* g,
                           const void* l, void* o, float* gcum, float* ht, void* ws, int B,
                           int T, int G, int H, int V, int L, int nlev, hipStream_t stream) {
  const int NT = T / kBT;
  const int slog = seg_log2(NT);
  const int S = 1 << slog;
  const int NSEG = (NT + S - 1) / S;
  const int rows = B * H;
  const int nvb64 = V / 64;
  float* segd = nullptr;
  float* sums = nullptr;
  if (NSEG > 1) {
    segd = (float*)ws;
    sums = (float*)((char*)ws + segd_bytes(rows, NSEG));
    auto sk = mamba2_seg_sum_kernel<TV, false>;
    hipLaunchKernelGGL(sk, dim3(rows * NSEG * nvb64), dim3(256), 0, stream, (const __bf16*)k, (const TV*)v, g, sums, segd, T, G, H, V, NT, S,
                       NSEG, nvb64);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int smem = main_smem_bytes(nlev - min(slog, nlev));
  const int rows8 = (rows * NSEG + 7) / 8;
  const int grid = rows8 * 8 * nvb64;
  auto kern = mamba2_fwd_main_kernel<TV, TL, TO>;
  hipError_t e =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), smem, stream, (const __bf16*)q,
                     (const __bf16*)k, (const TV*)v, g, (const TL*)l, (TO*)o, gcum, ht, sums,
                     segd, B, T, G, H, V, L, nlev, nvb64, slog, NSEG, ht != nullptr ? 1 : 0);
  return hipGetLastError();
}

}  // namespace hattn

hipError_t hattn_mamba2_fwd_launch(const void* q, const void* k, const void* v, const float* g,
                                   const void* l, void* o, float* gcum, float* ht, void* ws,
                                   int B, int T, int G, int H, int V, int L, int nlev, int dt_v,
                                   int dt_l, int dt_o, hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
#define HATTN_DISPATCH_O(TV_, TL_)                                                             \
  if (dt_o == DT_BF16)                                                                       \
    return launch_t<TV_, TL_, __bf16>(q, k, v, g, l, o, gcum, ht, ws, B, T, G, H, V, L, nlev, \
                                      stream);                                                \
  if (dt_o == DT_FP32)                                                                       \
    return launch_t<TV_, TL_, float>(q, k, v, g, l, o, gcum, ht, ws, B, T, G, H, V, L, nlev,  \
                                     stream);
  if (dt_v == DT_BF16 && dt_l == DT_BF16) { HATTN_DISPATCH_O(__bf16, __bf16) }
  if (dt_v == DT_BF16 && dt_l == DT_FP32) { HATTN_DISPATCH_O(__bf16, float) }
  if (dt_v == DT_FP32 && dt_l == DT_BF16) { HATTN_DISPATCH_O(float, __bf16) }
  if (dt_v == DT_FP32 && dt_l == DT_FP32) { HATTN_DISPATCH_O(float, float) }
#undef HATTN_DISPATCH_O
  *unsupported = 1;
  return hipSuccess;
}
