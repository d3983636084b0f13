// Log-linear Mamba-2 chunkwise forward, fused into one pass over the sequence.
//
// Replaces the reference's 1 + 2 * nlev Triton launches (chunkwise.py:1118-1275:
// chunk_fwd_kernel_o with USE_A, then per inter-chunk level chunk_fwd_kernel_h
// and chunk_fwd_kernel_o) with a single launch that reads q, k, v, g, lambda
// once and writes o once.
//
// One workgroup (4 wavefronts) owns one (batch, head) row and one 16-wide slice
// of V and walks the 64-token chunks in order:
//   * intra-chunk tile: S^T = K Q^T on MFMA, masked by the causal mask, scaled
//     by exp(Gc_t - Gc_s) and lambda[t, bit_length(t ^ s)] in registers, then
//     A V on MFMA (the D fragment of S^T is the A operand of A V);
//   * inter-chunk Fenwick levels: the per-level K x V states live in fp32
//     registers (wave w owns state rows 16w..16w+15) and are mirrored in LDS as
//     bf16 for the levels the next chunk reads; each chunk's decayed K^T V is
//     computed once and added to every level whose bit is clear (the reference
//     recomputes it once per level, chunkwise.py:256-266);
//   * reading levels (bits set in the chunk index) add
//     lambda[t, 7 + ell] * exp(Gc_t) * q_t h_ell to the same fp32 accumulator,
//     so o is stored once.
// Loads for chunk i+1 are issued before chunk i is computed (register
// prefetch); LDS holds two input stages and two state buffers, so one barrier
// per chunk suffices.
#include "common.h"

namespace hattn {

constexpr int kBT = 64;       // chunk length (the reference's only chunk size)
constexpr int kKD = 64;       // head dim of q / k
constexpr int kBV = 16;       // V columns per workgroup
constexpr int kMaxLev = 17;   // inter-chunk levels supported (T <= 64 * 2^17)
constexpr int kRow = 72;      // LDS row stride (bf16) of 64-wide tiles
constexpr int kLamPerLane = 6;  // lambda elements per lane per chunk (16 rows x <= 24 cols)

struct FwdSmem {
  int stage_bytes;
  int off_k, off_kt, off_vt, off_gc, off_lam;
  int off_h;      // state mirror: [2][nlev][kBV][kRow] bf16
  int total;
  int lam_stride;
};

__host__ __device__ inline FwdSmem fwd_smem_layout(int nlev) {
  FwdSmem s;
  const int lu = 7 + nlev;
  s.lam_stride = lu | 1;
  s.off_k = 0;
  s.off_kt = s.off_k + kBT * kRow * 2;
  s.off_vt = s.off_kt + kKD * kRow * 2;
  s.off_gc = s.off_vt + kBV * kRow * 2;
  s.off_lam = s.off_gc + kBT * 4;
  int end = s.off_lam + kBT * s.lam_stride * 4;
  s.stage_bytes = (end + 15) & ~15;
  s.off_h = 2 * s.stage_bytes;
  s.total = s.off_h + 2 * (nlev > 0 ? nlev : 1) * kBV * kRow * 2;
  return s;
}

// Registers holding one chunk's global loads until they are written to LDS.
template <typename TV, typename TL>
struct ChunkRegs {
  bf16x8 q[2];   // own rows of Q in the MFMA fragment layout
  uint4 k[2];    // two 16-byte units of K (row = u / 8, cols 8 * (u % 8) ..)
  uint4 v;       // one 16-byte unit of the V slice
  float g;       // g[t] for t = lane (wave 0 only)
  TL lam[kLamPerLane];
};

template <typename TV, typename TL>
__device__ __forceinline__ void load_chunk(ChunkRegs<TV, TL>& r, const __bf16* __restrict__ q,
                                           const __bf16* __restrict__ k, const TV* __restrict__ v,
                                           const float* __restrict__ g, const TL* __restrict__ l,
                                           int b, int h, int gq, int vb, int t0, int T, int G,
                                           int H, int V, int L, int lu) {
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const size_t rowq = (size_t)b * T + t0;
  // Q: lane (lq, ln) -> row 16w + ln, cols 32c + 8lq .. +7
  {
    const __bf16* p = q + ((rowq + 16 * w + ln) * G + gq) * kKD + 8 * lq;
    r.q[0] = *(const bf16x8*)(p);
    r.q[1] = *(const bf16x8*)(p + 32);
  }
  // K: units u = tid, tid + 256 ; row u >> 3, col 8 * (u & 7)
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int u = tid + 256 * rr;
    const __bf16* p = k + ((rowq + (u >> 3)) * G + gq) * kKD + 8 * (u & 7);
    r.k[rr] = *(const uint4*)p;
  }
  // V slice: 64 rows x 16 columns
  if constexpr (sizeof(TV) == 2) {
    if (tid < 128) {
      const TV* p = v + ((rowq + (tid >> 1)) * H + h) * V + vb * kBV + 8 * (tid & 1);
      r.v = *(const uint4*)p;
    }
  } else {
    const TV* p = v + ((rowq + (tid >> 2)) * H + h) * V + vb * kBV + 4 * (tid & 3);
    r.v = *(const uint4*)p;
  }
  if (w == 0) r.g = g[(rowq + lane) * H + h];
  // lambda: wave w loads its own 16 rows, lu columns
#pragma unroll
  for (int rr = 0; rr < kLamPerLane; ++rr) {
    const int e = lane + 64 * rr;
    if (e < 16 * lu) {
      const int row = 16 * w + e / lu, col = e % lu;
      r.lam[rr] = l[((rowq + row) * H + h) * L + col];
    }
  }
}

template <typename TV, typename TL>
__device__ __forceinline__ void store_chunk(const ChunkRegs<TV, TL>& r, unsigned char* stage,
                                            const FwdSmem& sm, int lu, float* __restrict__ gcum,
                                            size_t gcum_base, int H, bool write_gcum) {
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  __bf16* kS = (__bf16*)(stage + sm.off_k);
  __bf16* kT = (__bf16*)(stage + sm.off_kt);
  __bf16* vT = (__bf16*)(stage + sm.off_vt);
  float* gc = (float*)(stage + sm.off_gc);
  float* lam = (float*)(stage + sm.off_lam);
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int u = tid + 256 * rr;
    const int row = u >> 3, c0 = 8 * (u & 7);
    *(uint4*)(kS + row * kRow + c0) = r.k[rr];
    const __bf16* e = (const __bf16*)&r.k[rr];
#pragma unroll
    for (int j = 0; j < 8; ++j) kT[(c0 + j) * kRow + row] = e[j];
  }
  if constexpr (sizeof(TV) == 2) {
    if (tid < 128) {
      const int row = tid >> 1, c0 = 8 * (tid & 1);
      const TV* e = (const TV*)&r.v;
#pragma unroll
      for (int j = 0; j < 8; ++j) vT[(c0 + j) * kRow + row] = from_f32<__bf16>(to_f32<TV>(e[j]));
    }
  } else {
    const int row = tid >> 2, c0 = 4 * (tid & 3);
    const TV* e = (const TV*)&r.v;
#pragma unroll
    for (int j = 0; j < 4; ++j) vT[(c0 + j) * kRow + row] = from_f32<__bf16>(to_f32<TV>(e[j]));
  }
  if (w == 0) {
    // inclusive chunk-local cumsum of g (fla chunk_local_cumsum, chunkwise.py:1175)
    float x = r.g;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      float y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    gc[lane] = x;
    if (write_gcum) gcum[gcum_base + (size_t)lane * H] = x;
  }
#pragma unroll
  for (int rr = 0; rr < kLamPerLane; ++rr) {
    const int e = lane + 64 * rr;
    if (e < 16 * lu) {
      const int row = 16 * w + e / lu, col = e % lu;
      lam[row * sm.lam_stride + col] = to_f32<TL>(r.lam[rr]);
    }
  }
}

template <typename TV, typename TL, typename TO>
__global__ __launch_bounds__(256, 1) void mamba2_fwd_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const TV* __restrict__ v,
    const float* __restrict__ g, const TL* __restrict__ l, TO* __restrict__ o,
    float* __restrict__ gcum, float* __restrict__ ht, int B, int T, int G, int H, int V, int L,
    int nlev, int nvb, int final_state) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  const XcdMap m = xcd_map(blockIdx.x, nvb);
  const int BH = B * H;
  if (m.row >= BH) return;
  const int b = m.row / H, h = m.row % H, vb = m.slice;
  const int gq = h / (H / G);
  const int NT = T / kBT;
  const int lu = 7 + nlev;
  const FwdSmem sm = fwd_smem_layout(nlev);
  __bf16* hT = (__bf16*)(smem + sm.off_h);
  const int hbuf_elems = nlev * kBV * kRow;

  floatx4 st[kMaxLev];
#pragma unroll
  for (int e = 0; e < kMaxLev; ++e) st[e] = zero4();

  ChunkRegs<TV, TL> cur, nxt;
  load_chunk(cur, q, k, v, g, l, b, h, gq, vb, 0, T, G, H, V, L, lu);
  const bool write_gcum = (gcum != nullptr) && vb == 0;
  store_chunk(cur, smem, sm, lu, gcum, ((size_t)b * T) * H + h, H, write_gcum);
  if (NT > 1) load_chunk(nxt, q, k, v, g, l, b, h, gq, vb, kBT, T, G, H, V, L, lu);
  __syncthreads();

  for (int ic = 0; ic < NT; ++ic) {
    const unsigned char* stage = smem + (ic & 1) * sm.stage_bytes;
    const __bf16* kS = (const __bf16*)(stage + sm.off_k);
    const __bf16* kT = (const __bf16*)(stage + sm.off_kt);
    const __bf16* vT = (const __bf16*)(stage + sm.off_vt);
    const float* gc = (const float*)(stage + sm.off_gc);
    const float* lam = (const float*)(stage + sm.off_lam);
    const int LS = sm.lam_stride;

    // ---- intra-chunk: S^T tiles (s-tile j, t-tile w), j <= w -----------------
    const int t = 16 * w + ln;
    const float gct = gc[t];
    floatx4 sT[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sT[j] = zero4();
      if (j <= w) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const bf16x8 a = *(const bf16x8*)(kS + (16 * j + ln) * kRow + 32 * c + 8 * lq);
          sT[j] = mfma16x16x32(a, cur.q[c], sT[j]);
        }
        const floatx4 gs = *(const floatx4*)(gc + 16 * j + 4 * lq);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int s = 16 * j + 4 * lq + i;
          float val = 0.f;
          if (s <= t) val = sT[j][i] * fexp(gct - gs[i]) * lam[t * LS + intra_level(t, s)];
          sT[j][i] = val;
        }
      }
    }
    // ---- A V: contraction over s, pairs of s-tiles (2p, 2p + 1) ----------------
    floatx4 acc = zero4();
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (2 * p <= w) {
        bf16x8 a, bv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = (__bf16)sT[2 * p][i];
          a[4 + i] = (__bf16)sT[2 * p + 1][i];
        }
        const bf16x4 v0 = *(const bf16x4*)(vT + ln * kRow + 32 * p + 4 * lq);
        const bf16x4 v1 = *(const bf16x4*)(vT + ln * kRow + 32 * p + 16 + 4 * lq);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bv[i] = v0[i];
          bv[4 + i] = v1[i];
        }
        acc = mfma16x16x32(a, bv, acc);
      }
    }
    // ---- inter-chunk levels read by this chunk (bits set in ic) ----------------
    if (ic > 0) {
      const __bf16* hR = hT + (ic & 1) * hbuf_elems;
      float eg[4];
      const floatx4 g4 = *(const floatx4*)(gc + 16 * w + 4 * lq);
#pragma unroll
      for (int i = 0; i < 4; ++i) eg[i] = fexp(g4[i]);
#pragma unroll
      for (int e = 0; e < kMaxLev; ++e) {
        if (e < nlev && ((ic >> e) & 1)) {
          floatx4 tmp = zero4();
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const bf16x8 bh = *(const bf16x8*)(hR + (e * kBV + ln) * kRow + 32 * c + 8 * lq);
            tmp = mfma16x16x32(cur.q[c], bh, tmp);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[i] += tmp[i] * eg[i] * lam[(16 * w + 4 * lq + i) * LS + 7 + e];
        }
      }
    }
    // ---- store o ---------------------------------------------------------------
    {
      const size_t base = (((size_t)b * T + ic * kBT + 16 * w + 4 * lq) * H + h) * V + vb * kBV + ln;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[base + (size_t)i * H * V] = from_f32<TO>(acc[i]);
    }
    // ---- state update: wave w owns state rows k = 16w .. 16w + 15 --------------
    {
      const float glr = gc[kBT - 1];
      floatx4 kv = zero4();
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const bf16x8 a = *(const bf16x8*)(kT + (16 * w + ln) * kRow + 32 * c + 8 * lq);
        const bf16x8 vv = *(const bf16x8*)(vT + ln * kRow + 32 * c + 8 * lq);
        const floatx4 gA = *(const floatx4*)(gc + 32 * c + 8 * lq);
        const floatx4 gB = *(const floatx4*)(gc + 32 * c + 8 * lq + 4);
        bf16x8 bv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bv[j] = (__bf16)((float)vv[j] * fexp(glr - gA[j]));
          bv[4 + j] = (__bf16)((float)vv[4 + j] * fexp(glr - gB[j]));
        }
        kv = mfma16x16x32(a, bv, kv);
      }
      const float gl = fexp(glr);
      __bf16* hW = hT + ((ic + 1) & 1) * hbuf_elems;
      const bool last = (ic == NT - 1);
#pragma unroll
      for (int e = 0; e < kMaxLev; ++e) {
        if (e < nlev) {
          const int per = 2 << e;
          const bool reset = ((ic & (per - 1)) == per - 1) && !(last && final_state);
          const bool write_kv = !((ic >> e) & 1);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float x = reset ? 0.f : st[e][i] * gl;
            if (write_kv) x += kv[i];
            st[e][i] = x;
          }
          if (!last && (((ic + 1) >> e) & 1)) {
            bf16x4 hb;
#pragma unroll
            for (int i = 0; i < 4; ++i) hb[i] = (__bf16)st[e][i];
            *(bf16x4*)(hW + (e * kBV + ln) * kRow + 16 * w + 4 * lq) = hb;
          }
        }
      }
      if (last && ht != nullptr) {
        // ht[b, h, k, v, 7 + e] (chunkwise.py:1179, 277-279)
#pragma unroll
        for (int e = 0; e < kMaxLev; ++e) {
          if (e < nlev) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int kk = 16 * w + 4 * lq + i, vv = vb * kBV + ln;
              ht[((((size_t)b * H + h) * kKD + kk) * V + vv) * L + 7 + e] = st[e][i];
            }
          }
        }
      }
    }
    // ---- stage the next chunk --------------------------------------------------
    if (ic + 1 < NT) {
      cur = nxt;
      store_chunk(cur, smem + ((ic + 1) & 1) * sm.stage_bytes, sm, lu, gcum,
                  ((size_t)b * T + (ic + 1) * kBT) * H + h, H, write_gcum);
      if (ic + 2 < NT)
        load_chunk(nxt, q, k, v, g, l, b, h, gq, vb, (ic + 2) * kBT, T, G, H, V, L, lu);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// host launcher
// ---------------------------------------------------------------------------
template <typename TV, typename TL, typename TO>
static hipError_t launch_t(const void* q, const void* k, const void* v, const float* g,
                           const void* l, void* o, float* gcum, float* ht, int B, int T, int G,
                           int H, int V, int L, int nlev, hipStream_t stream) {
  const FwdSmem sm = fwd_smem_layout(nlev);
  const int nvb = V / kBV;
  const int rows8 = (B * H + 7) / 8;
  const int grid = rows8 * 8 * nvb;
  auto kern = mamba2_fwd_kernel<TV, TL, TO>;
  hipError_t e = hipFuncSetAttribute((const void*)kern,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, sm.total);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), sm.total, stream, (const __bf16*)q,
                     (const __bf16*)k, (const TV*)v, g, (const TL*)l, (TO*)o, gcum, ht, B, T, G,
                     H, V, L, nlev, nvb, ht != nullptr ? 1 : 0);
  return hipGetLastError();
}

}  // namespace hattn

// dtype codes shared with the C-ABI (include/hattn.h)
enum { DT_BF16 = 0, DT_FP16 = 1, DT_FP32 = 2 };

hipError_t hattn_mamba2_fwd_launch(const void* q, const void* k, const void* v, const float* g,
                                   const void* l, void* o, float* gcum, float* ht, int B, int T,
                                   int G, int H, int V, int L, int nlev, int dt_v, int dt_l,
                                   int dt_o, hipStream_t stream, int* unsupported) {
  using namespace hattn;
  *unsupported = 0;
#define HATTN_DISPATCH_O(TV_, TL_)                                                             \
  if (dt_o == DT_BF16)                                                                       \
    return launch_t<TV_, TL_, __bf16>(q, k, v, g, l, o, gcum, ht, B, T, G, H, V, L, nlev, stream); \
  if (dt_o == DT_FP32)                                                                       \
    return launch_t<TV_, TL_, float>(q, k, v, g, l, o, gcum, ht, B, T, G, H, V, L, nlev, stream);
  if (dt_v == DT_BF16 && dt_l == DT_BF16) { HATTN_DISPATCH_O(__bf16, __bf16) }
  if (dt_v == DT_BF16 && dt_l == DT_FP32) { HATTN_DISPATCH_O(__bf16, float) }
  if (dt_v == DT_FP32 && dt_l == DT_BF16) { HATTN_DISPATCH_O(float, __bf16) }
  if (dt_v == DT_FP32 && dt_l == DT_FP32) { HATTN_DISPATCH_O(float, float) }
#undef HATTN_DISPATCH_O
  *unsupported = 1;
  return hipSuccess;
}
