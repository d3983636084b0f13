// Recurrent (decode) path of log-linear attention for gfx950: one token step of
// the Fenwick level state HState and the prefill of its low levels.
//
// Replaces hattention_step / step_state / step_output (hattention/kernel.py:577-633,
// recurrent.py:9-166) and the MAMBA2 fast path of postprocess_prefill_hstate_
// (kernel.py:378-465).  The reference runs a torch einsum per level and a
// Python loop over levels that reads device counts back to the host at every
// level (recurrent.py:42-54); here the weak cascade is planned on the host from
// a host copy of the counts (the counts depend only on the step number) and the
// whole step, including GDELTA's l2norm of q and k, is one launch.
//
// States: fp32 [B, H, K, V, L] (level innermost), the reference's HState layout.
// Grid (B * H, V / 16): a workgroup owns 16 value columns of one (b, h) and all
// K rows.  Every quantity of the step is per value column (the state update,
// GDELTA's k^T S and the output's sum over k), so the column slices need no
// exchange.  Thread t owns column v0 + t % 16 and rows t / 16 + 16 i, all L
// levels of each (k, v) in registers.
//
// A step with cascade depth c (levels 0 .. c-1 are full and cascade upwards,
// recurrent.py:42-54) is, per (k, v):
//   S[c] += S[0] + ... + S[c-1];  S[0 .. c-1] = 0           (cascade_weak)
//   MAMBA2: S[l] *= exp(g)                                   (insert, :88-89)
//   GDELTA: S[l] <- exp(g) (S[l] - beta k (k^T S[l]))        (insert, :90-91; step_state :146-154)
//   S[0] = k v^T (MAMBA2) or beta k v^T (GDELTA)             (insert, :93)
//   o[v] = sum_k q[k] sum_l lambda[l] S[k][v][l]              (step_output, :159-166)
#include <hip/hip_runtime.h>

#include "common.h"

namespace hattn {

constexpr int kHsMaxL = 32;   // levels held in registers per (k, v)
constexpr int kHsCols = 16;   // value columns per workgroup
constexpr int kHsRowGroups = 256 / kHsCols;

template <typename T>
__device__ __forceinline__ float ld(const T* p, size_t i) { return to_f32<T>(p[i]); }

// Sum of x over the 256 threads of the workgroup (every thread gets the sum).
__device__ __forceinline__ float block_sum256(float x, float* scratch4) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) x += __shfl_xor(x, d, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch4[threadIdx.x >> 6] = x;
  __syncthreads();
  return scratch4[0] + scratch4[1] + scratch4[2] + scratch4[3];
}

// The level counts (shared by all rows) after the step: the cascade (weak: levels
// 0 .. c-1 merge into level c; strong: levels 0 .. m-1 move up one level, m - 1
// merging into m), then one more token at level 0.
__device__ inline void cascade_counts(int* counts, int L, int cascade, int strong) {
  if (strong) {
    int prev = 0;
    for (int e = 0; e < L; ++e) {
      const int cur = counts[e];
      counts[e] = e == 0 ? 0 : (e < cascade ? prev : (e == cascade ? cur + prev : cur));
      prev = cur;
    }
  } else {
    int moved = 0;
    for (int e = 0; e < cascade; ++e) {
      moved += counts[e];
      counts[e] = 0;
    }
    if (cascade > 0) counts[cascade] += moved;
  }
  counts[0] += 1;
}

template <typename TQ, typename TV, typename TL, typename TB, bool GDN>
__global__ __launch_bounds__(256) void hstate_step_kernel(
    float* __restrict__ states, int* __restrict__ counts, const TQ* __restrict__ q,
    const TQ* __restrict__ k, const TV* __restrict__ v, const TB* __restrict__ beta,
    const float* __restrict__ g, const TL* __restrict__ l, TV* __restrict__ o, int G, int H,
    int K, int V, int L, int cascade, int strong, int update, int output, int norm_qk, float scale) {
  __shared__ float sq[256], sk[256], sv[kHsCols], sl[kHsMaxL], snorm[8];
  __shared__ float red[256 * 4];   // [row group][column][4]: k^T S per level, then o
  const int tid = threadIdx.x;
  const int v0 = blockIdx.y * kHsCols, bh = blockIdx.x, b = bh / H, h = bh % H;
  const int gq = h / (H / G);
  const int vv = tid % kHsCols, kg = tid / kHsCols;

  // q, k (l2-normalised for GDELTA: q / |q| * scale, k / |k|, kernel.py:20-23,
  // 626-629 with the eps of fla's l2norm), v columns, lambda
  // (q, lambda are read only for the output, k, v only for the update)
  float qx = 0.f, kx = 0.f;
  if (output && tid < K) qx = ld(q, ((size_t)b * G + gq) * K + tid);
  if (update && tid < K) kx = ld(k, ((size_t)b * G + gq) * K + tid);
  if (norm_qk) {
    const float nq = block_sum256(qx * qx, snorm);
    const float nk = block_sum256(kx * kx, snorm + 4);
    // rounded to the input dtype after the norm and after the scale, as the
    // reference's l2norm_fwd / l2norm_and_scale_fwd store their outputs
    qx = to_f32<TQ>(from_f32<TQ>(to_f32<TQ>(from_f32<TQ>(qx * rsqrtf(nq + 1e-6f))) * scale));
    kx = to_f32<TQ>(from_f32<TQ>(kx * rsqrtf(nk + 1e-6f)));
  }
  if (tid < K) {
    sq[tid] = qx;
    sk[tid] = kx;
  }
  if (update && tid < kHsCols) sv[tid] = ld(v, (size_t)bh * V + v0 + tid);
  if (output && tid < L) sl[tid] = ld(l, (size_t)bh * L + tid);
  __syncthreads();
  const float a = update ? __expf(g[bh]) : 0.f;
  const float bt = GDN && update ? ld(beta, (size_t)bh) : 1.f;
  float* sbase = states + (size_t)bh * K * V * L;

  auto load_cascaded = [&](int kk, float (&s)[kHsMaxL]) {
    const float* p = sbase + ((size_t)kk * V + v0 + vv) * L;
#pragma unroll
    for (int e = 0; e < kHsMaxL; ++e) s[e] = e < L ? p[e] : 0.f;
    if (strong) {
      // cascade_strong (recurrent.py:56-74) with merge level m = cascade: levels
      // 0 .. m-1 move up one level, level m - 1 merging into level m (m = L: the
      // top level's content leaves the state); level 0 ends empty
      float prev = 0.f;
#pragma unroll
      for (int e = 0; e < kHsMaxL; ++e) {
        const float cur = s[e];
        s[e] = e == 0 ? 0.f : (e < cascade ? prev : (e == cascade ? cur + prev : cur));
        prev = cur;
      }
    } else if (cascade > 0) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < kHsMaxL; ++e)
        if (e < cascade) {
          acc += s[e];
          s[e] = 0.f;
        }
#pragma unroll
      for (int e = 0; e < kHsMaxL; ++e)
        if (e == cascade) s[e] += acc;
    }
  };

  // GDELTA: u[l] = sum_k k[k] S_cascaded[k][v][l], reduced over the row groups
  float u[kHsMaxL];
#pragma unroll
  for (int e = 0; e < kHsMaxL; ++e) u[e] = 0.f;
  if (GDN && update) {
    for (int kk = kg; kk < K; kk += kHsRowGroups) {
      float s[kHsMaxL];
      load_cascaded(kk, s);
#pragma unroll
      for (int e = 0; e < kHsMaxL; ++e) u[e] += sk[kk] * s[e];
    }
    for (int e0 = 0; e0 < L; e0 += 4) {
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x = 0.f;
#pragma unroll
        for (int e = 0; e < kHsMaxL; ++e)
          if (e == e0 + j) x = u[e];
        red[(kg * kHsCols + vv) * 4 + j] = x;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x = 0.f;
        for (int gi = 0; gi < kHsRowGroups; ++gi) x += red[(gi * kHsCols + vv) * 4 + j];
#pragma unroll
        for (int e = 0; e < kHsMaxL; ++e)
          if (e == e0 + j) u[e] = x;
      }
    }
  }

  float oacc = 0.f;
  for (int kk = kg; kk < K; kk += kHsRowGroups) {
    float s[kHsMaxL];
    float* p = sbase + ((size_t)kk * V + v0 + vv) * L;
    if (update) {
      load_cascaded(kk, s);
      const float bk = bt * sk[kk];
#pragma unroll
      for (int e = 0; e < kHsMaxL; ++e) s[e] = GDN ? a * (s[e] - bk * u[e]) : a * s[e];
      s[0] = bk * sv[vv];
#pragma unroll
      for (int e = 0; e < kHsMaxL; ++e)
        if (e < L) p[e] = s[e];
    } else {
#pragma unroll
      for (int e = 0; e < kHsMaxL; ++e) s[e] = e < L ? p[e] : 0.f;
    }
    if (output) {
      float w = 0.f;
#pragma unroll
      for (int e = 0; e < kHsMaxL; ++e)
        if (e < L) w += sl[e] * s[e];
      oacc += sq[kk] * w;
    }
  }
  if (output) {
    __syncthreads();
    red[kg * kHsCols + vv] = oacc;
    __syncthreads();
    if (kg == 0) {
      float x = 0.f;
      for (int gi = 0; gi < kHsRowGroups; ++gi) x += red[gi * kHsCols + vv];
      o[(size_t)bh * V + v0 + vv] = from_f32<TV>(x);
    }
  }
  // counts (shared by all rows): the same cascade, then one more token at level 0
  if (update && counts != nullptr && blockIdx.y == 0 && bh == 0 && tid == 0)
    cascade_counts(counts, L, cascade, strong);
}

// Sum over the lanes of one wave that share lane % VB (VB a power of two <= 32):
// butterfly over the lane bits above log2(VB).
__device__ __forceinline__ float wave_sum_same_col(float x, int VB) {
  for (int d = 32; d >= VB; d >>= 1) x += __shfl_xor(x, d, 64);
  return x;
}

// The same step as hstate_step_kernel with the workgroup's state slab staged
// in LDS: the slab (K rows of VB * L contiguous floats, row stride V * L) moves
// between HBM and LDS in 16-byte pieces, all of a thread's loads issued before
// the first is consumed, and the per-(k, v) work reads the slab from LDS with
// each (k, v) group of L levels padded to an odd stride (conflict-free reads).
// Grid (B * H, V / VB); VB in {4, 8, 16} is chosen by the host so that the slab
// fits in LDS; NL (16 or 32) bounds the levels held in registers.  Dynamic
// LDS: K * VB * (L | 1) floats.
constexpr int kHsBatch = 8;    // 16-byte pieces in flight per thread

template <typename TQ, typename TV, typename TL, typename TB, bool GDN, int NL>
__global__ __launch_bounds__(256) void hstate_step_lds_kernel(
    float* __restrict__ states, int* __restrict__ counts, const TQ* __restrict__ q,
    const TQ* __restrict__ k, const TV* __restrict__ v, const TB* __restrict__ beta,
    const float* __restrict__ g, const TL* __restrict__ l, TV* __restrict__ o, int G, int H,
    int K, int V, int L, int VB, int cascade, int strong, int update, int output, int norm_qk,
    float scale) {
  extern __shared__ float slab[];
  __shared__ float sq[256], sk[256], sv[kHsCols], sl[NL], snorm[8];
  __shared__ float red[4 * kHsCols * NL];   // [wave][column][level]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int v0 = blockIdx.y * VB, bh = blockIdx.x, b = bh / H, h = bh % H;
  const int gq = h / (H / G);
  const int Lp = L | 1, W = VB * L, W4 = W >> 2, n4 = K * W4;
  float* src = states + (size_t)bh * K * V * L + (size_t)v0 * L;
  const size_t rstride = (size_t)V * L;
  // piece f = tid + 256 i sits at (row, off) = divmod(f, W4); advanced without
  // dividing: 256 = dq * W4 + dr
  const int dq = 256 / W4, dr = 256 - dq * W4;
  int row = tid / W4, off = tid - (tid / W4) * W4;
  floatx4 x[kHsBatch];
  int brow = row, boff = off;   // (row, off) of the batch's first piece
  auto advance = [&](int& r, int& c) {
    r += dq;
    c += dr;
    if (c >= W4) {
      c -= W4;
      ++r;
    }
  };
  auto load_batch = [&]() {
    brow = row;
    boff = off;
#pragma unroll
    for (int i = 0; i < kHsBatch; ++i) {
      if (row < K) x[i] = *(const floatx4*)(src + row * rstride + 4 * off);
      advance(row, off);
    }
  };
  // padded LDS offset of element w of a row: group w / L, level w % L (the
  // quotient by a float reciprocal: exact for w < 2^16, L <= 32, as (w + 0.5) / L
  // is at least 1 / (2L) away from an integer)
  const float invL = 1.f / (float)L;
  auto pad = [&](int w) {
    const int grp = (int)((float)w * invL + 0.5f * invL);
    return grp * Lp + (w - grp * L);
  };
  auto store_batch_lds = [&]() {
    int r = brow, c = boff;
#pragma unroll
    for (int i = 0; i < kHsBatch; ++i) {
      if (r < K) {
        float* d = slab + r * VB * Lp;
#pragma unroll
        for (int j = 0; j < 4; ++j) d[pad(4 * c + j)] = x[i][j];
      }
      advance(r, c);
    }
  };

  // ---- HBM -> LDS: the first batch of state loads goes out before the small
  // operands are read, so their latencies overlap
  load_batch();
  float qx = 0.f, kx = 0.f;
  if (output && tid < K) qx = ld(q, ((size_t)b * G + gq) * K + tid);
  if (update && tid < K) kx = ld(k, ((size_t)b * G + gq) * K + tid);
  const float a = update ? __expf(g[bh]) : 0.f;
  const float bt = GDN && update ? ld(beta, (size_t)bh) : 1.f;
  if (update && tid < VB) sv[tid] = ld(v, (size_t)bh * V + v0 + tid);
  if (output && tid < L) sl[tid] = ld(l, (size_t)bh * L + tid);
  if (norm_qk) {
    const float nq = block_sum256(qx * qx, snorm);
    const float nk = block_sum256(kx * kx, snorm + 4);
    qx = to_f32<TQ>(from_f32<TQ>(to_f32<TQ>(from_f32<TQ>(qx * rsqrtf(nq + 1e-6f))) * scale));
    kx = to_f32<TQ>(from_f32<TQ>(kx * rsqrtf(nk + 1e-6f)));
  }
  if (tid < K) {
    sq[tid] = qx;
    sk[tid] = kx;
  }
  store_batch_lds();
  for (int f0 = 256 * kHsBatch; f0 < n4; f0 += 256 * kHsBatch) {
    load_batch();
    store_batch_lds();
  }
  __syncthreads();

  // ---- per (k, v) work: thread owns column vv = tid % VB, rows tid / VB + (256 / VB) i
  const int vv = tid & (VB - 1), kg = tid / VB, nkg = 256 / VB;
  auto load_cascaded = [&](int kk, float (&s)[NL]) {
    const float* p = slab + (kk * VB + vv) * Lp;
#pragma unroll
    for (int e = 0; e < NL; ++e) s[e] = e < L ? p[e] : 0.f;
    if (strong) {
      float prev = 0.f;   // cascade_strong, as in hstate_step_kernel
#pragma unroll
      for (int e = 0; e < NL; ++e) {
        const float cur = s[e];
        s[e] = e == 0 ? 0.f : (e < cascade ? prev : (e == cascade ? cur + prev : cur));
        prev = cur;
      }
    } else if (cascade > 0) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < NL; ++e)
        if (e < cascade) {
          acc += s[e];
          s[e] = 0.f;
        }
#pragma unroll
      for (int e = 0; e < NL; ++e)
        if (e == cascade) s[e] += acc;
    }
  };

  float u[NL];
#pragma unroll
  for (int e = 0; e < NL; ++e) u[e] = 0.f;
  if (GDN && update) {
    for (int kk = kg; kk < K; kk += nkg) {
      float s[NL];
      load_cascaded(kk, s);
#pragma unroll
      for (int e = 0; e < NL; ++e) u[e] += sk[kk] * s[e];
    }
#pragma unroll
    for (int e = 0; e < NL; ++e)
      if (e < L) {
        const float x = wave_sum_same_col(u[e], VB);
        if (lane < VB) red[(wave * kHsCols + vv) * NL + e] = x;
      }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < NL; ++e)
      if (e < L)
        u[e] = red[(0 * kHsCols + vv) * NL + e] + red[(1 * kHsCols + vv) * NL + e] +
               red[(2 * kHsCols + vv) * NL + e] + red[(3 * kHsCols + vv) * NL + e];
  }

  float oacc = 0.f;
  for (int kk = kg; kk < K; kk += nkg) {
    float s[NL];
    float* p = slab + (kk * VB + vv) * Lp;
    if (update) {
      load_cascaded(kk, s);
      const float bk = bt * sk[kk];
#pragma unroll
      for (int e = 0; e < NL; ++e) s[e] = GDN ? a * (s[e] - bk * u[e]) : a * s[e];
      s[0] = bk * sv[vv];
#pragma unroll
      for (int e = 0; e < NL; ++e)
        if (e < L) p[e] = s[e];
    } else {
#pragma unroll
      for (int e = 0; e < NL; ++e) s[e] = e < L ? p[e] : 0.f;
    }
    if (output) {
      float w = 0.f;
#pragma unroll
      for (int e = 0; e < NL; ++e)
        if (e < L) w += sl[e] * s[e];
      oacc += sq[kk] * w;
    }
  }
  if (output) {
    oacc = wave_sum_same_col(oacc, VB);
    __syncthreads();   // red is reused
    if (lane < VB) red[wave * kHsCols + vv] = oacc;
    __syncthreads();
    if (tid < VB)
      o[(size_t)bh * V + v0 + tid] =
          from_f32<TV>(red[tid] + red[kHsCols + tid] + red[2 * kHsCols + tid] +
                       red[3 * kHsCols + tid]);
  }

  // ---- LDS -> HBM
  if (update) {
    __syncthreads();
    row = tid / W4;
    off = tid - row * W4;
    for (int f0 = 0; f0 < n4; f0 += 256) {
      if (row < K) {
        const float* d = slab + row * VB * Lp;
        floatx4 x;
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = d[pad(4 * off + j)];
        *(floatx4*)(src + row * rstride + 4 * off) = x;
      }
      advance(row, off);
    }
    if (counts != nullptr && blockIdx.y == 0 && bh == 0 && tid == 0)
      cascade_counts(counts, L, cascade, strong);
  }
}

// Levels 0 .. nlo - 1 after a prefill of T tokens (MAMBA2 fast path of
// postprocess_prefill_hstate_, kernel.py:420-436): level 0 holds k v^T of token
// T - 1; level e >= 1 holds the 2^(e-1) tokens before the tokens of levels
// < e, i.e. chunk offsets [64 - 2^e, 64 - 2^(e-1)) of the last chunk, each token
// s weighted by exp(sum_{u = s+1}^{T-1} g_u) (the reverse chunk-local cumsum
// gr[s + 1] of :420).  Grid (B * H, V / 16); the last chunk's k rows and its
// weighted v columns are staged in LDS as fp32.
template <typename TK, typename TV>
__global__ __launch_bounds__(256) void mamba2_prefill_levels_kernel(
    float* __restrict__ states, const TK* __restrict__ k, const TV* __restrict__ v,
    const float* __restrict__ g, int T, int G, int H, int K, int V, int L, int nlo) {
  __shared__ float sk[64 * 256];      // [token][k]
  __shared__ float sv[64 * kHsCols];  // [token][column], weighted
  __shared__ float sw[64];            // sw[j]: weight of chunk offset j
  const int tid = threadIdx.x;
  const int v0 = blockIdx.y * kHsCols, bh = blockIdx.x, b = bh / H, h = bh % H;
  const int gq = h / (H / G);
  const int t0 = T - 64;     // the host guarantees T >= 64 (a prefill of whole chunks)
  if (tid < 64) {
    // lane i scans g of offset 63 - i: P_i = sum_{m <= i} g_{t0 + 63 - m}, the
    // suffix sum from offset 63 - i; offset j's weight is exp(P_{62 - j})
    float r = g[((size_t)b * T + t0 + 63 - tid) * H + h];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float z = __shfl_up(r, d, 64);
      if (tid >= d) r += z;
    }
    if (tid <= 62) sw[62 - tid] = __expf(r);
    else sw[63] = 1.f;
  }
  for (int i = tid; i < 64 * K; i += 256) {
    const int j = i / K, kk = i % K;
    sk[j * 256 + kk] = to_f32<TK>(k[(((size_t)b * T + t0 + j) * G + gq) * K + kk]);
  }
  __syncthreads();
  for (int i = tid; i < 64 * kHsCols; i += 256) {
    const int j = i / kHsCols, c = i % kHsCols;
    sv[i] = sw[j] * to_f32<TV>(v[(((size_t)b * T + t0 + j) * H + h) * V + v0 + c]);
  }
  __syncthreads();
  const int vv = tid % kHsCols, kg = tid / kHsCols;
  float* sbase = states + (size_t)bh * K * V * L;
  for (int kk = kg; kk < K; kk += kHsRowGroups) {
    float* p = sbase + ((size_t)kk * V + v0 + vv) * L;
    p[0] = sk[63 * 256 + kk] * sv[63 * kHsCols + vv];
    for (int e = 1; e < nlo; ++e) {
      float acc = 0.f;
      for (int j = 64 - (1 << e); j < 64 - (1 << (e - 1)); ++j)
        acc += sk[j * 256 + kk] * sv[j * kHsCols + vv];
      p[e] = acc;
    }
  }
}

}  // namespace hattn

enum { HS_BF16 = 0, HS_FP16 = 1, HS_FP32 = 2 };

namespace {

// Calls f with a value of the element type named by dtype code dt (bf16 or
// fp32); returns false for any other code.
template <typename F>
bool with_type(int dt, F&& f) {
  if (dt == HS_BF16) {
    f(__bf16{});
    return true;
  }
  if (dt == HS_FP32) {
    f(float{});
    return true;
  }
  return false;
}

}  // namespace

hipError_t hattn_hstate_step_launch(float* states, int* counts, const void* q, const void* k,
                                    const void* v, const void* beta, const float* g,
                                    const void* l, void* o, int B, int G, int H, int K, int V,
                                    int L, int gdn, int cascade, int strong, int update,
                                    int output, int norm_qk, float scale, int dt_qk, int dt_v,
                                    int dt_l, int dt_b, hipStream_t stream, int* unsupported) {
  using namespace hattn;
  const bool known = (dt_qk == HS_BF16 || dt_qk == HS_FP32) &&
                     (dt_v == HS_BF16 || dt_v == HS_FP32) &&
                     (dt_l == HS_BF16 || dt_l == HS_FP32) &&
                     (!gdn || dt_b == HS_BF16 || dt_b == HS_FP32);
  *unsupported = known ? 0 : 1;
  if (!known) return hipSuccess;
  // LDS-staged kernel when the slab of VB columns fits (VB = 16, halved while
  // the grid has fewer than 1024 workgroups or the slab exceeds 40 KB, so that
  // several workgroups share a CU and their load / compute / store phases
  // overlap); the register kernel otherwise (large K * L) or when the state
  // pointer is not 16-byte aligned
  const int Lp = L | 1;
  int VB = 16;
  auto slab_bytes = [&](int vb) { return (size_t)K * vb * Lp * sizeof(float); };
  while (VB > 4 && ((long)B * H * (V / VB) < 1024 || slab_bytes(VB) > 40 * 1024)) VB >>= 1;
  const bool use_lds = slab_bytes(VB) <= 144 * 1024 && ((uintptr_t)states & 15) == 0;
  const int smem = (int)slab_bytes(VB);
  hipError_t err = hipSuccess;
  auto launch = [&](auto kern_lds, auto kern_reg, auto tq, auto tv, auto tl, auto tb) {
    using TQ = decltype(tq);
    using TV = decltype(tv);
    using TL = decltype(tl);
    using TB = decltype(tb);
    if (use_lds) {
      if ((err = hipFuncSetAttribute((const void*)kern_lds,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, smem)) !=
          hipSuccess)
        return;
      hipLaunchKernelGGL(kern_lds, dim3(B * H, V / VB), dim3(256), smem, stream, states, counts,
                         (const TQ*)q, (const TQ*)k, (const TV*)v, (const TB*)beta, g,
                         (const TL*)l, (TV*)o, G, H, K, V, L, VB, cascade, strong, update, output,
                         norm_qk, scale);
    } else {
      hipLaunchKernelGGL(kern_reg, dim3(B * H, V / kHsCols), dim3(256), 0, stream, states,
                         counts, (const TQ*)q, (const TQ*)k, (const TV*)v, (const TB*)beta, g,
                         (const TL*)l, (TV*)o, G, H, K, V, L, cascade, strong, update, output, norm_qk,
                         scale);
    }
  };
  with_type(dt_qk, [&](auto tq) {
    using TQ = decltype(tq);
    with_type(dt_v, [&](auto tv) {
      using TV = decltype(tv);
      with_type(dt_l, [&](auto tl) {
        using TL = decltype(tl);
        if (!gdn) {
          if (L <= 16)
            launch(hstate_step_lds_kernel<TQ, TV, TL, float, false, 16>,
                   hstate_step_kernel<TQ, TV, TL, float, false>, tq, tv, tl, float{});
          else
            launch(hstate_step_lds_kernel<TQ, TV, TL, float, false, 32>,
                   hstate_step_kernel<TQ, TV, TL, float, false>, tq, tv, tl, float{});
          return;
        }
        with_type(dt_b, [&](auto tb) {
          using TB = decltype(tb);
          if (L <= 16)
            launch(hstate_step_lds_kernel<TQ, TV, TL, TB, true, 16>,
                   hstate_step_kernel<TQ, TV, TL, TB, true>, tq, tv, tl, tb);
          else
            launch(hstate_step_lds_kernel<TQ, TV, TL, TB, true, 32>,
                   hstate_step_kernel<TQ, TV, TL, TB, true>, tq, tv, tl, tb);
        });
      });
    });
  });
  if (err != hipSuccess) return err;
  return hipGetLastError();
}

hipError_t hattn_mamba2_prefill_levels_launch(float* states, const void* k, const void* v,
                                              const float* g, int B, int T, int G, int H, int K,
                                              int V, int L, int nlo, int dt_k, int dt_v,
                                              hipStream_t stream, int* unsupported) {
  using namespace hattn;
  const dim3 grid(B * H, V / kHsCols), block(256);
  *unsupported = 0;
  const bool known = (dt_k == HS_BF16 || dt_k == HS_FP32) && (dt_v == HS_BF16 || dt_v == HS_FP32);
  if (!known) {
    *unsupported = 1;
    return hipSuccess;
  }
  with_type(dt_k, [&](auto tk) {
    using TK = decltype(tk);
    with_type(dt_v, [&](auto tv) {
      using TV = decltype(tv);
      hipLaunchKernelGGL((mamba2_prefill_levels_kernel<TK, TV>), grid, block, 0, stream, states,
                         (const TK*)k, (const TV*)v, g, T, G, H, K, V, L, nlo);
    });
  });
  return hipGetLastError();
}
