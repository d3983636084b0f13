// Shared pieces of the log-linear Gated DeltaNet kernels (forward and backward).
#pragma once
#include "common.h"

namespace hattn {

constexpr int kGC = 64;       // chunk length
constexpr int kLd64 = 72;     // LDS row stride of 64-wide bf16 tiles
constexpr int kGMaxLev = 7;   // inter-chunk levels held by the scans (T <= 64 * 2^7)
constexpr int kBVs = 32;      // V columns per scan workgroup
constexpr int kLM = 65;       // row stride of 64 x 64 fp32 LDS matrices

// 16-byte units of a row-major [NR][N] bf16 tile, 256 threads (threads
// T0 .. T0 + 255 of the workgroup).  The unit loop has a compile-time trip
// count and every load is issued before the first LDS store, so the tile costs
// one memory round trip instead of one per unit.
template <int N, int NR = kGC, int T0 = 0>
__device__ __forceinline__ void g2s_tile(const __bf16* __restrict__ src, size_t row_stride,
                                         __bf16* dst, int ld) {
  constexpr int UPR = N / 8, NU = NR * UPR, IT = (NU + 255) / 256;   // units per row / in all / per thread
  const int t = (int)threadIdx.x - T0;
  u32x4 r[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int u = (NU % 256 == 0) ? t + 256 * i : min(t + 256 * i, NU - 1);
    r[i] = *(const u32x4*)(src + (size_t)(u / UPR) * row_stride + 8 * (u % UPR));
  }
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int u = t + 256 * i;
    if (NU % 256 == 0 || u < NU) *(u32x4*)(dst + (u / UPR) * ld + 8 * (u % UPR)) = r[i];
  }
}

// X = (I + A)^-1 for a strictly lower-triangular 64 x 64 fp32 A (row stride kLM),
// in fp32: the 16 x 16 diagonal blocks by forward substitution (lane ln of wave w
// owns column ln of block w), then the off-diagonal blocks by distance d,
//   X_ij = -X_ii sum_{m=j}^{i-1} A_im X_mj,
// with a per-wave 16 x 17 scratch t1all[w].  The upper blocks of X are set to
// zero.  256 threads; starts and ends with the caller's data in LDS and ends
// with a barrier.
// NTHR threads call it together; waves 0..3 do the block work (the others only
// take part in the zero fill and the barriers).
template <int NTHR = 256>
__device__ inline void tri_inv64(const float* A, float* X, float (*t1all)[16 * 17]) {
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  for (int u = tid; u < 6 * 256; u += NTHR) {   // the six upper 16 x 16 blocks
    const int blk = u >> 8, e = u & 255;
    const int bi = blk < 3 ? 0 : (blk < 5 ? 1 : 2);
    const int bj = blk < 3 ? blk + 1 : (blk < 5 ? blk - 1 : 3);
    X[(16 * bi + (e >> 4)) * kLM + 16 * bj + (e & 15)] = 0.f;
  }
  if (w < 4 && lq == 0) {
    const int o = 16 * w;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = (i == ln) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) acc -= A[(o + i) * kLM + o + j] * x[j];
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) X[(o + i) * kLM + o + ln] = x[i];
  }
  __syncthreads();
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    const int bj = w, bi = w + d;
    if (bi < 4) {
      float* t1 = t1all[w];
      // T1 = sum_m A[bi][m] X[m][bj]; lane: rows 4lq + ii, column ln
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int r = 4 * lq + ii;
        float acc = 0.f;
        for (int m = bj; m < bi; ++m)
#pragma unroll
          for (int x = 0; x < 16; ++x)
            acc += A[(16 * bi + r) * kLM + 16 * m + x] * X[(16 * m + x) * kLM + 16 * bj + ln];
        t1[r * 17 + ln] = acc;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int r = 4 * lq + ii;
        float acc = 0.f;
#pragma unroll
        for (int x = 0; x < 16; ++x) acc += X[(16 * bi + r) * kLM + 16 * bi + x] * t1[x * 17 + ln];
        X[(16 * bi + r) * kLM + 16 * bj + ln] = -acc;
      }
    }
    __syncthreads();
  }
}

// In-place l2 normalisation of the 64 rows of a staged bf16 tile [64][LD] with
// N columns: x <- x * scale / sqrt(||x||^2 + eps), eps = 1e-6 (fla's l2norm,
// used at kernel.py:20-23, 110-111), over fp32 sums.  Threads T0 .. T0 + 255
// take part, four per row (consecutive lanes); rinv (if not null) receives
// 1 / sqrt(||x||^2 + eps) of each row, for the backward's chain rule.
template <int N, int LD, int T0 = 0>
__device__ __forceinline__ void l2norm_rows(__bf16* X, float scale, float* rinv) {
  constexpr int PER = N / 4, NU = PER / 8;   // columns per thread, 16-byte units
  const int t = (int)threadIdx.x - T0, r = t >> 2, part = t & 3;
  __bf16* row = X + r * LD + part * PER;
  float ss = 0.f;
  bf16x8 u[NU];
#pragma unroll
  for (int j = 0; j < NU; ++j) {
    u[j] = *(const bf16x8*)(row + 8 * j);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (float)u[j][i] * (float)u[j][i];
  }
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  const float ri = __builtin_amdgcn_rsqf(ss + 1e-6f);
  const float f = ri * scale;
#pragma unroll
  for (int j = 0; j < NU; ++j) {
    bf16x8 y;
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = (__bf16)((float)u[j][i] * f);
    *(bf16x8*)(row + 8 * j) = y;
  }
  if (rinv != nullptr && part == 0) rinv[r] = ri;
}

}  // namespace hattn
