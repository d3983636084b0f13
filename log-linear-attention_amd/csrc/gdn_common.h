// Shared pieces of the log-linear Gated DeltaNet kernels (forward and backward).
#pragma once
#include "common.h"

namespace hattn {

constexpr int kGC = 64;       // chunk length
constexpr int kLd64 = 72;     // LDS row stride of 64-wide bf16 tiles
constexpr int kGMaxLev = 8;   // inter-chunk levels of the forward scan (T <= 64 * 2^8)
constexpr int kGBwdMaxLev = 8;   // inter-chunk levels of the backward scan (T <= 64 * 2^8)
constexpr int kBVs = 32;      // V columns per backward-scan workgroup
constexpr int kLM = 65;       // row stride of 64 x 64 fp32 LDS matrices

// HType.STRONG intra-chunk levels: the reference's chunkwise GDN path takes
// lambda of a pair inside a chunk at its strong level (make_levels_matrix with
// htype STRONG, chunkwise_hgdn.py:630), which on an aligned 64-token chunk is
// the strong function of the chunk-local positions; [t][s], 0 on and above
// the diagonal.
struct alignas(16) GdnStrongIntra {
  unsigned char lv[kGC * kGC];
  constexpr GdnStrongIntra() : lv() {
    for (int a = 0; a < kGC; ++a)
      for (int b = 0; b < kGC; ++b) lv[a * kGC + b] = (unsigned char)(b < a ? strong_level_ce(a, b) : 0);
  }
};
__device__ constexpr GdnStrongIntra kGdnStrongIntra{};

// Level of the pair (t, s) of one chunk (chunk-local, s <= t): the weak closed
// form, or the strong table (a cached global byte read; only the STRONG
// instantiations read it).
template <bool STRONG>
__device__ __forceinline__ int gdn_intra_level(int t, int s) {
  if constexpr (STRONG)
    return kGdnStrongIntra.lv[t * kGC + s];
  else
    return intra_level(t, s);
}

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
__device__ __forceinline__ void tri_inv64(const float* A, float* X, float (*t1all)[16 * 17]) {
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

// ---------------------------------------------------------------------------
// X = (I + A)^-1 on fp32 MFMA (v_mfma_f32_16x16x4_f32: exact fp32 products,
// fp32 accumulation) for a strictly lower-triangular 64 x 64 fp32 A.
//   Diagonal 16 x 16 blocks, N = A_ii nilpotent (N^16 = 0):
//     (I + N)^-1 = sum_{k < 16} (-N)^k = (I - N)(I + N^2)(I + N^4)(I + N^8)
//   (the factors commute), from N^2, N^4, N^8 and three more products.
//   Off-diagonal blocks by block forward substitution down each block column:
//     X_ij = -X_ii sum_{m=j}^{i-1} A_im X_mj,
//   which only needs X_mj of the same column (wave j) and the diagonal blocks.
// Wave w < 4 owns diagonal block w and block column w; every wave takes part
// in the zero fill of the upper blocks and in the two barriers.  scratch holds
// 3 x 16 x 17 floats per wave (waves 0..3).  Starts and ends with the
// caller's data in LDS and ends with a barrier.
// ---------------------------------------------------------------------------
constexpr int kInvScratchFloats = 4 * 3 * 16 * 17;

// C += L R for 16 x 16 fp32 blocks in LDS (row-major, strides ldl, ldr); C and
// the result in the D layout (lane (lq, ln): rows 4 lq + i, column ln).
__device__ __forceinline__ floatx4 mm16_f32(const float* L, int ldl, const float* R, int ldr,
                                            floatx4 c) {
  const int lane = threadIdx.x & 63, lq = lane >> 4, ln = lane & 15;
  float a[4], b[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    a[s] = L[ln * ldl + 4 * s + lq];     // A_s[m = ln][k = lq] = L[ln][4s + lq]
    b[s] = R[(4 * s + lq) * ldr + ln];   // B_s[k = lq][n = ln] = R[4s + lq][ln]
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], c, 0, 0, 0);
  return c;
}

__device__ __forceinline__ void st16_f32(float* D, int ld, floatx4 d) {
  const int lane = threadIdx.x & 63, lq = lane >> 4, ln = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) D[(4 * lq + i) * ld + ln] = d[i];
}

// LDS writes of this wave visible to its later LDS reads (the wave's LDS
// operations execute in order; the fences keep the compiler from moving them).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <int NTHR>
__device__ __forceinline__ void tri_inv64_mfma(const float* A, float* X, float* scratch) {
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, ln = lane & 15;
  for (int u = tid; u < 6 * 256; u += NTHR) {   // the six upper 16 x 16 blocks
    const int blk = u >> 8, e = u & 255;
    const int bi = blk < 3 ? 0 : (blk < 5 ? 1 : 2);
    const int bj = blk < 3 ? blk + 1 : (blk < 5 ? blk - 1 : 3);
    X[(16 * bi + (e >> 4)) * kLM + 16 * bj + (e & 15)] = 0.f;
  }
  if (w < 4) {
    constexpr int LS = 17;
    float* S0 = scratch + w * 3 * 16 * LS;
    float* S1 = S0 + 16 * LS;
    float* S2 = S1 + 16 * LS;
    const float* N = A + 16 * w * kLM + 16 * w;
    floatx4 p = mm16_f32(N, kLM, N, kLM, zero4());           // N^2
    st16_f32(S0, LS, p);
    wave_lds_sync();
    p = mm16_f32(S0, LS, S0, LS, zero4());                    // N^4
    st16_f32(S1, LS, p);
    wave_lds_sync();
    p = mm16_f32(S1, LS, S1, LS, zero4());                    // N^8
    st16_f32(S2, LS, p);
    wave_lds_sync();
    // R1 = (I - N)(I + N^2) = I - N + N^2 - N N^2
    floatx4 r = mm16_f32(N, kLM, S0, LS, zero4());
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * lq + i;
      r[i] = (row == ln ? 1.f : 0.f) - N[row * kLM + ln] + S0[row * LS + ln] - r[i];
    }
    wave_lds_sync();
    st16_f32(S0, LS, r);
    wave_lds_sync();
    r = mm16_f32(S0, LS, S1, LS, r);                          // R2 = R1 (I + N^4)
    wave_lds_sync();
    st16_f32(S1, LS, r);
    wave_lds_sync();
    r = mm16_f32(S1, LS, S2, LS, r);                          // R3 = R2 (I + N^8)
    st16_f32(X + 16 * w * kLM + 16 * w, kLM, r);
  }
  __syncthreads();
  if (w < 3) {
    constexpr int LS = 17;
    float* S0 = scratch + w * 3 * 16 * LS;
    const int j = w;
    for (int i = j + 1; i < 4; ++i) {
      floatx4 t = zero4();
      for (int m = j; m < i; ++m)
        t = mm16_f32(A + 16 * i * kLM + 16 * m, kLM, X + 16 * m * kLM + 16 * j, kLM, t);
      st16_f32(S0, LS, t);
      wave_lds_sync();
      floatx4 x = mm16_f32(X + 16 * i * kLM + 16 * i, kLM, S0, LS, zero4());
#pragma unroll
      for (int q = 0; q < 4; ++q) x[q] = -x[q];
      wave_lds_sync();
      st16_f32(X + 16 * i * kLM + 16 * j, kLM, x);
      wave_lds_sync();
    }
  }
  __syncthreads();
}

// In-place l2 normalisation of the 64 rows of a staged bf16 tile [64][LD] with
// N columns: x <- bf16(bf16(x / sqrt(||x||^2 + eps)) * scale), eps = 1e-6,
// over fp32 sums: fla's l2norm stores its output in the input dtype and the
// scale multiplies that (l2norm_and_scale_fwd, kernel.py:20-23, 110-111), so
// the value is rounded after the norm and again after the scale (the decode
// step rounds the same way).  Threads T0 .. T0 + 255 take part, four per row
// (consecutive lanes); rinv (if not null) receives 1 / sqrt(||x||^2 + eps) of
// each row, for the backward's chain rule.
// bf16(bf16(x * ri) * scale) of eight values (the stored l2norm output).
// E: the 16-bit format of the stored values (bf16, or fp16 for fp16 inputs).
template <typename E = __bf16>
__device__ __forceinline__ bf16x8 l2norm_scale8(bf16x8 x, float ri, float scale) {
  bf16x8 y;
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = to16<E>(from16<E>(to16<E>(from16<E>(x[i]) * ri)) * scale);
  return y;
}

template <int N, int LD, int T0 = 0, typename E = __bf16>
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
    for (int i = 0; i < 8; ++i) ss += from16<E>(u[j][i]) * from16<E>(u[j][i]);
  }
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  const float ri = __builtin_amdgcn_rsqf(ss + 1e-6f);
#pragma unroll
  for (int j = 0; j < NU; ++j) *(bf16x8*)(row + 8 * j) = l2norm_scale8<E>(u[j], ri, scale);
  if (rinv != nullptr && part == 0) rinv[r] = ri;
}

// 1 / sqrt(||x||^2 + eps) of the 64 rows of a global bf16 tile (row stride
// ld elements, N columns), with the arithmetic of l2norm_rows (same column
// split and sum order, so the same value): four threads per row, rinv[r].
template <int N, typename E = __bf16>
__device__ __forceinline__ void l2norm_rinv_global(const __bf16* X, size_t ld, float* rinv) {
  constexpr int PER = N / 4, NU = PER / 8;
  const int t = (int)threadIdx.x, r = t >> 2, part = t & 3;
  const __bf16* row = X + (size_t)r * ld + part * PER;
  bf16x8 u[NU];
#pragma unroll
  for (int j = 0; j < NU; ++j) u[j] = *(const bf16x8*)(row + 8 * j);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NU; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += from16<E>(u[j][i]) * from16<E>(u[j][i]);
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  if (part == 0) rinv[r] = __builtin_amdgcn_rsqf(ss + 1e-6f);
}

}  // namespace hattn
