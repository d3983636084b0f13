// Shared device helpers for the gfx950 (CDNA4) log-linear attention kernels.
//
// MFMA fragment conventions used throughout (v_mfma_f32_16x16x32_bf16, one
// 64-wide wavefront, lane = 16 * lq + ln with lq in [0,4), ln in [0,16)):
//   A operand : lane holds A[m = ln][k = 8*lq + j], j = 0..7   (bf16x8)
//   B operand : lane holds B[k = 8*lq + j][n = ln], j = 0..7   (bf16x8)
//   C/D       : lane holds D[m = 4*lq + i][n = ln], i = 0..3   (floatx4)
// Only the pairing "element j of lane group lq of A meets element j of lane
// group lq of B" matters for the contraction, so a kernel may assign any
// bijection k(lq, j) onto the 32 contraction indices as long as it loads both
// operands with the same map.  The kernels use that to feed a D fragment of
// one product straight into the A operand of the next without a transpose.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hattn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma16x16x32(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx4 zero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

// Element conversions used by the loaders / stores.
template <typename T> __device__ __forceinline__ float to_f32(T x);
template <> __device__ __forceinline__ float to_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ float to_f32<__bf16>(__bf16 x) { return (float)x; }
template <> __device__ __forceinline__ float to_f32<_Float16>(_Float16 x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float x) { return (__bf16)x; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }

// exp(x) for x <= 0 (all decays on the path are non-positive log-decays).
__device__ __forceinline__ float fexp(float x) { return __expf(x); }

// Weak Fenwick level of a pair inside one 64-token chunk (t, s chunk-local):
// 0 on the diagonal, bit_length(t ^ s) otherwise (closed form of
// hattention/base.py:41-46, exact for every pair).
__device__ __forceinline__ int intra_level(int t, int s) {
  int x = t ^ s;
  return x == 0 ? 0 : 32 - __clz(x);
}

// Workgroup -> (row, slice) map that keeps the slices of one (batch, head)
// row on one XCD (workgroups are dispatched round-robin over the 8 XCDs), so
// the rows they share (q, k, g, lambda) are fetched into that XCD's L2 once.
struct XcdMap {
  int row, slice;
};
__device__ __forceinline__ XcdMap xcd_map(int wg, int nslices) {
  const int xcd = wg & 7;
  const int r = wg >> 3;
  return XcdMap{(r / nslices) * 8 + xcd, r % nslices};
}

}  // namespace hattn
