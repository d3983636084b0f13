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

// The strong level function for t > s (base.py:49-62 with base 2), for the
// compile-time level tables of the HType.STRONG kernels.
constexpr int strong_level_ce(int t, int s) {
  for (;;) {
    int ell = 0;
    while ((2 << ell) <= t) ++ell;          // floor(log2 t)
    const int v = 1 << (ell > 0 ? ell - 1 : 0);
    const int r = t - (1 << ell);
    if (s < v) return ell + 1;
    if (s < 2 * v && r >= v) return ell + 1;
    if (s < 2 * v) {
      t -= v;
      s -= v;
    } else {
      t -= 2 * v;
      s -= 2 * v;
    }
  }
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

// Workgroup -> (group, head, slice) map for kernels over [group][head] work
// items: all H heads (and their slices) of one group run consecutively on one
// XCD, so the cache lines that interleave the heads of a token row (lambda
// [.., H, L], g [.., H]) are fetched into a single L2 and shared by the heads.
// Groups grp, grp + 8, .. go to XCD grp & 7; the grid has ceil(ngroups / 8) *
// 8 * H * nslices workgroups and a workgroup with grp >= ngroups has no work.
struct XcdHeadMap {
  int grp, h, slice;
};
__device__ __forceinline__ XcdHeadMap xcd_head_map(int wg, int H, int nslices) {
  const int xcd = wg & 7;
  const int r = wg >> 3;
  const int u = r / nslices;
  return XcdHeadMap{(u / H) * 8 + xcd, u % H, r % nslices};
}
__host__ __device__ inline int xcd_head_grid(int ngroups, int H, int nslices) {
  return (ngroups + 7) / 8 * 8 * H * nslices;
}

}  // namespace hattn

namespace hattn {

// Transposed MFMA fragment from a row-major bf16 tile in LDS (gfx950
// ds_read_b64_tr_b16).  Lane layout of the instruction, within each group of
// 16 lanes: lane i receives element (i & 3) of the 8-byte rows addressed by
// lanes 4j + (i >> 2), j = 0..3.  Lane (lq, ln) therefore addresses row
// r0 + 8lq + (ln >> 2), columns c0 + 4(ln & 3) .. +3, and receives
//     X[r0 + 8lq + j][c0 + ln],  j = 0..7   (two reads, rows +0..3 / +4..7),
// which is the A operand of a contraction over the row index (A[m][k] = X[k][m])
// or the B operand B[k][n] = X[k][n].  ld, r0, c0 must keep 8-byte alignment.
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

__device__ __forceinline__ bf16x4 ds_read_tr(const __bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
}

__device__ __forceinline__ bf16x8 tr_frag(const __bf16* X, int ld, int r0, int c0) {
  const int lane = threadIdx.x & 63, lq = lane >> 4, ln = lane & 15;
  const __bf16* p = X + (r0 + 8 * lq + (ln >> 2)) * ld + c0 + 4 * (ln & 3);
  const bf16x4 lo = ds_read_tr(p);
  const bf16x4 hi = ds_read_tr(p + 4 * ld);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Same read with the row order of a D-layout fragment pair: lane (lq, ln)
// receives X[r0 + 4lq + j][c0 + ln] (j = 0..3) and X[r0 + 16 + 4lq + j][c0 + ln],
// the k order {4lq + i, 16 + 4lq + i} in which two stacked 16x16 MFMA D tiles
// hold rows (see the forward kernel's state fragments).
__device__ __forceinline__ bf16x8 tr_frag_d(const __bf16* X, int ld, int r0, int c0) {
  const int lane = threadIdx.x & 63, lq = lane >> 4, ln = lane & 15;
  const __bf16* p = X + (r0 + 4 * lq + (ln >> 2)) * ld + c0 + 4 * (ln & 3);
  const bf16x4 lo = ds_read_tr(p);
  const bf16x4 hi = ds_read_tr(p + 16 * ld);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ bf16x4 cvt4(floatx4 x) {
  return bf16x4{(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]};
}

__device__ __forceinline__ bf16x8 cat8(floatx4 a, floatx4 b) {
  return bf16x8{(__bf16)a[0], (__bf16)a[1], (__bf16)a[2], (__bf16)a[3],
                (__bf16)b[0], (__bf16)b[1], (__bf16)b[2], (__bf16)b[3]};
}

// 16-bit MFMA operand formats.  The kernels move q, k, v, A and states as
// 16-bit patterns held in bf16x8 / bf16x4 registers and LDS tiles whatever
// their format; E (__bf16 or _Float16) selects the conversions to and from
// fp32 and the MFMA opcode (v_mfma_f32_16x16x32_bf16 / _f16), so fp16 inputs
// multiply natively, as the reference's fp16 dots do.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <typename E>
__device__ __forceinline__ floatx4 mfma16(bf16x8 a, bf16x8 b, floatx4 c) {
  if constexpr (sizeof(E) == 2 && __is_same(E, _Float16))
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return mfma16x16x32(a, b, c);
}

// fp32 -> format E, as a 16-bit pattern in a __bf16 slot
template <typename E>
__device__ __forceinline__ __bf16 to16(float x) {
  if constexpr (__is_same(E, _Float16))
    return __builtin_bit_cast(__bf16, (_Float16)x);
  else
    return (__bf16)x;
}

// a 16-bit pattern of format E -> fp32
template <typename E>
__device__ __forceinline__ float from16(__bf16 x) {
  if constexpr (__is_same(E, _Float16))
    return (float)__builtin_bit_cast(_Float16, x);
  else
    return (float)x;
}

template <typename E>
__device__ __forceinline__ bf16x4 cvt4e(floatx4 x) {
  if constexpr (__is_same(E, _Float16))
    return bf16x4{to16<E>(x[0]), to16<E>(x[1]), to16<E>(x[2]), to16<E>(x[3])};
  else
    return cvt4(x);
}

template <typename E>
__device__ __forceinline__ bf16x8 cat8e(floatx4 a, floatx4 b) {
  if constexpr (__is_same(E, _Float16))
    return bf16x8{to16<E>(a[0]), to16<E>(a[1]), to16<E>(a[2]), to16<E>(a[3]),
                  to16<E>(b[0]), to16<E>(b[1]), to16<E>(b[2]), to16<E>(b[3])};
  else
    return cat8(a, b);
}

}  // namespace hattn

namespace hattn {

// Raw buffer access: a 128-bit descriptor in SGPRs holds the (uniform) base
// address and byte range, so a load or store needs one 32-bit VGPR offset plus
// an SGPR offset instead of a 64-bit per-lane address.  Accesses beyond the
// range read zero / are dropped by the hardware.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, size_t bytes) {
  const unsigned int n = bytes > 0xffffffffull ? 0xffffffffu : (unsigned int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(rsrc_t r, unsigned int voff, unsigned int soff) {
  const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return uint4{x[0], x[1], x[2], x[3]};
}

template <typename T> __device__ __forceinline__ T buf_load(rsrc_t r, unsigned int voff, unsigned int soff);
template <> __device__ __forceinline__ float buf_load<float>(rsrc_t r, unsigned int voff, unsigned int soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
template <> __device__ __forceinline__ __bf16 buf_load<__bf16>(rsrc_t r, unsigned int voff, unsigned int soff) {
  return __builtin_bit_cast(__bf16, __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0));
}

template <typename T> __device__ __forceinline__ void buf_store(T x, rsrc_t r, unsigned int voff, unsigned int soff);
template <> __device__ __forceinline__ void buf_store<float>(float x, rsrc_t r, unsigned int voff, unsigned int soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, x), r, voff, soff, 0);
}
template <> __device__ __forceinline__ void buf_store<__bf16>(__bf16 x, rsrc_t r, unsigned int voff, unsigned int soff) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, x), r, voff, soff, 0);
}
template <> __device__ __forceinline__ void buf_store<_Float16>(_Float16 x, rsrc_t r, unsigned int voff, unsigned int soff) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, x), r, voff, soff, 0);
}

}  // namespace hattn

namespace hattn {

__device__ __forceinline__ uint2 buf_load8(rsrc_t r, unsigned int voff, unsigned int soff) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
  return uint2{x[0], x[1]};
}

__device__ __forceinline__ void buf_store8(uint2 x, rsrc_t r, unsigned int voff, unsigned int soff) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(u32x2{x.x, x.y}, r, voff, soff, 0);
}

__device__ __forceinline__ void buf_store16(uint4 x, rsrc_t r, unsigned int voff, unsigned int soff) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{x.x, x.y, x.z, x.w}, r, voff, soff, 0);
}

// Four fp32 values stored as T (bf16: one 8-byte store, fp32: one 16-byte store).
template <typename T>
__device__ __forceinline__ void buf_store4(floatx4 x, rsrc_t r, unsigned int voff, unsigned int soff) {
  if constexpr (sizeof(T) == 2) {
    const bf16x4 b = cvt4e<T>(x);
    buf_store8(__builtin_bit_cast(uint2, b), r, voff, soff);
  } else {
    buf_store16(__builtin_bit_cast(uint4, x), r, voff, soff);
  }
}

// DPP move of a float: lanes whose source is outside the row read 0, rows
// outside row_mask keep `old`.
template <int CTRL, int ROW_MASK, bool BOUND_ZERO>
__device__ __forceinline__ float dpp_f32(float old, float src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, src), CTRL,
                                                               ROW_MASK, 0xf, BOUND_ZERO));
}

// Inclusive cumsum of g over the 64 tokens of a chunk (fla chunk_local_cumsum,
// chunkwise.py:1175); lane l holds g[t = l] on entry and Gc[l] on exit.
// Hillis-Steele within each 16-lane row (DPP row_shr 1, 2, 4, 8), then the row
// totals are carried with row_bcast:15 (into rows 1, 3) and row_bcast:31 (into
// rows 2, 3): six VALU ops, no LDS round trips.
__device__ __forceinline__ float chunk_cumsum(float x) {
  x += dpp_f32<0x111, 0xf, true>(0.f, x);   // row_shr:1
  x += dpp_f32<0x112, 0xf, true>(0.f, x);   // row_shr:2
  x += dpp_f32<0x114, 0xf, true>(0.f, x);   // row_shr:4
  x += dpp_f32<0x118, 0xf, true>(0.f, x);   // row_shr:8
  x += dpp_f32<0x142, 0xa, false>(0.f, x);  // row_bcast:15
  x += dpp_f32<0x143, 0xc, false>(0.f, x);  // row_bcast:31
  return x;
}

// Inclusive suffix sum over the 64 lanes (lane l: sum of lanes l .. 63): the
// same Hillis-Steele steps toward lower lanes (row_shl), then each row adds the
// totals of the rows after it (read from lanes 16, 32, 48).
__device__ __forceinline__ float chunk_rsum(float x) {
  x += dpp_f32<0x101, 0xf, true>(0.f, x);   // row_shl:1
  x += dpp_f32<0x102, 0xf, true>(0.f, x);   // row_shl:2
  x += dpp_f32<0x104, 0xf, true>(0.f, x);   // row_shl:4
  x += dpp_f32<0x108, 0xf, true>(0.f, x);   // row_shl:8
  const int xi = __builtin_bit_cast(int, x);
  const float t1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 16));
  const float t2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 32));
  const float t3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 48));
  const int r = (threadIdx.x & 63) >> 4;
  return x + ((r < 3 ? t3 : 0.f) + (r < 2 ? t2 : 0.f) + (r < 1 ? t1 : 0.f));
}

// Sums over the lanes of a DPP quad (4 q .. 4 q + 3) and of a 16-lane row, in
// every lane of the quad / row: quad permutations, then the mirrored half-row
// and row.  VALU only, no LDS round trip.
__device__ __forceinline__ float quad_sum(float x) {
  x += dpp_f32<0xb1, 0xf, false>(0.f, x);   // quad_perm [1, 0, 3, 2]
  x += dpp_f32<0x4e, 0xf, false>(0.f, x);   // quad_perm [2, 3, 0, 1]
  return x;
}
__device__ __forceinline__ float row_sum16(float x) {
  x = quad_sum(x);
  x += dpp_f32<0x141, 0xf, false>(0.f, x);  // row_half_mirror
  x += dpp_f32<0x140, 0xf, false>(0.f, x);  // row_mirror
  return x;
}

// Sum over the four lanes ln, ln + 16, ln + 32, ln + 48 (the lq groups).
__device__ __forceinline__ float sum_lq(float x) {
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}

// Four sum_lq at once, transposed: lane (lq, ln) holds x[m] for m = 0..3 and
// receives sum_lq of x[lq], i.e. the sum over the four 16-lane rows of x[lq],
// in sum_lq's order ((row 0 + row 1) + (row 2 + row 3), each pair added in
// either order).  Three lane exchanges instead of eight.
__device__ __forceinline__ float sum_lq_t(const float (&x)[4], int lq) {
  const bool odd = lq & 1;
  // rows lq and lq ^ 1: keep m = lq & 1 and 2 + (lq & 1), send the other two
  const float a0 = (odd ? x[1] : x[0]) + __shfl_xor(odd ? x[0] : x[1], 16, 64);
  const float a1 = (odd ? x[3] : x[2]) + __shfl_xor(odd ? x[2] : x[3], 16, 64);
  // rows lq and lq ^ 2: keep m = lq, send the other
  const bool hi = lq & 2;
  return (hi ? a1 : a0) + __shfl_xor(hi ? a0 : a1, 32, 64);
}

}  // namespace hattn

namespace hattn {

// bf16x3 products (Henry, Tang & Heinecke 2019, "Leveraging the bfloat16
// artificial intelligence datatype for higher-precision computations"):
// x = hi + lo with hi = bf16(x), lo = bf16(x - hi) carries about 16 mantissa
// bits, and a.b = hi_a.hi_b + hi_a.lo_b + lo_a.hi_b up to the lo_a.lo_b term
// (relative 2^-16), accumulated in fp32 by the MFMA.
__device__ __forceinline__ __bf16 bf16_lo(float x, __bf16 hi) { return (__bf16)(x - (float)hi); }

// Product of fragment planes: NP = 1 (plain bf16) or 2 (hi, lo); the small
// terms are accumulated first.
template <int NP, typename E = __bf16>
__device__ __forceinline__ floatx4 mma(const bf16x8* a, const bf16x8* b, floatx4 c) {
  static_assert(NP == 1 || __is_same(E, __bf16), "bf16x3 splits into bf16 planes");
  if constexpr (NP == 2) {
    c = mfma16x16x32(a[1], b[0], c);
    c = mfma16x16x32(a[0], b[1], c);
  }
  return mfma16<E>(a[0], b[0], c);
}

// fp32 fragment (8 values) -> hi / lo planes.
template <int NP, typename E = __bf16>
__device__ __forceinline__ void split8(const float* x, bf16x8* out) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const __bf16 h = to16<E>(x[j]);
    out[0][j] = h;
    if constexpr (NP == 2) out[1][j] = bf16_lo(x[j], h);
  }
}

// Two D-layout quads -> one B fragment (as cat8), split into NP planes.
template <int NP, typename E = __bf16>
__device__ __forceinline__ void cat8s(floatx4 a, floatx4 b, bf16x8* out) {
  const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  split8<NP, E>(x, out);
}

}  // namespace hattn
