// Fused pre- and post-processing of the log-linear Mamba-2 layer scan for gfx950.
//
// Replaces the elementwise torch chain of hmamba_chunk_scan_combined
// (hattention/mamba_apis.py:346-403) around the chunkwise kernels:
//   dt'  = softplus(dt + dt_bias)              (:353-356; softplus threshold 20 as torch)
//   v    = x * dt'                             (:358)
//   g    = A[h] * dt'                          (:359)
//   lam  = compute_lambda(L[h], dl)            (:360-366, mamba_apis.py:70-85)
//          positive: softplus(L dl), bounded: exp(-exp(L) softplus(dl)), None: L dl
//   y    = o + x * D[h]                        (:346-349, :402-403)
// and the backward of that chain (what torch autograd computes through it):
//   dx = dv dt' + dy D,  ddt' = sum_p dv x + dg A,  ddt = ddt' softplus'(dt + dt_bias)
//   dA[h] = sum dg dt',  ddt_bias[h] = sum ddt,  dD[h] = sum dy x,
//   dlam -> ddl and dL[h, l] per lambda mode.
// Every kernel is one pass over its tensors (HBM-bound elementwise work); the
// per-head sums are reduced deterministically (fixed-order partials per
// workgroup, then one ordered sum per head), so repeated runs agree bit for bit.
//
// Rows are (b, t, h) in the time-first layout: x, v, dx [rows, P]; dt, g [rows];
// dl, lam [rows, L].  Element types are runtime flags (bf16 or fp32): the
// kernels are bound by HBM, and a uniform branch per load costs nothing there.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <algorithm>
#include <initializer_list>

#include "common.h"
#include "layer_math.h"

namespace hattn {

namespace {

__device__ __forceinline__ float ld1(const void* p, size_t i, int bf) {
  return bf ? (float)((const __bf16*)p)[i] : ((const float*)p)[i];
}
__device__ __forceinline__ void st1(void* p, size_t i, float x, int bf) {
  if (bf) ((__bf16*)p)[i] = (__bf16)x;
  else ((float*)p)[i] = x;
}
// four consecutive elements starting at a multiple of 4
__device__ __forceinline__ floatx4 ld4(const void* p, size_t i, int bf) {
  if (bf) {
    const bf16x4 a = *(const bf16x4*)((const __bf16*)p + i);
    return floatx4{(float)a[0], (float)a[1], (float)a[2], (float)a[3]};
  }
  return *(const floatx4*)((const float*)p + i);
}
__device__ __forceinline__ void st4(void* p, size_t i, floatx4 x, int bf) {
  if (bf) *(bf16x4*)((__bf16*)p + i) = bf16x4{(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]};
  else *(floatx4*)((float*)p + i) = x;
}

// eight consecutive elements starting at a multiple of 8 (16-byte aligned base)
__device__ __forceinline__ void ld8(const void* p, size_t i, int bf, float* o) {
  if (bf) {
    const bf16x8 a = *(const bf16x8*)((const __bf16*)p + i);
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = (float)a[k];
  } else {
    const floatx4 a = *(const floatx4*)((const float*)p + i);
    const floatx4 b = *(const floatx4*)((const float*)p + i + 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) { o[k] = a[k]; o[4 + k] = b[k]; }
  }
}
__device__ __forceinline__ void st8(void* p, size_t i, const float* x, int bf) {
  if (bf) {
    bf16x8 a;
#pragma unroll
    for (int k = 0; k < 8; ++k) a[k] = (__bf16)x[k];
    *(bf16x8*)((__bf16*)p + i) = a;
  } else {
    *(floatx4*)((float*)p + i) = floatx4{x[0], x[1], x[2], x[3]};
    *(floatx4*)((float*)p + i + 4) = floatx4{x[4], x[5], x[6], x[7]};
  }
}

// Ordered column sums of partial rows: out column c (of ncol) = sum over
// b < nblk of ws[b * stride + c].  Grid ceil(ncol / 64) workgroups of 16
// waves; wave g adds rows g, g + 16, ... in order, then the 16 wave sums are
// added in order, so the result does not depend on timing.
__device__ __forceinline__ float ordered_colsum(const float* __restrict__ ws, long stride,
                                                int nblk, int ncol, int c) {
  __shared__ float part[16][64];
  const int g = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float s0 = 0.f, s1 = 0.f;   // two interleaved chains, added at the end
  if (c < ncol) {
    int b = g;
    for (; b + 16 < nblk; b += 32) {
      s0 += ws[(size_t)b * stride + c];
      s1 += ws[(size_t)(b + 16) * stride + c];
    }
    if (b < nblk) s0 += ws[(size_t)b * stride + c];
  }
  part[g][lane] = s0 + s1;
  __syncthreads();
  float sum = 0.f;
  if (g == 0)
#pragma unroll
    for (int i = 0; i < 16; ++i) sum += part[i][lane];
  return sum;
}

}  // namespace

struct LayerDt {
  int x, dt, dl, lp, v, lam;   // 1 = bf16, 0 = fp32
};

// Blocks [0, nbx): four x elements per thread (v = x dt', and g at the row's
// first quad); blocks [nbx, ..): one lambda element per thread.
__global__ __launch_bounds__(256) void mamba2_layer_prologue_kernel(
    const void* __restrict__ x, const void* __restrict__ dt, const float* __restrict__ A,
    const float* __restrict__ dt_bias, const void* __restrict__ dl, const void* __restrict__ Lp,
    void* __restrict__ v, float* __restrict__ g, void* __restrict__ lam, long rows, int H,
    int P, int L, int softplus, int mode, LayerDt f, int nbx) {
  // 32-bit index arithmetic (the host keeps rows * max(P, L) below 2^31); P is a
  // power of two
  const unsigned int lp = 31 - __builtin_clz((unsigned int)P);
  if ((int)blockIdx.x < nbx) {
    const unsigned int e0 = 4u * (blockIdx.x * 256u + threadIdx.x);
    if (e0 >= (unsigned int)(rows * P)) return;
    const unsigned int r = e0 >> lp;
    const int h = (int)(r % (unsigned int)H);
    const float d = layer_dtp(ld1(dt, r, f.dt), dt_bias ? dt_bias[h] : 0.f, softplus);
    const floatx4 xv = ld4(x, e0, f.x);
    st4(v, e0, floatx4{xv[0] * d, xv[1] * d, xv[2] * d, xv[3] * d}, f.v);
    if (e0 == r * P) g[r] = layer_g(A[h], d);
  } else {
    const unsigned int e = (blockIdx.x - nbx) * 256u + threadIdx.x;
    if (e >= (unsigned int)(rows * L)) return;
    const unsigned int r = e / (unsigned int)L;
    const int l = (int)(e - r * L);
    const int h = (int)(r % (unsigned int)H);
    st1(lam, e, lambda_of(ld1(Lp, (size_t)h * L + l, f.lp), ld1(dl, e, f.dl), mode), f.lam);
  }
}

// Vector form (P % 8 == 0, 16-byte aligned x, v, dl, lam): eight x elements
// per thread in blocks [0, nbx), eight consecutive lambda elements per thread
// after them (the row / level of the first one divided out once, then
// stepped).
__global__ __launch_bounds__(256) void mamba2_layer_prologue_vec_kernel(
    const void* __restrict__ x, const void* __restrict__ dt, const float* __restrict__ A,
    const float* __restrict__ dt_bias, const void* __restrict__ dl, const void* __restrict__ Lp,
    void* __restrict__ v, float* __restrict__ g, void* __restrict__ lam, long rows, int H,
    int P, int L, int softplus, int mode, LayerDt f, int nbx) {
  const unsigned int lp = 31 - __builtin_clz((unsigned int)P);
  if ((int)blockIdx.x < nbx) {
    const unsigned int e0 = 8u * (blockIdx.x * 256u + threadIdx.x);
    if (e0 >= (unsigned int)(rows * P)) return;
    const unsigned int r = e0 >> lp;
    const int h = (int)(r % (unsigned int)H);
    const float d = layer_dtp(ld1(dt, r, f.dt), dt_bias ? dt_bias[h] : 0.f, softplus);
    float xv[8];
    ld8(x, e0, f.x, xv);
#pragma unroll
    for (int c = 0; c < 8; ++c) xv[c] *= d;
    st8(v, e0, xv, f.v);
    if (e0 == r * P) g[r] = layer_g(A[h], d);
  } else {
    const unsigned int n = (unsigned int)(rows * L);
    const unsigned int e0 = 8u * ((blockIdx.x - nbx) * 256u + threadIdx.x);
    if (e0 >= n) return;
    unsigned int r = e0 / (unsigned int)L;
    int l = (int)(e0 - r * L);
    int h = (int)(r % (unsigned int)H);
    if (e0 + 8 <= n) {
      float dv[8];
      ld8(dl, e0, f.dl, dv);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        dv[c] = lambda_of(ld1(Lp, (size_t)h * L + l, f.lp), dv[c], mode);
        if (++l == L) {
          l = 0;
          h = h + 1 == H ? 0 : h + 1;
        }
      }
      st8(lam, e0, dv, f.lam);
    } else {
      for (unsigned int e = e0; e < n; ++e) {
        st1(lam, e, lambda_of(ld1(Lp, (size_t)h * L + l, f.lp), ld1(dl, e, f.dl), mode), f.lam);
        if (++l == L) {
          l = 0;
          h = h + 1 == H ? 0 : h + 1;
        }
      }
    }
  }
}

// out = y + x * D[h], four elements per thread
__global__ __launch_bounds__(256) void mamba2_layer_epilogue_kernel(
    const void* __restrict__ y, const void* __restrict__ x, const float* __restrict__ D,
    void* __restrict__ out, long rows, int H, int P, int ybf, int xbf, int obf) {
  const unsigned int e0 = 4u * (blockIdx.x * 256u + threadIdx.x);
  if (e0 >= (unsigned int)(rows * P)) return;
  const int h = (int)((e0 >> (31 - __builtin_clz((unsigned int)P))) % (unsigned int)H);
  const float d = D[h];
  const floatx4 a = ld4(y, e0, ybf), b = ld4(x, e0, xbf);
  st4(out, e0, floatx4{layer_out(a[0], b[0], d), layer_out(a[1], b[1], d), layer_out(a[2], b[2], d),
                       layer_out(a[3], b[3], d)}, obf);
}

struct LayerBwdDt {
  int x, dt, dl, lp, dy, dv, dlam, dx, ddt, ddl;   // 1 = bf16, 0 = fp32
};

// Backward: grid (nblk, H); workgroup (blk, h) owns the rows bt*H + h for bt in
// its contiguous share of [0, B*T).  A row is handled by tpr = P / 4 threads
// (four elements each, P / 4 a power of two <= 64); lambda entry l of a row is
// handled by its thread l % tpr (NI >= ceil(L / tpr) entries per thread).
// Per-head partials [dA, ddt_bias, dD, dL[0..L)] go to ws[h][blk][3 + L].
template <int NI>
__global__ __launch_bounds__(256) void mamba2_layer_bwd_kernel(
    const void* __restrict__ x, const void* __restrict__ dt, const float* __restrict__ A,
    const float* __restrict__ dt_bias, const void* __restrict__ dl, const void* __restrict__ Lp,
    const float* __restrict__ D, const void* __restrict__ dy, const void* __restrict__ dv,
    const float* __restrict__ dg, const void* __restrict__ dlam, void* __restrict__ dx,
    void* __restrict__ ddt, void* __restrict__ ddl, float* __restrict__ ws, long BT, int H,
    int P, int L, int softplus, int mode, LayerBwdDt f) {
  __shared__ float red[3][256];
  __shared__ float redL[NI * 256];   // [l][ri]: L * rpi <= NI * tpr * rpi = NI * 256
  const int tid = threadIdx.x, h = blockIdx.y, blk = blockIdx.x, nblk = gridDim.x;
  const int tpr = P / 4, rpi = 256 / tpr;
  const int j = tid % tpr, ri = tid / tpr;
  const long per = (BT + nblk - 1) / nblk;
  const long bt0 = (long)blk * per, bt1 = min(BT, bt0 + per);
  const float Ah = A[h], bias = dt_bias ? dt_bias[h] : 0.f, Dh = D ? D[h] : 0.f;
  float accA = 0.f, accB = 0.f, accD = 0.f, accL[NI];   // lambda entries j + i tpr, i < NI
#pragma unroll
  for (int i = 0; i < NI; ++i) accL[i] = 0.f;
  for (long bt = bt0 + ri; bt < bt1; bt += rpi) {
    const long r = bt * H + h;
    const size_t e0 = (size_t)r * P + 4 * j;
    const float pre = ld1(dt, r, f.dt) + bias;
    const float d = softplus ? softplus20(pre) : pre;
    const floatx4 xv = ld4(x, e0, f.x), gv = ld4(dv, e0, f.dv);
    floatx4 yv = floatx4{0.f, 0.f, 0.f, 0.f};
    if (D) yv = ld4(dy, e0, f.dy);
    st4(dx, e0, floatx4{gv[0] * d + yv[0] * Dh, gv[1] * d + yv[1] * Dh, gv[2] * d + yv[2] * Dh,
                        gv[3] * d + yv[3] * Dh}, f.dx);
    float s = gv[0] * xv[0] + gv[1] * xv[1] + gv[2] * xv[2] + gv[3] * xv[3];
    accD += yv[0] * xv[0] + yv[1] * xv[1] + yv[2] * xv[2] + yv[3] * xv[3];
    // sum over the row's tpr lanes (consecutive lanes of one wave)
    for (int m = 1; m < tpr; m <<= 1) s += __shfl_xor(s, m, 64);
    if (j == 0) {
      const float dgr = dg[r];
      const float ddtv = s + dgr * Ah;
      const float dd = softplus ? ddtv * dsoftplus20(pre) : ddtv;
      st1(ddt, r, dd, f.ddt);
      accA += dgr * d;
      accB += dd;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int l = j + i * tpr;
      if (l < L) {
        const size_t el = (size_t)r * L + l;
        const float dlv = ld1(dl, el, f.dl), gl = ld1(dlam, el, f.dlam);
        const float Lv = ld1(Lp, (size_t)h * L + l, f.lp);
        float gdl, gL;
        if (mode == kLamPositive) {
          const float u = gl * dsoftplus20(Lv * dlv);   // d lam / d (L dl)
          gdl = u * Lv;
          gL = u * dlv;
        } else if (mode == kLamBounded) {
          const float eL = __expf(Lv), sp = softplus20(dlv);
          const float lamv = __expf(-eL * sp);
          gL = gl * lamv * (-eL * sp);
          gdl = gl * lamv * (-eL) * dsoftplus20(dlv);
        } else {
          gdl = gl * Lv;
          gL = gl * dlv;
        }
        st1(ddl, el, gdl, f.ddl);
        accL[i] += gL;
      }
    }
  }
  // fixed-order reduction of the workgroup's partials
  red[0][tid] = accA;
  red[1][tid] = accB;
  red[2][tid] = accD;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int l = j + i * tpr;
    if (l < L) redL[l * rpi + ri] = accL[i];   // slot ri of level l (rpi slots per level)
  }
  __syncthreads();
  const int nq = 3 + L;
  if (tid < nq) {
    const float* src = tid < 3 ? red[tid] : redL + (tid - 3) * rpi;
    const int n = tid < 3 ? 256 : rpi;
    float sum = 0.f;
    for (int i = 0; i < n; ++i) sum += src[i];
    ws[((size_t)h * nblk + blk) * nq + tid] = sum;
  }
}

// Per-head sums over the workgroups, in a fixed order; grid H.
// Vector form of the backward (P % 8 == 0, H P / 8 dividing 256, 3 H <= 256, H L <= 1024,
// 16-byte aligned x, dv, dy, dx): workgroup blk owns a contiguous share of the
// B T token rows, all heads.  x part: thread tid handles the eight elements
// 8 (tid % tpb) .. + 7 of rows bt = slot, slot + rpi, ... (tpb = H P / 8
// threads per row, rpi = 256 / tpb rows at a time), so its head is fixed; a
// (row, head) is summed over its P / 8 consecutive lanes.  lambda part:
// thread tid handles offsets tid + 256 k of every row's H L entries, so each
// (head, level) has one owner and dL needs no reduction in the workgroup.
// Partials go to ws[h][blk][3 + L] like the per-head kernel's.
template <int NL>
__global__ __launch_bounds__(256) void mamba2_layer_bwd_vec_kernel(
    const void* __restrict__ x, const void* __restrict__ dt, const float* __restrict__ A,
    const float* __restrict__ dt_bias, const void* __restrict__ dl, const void* __restrict__ Lp,
    const float* __restrict__ D, const void* __restrict__ dy, const void* __restrict__ dv,
    const float* __restrict__ dg, const void* __restrict__ dlam, void* __restrict__ dx,
    void* __restrict__ ddt, void* __restrict__ ddl, float* __restrict__ ws, long BT, int H,
    int P, int L, int softplus, int mode, LayerBwdDt f) {
  __shared__ float red[3][256];
  const int tid = threadIdx.x, blk = blockIdx.x, nblk = gridDim.x;
  const int HP = H * P, tpb = HP / 8, rpi = 256 / tpb, gl = P / 8;
  const int slot = tid / tpb, col = (tid % tpb) * 8, h = col / P, j = (col % P) / 8;
  const long per = (BT + nblk - 1) / nblk;
  const long bt0 = (long)blk * per, bt1 = min(BT, bt0 + per);
  const float Ah = A[h], bias = dt_bias ? dt_bias[h] : 0.f, Dh = D ? D[h] : 0.f;
  float accA = 0.f, accB = 0.f, accD = 0.f;
  for (long bt = bt0 + slot; bt < bt1; bt += rpi) {
    const long r = bt * H + h;
    const size_t e0 = (size_t)bt * HP + col;
    const float pre = ld1(dt, r, f.dt) + bias;
    const float d = softplus ? softplus20(pre) : pre;
    float xv[8], gv[8], yv[8], o[8];
    ld8(x, e0, f.x, xv);
    ld8(dv, e0, f.dv, gv);
    if (D) ld8(dy, e0, f.dy, yv);
    else
#pragma unroll
      for (int c = 0; c < 8; ++c) yv[c] = 0.f;
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      o[c] = gv[c] * d + yv[c] * Dh;
      s += gv[c] * xv[c];
      accD += yv[c] * xv[c];
    }
    st8(dx, e0, o, f.dx);
    for (int m = 1; m < gl; m <<= 1) s += __shfl_xor(s, m, 64);
    if (j == 0) {
      const float dgr = dg[r];
      const float ddtv = s + dgr * Ah;
      const float dd = softplus ? ddtv * dsoftplus20(pre) : ddtv;
      st1(ddt, r, dd, f.ddt);
      accA += dgr * d;
      accB += dd;
    }
  }
  // lambda entries: fixed (head, level) per thread and k
  const int HL = H * L;
  float accL[NL], Lv[NL];
  int lk[NL];
#pragma unroll
  for (int k = 0; k < NL; ++k) {
    const int oq = tid + 256 * k;
    accL[k] = 0.f;
    lk[k] = oq < HL ? oq % L : 0;
    Lv[k] = oq < HL ? ld1(Lp, oq, f.lp) : 0.f;   // Lp [H, L] row-major: offset oq
  }
#pragma unroll 4
  for (long bt = bt0; bt < bt1; ++bt) {
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const int oq = tid + 256 * k;
      if (oq < HL) {
        const size_t el = (size_t)bt * HL + oq;
        const float dlv = ld1(dl, el, f.dl), gq = ld1(dlam, el, f.dlam);
        float gdl, gL;
        if (mode == kLamPositive) {
          const float u = gq * dsoftplus20(Lv[k] * dlv);
          gdl = u * Lv[k];
          gL = u * dlv;
        } else if (mode == kLamBounded) {
          const float eL = __expf(Lv[k]), sp = softplus20(dlv);
          const float lamv = __expf(-eL * sp);
          gL = gq * lamv * (-eL * sp);
          gdl = gq * lamv * (-eL) * dsoftplus20(dlv);
        } else {
          gdl = gq * Lv[k];
          gL = gq * dlv;
        }
        st1(ddl, el, gdl, f.ddl);
        accL[k] += gL;
      }
    }
  }
  // dD: sum over the (row, head) group's lanes, then everything per head over
  // the rpi row slots in order
  for (int m = 1; m < gl; m <<= 1) accD += __shfl_xor(accD, m, 64);
  if (j == 0) {
    red[0][slot * H + h] = accA;
    red[1][slot * H + h] = accB;
    red[2][slot * H + h] = accD;
  }
  __syncthreads();
  const int nq = 3 + L;
  if (tid < 3 * H) {
    const int q = tid / H, hh = tid % H;
    float sum = 0.f;
    for (int sl = 0; sl < rpi; ++sl) sum += red[q][sl * H + hh];
    ws[((size_t)hh * nblk + blk) * nq + q] = sum;
  }
#pragma unroll
  for (int k = 0; k < NL; ++k) {
    const int oq = tid + 256 * k;
    if (oq < HL) ws[((size_t)(oq / L) * nblk + blk) * nq + 3 + lk[k]] = accL[k];
  }
}

__global__ __launch_bounds__(1024) void mamba2_layer_bwd_reduce_kernel(
    const float* __restrict__ ws, float* __restrict__ dA, float* __restrict__ ddt_bias,
    float* __restrict__ dD, float* __restrict__ dLp, int nblk, int L) {
  const int h = blockIdx.x, q = threadIdx.x & 63, nq = 3 + L;
  const float sum = ordered_colsum(ws + (size_t)h * nblk * nq, nq, nblk, nq, q);
  if (threadIdx.x >= 64 || q >= nq) return;
  if (q == 0) { if (dA) dA[h] = sum; }
  else if (q == 1) { if (ddt_bias) ddt_bias[h] = sum; }
  else if (q == 2) { if (dD) dD[h] = sum; }
  else if (dLp) dLp[(size_t)h * L + (q - 3)] = sum;
}

}  // namespace hattn

namespace {
int layer_bwd_nblk(long BT, int H) {
  // about 2048 workgroups in all, at least 8 rows each
  long n = 2048 / (H > 0 ? H : 1);
  if (n < 1) n = 1;
  const long cap = (BT + 7) / 8;
  if (n > cap) n = cap;
  return (int)(n < 1 ? 1 : n);
}
}  // namespace

// workgroups of the vector backward: about 1024, at least 16 rows each
int layer_bwd_vec_nblk(long BT) {
  long n = (BT + 15) / 16;
  if (n > 1024) n = 1024;
  return (int)(n < 1 ? 1 : n);
}
size_t hattn_mamba2_layer_bwd_ws_bytes(int B, int T, int H, int L) {
  const long BT = (long)B * T;
  const long nblk = std::max<long>(layer_bwd_nblk(BT, H), layer_bwd_vec_nblk(BT));
  return (size_t)H * nblk * (3 + L) * sizeof(float);
}

hipError_t hattn_mamba2_layer_prologue_launch(const void* x, const void* dt, const float* A,
                                              const float* dt_bias, const void* dl,
                                              const void* Lp, void* v, float* g, void* lam,
                                              int B, int T, int H, int P, int L, int softplus,
                                              int mode, const int* bf, hipStream_t stream) {
  using namespace hattn;
  const long rows = (long)B * T * H;
  const LayerDt f{bf[0], bf[1], bf[2], bf[3], bf[4], bf[5]};
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (P % 8 == 0 && a16(x) && a16(v) && a16(dl) && a16(lam)) {
    const long nx = (rows * P / 8 + 255) / 256, nl = ((rows * L + 7) / 8 + 255) / 256;
    hipLaunchKernelGGL(mamba2_layer_prologue_vec_kernel, dim3((unsigned)(nx + nl)), dim3(256), 0,
                       stream, x, dt, A, dt_bias, dl, Lp, v, g, lam, rows, H, P, L, softplus,
                       mode, f, (int)nx);
    return hipGetLastError();
  }
  const long nx = (rows * P / 4 + 255) / 256, nl = (rows * L + 255) / 256;
  hipLaunchKernelGGL(mamba2_layer_prologue_kernel, dim3((unsigned)(nx + nl)), dim3(256), 0, stream,
                     x, dt, A, dt_bias, dl, Lp, v, g, lam, rows, H, P, L, softplus, mode, f,
                     (int)nx);
  return hipGetLastError();
}

hipError_t hattn_mamba2_layer_epilogue_launch(const void* y, const void* x, const float* D,
                                              void* out, int B, int T, int H, int P, int ybf,
                                              int xbf, int obf, hipStream_t stream) {
  using namespace hattn;
  const long rows = (long)B * T * H;
  const long n = (rows * P / 4 + 255) / 256;
  hipLaunchKernelGGL(mamba2_layer_epilogue_kernel, dim3((unsigned)n), dim3(256), 0, stream, y, x,
                     D, out, rows, H, P, ybf, xbf, obf);
  return hipGetLastError();
}

hipError_t hattn_mamba2_layer_bwd_launch(const void* x, const void* dt, const float* A,
                                         const float* dt_bias, const void* dl, const void* Lp,
                                         const float* D, const void* dy, const void* dv,
                                         const float* dg, const void* dlam, void* dx, void* ddt,
                                         void* ddl, float* dA, float* ddt_bias, float* dD,
                                         float* dLp, float* ws, int B, int T, int H, int P, int L,
                                         int softplus, int mode, const int* bf,
                                         hipStream_t stream) {
  using namespace hattn;
  const long BT = (long)B * T;
  const LayerBwdDt f{bf[0], bf[1], bf[2], bf[3], bf[4], bf[5], bf[6], bf[7], bf[8], bf[9]};
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int tpb = H * P / 8;
  if (P % 8 == 0 && tpb <= 256 && 256 % tpb == 0 && 3 * H <= 256 && H * L <= 4 * 256 && a16(x) &&
      a16(dv) && (D == nullptr || a16(dy)) && a16(dx)) {
    const int vblk = layer_bwd_vec_nblk(BT), nl = (H * L + 255) / 256;
#define LAYER_BWD_VEC(NL_)                                                                      \
  hipLaunchKernelGGL((mamba2_layer_bwd_vec_kernel<NL_>), dim3(vblk), dim3(256), 0, stream, x,   \
                     dt, A, dt_bias, dl, Lp, D, dy, dv, dg, dlam, dx, ddt, ddl, ws, BT, H, P, L, \
                     softplus, mode, f)
    if (nl <= 1) LAYER_BWD_VEC(1);
    else if (nl <= 2) LAYER_BWD_VEC(2);
    else LAYER_BWD_VEC(4);
#undef LAYER_BWD_VEC
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(mamba2_layer_bwd_reduce_kernel, dim3(H), dim3(1024), 0, stream, ws, dA,
                       ddt_bias, dD, dLp, vblk, L);
    return hipGetLastError();
  }
  const int nblk = layer_bwd_nblk(BT, H);
  const int tpr = P / 4, ni = (L + tpr - 1) / tpr;   // lambda entries per thread
#define LAYER_BWD(NI_)                                                                         \
  hipLaunchKernelGGL((mamba2_layer_bwd_kernel<NI_>), dim3(nblk, H), dim3(256), 0, stream, x,   \
                     dt, A, dt_bias, dl, Lp, D, dy, dv, dg, dlam, dx, ddt, ddl, ws, BT, H, P, L, \
                     softplus, mode, f)
  if (ni <= 1) LAYER_BWD(1);
  else if (ni <= 2) LAYER_BWD(2);
  else if (ni <= 4) LAYER_BWD(4);
  else if (ni <= 8) LAYER_BWD(8);
  else LAYER_BWD(32);
#undef LAYER_BWD
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mamba2_layer_bwd_reduce_kernel, dim3(H), dim3(1024), 0, stream, ws, dA,
                     ddt_bias, dD, dLp, nblk, L);
  return hipGetLastError();
}

// ===========================================================================
// hmamba_split_conv1d_scan_combined (hattention/mamba_apis.py:116-260): the
// depthwise causal conv1d + SiLU of the xBC channels (causal_conv1d_fn, :206-213)
// and the gated RMSNorm of the scan output (rmsnorm_fn with z and
// norm_before_gate=False, :247-255), forward and backward.
//   conv:  pre[b,s,d] = bias[d] + sum_{w<W} weight[d,w] in[b, s-(W-1)+w, d]
//          (zero for negative positions), out = pre * sigmoid(pre)
//   norm:  u = y * silu(z), r = (mean_j u_j^2 + eps)^-1/2, out = u r weight
// The conv input is a column window of the packed zxbcdtdl rows (row stride
// `ld`); its output is written as three contiguous tensors x, B, C.
// ===========================================================================
namespace hattn {

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }
__device__ __forceinline__ float dsilu_f(float x) {
  const float s = 1.f / (1.f + expf(-x));
  return s * (1.f + x * (1.f - s));
}

// grid (B * S, ceil(Dc / 256)): one thread per (b, s, d), d fastest; the
// kernel width W (1..8) is a template argument
template <int W>
__global__ __launch_bounds__(256) void conv1d_silu_fwd_kernel(
    const void* __restrict__ in, long ld, long col0, const void* __restrict__ wt,
    const void* __restrict__ bias, void* __restrict__ o0, void* __restrict__ o1,
    void* __restrict__ o2, long BS, int S, int Dc, int d1, int d2, int fin, int fw, int fo) {
  const long bs = blockIdx.x;
  const int d = blockIdx.y * 256 + threadIdx.x;
  if (d >= Dc) return;
  const int s = (int)(blockIdx.x % (unsigned int)S);
  float xv[W], wv[W];
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const int sp = s - (W - 1) + w;
    wv[w] = ld1(wt, (size_t)d * W + w, fw);
    xv[w] = sp >= 0 ? ld1(in, (size_t)(bs - s + sp) * ld + col0 + d, fin) : 0.f;
  }
  float acc = bias ? ld1(bias, d, fw) : 0.f;
#pragma unroll
  for (int w = 0; w < W; ++w) acc += wv[w] * xv[w];
  const float y = silu_f(acc);
  if (d < d1) st1(o0, (size_t)bs * d1 + d, y, fo);
  else if (d < d2) st1(o1, (size_t)bs * (d2 - d1) + (d - d1), y, fo);
  else st1(o2, (size_t)bs * (Dc - d2) + (d - d2), y, fo);
}

// Vector form for bf16 input rows: each thread owns 8 consecutive channels
// (16-byte loads and stores, consecutive lanes on consecutive channel groups)
// and a run of kConvRun tokens of one sequence; the W - 1 input rows before the
// current one stay in registers, so every input element is loaded once per
// run (plus W - 1 halo rows).  Requires Dc, d1, d2, ld, col0 multiples of 8
// and 16-byte aligned bases (checked by the host).
constexpr int kConvRun = 32;

template <int W>
__global__ __launch_bounds__(256) void conv1d_silu_fwd_vec_kernel(
    const __bf16* __restrict__ in, long ld, long col0, const void* __restrict__ wt,
    const void* __restrict__ bias, void* __restrict__ o0, void* __restrict__ o1,
    void* __restrict__ o2, int B, int S, int Dc, int d1, int d2, int fw, int fo) {
  const int ng = Dc / 8;
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  const int cgp = (int)(gid % ng);
  const long run = gid / ng;
  const int nrun = (S + kConvRun - 1) / kConvRun;
  if (run >= (long)B * nrun) return;
  const int b = (int)(run / nrun), s0 = (int)(run % nrun) * kConvRun;
  const int s1 = min(s0 + kConvRun, S);
  const int d = 8 * cgp;
  float wv[8][W], bv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    bv[c] = bias ? ld1(bias, d + c, fw) : 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) wv[c][w] = ld1(wt, (size_t)(d + c) * W + w, fw);
  }
  // output tensor and row stride of this channel group
  void* ob = d < d1 ? o0 : (d < d2 ? o1 : o2);
  const int on = d < d1 ? d1 : (d < d2 ? d2 - d1 : Dc - d2);
  const int oc = d < d1 ? d : (d < d2 ? d - d1 : d - d2);
  const __bf16* src = in + (size_t)b * S * ld + col0 + d;
  auto cvt = [](const bf16x8& u, float (&x)[8]) {
#pragma unroll
    for (int c = 0; c < 8; ++c) x[c] = (float)u[c];
  };
  float win[W][8];   // rows s - (W - 1) .. s
#pragma unroll
  for (int w = 0; w < W - 1; ++w) {
    const int sp = s0 - (W - 1) + w;
    const bf16x8 u = sp >= 0 ? *(const bf16x8*)(src + (size_t)sp * ld) : bf16x8{};
    cvt(u, win[w]);
  }
  // rows in blocks of kConvBlk: the next block's loads are issued before the
  // current block is computed, so each has a block's work to land
  constexpr int kConvBlk = 8;
  bf16x8 nxt[kConvBlk];
  auto issue = [&](int sb) {
#pragma unroll
    for (int r = 0; r < kConvBlk; ++r)
      nxt[r] = sb + r < s1 ? *(const bf16x8*)(src + (size_t)(sb + r) * ld) : bf16x8{};
  };
  issue(s0);
  for (int sb = s0; sb < s1; sb += kConvBlk) {
    bf16x8 cur[kConvBlk];
#pragma unroll
    for (int r = 0; r < kConvBlk; ++r) cur[r] = nxt[r];
    if (sb + kConvBlk < s1) issue(sb + kConvBlk);
#pragma unroll
    for (int r = 0; r < kConvBlk; ++r) {
      const int s = sb + r;
      if (s < s1) {
        cvt(cur[r], win[W - 1]);
        float y[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float acc = bv[c];
#pragma unroll
          for (int w = 0; w < W; ++w) acc += wv[c][w] * win[w][c];
          y[c] = silu_f(acc);
        }
        const size_t oi = ((size_t)b * S + s) * on + oc;
        if (fo) {
          bf16x8 o;
#pragma unroll
          for (int c = 0; c < 8; ++c) o[c] = (__bf16)y[c];
          *(bf16x8*)((__bf16*)ob + oi) = o;
        } else {
          *(floatx4*)((float*)ob + oi) = floatx4{y[0], y[1], y[2], y[3]};
          *(floatx4*)((float*)ob + oi + 4) = floatx4{y[4], y[5], y[6], y[7]};
        }
#pragma unroll
        for (int w = 0; w < W - 1; ++w)
#pragma unroll
          for (int c = 0; c < 8; ++c) win[w][c] = win[w + 1][c];
      }
    }
  }
}

// Backward of the conv + SiLU.  Grid (Dc / 64, nblk): workgroup (cg, blk)
// owns channels 64 cg .. + 63 and the 64-token tiles blk, blk + nblk, ... of
// the flattened (b, s-tile) index.  Per tile it stages the input rows the
// tile needs, forms dpre = dout * silu'(pre) for the tile and the W - 1 rows
// after it, writes din and accumulates dweight / dbias partials, which go to
// ws[blk][64 cg + c][W + 1] and are summed in order afterwards.
constexpr int kConvTile = 64;

template <int W>
__global__ __launch_bounds__(256) void conv1d_silu_bwd_kernel(
    const void* __restrict__ in, long ld, long col0, const void* __restrict__ wt,
    const void* __restrict__ bias, const void* __restrict__ g0, const void* __restrict__ g1,
    const void* __restrict__ g2, void* __restrict__ din, long ldo, long colo,
    float* __restrict__ ws, int B, int S, int Dc, int d1, int d2, int fin, int fw,
    int fg0, int fg1, int fg2, int fdi) {
  constexpr int NX = kConvTile + 2 * (W - 1);   // staged input rows s0-(W-1) .. s0+63+(W-1)
  constexpr int NP = kConvTile + W - 1;         // dpre rows s0 .. s0+63+(W-1)
  __shared__ float xs[NX][64];
  __shared__ float dp[NP][64];
  __shared__ float red[4][64][W + 1];
  const int tid = threadIdx.x, c = tid & 63, sr = tid >> 6;
  const int cg = blockIdx.x, blk = blockIdx.y, nblk = gridDim.y;
  const int d = 64 * cg + c;
  const bool dok = d < Dc;
  const int ntile_s = (S + kConvTile - 1) / kConvTile;
  const long ntiles = (long)B * ntile_s;
  float wv[W];
#pragma unroll
  for (int w = 0; w < W; ++w) wv[w] = dok ? ld1(wt, (size_t)d * W + w, fw) : 0.f;
  const float bv = (dok && bias) ? ld1(bias, d, fw) : 0.f;
  float accw[W], accb = 0.f;
#pragma unroll
  for (int w = 0; w < W; ++w) accw[w] = 0.f;
  auto gout = [&](long bs) -> float {
    if (d < d1) return ld1(g0, (size_t)bs * d1 + d, fg0);
    if (d < d2) return ld1(g1, (size_t)bs * (d2 - d1) + (d - d1), fg1);
    return ld1(g2, (size_t)bs * (Dc - d2) + (d - d2), fg2);
  };
  // fixed trip counts (row sr + 4 i) so that each phase's loads issue together
  for (long tile = blk; tile < ntiles; tile += nblk) {
    const int b = (int)(tile / ntile_s), s0 = (int)(tile % ntile_s) * kConvTile;
    const long base = (long)b * S;
    float xr[(NX + 3) / 4];
#pragma unroll
    for (int i = 0; i < (NX + 3) / 4; ++i) {
      const int r = sr + 4 * i, sp = s0 - (W - 1) + r;
      xr[i] = (r < NX && dok && sp >= 0 && sp < S) ? ld1(in, (size_t)(base + sp) * ld + col0 + d, fin) : 0.f;
    }
    float gr[(NP + 3) / 4];
#pragma unroll
    for (int i = 0; i < (NP + 3) / 4; ++i) {
      const int r = sr + 4 * i, sp = s0 + r;
      gr[i] = (r < NP && dok && sp < S) ? gout(base + sp) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < (NX + 3) / 4; ++i)
      if (sr + 4 * i < NX) xs[sr + 4 * i][c] = xr[i];
    __syncthreads();
    // dpre = dout * silu'(pre) (zero beyond the sequence: gr is zero there)
#pragma unroll
    for (int i = 0; i < (NP + 3) / 4; ++i) {
      const int r = sr + 4 * i;
      if (r < NP) {
        float pre = bv;
#pragma unroll
        for (int w = 0; w < W; ++w) pre += wv[w] * xs[r + w][c];   // xs row r + w is s0 + r - (W-1) + w
        dp[r][c] = s0 + r < S ? gr[i] * dsilu_f(pre) : 0.f;
      }
    }
    __syncthreads();
    // din and the weight / bias partials for rows s0 .. s0 + 63
#pragma unroll
    for (int i = 0; i < kConvTile / 4; ++i) {
      const int r = sr + 4 * i, sp = s0 + r;
      if (dok && sp < S) {
        float gi = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) gi += wv[w] * dp[r + (W - 1) - w][c];   // out row sp + W-1-w
        st1(din, (size_t)(base + sp) * ldo + colo + d, gi, fdi);
        const float dpr = dp[r][c];
        accb += dpr;
#pragma unroll
        for (int w = 0; w < W; ++w) accw[w] += dpr * xs[r + w][c];        // input row sp-(W-1)+w
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int w = 0; w < W; ++w) red[sr][c][w] = accw[w];
  red[sr][c][W] = accb;
  __syncthreads();
  if (sr == 0 && dok) {
    float* out = ws + ((size_t)blk * Dc + d) * (W + 1);
#pragma unroll
    for (int w = 0; w <= W; ++w) out[w] = red[0][c][w] + red[1][c][w] + red[2][c][w] + red[3][c][w];
  }
}


// Vector form of the backward for bf16 rows (input, output gradients and din):
// each thread owns 8 consecutive channels and a run of kConvRun tokens; the
// W - 1 input rows and dpre values before the current row stay in registers,
// so one pass over rows s0 .. s0 + kConvRun + W - 2 yields dpre, din for the
// run and the weight / bias partials.  Workgroup (cb, rb): channel groups
// 16 cb + (tid & 15) and runs 16 rb + (tid >> 4) of the flattened (b, run)
// index; the partials of its 16 runs are summed in a fixed order (lane
// shuffles, then the four waves) into ws[rb][d][W + 1].
constexpr int kConvBwdRuns = 16;

template <int W>
__global__ __launch_bounds__(256) void conv1d_silu_bwd_vec_kernel(
    const __bf16* __restrict__ in, long ld, long col0, const void* __restrict__ wt,
    const void* __restrict__ bias, const __bf16* __restrict__ g0,
    const __bf16* __restrict__ g1, const __bf16* __restrict__ g2, __bf16* __restrict__ din,
    long ldo, long colo, float* __restrict__ ws, int B, int S, int Dc, int d1, int d2,
    int fw) {
  __shared__ float red[4][16][8][W + 1];
  const int tid = threadIdx.x, cl = tid & 15, rl = tid >> 4;
  const int ng = Dc / 8, nrun = (S + kConvRun - 1) / kConvRun;
  const int cg = blockIdx.x * 16 + cl;
  const long run = (long)blockIdx.y * kConvBwdRuns + rl;
  const bool ok = cg < ng && run < (long)B * nrun;
  const int d = 8 * min(cg, ng - 1);
  float wv[8][W], bv[8], accw[8][W], accb[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    bv[c] = bias ? ld1(bias, d + c, fw) : 0.f;
    accb[c] = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      wv[c][w] = ld1(wt, (size_t)(d + c) * W + w, fw);
      accw[c][w] = 0.f;
    }
  }
  if (ok) {
    const int b = (int)(run / nrun), s0 = (int)(run % nrun) * kConvRun;
    const int s1 = min(s0 + kConvRun, S);
    const int tend = min(s1 + W - 1, S);   // rows with a dpre value (zero past S)
    const __bf16* gb = d < d1 ? g0 : (d < d2 ? g1 : g2);
    const int gn = d < d1 ? d1 : (d < d2 ? d2 - d1 : Dc - d2);
    const int gc = d < d1 ? d : (d < d2 ? d - d1 : d - d2);
    const __bf16* src = in + (size_t)b * S * ld + col0 + d;
    const __bf16* gsrc = gb + (size_t)b * S * gn + gc;
    __bf16* dst = din + (size_t)b * S * ldo + colo + d;
    float xw[W][8], dw[W][8];   // x rows t-(W-1)..t, dpre rows t-(W-1)..t
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
      const int sp = s0 - (W - 1) + w;
      const bf16x8 u = sp >= 0 ? *(const bf16x8*)(src + (size_t)sp * ld) : bf16x8{};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        xw[w][c] = (float)u[c];
        dw[w][c] = 0.f;
      }
    }
    constexpr int kBlk = 4;
    bf16x8 nx[kBlk], ngr[kBlk];
    auto issue = [&](int tb) {
#pragma unroll
      for (int r = 0; r < kBlk; ++r) {
        const bool in_s = tb + r < tend;
        nx[r] = in_s ? *(const bf16x8*)(src + (size_t)(tb + r) * ld) : bf16x8{};
        ngr[r] = in_s ? *(const bf16x8*)(gsrc + (size_t)(tb + r) * gn) : bf16x8{};
      }
    };
    const int tlast = s1 + W - 1;   // rows s0 .. tlast - 1 are walked
    issue(s0);
    for (int tb = s0; tb < tlast; tb += kBlk) {
      bf16x8 cx[kBlk], cgr[kBlk];
#pragma unroll
      for (int r = 0; r < kBlk; ++r) {
        cx[r] = nx[r];
        cgr[r] = ngr[r];
      }
      if (tb + kBlk < tlast) issue(tb + kBlk);
#pragma unroll
      for (int r = 0; r < kBlk; ++r) {
        const int t = tb + r;
        if (t < tlast) {
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            xw[W - 1][c] = (float)cx[r][c];
            float pre = bv[c];
#pragma unroll
            for (int w = 0; w < W; ++w) pre += wv[c][w] * xw[w][c];
            // rows past S load as zero gradients, so dpre is zero there
            dw[W - 1][c] = (float)cgr[r][c] * dsilu_f(pre);
          }
          if (t < s1) {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              accb[c] += dw[W - 1][c];
#pragma unroll
              for (int w = 0; w < W; ++w) accw[c][w] += dw[W - 1][c] * xw[w][c];
            }
          }
          const int so = t - (W - 1);   // din row completed by this dpre
          if (so >= s0 && so < s1) {
            bf16x8 o;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              float gi = 0.f;
#pragma unroll
              for (int w = 0; w < W; ++w) gi += wv[c][w] * dw[W - 1 - w][c];
              o[c] = (__bf16)gi;
            }
            *(bf16x8*)(dst + (size_t)so * ldo) = o;
          }
#pragma unroll
          for (int w = 0; w < W - 1; ++w)
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              xw[w][c] = xw[w + 1][c];
              dw[w][c] = dw[w + 1][c];
            }
        }
      }
    }
  }
  // the wave's four runs (lanes 16 apart), then the four waves, in fixed order
  const int wv_id = tid >> 6;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int w = 0; w <= W; ++w) {
      float a = w < W ? accw[c][w] : accb[c];
      a += __shfl_xor(a, 16, 64);
      a += __shfl_xor(a, 32, 64);
      if ((tid & 63) < 16) red[wv_id][cl][c][w] = a;
    }
  }
  __syncthreads();
  for (int e = tid; e < 16 * 8 * (W + 1); e += 256) {
    const int l = e / (8 * (W + 1)), rem = e % (8 * (W + 1));
    const int c = rem / (W + 1), w = rem % (W + 1);
    const int cgo = blockIdx.x * 16 + l;
    if (cgo < ng) {
      const float sum = red[0][l][c][w] + red[1][l][c][w] + red[2][l][c][w] + red[3][l][c][w];
      ws[((size_t)blockIdx.y * Dc + 8 * cgo + c) * (W + 1) + w] = sum;
    }
  }
}

// Gated RMSNorm, one wave per row of n features: u = y silu(z), r = rsqrt(mean
// u^2 + eps), out = u r w; r is saved for the backward.
__global__ __launch_bounds__(256) void gated_rmsnorm_fwd_kernel(
    const void* __restrict__ y, const void* __restrict__ z, long ldz, const void* __restrict__ w,
    void* __restrict__ out, float* __restrict__ rstd, long rows, int n, float eps, int fy,
    int fz, int fw, int fo) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float ss = 0.f;
  for (int j = lane; j < n; j += 64) {
    const float u = ld1(y, (size_t)row * n + j, fy) * silu_f(ld1(z, (size_t)row * ldz + j, fz));
    ss += u * u;
  }
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  const float r = rsqrtf(ss / n + eps);
  if (lane == 0) rstd[row] = r;
  for (int j = lane; j < n; j += 64) {
    const float u = ld1(y, (size_t)row * n + j, fy) * silu_f(ld1(z, (size_t)row * ldz + j, fz));
    st1(out, (size_t)row * n + j, u * r * ld1(w, j, fw), fo);
  }
}

// Backward: g = dout w, du = r (g - u r^2 mean(g u)), dy = du silu(z),
// dz = du y silu'(z); dw partials [blk][n] summed in order afterwards.
// Grid nblk workgroups of 4 waves; wave (blk, q) handles rows blk*4 + q + 4*nblk*i.
__global__ __launch_bounds__(256) void gated_rmsnorm_bwd_kernel(
    const void* __restrict__ y, const void* __restrict__ z, long ldz, const void* __restrict__ w,
    const float* __restrict__ rstd, const void* __restrict__ dout, void* __restrict__ dy,
    void* __restrict__ dz, long lddz, float* __restrict__ ws, long rows, int n, int fy, int fz,
    int fw, int fdo, int fdy, int fdz) {
  extern __shared__ float wacc[];   // [4][n] per-wave dw partials
  const int q = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int blk = blockIdx.x, nblk = gridDim.x;
  for (int j = threadIdx.x; j < 4 * n; j += 256) wacc[j] = 0.f;
  __syncthreads();
  for (long row = (long)blk * 4 + q; row < rows; row += 4L * nblk) {
    const float r = rstd[row];
    float sgu = 0.f;
    for (int j = lane; j < n; j += 64) {
      const float zz = ld1(z, (size_t)row * ldz + j, fz);
      const float u = ld1(y, (size_t)row * n + j, fy) * silu_f(zz);
      sgu += ld1(dout, (size_t)row * n + j, fdo) * ld1(w, j, fw) * u;
    }
    for (int m = 32; m >= 1; m >>= 1) sgu += __shfl_xor(sgu, m, 64);
    const float mgu = sgu / n;
    for (int j = lane; j < n; j += 64) {
      const float zz = ld1(z, (size_t)row * ldz + j, fz), yy = ld1(y, (size_t)row * n + j, fy);
      const float sz = silu_f(zz), u = yy * sz;
      const float go = ld1(dout, (size_t)row * n + j, fdo);
      const float du = r * (go * ld1(w, j, fw) - u * r * r * mgu);
      st1(dy, (size_t)row * n + j, du * sz, fdy);
      st1(dz, (size_t)row * lddz + j, du * yy * dsilu_f(zz), fdz);
      wacc[q * n + j] += go * u * r;
    }
  }
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += 256)
    ws[(size_t)blk * n + j] = wacc[j] + wacc[n + j] + wacc[2 * n + j] + wacc[3 * n + j];
}

// Vector forms of the gated RMSNorm for n % 8 == 0, n <= 512 NC, 16-byte aligned
// rows: lane l of a row's wave owns elements 512 c + 8 l .. + 7 (c < NC) and
// keeps them in registers between the sum and the output.
template <int NC>
__global__ __launch_bounds__(256) void gated_rmsnorm_fwd_vec_kernel(
    const void* __restrict__ y, const void* __restrict__ z, long ldz, const void* __restrict__ w,
    void* __restrict__ out, float* __restrict__ rstd, long rows, int n, float eps, int fy,
    int fz, int fw, int fo) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float u[NC][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j = 512 * c + 8 * lane;
    if (j < n) {
      float yy[8], zz[8];
      ld8(y, (size_t)row * n + j, fy, yy);
      ld8(z, (size_t)row * ldz + j, fz, zz);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        u[c][k] = yy[k] * silu_f(zz[k]);
        ss += u[c][k] * u[c][k];
      }
    }
  }
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  const float r = rsqrtf(ss / n + eps);
  if (lane == 0) rstd[row] = r;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j = 512 * c + 8 * lane;
    if (j < n) {
      float wv[8], o[8];
      ld8(w, j, fw, wv);
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] = u[c][k] * r * wv[k];
      st8(out, (size_t)row * n + j, o, fo);
    }
  }
}

// Backward, vector form: as gated_rmsnorm_bwd_kernel, with each wave's dw
// partial kept in registers over its rows.
template <int NC>
__global__ __launch_bounds__(256) void gated_rmsnorm_bwd_vec_kernel(
    const void* __restrict__ y, const void* __restrict__ z, long ldz, const void* __restrict__ w,
    const float* __restrict__ rstd, const void* __restrict__ dout, void* __restrict__ dy,
    void* __restrict__ dz, long lddz, float* __restrict__ ws, long rows, int n, int fy, int fz,
    int fw, int fdo, int fdy, int fdz) {
  extern __shared__ float wacc[];   // [4][n] per-wave dw partials
  const int q = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int blk = blockIdx.x, nblk = gridDim.x;
  float wv[NC][8], acc[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j = 512 * c + 8 * lane;
    if (j < n) ld8(w, j, fw, wv[c]);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (j >= n) wv[c][k] = 0.f;
      acc[c][k] = 0.f;
    }
  }
  for (long row = (long)blk * 4 + q; row < rows; row += 4L * nblk) {
    const float r = rstd[row];
    float yy[NC][8], zz[NC][8], go[NC][8];
    float sgu = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int j = 512 * c + 8 * lane;
      if (j < n) {
        ld8(y, (size_t)row * n + j, fy, yy[c]);
        ld8(z, (size_t)row * ldz + j, fz, zz[c]);
        ld8(dout, (size_t)row * n + j, fdo, go[c]);
#pragma unroll
        for (int k = 0; k < 8; ++k) sgu += go[c][k] * wv[c][k] * (yy[c][k] * silu_f(zz[c][k]));
      }
    }
    for (int m = 32; m >= 1; m >>= 1) sgu += __shfl_xor(sgu, m, 64);
    const float mgu = sgu / n;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int j = 512 * c + 8 * lane;
      if (j < n) {
        float oy[8], oz[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float sz = silu_f(zz[c][k]), u = yy[c][k] * sz;
          const float du = r * (go[c][k] * wv[c][k] - u * r * r * mgu);
          oy[k] = du * sz;
          oz[k] = du * yy[c][k] * dsilu_f(zz[c][k]);
          acc[c][k] += go[c][k] * u * r;
        }
        st8(dy, (size_t)row * n + j, oy, fdy);
        st8(dz, (size_t)row * lddz + j, oz, fdz);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j = 512 * c + 8 * lane;
    if (j < n) {
#pragma unroll
      for (int k = 0; k < 8; ++k) wacc[q * n + j + k] = acc[c][k];
    }
  }
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += 256)
    ws[(size_t)blk * n + j] = wacc[j] + wacc[n + j] + wacc[2 * n + j] + wacc[3 * n + j];
}

// dweight[d][w], dbias[d] = ordered sums over the workgroups' partials
// ws[blk][d][W + 1]
__global__ __launch_bounds__(1024) void conv1d_bwd_reduce_kernel(const float* __restrict__ ws,
                                                                 float* __restrict__ dw,
                                                                 float* __restrict__ db,
                                                                 int nblk, int Dc, int W) {
  const int ncol = Dc * (W + 1), e = blockIdx.x * 64 + (threadIdx.x & 63);
  const float sum = ordered_colsum(ws, ncol, nblk, ncol, e);
  if (threadIdx.x >= 64 || e >= ncol) return;
  const int d = e / (W + 1), q = e % (W + 1);
  if (q < W) { if (dw) dw[(size_t)d * W + q] = sum; }
  else if (db) db[d] = sum;
}

__global__ __launch_bounds__(1024) void rows_sum_kernel(const float* __restrict__ ws,
                                                        float* __restrict__ out, int nblk, int n) {
  const int c = blockIdx.x * 64 + (threadIdx.x & 63);
  const float sum = ordered_colsum(ws, n, nblk, n, c);
  if (threadIdx.x < 64 && c < n) out[c] = sum;
}

}  // namespace hattn

namespace {
int conv_bwd_nblk(long tiles, int ncg) {
  long n = 2048 / (ncg > 0 ? ncg : 1);
  if (n > tiles) n = tiles;
  return (int)(n < 1 ? 1 : n);
}
// 512-element chunks per row for the vector RMSNorm kernels (1..4), or 0 for the
// scalar kernels: needs n % 8 == 0, row strides % 8 == 0 and 16-byte aligned bases
int norm_vec_chunks(int n, long ld1, long ld2, std::initializer_list<const void*> ptrs) {
  if (n % 8 != 0 || ld1 % 8 != 0 || ld2 % 8 != 0 || n > 2048) return 0;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return 0;
  return (n + 511) / 512;
}
int norm_bwd_nblk(long rows) {
  long n = (rows + 3) / 4;
  if (n > 1024) n = 1024;
  return (int)(n < 1 ? 1 : n);
}
}  // namespace

// run blocks of the vector backward (one partial row of ws each)
long conv_bwd_vec_nblk(int B, int S) {
  const long runs = (long)B * ((S + hattn::kConvRun - 1) / hattn::kConvRun);
  return (runs + hattn::kConvBwdRuns - 1) / hattn::kConvBwdRuns;
}
size_t hattn_conv1d_bwd_ws_bytes(int B, int S, int Dc, int W) {
  const long tiles = (long)B * ((S + hattn::kConvTile - 1) / hattn::kConvTile);
  const long nblk = std::max<long>(conv_bwd_nblk(tiles, (Dc + 63) / 64), conv_bwd_vec_nblk(B, S));
  return (size_t)nblk * Dc * (W + 1) * sizeof(float);
}
size_t hattn_rmsnorm_bwd_ws_bytes(long rows, int n) {
  return (size_t)norm_bwd_nblk(rows) * n * sizeof(float);
}

hipError_t hattn_conv1d_silu_fwd_launch(const void* in, long ld, long col0, const void* wt,
                                        const void* bias, void* o0, void* o1, void* o2, int B,
                                        int S, int Dc, int d1, int d2, int W, int fin, int fw,
                                        int fo, hipStream_t stream) {
  using namespace hattn;
  const long BS = (long)B * S;
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (fin == 1 && Dc % 8 == 0 && d1 % 8 == 0 && d2 % 8 == 0 && ld % 8 == 0 && col0 % 8 == 0 &&
      a16(in) && a16(o0) && a16(o1) && a16(o2) && W >= 1 && W <= 8) {
    const long threads = (long)B * ((S + kConvRun - 1) / kConvRun) * (Dc / 8);
    const dim3 vgrid((unsigned)((threads + 255) / 256));
    switch (W) {
#define CONV_FWD_VEC(W_)                                                                        \
  case W_:                                                                                      \
    hipLaunchKernelGGL((conv1d_silu_fwd_vec_kernel<W_>), vgrid, dim3(256), 0, stream,            \
                       (const __bf16*)in, ld, col0, wt, bias, o0, o1, o2, B, S, Dc, d1, d2, fw,  \
                       fo);                                                                      \
    break;
      CONV_FWD_VEC(1) CONV_FWD_VEC(2) CONV_FWD_VEC(3) CONV_FWD_VEC(4) CONV_FWD_VEC(5)
      CONV_FWD_VEC(6) CONV_FWD_VEC(7) CONV_FWD_VEC(8)
#undef CONV_FWD_VEC
    }
    return hipGetLastError();
  }
  const dim3 grid((unsigned)BS, (unsigned)((Dc + 255) / 256));
  switch (W) {
#define CONV_FWD(W_)                                                                          \
  case W_:                                                                                    \
    hipLaunchKernelGGL((conv1d_silu_fwd_kernel<W_>), grid, dim3(256), 0, stream, in, ld, col0, \
                       wt, bias, o0, o1, o2, BS, S, Dc, d1, d2, fin, fw, fo);                  \
    break;
    CONV_FWD(1) CONV_FWD(2) CONV_FWD(3) CONV_FWD(4) CONV_FWD(5) CONV_FWD(6) CONV_FWD(7)
    CONV_FWD(8)
#undef CONV_FWD
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t hattn_conv1d_silu_bwd_launch(const void* in, long ld, long col0, const void* wt,
                                        const void* bias, const void* g0, const void* g1,
                                        const void* g2, void* din, long ldo, long colo,
                                        float* dw, float* db, float* ws, int B, int S, int Dc,
                                        int d1, int d2, int W, int fin, int fw, int fg0, int fg1,
                                        int fg2, int fdi, hipStream_t stream) {
  using namespace hattn;
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (fin == 1 && fg0 == 1 && fg1 == 1 && fg2 == 1 && fdi == 1 && Dc % 8 == 0 && d1 % 8 == 0 &&
      d2 % 8 == 0 && ld % 8 == 0 && col0 % 8 == 0 && ldo % 8 == 0 && colo % 8 == 0 &&
      a16(in) && a16(g0) && a16(g1) && a16(g2) && a16(din) && W >= 1 && W <= 8) {
    const long vblk = conv_bwd_vec_nblk(B, S);
    const dim3 vgrid((unsigned)((Dc / 8 + 15) / 16), (unsigned)vblk);
    switch (W) {
#define CONV_BWD_VEC(W_)                                                                       \
  case W_:                                                                                     \
    hipLaunchKernelGGL((conv1d_silu_bwd_vec_kernel<W_>), vgrid, dim3(256), 0, stream,           \
                       (const __bf16*)in, ld, col0, wt, bias, (const __bf16*)g0,                \
                       (const __bf16*)g1, (const __bf16*)g2, (__bf16*)din, ldo, colo, ws, B, S, \
                       Dc, d1, d2, fw);                                                         \
    break;
      CONV_BWD_VEC(1) CONV_BWD_VEC(2) CONV_BWD_VEC(3) CONV_BWD_VEC(4) CONV_BWD_VEC(5)
      CONV_BWD_VEC(6) CONV_BWD_VEC(7) CONV_BWD_VEC(8)
#undef CONV_BWD_VEC
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(conv1d_bwd_reduce_kernel, dim3((Dc * (W + 1) + 63) / 64), dim3(1024), 0,
                       stream, ws, dw, db, (int)vblk, Dc, W);
    return hipGetLastError();
  }
  const int ncg = (Dc + 63) / 64;
  const long tiles = (long)B * ((S + kConvTile - 1) / kConvTile);
  const int nblk = conv_bwd_nblk(tiles, ncg);
  switch (W) {
#define CONV_BWD(W_)                                                                            \
  case W_:                                                                                      \
    hipLaunchKernelGGL((conv1d_silu_bwd_kernel<W_>), dim3(ncg, nblk), dim3(256), 0, stream, in, \
                       ld, col0, wt, bias, g0, g1, g2, din, ldo, colo, ws, B, S, Dc, d1, d2,    \
                       fin, fw, fg0, fg1, fg2, fdi);                                             \
    break;
    CONV_BWD(1) CONV_BWD(2) CONV_BWD(3) CONV_BWD(4) CONV_BWD(5) CONV_BWD(6) CONV_BWD(7)
    CONV_BWD(8)
#undef CONV_BWD
    default:
      return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(conv1d_bwd_reduce_kernel, dim3((Dc * (W + 1) + 63) / 64), dim3(1024), 0,
                     stream, ws, dw, db, nblk, Dc, W);
  return hipGetLastError();
}

hipError_t hattn_gated_rmsnorm_fwd_launch(const void* y, const void* z, long ldz, const void* w,
                                          void* out, float* rstd, long rows, int n, float eps,
                                          int fy, int fz, int fw, int fo, hipStream_t stream) {
  using namespace hattn;
  const dim3 grid((unsigned)((rows + 3) / 4));
  switch (norm_vec_chunks(n, ldz, ldz, {y, z, w, out})) {
#define NORM_FWD(NC_)                                                                       \
  case NC_:                                                                                 \
    hipLaunchKernelGGL((gated_rmsnorm_fwd_vec_kernel<NC_>), grid, dim3(256), 0, stream, y, z, \
                       ldz, w, out, rstd, rows, n, eps, fy, fz, fw, fo);                    \
    break;
    NORM_FWD(1) NORM_FWD(2) NORM_FWD(3) NORM_FWD(4)
#undef NORM_FWD
    default:
      hipLaunchKernelGGL(gated_rmsnorm_fwd_kernel, grid, dim3(256), 0, stream, y, z, ldz, w, out,
                         rstd, rows, n, eps, fy, fz, fw, fo);
  }
  return hipGetLastError();
}

hipError_t hattn_gated_rmsnorm_bwd_launch(const void* y, const void* z, long ldz, const void* w,
                                          const float* rstd, const void* dout, void* dy, void* dz,
                                          long lddz, float* dw, float* ws, long rows, int n,
                                          int fy, int fz, int fw, int fdo, int fdy, int fdz,
                                          hipStream_t stream) {
  using namespace hattn;
  const int nblk = norm_bwd_nblk(rows);
  const size_t smem = (size_t)4 * n * sizeof(float);
  const int nc = norm_vec_chunks(n, ldz, lddz, {y, z, w, dout, dy, dz});
  const void* fn = (const void*)gated_rmsnorm_bwd_kernel;
  if (nc == 1) fn = (const void*)gated_rmsnorm_bwd_vec_kernel<1>;
  else if (nc == 2) fn = (const void*)gated_rmsnorm_bwd_vec_kernel<2>;
  else if (nc == 3) fn = (const void*)gated_rmsnorm_bwd_vec_kernel<3>;
  else if (nc == 4) fn = (const void*)gated_rmsnorm_bwd_vec_kernel<4>;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  switch (nc) {
#define NORM_BWD(NC_)                                                                        \
  case NC_:                                                                                  \
    hipLaunchKernelGGL((gated_rmsnorm_bwd_vec_kernel<NC_>), dim3(nblk), dim3(256), smem,     \
                       stream, y, z, ldz, w, rstd, dout, dy, dz, lddz, ws, rows, n, fy, fz, fw, \
                       fdo, fdy, fdz);                                                        \
    break;
    NORM_BWD(1) NORM_BWD(2) NORM_BWD(3) NORM_BWD(4)
#undef NORM_BWD
    default:
      hipLaunchKernelGGL(gated_rmsnorm_bwd_kernel, dim3(nblk), dim3(256), smem, stream, y, z, ldz,
                         w, rstd, dout, dy, dz, lddz, ws, rows, n, fy, fz, fw, fdo, fdy, fdz);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(rows_sum_kernel, dim3((n + 63) / 64), dim3(1024), 0, stream, ws, dw, nblk, n);
  return hipGetLastError();
}
