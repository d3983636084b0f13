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

#include "common.h"

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

// torch.nn.functional.softplus (beta 1, threshold 20) and its derivative
__device__ __forceinline__ float softplus20(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float dsoftplus20(float x) {
  return x > 20.f ? 1.f : 1.f / (1.f + expf(-x));
}

enum { kLamLinear = 0, kLamPositive = 1, kLamBounded = 2 };

__device__ __forceinline__ float lambda_of(float Lv, float dlv, int mode) {
  if (mode == kLamPositive) return softplus20(Lv * dlv);
  if (mode == kLamBounded) return expf(-expf(Lv) * softplus20(dlv));
  return Lv * dlv;
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
  if ((int)blockIdx.x < nbx) {
    const long q4 = (long)blockIdx.x * 256 + threadIdx.x;
    const long e0 = 4 * q4;
    if (e0 >= rows * P) return;
    const long r = e0 / P;
    const int h = (int)(r % H);
    float d = ld1(dt, r, f.dt) + (dt_bias ? dt_bias[h] : 0.f);
    if (softplus) d = softplus20(d);
    const floatx4 xv = ld4(x, e0, f.x);
    st4(v, e0, floatx4{xv[0] * d, xv[1] * d, xv[2] * d, xv[3] * d}, f.v);
    if (e0 == r * P) g[r] = A[h] * d;
  } else {
    const long e = (long)(blockIdx.x - nbx) * 256 + threadIdx.x;
    if (e >= rows * L) return;
    const long r = e / L;
    const int l = (int)(e - r * L);
    const int h = (int)(r % H);
    st1(lam, e, lambda_of(ld1(Lp, (size_t)h * L + l, f.lp), ld1(dl, e, f.dl), mode), f.lam);
  }
}

// out = y + x * D[h], four elements per thread
__global__ __launch_bounds__(256) void mamba2_layer_epilogue_kernel(
    const void* __restrict__ y, const void* __restrict__ x, const float* __restrict__ D,
    void* __restrict__ out, long rows, int H, int P, int ybf, int xbf, int obf) {
  const long e0 = 4 * ((long)blockIdx.x * 256 + threadIdx.x);
  if (e0 >= rows * P) return;
  const int h = (int)((e0 / P) % H);
  const float d = D[h];
  const floatx4 a = ld4(y, e0, ybf), b = ld4(x, e0, xbf);
  st4(out, e0, floatx4{a[0] + b[0] * d, a[1] + b[1] * d, a[2] + b[2] * d, a[3] + b[3] * d}, obf);
}

struct LayerBwdDt {
  int x, dt, dl, lp, dy, dv, dlam, dx, ddt, ddl;   // 1 = bf16, 0 = fp32
};

constexpr int kLayerMaxL = 32;   // lambda levels
constexpr int kLayerNQ = 3 + kLayerMaxL;

// Backward: grid (nblk, H); workgroup (blk, h) owns the rows bt*H + h for bt in
// its contiguous share of [0, B*T).  A row is handled by tpr = P / 4 threads
// (four elements each, P / 4 a power of two <= 64).  Per-head partials
// [dA, ddt_bias, dD, dL[0..L)] go to ws[h][blk][3 + L].
__global__ __launch_bounds__(256) void mamba2_layer_bwd_kernel(
    const void* __restrict__ x, const void* __restrict__ dt, const float* __restrict__ A,
    const float* __restrict__ dt_bias, const void* __restrict__ dl, const void* __restrict__ Lp,
    const float* __restrict__ D, const void* __restrict__ dy, const void* __restrict__ dv,
    const float* __restrict__ dg, const void* __restrict__ dlam, void* __restrict__ dx,
    void* __restrict__ ddt, void* __restrict__ ddl, float* __restrict__ ws, long BT, int H,
    int P, int L, int softplus, int mode, LayerBwdDt f) {
  __shared__ float red[kLayerNQ][256];
  const int tid = threadIdx.x, h = blockIdx.y, blk = blockIdx.x, nblk = gridDim.x;
  const int tpr = P / 4, rpi = 256 / tpr;
  const int j = tid % tpr, ri = tid / tpr;
  const long per = (BT + nblk - 1) / nblk;
  const long bt0 = (long)blk * per, bt1 = min(BT, bt0 + per);
  const float Ah = A[h], bias = dt_bias ? dt_bias[h] : 0.f, Dh = D ? D[h] : 0.f;
  float accA = 0.f, accB = 0.f, accD = 0.f, accL[kLayerMaxL];
#pragma unroll
  for (int i = 0; i < kLayerMaxL; ++i) accL[i] = 0.f;
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
    for (int i = 0; i < kLayerMaxL; ++i) {
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
          const float eL = expf(Lv), sp = softplus20(dlv);
          const float lamv = expf(-eL * sp);
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
  for (int i = 0; i < kLayerMaxL; ++i) {
    const int l = j + i * tpr;
    if (l < L) red[3 + l][ri] = accL[i];   // slot ri of level l (rpi slots per level)
  }
  __syncthreads();
  const int nq = 3 + L;
  if (tid < nq) {
    const int n = tid < 3 ? 256 : rpi;
    float sum = 0.f;
    for (int i = 0; i < n; ++i) sum += red[tid][i];
    ws[((size_t)h * nblk + blk) * nq + tid] = sum;
  }
}

// Per-head sums over the workgroups, in order.
__global__ __launch_bounds__(64) void mamba2_layer_bwd_reduce_kernel(
    const float* __restrict__ ws, float* __restrict__ dA, float* __restrict__ ddt_bias,
    float* __restrict__ dD, float* __restrict__ dLp, int nblk, int L) {
  const int h = blockIdx.x, q = threadIdx.x, nq = 3 + L;
  if (q >= nq) return;
  float sum = 0.f;
  for (int b = 0; b < nblk; ++b) sum += ws[((size_t)h * nblk + b) * nq + q];
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

size_t hattn_mamba2_layer_bwd_ws_bytes(int B, int T, int H, int L) {
  const long BT = (long)B * T;
  return (size_t)H * layer_bwd_nblk(BT, H) * (3 + L) * sizeof(float);
}

hipError_t hattn_mamba2_layer_prologue_launch(const void* x, const void* dt, const float* A,
                                              const float* dt_bias, const void* dl,
                                              const void* Lp, void* v, float* g, void* lam,
                                              int B, int T, int H, int P, int L, int softplus,
                                              int mode, const int* bf, hipStream_t stream) {
  using namespace hattn;
  const long rows = (long)B * T * H;
  const LayerDt f{bf[0], bf[1], bf[2], bf[3], bf[4], bf[5]};
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
  const int nblk = layer_bwd_nblk(BT, H);
  const LayerBwdDt f{bf[0], bf[1], bf[2], bf[3], bf[4], bf[5], bf[6], bf[7], bf[8], bf[9]};
  hipLaunchKernelGGL(mamba2_layer_bwd_kernel, dim3(nblk, H), dim3(256), 0, stream, x, dt, A,
                     dt_bias, dl, Lp, D, dy, dv, dg, dlam, dx, ddt, ddl, ws, BT, H, P, L, softplus,
                     mode, f);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mamba2_layer_bwd_reduce_kernel, dim3(H), dim3(64), 0, stream, ws, dA,
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

constexpr int kConvMaxW = 8;

// one thread per (b, s, d); d fastest
__global__ __launch_bounds__(256) void conv1d_silu_fwd_kernel(
    const void* __restrict__ in, long ld, long col0, const void* __restrict__ wt,
    const void* __restrict__ bias, void* __restrict__ o0, void* __restrict__ o1,
    void* __restrict__ o2, long BS, int S, int Dc, int d1, int d2, int W, int fin, int fw,
    int fo) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= BS * Dc) return;
  const long bs = e / Dc;
  const int d = (int)(e - bs * Dc);
  const int s = (int)(bs % S);
  float acc = bias ? ld1(bias, d, fw) : 0.f;
  for (int w = 0; w < W; ++w) {
    const int sp = s - (W - 1) + w;
    if (sp >= 0) acc += ld1(wt, (size_t)d * W + w, fw) * ld1(in, (size_t)(bs - s + sp) * ld + col0 + d, fin);
  }
  const float y = silu_f(acc);
  if (d < d1) st1(o0, (size_t)bs * d1 + d, y, fo);
  else if (d < d2) st1(o1, (size_t)bs * (d2 - d1) + (d - d1), y, fo);
  else st1(o2, (size_t)bs * (Dc - d2) + (d - d2), y, fo);
}

// Backward of the conv + SiLU.  Grid (Dc / 64, nblk): workgroup (cg, blk)
// owns channels 64 cg .. + 63 and the 64-token tiles blk, blk + nblk, ... of
// the flattened (b, s-tile) index.  Per tile it stages the input rows the
// tile needs, forms dpre = dout * silu'(pre) for the tile and the W - 1 rows
// after it, writes din and accumulates dweight / dbias partials, which go to
// ws[blk][64 cg + c][W + 1] and are summed in order afterwards.
constexpr int kConvTile = 64;

__global__ __launch_bounds__(256) void conv1d_silu_bwd_kernel(
    const void* __restrict__ in, long ld, long col0, const void* __restrict__ wt,
    const void* __restrict__ bias, const void* __restrict__ g0, const void* __restrict__ g1,
    const void* __restrict__ g2, void* __restrict__ din, long ldo, long colo,
    float* __restrict__ ws, int B, int S, int Dc, int d1, int d2, int W, int fin, int fw,
    int fg0, int fg1, int fg2, int fdi) {
  __shared__ float xs[kConvTile + 2 * kConvMaxW][64];   // input rows s0-(W-1) .. s0+63+(W-1)
  __shared__ float dp[kConvTile + kConvMaxW][64];       // dpre rows s0 .. s0+63+(W-1)
  __shared__ float red[4][64][kConvMaxW + 1];
  const int tid = threadIdx.x, c = tid & 63, sr = tid >> 6;
  const int cg = blockIdx.x, blk = blockIdx.y, nblk = gridDim.y;
  const int d = 64 * cg + c;
  const bool dok = d < Dc;
  const int ntile_s = (S + kConvTile - 1) / kConvTile;
  const long ntiles = (long)B * ntile_s;
  float wv[kConvMaxW];
#pragma unroll
  for (int w = 0; w < kConvMaxW; ++w) wv[w] = (dok && w < W) ? ld1(wt, (size_t)d * W + w, fw) : 0.f;
  const float bv = (dok && bias) ? ld1(bias, d, fw) : 0.f;
  float accw[kConvMaxW], accb = 0.f;
#pragma unroll
  for (int w = 0; w < kConvMaxW; ++w) accw[w] = 0.f;
  auto gout = [&](long bs) -> float {
    if (d < d1) return ld1(g0, (size_t)bs * d1 + d, fg0);
    if (d < d2) return ld1(g1, (size_t)bs * (d2 - d1) + (d - d1), fg1);
    return ld1(g2, (size_t)bs * (Dc - d2) + (d - d2), fg2);
  };
  for (long tile = blk; tile < ntiles; tile += nblk) {
    const int b = (int)(tile / ntile_s), s0 = (int)(tile % ntile_s) * kConvTile;
    const long base = (long)b * S;
    // input rows s0 - (W-1) .. s0 + 63 + (W-1)
    const int nx = kConvTile + 2 * (W - 1);
    for (int r = sr; r < nx; r += 4) {
      const int sp = s0 - (W - 1) + r;
      xs[r][c] = (dok && sp >= 0 && sp < S) ? ld1(in, (size_t)(base + sp) * ld + col0 + d, fin) : 0.f;
    }
    __syncthreads();
    // dpre rows s0 .. s0 + 63 + (W-1)
    const int np = kConvTile + W - 1;
    for (int r = sr; r < np; r += 4) {
      const int sp = s0 + r;
      float v = 0.f;
      if (dok && sp < S) {
        float pre = bv;
        for (int w = 0; w < W; ++w) pre += wv[w] * xs[r + w][c];   // xs row r + w is s0 + r - (W-1) + w
        v = gout(base + sp) * dsilu_f(pre);
      }
      dp[r][c] = v;
    }
    __syncthreads();
    // din and the weight / bias partials for rows s0 .. s0 + 63
    for (int r = sr; r < kConvTile; r += 4) {
      const int sp = s0 + r;
      if (!dok || sp >= S) continue;
      float gi = 0.f;
      for (int w = 0; w < W; ++w) gi += wv[w] * dp[r + (W - 1) - w][c];   // out row sp + W-1-w
      st1(din, (size_t)(base + sp) * ldo + colo + d, gi, fdi);
      const float dpr = dp[r][c];
      accb += dpr;
      for (int w = 0; w < W; ++w) accw[w] += dpr * xs[r + w][c];        // input row sp-(W-1)+w
    }
    __syncthreads();
  }
#pragma unroll
  for (int w = 0; w < kConvMaxW; ++w) red[sr][c][w] = accw[w];
  red[sr][c][kConvMaxW] = accb;
  __syncthreads();
  if (sr == 0 && dok) {
    float* out = ws + ((size_t)blk * Dc + d) * (W + 1);
    for (int w = 0; w < W; ++w) out[w] = red[0][c][w] + red[1][c][w] + red[2][c][w] + red[3][c][w];
    out[W] = red[0][c][kConvMaxW] + red[1][c][kConvMaxW] + red[2][c][kConvMaxW] + red[3][c][kConvMaxW];
  }
}

// dweight[d][w], dbias[d] = ordered sums over the workgroups' partials
__global__ __launch_bounds__(256) void conv1d_bwd_reduce_kernel(const float* __restrict__ ws,
                                                                float* __restrict__ dw,
                                                                float* __restrict__ db,
                                                                int nblk, int Dc, int W) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= Dc * (W + 1)) return;
  const int d = e / (W + 1), q = e % (W + 1);
  float sum = 0.f;
  for (int b = 0; b < nblk; ++b) sum += ws[((size_t)b * Dc + d) * (W + 1) + q];
  if (q < W) { if (dw) dw[(size_t)d * W + q] = sum; }
  else if (db) db[d] = sum;
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

__global__ __launch_bounds__(256) void rows_sum_kernel(const float* __restrict__ ws,
                                                       float* __restrict__ out, int nblk, int n) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n) return;
  float sum = 0.f;
  for (int b = 0; b < nblk; ++b) sum += ws[(size_t)b * n + j];
  out[j] = sum;
}

}  // namespace hattn

namespace {
int conv_bwd_nblk(long tiles, int ncg) {
  long n = 2048 / (ncg > 0 ? ncg : 1);
  if (n > tiles) n = tiles;
  return (int)(n < 1 ? 1 : n);
}
int norm_bwd_nblk(long rows) {
  long n = (rows + 3) / 4;
  if (n > 1024) n = 1024;
  return (int)(n < 1 ? 1 : n);
}
}  // namespace

size_t hattn_conv1d_bwd_ws_bytes(int B, int S, int Dc, int W) {
  const long tiles = (long)B * ((S + hattn::kConvTile - 1) / hattn::kConvTile);
  return (size_t)conv_bwd_nblk(tiles, (Dc + 63) / 64) * Dc * (W + 1) * sizeof(float);
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
  const long n = (BS * Dc + 255) / 256;
  hipLaunchKernelGGL(conv1d_silu_fwd_kernel, dim3((unsigned)n), dim3(256), 0, stream, in, ld,
                     col0, wt, bias, o0, o1, o2, BS, S, Dc, d1, d2, W, fin, fw, fo);
  return hipGetLastError();
}

hipError_t hattn_conv1d_silu_bwd_launch(const void* in, long ld, long col0, const void* wt,
                                        const void* bias, const void* g0, const void* g1,
                                        const void* g2, void* din, long ldo, long colo,
                                        float* dw, float* db, float* ws, int B, int S, int Dc,
                                        int d1, int d2, int W, int fin, int fw, int fg0, int fg1,
                                        int fg2, int fdi, hipStream_t stream) {
  using namespace hattn;
  const int ncg = (Dc + 63) / 64;
  const long tiles = (long)B * ((S + kConvTile - 1) / kConvTile);
  const int nblk = conv_bwd_nblk(tiles, ncg);
  hipLaunchKernelGGL(conv1d_silu_bwd_kernel, dim3(ncg, nblk), dim3(256), 0, stream, in, ld, col0,
                     wt, bias, g0, g1, g2, din, ldo, colo, ws, B, S, Dc, d1, d2, W, fin, fw, fg0,
                     fg1, fg2, fdi);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(conv1d_bwd_reduce_kernel, dim3((Dc * (W + 1) + 255) / 256), dim3(256), 0,
                     stream, ws, dw, db, nblk, Dc, W);
  return hipGetLastError();
}

hipError_t hattn_gated_rmsnorm_fwd_launch(const void* y, const void* z, long ldz, const void* w,
                                          void* out, float* rstd, long rows, int n, float eps,
                                          int fy, int fz, int fw, int fo, hipStream_t stream) {
  using namespace hattn;
  hipLaunchKernelGGL(gated_rmsnorm_fwd_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     stream, y, z, ldz, w, out, rstd, rows, n, eps, fy, fz, fw, fo);
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
  hipError_t e = hipFuncSetAttribute((const void*)gated_rmsnorm_bwd_kernel,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(gated_rmsnorm_bwd_kernel, dim3(nblk), dim3(256), smem, stream, y, z, ldz, w,
                     rstd, dout, dy, dz, lddz, ws, rows, n, fy, fz, fw, fdo, fdy, fdz);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(rows_sum_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, ws, dw, nblk, n);
  return hipGetLastError();
}
