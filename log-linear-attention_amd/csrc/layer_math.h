// Elementwise math of the log-linear Mamba-2 layer pre- and post-processing
// (hmamba_chunk_scan_combined, mamba_apis.py:346-403), shared by the separate
// layer kernels (mamba2_layer.hip) and the forward scan that folds them into its
// loads and stores (mamba2_fwd.hip), so both compute the same values bit for bit:
//   dt'  = softplus(dt + dt_bias)     (softplus threshold 20 as torch)
//   v    = x dt',   g = A[h] dt'
//   lam  = compute_lambda(L[h], dl):  positive softplus(L dl), bounded
//          exp(-exp(L) softplus(dl)), None L dl (mamba_apis.py:70-85)
//   y    = o + x D[h]
#pragma once

#include <hip/hip_runtime.h>

namespace hattn {

// torch.nn.functional.softplus (beta 1, threshold 20) and its derivative.
// softplus(x) = log1p(e^x) from the hardware exp / log (v_exp_f32, v_log_f32)
// with log1p(y) = y log(u) / (u - 1), u = 1 + y (Goldberg's form: the rounding
// of 1 + y cancels, so small results keep full relative accuracy, a few ulp):
// about ten instructions instead of the library's log1pf(expf(x)), which
// matters where the forward scan computes lambda per element.
__device__ __forceinline__ float log1p_fast(float y) {
  const float u = 1.f + y;
  return u == 1.f ? y : __logf(u) * (y / (u - 1.f));
}
__device__ __forceinline__ float softplus20(float x) { return x > 20.f ? x : log1p_fast(__expf(x)); }
__device__ __forceinline__ float dsoftplus20(float x) {
  return x > 20.f ? 1.f : 1.f / (1.f + expf(-x));
}

enum { kLamLinear = 0, kLamPositive = 1, kLamBounded = 2 };

__device__ __forceinline__ float lambda_of(float Lv, float dlv, int mode) {
  if (mode == kLamPositive) return softplus20(Lv * dlv);
  if (mode == kLamBounded) return __expf(-__expf(Lv) * softplus20(dlv));
  return Lv * dlv;
}

// The layer inputs of a forward scan that computes v, g and lambda itself:
// the scan's v pointer is x, its lambda pointer dl, and g comes from dt.
struct LayerArgs {
  const void* dt;      // [B, T, H], fp32 (dt_f32) or bf16
  const float* A;      // [H]
  const float* bias;   // [H] or null
  const float* Lp;     // [H, L] fp32
  const float* D;      // [H] or null: y = bf16(o) + x D[h], else y = o
  int dt_f32, softplus, mode, lam_bf16;   // lam_bf16: lambda rounded to bf16 (its dtype)
};

// dt' of one token: dt read as a 32-bit word of the dt tensor (element el, the
// bf16 half selected by the element's byte offset) plus the head's bias.
__device__ __forceinline__ float layer_dt_word(unsigned int word, unsigned int el, int f32) {
  if (f32) return __builtin_bit_cast(float, word);
  return __builtin_bit_cast(float, (el & 1) ? (word & 0xffff0000u) : (word << 16));
}
__device__ __forceinline__ float layer_dtp(float dt, float bias_h, int softplus) {
  const float d = __fadd_rn(dt, bias_h);
  return softplus ? softplus20(d) : d;
}

// g = A[h] dt' and y = o + x D[h], each rounded as written (never contracted
// with the arithmetic around them), so the separate and the folded kernels agree
__device__ __forceinline__ float layer_g(float A_h, float d) { return __fmul_rn(A_h, d); }
__device__ __forceinline__ float layer_out(float o, float x, float D_h) {
  return __fadd_rn(o, __fmul_rn(x, D_h));
}

}  // namespace hattn
