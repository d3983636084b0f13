// C-ABI entry points of libhattn_hip.so (declared in include/hattn.h).
//
// Host-side validation mirrors the checks of the reference host drivers
// (chunkwise.py:1140-1153, 1211-1214; kernel.py:55-123) and reports them as
// status codes plus a thread-local message; the kernels themselves assume
// validated shapes.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <initializer_list>

#include "../../include/hattn.h"

hipError_t hattn_mamba2_fwd_launch(const void* q, const void* k, const void* v, const float* g,
                                   const void* l, void* o, float* gcum, float* ht, void* ws,
                                   int B, int T, int G, int H, int V, int L, int nlev, int dt_qk,
                                   int dt_v, int dt_l, int dt_o, hipStream_t stream,
                                   int* unsupported);
size_t hattn_mamba2_fwd_ws_bytes(int B, int T, int H, int V, int x3);
size_t hattn_mamba2_fwd_static_scratch_bytes();
hipError_t hattn_mamba2_fwd_static_scratch(void** ptr);
int hattn_mamba2_fwd_max_levels(int x3);
int hattn_mamba2_strong_max_levels();
hipError_t hattn_mamba2_strong_ht_launch(const void* k, const void* v, const float* g, float* ht,
                                         int B, int T, int G, int H, int V, int L,
                                         hipStream_t stream);
hipError_t hattn_mamba2_strong_fwd_launch(const void* q, const void* k, const void* v,
                                          const float* g, const void* l, void* o, float* gcum,
                                          void* ws, size_t ws_bytes, int B, int T, int G, int H,
                                          int V, int L, int dt_l, int dt_o, hipStream_t stream,
                                          int* unsupported);
size_t hattn_mamba2_strong_fwd_ws_bytes(int B, int T, int H, int V);
size_t hattn_mamba2_strong_bwd_ws_bytes(int B, int T, int H, int nlev);
hipError_t hattn_mamba2_layer_fwd_launch(const void* q, const void* k, const void* x,
                                         const void* dl, void* o, float* gcum, void* ws,
                                         const void* dt, const float* A, const float* dt_bias,
                                         const float* Lp, const float* D, int dt_f32,
                                         int softplus, int mode, int lam_bf16, int B, int T,
                                         int G, int H, int V, int L, int nlev, int dt_l,
                                         int dt_o, hipStream_t stream, int* unsupported);
hipError_t hattn_mamba2_strong_bwd_launch(const void* q, const void* k, const void* v,
                                          const float* gc, const void* l, const void* dO,
                                          void* dq, void* dk, void* dv, float* dg, float* dl,
                                          void* ws, int B, int T, int H, int L, int nlev,
                                          int dt_l, hipStream_t stream, int* unsupported);
size_t hattn_gdn_fwd_ws_bytes(int B, int T, int H, int K, int V);
int hattn_gdn_fwd_max_levels();
int hattn_gdn_fwd_supports_k(int K);
int hattn_gdn_bwd_max_levels();
hipError_t hattn_gdn_fwd_launch(const void* q, const void* k, const void* v, const void* beta,
                                const float* g, const void* l, void* o, float* gcum, void* aw,
                                void* au, float* ht, void* ws, int B, int T, int H, int K, int V,
                                int L, int nlev, int dt_b, int dt_l, int dt_o, int norm_qk,
                                float scale, int strong, int h16, hipStream_t stream,
                                int* unsupported);
size_t hattn_gdn_fwd_keep_ws_bytes(int B, int T, int H, int K, int V, int nlev);
hipError_t hattn_gdn_fwd_keep_launch(const void* q, const void* k, const void* v,
                                     const void* beta, const float* g, const void* l, void* o,
                                     float* gcum, void* aw, void* au, float* ht, void* ws, int B,
                                     int T, int H, int K, int V, int L, int nlev, int dt_b,
                                     int dt_l, int dt_o, int norm_qk, float scale, int strong,
                                     int h16, hipStream_t stream, int* unsupported);
void hattn_gdn_fwd_keep_buffers(const void* ws, int B, int T, int H, int K, int V, int nlev,
                                const __bf16** qn, const __bf16** wn, const __bf16** kn,
                                const __bf16** un, const __bf16** hs);
size_t hattn_gdn_bwd_kept_ws_bytes(int B, int T, int H, int K, int V, int nlev);
hipError_t hattn_gdn_bwd_kept_launch(const void* q, const void* k, const void* v,
                                     const void* beta, const float* gcum, const void* l,
                                     const void* dO, void* dq, void* dk, void* dv, void* db,
                                     float* dg, float* dl, const __bf16* qn, const __bf16* wn,
                                     const __bf16* kn, const __bf16* un, const __bf16* hs,
                                     void* ws, int B, int T, int H, int K, int V, int L, int nlev,
                                     int dt_b, int dt_l, int norm_qk, float scale, int strong,
                                     int h16, hipStream_t stream, int* unsupported);
size_t hattn_gdn_bwd_ws_bytes(int B, int T, int H, int K, int V, int nlev);
hipError_t hattn_gdn_bwd_launch(const void* q, const void* k, const void* v, const void* beta,
                                const float* gcum, const void* l, const void* dO, void* dq,
                                void* dk, void* dv, void* db, float* dg, float* dl, void* ws,
                                int B, int T, int H, int K, int V, int L, int nlev, int dt_b,
                                int dt_l, int norm_qk, float scale, int strong, int h16,
                                hipStream_t stream, int* unsupported);
size_t hattn_mamba2_bwd_ws_bytes(int B, int T, int H, int V, int nlev);
hipError_t hattn_mamba2_bwd_launch(const void* q, const void* k, const void* v, const float* gc,
                                   const void* l, const void* dO, void* dq, void* dk, void* dv,
                                   float* dg, float* dl, void* ws, const float* fsums,
                                   const float* fsegd, int B, int T, int H, int V, int L,
                                   int nlev, int dt_qk, int dt_v, int dt_l, hipStream_t stream,
                                   int* unsupported);
void hattn_mamba2_fwd_ws_summaries(void* ws, int B, int T, int H, int V, const float** sums,
                                   const float** segd);
void hattn_mamba2_fwd_set_lookback(int spin_limit, int publish);
const unsigned int* hattn_mamba2_fwd_status_word(const void* ws, int B, int T, int H, int V);

hipError_t hattn_hstate_step_launch(float* states, int* counts, const void* q, const void* k,
                                    const void* v, const void* beta, const float* g,
                                    const void* l, void* o, int B, int G, int H, int K, int V,
                                    int L, int gdn, int cascade, int strong, int update, int output,
                                    int norm_qk, float scale, int dt_qk, int dt_v, int dt_l,
                                    int dt_b, hipStream_t stream, int* unsupported);
hipError_t hattn_mamba2_prefill_levels_launch(float* states, const void* k, const void* v,
                                              const float* g, int B, int T, int G, int H, int K,
                                              int V, int L, int nlo, int dt_k, int dt_v,
                                              hipStream_t stream, int* unsupported);

size_t hattn_mamba2_layer_bwd_ws_bytes(int B, int T, int H, int L);
hipError_t hattn_mamba2_layer_prologue_launch(const void* x, const void* dt, const float* A,
                                              const float* dt_bias, const void* dl,
                                              const void* Lp, void* v, float* g, void* lam,
                                              int B, int T, int H, int P, int L, int softplus,
                                              int mode, const int* bf, hipStream_t stream);
hipError_t hattn_mamba2_layer_epilogue_launch(const void* y, const void* x, const float* D,
                                              void* out, int B, int T, int H, int P, int ybf,
                                              int xbf, int obf, hipStream_t stream);
hipError_t hattn_mamba2_layer_bwd_launch(const void* x, const void* dt, const float* A,
                                         const float* dt_bias, const void* dl, const void* Lp,
                                         const float* D, const void* dy, const void* dv,
                                         const float* dg, const void* dlam, void* dx, void* ddt,
                                         void* ddl, float* dA, float* ddt_bias, float* dD,
                                         float* dLp, float* ws, int B, int T, int H, int P, int L,
                                         int softplus, int mode, const int* bf,
                                         hipStream_t stream);

size_t hattn_conv1d_bwd_ws_bytes(int B, int S, int Dc, int W);
size_t hattn_rmsnorm_bwd_ws_bytes(long rows, int n);
hipError_t hattn_conv1d_silu_fwd_launch(const void* in, long ld, long col0, const void* wt,
                                        const void* bias, void* o0, void* o1, void* o2, int B,
                                        int S, int Dc, int d1, int d2, int W, int fin, int fw,
                                        int fo, hipStream_t stream);
hipError_t hattn_conv1d_silu_bwd_launch(const void* in, long ld, long col0, const void* wt,
                                        const void* bias, const void* g0, const void* g1,
                                        const void* g2, void* din, long ldo, long colo,
                                        float* dw, float* db, float* ws, int B, int S, int Dc,
                                        int d1, int d2, int W, int fin, int fw, int fg0, int fg1,
                                        int fg2, int fdi, hipStream_t stream);
hipError_t hattn_gated_rmsnorm_fwd_launch(const void* y, const void* z, long ldz, const void* w,
                                          void* out, float* rstd, long rows, int n, float eps,
                                          int fy, int fz, int fw, int fo, hipStream_t stream);
hipError_t hattn_gated_rmsnorm_bwd_launch(const void* y, const void* z, long ldz, const void* w,
                                          const float* rstd, const void* dout, void* dy, void* dz,
                                          long lddz, float* dw, float* ws, long rows, int n,
                                          int fy, int fz, int fw, int fdo, int fdy, int fdz,
                                          hipStream_t stream);

namespace {

thread_local char g_err[512] = {0};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = 0;
  return HATTN_OK;
}

// ceil(log2(n)) for n >= 1 (ceil_log(NT, 2), base.py:29-30; exact for integers)
int ceil_log2(int n) {
  int e = 0;
  while ((1 << e) < n) ++e;
  return e;
}

int check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(HATTN_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

size_t elem_bytes(int code) { return code == HATTN_FP32 ? 4 : 2; }

// The Mamba-2 kernels address one batch's [T, heads, D] slice of each tensor
// through a buffer descriptor whose byte range and offsets are 32-bit, so
// every slice must stay below 4 GiB.  row_bytes: the largest per-token row
// (all heads) of any tensor the call reads or writes.
int check_span(int T, size_t row_bytes) {
  if ((unsigned long long)T * row_bytes >= (1ull << 32))
    return fail(HATTN_ERR_NOT_IMPLEMENTED,
                "one batch's slice of T=%d rows of %zu bytes reaches 4 GiB (32-bit buffer range)",
                T, row_bytes);
  return HATTN_OK;
}

size_t max_of(std::initializer_list<size_t> xs) {
  size_t m = 0;
  for (size_t x : xs) m = x > m ? x : m;
  return m;
}

}  // namespace

extern "C" {

const char* hattn_version(void) { return "hattn-mi355x 0.1.0 gfx950"; }

const char* hattn_last_error(void) { return g_err; }

size_t hattn_mamba2_chunkwise_fwd_workspace(int B, int T, int G, int H, int K, int V, int L) {
  (void)G;
  (void)K;
  (void)L;
  if (B <= 0 || T < 64 || T % 64 != 0 || H <= 0 || V <= 0) return 0;
  // the bf16 kernels cut the sequence into the most segments: their workspace
  // also covers the fp32 (bf16x3) kernels; HType.STRONG's segment-parallel walks
  // take the per-segment block sums
  const size_t a = hattn_mamba2_fwd_ws_bytes(B, T, H, V, 0);
  const size_t b = hattn_mamba2_fwd_ws_bytes(B, T, H, V, 1);
  const size_t c = hattn_mamba2_strong_fwd_ws_bytes(B, T, H, V);
  return max_of({a, b, c});
}

}  // extern "C"

// The forward behind both entry points.  noalloc: the workspace is the static
// scratch of hattn_mamba2_chunkwise_fwd_noalloc, looked up (and its capacity
// checked) after every other check, so a bad shape reports the same status
// through either entry point.
static int mamba2_fwd_impl(const void* q, const void* k, const void* v, const float* g,
                           const void* l, void* o, float* g_cumsum, float* ht, int B, int T,
                           int G, int H, int K, int V, int L, int dtype_qk, int dtype_v,
                           int dtype_l, int dtype_o, int level_base, int htype, int chunk_size,
                           void* workspace, size_t workspace_bytes, bool noalloc, void* stream) {
  if (chunk_size != 64)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "chunk_size=%d (only 64 is supported)", chunk_size);
  if (level_base != 2)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "level_base=%d (only 2 is supported)", level_base);
  if (htype != HATTN_HTYPE_WEAK && htype != HATTN_HTYPE_STRONG)
    return fail(HATTN_ERR_VALUE, "htype=%d", htype);
  if (B <= 0 || H <= 0 || G <= 0 || K <= 0 || V <= 0 || L <= 0)
    return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (T < 64 || T % 64 != 0) return fail(HATTN_ERR_VALUE, "T=%d and BT=64", T);
  if (H % G != 0) return fail(HATTN_ERR_VALUE, "H=%d is not a multiple of G=%d", H, G);
  if (V % 64 != 0) return fail(HATTN_ERR_VALUE, "V=%d and BV could be 64", V);
  if (K != 64) return fail(HATTN_ERR_NOT_IMPLEMENTED, "K=%d (the MI355X kernel supports 64)", K);
  const int NT = T / 64;
  const int nlev = ceil_log2(NT);
  if (7 + nlev > L)
    return fail(HATTN_ERR_VALUE, "L=%d levels < 7 + ceil(log2(T/64))=%d", L, 7 + nlev);
  if (htype == HATTN_HTYPE_STRONG) {
    // chunkwise.py:1118-1275 with USE_A2 / USE_H2
    if (nlev > hattn_mamba2_strong_max_levels())
      return fail(HATTN_ERR_NOT_IMPLEMENTED, "T=%d exceeds 64 * 2^%d (HType.STRONG)", T,
                  hattn_mamba2_strong_max_levels());
    if (L > 32) return fail(HATTN_ERR_NOT_IMPLEMENTED, "L=%d > 32 (HType.STRONG)", L);
    if (dtype_qk != HATTN_BF16 || dtype_v != HATTN_BF16)
      return fail(HATTN_ERR_NOT_IMPLEMENTED, "HType.STRONG: q/k/v dtype codes %d/%d (bf16 required)",
                  dtype_qk, dtype_v);
    if (int st = check_span(T, max_of({(size_t)G * K * 2, (size_t)H * V * elem_bytes(dtype_o),
                                        (size_t)H * L * elem_bytes(dtype_l), (size_t)H * 4})))
      return st;
    if (!q || !k || !v || !g || !l || !o || !g_cumsum)
      return fail(HATTN_ERR_VALUE, "null tensor pointer");
    // segment-parallel walks when the workspace (or the static scratch) holds the
    // per-segment block sums, else one serial walk per row
    if (noalloc) {
      const size_t cap = hattn_mamba2_fwd_static_scratch_bytes();
      if (hattn_mamba2_strong_fwd_ws_bytes(B, T, H, V) <= cap) {
        const hipError_t e = hattn_mamba2_fwd_static_scratch(&workspace);
        if (e != hipSuccess) return check_hip(e, "static scratch address (hipGetSymbolAddress)");
        workspace_bytes = cap;
      } else {
        workspace = nullptr;
        workspace_bytes = 0;
      }
    }
    int unsupported = 0;
    hipError_t e = hattn_mamba2_strong_fwd_launch(q, k, v, g, l, o, g_cumsum, workspace,
                                                  workspace_bytes, B, T, G, H, V, L, dtype_l,
                                                  dtype_o, (hipStream_t)stream, &unsupported);
    if (unsupported)
      return fail(HATTN_ERR_NOT_IMPLEMENTED, "HType.STRONG: dtype combination l=%d o=%d", dtype_l,
                  dtype_o);
    if (e == hipSuccess && ht != nullptr)
      // the raw phase-0 state of each strong level (chunkwise.py:179-279)
      e = hattn_mamba2_strong_ht_launch(k, v, g, ht, B, T, G, H, V, L, (hipStream_t)stream);
    return check_hip(e, "hattn_mamba2_chunkwise_fwd (strong) launch");
  }
  if (dtype_qk != HATTN_BF16 && dtype_qk != HATTN_FP16 && dtype_qk != HATTN_FP32)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "q/k dtype code %d (bf16, fp16 or fp32 required)",
                dtype_qk);
  // fp32 q / k select the bf16x3 kernels (fp32-accurate products); fp16 q / k the
  // fused kernel on fp16 MFMA (fp16 or fp32 v and o, fp32 lambda)
  const int x3 = dtype_qk == HATTN_FP32;
  const int h16 = dtype_qk == HATTN_FP16;
  if (nlev > hattn_mamba2_fwd_max_levels(x3))
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "T=%d exceeds 64 * 2^%d%s", T,
                hattn_mamba2_fwd_max_levels(x3), x3 ? " in fp32" : "");
  // dtype combinations the kernels are instantiated for (checked again at dispatch)
  const bool bf_or_f32 = (dtype_v == HATTN_BF16 || dtype_v == HATTN_FP32) &&
                         (dtype_l == HATTN_BF16 || dtype_l == HATTN_FP32) &&
                         (dtype_o == HATTN_BF16 || dtype_o == HATTN_FP32);
  const bool h_or_f32 = (dtype_v == HATTN_FP16 || dtype_v == HATTN_FP32) &&
                        dtype_l == HATTN_FP32 && (dtype_o == HATTN_FP16 || dtype_o == HATTN_FP32);
  if (x3 ? !(dtype_v == HATTN_FP32 && dtype_l == HATTN_FP32 && dtype_o == HATTN_FP32)
         : h16 ? !h_or_f32 : !bf_or_f32)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype combination q/k=%d v=%d l=%d o=%d%s", dtype_qk,
                dtype_v, dtype_l, dtype_o,
                x3 ? " (fp32 q/k need fp32 v, lambda and o)"
                   : h16 ? " (fp16 q/k need fp16 or fp32 v and o, fp32 lambda)" : "");
  if (int st = check_span(T, max_of({(size_t)G * K * elem_bytes(dtype_qk),
                                      (size_t)H * V * elem_bytes(dtype_v),
                                      (size_t)H * V * elem_bytes(dtype_o),
                                      (size_t)H * L * elem_bytes(dtype_l), (size_t)H * 4})))
    return st;
  if (!q || !k || !v || !g || !l || !o) return fail(HATTN_ERR_VALUE, "null tensor pointer");
  const size_t need = hattn_mamba2_fwd_ws_bytes(B, T, H, V, x3);
  if (noalloc && need > 0) {
    const size_t cap = hattn_mamba2_fwd_static_scratch_bytes();
    if (need > cap)
      return fail(HATTN_ERR_VALUE,
                  "these sizes need %zu bytes of scratch, above the %zu-byte static scratch of "
                  "hattn_mamba2_chunkwise_fwd_noalloc (use hattn_mamba2_chunkwise_fwd)",
                  need, cap);
    const hipError_t e = hattn_mamba2_fwd_static_scratch(&workspace);
    if (e != hipSuccess) return check_hip(e, "static scratch address (hipGetSymbolAddress)");
    workspace_bytes = cap;
  }
  if (workspace_bytes < need || (need > 0 && workspace == nullptr))
    return fail(HATTN_ERR_VALUE, "workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  int unsupported = 0;
  hipError_t e = hattn_mamba2_fwd_launch(q, k, v, g, l, o, g_cumsum, ht, workspace, B, T, G, H,
                                         V, L, nlev, dtype_qk, dtype_v, dtype_l, dtype_o,
                                         (hipStream_t)stream, &unsupported);
  if (unsupported)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype combination q/k=%d v=%d l=%d o=%d%s", dtype_qk,
                dtype_v, dtype_l, dtype_o, x3 ? " (fp32 q/k need fp32 v, lambda and o)" : "");
  return check_hip(e, "hattn_mamba2_chunkwise_fwd launch");
}

extern "C" {

int hattn_mamba2_chunkwise_fwd(const void* q, const void* k, const void* v, const float* g,
                               const void* l, void* o, float* g_cumsum, float* ht, int B, int T,
                               int G, int H, int K, int V, int L, int dtype_qk, int dtype_v,
                               int dtype_l, int dtype_o, int level_base, int htype,
                               int chunk_size, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return mamba2_fwd_impl(q, k, v, g, l, o, g_cumsum, ht, B, T, G, H, K, V, L, dtype_qk, dtype_v,
                         dtype_l, dtype_o, level_base, htype, chunk_size, workspace,
                         workspace_bytes, false, stream);
}

int hattn_mamba2_chunkwise_fwd_noalloc(const void* q, const void* k, const void* v,
                                       const float* g, const void* l, void* o, float* g_cumsum,
                                       float* ht, int B, int T, int G, int H, int K, int V, int L,
                                       int dtype_qk, int dtype_v, int dtype_l, int dtype_o,
                                       int level_base, int htype, int chunk_size, void* stream) {
  // HType.STRONG takes no workspace; WEAK uses the static scratch, checked
  // against its capacity after the shape and dtype checks
  return mamba2_fwd_impl(q, k, v, g, l, o, g_cumsum, ht, B, T, G, H, K, V, L, dtype_qk, dtype_v,
                         dtype_l, dtype_o, level_base, htype, chunk_size, nullptr, 0, true,
                         stream);
}

int hattn_mamba2_chunkwise_fwd_status(const void* workspace, int B, int T, int H, int V,
                                      unsigned int* status, void* stream) {
  if (status == nullptr) return fail(HATTN_ERR_VALUE, "null status pointer");
  *status = 0;
  if (B <= 0 || T < 64 || T % 64 != 0 || H <= 0 || V <= 0 || V % 64 != 0)
    return fail(HATTN_ERR_VALUE, "sizes B=%d T=%d H=%d V=%d", B, T, H, V);
  if (workspace == nullptr) {
    if (hattn_mamba2_fwd_ws_bytes(B, T, H, V, 0) > 0)
      return fail(HATTN_ERR_VALUE, "null workspace for sizes that have one");
    return ok();
  }
  const unsigned int* word = hattn_mamba2_fwd_status_word(workspace, B, T, H, V);
  if (word == nullptr) return ok();   // one segment: no look-back
  hipError_t e = hipMemcpyAsync(status, word, sizeof(unsigned int), hipMemcpyDeviceToHost,
                                (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  return check_hip(e, "hattn_mamba2_chunkwise_fwd_status");
}

void hattn_debug_lookback(int spin_limit, int publish) {
  hattn_mamba2_fwd_set_lookback(spin_limit, publish);
}

size_t hattn_mamba2_chunkwise_bwd_workspace(int B, int T, int H, int K, int V, int L,
                                             int htype) {
  (void)K;
  (void)L;
  if (B <= 0 || T < 64 || T % 64 != 0 || H <= 0 || V <= 0) return 0;
  if (htype == HATTN_HTYPE_STRONG) return hattn_mamba2_strong_bwd_ws_bytes(B, T, H, ceil_log2(T / 64));
  return hattn_mamba2_bwd_ws_bytes(B, T, H, V, ceil_log2(T / 64));
}

// fwd_ws (or null): the workspace of the bf16 WEAK forward of the same inputs,
// whose segment summaries replace the backward's own summary pass
static int mamba2_bwd_impl(const void* q, const void* k, const void* v, const float* g_cumsum,
                           const void* l, const void* do_, void* dq, void* dk, void* dv,
                           float* dg, float* dl, int B, int T, int H, int K, int V, int L,
                           int dtype_qk, int dtype_v, int dtype_l, int dtype_do, int level_base,
                           int htype, int chunk_size, void* workspace, size_t workspace_bytes,
                           const void* fwd_ws, size_t fwd_ws_bytes, void* stream) {
  if (chunk_size != 64)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "chunk_size=%d (only 64 is supported)", chunk_size);
  if (level_base != 2)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "level_base=%d (only 2 is supported)", level_base);
  if (htype != HATTN_HTYPE_WEAK && htype != HATTN_HTYPE_STRONG)
    return fail(HATTN_ERR_VALUE, "htype=%d", htype);
  if (B <= 0 || H <= 0 || K <= 0 || V <= 0 || L <= 0)
    return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (T < 64 || T % 64 != 0) return fail(HATTN_ERR_VALUE, "T=%d and BT=64", T);
  if (K % 64 != 0 || V % 64 != 0)
    return fail(HATTN_ERR_VALUE, "K=%d, V=%d and BK, BV could be 64", K, V);
  if (K != 64 || V != 64)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "K=%d V=%d (the MI355X backward supports 64)", K, V);
  const int nlev = ceil_log2(T / 64);
  if (7 + nlev > L)
    return fail(HATTN_ERR_VALUE, "L=%d levels < 7 + ceil(log2(T/64))=%d", L, 7 + nlev);
  if (htype == HATTN_HTYPE_STRONG) {
    // chunkwise.py:1286-1597 with USE_A2 / USE_H2 (MODE_H2 = 3)
    if (nlev > hattn_mamba2_strong_max_levels())
      return fail(HATTN_ERR_NOT_IMPLEMENTED, "T=%d exceeds 64 * 2^%d (HType.STRONG)", T,
                  hattn_mamba2_strong_max_levels());
    if (dtype_qk != HATTN_BF16 || dtype_v != HATTN_BF16 || dtype_do != HATTN_BF16)
      return fail(HATTN_ERR_NOT_IMPLEMENTED,
                  "HType.STRONG: q/k, v, do dtype codes %d/%d/%d (bf16 required)", dtype_qk,
                  dtype_v, dtype_do);
    if (int st = check_span(T, max_of({(size_t)H * K * 2, (size_t)H * V * 2,
                                        (size_t)H * L * elem_bytes(dtype_l), (size_t)H * 4})))
      return st;
    if (!q || !k || !v || !g_cumsum || !l || !do_ || !dq || !dk || !dv || !dg || !dl)
      return fail(HATTN_ERR_VALUE, "null tensor pointer");
    const size_t need = hattn_mamba2_strong_bwd_ws_bytes(B, T, H, nlev);
    if (workspace_bytes < need || workspace == nullptr)
      return fail(HATTN_ERR_VALUE, "workspace of %zu bytes is smaller than the %zu required",
                  workspace_bytes, need);
    int unsupported = 0;
    hipError_t e = hattn_mamba2_strong_bwd_launch(q, k, v, g_cumsum, l, do_, dq, dk, dv, dg, dl,
                                                  workspace, B, T, H, L, nlev, dtype_l,
                                                  (hipStream_t)stream, &unsupported);
    if (unsupported)
      return fail(HATTN_ERR_NOT_IMPLEMENTED, "HType.STRONG: lambda dtype code %d", dtype_l);
    return check_hip(e, "hattn_mamba2_chunkwise_bwd (strong) launch");
  }
  if (nlev > hattn_mamba2_fwd_max_levels(0))
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "T=%d exceeds 64 * 2^%d", T,
                hattn_mamba2_fwd_max_levels(0));
  // bf16 q / k / dO: bf16 kernels; fp16: the same kernels on fp16 MFMA (fp16 or
  // fp32 v, fp32 lambda); fp32 q / k / dO: bf16x3 kernels (fp32 v and lambda)
  if (!((dtype_qk == HATTN_BF16 && dtype_do == HATTN_BF16) ||
        (dtype_qk == HATTN_FP16 && dtype_do == HATTN_FP16) ||
        (dtype_qk == HATTN_FP32 && dtype_do == HATTN_FP32)))
    return fail(HATTN_ERR_NOT_IMPLEMENTED,
                "q/k/do dtype codes %d/%d (bf16, fp16 or fp32, both alike)", dtype_qk, dtype_do);
  if (dtype_qk == HATTN_FP32 && !(dtype_v == HATTN_FP32 && dtype_l == HATTN_FP32))
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "fp32 q/k need fp32 v and lambda (v=%d l=%d)", dtype_v,
                dtype_l);
  if (dtype_qk == HATTN_FP16 &&
      !((dtype_v == HATTN_FP16 || dtype_v == HATTN_FP32) && dtype_l == HATTN_FP32))
    return fail(HATTN_ERR_NOT_IMPLEMENTED,
                "fp16 q/k need fp16 or fp32 v and fp32 lambda (v=%d l=%d)", dtype_v, dtype_l);
  if (int st = check_span(T, max_of({(size_t)H * K * elem_bytes(dtype_qk),
                                      (size_t)H * V * elem_bytes(dtype_v),
                                      (size_t)H * V * elem_bytes(dtype_do),
                                      (size_t)H * L * 4, (size_t)H * 4})))
    return st;
  if (!q || !k || !v || !g_cumsum || !l || !do_ || !dq || !dk || !dv || !dg || !dl)
    return fail(HATTN_ERR_VALUE, "null tensor pointer");
  const size_t need = hattn_mamba2_bwd_ws_bytes(B, T, H, V, nlev);
  if (workspace_bytes < need || workspace == nullptr)
    return fail(HATTN_ERR_VALUE, "workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  const float* fsums = nullptr;
  const float* fsegd = nullptr;
  if (fwd_ws != nullptr) {
    if (dtype_qk != HATTN_BF16)
      return fail(HATTN_ERR_NOT_IMPLEMENTED,
                  "forward summaries: q/k dtype code %d (the bf16 forward keeps them)", dtype_qk);
    const size_t fneed = hattn_mamba2_fwd_ws_bytes(B, T, H, V, 0);
    if (fwd_ws_bytes < fneed)
      return fail(HATTN_ERR_VALUE, "forward workspace of %zu bytes is smaller than the %zu its "
                  "forward used", fwd_ws_bytes, fneed);
    hattn_mamba2_fwd_ws_summaries(const_cast<void*>(fwd_ws), B, T, H, V, &fsums, &fsegd);
  }
  int unsupported = 0;
  hipError_t e = hattn_mamba2_bwd_launch(q, k, v, g_cumsum, l, do_, dq, dk, dv, dg, dl, workspace,
                                         fsums, fsegd, B, T, H, V, L, nlev, dtype_qk, dtype_v,
                                         dtype_l, (hipStream_t)stream, &unsupported);
  if (unsupported)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype combination v=%d l=%d", dtype_v, dtype_l);
  return check_hip(e, "hattn_mamba2_chunkwise_bwd launch");
}

int hattn_mamba2_chunkwise_bwd(const void* q, const void* k, const void* v, const float* g_cumsum,
                               const void* l, const void* do_, void* dq, void* dk, void* dv,
                               float* dg, float* dl, int B, int T, int H, int K, int V, int L,
                               int dtype_qk, int dtype_v, int dtype_l, int dtype_do,
                               int level_base, int htype, int chunk_size, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return mamba2_bwd_impl(q, k, v, g_cumsum, l, do_, dq, dk, dv, dg, dl, B, T, H, K, V, L,
                         dtype_qk, dtype_v, dtype_l, dtype_do, level_base, htype, chunk_size,
                         workspace, workspace_bytes, nullptr, 0, stream);
}

int hattn_mamba2_chunkwise_bwd_fwd_ws(const void* q, const void* k, const void* v,
                                      const float* g_cumsum, const void* l, const void* do_,
                                      void* dq, void* dk, void* dv, float* dg, float* dl, int B,
                                      int T, int H, int K, int V, int L, int dtype_qk,
                                      int dtype_v, int dtype_l, int dtype_do, int level_base,
                                      int htype, int chunk_size, void* workspace,
                                      size_t workspace_bytes, const void* fwd_workspace,
                                      size_t fwd_workspace_bytes, void* stream) {
  if (fwd_workspace == nullptr) return fail(HATTN_ERR_VALUE, "null forward workspace");
  if (htype != HATTN_HTYPE_WEAK)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "forward summaries: htype=%d (WEAK only)", htype);
  return mamba2_bwd_impl(q, k, v, g_cumsum, l, do_, dq, dk, dv, dg, dl, B, T, H, K, V, L,
                         dtype_qk, dtype_v, dtype_l, dtype_do, level_base, htype, chunk_size,
                         workspace, workspace_bytes, fwd_workspace, fwd_workspace_bytes, stream);
}

size_t hattn_gdn_chunkwise_fwd_workspace(int B, int T, int H, int K, int V, int L) {
  (void)L;
  if (B <= 0 || T < 64 || T % 64 != 0 || H <= 0 || K <= 0 || V <= 0) return 0;
  return hattn_gdn_fwd_ws_bytes(B, T, H, K, V);
}

// keep: also leave, in the workspace, what the backward's recompute would
// produce (hattn_gdn_chunkwise_fwd_keep)
static int gdn_fwd_impl(const void* q, const void* k, const void* v, const void* beta,
                        const float* g, const void* l, void* o, float* g_cumsum, void* Aw,
                        void* Au, float* ht, int B, int T, int H, int K, int V, int L,
                        int dtype_qkv, int dtype_beta, int dtype_l, int dtype_o, int level_base,
                        int htype, int chunk_size, int l2norm_qk, float qk_scale,
                        void* workspace, size_t workspace_bytes, bool keep, void* stream) {
  if (chunk_size != 64)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "chunk_size=%d (only 64 is supported)", chunk_size);
  if (level_base != 2)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "level_base=%d (only 2 is supported)", level_base);
  // HType.STRONG: the reference's strong chunkwise GDN path (strong intra-chunk
  // levels, levels >= 1, every chunk reading every level; chunkwise_hgdn.py:630,
  // 724-728, 782)
  if (htype != HATTN_HTYPE_WEAK && htype != HATTN_HTYPE_STRONG)
    return fail(HATTN_ERR_VALUE, "htype=%d", htype);
  if (B <= 0 || H <= 0 || K <= 0 || V <= 0 || L <= 0)
    return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (T < 64 || T % 64 != 0) return fail(HATTN_ERR_VALUE, "T=%d and BT=64", T);
  if (K > 256) return fail(HATTN_ERR_NOT_IMPLEMENTED, "K=%d > 256", K);
  if (K % 64 != 0 || V % 64 != 0)
    return fail(HATTN_ERR_VALUE, "K=%d, V=%d and BK, BV could be 64", K, V);
  if (!hattn_gdn_fwd_supports_k(K))
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "K=%d (the MI355X GDN forward supports 64, 128, 192, 256)",
                K);
  const int nlev = ceil_log2(T / 64);
  if (7 + nlev > L)
    return fail(HATTN_ERR_VALUE, "L=%d levels < 7 + ceil(log2(T/64))=%d", L, 7 + nlev);
  if (nlev > hattn_gdn_fwd_max_levels())
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "T=%d exceeds 64 * 2^%d", T, hattn_gdn_fwd_max_levels());
  if ((size_t)T * H * (K > V ? K : V) >= ((size_t)1 << 31))
    return fail(HATTN_ERR_VALUE, "T * H * max(K, V) = %zu exceeds 2^31", (size_t)T * H * (K > V ? K : V));
  // fp16 q/k/v (fp16 MFMA): HType.WEAK with fp32 beta / lambda and an fp16 o
  if (dtype_qkv != HATTN_BF16 && dtype_qkv != HATTN_FP16)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "q/k/v dtype code %d (bf16 or fp16 required)", dtype_qkv);
  if (keep && !(V == 64 || V == 128))
    return fail(HATTN_ERR_NOT_IMPLEMENTED,
                "V=%d: the kept buffers serve a backward in one V block (V in {64, 128})", V);
  if (keep && nlev > hattn_gdn_bwd_max_levels())
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "T=%d exceeds 64 * 2^%d (the backward's limit)", T,
                hattn_gdn_bwd_max_levels());
  if (!q || !k || !v || !beta || !g || !l || !o || !g_cumsum || !Aw || !Au)
    return fail(HATTN_ERR_VALUE, "null tensor pointer");
  const size_t need = keep ? hattn_gdn_fwd_keep_ws_bytes(B, T, H, K, V, nlev)
                           : hattn_gdn_fwd_ws_bytes(B, T, H, K, V);
  if (workspace_bytes < need || workspace == nullptr)
    return fail(HATTN_ERR_VALUE, "workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  int unsupported = 0;
  hipError_t e =
      (keep ? hattn_gdn_fwd_keep_launch : hattn_gdn_fwd_launch)(
          q, k, v, beta, g, l, o, g_cumsum, Aw, Au, ht, workspace, B, T, H, K, V, L, nlev,
          dtype_beta, dtype_l, dtype_o, l2norm_qk ? 1 : 0, qk_scale,
          htype == HATTN_HTYPE_STRONG ? 1 : 0, dtype_qkv == HATTN_FP16 ? 1 : 0,
          (hipStream_t)stream, &unsupported);
  if (unsupported)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype combination q/k/v=%d beta=%d l=%d o=%d%s",
                dtype_qkv, dtype_beta, dtype_l, dtype_o,
                dtype_qkv == HATTN_FP16 ? " (fp16 q/k/v need fp32 beta and lambda, an fp16 o and "
                                          "HType.WEAK)"
                                        : "");
  return check_hip(e, keep ? "hattn_gdn_chunkwise_fwd_keep launch" : "hattn_gdn_chunkwise_fwd launch");
}

int hattn_gdn_chunkwise_fwd(const void* q, const void* k, const void* v, const void* beta,
                            const float* g, const void* l, void* o, float* g_cumsum, void* Aw,
                            void* Au, float* ht, int B, int T, int H, int K, int V, int L,
                            int dtype_qkv, int dtype_beta, int dtype_l, int dtype_o,
                            int level_base, int htype, int chunk_size, int l2norm_qk,
                            float qk_scale, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return gdn_fwd_impl(q, k, v, beta, g, l, o, g_cumsum, Aw, Au, ht, B, T, H, K, V, L, dtype_qkv,
                      dtype_beta, dtype_l, dtype_o, level_base, htype, chunk_size, l2norm_qk,
                      qk_scale, workspace, workspace_bytes, false, stream);
}

size_t hattn_gdn_chunkwise_fwd_keep_workspace(int B, int T, int H, int K, int V, int L) {
  (void)L;
  if (B <= 0 || T < 64 || T % 64 != 0 || H <= 0 || K <= 0 || V <= 0) return 0;
  return hattn_gdn_fwd_keep_ws_bytes(B, T, H, K, V, ceil_log2(T / 64));
}

int hattn_gdn_chunkwise_fwd_keep(const void* q, const void* k, const void* v, const void* beta,
                                 const float* g, const void* l, void* o, float* g_cumsum,
                                 void* Aw, void* Au, float* ht, int B, int T, int H, int K, int V,
                                 int L, int dtype_qkv, int dtype_beta, int dtype_l, int dtype_o,
                                 int level_base, int htype, int chunk_size, int l2norm_qk,
                                 float qk_scale, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  return gdn_fwd_impl(q, k, v, beta, g, l, o, g_cumsum, Aw, Au, ht, B, T, H, K, V, L, dtype_qkv,
                      dtype_beta, dtype_l, dtype_o, level_base, htype, chunk_size, l2norm_qk,
                      qk_scale, workspace, workspace_bytes, true, stream);
}

size_t hattn_gdn_chunkwise_bwd_workspace(int B, int T, int H, int K, int V, int L) {
  (void)L;
  if (B <= 0 || T < 64 || T % 64 != 0 || H <= 0 || K <= 0 || V <= 0) return 0;
  return hattn_gdn_bwd_ws_bytes(B, T, H, K, V, ceil_log2(T / 64));
}

// fwd_ws != nullptr: q_new, W_new, K_new, U and the level states come from the
// workspace of hattn_gdn_chunkwise_fwd_keep (hattn_gdn_chunkwise_bwd_fwd_ws)
static int gdn_bwd_impl(const void* q, const void* k, const void* v, const void* beta,
                        const float* g_cumsum, const void* l, const void* do_, void* dq, void* dk,
                        void* dv, void* db, float* dg, float* dl, int B, int T, int H, int K,
                        int V, int L, int dtype_qkv, int dtype_beta, int dtype_l, int dtype_do,
                        int level_base, int htype, int chunk_size, int l2norm_qk,
                        float qk_scale, void* workspace, size_t workspace_bytes,
                        const void* fwd_ws, size_t fwd_ws_bytes, bool kept, void* stream) {
  // chunkwise_hgdn.py:818-858; HType.STRONG: the gradient of the strong forward
  // (level reads at every chunk for levels >= 1)
  if (chunk_size != 64)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "chunk_size=%d (only 64 is supported)", chunk_size);
  if (level_base != 2)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "level_base=%d (only 2 is supported)", level_base);
  if (htype != HATTN_HTYPE_WEAK && htype != HATTN_HTYPE_STRONG)
    return fail(HATTN_ERR_VALUE, "htype=%d", htype);
  if (B <= 0 || H <= 0 || K <= 0 || V <= 0 || L <= 0)
    return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (T < 64 || T % 64 != 0) return fail(HATTN_ERR_VALUE, "T=%d and BT=64", T);
  if (K > 256) return fail(HATTN_ERR_NOT_IMPLEMENTED, "K=%d > 256", K);
  if (K % 64 != 0 || V % 64 != 0)
    return fail(HATTN_ERR_VALUE, "K=%d, V=%d and BK, BV could be 64", K, V);
  if (!((K == 64 || K == 128 || K == 192 || K == 256) && (V == 64 || V == 128)))
    return fail(HATTN_ERR_NOT_IMPLEMENTED,
                "K=%d V=%d (the MI355X GDN backward supports K in {64, 128, 192, 256} and V in "
                "{64, 128}; the host driver splits larger V into blocks)", K, V);
  const int nlev = ceil_log2(T / 64);
  if (7 + nlev > L)
    return fail(HATTN_ERR_VALUE, "L=%d levels < 7 + ceil(log2(T/64))=%d", L, 7 + nlev);
  if (nlev > hattn_gdn_bwd_max_levels())
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "T=%d exceeds 64 * 2^%d", T, hattn_gdn_bwd_max_levels());
  if (!((dtype_qkv == HATTN_BF16 || dtype_qkv == HATTN_FP16) && dtype_do == dtype_qkv))
    return fail(HATTN_ERR_NOT_IMPLEMENTED,
                "q/k/v/do dtype codes %d/%d (bf16 or fp16, the same for all four)", dtype_qkv,
                dtype_do);
  if (!q || !k || !v || !beta || !g_cumsum || !l || !do_ || !dq || !dk || !dv || !db || !dg || !dl)
    return fail(HATTN_ERR_VALUE, "null tensor pointer");
  if (kept) {
    const size_t fneed = hattn_gdn_fwd_keep_ws_bytes(B, T, H, K, V, nlev);
    if (fwd_ws == nullptr || fwd_ws_bytes < fneed)
      return fail(HATTN_ERR_VALUE,
                  "forward workspace of %zu bytes is smaller than the %zu of the keeping forward",
                  fwd_ws_bytes, fneed);
  }
  const size_t need = kept ? hattn_gdn_bwd_kept_ws_bytes(B, T, H, K, V, nlev)
                           : hattn_gdn_bwd_ws_bytes(B, T, H, K, V, nlev);
  if (workspace_bytes < need || workspace == nullptr)
    return fail(HATTN_ERR_VALUE, "workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  int unsupported = 0;
  hipError_t e;
  if (kept) {
    const __bf16 *qn, *wn, *kn, *un, *hs;
    hattn_gdn_fwd_keep_buffers(fwd_ws, B, T, H, K, V, nlev, &qn, &wn, &kn, &un, &hs);
    e = hattn_gdn_bwd_kept_launch(q, k, v, beta, g_cumsum, l, do_, dq, dk, dv, db, dg, dl, qn, wn,
                                  kn, un, hs, workspace, B, T, H, K, V, L, nlev, dtype_beta,
                                  dtype_l, l2norm_qk ? 1 : 0, qk_scale,
                                  htype == HATTN_HTYPE_STRONG ? 1 : 0,
                                  dtype_qkv == HATTN_FP16 ? 1 : 0, (hipStream_t)stream,
                                  &unsupported);
  } else {
    e = hattn_gdn_bwd_launch(q, k, v, beta, g_cumsum, l, do_, dq, dk, dv, db, dg, dl, workspace,
                             B, T, H, K, V, L, nlev, dtype_beta, dtype_l, l2norm_qk ? 1 : 0,
                             qk_scale, htype == HATTN_HTYPE_STRONG ? 1 : 0,
                             dtype_qkv == HATTN_FP16 ? 1 : 0, (hipStream_t)stream, &unsupported);
  }
  if (unsupported)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype combination q/k/v=%d beta=%d l=%d%s", dtype_qkv,
                dtype_beta, dtype_l,
                dtype_qkv == HATTN_FP16 ? " (fp16 q/k/v need fp32 beta and lambda and HType.WEAK)"
                                        : "");
  return check_hip(e, kept ? "hattn_gdn_chunkwise_bwd_fwd_ws launch" : "hattn_gdn_chunkwise_bwd launch");
}

int hattn_gdn_chunkwise_bwd(const void* q, const void* k, const void* v, const void* beta,
                            const float* g_cumsum, const void* l, const void* Aw, const void* Au,
                            const void* do_, void* dq, void* dk, void* dv, void* db, float* dg,
                            float* dl, int B, int T, int H, int K, int V, int L, int dtype_qkv,
                            int dtype_beta, int dtype_l, int dtype_do, int level_base, int htype,
                            int chunk_size, int l2norm_qk, float qk_scale, void* workspace,
                            size_t workspace_bytes, void* stream) {
  (void)Aw;
  (void)Au;
  return gdn_bwd_impl(q, k, v, beta, g_cumsum, l, do_, dq, dk, dv, db, dg, dl, B, T, H, K, V, L,
                      dtype_qkv, dtype_beta, dtype_l, dtype_do, level_base, htype, chunk_size,
                      l2norm_qk, qk_scale, workspace, workspace_bytes, nullptr, 0, false, stream);
}

size_t hattn_gdn_chunkwise_bwd_fwd_ws_workspace(int B, int T, int H, int K, int V, int L) {
  (void)L;
  if (B <= 0 || T < 64 || T % 64 != 0 || H <= 0 || K <= 0 || V <= 0) return 0;
  return hattn_gdn_bwd_kept_ws_bytes(B, T, H, K, V, ceil_log2(T / 64));
}

int hattn_gdn_chunkwise_bwd_fwd_ws(const void* q, const void* k, const void* v, const void* beta,
                                   const float* g_cumsum, const void* l, const void* Aw,
                                   const void* Au, const void* do_, void* dq, void* dk, void* dv,
                                   void* db, float* dg, float* dl, int B, int T, int H, int K,
                                   int V, int L, int dtype_qkv, int dtype_beta, int dtype_l,
                                   int dtype_do, int level_base, int htype, int chunk_size,
                                   int l2norm_qk, float qk_scale, void* workspace,
                                   size_t workspace_bytes, const void* fwd_workspace,
                                   size_t fwd_workspace_bytes, void* stream) {
  (void)Aw;
  (void)Au;
  return gdn_bwd_impl(q, k, v, beta, g_cumsum, l, do_, dq, dk, dv, db, dg, dl, B, T, H, K, V, L,
                      dtype_qkv, dtype_beta, dtype_l, dtype_do, level_base, htype, chunk_size,
                      l2norm_qk, qk_scale, workspace, workspace_bytes, fwd_workspace,
                      fwd_workspace_bytes, true, stream);
}

int hattn_hstate_step(float* states, int* counts, const void* q, const void* k, const void* v,
                      const void* beta, const float* g, const void* l, void* o, int B, int G,
                      int H, int K, int V, int L, int hstruct, int htype, int cascade, int update,
                      int output, int l2norm_qk, float scale, int dtype_qk, int dtype_v,
                      int dtype_l, int dtype_beta, void* stream) {
  if (B <= 0 || G <= 0 || H <= 0 || K <= 0 || V <= 0 || L <= 0)
    return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (H % G != 0) return fail(HATTN_ERR_VALUE, "G=%d does not divide H=%d", G, H);
  if (hstruct != HATTN_HSTRUCT_MAMBA2 && hstruct != HATTN_HSTRUCT_GDELTA)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "hstruct=%d", hstruct);
  if (K > 256 || V % 16 != 0 || L > 32)
    return fail(HATTN_ERR_NOT_IMPLEMENTED,
                "K=%d V=%d L=%d (K <= 256, V a multiple of 16, L <= 32)", K, V, L);
  if (htype != HATTN_HTYPE_WEAK && htype != HATTN_HTYPE_STRONG)
    return fail(HATTN_ERR_VALUE, "htype=%d", htype);
  if (htype == HATTN_HTYPE_WEAK && (cascade < 0 || cascade >= L))
    return fail(HATTN_ERR_VALUE, "cascade depth %d with %d levels (level overflow)", cascade, L);
  if (htype == HATTN_HTYPE_STRONG && update && (cascade < 1 || cascade > L))
    return fail(HATTN_ERR_VALUE, "strong cascade merge level %d with %d levels", cascade, L);
  if (!states || (output && (!q || !l || !o)) ||
      (update && (!k || !v || !g || (hstruct == HATTN_HSTRUCT_GDELTA && !beta))))
    return fail(HATTN_ERR_VALUE, "null tensor pointer");
  int unsupported = 0;
  hipError_t e = hattn_hstate_step_launch(
      states, counts, q, k, v, beta, g, l, o, B, G, H, K, V, L,
      hstruct == HATTN_HSTRUCT_GDELTA ? 1 : 0, update ? cascade : 0,
      (htype == HATTN_HTYPE_STRONG && update) ? 1 : 0,
      update ? 1 : 0, output ? 1 : 0,
      l2norm_qk ? 1 : 0, scale, dtype_qk, dtype_v, dtype_l, dtype_beta, (hipStream_t)stream,
      &unsupported);
  if (unsupported)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype codes qk=%d v=%d l=%d beta=%d", dtype_qk,
                dtype_v, dtype_l, dtype_beta);
  return check_hip(e, "hattn_hstate_step launch");
}

int hattn_mamba2_prefill_levels(float* states, const void* k, const void* v, const float* g,
                                int B, int T, int G, int H, int K, int V, int L, int nlo,
                                int dtype_k, int dtype_v, void* stream) {
  if (B <= 0 || G <= 0 || H <= 0 || K <= 0 || V <= 0 || L <= 0)
    return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (H % G != 0) return fail(HATTN_ERR_VALUE, "G=%d does not divide H=%d", G, H);
  if (T < 64 || T % 64 != 0) return fail(HATTN_ERR_VALUE, "T=%d is not a positive multiple of 64", T);
  if (nlo < 1 || nlo > 7 || nlo > L) return fail(HATTN_ERR_VALUE, "nlo=%d with L=%d", nlo, L);
  if (K > 256 || V % 16 != 0)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "K=%d V=%d (K <= 256, V a multiple of 16)", K, V);
  if (!states || !k || !v || !g) return fail(HATTN_ERR_VALUE, "null tensor pointer");
  int unsupported = 0;
  hipError_t e = hattn_mamba2_prefill_levels_launch(states, k, v, g, B, T, G, H, K, V, L, nlo,
                                                    dtype_k, dtype_v, (hipStream_t)stream,
                                                    &unsupported);
  if (unsupported)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype codes k=%d v=%d", dtype_k, dtype_v);
  return check_hip(e, "hattn_mamba2_prefill_levels launch");
}

namespace {
// dtype code -> 1 for bf16, 0 for fp32, -1 otherwise
int bf_flag(int code) { return code == HATTN_BF16 ? 1 : code == HATTN_FP32 ? 0 : -1; }
bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
int layer_dims_check(int B, int T, int H, int P, int L) {
  if (B <= 0 || T <= 0 || H <= 0 || P <= 0 || L <= 0)
    return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (P % 4 != 0 || (P / 4) > 64 || ((P / 4) & (P / 4 - 1)) != 0)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "P=%d (a multiple of 4 with P/4 a power of two <= 64)", P);
  if (L > 32) return fail(HATTN_ERR_NOT_IMPLEMENTED, "L=%d above 32", L);
  // the elementwise kernels index elements in 32 bits
  if ((long long)B * T * H * (P > L ? P : L) >= (1LL << 31))
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "B*T*H*max(P, L) = %lld elements (below 2^31)",
                (long long)B * T * H * (P > L ? P : L));
  return HATTN_OK;
}
}  // namespace

int hattn_mamba2_layer_prologue(const void* x, const void* dt, const float* A,
                                const float* dt_bias, const void* dl, const void* Lp, void* v,
                                float* g, void* lam, int B, int T, int H, int P, int L,
                                int dt_softplus, int lambda_mode, int dtype_x, int dtype_dt,
                                int dtype_dl, int dtype_lp, int dtype_v, int dtype_lam,
                                void* stream) {
  if (int st = layer_dims_check(B, T, H, P, L)) return st;
  if (lambda_mode < 0 || lambda_mode > 2) return fail(HATTN_ERR_VALUE, "lambda_mode=%d", lambda_mode);
  if (!x || !dt || !A || !dl || !Lp || !v || !g || !lam) return fail(HATTN_ERR_VALUE, "null tensor pointer");
  if (!aligned16(x) || !aligned16(v)) return fail(HATTN_ERR_VALUE, "x / v not 16-byte aligned");
  const int bf[6] = {bf_flag(dtype_x), bf_flag(dtype_dt), bf_flag(dtype_dl), bf_flag(dtype_lp),
                     bf_flag(dtype_v), bf_flag(dtype_lam)};
  for (int i = 0; i < 6; ++i)
    if (bf[i] < 0) return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype code (bf16 or fp32 only)");
  return check_hip(hattn_mamba2_layer_prologue_launch(x, dt, A, dt_bias, dl, Lp, v, g, lam, B, T,
                                                      H, P, L, dt_softplus ? 1 : 0, lambda_mode,
                                                      bf, (hipStream_t)stream),
                   "hattn_mamba2_layer_prologue launch");
}

int hattn_mamba2_layer_epilogue(const void* y, const void* x, const float* D, void* out, int B,
                                int T, int H, int P, int dtype_y, int dtype_x, int dtype_out,
                                void* stream) {
  if (int st = layer_dims_check(B, T, H, P, 1)) return st;
  if (!y || !x || !D || !out) return fail(HATTN_ERR_VALUE, "null tensor pointer");
  if (!aligned16(y) || !aligned16(x) || !aligned16(out))
    return fail(HATTN_ERR_VALUE, "y / x / out not 16-byte aligned");
  const int yb = bf_flag(dtype_y), xb = bf_flag(dtype_x), ob = bf_flag(dtype_out);
  if (yb < 0 || xb < 0 || ob < 0) return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype code (bf16 or fp32 only)");
  return check_hip(hattn_mamba2_layer_epilogue_launch(y, x, D, out, B, T, H, P, yb, xb, ob,
                                                      (hipStream_t)stream),
                   "hattn_mamba2_layer_epilogue launch");
}

int hattn_mamba2_layer_scan_fwd(const void* x, const void* dt, const float* A,
                                const float* dt_bias, const void* Bm, const void* Cm,
                                const void* dl, const float* Lp, const float* D, void* y,
                                float* g_cumsum, int B, int T, int G, int H, int P, int N, int L,
                                int dtype_x, int dtype_dt, int dtype_bc, int dtype_dl,
                                int dtype_lam, int dtype_y, int dt_softplus, int lambda_mode,
                                int level_base, int htype, int chunk_size, void* workspace,
                                size_t workspace_bytes, void* stream) {
  // mamba_apis.py:263-404 (the layer scan of hmamba_chunk_scan_combined, no final state)
  if (chunk_size != 64)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "chunk_size=%d (only 64 is supported)", chunk_size);
  if (level_base != 2)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "level_base=%d (only 2 is supported)", level_base);
  if (htype != HATTN_HTYPE_WEAK)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "the folded layer scan runs HType.WEAK only");
  if (B <= 0 || T <= 0 || G <= 0 || H <= 0 || P <= 0 || N <= 0 || L <= 0)
    return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (T % 64 != 0) return fail(HATTN_ERR_VALUE, "T=%d and BT=64", T);
  if (H % G != 0) return fail(HATTN_ERR_VALUE, "H=%d is not a multiple of G=%d", H, G);
  if (P % 64 != 0) return fail(HATTN_ERR_VALUE, "P=%d and BV could be 64", P);
  if (N != 64) return fail(HATTN_ERR_NOT_IMPLEMENTED, "N=%d (the folded layer scan takes 64)", N);
  if (lambda_mode < 0 || lambda_mode > 2) return fail(HATTN_ERR_VALUE, "lambda_mode=%d", lambda_mode);
  const int nlev = ceil_log2(T / 64);
  if (7 + nlev > L)
    return fail(HATTN_ERR_VALUE, "L=%d levels < 7 + ceil(log2(T/64))=%d", L, 7 + nlev);
  if (nlev > hattn_mamba2_fwd_max_levels(0))
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "T=%d exceeds 64 * 2^%d", T, hattn_mamba2_fwd_max_levels(0));
  if (L > 32) return fail(HATTN_ERR_NOT_IMPLEMENTED, "L=%d > 32 (folded layer scan)", L);
  if (dtype_x != HATTN_BF16 || dtype_bc != HATTN_BF16)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "x / B / C dtype codes %d / %d (bf16 required)",
                dtype_x, dtype_bc);
  const int dtb = bf_flag(dtype_dt), lb = bf_flag(dtype_lam);
  if (dtb < 0 || lb < 0 || bf_flag(dtype_dl) < 0 || bf_flag(dtype_y) < 0)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype code (bf16 or fp32 only)");
  if (int st = check_span(T, max_of({(size_t)G * N * 2, (size_t)H * P * elem_bytes(dtype_y),
                                      (size_t)H * L * elem_bytes(dtype_dl), (size_t)H * 4})))
    return st;
  if (!x || !dt || !A || !Bm || !Cm || !dl || !Lp || !y || !g_cumsum)
    return fail(HATTN_ERR_VALUE, "null tensor pointer");
  const size_t need = hattn_mamba2_fwd_ws_bytes(B, T, H, P, 0);
  if (need > 0 && (workspace_bytes < need || workspace == nullptr))
    return fail(HATTN_ERR_VALUE, "workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  int unsupported = 0;
  hipError_t e = hattn_mamba2_layer_fwd_launch(
      Cm, Bm, x, dl, y, g_cumsum, workspace, dt, A, dt_bias, Lp, D, dtb ? 0 : 1,
      dt_softplus ? 1 : 0, lambda_mode, lb, B, T, G, H, P, L, nlev, dtype_dl, dtype_y,
      (hipStream_t)stream, &unsupported);
  if (unsupported)
    return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype combination dl=%d y=%d", dtype_dl, dtype_y);
  return check_hip(e, "hattn_mamba2_layer_scan_fwd launch");
}

size_t hattn_mamba2_layer_bwd_workspace(int B, int T, int H, int L) {
  if (B <= 0 || T <= 0 || H <= 0 || L <= 0 || L > 32) return 0;
  return hattn_mamba2_layer_bwd_ws_bytes(B, T, H, L);
}

int hattn_mamba2_layer_bwd(const void* x, const void* dt, const float* A, const float* dt_bias,
                           const void* dl, const void* Lp, const float* D, const void* dy,
                           const void* dv, const float* dg, const void* dlam, void* dx,
                           void* ddt, void* ddl, float* dA, float* ddt_bias, float* dD,
                           float* dLp, int B, int T, int H, int P, int L, int dt_softplus,
                           int lambda_mode, int dtype_x, int dtype_dt, int dtype_dl,
                           int dtype_lp, int dtype_dy, int dtype_dv, int dtype_dlam,
                           int dtype_dx, int dtype_ddt, int dtype_ddl, void* ws,
                           size_t ws_bytes, void* stream) {
  if (int st = layer_dims_check(B, T, H, P, L)) return st;
  if (lambda_mode < 0 || lambda_mode > 2) return fail(HATTN_ERR_VALUE, "lambda_mode=%d", lambda_mode);
  if (!x || !dt || !A || !dl || !Lp || !dv || !dg || !dlam || !dx || !ddt || !ddl ||
      (D && !dy))
    return fail(HATTN_ERR_VALUE, "null tensor pointer");
  if (!aligned16(x) || !aligned16(dv) || !aligned16(dx) || (D && !aligned16(dy)))
    return fail(HATTN_ERR_VALUE, "x / dv / dx / dy not 16-byte aligned");
  const size_t need = hattn_mamba2_layer_bwd_ws_bytes(B, T, H, L);
  if (!ws || ws_bytes < need)
    return fail(HATTN_ERR_VALUE, "workspace of %zu bytes, %zu needed", ws_bytes, need);
  const int bf[10] = {bf_flag(dtype_x), bf_flag(dtype_dt), bf_flag(dtype_dl), bf_flag(dtype_lp),
                      bf_flag(dtype_dy), bf_flag(dtype_dv), bf_flag(dtype_dlam), bf_flag(dtype_dx),
                      bf_flag(dtype_ddt), bf_flag(dtype_ddl)};
  for (int i = 0; i < 10; ++i)
    if (bf[i] < 0 && !(i == 4 && !D)) return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype code (bf16 or fp32 only)");
  int bfx[10];
  for (int i = 0; i < 10; ++i) bfx[i] = bf[i] < 0 ? 0 : bf[i];
  return check_hip(hattn_mamba2_layer_bwd_launch(x, dt, A, dt_bias, dl, Lp, D, dy, dv, dg, dlam, dx,
                                                 ddt, ddl, dA, ddt_bias, dD, dLp, (float*)ws, B,
                                                 T, H, P, L, dt_softplus ? 1 : 0, lambda_mode, bfx,
                                                 (hipStream_t)stream),
                   "hattn_mamba2_layer_bwd launch");
}

namespace {
int flags(const int* codes, int* out, int n) {
  for (int i = 0; i < n; ++i) {
    out[i] = bf_flag(codes[i]);
    if (out[i] < 0) return fail(HATTN_ERR_NOT_IMPLEMENTED, "dtype code %d (bf16 or fp32 only)", codes[i]);
  }
  return HATTN_OK;
}
int conv_check(int B, int S, int Dc, int d1, int d2, int W, long long ld, long long col0) {
  if (B <= 0 || S <= 0 || Dc <= 0 || W <= 0) return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (W > 8) return fail(HATTN_ERR_NOT_IMPLEMENTED, "conv width %d above 8", W);
  if ((long long)B * S >= (1LL << 31)) return fail(HATTN_ERR_NOT_IMPLEMENTED, "B*S above 2^31 - 1");
  if (!(0 <= d1 && d1 <= d2 && d2 <= Dc)) return fail(HATTN_ERR_VALUE, "channel split %d %d of %d", d1, d2, Dc);
  if (col0 < 0 || ld < col0 + Dc) return fail(HATTN_ERR_VALUE, "row stride %lld too small", ld);
  return HATTN_OK;
}
}  // namespace

int hattn_causal_conv1d_silu_fwd(const void* in, long long ld, long long col0, const void* weight,
                                 const void* bias, void* out0, void* out1, void* out2, int B,
                                 int S, int Dc, int d1, int d2, int W, int dtype_in,
                                 int dtype_w, int dtype_out, void* stream) {
  if (int st = conv_check(B, S, Dc, d1, d2, W, ld, col0)) return st;
  if (!in || !weight || (d1 > 0 && !out0) || (d2 > d1 && !out1) || (Dc > d2 && !out2))
    return fail(HATTN_ERR_VALUE, "null tensor pointer");
  const int codes[3] = {dtype_in, dtype_w, dtype_out};
  int f[3];
  if (int st = flags(codes, f, 3)) return st;
  return check_hip(hattn_conv1d_silu_fwd_launch(in, (long)ld, (long)col0, weight, bias, out0, out1,
                                                out2, B, S, Dc, d1, d2, W, f[0], f[1], f[2],
                                                (hipStream_t)stream),
                   "hattn_causal_conv1d_silu_fwd launch");
}

size_t hattn_causal_conv1d_silu_bwd_workspace(int B, int S, int Dc, int W) {
  if (B <= 0 || S <= 0 || Dc <= 0 || W <= 0 || W > 8) return 0;
  return hattn_conv1d_bwd_ws_bytes(B, S, Dc, W);
}

int hattn_causal_conv1d_silu_bwd(const void* in, long long ld, long long col0,
                                 const void* weight, const void* bias, const void* g0,
                                 const void* g1, const void* g2, void* din, long long ldo,
                                 long long colo, float* dweight, float* dbias, int B, int S,
                                 int Dc, int d1, int d2, int W, int dtype_in, int dtype_w,
                                 int dtype_g0, int dtype_g1, int dtype_g2, int dtype_din,
                                 void* ws, size_t ws_bytes, void* stream) {
  if (int st = conv_check(B, S, Dc, d1, d2, W, ld, col0)) return st;
  if (colo < 0 || ldo < colo + Dc) return fail(HATTN_ERR_VALUE, "gradient row stride %lld too small", ldo);
  if (!in || !weight || !din || (d1 > 0 && !g0) || (d2 > d1 && !g1) || (Dc > d2 && !g2))
    return fail(HATTN_ERR_VALUE, "null tensor pointer");
  const size_t need = hattn_conv1d_bwd_ws_bytes(B, S, Dc, W);
  if (!ws || ws_bytes < need) return fail(HATTN_ERR_VALUE, "workspace of %zu bytes, %zu needed", ws_bytes, need);
  const int codes[6] = {dtype_in, dtype_w, d1 > 0 ? dtype_g0 : HATTN_FP32,
                        d2 > d1 ? dtype_g1 : HATTN_FP32, Dc > d2 ? dtype_g2 : HATTN_FP32, dtype_din};
  int f[6];
  if (int st = flags(codes, f, 6)) return st;
  return check_hip(hattn_conv1d_silu_bwd_launch(in, (long)ld, (long)col0, weight, bias, g0, g1, g2, din,
                                                (long)ldo, (long)colo, dweight, dbias, (float*)ws, B, S,
                                                Dc, d1, d2, W, f[0], f[1], f[2], f[3], f[4], f[5],
                                                (hipStream_t)stream),
                   "hattn_causal_conv1d_silu_bwd launch");
}

int hattn_gated_rmsnorm_fwd(const void* y, const void* z, long long ldz, const void* weight,
                            void* out, float* rstd, long long rows, int n, float eps,
                            int dtype_y, int dtype_z, int dtype_w, int dtype_out, void* stream) {
  if (rows <= 0 || n <= 0) return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (ldz < n) return fail(HATTN_ERR_VALUE, "z row stride %lld below n=%d", ldz, n);
  if (!y || !z || !weight || !out || !rstd) return fail(HATTN_ERR_VALUE, "null tensor pointer");
  const int codes[4] = {dtype_y, dtype_z, dtype_w, dtype_out};
  int f[4];
  if (int st = flags(codes, f, 4)) return st;
  return check_hip(hattn_gated_rmsnorm_fwd_launch(y, z, (long)ldz, weight, out, rstd, (long)rows, n,
                                                  eps, f[0], f[1], f[2], f[3], (hipStream_t)stream),
                   "hattn_gated_rmsnorm_fwd launch");
}

size_t hattn_gated_rmsnorm_bwd_workspace(long long rows, int n) {
  if (rows <= 0 || n <= 0) return 0;
  return hattn_rmsnorm_bwd_ws_bytes((long)rows, n);
}

int hattn_gated_rmsnorm_bwd(const void* y, const void* z, long long ldz, const void* weight,
                            const float* rstd, const void* dout, void* dy, void* dz,
                            long long lddz, float* dweight, long long rows, int n, int dtype_y,
                            int dtype_z, int dtype_w, int dtype_dout, int dtype_dy,
                            int dtype_dz, void* ws, size_t ws_bytes, void* stream) {
  if (rows <= 0 || n <= 0) return fail(HATTN_ERR_VALUE, "non-positive dimension");
  if (ldz < n || lddz < n) return fail(HATTN_ERR_VALUE, "row stride below n=%d", n);
  if (n > 8192) return fail(HATTN_ERR_NOT_IMPLEMENTED, "n=%d above 8192", n);
  if (!y || !z || !weight || !rstd || !dout || !dy || !dz || !dweight)
    return fail(HATTN_ERR_VALUE, "null tensor pointer");
  const size_t need = hattn_rmsnorm_bwd_ws_bytes((long)rows, n);
  if (!ws || ws_bytes < need) return fail(HATTN_ERR_VALUE, "workspace of %zu bytes, %zu needed", ws_bytes, need);
  const int codes[6] = {dtype_y, dtype_z, dtype_w, dtype_dout, dtype_dy, dtype_dz};
  int f[6];
  if (int st = flags(codes, f, 6)) return st;
  return check_hip(hattn_gated_rmsnorm_bwd_launch(y, z, (long)ldz, weight, rstd, dout, dy, dz,
                                                  (long)lddz, dweight, (float*)ws, (long)rows, n,
                                                  f[0], f[1], f[2], f[3], f[4], f[5],
                                                  (hipStream_t)stream),
                   "hattn_gated_rmsnorm_bwd launch");
}

}  // extern "C"
