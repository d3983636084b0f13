/*
 * hattn.h -- C-ABI of libhattn_hip.so, the MI355X (gfx950) chunkwise path of
 * log-linear (Fenwick-tree hierarchical) attention.
 *
 * Every entry point takes plain device pointers, sizes and dtype codes, runs
 * stream-ordered on the caller's HIP stream, never allocates, frees or
 * synchronises, and returns an hattn_status.  Tensors are time-first and
 * contiguous (the reference's head_first=False layout):
 *
 *   q, k   [B, T, G, K]        G divides H (head h reads group h / (H / G))
 *   v, o   [B, T, H, V]
 *   g      [B, T, H]   fp32    per-step log-decay
 *   l      [B, T, H, L]        level weights lambda (linear)
 *   ht     [B, H, K, V, L] fp32 final per-level states
 *
 * The caller (the Python host layer, or any FFI binding) allocates every
 * output.  A failed call leaves a message retrievable with hattn_last_error()
 * (thread-local) and returns the status the reference's Python would have
 * raised as an exception (see hattn_status).
 */
#ifndef HATTN_H_
#define HATTN_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The Python layer maps them to the exception types the
 * reference raises for the same condition. */
typedef enum {
  HATTN_OK = 0,
  HATTN_ERR_VALUE = 1,           /* ValueError (chunkwise.py:1140-1153, 1211-1214) */
  HATTN_ERR_NOT_IMPLEMENTED = 2, /* NotImplementedError (kernel.py:55-123) */
  HATTN_ERR_HIP = 3              /* HIP runtime error (launch / attribute) */
} hattn_status;

/* Element types of the tensors crossing the boundary. */
typedef enum { HATTN_BF16 = 0, HATTN_FP16 = 1, HATTN_FP32 = 2 } hattn_dtype;

/* HType / HStruct of hattention/base.py:12-19. */
enum { HATTN_HTYPE_WEAK = 0, HATTN_HTYPE_STRONG = 1 };
enum { HATTN_HSTRUCT_MAMBA2 = 0, HATTN_HSTRUCT_GDELTA = 1 };

/* Library version string, e.g. "hattn-mi355x 0.1.0 gfx950". */
const char* hattn_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* hattn_last_error(void);

/*
 * Log-linear Mamba-2 chunkwise forward.
 *
 * Replaces hattention/chunkwise.py:1118-1275 `chunkwise_fwd(q, k, v, g, l,
 * head_first, level_base, htype, chunk_size, output_final_state)
 * -> (o, g_cumsum, ht)`, the function HAttentionFunction.forward calls for
 * HStruct.MAMBA2 with chunkwise=True (kernel.py:77-98).
 *
 *   o         [B, T, H, V] in dtype_o (the reference allocates it in v.dtype)
 *   g_cumsum  [B, T, H] fp32 chunk-local inclusive cumsum of g, or NULL
 *             (the reference returns it and saves it for backward)
 *   ht        [B, H, K, V, L] fp32 final inter-chunk level states (levels
 *             7 .. 6 + ceil(log2(T / 64))), or NULL for output_final_state=False.
 *             Levels not written by the kernel are left untouched (the
 *             reference zero-initialises ht, chunkwise.py:1179).
 *   workspace device scratch of at least
 *             hattn_mamba2_chunkwise_fwd_workspace(...) bytes (may be NULL
 *             when that is 0); contents on entry are ignored.  HType.STRONG
 *             takes any size: with the full size its chunk walks run per
 *             32-chunk segment in parallel (per-segment block sums in the
 *             workspace), with less one serial walk per row.
 *
 * Constraints (status on violation):
 *   T % 64 == 0, T >= 64, H % G == 0, L >= 7 + ceil(log2(T / 64)),
 *   V % 64 == 0, workspace large enough               -> HATTN_ERR_VALUE
 *   htype not HATTN_HTYPE_WEAK / HATTN_HTYPE_STRONG  -> HATTN_ERR_VALUE
 *   chunk_size == 64, level_base == 2, K == 64 (the Python host layer runs a
 *   larger K as one call per 64-wide block of q and k and sums the outputs),
 *   dtype_qk BF16 (bf16 MFMA; dtype_v / dtype_l / dtype_o in {BF16, FP32}),
 *   FP16 (fp16 MFMA, HType.WEAK: dtype_v / dtype_o in {FP16, FP32}, dtype_l
 *   FP32) or FP32 (bf16x3, fp32-accurate; v, l, o FP32)
 *                                                    -> HATTN_ERR_NOT_IMPLEMENTED
 * htype HATTN_HTYPE_STRONG (the reference's USE_A2 / USE_H2 forward,
 * chunkwise.py:1118-1275 with the strong level function, base.py:49-62): BF16
 * q, k, v, L <= 32, T <= 64 * 2^9; else HATTN_ERR_NOT_IMPLEMENTED.  Its ht
 * holds what the reference stores for the strong hierarchy: at level 7 + ell,
 * ell = 1 .. ceil(log2(T / 64)) - 1, the raw phase-0 state of the strong state
 * loop after the last chunk (chunkwise.py:179-279); level 7 and the intra-chunk
 * levels are left untouched (zero in the reference).  It is no HState (the
 * decode step builds strong states itself).
 */
int hattn_mamba2_chunkwise_fwd(const void* q, const void* k, const void* v, const float* g,
                               const void* l, void* o, float* g_cumsum, float* ht, int B, int T,
                               int G, int H, int K, int V, int L, int dtype_qk, int dtype_v,
                               int dtype_l, int dtype_o, int level_base, int htype,
                               int chunk_size, void* workspace, size_t workspace_bytes,
                               void* stream);

/* Workspace bytes hattn_mamba2_chunkwise_fwd needs for these sizes, for
 * either htype and any dtype (the per-segment K x V summaries of the
 * segment-parallel scan; HType.STRONG: six block sums per segment).  No counterpart
 * in the reference, which allocates its intermediates with torch inside
 * chunkwise_fwd (chunkwise.py:1176-1179). */
size_t hattn_mamba2_chunkwise_fwd_workspace(int B, int T, int G, int H, int K, int V, int L);

/*
 * Log-linear Mamba-2 chunkwise forward that allocates nothing and takes no
 * workspace.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, results and status codes
 * as hattn_mamba2_chunkwise_fwd without the workspace pair; its scratch is a
 * file-scope static device array of 64 MiB per GPU (held until the process
 * ends), so HType.WEAK sizes whose segment summaries exceed 64 MiB return
 * HATTN_ERR_VALUE; HType.STRONG sizes whose per-segment block sums exceed it
 * run one serial walk per row instead (same results, slower).  Every call on one GPU shares that array:
 * calls that overlap on one GPU (concurrent streams or threads) race.
 */
int hattn_mamba2_chunkwise_fwd_noalloc(const void* q, const void* k, const void* v,
                                       const float* g, const void* l, void* o, float* g_cumsum,
                                       float* ht, int B, int T, int G, int H, int K, int V, int L,
                                       int dtype_qk, int dtype_v, int dtype_l, int dtype_o,
                                       int level_base, int htype, int chunk_size, void* stream);

/*
 * Health word of the last bf16 hattn_mamba2_chunkwise_fwd on this workspace
 * (no counterpart in the reference, whose forward is a sequence of launches
 * with no cross-workgroup waits).  The single-pass forward waits for the
 * segment summaries of earlier workgroups with a bounded poll; a wait that
 * gives up sets bit 0 (1 = look-back timeout) and that workgroup writes NaN
 * over its part of o, g_cumsum and ht.  A timeout means the results are
 * invalid (a lost flag, or two calls overlapping on one workspace or on the
 * no-allocation entry point's static scratch).  Copies the word to *status
 * and synchronises `stream` (a diagnostic, not for the hot path); 0 when the
 * sizes have one segment (no waits).  For hattn_mamba2_chunkwise_fwd_noalloc,
 * whose workspace is not exported, the NaN outputs are the signal.
 */
int hattn_mamba2_chunkwise_fwd_status(const void* workspace, int B, int T, int H, int V,
                                      unsigned int* status, void* stream);

/*
 * Test hook, no counterpart in the reference: sets the look-back controls of
 * the later forward launches of this process.  spin_limit: polls before a
 * wait gives up (<= 0 restores the default, about 1 s); publish = 0 makes the
 * summary phase skip its flags, so every look-back wait gives up.  With both
 * the tests exercise the timeout path while every kernel still exits
 * normally.  Not thread-safe with respect to concurrent forward calls.
 */
void hattn_debug_lookback(int spin_limit, int publish);

/*
 * Log-linear Mamba-2 chunkwise backward.
 *
 * Replaces hattention/chunkwise.py:1286-1597 `chunkwise_bwd(q, k, v, g, l, do,
 * head_first, level_base, htype, chunk_size) -> (dq, dk, dv, dg, dl)`, called
 * by HAttentionFunction.backward for HStruct.MAMBA2 (kernel.py:180-199).
 * Inputs are per head (the reference expands grouped q / k before its
 * kernels, chunkwise.py:1360-1362; the host layer does the same and sums the
 * group's dq / dk afterwards):
 *
 *   q, k, dq, dk [B, T, H, K] in dtype_qk  v, dv [B, T, H, V] in dtype_v
 *   g_cumsum     [B, T, H] fp32 chunk-local inclusive cumsum (the forward's output)
 *   l            [B, T, H, L] in dtype_l   do [B, T, H, V] in dtype_do (= dtype_qk)
 *   dg           [B, T, H] fp32: gradient w.r.t. the per-step g (what the
 *                reference returns after its reverse chunk-local cumsum)
 *   dl           [B, T, H, L] fp32 (every element written; levels no pair
 *                uses are 0)
 *   workspace    >= hattn_mamba2_chunkwise_bwd_workspace(...) bytes
 *
 * Constraints: as the forward (T % 64, L >= 7 + ceil(log2(T/64)), K and V
 * multiples of 64 -> HATTN_ERR_VALUE); K == V == 64 (the Python host layer
 * runs larger K and V as one call per 64-wide block), q/k/do either all BF16
 * (bf16 MFMA; v and l in {BF16, FP32}), all FP16 (fp16 MFMA; v FP16 or FP32,
 * l FP32) or all FP32 (bf16x3 kernels, fp32-accurate; v and l FP32, dq / dk /
 * dv written in fp32)
 *                                                  -> HATTN_ERR_NOT_IMPLEMENTED.
 * htype HATTN_HTYPE_STRONG (the reference's USE_A2 / USE_H2 backward,
 * chunkwise.py:1377-1580): BF16 q, k, v and do (l BF16 or FP32), T <= 64 *
 * 2^9; else HATTN_ERR_NOT_IMPLEMENTED.  Any other htype -> HATTN_ERR_VALUE.
 */
int hattn_mamba2_chunkwise_bwd(const void* q, const void* k, const void* v, const float* g_cumsum,
                               const void* l, const void* do_, void* dq, void* dk, void* dv,
                               float* dg, float* dl, int B, int T, int H, int K, int V, int L,
                               int dtype_qk, int dtype_v, int dtype_l, int dtype_do,
                               int level_base, int htype, int chunk_size, void* workspace,
                               size_t workspace_bytes, void* stream);

/*
 * hattn_mamba2_chunkwise_bwd that reuses the forward's segment summaries.
 *
 * No counterpart in the reference (its backward recomputes its states,
 * chunkwise.py:1371-1384); for callers that keep the forward's workspace until
 * the backward, as HAttentionFunction does between its forward and backward
 * (kernel.py:32-244).  Same arguments, results and status codes as
 * hattn_mamba2_chunkwise_bwd, plus fwd_workspace / fwd_workspace_bytes: the
 * workspace of the hattn_mamba2_chunkwise_fwd call (bf16 q / k, WEAK) on the
 * same q, k, v, g, l, with the same B, T, H, K = V = 64 and L, unchanged
 * since.  Its segment summaries and log-decays replace the backward's summary
 * pass (one read of K and V).  htype STRONG -> HATTN_ERR_NOT_IMPLEMENTED; q/k
 * not BF16 -> HATTN_ERR_NOT_IMPLEMENTED; fwd_workspace null or
 * fwd_workspace_bytes below hattn_mamba2_chunkwise_fwd_workspace(...) ->
 * HATTN_ERR_VALUE.  A workspace of another call gives wrong gradients.
 */
int hattn_mamba2_chunkwise_bwd_fwd_ws(const void* q, const void* k, const void* v,
                                      const float* g_cumsum, const void* l, const void* do_,
                                      void* dq, void* dk, void* dv, float* dg, float* dl, int B,
                                      int T, int H, int K, int V, int L, int dtype_qk,
                                      int dtype_v, int dtype_l, int dtype_do, int level_base,
                                      int htype, int chunk_size, void* workspace,
                                      size_t workspace_bytes, const void* fwd_workspace,
                                      size_t fwd_workspace_bytes, void* stream);

/* Workspace bytes of hattn_mamba2_chunkwise_bwd for the given htype (WEAK:
 * segment summaries of both scan directions and the q . dq row sums; STRONG:
 * the far dq / dlambda partials of the chunk walks and the adjoint of every
 * chunk's state insertion).  No counterpart in the reference, which allocates
 * fp32 h / dh (and hr / dhr for STRONG) per level inside chunkwise_bwd
 * (chunkwise.py:1371-1384). */
size_t hattn_mamba2_chunkwise_bwd_workspace(int B, int T, int H, int K, int V, int L, int htype);

/*
 * Log-linear Gated DeltaNet chunkwise forward.
 *
 * Replaces hattention/chunkwise_hgdn.py:566-788 `chunkwise_fwd(q, k, v, b, g, l,
 * head_first, level_base, htype, chunk_size, output_final_state)
 * -> (g_cumsum, o, Aw, Au, ht)`, called by HAttentionFunction.forward for
 * HStruct.GDELTA (kernel.py:100-123) with q = l2norm(q) * scale, k = l2norm(k).
 * Per head (the reference expands grouped q / k first, chunkwise_hgdn.py:614-623):
 *
 *   q, k [B, T, H, K] bf16   v, o [B, T, H, V] bf16   beta [B, T, H] in dtype_beta
 *   g [B, T, H] fp32 per-step log-decay     l [B, T, H, L] in dtype_l
 *   g_cumsum [B, T, H] fp32 (output, chunk-local inclusive cumsum)
 *   Aw, Au [B, T, H, 64] bf16 (outputs): per chunk (I + A)^-1 and (I + A)^-1 o gamma,
 *          A = strict-tril(diag(beta) K K^T), gamma[t,s] = exp(Gc_t - Gc_s)
 *   ht [B, H, K, V, L] fp32 final level states or NULL
 *   l2norm_qk, qk_scale: nonzero l2norm_qk normalises inside the kernels,
 *          q <- q * qk_scale / ||q||, k <- k / ||k|| (||x|| = sqrt(sum x^2 +
 *          1e-6)), which is what HAttentionFunction does before the call
 *          (kernel.py:110-111, use_qk_l2norm_in_kernel); 0 takes q and k as
 *          given, as the reference's chunkwise_fwd does
 *   workspace >= hattn_gdn_chunkwise_fwd_workspace(...) bytes
 *
 * htype HATTN_HTYPE_WEAK, or HATTN_HTYPE_STRONG: what the reference's chunkwise
 * GDN path computes with the strong level table (chunkwise_hgdn.py:630,
 * 724-728, 782): lambda of an intra-chunk pair at its strong level, the
 * inter-chunk levels from 1 with the same (weak) delta-rule states, and every
 * chunk reading every level >= 1; ht then holds levels 8 .. 6 + nlev (level 7
 * is left as the caller set it, zero in the reference).  Any other htype ->
 * HATTN_ERR_VALUE.
 *
 * Constraints: T % 64, L >= 7 + ceil(log2(T/64)), K and V multiples of 64,
 * T * H * max(K, V) < 2^31 -> HATTN_ERR_VALUE; K in {64, 128, 192, 256} (the
 * reference's limit is K <= 256, chunkwise_hgdn.py:600-601), any V multiple of
 * 64, T <= 64 * 2^8 (16384) -> HATTN_ERR_NOT_IMPLEMENTED.  dtype_qkv BF16: beta / l in
 * {BF16, FP32}, o BF16 (bf16 MFMA); dtype_qkv FP16 (fp16 MFMA; q, k, v, o, Aw, Au
 * and the saved states in fp16, as the reference's fp16 dots): HType.WEAK, beta
 * and l FP32, o FP16; any other combination -> HATTN_ERR_NOT_IMPLEMENTED.
 */
int hattn_gdn_chunkwise_fwd(const void* q, const void* k, const void* v, const void* beta,
                            const float* g, const void* l, void* o, float* g_cumsum, void* Aw,
                            void* Au, float* ht, int B, int T, int H, int K, int V, int L,
                            int dtype_qkv, int dtype_beta, int dtype_l, int dtype_o,
                            int level_base, int htype, int chunk_size, int l2norm_qk,
                            float qk_scale, void* workspace, size_t workspace_bytes,
                            void* stream);

/* Workspace bytes of hattn_gdn_chunkwise_fwd (q_new, w_new, per-chunk transposed
 * k_new, u and the intra-chunk matrix P, all bf16).  No counterpart in the
 * reference, which allocates these with torch inside chunkwise_fwd
 * (chunkwise_hgdn.py:636-642). */
size_t hattn_gdn_chunkwise_fwd_workspace(int B, int T, int H, int K, int V, int L);

/*
 * hattn_gdn_chunkwise_fwd that also leaves, in its workspace, what the
 * backward's recompute would produce: q_new, W_new, K_new, U and every level's
 * state at every chunk start (bf16), the same values bit for bit.  No
 * counterpart in the reference (its backward recomputes them,
 * chunkwise_hgdn.py:860-893); for callers that keep the forward's workspace
 * until the backward, as HAttentionFunction does between its forward and
 * backward (kernel.py:32-244).  Same arguments, outputs and status codes as
 * hattn_gdn_chunkwise_fwd with workspace >= hattn_gdn_chunkwise_fwd_keep_workspace(...)
 * bytes; additionally V in {64, 128} and T <= 64 * 2^8 (the backward's
 * limits) -> else HATTN_ERR_NOT_IMPLEMENTED.
 */
int hattn_gdn_chunkwise_fwd_keep(const void* q, const void* k, const void* v, const void* beta,
                                 const float* g, const void* l, void* o, float* g_cumsum,
                                 void* Aw, void* Au, float* ht, int B, int T, int H, int K, int V,
                                 int L, int dtype_qkv, int dtype_beta, int dtype_l, int dtype_o,
                                 int level_base, int htype, int chunk_size, int l2norm_qk,
                                 float qk_scale, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* Workspace bytes of hattn_gdn_chunkwise_fwd_keep (the forward's, plus the
 * token-major k_new and the per-chunk level states).  No counterpart in the
 * reference. */
size_t hattn_gdn_chunkwise_fwd_keep_workspace(int B, int T, int H, int K, int V, int L);

/*
 * Log-linear Gated DeltaNet chunkwise backward.
 *
 * Replaces hattention/chunkwise_hgdn.py:791-1222 `chunkwise_bwd(q, k, v, b, g, l,
 * Aw, Au, do, head_first, level_base, htype, chunk_size) -> (dq, dk, dv, db, dg, dl)`,
 * called by HAttentionFunction.backward for HStruct.GDELTA (kernel.py:201-225)
 * with the same normalised q, k as the forward.  Per head:
 *
 *   q, k [B, T, H, K] bf16   v, do [B, T, H, V] bf16   beta [B, T, H] in dtype_beta
 *   g_cumsum [B, T, H] fp32 (the forward's chunk-local cumsum)   l [B, T, H, L] in dtype_l
 *   Aw, Au: the forward's outputs; accepted for the reference's signature and not
 *           read (the kernels recompute (I + A)^-1 in fp32)
 *   dq, dk [B, T, H, K] bf16   dv [B, T, H, V] bf16   db [B, T, H] in dtype_beta
 *   dg [B, T, H] fp32 (w.r.t. the per-step g: reverse chunk-local cumsum applied,
 *   chunkwise_hgdn.py:1219)   dl [B, T, H, L] fp32
 *   l2norm_qk, qk_scale: as the forward; with l2norm_qk nonzero, q and k are the
 *   raw inputs and dq, dk are w.r.t. them (the l2norm chain rule of
 *   kernel.py:24-29, 224-225 applied inside the kernel)
 *   workspace >= hattn_gdn_chunkwise_bwd_workspace(...) bytes
 *
 * htype STRONG: the gradient of the strong forward above (the level reads at
 * every chunk for levels >= 1 enter dq, dlambda and the dh scan).  The
 * reference's backward for that mode masks the level reads with the weak
 * skip_q (chunkwise_hgdn.py:1034, 1066-1067) and adds du on chunks whose u the
 * forward masked (chunkwise.py:1008-1012), so it is not the derivative of its
 * own forward; this one is.
 *
 * Constraints as hattn_gdn_chunkwise_fwd, except K in {64, 128, 192, 256} and V in
 * {64, 128} -> HATTN_ERR_NOT_IMPLEMENTED (the gradients are sums over independent column
 * blocks of V, so a caller splits a larger V into blocks of 128 / 64 and sums
 * dq, dk, db, dg, dl; hattention.chunkwise_hgdn.chunkwise_bwd does); dtype_do equal to
 * dtype_qkv; FP16 (dq, dk, dv in fp16) with HType.WEAK and FP32 beta / l only;
 * else HATTN_ERR_NOT_IMPLEMENTED.
 */
int hattn_gdn_chunkwise_bwd(const void* q, const void* k, const void* v, const void* beta,
                            const float* g_cumsum, const void* l, const void* Aw, const void* Au,
                            const void* do_, void* dq, void* dk, void* dv, void* db, float* dg,
                            float* dl, int B, int T, int H, int K, int V, int L, int dtype_qkv,
                            int dtype_beta, int dtype_l, int dtype_do, int level_base, int htype,
                            int chunk_size, int l2norm_qk, float qk_scale, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Workspace bytes of hattn_gdn_chunkwise_bwd: the recomputed q_new, k_new (token-major
 * and per-chunk transposed), w_new, u (bf16), every level's state at every chunk start (bf16), and the
 * per-V-slice partial gradients of the level scan.  No counterpart in the
 * reference, which allocates h / dh and its temporaries with torch inside
 * chunkwise_bwd (chunkwise_hgdn.py:894-913). */
size_t hattn_gdn_chunkwise_bwd_workspace(int B, int T, int H, int K, int V, int L);

/*
 * hattn_gdn_chunkwise_bwd without the recompute: q_new, W_new, K_new, U and
 * the level states come from fwd_workspace, the workspace of the
 * hattn_gdn_chunkwise_fwd_keep call on the same q, k, v, beta, g, l, B, T, H,
 * K, V, L, l2norm_qk and qk_scale, unchanged since.  No counterpart in the
 * reference (see hattn_gdn_chunkwise_fwd_keep).  Same arguments, results and
 * status codes as hattn_gdn_chunkwise_bwd, with workspace >=
 * hattn_gdn_chunkwise_bwd_fwd_ws_workspace(...) bytes (the level scan's
 * partial gradients only), plus fwd_workspace null or fwd_workspace_bytes
 * below hattn_gdn_chunkwise_fwd_keep_workspace(...) -> HATTN_ERR_VALUE.  The
 * results equal hattn_gdn_chunkwise_bwd's bit for bit; a workspace of another
 * call gives wrong gradients.
 */
int hattn_gdn_chunkwise_bwd_fwd_ws(const void* q, const void* k, const void* v, const void* beta,
                                   const float* g_cumsum, const void* l, const void* Aw,
                                   const void* Au, const void* do_, void* dq, void* dk, void* dv,
                                   void* db, float* dg, float* dl, int B, int T, int H, int K,
                                   int V, int L, int dtype_qkv, int dtype_beta, int dtype_l,
                                   int dtype_do, int level_base, int htype, int chunk_size,
                                   int l2norm_qk, float qk_scale, void* workspace,
                                   size_t workspace_bytes, const void* fwd_workspace,
                                   size_t fwd_workspace_bytes, void* stream);

/* Workspace bytes of hattn_gdn_chunkwise_bwd_fwd_ws: the level scan's partial
 * gradients (no recompute regions).  No counterpart in the reference. */
size_t hattn_gdn_chunkwise_bwd_fwd_ws_workspace(int B, int T, int H, int K, int V, int L);

/*
 * One decode step of the Fenwick level state (HState) for every (b, h).
 *
 * Replaces hattention/kernel.py:577-633 `hattention_step(hstate, q, k, v, b, g, l,
 * scale, level_base, htype, hstruct, use_qk_l2norm_in_kernel) -> (o, hstate)`
 * with its step_state / step_output (hattention/recurrent.py:134-166), called by
 * hattention_prefill (kernel.py:555-570) and hselective_state_update
 * (mamba_apis.py:407-566).  HType.WEAK or HType.STRONG, level base 2.
 *
 *   states [B, H, K, V, L] fp32 (read and written)   counts [L] int32 or NULL
 *   q, k [B, G, K] in dtype_qk   v, o [B, H, V] in dtype_v   l [B, H, L] in dtype_l
 *   g [B, H] fp32 log-decay (gate exp(g))   beta [B, H] in dtype_beta (GDELTA) or NULL
 *   hstruct HATTN_HSTRUCT_MAMBA2 or HATTN_HSTRUCT_GDELTA
 *   htype HATTN_HTYPE_WEAK or HATTN_HTYPE_STRONG
 *   cascade, planned by the caller from its copy of counts (the cascade depends
 *            only on the counts):
 *            WEAK: number of full levels that merge upwards before the insert
 *            (HState.cascade_weak, recurrent.py:42-54); 0 <= cascade < L.
 *            STRONG: the level m where HState.cascade_strong's carry merges
 *            (recurrent.py:56-74): levels 0 .. m-1 move up one level, level
 *            m - 1 merging into level m; m = L when the carry leaves the top
 *            level; 1 <= cascade <= L.
 *   update / output: 1 to advance the state (step_state) / write o (step_output);
 *            k, v, g, beta are read only with update, q, l, o only with output
 *            (the others may be NULL)
 *   l2norm_qk: 1 to use q / |q| * scale and k / |k| (|x| = sqrt(sum x^2 + 1e-6),
 *            kernel.py:20-23, 626-629); scale is ignored otherwise
 *
 * Constraints: K <= 256, V a multiple of 16, L <= 32, dtype codes BF16 or FP32
 * -> else HATTN_ERR_NOT_IMPLEMENTED.
 */
int hattn_hstate_step(float* states, int* counts, const void* q, const void* k, const void* v,
                      const void* beta, const float* g, const void* l, void* o, int B, int G,
                      int H, int K, int V, int L, int hstruct, int htype, int cascade,
                      int update, int output, int l2norm_qk, float scale, int dtype_qk,
                      int dtype_v, int dtype_l, int dtype_beta, void* stream);

/*
 * Levels 0 .. nlo - 1 of the HState after a chunkwise prefill of T tokens
 * (T % 64 == 0), MAMBA2.
 *
 * Replaces the MAMBA2 fast path of hattention/kernel.py:378-465
 * `postprocess_prefill_hstate_` (the torch einsums of :420-436): level 0 is
 * k_{T-1} v_{T-1}^T, level e >= 1 the 2^(e-1) tokens before the tokens of the
 * lower levels, each weighted by exp(sum of g after it).  The levels >= nlo come
 * from the chunkwise forward's final states.
 *
 *   states [B, H, K, V, L] fp32 (levels < nlo written)   k [B, T, G, K] in dtype_k
 *   v [B, T, H, V] in dtype_v   g [B, T, H] fp32 per-step log-decay
 *
 * Constraints: K <= 256, V a multiple of 16, 1 <= nlo <= min(7, L).
 */
int hattn_mamba2_prefill_levels(float* states, const void* k, const void* v, const float* g,
                                int B, int T, int G, int H, int K, int V, int L, int nlo,
                                int dtype_k, int dtype_v, void* stream);

/*
 * Layer pre-processing of hmamba_chunk_scan_combined, one pass
 * (hattention/mamba_apis.py:346-366, compute_lambda :70-85):
 *   d = dt + dt_bias (dt_bias may be NULL), softplus(d) if dt_softplus;
 *   v = x * d;  g = A[h] * d (fp32);  lam = compute_lambda(Lp[h], dl, lambda_mode).
 * x, v [B, T, H, P]; dt [B, T, H]; dl, lam [B, T, H, L]; A [H] fp32; Lp [H, L].
 * lambda_mode: HATTN_LAMBDA_LINEAR (None), _POSITIVE, _BOUNDED.  P a multiple of
 * 4 with P / 4 a power of two <= 64, L <= 32; every tensor 16-byte aligned.
 * Element types (BF16 / FP32) per tensor: dtype_x, dtype_dt, dtype_dl, dtype_lp,
 * dtype_v, dtype_lam.
 */
enum { HATTN_LAMBDA_LINEAR = 0, HATTN_LAMBDA_POSITIVE = 1, HATTN_LAMBDA_BOUNDED = 2 };
int hattn_mamba2_layer_prologue(const void* x, const void* dt, const float* A,
                                const float* dt_bias, const void* dl, const void* Lp, void* v,
                                float* g, void* lam, int B, int T, int H, int P, int L,
                                int dt_softplus, int lambda_mode, int dtype_x, int dtype_dt,
                                int dtype_dl, int dtype_lp, int dtype_v, int dtype_lam,
                                void* stream);

/*
 * Layer post-processing, out = y + x * D[h] (mamba_apis.py:346-349, :402-403).
 * y, x, out [B, T, H, P] in dtype_y, dtype_x, dtype_out; D [H] fp32.
 */
int hattn_mamba2_layer_epilogue(const void* y, const void* x, const float* D, void* out, int B,
                                int T, int H, int P, int dtype_y, int dtype_x, int dtype_out,
                                void* stream);

/*
 * The layer scan of hmamba_chunk_scan_combined with its pre- and
 * post-processing folded into the scan's loads and stores (replaces
 * mamba_apis.py:263-404 without final states: layer prologue ->
 * HAttentionFunction (q = C, k = B, v = x dt', g = A dt', lambda) -> y = o + x D):
 * the forward scan reads x, dt and dl in place of v, g and lambda and writes
 *   y = bf16(o) + x D[h]   (D != NULL; y in dtype_y), or y = o (D == NULL).
 * v and lambda are computed with the prologue's formulas (v rounded to bf16,
 * lambda to dtype_lam), so y equals the separate prologue -> chunkwise forward
 * -> epilogue chain.  g_cumsum [B, T, H] fp32 as the chunkwise forward's.
 *   x [B, T, H, P] bf16, dt [B, T, H] dtype_dt, A [H] fp32, dt_bias [H] fp32 or
 *   NULL, B / C [B, T, G, N] bf16, dl [B, T, H, L] dtype_dl, Lp [H, L] fp32,
 *   D [H] fp32 or NULL.
 * Constraints: N == 64, P % 64 == 0, L <= 32, HType.WEAK, chunk 64, base 2,
 * x / B / C bf16 (-> HATTN_ERR_NOT_IMPLEMENTED); workspace as
 * hattn_mamba2_chunkwise_fwd_workspace(B, T, G, H, N, P, L).
 */
int hattn_mamba2_layer_scan_fwd(const void* x, const void* dt, const float* A,
                                const float* dt_bias, const void* Bm, const void* Cm,
                                const void* dl, const float* Lp, const float* D, void* y,
                                float* g_cumsum, int B, int T, int G, int H, int P, int N, int L,
                                int dtype_x, int dtype_dt, int dtype_bc, int dtype_dl,
                                int dtype_lam, int dtype_y, int dt_softplus, int lambda_mode,
                                int level_base, int htype, int chunk_size, void* workspace,
                                size_t workspace_bytes, void* stream);

/*
 * Backward of the layer pre- and post-processing: what torch autograd computes
 * through mamba_apis.py:346-366 and :402-403 given the scan's gradients dv,
 * dg (fp32), dlam and the layer output gradient dy (read only when D != NULL):
 *   dx = dv d + dy D,  ddt = (sum_p dv x + dg A) softplus'(dt + dt_bias),
 *   ddl from dlam per lambda mode; per-head sums dA, ddt_bias, dD [H] and
 *   dLp [H, L] in fp32 (any of them may be NULL), reduced in a fixed order.
 * Workspace: hattn_mamba2_layer_bwd_workspace(B, T, H, L) bytes.
 */
size_t hattn_mamba2_layer_bwd_workspace(int B, int T, int H, int L);
int hattn_mamba2_layer_bwd(const void* x, const void* dt, const float* A, const float* dt_bias,
                           const void* dl, const void* Lp, const float* D, const void* dy,
                           const void* dv, const float* dg, const void* dlam, void* dx,
                           void* ddt, void* ddl, float* dA, float* ddt_bias, float* dD,
                           float* dLp, int B, int T, int H, int P, int L, int dt_softplus,
                           int lambda_mode, int dtype_x, int dtype_dt, int dtype_dl,
                           int dtype_lp, int dtype_dy, int dtype_dv, int dtype_dlam,
                           int dtype_dx, int dtype_ddt, int dtype_ddl, void* ws,
                           size_t ws_bytes, void* stream);

/*
 * Depthwise causal conv1d + SiLU of hmamba_split_conv1d_scan_combined
 * (hattention/mamba_apis.py:206-213, causal_conv1d_fn with activation "silu"):
 *   pre[b,s,d] = bias[d] + sum_{w<W} weight[d,w] in[b, s-(W-1)+w, d],  out = silu(pre)
 * The input is the column window [col0, col0 + Dc) of rows of stride ld
 * (elements) of a [B, S, ld] tensor (the xBC channels of zxbcdtdl); the output
 * channels [0, d1), [d1, d2), [d2, Dc) go to the contiguous tensors out0
 * [B,S,d1], out1 [B,S,d2-d1], out2 [B,S,Dc-d2] (x, B, C).  weight [Dc, W],
 * bias [Dc] or NULL; W <= 8.
 */
int hattn_causal_conv1d_silu_fwd(const void* in, long long ld, long long col0, const void* weight,
                                 const void* bias, void* out0, void* out1, void* out2, int B,
                                 int S, int Dc, int d1, int d2, int W, int dtype_in,
                                 int dtype_w, int dtype_out, void* stream);

/*
 * Backward of the conv + SiLU given the gradients g0, g1, g2 of out0 / out1 /
 * out2: din is written into the column window [colo, colo + Dc) of rows of
 * stride ldo (the xBC slice of the zxbcdtdl gradient); dweight [Dc, W] and
 * dbias [Dc] (fp32, either may be NULL) are reduced in a fixed order.
 * Workspace: hattn_causal_conv1d_silu_bwd_workspace(B, S, Dc, W) bytes.
 */
size_t hattn_causal_conv1d_silu_bwd_workspace(int B, int S, int Dc, int W);
int hattn_causal_conv1d_silu_bwd(const void* in, long long ld, long long col0,
                                 const void* weight, const void* bias, const void* g0,
                                 const void* g1, const void* g2, void* din, long long ldo,
                                 long long colo, float* dweight, float* dbias, int B, int S,
                                 int Dc, int d1, int d2, int W, int dtype_in, int dtype_w,
                                 int dtype_g0, int dtype_g1, int dtype_g2, int dtype_din,
                                 void* ws, size_t ws_bytes, void* stream);

/*
 * Gated RMSNorm of hmamba_split_conv1d_scan_combined (mamba_apis.py:247-255,
 * rmsnorm_fn with z, no bias, norm_before_gate=False, one group):
 *   u = y * silu(z),  r = (mean_j u_j^2 + eps)^-1/2,  out = u * r * weight
 * y, out [rows, n] contiguous; z rows of stride ldz (the z slice of zxbcdtdl);
 * weight [n]; rstd [rows] fp32 receives r for the backward.
 */
int hattn_gated_rmsnorm_fwd(const void* y, const void* z, long long ldz, const void* weight,
                            void* out, float* rstd, long long rows, int n, float eps,
                            int dtype_y, int dtype_z, int dtype_w, int dtype_out, void* stream);

/*
 * Backward of the gated RMSNorm: dy [rows, n]; dz into rows of stride lddz;
 * dweight [n] fp32 reduced in a fixed order.  Workspace:
 * hattn_gated_rmsnorm_bwd_workspace(rows, n) bytes.
 */
size_t hattn_gated_rmsnorm_bwd_workspace(long long rows, int n);
int hattn_gated_rmsnorm_bwd(const void* y, const void* z, long long ldz, const void* weight,
                            const float* rstd, const void* dout, void* dy, void* dz,
                            long long lddz, float* dweight, long long rows, int n, int dtype_y,
                            int dtype_z, int dtype_w, int dtype_dout, int dtype_dy,
                            int dtype_dz, void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HATTN_H_ */
