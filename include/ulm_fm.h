/*
 * ulm_fm.h - C ABI of libulm_fm.so, the MI355X (gfx950) implementation of
 * UnifiedLM's fast-memory path.
 *
 * The reference has no C ABI for this path: its boundary is the Python
 * autograd Function `unified_memory(r, v, g, w) -> (q, fast)`
 * (kernel.py:199-238) called from UnifiedBlock.forward (model.py:84), and the
 * token-by-token UnifiedBlock.step / forward_recurrent (model.py:87-111,
 * 164-175) mirrored in C by run.c:193-265. Each entry point below names the
 * reference code it replaces.
 *
 * Conventions:
 *   - all pointers are device pointers (HBM of the current HIP device);
 *   - `stream` is a hipStream_t; every kernel is enqueued on it and the call
 *     returns without synchronising;
 *   - nothing is allocated inside; temporaries live in a caller-provided
 *     workspace whose size the matching *_workspace_bytes function returns;
 *   - tensors are dense row-major: (B,T,A) means A fastest;
 *   - `g` is a device pointer to one fp32 scalar g = -exp(log_rate), so
 *     lam = exp(g) is read on the device and no host sync happens
 *     (kernel.py:31, model.py:84);
 *   - return 0 (ULM_OK) or a nonzero ulm_status; ulm_last_error() gives the
 *     calling thread's last message. Arguments are validated before any HIP
 *     call, so an invalid call never touches the GPU.
 */
#ifndef ULM_FM_H
#define ULM_FM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum ulm_status { ULM_OK = 0, ULM_ERR_INVALID = 1, ULM_ERR_UNSUPPORTED = 2, ULM_ERR_LAUNCH = 3 };

/* Element types for arguments whose dtype follows the caller's tensor. */
enum ulm_dtype { ULM_F32 = 0, ULM_BF16 = 1, ULM_F16 = 2 };

/* Chunk length of the chunked kernels (kernel.py:20, CHUNK = 64). */
#define ULM_CHUNK 64

int ulm_abi_version(void);
const char *ulm_last_error(void);

/* Which evaluation of the products ulm_fm_fwd / ulm_fm_bwd and the block
 * entries use at this shape: 1 the chunked state form (`_la`'s algorithm, the
 * K-group kernel; A and D multiples of 32), 2 the block-pair form (the same
 * sums over pairs of 128-position blocks, six tile GEMMs; T <= 4096, any A and
 * D on zero-padded tiles), whichever needs fewer flops where both apply: about
 * 4 A D per token and product for the first, T (A + D) / 2 for the second;
 * 0 the generic kernel (widths off the 32 grid past 2048 positions where the
 * pair form would need more than twice the state form's flops, or past 4096
 * positions). The
 * environment variable ULM_FM_PATH=chunked, =pair or =generic forces one of
 * them where it applies. The choice is made when the saved buffer is sized
 * (ulm_fm_saved_bytes) and travels with it: a forward and its backward always
 * use one form. -1 for invalid sizes. No counterpart in the reference (one
 * algorithm, kernel.py:183-196). */
int ulm_fm_path(int B, int T, int A, int D);

/* ------------------------------------------------------------------------
 * Training: fused fast memory. Replaces UnifiedMemory.forward
 * (kernel.py:202-213): q = r / c with c = w + decayed cumsum of k = shift(r),
 * fast = causal scalar-decay linear attention of (q, k, v).
 *
 *   r      (B,T,A) fp32          read addresses
 *   v      (B,T,D) v_dtype       values (the reference casts them to bf16 in
 *                                 Python, kernel.py:205; here the cast is
 *                                 inside, so the chunked form's backward can
 *                                 also keep the bf16 remainder of an fp32 v)
 *   w      (A,)    fp32          prior mass
 *   q      (B,T,A) fp32   out    returned and saved
 *   fast   (B,T,D) fast_dtype out  (v.dtype in the reference, kernel.py:211)
 *   saved  ulm_fm_saved_bytes() bytes, out: what the backward needs besides
 *          r, g and w (the reference saves v16, q, c, q16, k16, kernel.py:212;
 *          this holds bf16 operand tiles of q, k and v, the evidence n at
 *          every chunk start in place of c, and, by the evaluation
 *          ulm_fm_path chooses, the bf16 scores P (with their transpose and
 *          bf16 residual) of the block-pair form or the dv product's score
 *          tiles of the chunked form). Opaque; pass it unchanged to ulm_fm_bwd.
 *          saved_bytes must be exactly the value ulm_fm_saved_bytes returned:
 *          that size names the form (ulm_fm_path at the time of the call)
 *          that the forward evaluates and the backward reads the buffer in.
 *          A size that names no form at this shape is rejected
 *          (ULM_ERR_INVALID).
 */
size_t ulm_fm_saved_bytes(int B, int T, int A, int D, int v_dtype);

/* The form (as ulm_fm_path numbers them) a saved buffer of saved_bytes bytes
 * holds at this shape and v_dtype, or -1 if no form has that size. No
 * counterpart in the reference. */
int ulm_fm_saved_path(size_t saved_bytes, int B, int T, int A, int D, int v_dtype);
size_t ulm_fm_fwd_workspace_bytes(int B, int T, int A, int D, int fast_dtype);
int ulm_fm_fwd(const float *r, const void *v, int v_dtype, const float *g, const float *w,
               float *q, void *fast, int fast_dtype, void *saved, size_t saved_bytes,
               void *workspace, size_t workspace_bytes, int B, int T, int A, int D, void *stream);

/* Prefill: the forward of ulm_fm_fwd (no autograd state kept) plus the
 * decode state after position T-1, so decoding can continue from a prompt
 * processed in one parallel pass instead of the token-by-token loop of
 * UnifiedLM.forward_recurrent (model.py:164-175; the state of
 * UnifiedBlock.init_state / step, model.py:88-111).
 *
 *   S      (B,D,A) fp32 out, 16-byte aligned: sum_{s<T} lam^(T-1-s) v_s k_s^T,
 *          the S of ulm_decode_state
 *   c_last (B,A)   fp32 out: w + sum_{s<T} lam^(T-1-s) k_s, the decode c
 *   r, v, g, w, q, fast as for ulm_fm_fwd; workspace of
 *   ulm_fm_prefill_workspace_bytes() bytes (0: unsupported shape).
 * Any A and D (widths off the 32 grid run on zero-padded tiles).
 * ulm_fm_prefill_path reports the form: 1 the chunked state form (S is the end
 * of its walk), 2 the block-pair products for fast plus S as one product of v
 * with the keys decayed to T-1, where those need fewer flops (at the 110M
 * widths up to about 768 positions); ULM_FM_PATH=chunked|pair forces one.
 * -1: unsupported shape. */
int ulm_fm_prefill_path(int B, int T, int A, int D);
size_t ulm_fm_prefill_workspace_bytes(int B, int T, int A, int D, int v_dtype, int fast_dtype);
int ulm_fm_prefill(const float *r, const void *v, int v_dtype, const float *g, const float *w,
                   float *q, void *fast, int fast_dtype, float *S, float *c_last,
                   void *workspace, size_t workspace_bytes, int B, int T, int A, int D, void *stream);

/* Replaces UnifiedMemory.backward (kernel.py:216-233): the products dq, dk
 * (reverse) and dv (reverse), as chunked products or, on the block-pair form,
 * as the dscores, dq_f, dk_f and dv tile GEMMs, and the denominator chain rule
 * (on the block-pair form inside the dq_f and dk_f products' epilogues).
 *
 *   saved   the buffer ulm_fm_fwd filled for the same r, g, w (q is not
 *           needed: it is recomputed as r / c from the saved checkpoints)
 *   v_dtype the dtype of the v given to ulm_fm_fwd
 *   dfast   (B,T,D) dfast_dtype  upstream gradient of fast
 *   dq_out  (B,T,A) fp32 or NULL upstream gradient of the returned q
 *                                 (HAS_DQO, kernel.py:166-167, 228)
 *   dr      (B,T,A) fp32  out
 *   dv      (B,T,D) dv_dtype out (dfast.dtype in the reference, kernel.py:223)
 *   dg      (1,)    fp32  out    d loss / d g
 *   dw      (A,)    fp32  out
 * Every output is reduced in a fixed order (no atomics): repeated calls agree
 * bit for bit. The workspace is ulm_fm_bwd_workspace_bytes(..., saved_bytes,
 * v_dtype) bytes: the need of the form the saved buffer holds (saved_bytes = 0:
 * of the form ulm_fm_path picks now; 0 is returned for a size that names no
 * form). */
size_t ulm_fm_bwd_workspace_bytes(int B, int T, int A, int D, int dfast_dtype, size_t saved_bytes,
                                  int v_dtype);
int ulm_fm_bwd(const float *r, const float *g, const float *w,
               const void *saved, size_t saved_bytes, int v_dtype,
               const void *dfast, int dfast_dtype, const float *dq_out,
               float *dr, void *dv, int dv_dtype, float *dg, float *dw,
               void *workspace, size_t workspace_bytes, int B, int T, int A, int D, void *stream);

/* Building block of both: out = o, o_t = sum_{s<=t} lam^(t-s) (a_t . b_s) c_s
 * (s >= t when reverse != 0). Replaces `_la` (kernel.py:183-196) with the
 * chunk state kept in fp32 on chip. a, b (B,T,K) bf16; c (B,T,V) bf16;
 * out (B,T,V) fp32, overwritten. split != 0 carries the decayed state-update
 * operand as a bf16 hi + lo pair (used by the backward's dq and dk). K or V
 * off the 32 grid run the generic kernel, whose key tiles' partial outputs
 * (workspace) are summed in a fixed order. */
size_t ulm_la_workspace_bytes(int B, int T, int K, int V);
int ulm_la(const uint16_t *a, const uint16_t *b, const uint16_t *c, const float *g, float *out,
           int B, int T, int K, int V, int reverse, int split,
           void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------
 * relu^2 slot address. Replaces UnifiedBlock.code (model.py:70-72) after
 * the key GEMM: r = z / (exp(clamp(log_eps,-10,10)) + sum_a z),
 * z = relu(pre + bias)^2, one row per token.
 *
 *   pre   (M,A) pre_dtype        K u without the bias
 *   bias  (A,)  fp32 or NULL
 *   log_eps (1,) fp32 device scalar
 *   r     (M,A) fp32 out, or NULL: only denom (ulm_block_fm_fwd forms r itself)
 *   denom (M,)  fp32 out         exp(clamp(log_eps)) + sum_a z, saved for backward
 */
int ulm_addr_fwd(const void *pre, int pre_dtype, const float *bias, const float *log_eps,
                 float *r, float *denom, int M, int A, void *stream);

/* Backward of ulm_addr_fwd: dpre (M,A) pre_dtype, dbias (A,) fp32 (may be
 * NULL when bias is NULL), dlog_eps (1,) fp32, both summed in a fixed order.
 * r may be NULL: it is then formed again from pre, bias and denom. A <= 8192. */
size_t ulm_addr_bwd_workspace_bytes(int M, int A);
int ulm_addr_bwd(const void *pre, int pre_dtype, const float *bias, const float *log_eps,
                 const float *r, const float *denom, const float *dr,
                 void *dpre, float *dbias, float *dlog_eps,
                 void *workspace, size_t workspace_bytes, int M, int A, void *stream);

/* ulm_addr_bwd with no workspace argument and no allocation of any kind, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The scratch (ulm_addr_bwd_workspace_bytes(M, A) bytes) lives in a
 * static device array of ULM_ADDR_BWD_NOALLOC_SCRATCH_BYTES bytes, one per
 * GPU, held until the process ends; larger M x A are rejected
 * (ULM_ERR_INVALID). Results are bitwise those of ulm_addr_bwd. Every call on
 * one GPU shares that GPU's array: calls that overlap in time on one GPU (on
 * different streams, or from several threads) race and must not be issued. */
#define ULM_ADDR_BWD_NOALLOC_SCRATCH_BYTES (8u << 20)
int ulm_addr_bwd_noalloc(const void *pre, int pre_dtype, const float *bias, const float *log_eps,
                         const float *r, const float *denom, const float *dr,
                         void *dpre, float *dbias, float *dlog_eps, int M, int A, void *stream);

/* ------------------------------------------------------------------------
 * Training: the rest of UnifiedBlock.forward (model.py:77-85) around the fast
 * memory. The block runs as
 *   h, u  = ulm_norm_conv_fwd(x)               RMSNorm + causal conv (78-79)
 *   pre   = u K^T,  v = h W_v^T                 caller's GEMMs (key, val)
 *   denom = ulm_addr_fwd(pre), r = NULL         relu^2 address (code, 70-72)
 *   qw, y = ulm_block_fm_fwd(pre, denom, v, x)  qw = w q, y = x + fast (84-85)
 *   out   = y + qw mu^T                         caller's GEMM, accumulating into y
 * and backward in reverse, with ulm_block_fm_bwd taking d(w q) = dout mu and
 * ulm_norm_conv_bwd joining the conv, RMSNorm and residual gradients. The
 * address r (B,T,A) fp32 is never written: the fast memory's statistics form
 * r = relu(pre + bias)^2 / denom where they read it, and ulm_addr_bwd forms
 * it again, from the bf16 pre-activation (half of r's bytes).
 */

/* h = (x rstd) * norm_w with rstd = (mean x^2 + eps)^-1/2 per position
 * (RMSNorm, model.py:31-42); u = the depthwise causal conv of h with Kc taps,
 * conv_w (D, Kc) oldest tap first, zero before position 0 (nn.Conv1d with
 * groups = D, padding Kc - 1, truncated to T: model.py:63, 79).
 *   x (B,T,D) x_dtype (F32 or BF16); h, u (B,T,D) out, in one dtype
 *   (h_dtype == u_dtype); rstd (B,T) fp32 out, saved for the backward.
 *   1 <= Kc <= 8. */
int ulm_norm_conv_fwd(const void *x, int x_dtype, const float *norm_w, const float *conv_w, int Kc,
                      float norm_eps, void *h, int h_dtype, void *u, int u_dtype, float *rstd,
                      int B, int T, int D, void *stream);

/* Backward of ulm_norm_conv_fwd plus the residual branch:
 *   dx = dres + d(RMSNorm)(dhv + conv^T du),
 *   dnorm_w (D,) and dconv_w (D, Kc) fp32 out, summed deterministically.
 *   du (B,T,D) du_dtype; dhv (B,T,D) or NULL, the value GEMM's gradient of
 *   h, in the same dtype (dhv_dtype == du_dtype); dres (B,T,D) fp32 or
 *   NULL; dx (B,T,D) fp32 out, may be
 *   dres itself. Workspace of ulm_norm_conv_bwd_workspace_bytes() bytes
 *   (0: D too large). */
size_t ulm_norm_conv_bwd_workspace_bytes(int B, int T, int D, int Kc);
int ulm_norm_conv_bwd(const void *x, int x_dtype, const float *rstd, const float *norm_w,
                      const float *conv_w, int Kc, const void *du, int du_dtype, const void *dhv,
                      int dhv_dtype, const float *dres, float *dx, float *dnorm_w, float *dconv_w,
                      void *workspace, size_t workspace_bytes, int B, int T, int D, void *stream);

/* ulm_fm_fwd inside the block. r is given by the address inputs, pre (B,T,A)
 * pre_dtype, bias (A,) fp32 or NULL and denom (B,T) from ulm_addr_fwd, as
 * r = relu(pre + bias)^2 * (1 / denom) (within 1 ulp of ulm_addr_fwd's r).
 * Instead of q and fast it writes
 *   qw (B,T,A) qw_dtype out: w q, the operand of the mu GEMM ((q*w), model.py:85)
 *   y  (B,T,D) fp32 out:     x + fast, x (B,T,D) fp32 the residual (y != x)
 * saved as for ulm_fm_fwd (ulm_fm_saved_bytes). */
size_t ulm_block_fm_fwd_workspace_bytes(int B, int T, int A, int D);
int ulm_block_fm_fwd(const void *pre, int pre_dtype, const float *bias, const float *denom,
                     const void *v, int v_dtype, const float *g, const float *w, void *qw, int qw_dtype,
                     const float *x, float *y, void *saved, size_t saved_bytes, void *workspace,
                     size_t workspace_bytes, int B, int T, int A, int D, void *stream);

/* ulm_fm_bwd inside the block: r given by the address inputs as for
 * ulm_block_fm_fwd; dqw (B,T,A) dqw_dtype is d loss / d(w q), the q gradient
 * is w dqw and dw also gets sum_t q dqw. Workspace of
 * ulm_fm_bwd_workspace_bytes(..., saved_bytes, v_dtype) bytes; other
 * arguments as for ulm_fm_bwd. */
int ulm_block_fm_bwd(const void *pre, int pre_dtype, const float *bias, const float *denom,
                     const float *g, const float *w, const void *saved, size_t saved_bytes,
                     int v_dtype, const void *dfast, int dfast_dtype, const void *dqw, int dqw_dtype,
                     float *dr, void *dv, int dv_dtype, float *dg, float *dw, void *workspace,
                     size_t workspace_bytes, int B, int T, int A, int D, void *stream);

/* The block's chunked prefill (UnifiedBlock.prefill, no autograd state):
 * ulm_block_fm_fwd plus the decode state after position T-1, S (B,D,A) and
 * c_last (B,A) as for ulm_fm_prefill. A and D multiples of 32; workspace of
 * ulm_block_fm_prefill_workspace_bytes() bytes (0: unsupported shape). */
size_t ulm_block_fm_prefill_workspace_bytes(int B, int T, int A, int D, int v_dtype);
int ulm_block_fm_prefill(const void *pre, int pre_dtype, const float *bias, const float *denom,
                         const void *v, int v_dtype, const float *g, const float *w, void *qw,
                         int qw_dtype, const float *x, float *y, float *S, float *c_last, void *workspace,
                         size_t workspace_bytes, int B, int T, int A, int D, void *stream);

/* Weight gradient of a linear layer over the token dimension: C = A^T B, i.e.
 * C[i][j] = sum_k A[k][i] B[k][j], A (K,N1) and B (K,N2) bf16 row-major,
 * C (N1,N2) fp32 out. The backward of F.linear's weight under bf16 autocast
 * (model.py:64-68: key, val, mu), with K = batch x positions. N1 and N2
 * multiples of 8, A and B 16-byte aligned; split over K, summed in a fixed
 * order. Workspace of ulm_wgrad_workspace_bytes() bytes (may be 0). */
size_t ulm_wgrad_workspace_bytes(int K, int N1, int N2);
int ulm_wgrad(const void *a, const void *b, float *c, int K, int N1, int N2, void *workspace,
              size_t workspace_bytes, void *stream);

/* dst = src converted elementwise (n elements; F32/BF16/F16, bf16 rounding to
 * nearest even): the autocast casts around the block's GEMMs. */
int ulm_cast(const void *src, int src_dtype, void *dst, int dst_dtype, size_t n, void *stream);

/* The block's fast-memory parameters from their logs, g[0] = -exp(log_rate[0])
 * and w = exp(clamp(log_w, log_w_min, log_w_max)) over A slots (model.py:75,
 * 84; the reference clamps to [-7, 12]), and the chain rule back from dg, dw:
 * dlog_rate = dg g, dlog_w = dw w inside the clamp range and 0 outside it (the
 * gradient of torch.clamp). One launch each instead of the parameter
 * expressions' elementwise kernels and their autograd. */
int ulm_block_params(const float *log_rate, const float *log_w, float log_w_min, float log_w_max, int A,
                     float *g, float *w, void *stream);
int ulm_block_params_bwd(const float *log_rate, const float *log_w, float log_w_min, float log_w_max,
                         const float *dg, const float *dw, int A, float *dlog_rate, float *dlog_w, void *stream);

/* ------------------------------------------------------------------------
 * Batched recurrent decode, N sequences, one block, one position. Together
 * these replace UnifiedBlock.step (model.py:96-111) / run.c:193-265. The
 * slot contents are held as S = U - mu*w, so the stored state is exactly the
 * recurrence S_t = lam S_{t-1} + v_t r_{t-1}^T and y = S q + mu (w*q).
 *
 * ulm_decode_pre: h = RMSNorm(x) (model.py:31-42), u = causal depthwise conv
 *   over [conv_buf, h] (model.py:100-102), conv_buf shifted in place.
 *   x (N,D), norm_w (D,), conv_w (D,Kc) oldest->newest, conv_buf (N,D,Kc-1),
 *   h (N,D) out, u (N,D) out.
 */
int ulm_decode_pre(const float *x, const float *norm_w, const float *conv_w, float *conv_buf,
                   float *h, float *u, int N, int D, int Kc, float norm_eps, void *stream);

/* ulm_decode_addr: r = relu^2 address of pre + bias (model.py:103);
 *   c <- lam c + (1-lam) w + r_prev (model.py:108); q = r / c; wq = w * q.
 *   pre (N,A) fp32 (K u), c (N,A) in/out, r_prev (N,A), r/q/wq (N,A) out. */
int ulm_decode_addr(const float *pre, const float *bias, const float *log_eps, const float *w,
                    const float *g, const float *r_prev, float *c, float *r, float *q, float *wq,
                    int N, int A, void *stream);

/* ulm_decode_state: S <- lam S + v r_prev^T (model.py:107 minus its constant
 *   prior term), y = S q (model.py:109), out = x + y + ymu where
 *   ymu = mu (w*q) is computed by the caller's GEMM.
 *   S (N,D,A) fp32 in/out, v/x/ymu/out (N,D), r_prev/q (N,A). */
int ulm_decode_state(float *S, const float *v, const float *r_prev, const float *q,
                     const float *g, const float *x, const float *ymu, float *out,
                     int N, int D, int A, void *stream);

/* Deferred write-back of the decode state (the same position-by-position
 * maths as ulm_decode_state, model.py:107-109 / run.c:244-255, in another
 * order). The state is S_base (N,D,A) plus the m most recent write terms,
 * j = 0 (oldest) .. m-1: pv (m,N,D) their values v_j and pr (m,N,A) their
 * keys r_prev_j, so that
 *   S_t = lam^m S_base + sum_j lam^(m-1-j) v_j r_prev_j^T.
 * A position appends its term (v, r_prev) as term m-1 and then either reads
 * (ulm_decode_read, S_base unchanged) or, once the terms reach the capacity
 * its caller chose (at most ulm_decode_max_pending()), writes S_t back as the
 * new S_base (ulm_decode_flush) and starts over with no terms. Over J
 * positions S then moves J reads and one write instead of J reads and J
 * writes. A % 4 == 0, A <= 4096, S, q and pr 16-byte aligned; 1 <= m.
 *
 * ulm_decode_dots: cj (m,N) = pr_j[n,:] . q[n,:], the terms' read-out weights.
 * ulm_decode_read: out = x + lam^m S_base q + sum_j lam^(m-1-j) v_j cj_j + ymu.
 * ulm_decode_flush: S_base <- S_t (in place); out = x + S_t q + ymu. */
int ulm_decode_max_pending(void);
/* ulm_decode_addr_deferred: ulm_decode_addr for a deferred state, which also
 *   appends r_prev as the pending key of term `slot` (pr (slot+1,N,A) at least)
 *   and, with cj given, writes cj (slot+1,N) = pr_j[n,:] . q[n,:] for
 *   j = 0 .. slot (what ulm_decode_dots forms, from the q it has just made).
 *   A % 4 == 0, A <= 4096, every vector 16-byte aligned. */
int ulm_decode_addr_deferred(const float *pre, const float *bias, const float *log_eps, const float *w,
                             const float *g, const float *r_prev, float *c, float *r, float *q, float *wq,
                             float *pr, int slot, float *cj, int N, int A, void *stream);
int ulm_decode_dots(const float *pr, const float *q, float *cj, int m, int N, int A, void *stream);
int ulm_decode_read(const float *S, const float *pv, const float *cj, int m, const float *q, const float *g,
                    const float *x, const float *ymu, float *out, int N, int D, int A, void *stream);
int ulm_decode_flush(float *S, const float *pv, const float *pr, int m, const float *q, const float *g,
                     const float *x, const float *ymu, float *out, int N, int D, int A, void *stream);

/* ------------------------------------------------------------------------
 * Diagnostics: HIP-event timing of every chunked-kernel launch (ulm_la and
 * the launches inside ulm_fm_fwd / ulm_fm_bwd) between start and stop, on
 * the stream each launch uses. stop() synchronises on the recorded events
 * and returns the summed kernel time and the number of launches timed.
 * Process-wide and not thread-safe; no counterpart in the reference
 * (its timings come from external scripts, docs/kernel.md:55-70). */
int ulm_la_timer_start(int max_launches);
int ulm_la_timer_stop(double *total_ms, int *launches);
/* The share of the last stop()'s launches that one block-pair product made
 * (tag one of ULM_PRODUCT_*; the chunked products carry no tag): their summed
 * kernel time and their number. */
enum {
    ULM_PRODUCT_SCORES = 1,  /* P = lam^(t-s) q.k, with the v tile copies */
    ULM_PRODUCT_APPLY = 2,   /* fast = P v */
    ULM_PRODUCT_DSCORES = 3, /* dS = lam^(t-s) dfast.v, the decay gradient's pair sum */
    ULM_PRODUCT_DV = 4,      /* dv = P^T dfast */
    ULM_PRODUCT_DQSTATS = 5, /* dq_f = dS k with the backward statistics (writes dr) */
    ULM_PRODUCT_DKDR = 6,    /* dk_f = dS^T q added into dr with the carry */
    ULM_PRODUCT_STATE = 7    /* a prefill's decode state, one product over positions */
};
int ulm_la_timer_product(int tag, double *total_ms, int *launches);

#ifdef __cplusplus
}
#endif
#endif /* ULM_FM_H */
