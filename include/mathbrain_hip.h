/*
 * mathbrain_hip.h -- C ABI of the MI355X (gfx950) Per-Slot EMA hot path.
 *
 * Every entry point takes device pointers, plain sizes and strides, and a HIP stream
 * (hipStream_t passed as void*; NULL = the null stream).  Nothing here allocates:
 * callers pass every output buffer, and the one call that needs device scratch
 * (mb_corpus_states) takes it as a workspace argument, or, in its _noalloc variant, uses
 * a fixed scratch array inside the library.  Calls are asynchronous on the stream.
 *
 * Return value: MB_OK (0) on success; a negative MB_ERR_* code for an argument the call
 * rejects before launching anything; a positive hipError_t code when the HIP runtime
 * reports a launch failure.  mb_last_error() returns a message for the last failing
 * call on the calling thread.
 *
 * Token ids are int64 (the reference's torch.long); -1 marks padding in slot lists.
 * Float tensors are fp32 unless a name says otherwise.  "Contiguous" means C order.
 */
#ifndef MATHBRAIN_HIP_H
#define MATHBRAIN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MB_OK 0
#define MB_ERR_INVALID_ARGUMENT (-1)
#define MB_ERR_UNSUPPORTED (-2)
#define MB_ERR_WORKSPACE (-3)

/* Message of the last failing call on this thread ("" if none). */
const char *mb_last_error(void);

/* ABI version of this library (bumped on any signature or flag change). */
int mb_abi_version(void);

/*
 * EMA query scan.  Replaces compute_query_ema_history (mathbrain/triton_ema_query.py:
 * 120-169) and its kernel _ema_seq_scan_kernel (:11-64); semantics of the CPU path
 * compute_query_ema_history_pt (:67-117):
 *
 *   C_seq[b,t,:] = c0[b,x_t,:] * rho^t + sum_{s<t, x_s = x_t} rho^(t-s)
 *
 * where the c0 term is present only if x_t is one of c_init_keys[b,:] (the last listed
 * duplicate wins; -1 keys are ignored).  With doc_ids, a token whose previous
 * occurrence lies in another document restarts from 0 (:51-57); c_init rows count as
 * occurring in doc_ids[b,0].
 *
 *   x            [B, L] int64, element strides (x_stride_b, x_stride_l)
 *   rhos         [N] fp32, 0 < rho <= 1
 *   c_init       [B, K, N] contiguous or NULL (then c_init_keys is ignored and K = 0)
 *   c_init_keys  [B, K] int64 contiguous or NULL
 *   doc_ids      [B, L] int64 contiguous or NULL
 *   C_seq        [B, L, N] contiguous output
 *   state_out    [B, K, N] or NULL: for every key whose token occurs in the chunk, the
 *                lazy EMA state after its last occurrence (C_seq at that position + 1);
 *                rows of other keys are not written.  May alias c_init.
 *   stamp_out    [B, K] int32 or NULL: position of that last occurrence, else -1.
 *
 * Limits: L <= 8192 (the per-sequence index lives in the 160 KB LDS of one CU); longer
 * sequences take mb_ema_query_scan_ws.
 */
int mb_ema_query_scan(const int64_t *x, int64_t x_stride_b, int64_t x_stride_l, int B, int L,
                      const float *rhos, int N, int64_t vocab_size, const float *c_init,
                      const int64_t *c_init_keys, int K, const int64_t *doc_ids, float *C_seq,
                      float *state_out, int32_t *stamp_out, void *stream);

/*
 * The same scan for any L.  Replaces compute_query_ema_history (mathbrain/triton_ema_query.py:
 * 120-169), whose kernel walks any length (:34).  Up to 8192 steps it is mb_ema_query_scan;
 * longer sequences run as consecutive 2048-step pieces on the stream, each chain of a piece
 * starting from its token's last occurrence before the piece (C_seq there + 1, decayed), and
 * need a workspace of mb_ema_query_scan_workspace(B, L, vocab_size) bytes (4-byte aligned,
 * contents irrelevant): a [B, vocab_size] int32 table of last positions.  Token ids must
 * then lie in [0, vocab_size) (ids outside count as never seen before).
 */
int mb_ema_query_scan_ws(const int64_t *x, int64_t x_stride_b, int64_t x_stride_l, int B, int L,
                         const float *rhos, int N, int64_t vocab_size, const float *c_init,
                         const int64_t *c_init_keys, int K, const int64_t *doc_ids, float *C_seq,
                         float *state_out, int32_t *stamp_out, void *workspace,
                         int64_t workspace_bytes, void *stream);

/*
 * Workspace bytes mb_ema_query_scan_ws needs: 0 for L <= 8192, else B * vocab_size * 4 (-1,
 * with mb_last_error set, for negative sizes or L > 8192 with vocab_size < 1).  No
 * counterpart in the reference, whose scan allocates its [B, V+1] tables per call
 * (triton_ema_query.py:141-143).
 */
int64_t mb_ema_query_scan_workspace(int B, int L, int64_t vocab_size);

/*
 * Key-side EMA states at chunk starts.  Replaces precompute_boundaries and its kernel
 * _c_boundary_scan (mathbrain/triton_flash_ema.py:81-113, :29-78):
 *
 *   C_bounds[b,j,k,:] = c0[b,k,:] * rho^(j*Br) + sum_{s < j*Br, x_s = u_k} rho^(j*Br-1-s)
 *
 * i.e. the state stored before chunk j is processed, with C <- C*rho + I(x_t = u_k) per
 * step.  With doc_ids the state is zeroed when the document changes (:69-75).
 *
 *   x        [B, L] int64, element strides (x_stride_b, x_stride_l)
 *   unique   [B, K] int64 contiguous, -1 = padding slot (its state stays c0)
 *   rhos     [N] fp32
 *   c_init   [B, K, c_init_stride_k] fp32 (first N columns used) or NULL (zeros)
 *   doc_ids  [B, L] int64 contiguous or NULL
 *   C_bounds [B, nc, K, Np] output, nc = max(1, ceil(L/Br)), Np >= N; columns N..Np-1
 *            are written as 0 (the reference pads N to max(N, 16) for tl.dot).
 *
 * Any L (the sequence's tokens are staged in LDS 8192 at a time).
 */
int mb_ema_boundary_states(const int64_t *x, int64_t x_stride_b, int64_t x_stride_l, int B,
                           int L, const int64_t *unique, int K, const float *rhos, int N, int Br,
                           const float *c_init, int64_t c_init_stride_k, const int64_t *doc_ids,
                           float *C_bounds, int Np, void *stream);

/*
 * Sorted distinct ids of each row.  Replaces the body of _build_unique_index
 * (mathbrain/triton_flash_ema.py:475-507):
 *
 *   out[b, 0:counts[b]]     = the distinct values of x[b, :] in increasing order
 *   out[b, counts[b]:width] = -1
 *
 *   x       [B, L] int64, element strides (x_stride_b, x_stride_l)
 *   out     [B, width] int64 contiguous output (a row's ids beyond width are dropped;
 *           width >= L keeps all of them)
 *   counts  [B] int32 output: distinct values per row
 *
 * Limits: L <= 16384 (a row is sorted in the LDS of one CU); beyond 8192 ids a row whose
 * values span 2^32 or more gets counts[b] = -1 and an all -1 list (token ids always fit).
 */
int mb_unique_rows(const int64_t *x, int64_t x_stride_b, int64_t x_stride_l, int B, int L,
                   int64_t *out, int width, int32_t *counts, void *stream);

/* Flags of the flash-EMA entry points. */
#define MB_FLASH_SILU 1        /* gate = SiLU(pre); otherwise the linear gate (use_silu=False) */
#define MB_FLASH_ABSENT_MASS 2 /* softmax also over the V - K_b absent slots (score 0) */
#define MB_FLASH_VOCAB_ROWS 4  /* E_k, E_v (dE_k, dE_v) are [V_total, H*hd] tables indexed by
                                  the slot's token id instead of [B, K, H*hd] gathered rows */
#define MB_FLASH_FP32 8        /* fp32 mode: the gate GEMM takes fp16 hi + lo operand pairs (three
                                  products, ~2^-22 relative) and the dW_pe product bf16 hi + lo
                                  pairs (~2^-16).  Needs N <= 64 and hd <= 64. */
#define MB_FLASH_FAST_GATE 16  /* the gate GEMM takes single fp16 operands (one product, 2^-11
                                  relative each): faster, and accurate only while the scores
                                  stay small enough that the softmax does not amplify that
                                  rounding (see the forward's comment) */

/*
 * Flash-EMA gated cross-attention forward.  Replaces flash_ema_forward and its kernel
 * _flash_ema_fwd (mathbrain/triton_flash_ema.py:529-568, :121-241).  For sequence b,
 * head h, step t and valid slot k (unique[b,k] >= 0):
 *
 *   c_dec[t,k,:] = C_bounds[b, t/Br, k, :N] rho^(t - Br*(t/Br) + 1)
 *                  + sum_{Br*(t/Br) <= s < t, x_s = unique[b,k]} rho^(t-s)
 *   g[t,k,:]     = SiLU(c_dec[t,k,:] . W_pe[:, h*hd:(h+1)*hd])   (fp16 operands)
 *   s[t,k]       = Q[b,h,t] . (E_k[b,k,h] * g[t,k]) / sqrt(hd)
 *   O[b,h,t]     = sum_k softmax_k(s) E_v[b,k,h] * g[t,k]
 *   LSE[b,h,t]   = log(sum_k exp s[t,k] (+ V_total - K_b with MB_FLASH_ABSENT_MASS))
 *
 * With MB_FLASH_ABSENT_MASS the softmax holds all V_total slots as the dense PyTorch
 * reference does (mathbrain/flash_ema_attention.py:76-77); without it, only the valid
 * slots, as the Triton kernel computes (triton_flash_ema.py:215-229).
 *
 *   Q         [B, H, L, hd] fp32, element strides q_sb, q_sh, q_sl, q_sd
 *   x         [B, L] int64, element strides x_sb, x_sl
 *   E_k, E_v  [B, K, H*hd] fp32 contiguous: row (b, k) is slot k of sequence b; with
 *             MB_FLASH_VOCAB_ROWS [V_total, H*hd], row unique[b,k] (ids are clamped to
 *             [0, V_total); padding slots read row 0 and contribute nothing).  The
 *             projections k_proj(ln_kv(E)) act row by row, so projecting the vocabulary
 *             table once gives the rows the slots would gather (fewer rows when
 *             B*K > V_total, and no gather).
 *   W_pe      [N, H*hd] fp32 contiguous (pe_proj.weight transposed)
 *   rhos      [N] fp32
 *   unique    [B, K] int64 contiguous, -1 = padding slot
 *   C_bounds  [B, nc, K, Np] fp32 contiguous (mb_ema_boundary_states), nc >= ceil(L/Br)
 *   O         [B, H, L, hd] fp32 contiguous output; LSE [B, H, L] fp32 output
 *   scores    NULL, or [B, H, K, L] fp32 output: s[t,k] * log2(e) for every valid slot
 *             (rows of padding slots are not written).  Passed to mb_flash_ema_bwd, it
 *             spares the backward the score recomputation.
 *   workspace NULL, or workspace_bytes >= mb_flash_ema_fwd_workspace(...) bytes of device
 *             memory (16-byte aligned, contents irrelevant): room for the partial softmax
 *             states when the launch splits each workgroup's slots into parts so that the
 *             workgroups fill the device's last round (e.g. 896 workgroups of one per CU
 *             on 256 CUs).  Without it (or when smaller) the launch runs unsplit; O and LSE
 *             agree either way up to the order of the softmax sums.
 *
 * Gate arithmetic.  By default (N <= 64 and hd <= 64) the gate GEMM splits both operands,
 * c_dec and W_pe * log2(e), into fp16 hi + lo pairs and takes three products (W_lo c_hi +
 * W_hi c_lo + W_hi c_hi) with fp32 accumulation, ~2^-22 relative: where scores reach
 * ~100 (a model's own initialisation can do that) the softmax turns a relative gate error
 * e into ~100 e of the weights, and single fp16 operands (2^-11) moved a 6-layer model's
 * logits by 2e-2 and its gradients by 0.1 from the exact model.  The two lo products are
 * taken only on the 32-rate tiles whose counters can be large: an EMA of counts stays near
 * or below B = 1/(1 - rho), and with two tiles the first takes the single product when its
 * largest B is below 1/32 of the second's (rates from half-life 1 to 4096: 87 against 5900;
 * the 6-layer model then sits 6e-4 / 5e-3 from the exact one).  Each workgroup decides from
 * `rhos`, and the launch runs one kernel instantiation per choice.  MB_FLASH_FP32 splits
 * every tile.  With MB_FLASH_FAST_GATE,
 * and by default for N > 64 or hd 128 (where the lo tiles do not fit in LDS), the gate
 * takes single fp16 operands.  The fp16 counters are clamped to 65440 at the chunk start;
 * an EMA of counts stays below 1/(1 - rho), under that bound for half-lives up to ~45,000
 * steps, which the Python entry points check (rates with longer half-lives are refused
 * there), so only a caller-supplied initial state (C_bounds from a c_init) above 65440
 * reaches the clamp.
 *
 * Supported: hd in {32, 64, 128} (32 or 64 with MB_FLASH_FP32), 1 <= H <= 64, N <= 128 (N <= 64
 * with MB_FLASH_FP32), Br <= 32 or Br == 64.  At hd 128 each head takes two waves, one per
 * 16-step tile of the workgroup's 32 steps.
 */
int mb_flash_ema_fwd(const float *Q, int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t q_sd,
                     const int64_t *x, int64_t x_sb, int64_t x_sl, const float *E_k,
                     const float *E_v, const float *W_pe, const float *rhos,
                     const int64_t *unique, const float *C_bounds, int B, int H, int L, int hd,
                     int K, int N, int Np, int nc, int Br, int64_t V_total, int flags, float *O,
                     float *LSE, float *scores, void *workspace, int64_t workspace_bytes,
                     void *stream);

/*
 * Workspace bytes mb_flash_ema_fwd wants on the current device for these shapes and flags
 * (0: it would not split), or -1 for arguments mb_flash_ema_fwd rejects (mb_last_error).
 * No counterpart in the reference, whose Triton grid needs no workspace.
 */
int64_t mb_flash_ema_fwd_workspace(int B, int H, int L, int hd, int K, int N, int flags);

/*
 * Flash-EMA gated cross-attention backward.  Replaces FlashEMAFunction.backward and its
 * kernels _flash_ema_bwd_dq_de / _flash_ema_bwd_dw (mathbrain/triton_flash_ema.py:586-650,
 * :250-355, :359-469) with one fused pass.  Arguments as mb_flash_ema_fwd, plus
 *
 *   dO        [B, H, L, hd] fp32, same element strides as Q
 *   O, LSE    the forward's outputs (contiguous)
 *   scores    NULL (recompute the scores), or the forward's scores output
 *   dQ        [B, H, L, hd] fp32 contiguous output
 *   dE_k/dE_v [B, K, H*hd] fp32 contiguous outputs (zero for padding slots); with
 *             MB_FLASH_VOCAB_ROWS [V_total, H*hd], the sums over every slot of each token
 *   dW_pe     [N, H*hd] fp32 contiguous output
 *
 * dQ is written once per element.  dE_k, dE_v and dW_pe are cleared by the call (with a
 * fill kernel, no memset) and then accumulated with fp32 atomics, so their summation
 * order is not fixed, as in the reference's tl.atomic_add.  The gate is recomputed as
 * in the forward (the same arithmetic for the same flags), except that by default, when
 * `scores` is given, a slot takes the split gate only in the waves (16 steps of one head)
 * where the forward's probability reaches 2^-7 at one of the steps, and the single fp16
 * product elsewhere: every gradient term of a slot carries its probability, so the single
 * product's rounding enters scaled by it (at a 6-layer model's initialisation 99.9 % of the
 * slot-steps qualify, and the gradients' distance from the exact model's stays 4.6e-3, as
 * with the split everywhere).  The backward's split is the forward's gate (lo products on the
 * same rate tiles), so recomputed scores are the forward's.  MB_FLASH_FP32 always splits,
 * every tile.  The dW_pe product takes bf16
 * c_dec and bf16 dpre (as the reference's triton_flash_ema.py:463-465 does), or with
 * MB_FLASH_FP32 bf16 hi + lo pairs of both, with fp32 accumulation.  Supported: as
 * mb_flash_ema_fwd.  At hd 128 each head runs as two 64-dim halves on two waves that add
 * their score and dO . v partial sums through LDS.
 */
int mb_flash_ema_bwd(const float *Q, int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t q_sd,
                     const float *dO, const int64_t *x, int64_t x_sb, int64_t x_sl,
                     const float *E_k, const float *E_v, const float *W_pe, const float *rhos,
                     const int64_t *unique, const float *C_bounds, const float *O,
                     const float *LSE, int B, int H, int L, int hd, int K, int N, int Np, int nc,
                     int Br, int64_t V_total, int flags, const float *scores, float *dQ,
                     float *dE_k, float *dE_v, float *dW_pe, void *stream);

/*
 * Flash-EMA attention forward with the query gating folded into its prologue.  Replaces
 * fused_apply_symmetric_query_gating followed by q_proj and flash_ema_forward
 * (mathbrain/triton_fused_gating.py:179-197, model.py:75-87): each workgroup computes its
 * own queries
 *
 *   Q[b,t,:] = q_proj(LayerNorm_eps(x_q[b,t] * SiLU((C_seq[b,t] + 1) . W_pe)) * ln_w + ln_b)
 *
 * (the LayerNorm output bit for bit as mb_gating_fwd computes it; q_proj on the matrix
 * cores from fp16 hi + lo operand pairs, ~2^-22 relative per product), viewed as
 * [B, H, L, hd] (column h*hd + d of Q is head h, dim d), and then runs the attention of
 * mb_flash_ema_fwd on it.  Q is never written.  Arguments as mb_flash_ema_fwd without
 * Q and scores, plus
 *
 *   x_q       [B, L, D] fp32 (D = H*hd), element strides xq_sb, xq_sl, columns contiguous
 *   C_seq     [B, L, N] fp32, element strides c_sb, c_sl, columns contiguous
 *   ln_w, ln_b [D] fp32 (ln_q), eps > 0
 *   W_q       [D, D] fp32 contiguous (q_proj.weight: row = output column of Q)
 *
 * W_pe serves both the query gate and the key gate, as in the reference.  The backward is
 * mb_flash_ema_bwd on Q recomputed from x_ln (the q_proj and gating gradients need x_ln, so
 * the caller recomputes it with mb_gating_fwd).  Supported: as mb_flash_ema_fwd with hd 32
 * or 64 and D a multiple of 32 and at most 1024.
 */
int mb_flash_ema_fwd_gq(const float *x_q, int64_t xq_sb, int64_t xq_sl, const float *C_seq,
                        int64_t c_sb, int64_t c_sl, const float *ln_w, const float *ln_b, float eps,
                        const float *W_q, const int64_t *x, int64_t x_sb, int64_t x_sl,
                        const float *E_k, const float *E_v, const float *W_pe, const float *rhos,
                        const int64_t *unique, const float *C_bounds, int B, int H, int L, int hd,
                        int K, int N, int Np, int nc, int Br, int64_t V_total, int flags, float *O,
                        float *LSE, void *stream);

/*
 * Fused symmetric query gating, forward.  Replaces _fused_gating_fwd and the forward of
 * FusedGatingFunction (mathbrain/triton_fused_gating.py:12-57, :122-148); with the
 * projection folded in, also the pe_proj GEMM and bias of
 * fused_apply_symmetric_query_gating (:179-186).  Per row r and column d:
 *
 *   pre[r,d] = p_pre[r,d] + bias[d]                    when p_pre != NULL
 *            = sum_n (C_seq[r,n] + 1) W_pe[n,d]         when p_pre == NULL
 *   y[r,:]   = LayerNorm_eps(x_q[r,:] * SiLU(pre[r,:])) * ln_w + ln_b
 *
 * (the linear gate pre instead of SiLU(pre) when use_silu == 0).
 *
 *   x_q     [rows, D] fp32, row stride xq_row_stride (columns contiguous)
 *   p_pre   [rows, D] fp32, row stride pp_row_stride, or NULL; bias [D] with p_pre
 *   C_seq   [rows, N] fp32, row stride c_row_stride, and W_pe [N, D] contiguous
 *           (pe_proj.weight transposed): used when p_pre is NULL
 *   y       [rows, D] contiguous output; mu, rstd [rows] outputs (LayerNorm statistics,
 *           consumed by mb_gating_bwd)
 *   pre_out [rows, D] contiguous output, or NULL: the pre-activation pre[r,d], kept for
 *           the backward as the reference keeps its gate (written at
 *           triton_fused_gating.py:38, read back at :90); passed to mb_gating_bwd as p_pre
 *           with a NULL bias, it spares the backward the projection
 *
 * bias may be NULL with p_pre (read as zero).  Supported: D <= 1024, N <= 1024.
 */
int mb_gating_fwd(const float *x_q, int64_t xq_row_stride, const float *p_pre,
                  int64_t pp_row_stride, const float *bias, const float *C_seq,
                  int64_t c_row_stride, const float *W_pe, int N, const float *ln_w,
                  const float *ln_b, int64_t rows, int D, int use_silu, float eps, float *y,
                  float *mu, float *rstd, float *pre_out, void *stream);

/*
 * Fused symmetric query gating, backward.  Replaces _fused_gating_bwd and the backward of
 * FusedGatingFunction (mathbrain/triton_fused_gating.py:61-119, :150-177).  Inputs as
 * mb_gating_fwd (the same p_pre / C_seq choice), plus dy [rows, D] contiguous and the
 * forward's mu, rstd.  Outputs, all contiguous:
 *
 *   dx_q   [rows, D]   dx_emb * g
 *   dp_pre [rows, D]   dx_emb * x_q * SiLU'(pre): the gradient of p_pre, or, with the
 *                      folded projection, of pre (then dW_pe = dp_pre^T (C_seq + 1))
 *   dbias, dln_w, dln_b [D]  column sums of dp_pre, dy * x_hat and dy
 *
 * The column sums are cleared by the call (fill kernel) and accumulated with fp32
 * atomics, one per column and workgroup: their summation order is not fixed.  With p_pre
 * given (bias may be NULL) and D a multiple of 256 (16-byte aligned rows), one wave
 * takes each row.
 */
int mb_gating_bwd(const float *dy, const float *x_q, int64_t xq_row_stride, const float *p_pre,
                  int64_t pp_row_stride, const float *bias, const float *C_seq,
                  int64_t c_row_stride, const float *W_pe, int N, const float *ln_w,
                  const float *mu, const float *rstd, int64_t rows, int D, int use_silu,
                  float *dx_q, float *dp_pre, float *dbias, float *dln_w, float *dln_b,
                  void *stream);

/*
 * Data pipeline on the device (the producers of the hot path's inputs).
 *
 * Per-position EMA states of a whole corpus.  Replaces the preprocessing scan of
 * preprocess_corpus (mathbrain/data.py:276-303):
 *
 *   states[t,:] = sum_{s <= t, tokens[s] = tokens[t], s in t's document segment} rho^(t-s)
 *
 * the state of token tokens[t] just after its occurrence at t, restarted wherever the
 * document changes (data.py:287-290).  The corpus comes as its positions sorted by chain:
 *
 *   order    [T] int64: the positions 0..T-1 sorted by (document segment, token), ascending
 *            positions inside one key (a stable sort of the key)
 *   chain    [T] int64: the key of each sorted entry (equal keys = one token in one
 *            document segment; any encoding, e.g. segment << 32 | token)
 *   rhos     [N] fp32, 1 <= N <= 128
 *   states   [T, N] fp32 output
 *   work     device workspace of at least mb_corpus_states_workspace(T, N) bytes
 *
 * Limits: T <= 2^31 - 1 (positions are int32, as in pos_dict.pkl).
 */
int64_t mb_corpus_states_workspace(int64_t T, int N);
int mb_corpus_states(const int64_t *order, const int64_t *chain, int64_t T, const float *rhos,
                     int N, float *states, void *work, int64_t work_bytes, void *stream);

/*
 * mb_corpus_states without a workspace argument: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * mb_corpus_states; the scratch is a 32 MiB device array inside the library (one per GPU,
 * held until the process ends), so mb_corpus_states_workspace(T, N) must not exceed
 * 32 MiB (about 44 M tokens at N = 64): larger calls return MB_ERR_WORKSPACE.  The call
 * allocates nothing.  Calls on one GPU take the scratch one after the other in the order
 * the host makes them, whatever their streams: each call's stream waits for an event the
 * previous call recorded after its last pass (the event is created once per device, with
 * the scratch address).  Under graph capture that ordering is left to the graph, and
 * replays that overlap on one GPU race.
 */
int mb_corpus_states_noalloc(const int64_t *order, const int64_t *chain, int64_t T,
                             const float *rhos, int N, float *states, void *stream);

/*
 * Slot lists of a batch of chunks (first half of the batch builder).  Replaces the slot
 * expansion of WikiTextMMapDataset.__getitem__ (mathbrain/data.py:101-125).  Chunk b is
 * tokens[start[b]:end[b]) of a document that begins at doc_start[b]; its slots are the
 * distinct tokens of the chunk in increasing id order (torch.unique, :103-105), then the
 * distinct tokens of tokens[doc_start[b]:start[b]) that are not in the chunk, in
 * increasing id order (:110-123).
 *
 *   tokens     [T] int32, ids in [0, V) (others are ignored)
 *   next_pos   [T] int32: position of the next occurrence of the same token, >= T if none
 *   doc_start, start, end  [B] int64 on the device; a row without
 *              0 <= doc_start <= start < end <= T is treated as empty
 *   last       [B, V] int32 out: last occurrence before start[b] in the document, or -1
 *   slot_of    [B, V] int32 out: slot of each token in row b, or -1
 *   slot_tok   [B, V] int64 out: token of each slot (the first counts[b][1] entries)
 *   counts     [B, 2] int32 out: (number of chunk tokens, number of slots)
 */
int mb_slot_lists(const int32_t *tokens, const int32_t *next_pos, int64_t T, int64_t V,
                  const int64_t *doc_start, const int64_t *start, const int64_t *end, int B,
                  int32_t *last, int32_t *slot_of, int64_t *slot_tok, int32_t *counts,
                  void *stream);

/*
 * The collated batch (second half).  Replaces the c_base lookup of __getitem__
 * (mathbrain/data.py:127-140) and dynamic_collate_fn (:205-232):
 *
 *   c_base[b,k,:] = states[p,:] * rho^(start[b] - p),  p = last[b, slot_tok[b,k]]
 *
 * (zero when p < 0 or k >= counts[b][1]); unique_slots [B, K_max] int64 (0 past the
 * slots), pad_mask [B, K_max] uint8, and per chunk position chunks [B, L] int64 (0
 * past the chunk), doc_out [B, L] int64 (-1 past), inverse [B, L] int64 (the slot of the
 * token, 0 past).  Inputs as mb_slot_lists plus doc_ids [T] int32, states [T, N] fp32
 * and rhos [N]; K_max >= max_b counts[b][1] and L >= max_b (end[b] - start[b]) give
 * full rows (smaller values truncate).
 */
int mb_slot_batch(const int32_t *tokens, const int32_t *doc_ids, const float *states,
                  const float *rhos, int N, int64_t T, int64_t V, const int64_t *doc_start,
                  const int64_t *start, const int64_t *end, int B, const int32_t *last,
                  const int32_t *slot_of, const int64_t *slot_tok, const int32_t *counts, int L,
                  int K_max, int64_t *chunks, int64_t *doc_out, int64_t *unique_slots,
                  uint8_t *pad_mask, int64_t *inverse, float *c_base, void *stream);

/*
 * Factored linear EMA (mathbrain/factored_ema.py:22-96; the reference is a PyTorch loop
 * with an [N, hd, hd] state per (b, h) updated at every step).  Per sequence b and head h,
 * with q_t = Q[b,t,h*hd:], W_n = W_pe[n,h*hd:], e = E[x[b,s], h*hd:] rows of E_k / E_v:
 *
 *   o_t = sum_{s<t} A[t,s] e_v[x_s] + sum_n rho_n^(t+1) sum_i q_t[i] W_n[i] S_n[i,:]
 *   A[t,s] = sum_i q_t[i] e_k[x_s][i] G[t-s][i],  G[d] = sum_n rho_n^d W_n  ([L+1, D])
 *   S_n = sum_k c_base[b,k,n] e_k[u_k] ⊗ e_v[u_k]   (the initial state, factored_ema.py:52-67)
 *
 * fp32 tensors, rows of D = H*hd elements; head_dim 32 or 64 (at 64 mb_factored_outer and
 * mb_factored_apply run on the bf16 matrix cores with every fp32 operand split into bf16
 * hi + lo, three products and fp32 accumulation: about 2^-16 relative error per product).
 * Token ids outside [0, V) are
 * skipped; gathered row indices are clamped below at 0 (the reference's clamp of -1 slot
 * ids) and skipped at or above nrows.
 *
 * mb_factored_outer: out[b,h,n,i,j] = sum_{r<R} alpha[b*as_b + r*as_r + n*as_n]
 *     * X[row_x(b,r)*ld + h*hd + i] * Y[row_y(b,r)*ld + h*hd + j], row(b,r) = idx[b*R+r] or
 *     b*R + r when idx is NULL; out [B, H, N, hd, hd].  Builds S_n (alpha = c_base, rows =
 *     slots) and, in the backward, M_n = sum_t rho_n^(t+1) q_t ⊗ dO_t.
 */
int mb_factored_outer(const float *X, const int64_t *xrow, const float *Y, const int64_t *yrow,
                      int64_t ld, int64_t nrows, const float *alpha, int64_t as_b, int64_t as_r,
                      int64_t as_n, int B, int R, int H, int N, int hd, float *out, void *stream);

/*
 * mb_factored_apply: contracts a state [B, H, N, hd, hd] with rows,
 *   transpose = 0: out[b,r,h*hd+i] (+)= sum_n alpha[..] sum_j w[n*ldw+h*hd+i] M[b,h,n,i,j] Y[row(b,r),h*hd+j]
 *   transpose = 1: out[b,r,h*hd+j] (+)= sum_n alpha[..] sum_i w[n*ldw+h*hd+i] M[b,h,n,i,j] Y[row(b,r),h*hd+i]
 * (w NULL: 1; accumulate = 1 adds to out, row stride ldo).  The c_base part of the output
 * (M = S, rows Q, transpose 1) and of dQ (rows dO, transpose 0), and the slot gradients
 * from M (rows E_v / E_k of the slots, alpha = c_base).
 */
int mb_factored_apply(const float *M, const float *w, int64_t ldw, const float *Y,
                      const int64_t *yrow, int64_t ld, int64_t nrows, const float *alpha,
                      int64_t as_b, int64_t as_r, int64_t as_n, int B, int R, int H, int N, int hd,
                      int transpose, float *out, int64_t ldo, int accumulate, void *stream);

/*
 * mb_factored_tok_fwd: the token part of o (written, not added): Q [B, L, D], x [B, L]
 * int64, E_k / E_v [V, D], G [L+1, D], O [B, L, D].
 * mb_factored_tok_bwd: its gradients for dO [B, L, D]: dQ [B, L, D] (written), the
 * per-position embedding gradients dEk_tok / dEv_tok [B, L, D] (to be added into rows
 * x[b,s] of dE_k / dE_v) and dG_b [B, L, D] = sum_t dA[t,t-d] q_t ⊙ e_k[x_{t-d}] per
 * sequence (row 0 zero), from which dW_pe = sum_d rho^d sum_b dG_b[b,d].
 */
int mb_factored_tok_fwd(const float *Q, const int64_t *x, int64_t V, const float *E_k,
                        const float *E_v, const float *G, int B, int L, int H, int hd, float *O,
                        void *stream);
int mb_factored_tok_bwd(const float *Q, const float *dO, const int64_t *x, int64_t V,
                        const float *E_k, const float *E_v, const float *G, int B, int L, int H,
                        int hd, float *dQ, float *dEk_tok, float *dEv_tok, float *dG_b,
                        void *stream);

/*
 * RMSNorm.  Replaces RMSNorm.forward (mathbrain/model.py:11-19) and its autograd backward:
 *
 *   mb_rmsnorm_fwd:  rstd[r] = rsqrt(mean_d x[r,d]^2 + eps),  y[r,d] = w[d] * (x[r,d] * rstd[r])
 *   mb_rmsnorm_bwd:  dx[r,d] = rstd (w[d] dy[r,d]) - rstd^3 / D * x[r,d] * sum_e w[e] dy[r,e] x[r,e]
 *                    dw[d]   = sum_r dy[r,d] x[r,d] rstd[r]  (cleared by the call with a fill
 *                    kernel, then accumulated with fp32 atomics: summation order not fixed)
 *
 *   x, dy, y, dx  [rows, D] fp32 contiguous;  w, dw [D] fp32;  rstd [rows] fp32 (written by
 *                 the forward, read by the backward)
 *
 * Supported: 1 <= D <= 1024.
 */
int mb_rmsnorm_fwd(const float *x, const float *w, int64_t rows, int D, float eps, float *y,
                   float *rstd, void *stream);
int mb_rmsnorm_bwd(const float *x, const float *w, const float *dy, const float *rstd,
                   int64_t rows, int D, float *dx, float *dw, void *stream);

/*
 * LayerNorm (the model's ln_kv over the embedding rows, mathbrain/model.py:63-64):
 *
 *   mb_layernorm_fwd:  mean[r] = mean_d x[r,d],  rstd[r] = rsqrt(mean_d (x - mean)^2 + eps),
 *                      y[r,d] = (x[r,d] - mean[r]) rstd[r] w[d] + b[d]
 *   mb_layernorm_bwd:  with xh = (x - mean) rstd and g = dy w:
 *                      dx = rstd (g - mean_d g - xh mean_d(g xh)),
 *                      dw = sum_r dy xh,  db = sum_r dy  (cleared by the call with a fill
 *                      kernel, then accumulated with fp32 atomics: summation order not fixed)
 *
 *   x, dy, y, dx [rows, D] fp32 contiguous;  w, b, dw, db [D] fp32;  mean, rstd [rows] fp32
 *   (written by the forward, read by the backward).  Supported: 1 <= D <= 1024.
 */
int mb_layernorm_fwd(const float *x, const float *w, const float *b, int64_t rows, int D, float eps,
                     float *y, float *mean, float *rstd, void *stream);
int mb_layernorm_bwd(const float *x, const float *w, const float *dy, const float *mean,
                     const float *rstd, int64_t rows, int D, float *dx, float *dw, float *db,
                     void *stream);

/* Element types of the entry points that take either. */
#define MB_DTYPE_F32 0
#define MB_DTYPE_BF16 1

/*
 * SwiGLU gate product.  Replaces the elementwise part of SwiGLU.forward
 * (mathbrain/model.py:21-29), F.silu(w1(x)) * w3(x), and its autograd backward:
 *
 *   mb_swiglu_fwd:  m  = SiLU(a) * b
 *   mb_swiglu_bwd:  da = dm * b * s (1 + a (1 - s)),  db = dm * SiLU(a),  s = sigmoid(a)
 *
 *   a = w1(x), b = w3(x), m, dm, da, db: n elements each, contiguous, all of one dtype
 *   (MB_DTYPE_F32 or MB_DTYPE_BF16), 32-byte aligned (vector loads; others are rejected);
 *   evaluated in fp32, rounded once to the dtype.
 */
int mb_swiglu_fwd(const void *a, const void *b, int64_t n, int dtype, void *m, void *stream);
int mb_swiglu_bwd(const void *a, const void *b, const void *dm, int64_t n, int dtype, void *da,
                  void *db, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MATHBRAIN_HIP_H */
