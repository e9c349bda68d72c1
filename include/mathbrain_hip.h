/*
 * mathbrain_hip.h -- C ABI of the MI355X (gfx950) Per-Slot EMA hot path.
 *
 * Every entry point takes device pointers, plain sizes and strides, and a HIP stream
 * (hipStream_t passed as void*; NULL = the null stream).  Nothing here allocates:
 * callers pass every output buffer and, where a call needs one, a workspace whose size
 * the matching *_workspace_size() call returns.  Calls are asynchronous on the stream.
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

/* ABI version of this library (bumped on any signature change). */
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
 * Limits: L <= 8192 (the per-sequence index lives in the 160 KB LDS of one CU).
 */
int mb_ema_query_scan(const int64_t *x, int64_t x_stride_b, int64_t x_stride_l, int B, int L,
                      const float *rhos, int N, int64_t vocab_size, const float *c_init,
                      const int64_t *c_init_keys, int K, const int64_t *doc_ids, float *C_seq,
                      float *state_out, int32_t *stamp_out, void *stream);

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
 * Limits: L <= 8192.
 */
int mb_ema_boundary_states(const int64_t *x, int64_t x_stride_b, int64_t x_stride_l, int B,
                           int L, const int64_t *unique, int K, const float *rhos, int N, int Br,
                           const float *c_init, int64_t c_init_stride_k, const int64_t *doc_ids,
                           float *C_bounds, int Np, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MATHBRAIN_HIP_H */
