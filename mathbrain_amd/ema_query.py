"""Query-side EMA history: the per-position counter rows C_seq that gate the queries.

Drop-in for mathbrain/triton_ema_query.py:120-169 (``compute_query_ema_history``) and
:67-117 (``compute_query_ema_history_pt``, the same scan under the reference's second
name); the work runs in the gfx950 kernel behind ``mb_ema_query_scan``.
"""
import torch

from . import _lib


def compute_query_ema_history(x, rhos, vocab_size, c_init=None, c_init_keys=None, doc_ids=None,
                              return_state=False):
    """EMA history of x_t just before t, for every position (triton_ema_query.py:120).

    C_seq[b,t,:] = c0[b,x_t,:] rho^t + sum_{s<t, x_s=x_t} rho^(t-s), the c0 term present
    when x_t is one of c_init_keys[b] (-1 keys are padding; a repeated key keeps its last
    row).  With doc_ids a token whose previous occurrence is in another document restarts
    from 0 (triton_ema_query.py:51-57, 104-110).

    x [B, L] int64, rhos [N], c_init [B, K, N], c_init_keys [B, K], doc_ids [B, L].
    Returns C_seq [B, L, N] float32.  With ``return_state=True`` also returns
    (state, stamps): ``state`` [B, K, N] is c_init with each key that occurs in the chunk
    replaced by its lazy state after its last occurrence (C_seq there + 1) and ``stamps``
    [B, K] int32 is that position (-1 for keys that do not occur); the state at position p
    is state * rho^(p - stamp).
    """
    dev = _lib.require_gpu(x, rhos, c_init, c_init_keys, doc_ids, what="compute_query_ema_history")
    B, L = x.shape
    N = rhos.shape[0]
    x = x if x.dtype == torch.int64 else x.long()
    rhos_f = rhos.detach().to(torch.float32).contiguous()
    has_init = c_init is not None and c_init_keys is not None
    if has_init:
        ci = c_init.detach().to(torch.float32).contiguous()
        keys = c_init_keys.to(torch.int64).contiguous()
        if ci.shape[0] != B or ci.shape[2] != N or keys.shape != ci.shape[:2]:
            raise ValueError(f"c_init {tuple(ci.shape)} / c_init_keys {tuple(keys.shape)} "
                             f"do not match B={B}, N={N}")
        K = keys.shape[1]
    else:
        ci = keys = None
        K = 0
    docs = None
    if doc_ids is not None:
        docs = doc_ids.to(torch.int64).contiguous()
        if docs.shape != (B, L):
            raise ValueError(f"doc_ids {tuple(docs.shape)} must be [B, L] = {(B, L)}")
    C_seq = torch.empty(B, L, N, dtype=torch.float32, device=dev)
    state = stamps = None
    if return_state:
        state = ci.clone() if has_init else torch.empty(B, 0, N, dtype=torch.float32, device=dev)
        stamps = torch.empty(B, K, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_ema_query_scan", _lib.ptr(x), x.stride(0), x.stride(1), B, L,
                  _lib.ptr(rhos_f), N, int(vocab_size), _lib.ptr(ci), _lib.ptr(keys), K,
                  _lib.ptr(docs), _lib.ptr(C_seq),
                  _lib.ptr(state) if (return_state and K) else None,
                  _lib.ptr(stamps) if (return_state and K) else None, _lib.stream(dev))
    if return_state:
        return C_seq, state, stamps
    return C_seq


def compute_query_ema_history_pt(x, rhos, vocab_size, c_init=None, c_init_keys=None, doc_ids=None):
    """The reference's second name for the same scan (triton_ema_query.py:67-117, its
    PyTorch loop).  Same semantics and arguments; here it runs the same HIP kernel as
    ``compute_query_ema_history`` and, like it, needs GPU tensors (there is no CPU path)."""
    return compute_query_ema_history(x, rhos, vocab_size, c_init, c_init_keys, doc_ids)
