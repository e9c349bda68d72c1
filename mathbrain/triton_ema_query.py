"""Query-side EMA history: the per-position counter rows C_seq that gate the queries.

Drop-in for mathbrain/triton_ema_query.py:120-169 (``compute_query_ema_history``) and
:67-117 (``compute_query_ema_history_pt``, the same scan under the reference's second
name); the work runs in the gfx950 kernel behind ``mb_ema_query_scan``, registered as the torch op
mathbrain::ema_query_scan for tracing.
"""
from typing import Optional

import torch

from . import _lib


def _check(x, rhos, c_init, c_init_keys, doc_ids):
    B, L = x.shape
    N = rhos.shape[0]
    if c_init is not None and c_init_keys is not None:
        if c_init.shape[0] != B or c_init.shape[2] != N or tuple(c_init_keys.shape) != tuple(c_init.shape[:2]):
            raise ValueError(f"c_init {tuple(c_init.shape)} / c_init_keys {tuple(c_init_keys.shape)} "
                             f"do not match B={B}, N={N}")
    if doc_ids is not None and tuple(doc_ids.shape) != (B, L):
        raise ValueError(f"doc_ids {tuple(doc_ids.shape)} must be [B, L] = {(B, L)}")


def _scan(x, rhos, vocab_size, c_init, c_init_keys, doc_ids, state, stamps):
    dev = _lib.require_gpu(x, rhos, c_init, c_init_keys, doc_ids, what="compute_query_ema_history")
    _check(x, rhos, c_init, c_init_keys, doc_ids)
    B, L = x.shape
    N = rhos.shape[0]
    x = x if x.dtype == torch.int64 else x.long()
    rhos_f = rhos.detach().to(torch.float32).contiguous()
    ci = keys = None
    K = 0
    if c_init is not None and c_init_keys is not None:
        ci = c_init.detach().to(torch.float32).contiguous()
        keys = c_init_keys.to(torch.int64).contiguous()
        K = keys.shape[1]
    docs = None if doc_ids is None else doc_ids.to(torch.int64).contiguous()
    C_seq = torch.empty(B, L, N, dtype=torch.float32, device=dev)
    # Sequences longer than the one-launch limit run in pieces with a [B, vocab_size] int32
    # table of each token's last position between them (mb_ema_query_scan_workspace bytes).
    nws = _lib.lib().mb_ema_query_scan_workspace(B, L, int(vocab_size))
    if nws < 0:
        raise _lib.HipKernelError("mb_ema_query_scan_workspace: " + _lib.lib().mb_last_error().decode(errors="replace"))
    ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws > 0 else None
    with torch.cuda.device(dev):
        _lib.call("mb_ema_query_scan_ws", _lib.ptr(x), x.stride(0), x.stride(1), B, L,
                  _lib.ptr(rhos_f), N, int(vocab_size), _lib.ptr(ci), _lib.ptr(keys), K,
                  _lib.ptr(docs), _lib.ptr(C_seq), _lib.ptr(state) if K else None,
                  _lib.ptr(stamps) if K else None, _lib.ptr(ws), int(nws), _lib.stream(dev))
    return C_seq


def _scan_fake(x, rhos, vocab_size, c_init, c_init_keys, doc_ids):
    return x.new_empty((x.shape[0], x.shape[1], rhos.shape[0]), dtype=torch.float32)


@_lib.traced_op("ema_query_scan", _scan_fake)
def ema_query_scan(x: torch.Tensor, rhos: torch.Tensor, vocab_size: int, c_init: Optional[torch.Tensor],
                   c_init_keys: Optional[torch.Tensor], doc_ids: Optional[torch.Tensor]) -> torch.Tensor:
    """C_seq [B, L, N] of compute_query_ema_history (one mb_ema_query_scan launch)."""
    return _scan(x, rhos, vocab_size, c_init, c_init_keys, doc_ids, None, None)


def compute_query_ema_history(x, rhos, vocab_size, c_init=None, c_init_keys=None, doc_ids=None,
                              return_state=False):
    """EMA history of x_t just before t, for every position (triton_ema_query.py:120).

    C_seq[b,t,:] = c0[b,x_t,:] rho^t + sum_{s<t, x_s=x_t} rho^(t-s), the c0 term present
    when x_t is one of c_init_keys[b] (-1 keys are padding; a repeated key keeps its last
    row).  With doc_ids a token whose previous occurrence is in another document restarts
    from 0 (triton_ema_query.py:51-57, 104-110).

    x [B, L] int64, rhos [N], c_init [B, K, N], c_init_keys [B, K], doc_ids [B, L].
    Token ids must lie in [0, vocab_size) (as the reference's [B, V+1] tables need).  Any L:
    beyond 8192 steps the scan runs in 2048-step pieces.
    Returns C_seq [B, L, N] float32.  With ``return_state=True`` also returns
    (state, stamps): ``state`` [B, K, N] is c_init with each key that occurs in the chunk
    replaced by its lazy state after its last occurrence (C_seq there + 1) and ``stamps``
    [B, K] int32 is that position (-1 for keys that do not occur); the state at position p
    is state * rho^(p - stamp).
    """
    if c_init is None or c_init_keys is None:
        c_init = c_init_keys = None
    if not return_state:
        return ema_query_scan(x, rhos, int(vocab_size), c_init, c_init_keys, doc_ids)
    dev = _lib.require_gpu(x, rhos, c_init, c_init_keys, doc_ids, what="compute_query_ema_history")
    B, N = x.shape[0], rhos.shape[0]
    if c_init is not None:
        state = c_init.detach().to(torch.float32).contiguous().clone()
        stamps = torch.empty(c_init_keys.shape, dtype=torch.int32, device=dev)
    else:
        state = torch.empty(B, 0, N, dtype=torch.float32, device=dev)
        stamps = torch.empty(B, 0, dtype=torch.int32, device=dev)
    C_seq = _scan(x, rhos, vocab_size, c_init, c_init_keys, doc_ids, state, stamps)
    return C_seq, state, stamps


def compute_query_ema_history_pt(x, rhos, vocab_size, c_init=None, c_init_keys=None, doc_ids=None):
    """The reference's second name for the same scan (triton_ema_query.py:67-117, its
    PyTorch loop).  Same semantics and arguments; here it runs the same HIP kernel as
    ``compute_query_ema_history`` and, like it, needs GPU tensors (there is no CPU path)."""
    return compute_query_ema_history(x, rhos, vocab_size, c_init, c_init_keys, doc_ids)
