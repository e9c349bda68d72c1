"""Flash-EMA gated cross-attention over the unique slots of each sequence.

Drop-in for mathbrain/triton_flash_ema.py: ``precompute_boundaries`` (:81-113),
``_build_unique_index`` (:475-507), ``flash_ema_forward`` (:529-568),
``FlashEMAFunction`` (:571-650) and the module flag ``HAS_TRITON`` (:16-21).  The
kernels are the gfx950 ones behind the C ABI in include/mathbrain_hip.h.
"""
import math

import torch

from . import _lib

# model.py dispatches its device path on `HAS_TRITON and device.type == 'cuda'`
# (model.py:78, 162).  Here the device path is always the HIP one; it raises when its
# library is missing rather than falling back, so the flag is a constant.
HAS_TRITON = True


def precompute_boundaries(x, unique_tensor, rhos, Br, c_init=None, doc_ids=None):
    """Key-side EMA state of every slot at the start of each Br-step chunk
    (triton_flash_ema.py:81-113).

    C_bounds[b,j,k,:] = c0[b,k] rho^(jBr) + sum_{s<jBr, x_s=u_k} rho^(jBr-1-s), stored
    before chunk j runs, as [B, max(1, ceil(L/Br)), K, max(N, 16)] float32 (the N
    padding columns are zero).
    """
    dev = _lib.require_gpu(x, unique_tensor, rhos, c_init, doc_ids, what="precompute_boundaries")
    B, L = x.shape
    K = unique_tensor.shape[1]
    N = rhos.shape[0]
    Np = max(N, 16)
    nc = max(1, -(-L // Br))
    x = x if x.dtype == torch.int64 else x.long()
    uniq = unique_tensor.to(torch.int64).contiguous()
    rhos_f = rhos.detach().to(torch.float32).contiguous()
    ci = None
    if c_init is not None:
        ci = c_init.detach().to(torch.float32).contiguous()
        if ci.shape[0] != B or ci.shape[1] != K or ci.shape[2] < N:
            raise ValueError(f"c_init {tuple(ci.shape)} must be [B={B}, K={K}, >=N={N}]")
    docs = None if doc_ids is None else doc_ids.to(torch.int64).contiguous()
    out = torch.empty(B, nc, K, Np, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_ema_boundary_states", _lib.ptr(x), x.stride(0), x.stride(1), B, L,
                  _lib.ptr(uniq), K, _lib.ptr(rhos_f), N, int(Br), _lib.ptr(ci),
                  ci.shape[2] if ci is not None else 0, _lib.ptr(docs), _lib.ptr(out), Np,
                  _lib.stream(dev))
    return out


def _build_unique_index(x, device):
    """Sorted unique ids of each row, compacted to the front and -1 padded, with
    K_max = max(max unique count, 16) (triton_flash_ema.py:475-507)."""
    B, L = x.shape
    x_sorted, _ = torch.sort(x, dim=1)
    is_first = torch.ones(B, L, dtype=torch.bool, device=device)
    is_first[:, 1:] = x_sorted[:, 1:] != x_sorted[:, :-1]
    counts = is_first.sum(dim=1)
    K_max = max(int(counts.max().item()), 16)
    perm = (~is_first).long().argsort(dim=1, stable=True)
    out = torch.full((B, K_max), -1, dtype=x.dtype, device=device)
    n_take = min(perm.shape[1], K_max)
    out[:, :n_take] = x_sorted.gather(1, perm)[:, :n_take]
    pad = torch.arange(K_max, device=device).unsqueeze(0) >= counts.unsqueeze(1)
    out.masked_fill_(pad, -1)
    return out, K_max
