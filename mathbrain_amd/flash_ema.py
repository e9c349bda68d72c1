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


def _flash_flags(use_silu, absent_mass, vocab_rows=False):
    return ((_lib.MB_FLASH_SILU if use_silu else 0) | (_lib.MB_FLASH_ABSENT_MASS if absent_mass else 0)
            | (_lib.MB_FLASH_VOCAB_ROWS if vocab_rows else 0))


def _slot_rows(E, B, K, D, V_total, what):
    """E_k / E_v in fp32: [B, K, D] gathered slot rows, or a [V_total, D] vocabulary table
    whose row unique[b, k] is slot (b, k)'s (returns the tensor and whether it is a table)."""
    Ef = E.to(torch.float32)
    if Ef.dim() == 2:
        if Ef.shape != (V_total, D):
            raise ValueError(f"{what}: a vocabulary table must be [V_total, H*hd] = {(V_total, D)}, "
                             f"got {tuple(Ef.shape)}")
        return Ef.contiguous(), True
    Ef = Ef.reshape(B, K, D) if Ef.dim() == 4 and Ef.shape[:2] == (B, K) else Ef
    if Ef.shape != (B, K, D):
        raise ValueError(f"{what}: E_k/E_v must be [B, K_max, H*hd] = {(B, K, D)} or a "
                         f"[V_total, H*hd] table, got {tuple(E.shape)}")
    return Ef.contiguous(), False


def flash_ema_forward(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor, K_max,
                      C_bounds, use_silu=True, Br=64, absent_mass=True, return_scores=False):
    """Gated flash-EMA attention forward (triton_flash_ema.py:529-568).

    Q [B, H, L, hd]; x [B, L]; E_k_active / E_v_active [B, K_max, H*hd]; W_pe [N, H*hd]
    (pe_proj.weight.t()); rhos [N]; unique_tensor [B, K_max] (-1 = padding); C_bounds
    from ``precompute_boundaries(x, unique_tensor, rhos, Br, c_init)``.  Float inputs are
    used in fp32, as the reference's ``custom_fwd(cast_inputs=float32)`` does.
    E_k_active / E_v_active may instead be [V_total, H*hd] vocabulary tables (the
    projections of every embedding row): slot (b, k) then reads row unique_tensor[b, k],
    the same values the [B, K_max] gather would hold, without the gather.

    Returns (O [B, H, L, hd] fp32, LSE [B, H, L], C_bounds, E_k, E_v) with E_k/E_v viewed
    [B, K_max, H, hd], as the reference does (tables are returned as given, in fp32).  With ``absent_mass`` (the default) the
    softmax covers all V_total slots as the dense PyTorch reference
    (flash_ema_attention.py:76-77) does; ``absent_mass=False`` gives the Triton kernel's
    softmax over the valid slots only (triton_flash_ema.py:215-229).  With
    ``return_scores`` a sixth element holds the scores * log2(e) as [B, H, K_max, L]
    (what ``flash_ema_backward(scores=...)`` consumes instead of recomputing them).
    """
    dev = _lib.require_gpu(Q, x, E_k_active, E_v_active, W_pe, rhos, unique_tensor, C_bounds,
                           what="flash_ema_forward")
    B, H, L, hd = Q.shape
    K = unique_tensor.shape[1]
    if K != K_max:
        raise ValueError(f"unique_tensor has {K} slots but K_max={K_max}")
    N = rhos.shape[0]
    D = H * hd
    Qf = Q.to(torch.float32)
    Ek, table = _slot_rows(E_k_active, B, K, D, int(V_total), "flash_ema_forward")
    Ev, table_v = _slot_rows(E_v_active, B, K, D, int(V_total), "flash_ema_forward")
    if table != table_v:
        raise ValueError("flash_ema_forward: E_k and E_v must both be tables or both gathered rows")
    W = W_pe.to(torch.float32).contiguous()
    if W.shape[0] < N or W.shape[1] != D:
        raise ValueError(f"W_pe must be [N, H*hd] = {(N, D)}, got {tuple(W.shape)}")
    W = W[:N].contiguous()
    rh = rhos.detach().to(torch.float32).contiguous()
    uniq = unique_tensor.to(torch.int64).contiguous()
    xl = x if x.dtype == torch.int64 else x.long()
    Cb = C_bounds.to(torch.float32).contiguous()
    if Cb.dim() != 4 or Cb.shape[0] != B or Cb.shape[2] != K or Cb.shape[3] < N:
        raise ValueError(f"C_bounds must be [B, nc, K_max, >=N], got {tuple(Cb.shape)}")
    O = torch.empty(B, H, L, hd, dtype=torch.float32, device=dev)
    LSE = torch.empty(B, H, L, dtype=torch.float32, device=dev)
    S2 = torch.empty(B, H, K, L, dtype=torch.float32, device=dev) if return_scores else None
    with torch.cuda.device(dev):
        _lib.call("mb_flash_ema_fwd", _lib.ptr(Qf), *Qf.stride(), _lib.ptr(xl), xl.stride(0),
                  xl.stride(1), _lib.ptr(Ek), _lib.ptr(Ev), _lib.ptr(W), _lib.ptr(rh),
                  _lib.ptr(uniq), _lib.ptr(Cb), B, H, L, hd, K, N, Cb.shape[3], Cb.shape[1],
                  int(Br), int(V_total), _flash_flags(use_silu, absent_mass, table), _lib.ptr(O),
                  _lib.ptr(LSE), _lib.ptr(S2), _lib.stream(dev))
    if table:
        out = (O, LSE, C_bounds, Ek, Ev)
    else:
        out = (O, LSE, C_bounds, Ek.view(B, K, H, hd), Ev.view(B, K, H, hd))
    return out + (S2,) if return_scores else out


def flash_ema_backward(Q, x, E_k, E_v, W_pe, rhos, V_total, unique_tensor, C_bounds, O, LSE, dO,
                       use_silu=True, Br=64, absent_mass=True, scores=None):
    """Gradients of flash_ema_forward (triton_flash_ema.py:586-650) in one fused HIP pass.

    E_k / E_v are [B, K, H*hd] or [B, K, H, hd], or [V_total, H*hd] vocabulary tables (then
    dE_k / dE_v are tables too: each row sums the gradients of every slot of that token);
    ``scores`` is the forward's optional scores output (recomputed when None).  Returns
    (dQ [B,H,L,hd], dE_k [B,K,H*hd], dE_v [B,K,H*hd], dW_pe [N, H*hd]), all fp32.
    """
    dev = _lib.require_gpu(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO,
                           what="flash_ema_backward")
    B, H, L, hd = Q.shape
    K = unique_tensor.shape[1]
    N = rhos.shape[0]
    D = H * hd
    Qf = Q.to(torch.float32)
    dOf = dO.to(torch.float32)
    if dOf.stride() != Qf.stride():
        Qf = Qf.contiguous()
        dOf = dOf.contiguous()
    Ek, table = _slot_rows(E_k, B, K, D, int(V_total), "flash_ema_backward")
    Ev, table_v = _slot_rows(E_v, B, K, D, int(V_total), "flash_ema_backward")
    if table != table_v:
        raise ValueError("flash_ema_backward: E_k and E_v must both be tables or both gathered rows")
    W = W_pe.to(torch.float32)[:N].contiguous()
    rh = rhos.detach().to(torch.float32).contiguous()
    uniq = unique_tensor.to(torch.int64).contiguous()
    xl = x if x.dtype == torch.int64 else x.long()
    Cb = C_bounds.to(torch.float32).contiguous()
    Of = O.to(torch.float32).contiguous()
    Lf = LSE.to(torch.float32).contiguous()
    dQ = torch.empty(B, H, L, hd, dtype=torch.float32, device=dev)
    dEk = torch.empty(Ek.shape, dtype=torch.float32, device=dev)
    dEv = torch.empty(Ev.shape, dtype=torch.float32, device=dev)
    dW = torch.empty(N, D, dtype=torch.float32, device=dev)
    if scores is not None and (scores.shape != (B, H, K, L) or scores.dtype != torch.float32
                               or not scores.is_contiguous()):
        raise ValueError(f"scores must be contiguous fp32 [B, H, K_max, L], got {tuple(scores.shape)}")
    with torch.cuda.device(dev):
        _lib.call("mb_flash_ema_bwd", _lib.ptr(Qf), *Qf.stride(), _lib.ptr(dOf), _lib.ptr(xl),
                  xl.stride(0), xl.stride(1), _lib.ptr(Ek), _lib.ptr(Ev), _lib.ptr(W),
                  _lib.ptr(rh), _lib.ptr(uniq), _lib.ptr(Cb), _lib.ptr(Of), _lib.ptr(Lf), B, H, L,
                  hd, K, N, Cb.shape[3], Cb.shape[1], int(Br), int(V_total),
                  _flash_flags(use_silu, absent_mass, table), _lib.ptr(scores), _lib.ptr(dQ),
                  _lib.ptr(dEk), _lib.ptr(dEv), _lib.ptr(dW), _lib.stream(dev))
    return dQ, dEk, dEv, dW


# With SAVE_SCORES, FlashEMAFunction keeps the forward's scores ([B, H, K_max, L] fp32,
# 1.4 GB at B=56, T=512, H=8, K_max=1638) and the backward skips recomputing them.  Off by
# default: on gfx950 the extra live registers of that variant cost more than the skipped
# score arithmetic (configuration 2: backward 23.0 ms recomputing vs 23.5 ms reading them,
# and 0.3 ms more in the forward to write them).
SAVE_SCORES = False


class FlashEMAFunction(torch.autograd.Function):
    """Autograd entry point with the reference's 12 arguments (triton_flash_ema.py:571-650):
    apply(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor, K_max, C_bounds,
    use_silu=True, Br=64) -> O [B, H, L, hd].  Inputs are used in fp32 (the reference's
    custom_fwd(cast_inputs=float32)); gradients flow to Q, E_k_active, E_v_active, W_pe."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda", cast_inputs=torch.float32)
    def forward(ctx, Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor, K_max,
                C_bounds, use_silu=True, Br=64):
        res = flash_ema_forward(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor,
                                K_max, C_bounds, use_silu, Br, return_scores=SAVE_SCORES)
        O, LSE, C_bounds, E_k, E_v = res[:5]
        ctx.save_for_backward(Q, x, E_k, E_v, W_pe, rhos, C_bounds, unique_tensor, O, LSE,
                              res[5] if SAVE_SCORES else None)
        ctx.V_total = V_total
        ctx.use_silu = use_silu
        ctx.Br = Br
        ctx.W_rows = W_pe.shape[0]
        return O

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dO):
        Q, x, E_k, E_v, W_pe, rhos, C_bounds, unique_tensor, O, LSE, S2 = ctx.saved_tensors
        dQ, dEk, dEv, dW = flash_ema_backward(Q, x, E_k, E_v, W_pe, rhos, ctx.V_total,
                                              unique_tensor, C_bounds, O, LSE, dO.contiguous(),
                                              ctx.use_silu, ctx.Br, scores=S2)
        if ctx.W_rows > dW.shape[0]:  # W_pe passed with padded rows: their gradient is 0
            dW = torch.cat([dW, dW.new_zeros(ctx.W_rows - dW.shape[0], dW.shape[1])])
        return dQ, None, dEk, dEv, dW, None, None, None, None, None, None, None
