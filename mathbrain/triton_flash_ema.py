"""Flash-EMA gated cross-attention over the unique slots of each sequence.

Drop-in for the reference's mathbrain/triton_flash_ema.py: ``precompute_boundaries``
(:81-113), ``_build_unique_index`` (:475-507), ``flash_ema_forward`` (:529-568),
``FlashEMAFunction`` (:571-650) and the module flag ``HAS_TRITON`` (:16-21).  The kernels
are the gfx950 ones behind the C ABI in include/mathbrain_hip.h; each launch is also
registered as a torch op (mathbrain::boundary_states, unique_rows, flash_ema_fwd,
flash_ema_bwd) so that torch.compile traces through the attention instead of breaking
the graph at the ctypes call.
"""
import functools
from typing import Optional

import torch

from . import _lib

# model.py dispatches its device path on `HAS_TRITON and device.type == 'cuda'`
# (model.py:78, 162).  Here the device path is always the HIP one; it raises when its
# library is missing rather than falling back, so the flag is a constant.
HAS_TRITON = True


def _boundary_fake(x, unique_tensor, rhos, Br, c_init, doc_ids):
    B, L = x.shape
    nc = max(1, -(-L // Br))
    return x.new_empty((B, nc, unique_tensor.shape[1], max(rhos.shape[0], 16)), dtype=torch.float32)


@_lib.traced_op("boundary_states", _boundary_fake)
def boundary_states(x: torch.Tensor, unique_tensor: torch.Tensor, rhos: torch.Tensor, Br: int,
                    c_init: Optional[torch.Tensor], doc_ids: Optional[torch.Tensor]) -> torch.Tensor:
    """C_bounds of precompute_boundaries (one mb_ema_boundary_states launch)."""
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


def precompute_boundaries(x, unique_tensor, rhos, Br, c_init=None, doc_ids=None):
    """Key-side EMA state of every slot at the start of each Br-step chunk
    (triton_flash_ema.py:81-113).

    C_bounds[b,j,k,:] = c0[b,k] rho^(jBr) + sum_{s<jBr, x_s=u_k} rho^(jBr-1-s), stored
    before chunk j runs, as [B, max(1, ceil(L/Br)), K, max(N, 16)] float32 (the N
    padding columns are zero).
    """
    return boundary_states(x, unique_tensor, rhos, int(Br), c_init, doc_ids)


def _unique_fake(x, width):
    return (x.new_empty((x.shape[0], width), dtype=torch.int64),
            x.new_empty((x.shape[0],), dtype=torch.int32))


@_lib.traced_op("unique_rows", _unique_fake)
def unique_rows(x: torch.Tensor, width: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(ids [B, width] int64, counts [B] int32): each row's distinct ids in increasing order,
    then -1 (one mb_unique_rows launch, a workgroup per row)."""
    dev = _lib.require_gpu(x, what="_build_unique_index")
    B, L = x.shape
    xl = x if x.dtype == torch.int64 else x.long()
    out = torch.empty(B, width, dtype=torch.int64, device=dev)
    counts = torch.empty(B, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_unique_rows", _lib.ptr(xl), xl.stride(0), xl.stride(1), B, L, _lib.ptr(out),
                  width, _lib.ptr(counts), _lib.stream(dev))
    return out, counts


def _build_unique_index(x, device, width=None):
    """Each row's distinct token ids in increasing order, then -1 padding, and K_max, the
    padded width (triton_flash_ema.py:475-507; the same output).

    By default K_max = max(largest distinct count, 16), as the reference computes it, which
    takes one read of that count back to the host.  With ``width`` the rows are padded to
    K_max = max(width, 16) instead and nothing is read back (``width`` >= L keeps every id;
    the attention skips the extra -1 slots).
    """
    if x.device.type != "cuda":
        raise NotImplementedError("_build_unique_index: tensors must be on an MI355X GPU; this "
                                  "implementation has no CPU path")
    L = x.shape[1]
    if width is not None:
        K_max = max(int(width), 16)
        ids, _ = unique_rows(x, K_max)
        return ids.to(x.dtype), K_max
    ids, counts = unique_rows(x, max(L, 16))
    K_max = max(int(counts.max()) if counts.numel() else 0, 16)
    return ids[:, :K_max].contiguous().to(x.dtype), K_max


PRECISIONS = ("bf16", "fp32")


def _fp32(precision):
    if precision not in PRECISIONS:
        raise ValueError(f"precision must be one of {PRECISIONS}, got {precision!r}")
    return precision == "fp32"


def _flash_flags(use_silu, absent_mass, vocab_rows=False, fp32=False):
    return ((_lib.MB_FLASH_SILU if use_silu else 0) | (_lib.MB_FLASH_ABSENT_MASS if absent_mass else 0)
            | (_lib.MB_FLASH_VOCAB_ROWS if vocab_rows else 0) | (_lib.MB_FLASH_FP32 if fp32 else 0))


def _slot_rows(E, B, K, D, V_total, what):
    """E_k / E_v in fp32: [B, K, D] gathered slot rows, or a [V_total, D] vocabulary table
    whose row unique[b, k] is slot (b, k)'s (returns the tensor and whether it is a table)."""
    Ef = E.to(torch.float32)
    if Ef.dim() == 2:
        if tuple(Ef.shape) != (V_total, D):
            raise ValueError(f"{what}: a vocabulary table must be [V_total, H*hd] = {(V_total, D)}, "
                             f"got {tuple(Ef.shape)}")
        return Ef.contiguous(), True
    Ef = Ef.reshape(B, K, D) if Ef.dim() == 4 and tuple(Ef.shape[:2]) == (B, K) else Ef
    if tuple(Ef.shape) != (B, K, D):
        raise ValueError(f"{what}: E_k/E_v must be [B, K_max, H*hd] = {(B, K, D)} or a "
                         f"[V_total, H*hd] table, got {tuple(E.shape)}")
    return Ef.contiguous(), False


def _fwd_impl(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, V_total, use_silu, Br,
              absent_mass, return_scores, fp32=False):
    dev = _lib.require_gpu(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds,
                           what="flash_ema_forward")
    B, H, L, hd = Q.shape
    K = unique_tensor.shape[1]
    N = rhos.shape[0]
    D = H * hd
    Qf = Q.to(torch.float32)
    Ek, table = _slot_rows(E_k, B, K, D, int(V_total), "flash_ema_forward")
    Ev, table_v = _slot_rows(E_v, B, K, D, int(V_total), "flash_ema_forward")
    if table != table_v:
        raise ValueError("flash_ema_forward: E_k and E_v must both be tables or both gathered rows")
    W = W_pe.to(torch.float32)
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
    flags = _flash_flags(use_silu, absent_mass, table, fp32)
    with torch.cuda.device(dev):
        nws = _fwd_workspace_bytes(B, H, L, hd, K, N, flags, dev.index)
        ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws > 0 else None
        _lib.call("mb_flash_ema_fwd", _lib.ptr(Qf), *Qf.stride(), _lib.ptr(xl), xl.stride(0),
                  xl.stride(1), _lib.ptr(Ek), _lib.ptr(Ev), _lib.ptr(W), _lib.ptr(rh),
                  _lib.ptr(uniq), _lib.ptr(Cb), B, H, L, hd, K, N, Cb.shape[3], Cb.shape[1],
                  int(Br), int(V_total), flags, _lib.ptr(O), _lib.ptr(LSE), _lib.ptr(S2), _lib.ptr(ws), nws,
                  _lib.stream(dev))
    return O, LSE, S2, Ek, Ev, table


@functools.lru_cache(maxsize=256)
def _fwd_workspace_bytes(B, H, L, hd, K, N, flags, device_index):
    """Bytes of the forward's slot-split workspace (mb_flash_ema_fwd_workspace) on the
    current device, which is `device_index`."""
    n = _lib.lib().mb_flash_ema_fwd_workspace(B, H, L, hd, K, N, flags)
    if n < 0:
        raise _lib.HipKernelError("mb_flash_ema_fwd_workspace: " + _lib.lib().mb_last_error().decode(errors="replace"))
    return int(n)


def _fwd_fake(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, V_total, use_silu, Br, absent_mass,
              fp32):
    B, H, L, hd = Q.shape
    return Q.new_empty((B, H, L, hd), dtype=torch.float32), Q.new_empty((B, H, L), dtype=torch.float32)


@_lib.traced_op("flash_ema_fwd", _fwd_fake)
def flash_ema_fwd(Q: torch.Tensor, x: torch.Tensor, E_k: torch.Tensor, E_v: torch.Tensor,
                  W_pe: torch.Tensor, rhos: torch.Tensor, unique_tensor: torch.Tensor,
                  C_bounds: torch.Tensor, V_total: int, use_silu: bool, Br: int,
                  absent_mass: bool, fp32: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE) of flash_ema_forward (mb_flash_ema_fwd: one launch, and a merge launch when it
    splits the slots into parts)."""
    O, LSE = _fwd_impl(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, V_total, use_silu, Br,
                       absent_mass, False, fp32)[:2]
    return O, LSE


def flash_ema_forward(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor, K_max,
                      C_bounds, use_silu=True, Br=64, absent_mass=True, return_scores=False,
                      precision="bf16"):
    """Gated flash-EMA attention forward (triton_flash_ema.py:529-568).

    Q [B, H, L, hd]; x [B, L]; E_k_active / E_v_active [B, K_max, H*hd]; W_pe [N, H*hd]
    (pe_proj.weight.t()); rhos [N]; unique_tensor [B, K_max] (-1 = padding); C_bounds
    from ``precompute_boundaries(x, unique_tensor, rhos, Br, c_init)``.  Float inputs are
    used in fp32, as the reference's ``custom_fwd(cast_inputs=float32)`` does.
    E_k_active / E_v_active may instead be [V_total, H*hd] vocabulary tables (the
    projections of every embedding row): slot (b, k) then reads row unique_tensor[b, k],
    the same values the [B, K_max] gather would hold, without the gather.

    Returns (O [B, H, L, hd] fp32, LSE [B, H, L], C_bounds, E_k, E_v) with E_k/E_v viewed
    [B, K_max, H, hd], as the reference does (tables are returned as given, in fp32).  With
    ``absent_mass`` (the default) the softmax covers all V_total slots as the dense PyTorch
    reference (flash_ema_attention.py:76-77) does; ``absent_mass=False`` gives the Triton
    kernel's softmax over the valid slots only (triton_flash_ema.py:215-229).  With
    ``return_scores`` a sixth element holds the scores * log2(e) as [B, H, K_max, L]
    (what ``flash_ema_backward(scores=...)`` consumes instead of recomputing them).
    ``precision``: "bf16" (default) feeds the gate GEMM fp16 operands; "fp32" feeds it fp16
    hi + lo pairs (three products, ~2^-22 relative, N <= 64), the mode to use where scores
    are large enough that the softmax amplifies operand rounding.
    """
    fp32 = _fp32(precision)
    B, H, L, hd = Q.shape
    K = unique_tensor.shape[1]
    if K != K_max:
        raise ValueError(f"unique_tensor has {K} slots but K_max={K_max}")
    if not return_scores:
        O, LSE = flash_ema_fwd(Q, x, E_k_active, E_v_active, W_pe, rhos, unique_tensor, C_bounds,
                               int(V_total), bool(use_silu), int(Br), bool(absent_mass), fp32)
        Ek, Ev = E_k_active.to(torch.float32), E_v_active.to(torch.float32)
        if Ek.dim() == 2:
            return O, LSE, C_bounds, Ek, Ev
        return O, LSE, C_bounds, Ek.reshape(B, K, H, hd), Ev.reshape(B, K, H, hd)
    O, LSE, S2, Ek, Ev, table = _fwd_impl(Q, x, E_k_active, E_v_active, W_pe, rhos, unique_tensor,
                                          C_bounds, V_total, use_silu, Br, absent_mass, True, fp32)
    if table:
        return O, LSE, C_bounds, Ek, Ev, S2
    return O, LSE, C_bounds, Ek.view(B, K, H, hd), Ev.view(B, K, H, hd), S2


def _bwd_impl(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO, V_total, use_silu,
              Br, absent_mass, scores, fp32=False):
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
    if scores is not None and (tuple(scores.shape) != (B, H, K, L) or scores.dtype != torch.float32
                               or not scores.is_contiguous()):
        raise ValueError(f"scores must be contiguous fp32 [B, H, K_max, L], got {tuple(scores.shape)}")
    with torch.cuda.device(dev):
        _lib.call("mb_flash_ema_bwd", _lib.ptr(Qf), *Qf.stride(), _lib.ptr(dOf), _lib.ptr(xl),
                  xl.stride(0), xl.stride(1), _lib.ptr(Ek), _lib.ptr(Ev), _lib.ptr(W),
                  _lib.ptr(rh), _lib.ptr(uniq), _lib.ptr(Cb), _lib.ptr(Of), _lib.ptr(Lf), B, H, L,
                  hd, K, N, Cb.shape[3], Cb.shape[1], int(Br), int(V_total),
                  _flash_flags(use_silu, absent_mass, table, fp32), _lib.ptr(scores), _lib.ptr(dQ),
                  _lib.ptr(dEk), _lib.ptr(dEv), _lib.ptr(dW), _lib.stream(dev))
    return dQ, dEk, dEv, dW


def _bwd_fake(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO, V_total, use_silu,
              Br, absent_mass, fp32):
    B, H, L, hd = Q.shape
    D = H * hd
    rows = (E_k.shape[0], D) if E_k.dim() == 2 else (B, unique_tensor.shape[1], D)
    f = torch.float32
    return (Q.new_empty((B, H, L, hd), dtype=f), Q.new_empty(rows, dtype=f),
            Q.new_empty(rows, dtype=f), Q.new_empty((rhos.shape[0], D), dtype=f))


@_lib.traced_op("flash_ema_bwd", _bwd_fake)
def flash_ema_bwd(Q: torch.Tensor, x: torch.Tensor, E_k: torch.Tensor, E_v: torch.Tensor,
                  W_pe: torch.Tensor, rhos: torch.Tensor, unique_tensor: torch.Tensor,
                  C_bounds: torch.Tensor, O: torch.Tensor, LSE: torch.Tensor, dO: torch.Tensor,
                  V_total: int, use_silu: bool, Br: int, absent_mass: bool,
                  fp32: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dQ, dE_k, dE_v, dW_pe) of flash_ema_backward (fills and one mb_flash_ema_bwd launch)."""
    return _bwd_impl(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO, V_total,
                     use_silu, Br, absent_mass, None, fp32)


def flash_ema_backward(Q, x, E_k, E_v, W_pe, rhos, V_total, unique_tensor, C_bounds, O, LSE, dO,
                       use_silu=True, Br=64, absent_mass=True, scores=None, precision="bf16"):
    """Gradients of flash_ema_forward (triton_flash_ema.py:586-650) in one fused HIP pass.

    E_k / E_v are [B, K, H*hd] or [B, K, H, hd], or [V_total, H*hd] vocabulary tables (then
    dE_k / dE_v are tables too: each row sums the gradients of every slot of that token);
    ``scores`` is the forward's optional scores output (recomputed when None).  Returns
    (dQ [B,H,L,hd], dE_k [B,K,H*hd], dE_v [B,K,H*hd], dW_pe [N, H*hd]), all fp32.
    ``precision`` as in flash_ema_forward ("fp32" also takes the dW_pe product from bf16
    hi + lo pairs of both operands).
    """
    fp32 = _fp32(precision)
    if scores is None:
        return flash_ema_bwd(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO,
                             int(V_total), bool(use_silu), int(Br), bool(absent_mass), fp32)
    return _bwd_impl(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO, V_total,
                     use_silu, Br, absent_mass, scores, fp32)


# With SAVE_SCORES, FlashEMAFunction keeps the forward's scores ([B, H, K_max, L] fp32,
# 1.5 GB at B=56, T=512, H=8, K_max=1638) when they take at most SAVE_SCORES_MAX_BYTES, and
# the backward reads them instead of recomputing them: configuration 2 measured forward
# 9.09 -> 9.45 ms (writing them) and backward 22.49 -> 21.05 ms (no score products and half
# the cross-lane sums), 31.6 -> 30.5 ms per layer.  Traced graphs never save them.
SAVE_SCORES = True
SAVE_SCORES_MAX_BYTES = 16 << 30


def keep_scores(B, H, K_max, L):
    """Whether FlashEMAFunction keeps the forward's scores for a call of this shape."""
    return (SAVE_SCORES and not torch.compiler.is_compiling()
            and 4 * int(B) * int(H) * int(K_max) * int(L) <= SAVE_SCORES_MAX_BYTES)


class FlashEMAFunction(torch.autograd.Function):
    """Autograd entry point with the reference's 12 arguments (triton_flash_ema.py:571-650)
    and two more: apply(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor,
    K_max, C_bounds, use_silu=True, Br=64, absent_mass=True, precision="bf16") -> O [B, H, L, hd].  Inputs are
    used in fp32 (the reference's custom_fwd(cast_inputs=float32)); gradients flow to Q,
    E_k_active, E_v_active, W_pe.  ``absent_mass=True`` (the default) is the softmax over
    all V_total slots of the dense PyTorch reference; False reproduces the reference's
    Triton kernel, which drops the absent slots' mass (triton_flash_ema.py:215-229).
    ``precision`` picks the gate GEMM's operands (see flash_ema_forward)."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda", cast_inputs=torch.float32)
    def forward(ctx, Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor, K_max,
                C_bounds, use_silu=True, Br=64, absent_mass=True, precision="bf16"):
        keep = keep_scores(Q.shape[0], Q.shape[1], unique_tensor.shape[1], Q.shape[2])
        res = flash_ema_forward(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor,
                                K_max, C_bounds, use_silu, Br, absent_mass, return_scores=keep,
                                precision=precision)
        O, LSE, C_bounds, E_k, E_v = res[:5]
        ctx.save_for_backward(Q, x, E_k, E_v, W_pe, rhos, C_bounds, unique_tensor, O, LSE,
                              res[5] if keep else None)
        ctx.V_total = V_total
        ctx.use_silu = use_silu
        ctx.Br = Br
        ctx.absent_mass = absent_mass
        ctx.precision = precision
        ctx.W_rows = W_pe.shape[0]
        return O

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dO):
        Q, x, E_k, E_v, W_pe, rhos, C_bounds, unique_tensor, O, LSE, S2 = ctx.saved_tensors
        dQ, dEk, dEv, dW = flash_ema_backward(Q, x, E_k, E_v, W_pe, rhos, ctx.V_total,
                                              unique_tensor, C_bounds, O, LSE, dO.contiguous(),
                                              ctx.use_silu, ctx.Br, ctx.absent_mass, scores=S2,
                                              precision=ctx.precision)
        if ctx.W_rows > dW.shape[0]:  # W_pe passed with padded rows: their gradient is 0
            dW = torch.cat([dW, dW.new_zeros(ctx.W_rows - dW.shape[0], dW.shape[1])])
        return dQ, None, dEk, dEv, dW, None, None, None, None, None, None, None, None, None


# ---- the query gating folded into the attention ------------------------------------------

def _gq_prepare(x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, V_total, B, K, N, D, what):
    Ek, table = _slot_rows(E_k, B, K, D, int(V_total), what)
    Ev, table_v = _slot_rows(E_v, B, K, D, int(V_total), what)
    if table != table_v:
        raise ValueError(f"{what}: E_k and E_v must both be tables or both gathered rows")
    W = W_pe.to(torch.float32)
    if W.shape[0] < N or W.shape[1] != D:
        raise ValueError(f"{what}: W_pe must be [N, H*hd] = {(N, D)}, got {tuple(W.shape)}")
    W = W[:N].contiguous()
    rh = rhos.detach().to(torch.float32).contiguous()
    uniq = unique_tensor.to(torch.int64).contiguous()
    xl = x if x.dtype == torch.int64 else x.long()
    Cb = C_bounds.to(torch.float32).contiguous()
    if Cb.dim() != 4 or Cb.shape[0] != B or Cb.shape[2] != K or Cb.shape[3] < N:
        raise ValueError(f"{what}: C_bounds must be [B, nc, K_max, >=N], got {tuple(Cb.shape)}")
    return Ek, Ev, table, W, rh, uniq, xl, Cb


def _rows_f32(t, width):
    """fp32 view with contiguous columns and whole-row strides (copied if needed)."""
    t = t.to(torch.float32)
    if t.stride(-1) != 1 or t.stride(-2) < width:
        t = t.contiguous()
    return t


def _fwd_gq_fake(x_q, C_seq, W_pe, ln_w, ln_b, W_q, eps, x, E_k, E_v, rhos, unique_tensor, C_bounds,
                 V_total, n_heads, use_silu, Br, absent_mass, fp32):
    B, L, D = x_q.shape
    hd = D // n_heads
    return (x_q.new_empty((B, n_heads, L, hd), dtype=torch.float32),
            x_q.new_empty((B, n_heads, L), dtype=torch.float32))


@_lib.traced_op("flash_ema_fwd_gq", _fwd_gq_fake)
def flash_ema_fwd_gq(x_q: torch.Tensor, C_seq: torch.Tensor, W_pe: torch.Tensor, ln_w: torch.Tensor,
                     ln_b: torch.Tensor, W_q: torch.Tensor, eps: float, x: torch.Tensor, E_k: torch.Tensor,
                     E_v: torch.Tensor, rhos: torch.Tensor, unique_tensor: torch.Tensor,
                     C_bounds: torch.Tensor, V_total: int, n_heads: int, use_silu: bool, Br: int,
                     absent_mass: bool, fp32: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE) of the attention on Q = q_proj(LayerNorm(x_q * gate((C_seq + 1) @ W_pe))), the
    queries computed inside the attention kernel (one mb_flash_ema_fwd_gq launch)."""
    dev = _lib.require_gpu(x_q, C_seq, W_pe, ln_w, ln_b, W_q, x, E_k, E_v, rhos, unique_tensor,
                           C_bounds, what="flash_ema_forward (gated queries)")
    B, L, D = x_q.shape
    H = int(n_heads)
    if D % H:
        raise ValueError(f"d_model {D} is not a multiple of n_heads {H}")
    hd = D // H
    K = unique_tensor.shape[1]
    N = rhos.shape[0]
    if C_seq.shape[:2] != (B, L) or C_seq.shape[2] != N:
        raise ValueError(f"C_seq must be [B, L, N] = {(B, L, N)}, got {tuple(C_seq.shape)}")
    if tuple(W_q.shape) != (D, D):
        raise ValueError(f"W_q (q_proj.weight) must be [D, D] = {(D, D)}, got {tuple(W_q.shape)}")
    Ek, Ev, table, W, rh, uniq, xl, Cb = _gq_prepare(x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds,
                                                      V_total, B, K, N, D, "flash_ema_forward")
    xq = _rows_f32(x_q, D)
    C = _rows_f32(C_seq, N)
    lw = ln_w.to(torch.float32).contiguous()
    lb = ln_b.to(torch.float32).contiguous()
    Wq = W_q.to(torch.float32).contiguous()
    O = torch.empty(B, H, L, hd, dtype=torch.float32, device=dev)
    LSE = torch.empty(B, H, L, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_flash_ema_fwd_gq", _lib.ptr(xq), xq.stride(0), xq.stride(1), _lib.ptr(C), C.stride(0),
                  C.stride(1), _lib.ptr(lw), _lib.ptr(lb), float(eps), _lib.ptr(Wq), _lib.ptr(xl),
                  xl.stride(0), xl.stride(1), _lib.ptr(Ek), _lib.ptr(Ev), _lib.ptr(W), _lib.ptr(rh),
                  _lib.ptr(uniq), _lib.ptr(Cb), B, H, L, hd, K, N, Cb.shape[3], Cb.shape[1], int(Br),
                  int(V_total), _flash_flags(use_silu, absent_mass, table, fp32), _lib.ptr(O), _lib.ptr(LSE),
                  _lib.stream(dev))
    return O, LSE


class GatedQueryFlashEMAFunction(torch.autograd.Function):
    """The query side and the attention of SlotAttentionLayer (model.py:75-87) in one launch:
    apply(x_q, C_seq, W_pe, ln_w, ln_b, W_q, x, E_k_active, E_v_active, rhos, V_total,
    unique_tensor, K_max, C_bounds, n_heads, use_silu=True, Br=64, absent_mass=True,
    precision="bf16", eps=1e-5) -> O [B, H, L, hd], equal to

        Q = q_proj(LayerNorm_eps(x_q * SiLU((C_seq + 1) @ W_pe)))      (fused_apply_symmetric_query_gating)
        FlashEMAFunction.apply(Q.view(B, L, H, hd).transpose(1, 2), x, E_k_active, E_v_active, W_pe, ...)

    with W_pe = pe_proj.weight.t() [N, D] (shared by the query gate and the key gate, as in
    the reference), ln_w / ln_b = ln_q's parameters, W_q = q_proj.weight [D, D].  The forward
    kernel computes Q itself: the gating kernel, the q_proj GEMM and Q's trip through HBM are
    gone.  The backward recomputes the LayerNorm output x_ln (which the q_proj and gating
    gradients need) and Q from it, runs the attention backward, and dQ then gives
    dW_q = dQ^T x_ln, dx_ln = dQ W_q and the gating gradients.  Gradients flow to x_q, W_pe,
    ln_w, ln_b, W_q, E_k_active and E_v_active (and C_seq if it requires one).  Supported:
    d_model a multiple of 32, at most 1024."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda", cast_inputs=torch.float32)
    def forward(ctx, x_q, C_seq, W_pe, ln_w, ln_b, W_q, x, E_k_active, E_v_active, rhos, V_total,
                unique_tensor, K_max, C_bounds, n_heads, use_silu=True, Br=64, absent_mass=True,
                precision="bf16", eps=1e-5):
        fp32 = _fp32(precision)
        if unique_tensor.shape[1] != K_max:
            raise ValueError(f"unique_tensor has {unique_tensor.shape[1]} slots but K_max={K_max}")
        O, LSE = flash_ema_fwd_gq(x_q, C_seq, W_pe, ln_w, ln_b, W_q, float(eps), x, E_k_active, E_v_active,
                                  rhos, unique_tensor, C_bounds, int(V_total), int(n_heads), bool(use_silu),
                                  int(Br), bool(absent_mass), fp32)
        ctx.save_for_backward(x_q, C_seq, W_pe, ln_w, ln_b, W_q, x, E_k_active, E_v_active, rhos,
                              unique_tensor, C_bounds, O, LSE)
        ctx.cfg = (int(V_total), bool(use_silu), int(Br), bool(absent_mass), fp32, float(eps), int(n_heads))
        return O

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dO):
        from .triton_fused_gating import gating_bwd, gating_fwd
        (x_q, C_seq, W_pe, ln_w, ln_b, W_q, x, E_k, E_v, rhos, unique_tensor, C_bounds, O,
         LSE) = ctx.saved_tensors
        V_total, use_silu, Br, absent_mass, fp32, eps, H = ctx.cfg
        B, L, D = x_q.shape
        hd = D // H
        N = rhos.shape[0]
        Wpe = W_pe[:N]
        x_ln, mu, rstd = gating_fwd(x_q, None, None, C_seq, Wpe, ln_w, ln_b, use_silu, eps)
        xr = x_ln.reshape(B * L, D)
        Q = (xr @ W_q.t()).view(B, L, H, hd).transpose(1, 2)
        dQ, dEk, dEv, dWa = flash_ema_bwd(Q, x, E_k, E_v, Wpe, rhos, unique_tensor, C_bounds, O, LSE,
                                          dO.contiguous(), V_total, use_silu, Br, absent_mass, fp32)
        dQr = dQ.transpose(1, 2).reshape(B * L, D)  # row (b, t), column h hd + d
        dW_q = dQr.t() @ xr
        dx_ln = dQr @ W_q
        dxq, dpre, dbias, dlnw, dlnb = gating_bwd(dx_ln.view(B, L, D), x_q, None, None, C_seq, Wpe, ln_w,
                                                  mu, rstd, use_silu)
        # the gate's weight gradient: sum_r (C_seq[r] + 1)^T dpre[r] (the bias term's column sum
        # came reduced from the kernel), plus the attention's
        dW = torch.addmm(dbias.unsqueeze(0).expand(N, D), C_seq.reshape(-1, N).t(), dpre) + dWa
        if W_pe.shape[0] > N:  # W_pe passed with padded rows: their gradient is 0
            dW = torch.cat([dW, dW.new_zeros(W_pe.shape[0] - N, D)])
        dC = (dpre @ Wpe.t()).reshape(C_seq.shape) if ctx.needs_input_grad[1] else None
        return (dxq, dC, dW, dlnw, dlnb, dW_q, None, dEk, dEv, None, None, None, None, None, None, None,
                None, None, None, None)
