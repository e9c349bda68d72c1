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
import math
import threading
import weakref
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
    lo, hi = (int(v) for v in counts.aminmax()) if counts.numel() else (0, 0)
    if lo < 0:
        raise _lib.HipKernelError("_build_unique_index: a row of more than 8192 ids spans 2^32 or more "
                                  "(rows that long are sorted as 32-bit offsets)")
    K_max = max(hi, 16)
    return ids[:, :K_max].contiguous().to(x.dtype), K_max


# The gate GEMM takes the decayed key counters as fp16 operands (both precision modes: the
# fp32 mode splits them into fp16 hi + lo parts).  A slot's counter at a chunk start is an
# EMA of at most one occurrence per step, so it never exceeds 1 / (1 - rho) when c_base is
# itself such a count (as the data pipeline's states are), and a window adds at most 64
# occurrences on top.  COUNTER_MAX is fp16's largest finite value less those 64; rates with
# 1 / (1 - rho) above it (half-lives above MAX_HALF_LIFE steps: 1 / (1 - rho) is about
# hl / ln 2 + 1/2) are refused, because their counters could leave the fp16 range.
COUNTER_MAX = 65504.0 - 64
MAX_HALF_LIFE = math.log(2.0) / -math.log1p(-1.0 / COUNTER_MAX)
_rates_checked = {}  # id(tensor) -> (weak reference, version) of rate tensors found in range
_rates_lock = threading.Lock()


def check_counter_range(rhos, what="flash-EMA attention"):
    """Raises HipKernelError if a rate's counters can exceed the gate operands' fp16 range.

    ``rhos``: a tensor (any device) or a sequence of floats.  The check reads the largest
    rate once per tensor object and version (a device tensor is read back the first time
    only), and is skipped while torch.compile traces or a CUDA graph is captured."""
    if isinstance(rhos, torch.Tensor):
        if torch.compiler.is_compiling():
            return
        if rhos.device.type == "cuda" and torch.cuda.is_current_stream_capturing():
            return
        with _rates_lock:
            seen = _rates_checked.get(id(rhos))
        if seen is not None and seen[0]() is rhos and seen[1] == rhos._version:
            return
        rho_max = float(rhos.detach().max()) if rhos.numel() else 0.0
    else:
        rho_max = max((float(r) for r in rhos), default=0.0)
    if not rho_max < 1.0 or 1.0 / (1.0 - rho_max) > COUNTER_MAX:
        hl = math.inf if not rho_max < 1.0 else math.log(2.0) / -math.log(rho_max)
        raise _lib.HipKernelError(
            f"{what}: the slowest EMA rate (rho = {rho_max!r}, half-life {hl:.6g} steps) lets the "
            f"key counters reach 1/(1 - rho) = {1.0 / max(1.0 - rho_max, 1e-300):.6g}, above the "
            f"{COUNTER_MAX:g} that the gate's fp16 operands hold; half-lives up to "
            f"{MAX_HALF_LIFE:.0f} steps are supported")
    if isinstance(rhos, torch.Tensor):
        key = id(rhos)
        with _rates_lock:
            if key not in _rates_checked:
                weakref.finalize(rhos, _forget_rates, key)
            _rates_checked[key] = (weakref.ref(rhos), rhos._version)


def _forget_rates(key):
    with _rates_lock:
        _rates_checked.pop(key, None)


# Gate arithmetic of the attention kernels:
#   "bf16" (default)  the gate GEMM splits c_dec and W_pe * log2 e into fp16 hi + lo pairs
#                     (three products, ~2^-22 relative) where the kernels take it (N <= 64,
#                     head_dim <= 64; single fp16 operands otherwise), on the 32-rate tiles
#                     whose counters can be large (a tile whose largest 1/(1 - rho) is below
#                     1/32 of the largest takes the single product); the backward, when it
#                     reads the forward's scores, splits only for the slots whose probability
#                     reaches 2^-7 at one of a wave's 16 steps (every gradient term of a slot
#                     carries its p); dW_pe from bf16 operands, as the reference's kernel;
#   "fp16"            single fp16 gate operands (2^-11): faster, for models whose scores stay
#                     small (the softmax multiplies a relative gate error by the score scale);
#   "fp32"            the split gate and a split dW_pe product (bf16 hi + lo), everything else
#                     fp32: north_star's 1e-4 mode (N <= 64, head_dim <= 64).
PRECISIONS = ("bf16", "fp16", "fp32")


def _prec(precision):
    """The C ABI flag bits of a precision name."""
    if precision not in PRECISIONS:
        raise ValueError(f"precision must be one of {PRECISIONS}, got {precision!r}")
    return {"bf16": 0, "fp16": _lib.MB_FLASH_FAST_GATE, "fp32": _lib.MB_FLASH_FP32}[precision]


def _flash_flags(use_silu, absent_mass, vocab_rows=False, prec=0):
    return ((_lib.MB_FLASH_SILU if use_silu else 0) | (_lib.MB_FLASH_ABSENT_MASS if absent_mass else 0)
            | (_lib.MB_FLASH_VOCAB_ROWS if vocab_rows else 0) | int(prec))


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
              absent_mass, return_scores, prec=0):
    dev = _lib.require_gpu(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds,
                           what="flash_ema_forward")
    check_counter_range(rhos, "flash_ema_forward")
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
    flags = _flash_flags(use_silu, absent_mass, table, prec)
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
              prec):
    B, H, L, hd = Q.shape
    return Q.new_empty((B, H, L, hd), dtype=torch.float32), Q.new_empty((B, H, L), dtype=torch.float32)


@_lib.traced_op("flash_ema_fwd", _fwd_fake)
def flash_ema_fwd(Q: torch.Tensor, x: torch.Tensor, E_k: torch.Tensor, E_v: torch.Tensor,
                  W_pe: torch.Tensor, rhos: torch.Tensor, unique_tensor: torch.Tensor,
                  C_bounds: torch.Tensor, V_total: int, use_silu: bool, Br: int,
                  absent_mass: bool, prec: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE) of flash_ema_forward (mb_flash_ema_fwd: one launch, and a merge launch when it
    splits the slots into parts)."""
    O, LSE = _fwd_impl(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, V_total, use_silu, Br,
                       absent_mass, False, prec)[:2]
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
    ``return_scores`` a sixth element holds the scores * log2(e) as [B, H, K_max, L], -inf in
    the rows of padding slots (what ``flash_ema_backward(scores=...)`` consumes instead of
    recomputing them).
    ``precision``: the gate arithmetic (see PRECISIONS): "bf16" (default) splits the gate
    operands into fp16 hi + lo pairs (N <= 64, head_dim <= 64; single fp16 operands
    beyond), "fp16" takes single fp16 operands (faster; for small scores only), "fp32" also
    splits the backward's dW_pe product.
    """
    prec = _prec(precision)
    B, H, L, hd = Q.shape
    K = unique_tensor.shape[1]
    if K != K_max:
        raise ValueError(f"unique_tensor has {K} slots but K_max={K_max}")
    if not return_scores:
        O, LSE = flash_ema_fwd(Q, x, E_k_active, E_v_active, W_pe, rhos, unique_tensor, C_bounds,
                               int(V_total), bool(use_silu), int(Br), bool(absent_mass), prec)
        Ek, Ev = E_k_active.to(torch.float32), E_v_active.to(torch.float32)
        if Ek.dim() == 2:
            return O, LSE, C_bounds, Ek, Ev
        return O, LSE, C_bounds, Ek.reshape(B, K, H, hd), Ev.reshape(B, K, H, hd)
    res = _forward_with_scores(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor, C_bounds,
                               use_silu, Br, absent_mass, prec)
    # the kernel writes the rows of valid slots only: padding slots' rows hold -inf (score
    # of no slot), as a softmax over them expects
    res[5].masked_fill_((unique_tensor < 0)[:, None, :, None], float("-inf"))
    return res


def _forward_with_scores(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor, C_bounds,
                         use_silu, Br, absent_mass, prec):
    """flash_ema_forward's six outputs with the scores [B, H, K_max, L]; the rows of padding
    slots are left unwritten (the backward never reads them)."""
    B, H, L, hd = Q.shape
    K = unique_tensor.shape[1]
    O, LSE, S2, Ek, Ev, table = _fwd_impl(Q, x, E_k_active, E_v_active, W_pe, rhos, unique_tensor,
                                          C_bounds, V_total, use_silu, Br, absent_mass, True, prec)
    if table:
        return O, LSE, C_bounds, Ek, Ev, S2
    return O, LSE, C_bounds, Ek.view(B, K, H, hd), Ev.view(B, K, H, hd), S2


def _bwd_impl(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO, V_total, use_silu,
              Br, absent_mass, scores, prec=0):
    dev = _lib.require_gpu(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO,
                           what="flash_ema_backward")
    check_counter_range(rhos, "flash_ema_backward")
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
                  _flash_flags(use_silu, absent_mass, table, prec), _lib.ptr(scores), _lib.ptr(dQ),
                  _lib.ptr(dEk), _lib.ptr(dEv), _lib.ptr(dW), _lib.stream(dev))
    return dQ, dEk, dEv, dW


def _bwd_fake(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO, V_total, use_silu,
              Br, absent_mass, prec):
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
                  prec: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dQ, dE_k, dE_v, dW_pe) of flash_ema_backward (fills and one mb_flash_ema_bwd launch)."""
    return _bwd_impl(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO, V_total,
                     use_silu, Br, absent_mass, None, prec)


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
    prec = _prec(precision)
    if scores is None:
        return flash_ema_bwd(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO,
                             int(V_total), bool(use_silu), int(Br), bool(absent_mass), prec)
    return _bwd_impl(Q, x, E_k, E_v, W_pe, rhos, unique_tensor, C_bounds, O, LSE, dO, V_total,
                     use_silu, Br, absent_mass, scores, prec)


# With SAVE_SCORES, FlashEMAFunction keeps the forward's scores ([B, H, K_max, L] fp32,
# 1.5 GB at B=56, T=512, H=8, K_max=1638) and the backward reads them instead of recomputing
# them: configuration 2 measured forward 9.09 -> 9.45 ms (writing them) and backward 22.49 ->
# 21.05 ms (no score products and half the cross-lane sums), 31.6 -> 30.5 ms per layer.
# SAVE_SCORES_MAX_BYTES is a budget per device shared by every saved score tensor still
# alive (a model's layers each keep theirs until the backward reaches them): a call whose
# scores would take the held total past it recomputes them in the backward instead.  A
# saved tensor returns its bytes when it is freed (after the backward, or when the graph is
# dropped).  Traced graphs never save them.
SAVE_SCORES = True
SAVE_SCORES_MAX_BYTES = 16 << 30


class ScoreBudget:
    """Bytes of saved score tensors held per device, against a shared limit."""

    def __init__(self):
        self._held = {}
        self._lock = threading.Lock()

    def held(self, device):
        with self._lock:
            return self._held.get(str(device), 0)

    def reserve(self, device, nbytes, limit):
        """Takes ``nbytes`` for ``device`` if the total stays within ``limit``; returns whether
        it did."""
        key = str(device)
        with self._lock:
            held = self._held.get(key, 0)
            if held + nbytes > limit:
                return False
            self._held[key] = held + nbytes
            return True

    def release(self, device, nbytes):
        key = str(device)
        with self._lock:
            self._held[key] = max(self._held.get(key, 0) - nbytes, 0)

    def hold(self, tensor, nbytes):
        """Returns ``nbytes`` reserved for ``tensor``'s device when ``tensor`` is freed."""
        weakref.finalize(tensor, self.release, tensor.device, nbytes)


score_budget = ScoreBudget()


def keep_scores(B, H, K_max, L):
    """Whether FlashEMAFunction would keep the forward's scores for a call of this shape with
    nothing else held (the budget check of a real call also counts the scores already held)."""
    return (SAVE_SCORES and not torch.compiler.is_compiling()
            and 4 * int(B) * int(H) * int(K_max) * int(L) <= SAVE_SCORES_MAX_BYTES)


def _reserve_scores(Q, K_max):
    """Reserves the score bytes of this call in the shared budget; returns the byte count, or
    0 when the scores are to be recomputed by the backward instead."""
    B, H, L = Q.shape[0], Q.shape[1], Q.shape[2]
    if not keep_scores(B, H, K_max, L):
        return 0
    nbytes = 4 * int(B) * int(H) * int(K_max) * int(L)
    return nbytes if score_budget.reserve(Q.device, nbytes, SAVE_SCORES_MAX_BYTES) else 0


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
        nbytes = _reserve_scores(Q, unique_tensor.shape[1])
        keep = nbytes > 0
        try:
            if keep:
                if unique_tensor.shape[1] != K_max:
                    raise ValueError(f"unique_tensor has {unique_tensor.shape[1]} slots but K_max={K_max}")
                res = _forward_with_scores(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor,
                                           C_bounds, use_silu, Br, absent_mass, _prec(precision))
            else:
                res = flash_ema_forward(Q, x, E_k_active, E_v_active, W_pe, rhos, V_total, unique_tensor,
                                        K_max, C_bounds, use_silu, Br, absent_mass, precision=precision)
        except BaseException:
            if keep:
                score_budget.release(Q.device, nbytes)
            raise
        if keep:
            score_budget.hold(res[5], nbytes)
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
                 V_total, n_heads, use_silu, Br, absent_mass, prec):
    B, L, D = x_q.shape
    hd = D // n_heads
    return (x_q.new_empty((B, n_heads, L, hd), dtype=torch.float32),
            x_q.new_empty((B, n_heads, L), dtype=torch.float32))


@_lib.traced_op("flash_ema_fwd_gq", _fwd_gq_fake)
def flash_ema_fwd_gq(x_q: torch.Tensor, C_seq: torch.Tensor, W_pe: torch.Tensor, ln_w: torch.Tensor,
                     ln_b: torch.Tensor, W_q: torch.Tensor, eps: float, x: torch.Tensor, E_k: torch.Tensor,
                     E_v: torch.Tensor, rhos: torch.Tensor, unique_tensor: torch.Tensor,
                     C_bounds: torch.Tensor, V_total: int, n_heads: int, use_silu: bool, Br: int,
                     absent_mass: bool, prec: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE) of the attention on Q = q_proj(LayerNorm(x_q * gate((C_seq + 1) @ W_pe))), the
    queries computed inside the attention kernel (one mb_flash_ema_fwd_gq launch)."""
    dev = _lib.require_gpu(x_q, C_seq, W_pe, ln_w, ln_b, W_q, x, E_k, E_v, rhos, unique_tensor,
                           C_bounds, what="flash_ema_forward (gated queries)")
    check_counter_range(rhos, "flash_ema_forward (gated queries)")
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
                  int(V_total), _flash_flags(use_silu, absent_mass, table, prec), _lib.ptr(O), _lib.ptr(LSE),
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
        prec = _prec(precision)
        if unique_tensor.shape[1] != K_max:
            raise ValueError(f"unique_tensor has {unique_tensor.shape[1]} slots but K_max={K_max}")
        O, LSE = flash_ema_fwd_gq(x_q, C_seq, W_pe, ln_w, ln_b, W_q, float(eps), x, E_k_active, E_v_active,
                                  rhos, unique_tensor, C_bounds, int(V_total), int(n_heads), bool(use_silu),
                                  int(Br), bool(absent_mass), prec)
        ctx.save_for_backward(x_q, C_seq, W_pe, ln_w, ln_b, W_q, x, E_k_active, E_v_active, rhos,
                              unique_tensor, C_bounds, O, LSE)
        ctx.cfg = (int(V_total), bool(use_silu), int(Br), bool(absent_mass), prec, float(eps), int(n_heads))
        return O

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dO):
        from .triton_fused_gating import gating_bwd, gating_fwd
        (x_q, C_seq, W_pe, ln_w, ln_b, W_q, x, E_k, E_v, rhos, unique_tensor, C_bounds, O,
         LSE) = ctx.saved_tensors
        V_total, use_silu, Br, absent_mass, prec, eps, H = ctx.cfg
        B, L, D = x_q.shape
        hd = D // H
        N = rhos.shape[0]
        Wpe = W_pe[:N]
        x_ln, mu, rstd = gating_fwd(x_q, None, None, C_seq, Wpe, ln_w, ln_b, use_silu, eps)
        xr = x_ln.reshape(B * L, D)
        Q = (xr @ W_q.t()).view(B, L, H, hd).transpose(1, 2)
        dQ, dEk, dEv, dWa = flash_ema_bwd(Q, x, E_k, E_v, Wpe, rhos, unique_tensor, C_bounds, O, LSE,
                                          dO.contiguous(), V_total, use_silu, Br, absent_mass, prec)
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
