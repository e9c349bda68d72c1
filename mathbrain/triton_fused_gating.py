"""Fused symmetric query gating: Q = q_proj(LayerNorm(x_q * SiLU(pe_proj(C_seq + 1)))).

Drop-in for mathbrain/triton_fused_gating.py: ``FusedGatingFunction`` (:122-177) keeps
the reference's autograd signature (x_q, p_pre, bias, ln_w, ln_b, use_silu), and
``fused_apply_symmetric_query_gating`` (:179-197) keeps its call signature.  The latter
folds the pe_proj projection (a K = N contraction) and its bias into the gating kernel
(``GatedQueryFunction``), so the pre-activation is never a separate GEMM's output; the
forward keeps it for the backward (as the reference keeps its gate, :38 and :90), whose
kernel then takes one row per wave without the projection; q_proj stays a library GEMM.  The row kernels are the gfx950 ones behind
``mb_gating_fwd`` / ``mb_gating_bwd``, registered as torch ops (mathbrain::gating_fwd /
gating_bwd) for tracing.
"""
from typing import Optional

import torch

from . import _lib


def _rows(t, D):
    """[.., D] -> ([rows, D] view with contiguous columns, row stride)."""
    t2 = t.reshape(-1, D)
    if t2.stride(1) != 1 or t2.stride(0) < D:
        t2 = t2.contiguous()
    return t2, t2.stride(0)


def _gate_fwd_fake(x_q, p_pre, bias, C_seq, W_pe, ln_w, ln_b, use_silu, eps):
    rows = x_q.numel() // x_q.shape[-1]
    mu = x_q.new_empty((rows,), dtype=torch.float32)
    return x_q.new_empty(x_q.shape, dtype=torch.float32), mu, mu.new_empty((rows,))


def _gating_fwd(x_q, p_pre, bias, C_seq, W_pe, ln_w, ln_b, use_silu, eps, keep_pre):
    dev = _lib.require_gpu(x_q, p_pre, bias, C_seq, W_pe, ln_w, ln_b, what="query gating")
    D = x_q.shape[-1]
    xq, xs = _rows(x_q.to(torch.float32), D)
    rows = xq.shape[0]
    pp = ps = cs = css = W = None
    N = 0
    if p_pre is not None:
        pp, ps = _rows(p_pre.to(torch.float32), D)
        bias = bias.to(torch.float32).contiguous() if bias is not None else None
    else:
        N = C_seq.shape[-1]
        if W_pe.shape != (N, D):
            raise ValueError(f"W_pe must be [N, D] = {(N, D)}, got {tuple(W_pe.shape)}")
        cs, css = _rows(C_seq.to(torch.float32), N)
        if cs.shape[0] != rows:
            raise ValueError(f"C_seq {tuple(C_seq.shape)} and x_q {tuple(x_q.shape)} disagree in rows")
        W = W_pe.to(torch.float32).contiguous()
    ln_w = ln_w.to(torch.float32).contiguous()
    ln_b = ln_b.to(torch.float32).contiguous()
    y = torch.empty(x_q.shape, dtype=torch.float32, device=dev)
    mu = torch.empty(rows, dtype=torch.float32, device=dev)
    rstd = torch.empty(rows, dtype=torch.float32, device=dev)
    pre = torch.empty(rows if keep_pre else 0, D, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_gating_fwd", _lib.ptr(xq), xs, _lib.ptr(pp), ps or 0, _lib.ptr(bias),
                  _lib.ptr(cs), css or 0, _lib.ptr(W), N, _lib.ptr(ln_w), _lib.ptr(ln_b), rows, D,
                  int(bool(use_silu)), float(eps), _lib.ptr(y), _lib.ptr(mu), _lib.ptr(rstd),
                  _lib.ptr(pre) if keep_pre else None, _lib.stream(dev))
    return y, mu, rstd, pre


@_lib.traced_op("gating_fwd", _gate_fwd_fake)
def gating_fwd(x_q: torch.Tensor, p_pre: Optional[torch.Tensor], bias: Optional[torch.Tensor],
               C_seq: Optional[torch.Tensor], W_pe: Optional[torch.Tensor], ln_w: torch.Tensor,
               ln_b: torch.Tensor, use_silu: bool, eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y, mu, rstd): y = LayerNorm_eps(x_q * gate(pre)) * ln_w + ln_b with pre = p_pre + bias
    (p_pre given; a None bias is zero) or (C_seq + 1) @ W_pe (W_pe [N, D] =
    pe_proj.weight transposed)."""
    return _gating_fwd(x_q, p_pre, bias, C_seq, W_pe, ln_w, ln_b, use_silu, eps, False)[:3]


def _gate_fwd_keep_fake(x_q, C_seq, W_pe, ln_w, ln_b, use_silu, eps):
    y, mu, rstd = _gate_fwd_fake(x_q, None, None, C_seq, W_pe, ln_w, ln_b, use_silu, eps)
    return y, mu, rstd, y.new_empty((mu.shape[0], x_q.shape[-1]))


@_lib.traced_op("gating_fwd_keep_pre", _gate_fwd_keep_fake)
def gating_fwd_keep_pre(x_q: torch.Tensor, C_seq: torch.Tensor, W_pe: torch.Tensor, ln_w: torch.Tensor,
                        ln_b: torch.Tensor, use_silu: bool,
                        eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """gating_fwd with the projection folded in, also returning the pre-activation
    (C_seq + 1) @ W_pe as [rows, D] for the backward (which then needs no projection)."""
    return _gating_fwd(x_q, None, None, C_seq, W_pe, ln_w, ln_b, use_silu, eps, True)


def _gate_bwd_fake(dy, x_q, p_pre, bias, C_seq, W_pe, ln_w, mu, rstd, use_silu):
    D = x_q.shape[-1]
    rows = x_q.numel() // D
    col = x_q.new_empty((D,), dtype=torch.float32)
    return (x_q.new_empty(x_q.shape, dtype=torch.float32),
            x_q.new_empty((rows, D), dtype=torch.float32), col, col.new_empty((D,)), col.new_empty((D,)))


@_lib.traced_op("gating_bwd", _gate_bwd_fake)
def gating_bwd(dy: torch.Tensor, x_q: torch.Tensor, p_pre: Optional[torch.Tensor],
               bias: Optional[torch.Tensor], C_seq: Optional[torch.Tensor], W_pe: Optional[torch.Tensor],
               ln_w: torch.Tensor, mu: torch.Tensor, rstd: torch.Tensor,
               use_silu: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dx_q, dpre [rows, D], dbias, dln_w, dln_b) of gating_fwd for the output gradient dy;
    dpre is the gradient of p_pre, or of the folded pre-activation."""
    dev = x_q.device
    D = x_q.shape[-1]
    xq, xs = _rows(x_q.to(torch.float32), D)
    rows = xq.shape[0]
    pp = ps = cs = css = W = None
    N = 0
    if p_pre is not None:
        pp, ps = _rows(p_pre.to(torch.float32), D)
        bias = bias.to(torch.float32).contiguous() if bias is not None else None
    else:
        N = C_seq.shape[-1]
        cs, css = _rows(C_seq.to(torch.float32), N)
        W = W_pe.to(torch.float32).contiguous()
    ln_w = ln_w.to(torch.float32).contiguous()
    g = dy.to(torch.float32).reshape(rows, D).contiguous()
    dxq = torch.empty(x_q.shape, dtype=torch.float32, device=dev)
    dpre = torch.empty(rows, D, dtype=torch.float32, device=dev)
    dbias = torch.empty(D, dtype=torch.float32, device=dev)
    dlnw = torch.empty(D, dtype=torch.float32, device=dev)
    dlnb = torch.empty(D, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_gating_bwd", _lib.ptr(g), _lib.ptr(xq), xs, _lib.ptr(pp), ps or 0,
                  _lib.ptr(bias), _lib.ptr(cs), css or 0, _lib.ptr(W), N, _lib.ptr(ln_w),
                  _lib.ptr(mu), _lib.ptr(rstd), rows, D, int(bool(use_silu)), _lib.ptr(dxq),
                  _lib.ptr(dpre), _lib.ptr(dbias), _lib.ptr(dlnw), _lib.ptr(dlnb), _lib.stream(dev))
    return dxq, dpre, dbias, dlnw, dlnb


class FusedGatingFunction(torch.autograd.Function):
    """apply(x_q, p_pre, bias, ln_w, ln_b, use_silu=True) -> x_ln [B, L, D]
    (triton_fused_gating.py:122-177): LayerNorm_{1e-5}(x_q * SiLU(p_pre + bias)).
    Inputs are used in fp32 (the reference's custom_fwd(cast_inputs=float32))."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda", cast_inputs=torch.float32)
    def forward(ctx, x_q, p_pre, bias, ln_w, ln_b, use_silu=True):
        y, mu, rstd = gating_fwd(x_q, p_pre, bias, None, None, ln_w, ln_b, bool(use_silu), 1e-5)
        ctx.save_for_backward(x_q, p_pre, bias, ln_w, mu, rstd)
        ctx.use_silu = bool(use_silu)
        return y

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        x_q, p_pre, bias, ln_w, mu, rstd = ctx.saved_tensors
        dxq, dpp, dbias, dlnw, dlnb = gating_bwd(dy, x_q, p_pre, bias, None, None, ln_w, mu, rstd,
                                                 ctx.use_silu)
        return dxq, dpp.view(p_pre.shape), dbias, dlnw, dlnb, None


class GatedQueryFunction(torch.autograd.Function):
    """apply(x_q, C_seq, W_pe, ln_w, ln_b, use_silu=True, eps=1e-5) -> x_ln [B, L, D] with
    the projection folded in: LayerNorm(x_q * SiLU((C_seq + 1) @ W_pe)), W_pe [N, D]
    (pe_proj.weight transposed).  This is pe_proj(C_seq) + pe_proj.weight.sum(1)
    followed by FusedGatingFunction (triton_fused_gating.py:180-186).  Gradients flow to
    x_q, W_pe, ln_w, ln_b (and C_seq when it requires one)."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda", cast_inputs=torch.float32)
    def forward(ctx, x_q, C_seq, W_pe, ln_w, ln_b, use_silu=True, eps=1e-5):
        # the pre-activation is kept ([rows, D] fp32, as the reference keeps its gate): the
        # backward then runs on it instead of recomputing the projection
        y, mu, rstd, pre = gating_fwd_keep_pre(x_q, C_seq, W_pe, ln_w, ln_b, bool(use_silu), float(eps))
        ctx.save_for_backward(x_q, C_seq, W_pe, ln_w, mu, rstd, pre)
        ctx.use_silu = bool(use_silu)
        return y

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        x_q, C_seq, W_pe, ln_w, mu, rstd, pre = ctx.saved_tensors
        dxq, dpre, dbias, dlnw, dlnb = gating_bwd(dy, x_q, pre, None, None, None, ln_w, mu, rstd,
                                                  ctx.use_silu)
        N, D = W_pe.shape
        dW = None
        if ctx.needs_input_grad[2]:
            # dW[n, d] = sum_r (C[r, n] + 1) dpre[r, d]: a plain GEMM (K = rows) plus the
            # bias term's column sum, which the kernel already reduced.
            dW = torch.addmm(dbias.unsqueeze(0).expand(N, D), C_seq.reshape(-1, N).t(), dpre)
        dC = None
        if ctx.needs_input_grad[1]:
            dC = (dpre @ W_pe.t()).reshape(C_seq.shape)
        return dxq, dC, dW, dlnw, dlnb, None, None


def fused_apply_symmetric_query_gating(x_q, C_seq, pe_proj, ln_q, q_proj, use_silu=True):
    """q_proj(LayerNorm(x_q * SiLU(pe_proj(C_seq) + pe_proj.weight.sum(1))))
    (triton_fused_gating.py:179-197): the gate is taken on C_seq + 1.  pe_proj's own bias,
    if it has one, is added to the pre-activation as the reference's pe_proj(C_seq) does."""
    if pe_proj.bias is not None:
        bias = pe_proj.weight.sum(dim=1)
        p_pre = pe_proj(C_seq)
        q_ln = FusedGatingFunction.apply(x_q, p_pre, bias, ln_q.weight, ln_q.bias, use_silu)
    else:
        q_ln = GatedQueryFunction.apply(x_q, C_seq, pe_proj.weight.t(), ln_q.weight, ln_q.bias,
                                        use_silu, ln_q.eps)
    return q_proj(q_ln)
