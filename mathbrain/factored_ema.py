"""Factored linear EMA: the linear-gate form of per-slot EMA attention without a
per-slot gate.

Drop-in for mathbrain/factored_ema.py: ``factored_ema_forward`` (:22-96) with autograd
for Q, E_k_slots, E_v_slots and W_pe, and ``FactoredLinearEMALayer`` (:99-146) with the
same module tree.  The reference runs a Python loop over steps that decays and updates an
[B, H, N, hd, hd] state at every step; here the output is computed exactly from

    o_t = sum_{s<t} A[t,s] e_v[x_s] + sum_n rho_n^(t+1) (q_t ⊙ W_n)^T S_n,
    A[t,s] = sum_i q_t[i] e_k[x_s][i] G_{t-s}[i],   G_d = sum_n rho_n^d W_n,
    S_n = sum_k c_base[k,n] e_k[u_k] ⊗ e_v[u_k]   (the reference's initial state),

by the gfx950 kernels behind mb_factored_tok_fwd / mb_factored_tok_bwd (the token pairs,
fp32) and mb_factored_outer / mb_factored_apply (the c_base state; at head_dim 64 on the
bf16 matrix cores with every fp32 operand split into bf16 hi + lo, three products and fp32
accumulation, about 2^-16 relative error per product).  The small
[L+1, N] x [N, D] products with P[n,d] = rho_n^d (G and dW_pe's token part) are library
GEMMs in float64.  CPU tensors raise NotImplementedError: there is no CPU path.
"""
import torch
import torch.nn as nn

from . import _lib


def _powers(rhos, L, dev):
    """P[n, d] = rho_n^d for d in [0, L], float64."""
    d = torch.arange(L + 1, device=dev, dtype=torch.float64)
    return rhos.to(torch.float64).unsqueeze(1) ** d.unsqueeze(0)


class FactoredEMAFunction(torch.autograd.Function):
    """autograd for factored_ema_forward: gradients for Q, E_k_slots, E_v_slots, W_pe."""

    @staticmethod
    def forward(ctx, Q, x, E_k, E_v, rhos, W_pe, n_heads, c_base, unique_slots, pad_mask):
        dev = _lib.require_gpu(Q, x, E_k, E_v, rhos, W_pe, c_base, unique_slots, pad_mask,
                               what="factored_ema_forward")
        B, L, D = Q.shape
        H = int(n_heads)
        hd = D // H
        N = rhos.shape[0]
        V = E_k.shape[0]
        if D % H or E_k.shape != (V, D) or E_v.shape != (V, D) or W_pe.shape != (N, D):
            raise ValueError(f"factored_ema_forward: shapes Q {tuple(Q.shape)}, E_k "
                             f"{tuple(E_k.shape)}, E_v {tuple(E_v.shape)}, W_pe {tuple(W_pe.shape)}")
        f32 = torch.float32
        Qc = Q.detach().to(f32).contiguous()
        Ek = E_k.detach().to(f32).contiguous()
        Ev = E_v.detach().to(f32).contiguous()
        W = W_pe.detach().to(f32).contiguous()
        xx = x.to(torch.int64).contiguous()
        P = _powers(rhos.detach(), L, dev)
        G = (P.t() @ W.to(torch.float64)).to(f32).contiguous()        # [L+1, D]
        R = P[:, 1:].t().to(f32).contiguous()                          # [L, N]: rho^(t+1)
        O = torch.empty(B, L, D, dtype=f32, device=dev)
        st = _lib.stream(dev)
        p = _lib.ptr
        S = c = u = None
        with torch.cuda.device(dev):
            _lib.call("mb_factored_tok_fwd", p(Qc), p(xx), V, p(Ek), p(Ev), p(G), B, L, H, hd, p(O), st)
            if c_base is not None and unique_slots is not None:
                u = unique_slots.to(torch.int64).contiguous()
                K = u.shape[1]
                c = c_base.detach().to(f32)
                if pad_mask is not None:
                    c = c * pad_mask.to(f32).unsqueeze(-1)
                c = c.contiguous()
                if c.shape != (B, K, N):
                    raise ValueError(f"c_base {tuple(c.shape)} must be [B={B}, K={K}, N={N}]")
                S = torch.empty(B, H, N, hd, hd, dtype=f32, device=dev)
                _lib.call("mb_factored_outer", p(Ek), p(u), p(Ev), p(u), D, V, p(c), K * N, N, 1,
                          B, K, H, N, hd, p(S), st)
                _lib.call("mb_factored_apply", p(S), p(W), D, p(Qc), None, D, B * L, p(R), 0, N, 1,
                          B, L, H, N, hd, 1, p(O), D, 1, st)
        ctx.save_for_backward(Qc, xx, Ek, Ev, W, G, R, P, S, c, u)
        ctx.dims = (B, L, D, H, hd, N, V)
        ctx.in_dtypes = (Q.dtype, E_k.dtype, E_v.dtype, W_pe.dtype)
        return O.to(Q.dtype)

    @staticmethod
    def backward(ctx, dO):
        Qc, xx, Ek, Ev, W, G, R, P, S, c, u = ctx.saved_tensors
        B, L, D, H, hd, N, V = ctx.dims
        dev = Qc.device
        f32 = torch.float32
        g = dO.detach().to(f32).contiguous()
        dQ = torch.empty(B, L, D, dtype=f32, device=dev)
        dEk_t = torch.empty(B, L, D, dtype=f32, device=dev)
        dEv_t = torch.empty(B, L, D, dtype=f32, device=dev)
        dGb = torch.empty(B, L, D, dtype=f32, device=dev)
        st = _lib.stream(dev)
        p = _lib.ptr
        with torch.cuda.device(dev):
            _lib.call("mb_factored_tok_bwd", p(Qc), p(g), p(xx), V, p(Ek), p(Ev), p(G), B, L, H, hd,
                      p(dQ), p(dEk_t), p(dEv_t), p(dGb), st)
            dW = (P[:, :L] @ dGb.sum(0).to(torch.float64)).to(f32)
            dE_k = torch.zeros(V, D, dtype=f32, device=dev)
            dE_v = torch.zeros(V, D, dtype=f32, device=dev)
            # ids outside [0, V) were skipped by the kernels (their rows are zero): clamped
            # here only so that index_add_ stays in range
            tok_rows = xx.reshape(-1).clamp(0, V - 1)
            dE_k.index_add_(0, tok_rows, dEk_t.view(-1, D))
            dE_v.index_add_(0, tok_rows, dEv_t.view(-1, D))
            if S is not None:
                K = u.shape[1]
                _lib.call("mb_factored_apply", p(S), p(W), D, p(g), None, D, B * L, p(R), 0, N, 1,
                          B, L, H, N, hd, 0, p(dQ), D, 1, st)
                M = torch.empty(B, H, N, hd, hd, dtype=f32, device=dev)
                _lib.call("mb_factored_outer", p(Qc), None, p(g), None, D, B * L, p(R), 0, N, 1,
                          B, L, H, N, hd, p(M), st)
                dW += (S * M).sum(-1).sum(0).permute(1, 0, 2).reshape(N, D)
                dk_u = torch.empty(B, K, D, dtype=f32, device=dev)
                dv_u = torch.empty(B, K, D, dtype=f32, device=dev)
                _lib.call("mb_factored_apply", p(M), p(W), D, p(Ev), p(u), D, V, p(c), K * N, N, 1,
                          B, K, H, N, hd, 0, p(dk_u), D, 0, st)
                _lib.call("mb_factored_apply", p(M), p(W), D, p(Ek), p(u), D, V, p(c), K * N, N, 1,
                          B, K, H, N, hd, 1, p(dv_u), D, 0, st)
                rows = u.clamp(0, V - 1).reshape(-1)
                dE_k.index_add_(0, rows, dk_u.view(-1, D))
                dE_v.index_add_(0, rows, dv_u.view(-1, D))
        qd, kd, vd, wd = ctx.in_dtypes
        return (dQ.to(qd), None, dE_k.to(kd), dE_v.to(vd), None, dW.to(wd), None, None, None, None)


def factored_ema_forward(Q, x, E_k_slots, E_v_slots, rhos, W_pe, n_heads,
                         c_base=None, unique_slots=None, pad_mask=None):
    """Factored linear EMA forward (factored_ema.py:22-96), differentiable.

    Q [B, L, D] (already projected), x [B, L] token ids, E_k_slots / E_v_slots [V, D],
    rhos [N], W_pe [N, D] (pe_proj.weight.t()), c_base [B, K, N] with unique_slots [B, K]
    (-1 = padding, read as row 0 as the reference's clamp does) and pad_mask [B, K].
    Returns [B, L, D].  Token ids outside [0, V) contribute nothing (the reference's
    indexing would raise; checking here would cost a device-to-host sync per call).
    """
    if Q.device.type != "cuda":
        raise NotImplementedError("factored_ema_forward: tensors must be on an MI355X GPU; "
                                  "this implementation has no CPU path")
    if c_base is None or unique_slots is None:
        c_base = unique_slots = pad_mask = None
    return FactoredEMAFunction.apply(Q, x, E_k_slots, E_v_slots, rhos, W_pe, n_heads, c_base,
                                     unique_slots, pad_mask)


class FactoredLinearEMALayer(nn.Module):
    """Drop-in for SlotAttentionLayer when use_silu=False (factored_ema.py:99-146): the same
    parameters (q/k/v/o_proj, pe_proj, ln_kv, ln_q) and forward signature."""

    def __init__(self, d_model: int, n_heads: int, dropout: float, n_scales: int):
        super().__init__()
        assert d_model % n_heads == 0
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.n_scales = n_scales
        self.q_proj = nn.Linear(d_model, d_model, bias=False)
        self.k_proj = nn.Linear(d_model, d_model, bias=False)
        self.v_proj = nn.Linear(d_model, d_model, bias=False)
        self.o_proj = nn.Linear(d_model, d_model, bias=False)
        self.pe_proj = nn.Linear(n_scales, d_model, bias=False)
        self.ln_kv = nn.LayerNorm(d_model)
        self.ln_q = nn.LayerNorm(d_model)
        self.resid_dropout = nn.Dropout(dropout)

    def forward(self, x_q, x, E_slots, rhos, C_seq, c_base=None, unique_slots=None,
                pad_mask=None, **kwargs):
        memory_base = self.ln_kv(E_slots)                       # factored_ema.py:127-130
        E_k_slots = self.k_proj(memory_base)
        E_v_slots = self.v_proj(memory_base)
        P_gate_Q = self.pe_proj(C_seq + 1.0)                    # :133-136, linear gate
        Q_t = self.q_proj(self.ln_q(x_q * P_gate_Q))
        out = factored_ema_forward(Q_t, x, E_k_slots, E_v_slots, rhos,
                                   self.pe_proj.weight.t(), self.n_heads, c_base=c_base,
                                   unique_slots=unique_slots, pad_mask=pad_mask)
        return self.resid_dropout(self.o_proj(out))
