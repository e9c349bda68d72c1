"""TEST INFRASTRUCTURE ONLY: CPU restatement of the factored linear EMA
(mathbrain/factored_ema.py), the checker, never the product.

``loop_forward`` follows factored_ema_forward (factored_ema.py:22-96) step by step in torch
(any dtype, differentiable): the per-scale state S[b,h,n] = sum_k c_base[b,k,n] e_k ⊗ e_v of
the slots (:52-67), then per step t "decay, read, write" (variant C, :75-94):

    S_n <- rho_n S_n;   o_t = sum_n (q_t ⊙ W_n)^T S_n;   S_n <- S_n + e_k[x_t] ⊗ e_v[x_t].

``closed_form`` evaluates the same output from its closed form, written independently:

    o_t = sum_{s<t} A[t,s] e_v[x_s] + sum_n rho_n^(t+1) (q_t ⊙ W_n)^T S_n(init),
    A[t,s] = sum_i q_t[i] e_k[x_s][i] G_{t-s}[i],   G_d = sum_n rho_n^d W_n.

The two agree to rounding (tests/test_oracle_factored.py), which pins both; float64
gradcheck pins the gradients of ``loop_forward``.
"""
import torch


def loop_forward(Q, x, E_k, E_v, rhos, W_pe, n_heads, c_base=None, unique_slots=None,
                 pad_mask=None):
    """factored_ema_forward (factored_ema.py:22-96): Q [B,L,D], x [B,L], E_k/E_v [V,D],
    rhos [N], W_pe [N,D], c_base [B,K,N], unique_slots [B,K], pad_mask [B,K]."""
    B, L, D = Q.shape
    N = rhos.shape[0]
    H = n_heads
    hd = D // H
    Ek = E_k.view(-1, H, hd)
    Ev = E_v.view(-1, H, hd)
    Wh = W_pe.view(N, H, hd)
    if c_base is not None and unique_slots is not None:
        K = c_base.shape[1]
        safe = unique_slots.clamp(min=0).long()
        ek = Ek[safe.reshape(-1)].view(B, K, H, hd)
        ev = Ev[safe.reshape(-1)].view(B, K, H, hd)
        c = c_base
        if pad_mask is not None:
            c = c * pad_mask.unsqueeze(-1).to(c.dtype)
        S = torch.einsum("bkn,bkhi,bkhj->bhnij", c, ek, ev)
    else:
        S = torch.zeros(B, H, N, hd, hd, dtype=Q.dtype)
    r5 = rhos.view(1, 1, N, 1, 1).to(Q.dtype)
    outs = []
    for t in range(L):
        S = S * r5
        q = Q[:, t].view(B, H, hd)
        qm = q.unsqueeze(2) * Wh.permute(1, 0, 2).unsqueeze(0)          # [B,H,N,hd]
        outs.append(torch.matmul(qm.unsqueeze(3), S).squeeze(3).sum(2))  # [B,H,hd]
        tok = x[:, t]
        S = S + (Ek[tok].unsqueeze(-1) * Ev[tok].unsqueeze(-2)).unsqueeze(2)
    return torch.stack(outs, 1).reshape(B, L, D)


def closed_form(Q, x, E_k, E_v, rhos, W_pe, n_heads, c_base=None, unique_slots=None,
                pad_mask=None):
    """The closed form above, in the dtype of Q (float64 for checking)."""
    B, L, D = Q.shape
    N = rhos.shape[0]
    H = n_heads
    hd = D // H
    f = Q.dtype
    rh = rhos.to(f)
    d = torch.arange(L + 1, dtype=f)
    P = rh.unsqueeze(1) ** d.unsqueeze(0)                 # [N, L+1]: rho_n^d
    G = (P.t() @ W_pe.to(f)).view(L + 1, H, hd)           # G_d
    q = Q.view(B, L, H, hd)
    ek = E_k.to(f)[x].view(B, L, H, hd)
    ev = E_v.to(f)[x].view(B, L, H, hd)
    tt = torch.arange(L).view(L, 1)
    ss = torch.arange(L).view(1, L)
    delta = (tt - ss).clamp(min=0)
    Gts = G[delta]                                        # [L, L, H, hd]
    A = torch.einsum("bthi,bshi,tshi->bhts", q, ek, Gts) * (tt > ss).to(f)
    out = torch.einsum("bhts,bshj->bthj", A, ev)
    if c_base is not None and unique_slots is not None:
        safe = unique_slots.clamp(min=0).long()
        c = c_base.to(f)
        if pad_mask is not None:
            c = c * pad_mask.to(f).unsqueeze(-1)
        eku = E_k.to(f)[safe].view(*safe.shape, H, hd)
        evu = E_v.to(f)[safe].view(*safe.shape, H, hd)
        S = torch.einsum("bkn,bkhi,bkhj->bhnij", c, eku, evu)
        R = P[:, 1:L + 1].t()                             # [L, N]: rho_n^(t+1)
        Wh = W_pe.to(f).view(N, H, hd)
        out = out + torch.einsum("tn,bthi,nhi,bhnij->bthj", R, q, Wh, S)
    return out.reshape(B, L, D)
