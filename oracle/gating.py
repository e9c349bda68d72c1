"""TEST INFRASTRUCTURE ONLY: CPU restatement of the fused symmetric query gating.

``forward``   Q_ln = LayerNorm_{eps=1e-5}(x_q * SiLU(P_pre + bias)) with
              P_pre = C_seq @ W_pe^T and bias = W_pe.sum(1), i.e. the gate is
              taken on C_seq + 1 (mathbrain/triton_fused_gating.py:264-282, the
              CPU branch; the kernel form is :96-142).
``backward_formulas``
              the reference kernel's closed-form backward
              (triton_fused_gating.py:145-204, reductions :258-260), evaluated in
              torch; autograd of ``forward`` must agree with it.
"""
import torch
import torch.nn.functional as F


def gate_ln(x_q, p_pre, bias, ln_w, ln_b, use_silu=True, eps=1e-5):
    """FusedGatingFunction.forward semantics: returns x_ln [B, L, D]."""
    p_lin = p_pre + bias
    g = F.silu(p_lin) if use_silu else p_lin
    x_emb = x_q * g
    return F.layer_norm(x_emb, (x_q.shape[-1],), ln_w, ln_b, eps)


def forward(x_q, C_seq, pe_weight, ln_w, ln_b, q_weight, use_silu=True):
    """fused_apply_symmetric_query_gating (triton_fused_gating.py:264-282)."""
    bias = pe_weight.sum(dim=1)                      # :265
    p_pre = C_seq @ pe_weight.t()                    # :268
    q_ln = gate_ln(x_q, p_pre, bias, ln_w, ln_b, use_silu)
    return q_ln @ q_weight.t()                       # :282


@torch.no_grad()
def backward_formulas(dy, x_q, p_pre, bias, ln_w, ln_b, use_silu=True, eps=1e-5):
    """Returns (dx_q, dp_pre, dbias, dln_w, dln_b) as _fused_gating_bwd computes them."""
    D = x_q.shape[-1]
    p_lin = p_pre + bias
    sig = torch.sigmoid(p_lin)
    g = p_lin * sig if use_silu else p_lin
    x_emb = x_q * g
    mu = x_emb.mean(-1, keepdim=True)
    var = ((x_emb - mu) ** 2).mean(-1, keepdim=True)
    rstd = 1.0 / torch.sqrt(var + eps)
    x_hat = (x_emb - mu) * rstd                      # :180
    dln_w = (dy * x_hat).reshape(-1, D).sum(0)       # :181, :258
    dln_b = dy.reshape(-1, D).sum(0)                 # :182, :259
    dx_hat = dy * ln_w                               # :186
    c1 = dx_hat.mean(-1, keepdim=True)               # :187
    c2 = (dx_hat * x_hat).mean(-1, keepdim=True)     # :188
    dx_emb = (dx_hat - c1 - x_hat * c2) * rstd       # :189
    dx_q = dx_emb * g                                # :191
    dp_gate = dx_emb * x_q                           # :194
    dsilu = (g + sig * (1.0 - g)) if use_silu else torch.ones_like(g)   # :199
    dp_pre = dp_gate * dsilu                         # :203
    dbias = dp_pre.reshape(-1, D).sum(0)             # :260
    return dx_q, dp_pre, dbias, dln_w, dln_b
