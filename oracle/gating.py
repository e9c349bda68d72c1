"""TEST INFRASTRUCTURE ONLY: CPU restatement of the fused symmetric query gating (the checker).

``forward``   Q_ln = LayerNorm_{eps=1e-5}(x_q * SiLU(P_pre + bias)) with
              P_pre = C_seq @ W_pe^T and bias = W_pe.sum(1), i.e. the gate is
              taken on C_seq + 1 (mathbrain/triton_fused_gating.py:179-197, the
              CPU branch :187-195; the kernel form is :12-57).
``backward_formulas``
              the reference kernel's closed-form backward
              (triton_fused_gating.py:61-119, reductions :173-175), evaluated in
              torch; autograd of ``forward`` must agree with it.
"""
import torch
import torch.nn.functional as F


def gate_ln(x_q, p_pre, bias, ln_w, ln_b, use_silu=True, eps=1e-5):
    """FusedGatingFunction.forward semantics (triton_fused_gating.py:29-57): x_ln [B, L, D]."""
    p_lin = p_pre + bias
    g = F.silu(p_lin) if use_silu else p_lin
    x_emb = x_q * g
    return F.layer_norm(x_emb, (x_q.shape[-1],), ln_w, ln_b, eps)


def forward(x_q, C_seq, pe_weight, ln_w, ln_b, q_weight, use_silu=True, linear=None, pe_linear=None):
    """fused_apply_symmetric_query_gating (triton_fused_gating.py:179-197).  ``linear`` /
    ``pe_linear`` (u, w) -> u @ w.T evaluate the q_proj / pe_proj Linears (default: exact)."""
    mm = lambda u, w: u @ w.t()
    bias = pe_weight.sum(dim=1)                      # :180
    p_pre = (pe_linear or mm)(C_seq, pe_weight)      # :183
    q_ln = gate_ln(x_q, p_pre, bias, ln_w, ln_b, use_silu)
    return (linear or mm)(q_ln, q_weight)            # :197


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
    x_hat = (x_emb - mu) * rstd                      # :95
    dln_w = (dy * x_hat).reshape(-1, D).sum(0)       # :96, :173
    dln_b = dy.reshape(-1, D).sum(0)                 # :97, :174
    dx_hat = dy * ln_w                               # :101
    c1 = dx_hat.mean(-1, keepdim=True)               # :102
    c2 = (dx_hat * x_hat).mean(-1, keepdim=True)     # :103
    dx_emb = (dx_hat - c1 - x_hat * c2) * rstd       # :104
    dx_q = dx_emb * g                                # :106
    dp_gate = dx_emb * x_q                           # :109
    dsilu = (g + sig * (1.0 - g)) if use_silu else torch.ones_like(g)   # :113-116
    dp_pre = dp_gate * dsilu                         # :118
    dbias = dp_pre.reshape(-1, D).sum(0)             # :175
    return dx_q, dp_pre, dbias, dln_w, dln_b
