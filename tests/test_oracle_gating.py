"""Pins the gating oracle (oracle/gating.py) to torch's own library modules and to what
the mathematics fixes, so that the GPU gating tests compare against something checked.

* ``forward`` equals the reference's CPU branch written with torch modules
  (nn.Linear pe_proj and q_proj, F.silu, nn.LayerNorm; triton_fused_gating.py:179-197).
* ``backward_formulas`` (the reference kernel's closed form, :61-119, :173-175) equals
  torch autograd of the module forward in float64, and float64 gradcheck passes.
* Special cases: W_pe = 0 gives a zero gate, so every LayerNorm row is ln_b; with
  ln_w = 1, ln_b = 0 every output row has mean 0 and variance var / (var + eps).
"""
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import gating


def modules(D, N, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    pe = nn.Linear(N, D, bias=False).to(dtype)
    lnq = nn.LayerNorm(D).to(dtype)
    qp = nn.Linear(D, D, bias=False).to(dtype)
    with torch.no_grad():
        pe.weight.copy_(torch.randn(D, N, generator=g, dtype=dtype) * 0.3)
        lnq.weight.copy_(1 + 0.1 * torch.randn(D, generator=g, dtype=dtype))
        lnq.bias.copy_(0.1 * torch.randn(D, generator=g, dtype=dtype))
        qp.weight.copy_(torch.randn(D, D, generator=g, dtype=dtype) * 0.05)
    return pe, lnq, qp


def reference_cpu_branch(x_q, C_seq, pe, lnq, qp, use_silu):
    # triton_fused_gating.py:180-197 with HAS_TRITON false
    bias_offset = pe.weight.sum(dim=1)
    P_pre = pe(C_seq)
    p_lin = P_pre + bias_offset
    P_gate = F.silu(p_lin) if use_silu else p_lin
    return qp(lnq(x_q * P_gate))


@pytest.mark.parametrize("use_silu", [True, False])
def test_forward_equals_module_composition(use_silu):
    B, L, D, N = 2, 7, 48, 5
    pe, lnq, qp = modules(D, N, 0)
    g = torch.Generator().manual_seed(1)
    x_q = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    C = torch.rand(B, L, N, generator=g, dtype=torch.float64) * 5
    want = reference_cpu_branch(x_q, C, pe, lnq, qp, use_silu)
    got = gating.forward(x_q, C, pe.weight, lnq.weight, lnq.bias, qp.weight, use_silu)
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_zero_projection_gives_ln_bias_rows():
    B, L, D, N = 1, 5, 32, 4
    g = torch.Generator().manual_seed(2)
    x_q = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    C = torch.rand(B, L, N, generator=g, dtype=torch.float64)
    ln_w = torch.randn(D, generator=g, dtype=torch.float64)
    ln_b = torch.randn(D, generator=g, dtype=torch.float64)
    y = gating.gate_ln(x_q, C @ torch.zeros(N, D, dtype=torch.float64), torch.zeros(D, dtype=torch.float64),
                       ln_w, ln_b)
    assert torch.allclose(y, ln_b.expand_as(y), atol=1e-15)


def test_unit_affine_rows_are_standardised():
    B, L, D = 3, 4, 64
    g = torch.Generator().manual_seed(3)
    x_q = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    p_pre = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    bias = torch.randn(D, generator=g, dtype=torch.float64)
    y = gating.gate_ln(x_q, p_pre, bias, torch.ones(D, dtype=torch.float64), torch.zeros(D, dtype=torch.float64))
    e = x_q * F.silu(p_pre + bias)
    var = e.var(-1, unbiased=False)
    assert torch.allclose(y.mean(-1), torch.zeros(B, L, dtype=torch.float64), atol=1e-12)
    assert torch.allclose(y.pow(2).mean(-1), var / (var + 1e-5), rtol=1e-10)


@pytest.mark.parametrize("use_silu", [True, False])
def test_closed_form_backward_equals_autograd(use_silu):
    B, L, D = 2, 6, 40
    g = torch.Generator().manual_seed(4)
    x_q = torch.randn(B, L, D, generator=g, dtype=torch.float64, requires_grad=True)
    p_pre = torch.randn(B, L, D, generator=g, dtype=torch.float64, requires_grad=True)
    bias = torch.randn(D, generator=g, dtype=torch.float64, requires_grad=True)
    ln_w = (1 + 0.2 * torch.randn(D, generator=g, dtype=torch.float64)).requires_grad_()
    ln_b = (0.2 * torch.randn(D, generator=g, dtype=torch.float64)).requires_grad_()
    dy = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    # the module forward: nn.LayerNorm semantics through F.layer_norm, F.silu
    p_lin = p_pre + bias
    y = F.layer_norm(x_q * (F.silu(p_lin) if use_silu else p_lin), (D,), ln_w, ln_b, 1e-5)
    want = torch.autograd.grad(y, (x_q, p_pre, bias, ln_w, ln_b), dy)
    got = gating.backward_formulas(dy, x_q.detach(), p_pre.detach(), bias.detach(), ln_w.detach(),
                                   ln_b.detach(), use_silu)
    for a, b in zip(got, want):
        assert torch.allclose(a, b, rtol=1e-9, atol=1e-11)


def test_gradcheck():
    B, L, D = 1, 3, 8
    g = torch.Generator().manual_seed(5)
    args = [torch.randn(B, L, D, generator=g, dtype=torch.float64, requires_grad=True),
            torch.randn(B, L, D, generator=g, dtype=torch.float64, requires_grad=True),
            torch.randn(D, generator=g, dtype=torch.float64, requires_grad=True),
            torch.randn(D, generator=g, dtype=torch.float64, requires_grad=True),
            torch.randn(D, generator=g, dtype=torch.float64, requires_grad=True)]
    assert torch.autograd.gradcheck(lambda *a: gating.gate_ln(*a), args)
