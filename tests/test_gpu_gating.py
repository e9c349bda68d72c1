"""Parity of the HIP query gating (mb_gating_fwd / mb_gating_bwd) with the CPU oracle
(oracle/gating.py, float64) on seeded inputs.

Everything in these kernels is fp32 (no bf16 operand anywhere), so the bar is the task's
fp32 one, 1e-4 relative, measured norm-wise as max|got - want| / max|want|.  Inputs are
at the model's own scales: x_q ~ N(0, 1) embeddings, counters C_seq from the EMA scan of
a Zipf sequence (0 .. a few hundred), W_pe ~ N(0, 0.02).
"""
import pytest
import torch
import torch.nn as nn

from oracle import gating
from oracle import scan as oscan

pytestmark = pytest.mark.gpu

TOL_FP32 = 1e-4


def norm_err(got, want):
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    return float((got - want).abs().max() / want.abs().max().clamp(min=1e-300))


def case(B, L, D, N, V=500, seed=0, ws=0.02):
    from mathbrain.synthetic import make_batch
    d = make_batch(B, L, V, N, 256, seed=seed)
    C = torch.from_numpy(oscan.query_scan(d["x"], d["rhos"], V, d["c_base"], d["unique"])).float()
    g = torch.Generator().manual_seed(seed + 1)
    x_q = torch.randn(B, L, D, generator=g)
    W = torch.randn(D, N, generator=g) * ws          # pe_proj.weight [D, N]
    ln_w = 1 + 0.1 * torch.randn(D, generator=g)
    ln_b = 0.1 * torch.randn(D, generator=g)
    dy = torch.randn(B, L, D, generator=g)
    return dict(x_q=x_q, C=C, W=W, ln_w=ln_w, ln_b=ln_b, dy=dy)


def oracle_grads(c, use_silu):
    dt = torch.float64
    x_q = c["x_q"].to(dt).requires_grad_()
    W = c["W"].to(dt).requires_grad_()
    ln_w = c["ln_w"].to(dt).requires_grad_()
    ln_b = c["ln_b"].to(dt).requires_grad_()
    p_pre = c["C"].to(dt) @ W.t()
    y = gating.gate_ln(x_q, p_pre, W.sum(1), ln_w, ln_b, use_silu)
    grads = torch.autograd.grad(y, (x_q, W, ln_w, ln_b), c["dy"].to(dt))
    return y.detach(), grads


@pytest.mark.parametrize("D,N", [(128, 16), (512, 64), (384, 128), (1000, 7), (256, 32), (768, 64),
                                 (1024, 16), (512, 30), (256, 1)])
@pytest.mark.parametrize("use_silu", [True, False])
def test_folded_projection_fwd_bwd(D, N, use_silu):
    from mathbrain.triton_fused_gating import GatedQueryFunction
    c = case(2, 67, D, N, seed=D + N)
    want_y, want_g = oracle_grads(c, use_silu)
    x_q = c["x_q"].cuda().requires_grad_()
    Wt = c["W"].cuda().t().contiguous().requires_grad_()
    ln_w = c["ln_w"].cuda().requires_grad_()
    ln_b = c["ln_b"].cuda().requires_grad_()
    y = GatedQueryFunction.apply(x_q, c["C"].cuda(), Wt, ln_w, ln_b, use_silu)
    y.backward(c["dy"].cuda())
    torch.cuda.synchronize()
    errs = {"y": norm_err(y, want_y), "dx_q": norm_err(x_q.grad, want_g[0]),
            "dW": norm_err(Wt.grad.t(), want_g[1]), "dln_w": norm_err(ln_w.grad, want_g[2]),
            "dln_b": norm_err(ln_b.grad, want_g[3])}
    print(errs)
    assert max(errs.values()) < TOL_FP32, errs


@pytest.mark.parametrize("use_silu", [True, False])
@pytest.mark.parametrize("D", [512, 200])
def test_fused_gating_function_matches_reference_formulas(use_silu, D):
    """FusedGatingFunction keeps the reference autograd signature: gradients of
    (x_q, p_pre, bias, ln_w, ln_b) equal the reference kernel's closed form (D = 512: the
    one-row-per-wave backward; D = 200: the tiled one)."""
    from mathbrain.triton_fused_gating import FusedGatingFunction
    c = case(3, 41, D, 64, seed=7)
    dt = torch.float64
    p_pre = c["C"] @ c["W"].t()
    bias = c["W"].sum(1)
    want_y = gating.gate_ln(c["x_q"].to(dt), p_pre.to(dt), bias.to(dt), c["ln_w"].to(dt),
                            c["ln_b"].to(dt), use_silu)
    want = gating.backward_formulas(c["dy"].to(dt), c["x_q"].to(dt), p_pre.to(dt), bias.to(dt),
                                    c["ln_w"].to(dt), c["ln_b"].to(dt), use_silu)
    args = [t.cuda().requires_grad_() for t in (c["x_q"], p_pre, bias, c["ln_w"], c["ln_b"])]
    y = FusedGatingFunction.apply(*args, use_silu)
    y.backward(c["dy"].cuda())
    assert norm_err(y, want_y) < TOL_FP32
    for name, a, w in zip(("dx_q", "dp_pre", "dbias", "dln_w", "dln_b"), args, want):
        assert norm_err(a.grad, w) < TOL_FP32, name


def test_module_entry_point_and_strided_rows():
    """fused_apply_symmetric_query_gating with the model's modules, a strided x_q view and
    a single row; equals the reference CPU branch composed from torch modules."""
    from mathbrain.triton_fused_gating import fused_apply_symmetric_query_gating
    D, N = 256, 32
    c = case(2, 33, D, N, seed=3)
    pe = nn.Linear(N, D, bias=False)
    lnq = nn.LayerNorm(D)
    qp = nn.Linear(D, D, bias=False)
    with torch.no_grad():
        pe.weight.copy_(c["W"][:D, :N])
        lnq.weight.copy_(c["ln_w"][:D])
        lnq.bias.copy_(c["ln_b"][:D])
    big = torch.randn(2, 33, 2 * D)
    x_q = big[..., ::2]                               # column stride 2: copied to rows
    x_rows = big[..., :D]                             # row stride 2D, contiguous columns
    for xq in (x_q, x_rows, x_rows[:1, :1]):
        C = c["C"][: xq.shape[0], : xq.shape[1]]
        want = qp(lnq(xq * torch.nn.functional.silu(pe(C) + pe.weight.sum(1))))
        got = fused_apply_symmetric_query_gating(xq.cuda(), C.cuda(), pe.cuda(), lnq.cuda(),
                                                 qp.cuda())
        pe.cpu(), lnq.cpu(), qp.cpu()
        assert norm_err(got, want) < TOL_FP32


def test_empty_rows():
    from mathbrain.triton_fused_gating import GatedQueryFunction
    x = torch.zeros(0, 5, 64, device="cuda", requires_grad=True)
    y = GatedQueryFunction.apply(x, torch.zeros(0, 5, 8, device="cuda"),
                                 torch.zeros(8, 64, device="cuda"), torch.ones(64, device="cuda"),
                                 torch.zeros(64, device="cuda"))
    assert y.shape == (0, 5, 64)
