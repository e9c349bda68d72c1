"""Pins the model-level oracle (oracle/model.py): with no carried state, the reference's
CPU path (dense attention over the whole vocabulary, model.py:88-99) and the device
path (unique-slot attention with the absent-slot mass, model.py:63-87) are the same
function, in float64.  Also checks the CPU guard of the product model."""
import math

import pytest
import torch

from oracle import model as omodel


def params(V, D, n_layers, H, N, d_ff, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=0.3: (torch.randn(*s, generator=g, dtype=dtype) * sc)
    p = {"embed.weight": r(V, D, sc=1.0), "final_norm.weight": 1 + r(D, sc=0.1)}
    for l in range(n_layers):
        pre = f"layers.{l}."
        p.update({
            pre + "attn_norm.weight": 1 + r(D, sc=0.1), pre + "ffn_norm.weight": 1 + r(D, sc=0.1),
            pre + "attn.q_proj.weight": r(D, D), pre + "attn.k_proj.weight": r(D, D),
            pre + "attn.v_proj.weight": r(D, D), pre + "attn.o_proj.weight": r(D, D),
            pre + "attn.pe_proj.weight": r(D, N), pre + "attn.ln_kv.weight": 1 + r(D, sc=0.1),
            pre + "attn.ln_kv.bias": r(D, sc=0.1), pre + "attn.ln_q.weight": 1 + r(D, sc=0.1),
            pre + "attn.ln_q.bias": r(D, sc=0.1), pre + "ffn.w1.weight": r(d_ff, D),
            pre + "ffn.w2.weight": r(D, d_ff), pre + "ffn.w3.weight": r(d_ff, D)})
    return p


@pytest.mark.parametrize("use_silu", [True, False])
def test_dense_cpu_path_equals_sparse_device_path(use_silu):
    V, D, H, N, L, B = 40, 16, 2, 4, 12, 2
    p = params(V, D, 2, H, N, 32, seed=0)
    g = torch.Generator().manual_seed(1)
    x = torch.randint(0, V, (B, L), generator=g)
    hl = torch.logspace(0, math.log10(64), N, dtype=torch.float64)
    rhos = torch.exp(-math.log(2.0) / hl)
    dense = omodel.lm_forward(p, x, 2, H, rhos, V, use_silu=use_silu, attention="dense")
    sparse = omodel.lm_forward(p, x, 2, H, rhos, V, use_silu=use_silu, attention="sparse")
    assert dense.shape == (B, L, V)
    assert torch.allclose(dense, sparse, rtol=1e-10, atol=1e-10)


def test_product_model_has_no_cpu_path():
    from mathbrain.model import SlotTransformerLM
    m = SlotTransformerLM(50, 64, 1, 2, N=4, dropout=0.0)
    with pytest.raises(NotImplementedError):
        m(torch.randint(0, 50, (1, 8)))


def test_autocast_linear_matches_torch_bf16_matmul():
    """oracle.model.linear with dtype bf16 (the model oracle's autocast roundings) against
    torch's own bf16 matmul and its autograd on the CPU (float32 accumulation, one bf16
    rounding of the output and of each gradient product): equal up to the accumulation order,
    i.e. at most one bf16 step apart, and equal on nearly every element."""
    g = torch.Generator().manual_seed(0)
    a = torch.randn(3, 40, 96, generator=g, dtype=torch.float64)
    w = torch.randn(72, 96, generator=g, dtype=torch.float64)
    dy = torch.randn(3, 40, 72, generator=g, dtype=torch.float64)
    ao, wo = a.clone().requires_grad_(), w.clone().requires_grad_()
    y = omodel.linear(ao, wo, torch.bfloat16)
    y.backward(dy)
    ab, wb = a.to(torch.bfloat16).requires_grad_(), w.to(torch.bfloat16).requires_grad_()
    yb = ab @ wb.t()
    yb.backward(dy.to(torch.bfloat16))
    r = lambda t: t.to(torch.bfloat16).double().abs()
    mag = (r(a) @ r(w).t(), r(dy) @ r(w), r(dy).reshape(-1, 72).t() @ r(a).reshape(-1, 96))
    for (got, want), m in zip(((y, yb), (ao.grad, ab.grad), (wo.grad, wb.grad)), mag):
        want = want.double()
        assert got.dtype == torch.float64
        # values are bf16 numbers
        assert torch.equal(got, got.to(torch.bfloat16).double())
        # one bf16 step (8 significant bits) plus float32 accumulation over <= 120 terms
        bound = want.abs() * 2.0**-7 + m * 120 * 2.0**-24
        assert ((got - want).abs() <= bound).all()
        assert (got == want).double().mean() > 0.97
    # no rounding without a dtype, and the rounding helper rounds both ways
    assert torch.equal(omodel.linear(a, w), a @ w.t())
    t = a.clone().requires_grad_()
    omodel.rounded(t, torch.bfloat16).backward(torch.ones_like(a) / 3)
    assert torch.equal(t.grad, (torch.ones_like(a) / 3).to(torch.bfloat16).double())
