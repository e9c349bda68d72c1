"""Pins the CPU oracle of the factored linear EMA (oracle/factored.py): the step-by-step
restatement of factored_ema_forward (factored_ema.py:22-96) against its independently
written closed form, special cases that reduce to textbook forms, and float64 gradcheck."""
import math

import pytest
import torch

from oracle import factored as of


def case(B=2, L=9, V=13, H=2, hd=4, N=3, K=5, seed=0, dtype=torch.float64, cbase=True):
    g = torch.Generator().manual_seed(seed)
    D = H * hd
    Q = torch.randn(B, L, D, generator=g, dtype=dtype)
    x = torch.randint(0, V, (B, L), generator=g)
    Ek = torch.randn(V, D, generator=g, dtype=dtype) * 0.5
    Ev = torch.randn(V, D, generator=g, dtype=dtype) * 0.5
    rhos = torch.exp(-math.log(2.0) / torch.logspace(0, math.log10(16.0), N, dtype=dtype))
    W = torch.randn(N, D, generator=g, dtype=dtype) * 0.5
    extra = {}
    if cbase:
        u = torch.randint(-1, V, (B, K), generator=g)
        pm = u >= 0
        extra = dict(c_base=torch.rand(B, K, N, generator=g, dtype=dtype) * 3,
                     unique_slots=u, pad_mask=pm)
    return (Q, x, Ek, Ev, rhos, W, H), extra


@pytest.mark.parametrize("seed,cbase", [(0, False), (1, True), (2, True)])
def test_loop_equals_closed_form(seed, cbase):
    args, kw = case(seed=seed, cbase=cbase)
    a = of.loop_forward(*args, **kw)
    b = of.closed_form(*args, **kw)
    assert torch.allclose(a, b, rtol=1e-10, atol=1e-12)


def test_single_rate_is_decayed_linear_attention():
    # N = 1, no c_base: o_t = sum_{s<t} rho^(t-s) ((q_t ⊙ w) . e_k[x_s]) e_v[x_s], i.e. causal
    # linear attention with a strictly-lower decay mask, per head
    (Q, x, Ek, Ev, rhos, W, H), _ = case(N=1, cbase=False, seed=3)
    rho = float(rhos[0])
    B, L, D = Q.shape
    hd = D // H
    out = of.loop_forward(Q, x, Ek, Ev, rhos, W, H)
    t = torch.arange(L, dtype=torch.float64)
    mask = torch.where(t[:, None] > t[None, :], rho ** (t[:, None] - t[None, :]), torch.zeros(()))
    for h in range(H):
        sl = slice(h * hd, (h + 1) * hd)
        qw = Q[..., sl] * W[0, sl]
        want = ((qw @ Ek[x][..., sl].transpose(1, 2)) * mask) @ Ev[x][..., sl]
        assert torch.allclose(out[..., sl], want, rtol=1e-10, atol=1e-12)


def test_first_step_reads_only_c_base():
    # o_0 = sum_n rho_n (q_0 ⊙ W_n)^T S_n(init): the chunk's tokens are not seen yet (:84-94)
    args, kw = case(seed=4)
    Q, x, Ek, Ev, rhos, W, H = args
    o = of.loop_forward(*args, **kw)
    no_tok = of.loop_forward(Q[:, :1], x[:, :1], Ek, Ev, rhos, W, H, **kw)
    assert torch.allclose(o[:, 0], no_tok[:, 0])
    z = of.loop_forward(Q, x, Ek, Ev, rhos, W, H)
    assert torch.all(z[:, 0] == 0)


def test_pad_mask_drops_slots():
    args, kw = case(seed=5)
    kw2 = dict(kw)
    kw2["c_base"] = kw["c_base"] * kw["pad_mask"].unsqueeze(-1)
    kw2["pad_mask"] = None
    assert torch.allclose(of.loop_forward(*args, **kw), of.loop_forward(*args, **kw2))


def test_gradcheck_float64():
    (Q, x, Ek, Ev, rhos, W, H), kw = case(B=1, L=5, V=6, H=1, hd=3, N=2, K=3, seed=6)
    for t in (Q, Ek, Ev, W):
        t.requires_grad_(True)
    f = lambda q, ek, ev, w: of.loop_forward(q, x, ek, ev, rhos, w, H, **kw)
    assert torch.autograd.gradcheck(f, (Q, Ek, Ev, W), eps=1e-6, atol=1e-7)
    g = lambda q, ek, ev, w: of.closed_form(q, x, ek, ev, rhos, w, H, **kw)
    assert torch.autograd.gradcheck(g, (Q, Ek, Ev, W), eps=1e-6, atol=1e-7)
