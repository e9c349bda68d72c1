"""Parity of the HIP factored linear EMA (mb_factored_* behind
mathbrain/factored_ema.py) with the CPU oracle of factored_ema.py (oracle/factored.py,
float64): outputs and the gradients of Q, E_k, E_v and W_pe, with and without c_base, at
tile edges and at the model's head shape, plus the layer.  Tolerance (fp32 kernels against
float64): 1e-4 relative, norm-wise (max |diff| / max |ref|)."""
import math

import pytest
import torch

from oracle import factored as of

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rel(a, b):
    a = a.detach().cpu().to(torch.float64)
    b = b.detach().cpu().to(torch.float64)
    return float((a - b).abs().max() / b.abs().max().clamp(min=1e-300))


def make(B, L, V, H, hd, N, K, seed, cbase=True, scale=0.5):
    g = torch.Generator().manual_seed(seed)
    D = H * hd
    Q = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    x = torch.randint(0, V, (B, L), generator=g)
    Ek = torch.randn(V, D, generator=g, dtype=torch.float64) * scale
    Ev = torch.randn(V, D, generator=g, dtype=torch.float64) * scale
    rhos = torch.exp(-math.log(2.0) / torch.logspace(0, math.log10(1024.0), N, dtype=torch.float64))
    W = torch.randn(N, D, generator=g, dtype=torch.float64) * scale
    kw = {}
    if cbase:
        u = torch.randint(-1, V, (B, K), generator=g)
        kw = dict(c_base=torch.rand(B, K, N, generator=g, dtype=torch.float64) * 4,
                  unique_slots=u, pad_mask=u >= 0)
    return (Q, x, Ek, Ev, rhos, W, H), kw


def run_both(args, kw, dO_seed=99):
    from mathbrain.factored_ema import factored_ema_forward
    Q, x, Ek, Ev, rhos, W, H = args
    leaves = [t.clone().requires_grad_(True) for t in (Q, Ek, Ev, W)]
    want = of.closed_form(leaves[0], x, leaves[1], leaves[2], rhos, leaves[3], H, **kw)
    g = torch.Generator().manual_seed(dO_seed)
    dO = torch.randn(want.shape, generator=g, dtype=torch.float64)
    want.backward(dO)
    cu = lambda t: None if t is None else t.to(torch.float32).cuda() if t.is_floating_point() else t.cuda()
    dl = [cu(t).requires_grad_(True) for t in (Q, Ek, Ev, W)]
    kwd = {k: cu(v) for k, v in kw.items()}
    got = factored_ema_forward(dl[0], x.cuda(), dl[1], dl[2], cu(rhos), dl[3], H, **kwd)
    got.backward(cu(dO))
    errs = {"O": rel(got, want)}
    for name, a, b in zip(("dQ", "dE_k", "dE_v", "dW_pe"), dl, leaves):
        errs[name] = rel(a.grad, b.grad)
    return errs


@pytest.mark.parametrize("L", [1, 2, 63, 64, 65, 130])
@pytest.mark.parametrize("hd", [32, 64])
def test_gpu_factored_matches_oracle_edges(L, hd):
    args, kw = make(2, L, 37, 2, hd, 5, 9, seed=L + hd)
    print(f"factored L={L} hd={hd}", flush=True)
    errs = run_both(args, kw)
    assert max(errs.values()) < TOL, errs


@pytest.mark.parametrize("N,cbase", [(1, False), (16, True), (64, True), (64, False)])
def test_gpu_factored_rates_and_c_base(N, cbase):
    args, kw = make(3, 96, 50, 4, 64, N, 40, seed=N, cbase=cbase)
    print(f"factored N={N} c_base={cbase}", flush=True)
    errs = run_both(args, kw)
    assert max(errs.values()) < TOL, errs


def test_gpu_factored_model_shape():
    # the model's head shape (D=512, 8 heads of 64, N=64), 256 steps, 300 slots, Zipf-like ids
    args, kw = make(2, 256, 2000, 8, 64, 64, 300, seed=7, scale=0.05)
    print("factored model shape", flush=True)
    errs = run_both(args, kw)
    assert max(errs.values()) < TOL, errs


def test_gpu_factored_matches_loop_restatement():
    # the step-by-step restatement of factored_ema.py:22-96 (not only its closed form)
    from mathbrain.factored_ema import factored_ema_forward
    (Q, x, Ek, Ev, rhos, W, H), kw = make(2, 70, 30, 2, 32, 6, 12, seed=11)
    want = of.loop_forward(Q, x, Ek, Ev, rhos, W, H, **kw)
    f = lambda t: t.to(torch.float32).cuda()
    got = factored_ema_forward(f(Q), x.cuda(), f(Ek), f(Ev), f(rhos), f(W), H,
                               c_base=f(kw["c_base"]), unique_slots=kw["unique_slots"].cuda(),
                               pad_mask=kw["pad_mask"].cuda())
    assert rel(got, want) < TOL


def test_gpu_factored_layer_matches_reference_composition():
    # FactoredLinearEMALayer (factored_ema.py:99-146) against the same composition with the
    # oracle in float64
    from mathbrain.factored_ema import FactoredLinearEMALayer
    torch.manual_seed(0)
    B, L, V, D, H, N, K = 2, 48, 40, 128, 2, 8, 10
    layer = FactoredLinearEMALayer(D, H, 0.0, N).cuda()
    g = torch.Generator().manual_seed(1)
    x_q = torch.randn(B, L, D, generator=g)
    x = torch.randint(0, V, (B, L), generator=g)
    E = torch.randn(V, D, generator=g)
    rhos = torch.exp(-math.log(2.0) / torch.logspace(0, 2, N))
    C = torch.rand(B, L, N, generator=g) * 3
    u = torch.randint(-1, V, (B, K), generator=g)
    cb = torch.rand(B, K, N, generator=g)
    out = layer(x_q.cuda(), x.cuda(), E.cuda(), rhos.cuda(), C.cuda(), c_base=cb.cuda(),
                unique_slots=u.cuda(), pad_mask=(u >= 0).cuda())
    ref = {k: v.detach().cpu().double() for k, v in layer.state_dict().items()}
    f = torch.float64
    mem = torch.nn.functional.layer_norm(E.to(f), (D,), ref["ln_kv.weight"], ref["ln_kv.bias"])
    Ek, Ev = mem @ ref["k_proj.weight"].t(), mem @ ref["v_proj.weight"].t()
    gate = (C.to(f) + 1.0) @ ref["pe_proj.weight"].t()
    Qt = torch.nn.functional.layer_norm(x_q.to(f) * gate, (D,), ref["ln_q.weight"], ref["ln_q.bias"])
    Qt = Qt @ ref["q_proj.weight"].t()
    o = of.closed_form(Qt, x, Ek, Ev, rhos.to(f), ref["pe_proj.weight"].t(), H, c_base=cb.to(f),
                       unique_slots=u, pad_mask=u >= 0)
    want = o @ ref["o_proj.weight"].t()
    assert rel(out, want) < TOL
    out.sum().backward()
    assert all(torch.isfinite(p.grad).all() for p in layer.parameters() if p.grad is not None)
