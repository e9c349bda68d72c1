"""The dense entry point flash_ema_attention.flash_ema_forward (flash_ema_attention.py:19-85)
on the HIP path against the oracle's restatement of it, at the reference's own CPU-runnable
configuration (configuration 1: B=2, T=128, d_model 128, 4 heads x 32, N=16, V=1000,
uniform ids, half-lives 4..1024, weights N(0, 0.02)), outputs and gradients; and
compute_query_ema_history_pt.  Tolerance: 2e-2 norm-wise against the exact float64 oracle
(the gate GEMM takes fp16 operands), the scan 1e-5."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as att
from oracle import scan as oscan

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / b.abs().max())


def test_gpu_dense_entry_point_matches_dense_oracle():
    from mathbrain.flash_ema_attention import flash_ema_forward
    B, L, D, H, N, V = 2, 128, 128, 4, 16, 1000
    g = torch.Generator().manual_seed(0)
    x = torch.randint(0, V, (B, L), generator=g)
    hl = torch.logspace(math.log10(4.0), math.log10(1024.0), N, dtype=torch.float64)
    rhos = torch.exp(-math.log(2.0) / hl)
    Q = torch.randn(B, L, D, generator=g, dtype=torch.float64) * 0.02
    Ek = torch.randn(V, D, generator=g, dtype=torch.float64) * 0.02
    Ev = torch.randn(V, D, generator=g, dtype=torch.float64) * 0.02
    pe = torch.nn.Linear(N, D, bias=False)
    with torch.no_grad():
        pe.weight.copy_(torch.randn(D, N, generator=g) * 0.02)
    leaves = [t.clone().requires_grad_(True) for t in (Q, Ek, Ev)]
    Wd = pe.weight.detach().double().requires_grad_(True)
    want = att.dense(leaves[0], x, leaves[1], leaves[2], rhos, Wd, H)
    dO = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    want.backward(dO)
    pe = pe.cuda()
    dl = [t.float().cuda().requires_grad_(True) for t in (Q, Ek, Ev)]
    got = flash_ema_forward(dl[0], x.cuda(), dl[1], dl[2], rhos.float().cuda(), pe, H)
    got.backward(dO.float().cuda())
    errs = [rel(got, want)] + [rel(a.grad, b.grad) for a, b in zip(dl, leaves)]
    errs.append(rel(pe.weight.grad, Wd.grad))
    assert max(errs) < 2e-2, errs


def test_gpu_dense_entry_rejects_a_gate_bias():
    from mathbrain.flash_ema_attention import flash_ema_forward
    pe = torch.nn.Linear(4, 32).cuda()
    with pytest.raises(NotImplementedError, match="bias"):
        flash_ema_forward(torch.zeros(1, 8, 32).cuda(), torch.zeros(1, 8, dtype=torch.long).cuda(),
                          torch.zeros(5, 32).cuda(), torch.zeros(5, 32).cuda(), torch.ones(4).cuda(),
                          pe, 1)


def test_gpu_query_scan_pt_name():
    from mathbrain.triton_ema_query import compute_query_ema_history_pt
    rng = np.random.default_rng(3)
    x = rng.integers(0, 20, (2, 50))
    rh = np.array([0.9, 0.6, 0.3], np.float32)
    got = compute_query_ema_history_pt(torch.from_numpy(x).cuda(), torch.from_numpy(rh).cuda(), 20)
    want = oscan.query_scan(x, rh, 20)
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-5, atol=1e-30)
