"""Head counts beyond the configurations' eight: the forward runs whole head groups of at
most eight heads (one wave each) and the backward groups of at most four, with spare waves
that only stage and synchronise, so any H from 1 up is served.  Forward and backward
against the oracle with the kernel's rounding (2e-3, the tolerance of test_gpu_flash.py) and
in fp32 mode against the exact oracle (1e-4); a 12-head d_model 768 SlotTransformerLM
against the model oracle; head_dim outside {32, 64, 128} is refused with a clear error
(head_dim 128 itself: test_gpu_hd128.py)."""
import pytest
import torch

from oracle import model as omodel
from tests.test_gpu_flash import (TOL_KERNEL_ROUNDING, check_backward, check_forward, kernel_rounding, make_case,
                                  norm_err)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,hd", [(1, 64), (2, 32), (3, 64), (5, 32), (6, 64), (7, 32), (9, 32),
                                  (12, 64), (16, 32), (11, 64)])
def test_head_counts_forward_backward(H, hd):
    c = make_case(2, 70, 150, H, hd, 16, warmup=60, seed=100 + H)
    check_forward(c)
    check_backward(c, seed=H)


@pytest.mark.parametrize("H", [3, 12])
def test_head_counts_fp32_mode(H):
    from tests.test_gpu_fp32_mode import check
    check(make_case(2, 64, 120, H, 64, 32, warmup=50, seed=200 + H), seed=H)


@pytest.mark.parametrize("H", [2, 6])
def test_head_counts_rates_above_64(H):
    """N = 128: the backward's half-waves exchange dpre through LDS at a barrier that the
    spare waves of a partial group also reach."""
    c = make_case(1, 80, 150, H, 64, 128, warmup=60, seed=300 + H)
    check_forward(c)
    check_backward(c, seed=H)


def test_model_twelve_heads_d768():
    from mathbrain.model import SlotTransformerLM
    from mathbrain.synthetic import make_batch
    V, D, H, N, B, L = 300, 768, 12, 16, 2, 48
    torch.manual_seed(7)
    m = SlotTransformerLM(V, D, 1, H, N=N, dropout=0.0, max_hl=1024.0).cuda()
    d = make_batch(B, L, V, N, 100, seed=8, max_hl=1024.0)
    x, uniq, cb = d["x"], d["unique"], d["c_base"]
    pm = uniq >= 0
    g = torch.Generator().manual_seed(9)
    R = torch.randn(B, L, V, generator=g)
    logits = m(x.cuda(), uniq.cuda(), None, cb.cuda(), None, pm.cuda())
    (logits * R.cuda()).sum().backward()
    p = {k: v.detach().cpu().double().requires_grad_() for k, v in m.state_dict().items()
         if k not in ("ema_rhos", "lm_head.weight")}
    want = omodel.lm_forward(p, x, 1, H, m.ema_rhos.cpu(), V, unique_slots=uniq, c_base=cb.double(),
                             pad_mask=pm, gate_round=kernel_rounding(N, D // H), t_eval=list(range(L)))
    (want * R.double()).sum().backward()
    assert norm_err(logits, want) < 1e-4
    grads = dict(m.named_parameters())
    for k, v in p.items():
        tol = 1e-2 if k.endswith("pe_proj.weight") else 1e-4
        assert norm_err(grads[k].grad, v.grad) < tol, k


@pytest.mark.parametrize("hd", [16, 96])
def test_unsupported_head_dim_is_refused(hd):
    from mathbrain._lib import HipKernelError
    from tests.test_gpu_flash import gpu_forward
    c = make_case(1, 16, 50, 2, 32, 16, warmup=0, seed=1)
    H = 2
    c["Q"] = torch.randn(1, H, 16, hd)
    c["E_k"] = torch.randn(1, c["K"], H * hd)
    c["E_v"] = torch.randn(1, c["K"], H * hd)
    c["W"] = torch.randn(16, H * hd)
    with pytest.raises(HipKernelError, match=f"head_dim {hd}"):
        gpu_forward(c)
