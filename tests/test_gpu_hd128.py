"""head_dim 128.  The forward runs two waves per head, one 16-step tile each (a lane's queries,
outputs and gate tiles for 128 dims fill the register budget that two tiles of 64 dims do),
with the group's W fragments in LDS; groups hold up to four heads, fewer where that LDS would
not fit (N = 128).  The backward runs each head as two 64-dim sub-heads on two waves that add
their score and dO . v partial sums (and D = dO . O) through LDS.  Checked against the oracle
with the kernel's rounding (2e-3, the tolerance of test_gpu_flash.py) over head counts, rates
(N = 128 takes the backward's half-wave exchange as well), softmax modes, stored or
recomputed scores, ragged lengths, padding slots and vocabulary rows, against the exact
oracle at the configurations' own scales (2e-2), and a 2-head d_model 256 SlotTransformerLM
against the model oracle."""
import pytest
import torch

from oracle import model as omodel
from tests.test_gpu_flash import CFG, check_backward, check_forward, kernel_rounding, make_case, norm_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H", [1, 2, 3, 4, 8])
def test_hd128_forward_head_counts(H):
    check_forward(make_case(2, 70, 150, H, 128, 16, warmup=60, seed=500 + H))


@pytest.mark.parametrize("N", [16, 64, 128])
def test_hd128_forward_rates(N):
    check_forward(make_case(2, 96, 400, 4, 128, N, warmup=200, seed=510 + N))


@pytest.mark.parametrize("use_silu", [True, False])
@pytest.mark.parametrize("absent_mass", [True, False])
def test_hd128_forward_flags(use_silu, absent_mass):
    check_forward(make_case(2, 50, 120, 2, 128, 32, warmup=40, seed=520), use_silu, absent_mass)


@pytest.mark.parametrize("L", [1, 17, 33, 100])
def test_hd128_forward_ragged(L):
    check_forward(make_case(2, L, 200, 4, 128, 16, warmup=100, seed=530 + L))


def test_hd128_forward_padding_slots():
    check_forward(make_case(2, 64, 150, 4, 128, 32, warmup=50, seed=540, pad_slots=23))


def test_hd128_forward_exact_scales():
    check_forward(make_case(2, 256, 2000, 4, 128, 64, warmup=1024, seed=550, **CFG), exact=True)


@pytest.mark.parametrize("H", [1, 2, 3, 4])
def test_hd128_backward_head_counts(H):
    check_backward(make_case(2, 70, 150, H, 128, 16, warmup=60, seed=600 + H), seed=H)


@pytest.mark.parametrize("N", [16, 64, 128])
@pytest.mark.parametrize("stored_scores", [True, False])
def test_hd128_backward_rates(N, stored_scores):
    check_backward(make_case(2, 80, 300, 2, 128, N, warmup=150, seed=610 + N), seed=N,
                   stored_scores=stored_scores)


@pytest.mark.parametrize("use_silu", [True, False])
@pytest.mark.parametrize("absent_mass", [True, False])
def test_hd128_backward_flags(use_silu, absent_mass):
    check_backward(make_case(2, 50, 120, 2, 128, 32, warmup=40, seed=620), use_silu, absent_mass, seed=3,
                   stored_scores=False)


@pytest.mark.parametrize("L", [1, 17, 77])
def test_hd128_backward_ragged(L):
    check_backward(make_case(2, L, 200, 2, 128, 16, warmup=100, seed=630 + L), seed=L)


def test_hd128_backward_padding_slots():
    check_backward(make_case(2, 64, 150, 4, 128, 32, warmup=50, seed=640, pad_slots=23), seed=5)


def test_hd128_backward_exact_scales():
    check_backward(make_case(1, 256, 2000, 2, 128, 64, warmup=1024, seed=650, **CFG), exact=True, seed=6)


@pytest.mark.parametrize("kv_table", [False, True])
def test_hd128_model(kv_table):
    """SlotTransformerLM with two heads of 128 (vocabulary rows when kv_table) against the
    model oracle with the kernel's gate rounding: logits and every parameter gradient."""
    from mathbrain.model import SlotTransformerLM
    from mathbrain.synthetic import make_batch
    V, D, H, N, B, L = 300, 256, 2, 16, 2, 48
    torch.manual_seed(17)
    m = SlotTransformerLM(V, D, 1, H, N=N, dropout=0.0, max_hl=1024.0).cuda()
    m.kv_table = kv_table
    d = make_batch(B, L, V, N, 100, seed=18, max_hl=1024.0)
    x, uniq, cb = d["x"], d["unique"], d["c_base"]
    pm = uniq >= 0
    R = torch.randn(B, L, V, generator=torch.Generator().manual_seed(19))
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


def test_hd128_fp32_mode_is_refused():
    from mathbrain._lib import HipKernelError
    from mathbrain.triton_flash_ema import flash_ema_forward
    c = make_case(1, 16, 50, 2, 128, 16, warmup=0, seed=1)
    with pytest.raises(HipKernelError, match="head_dim"):
        flash_ema_forward(c["Q"].cuda(), c["x"].cuda(), c["E_k"].cuda(), c["E_v"].cuda(), c["W"].cuda(),
                          c["rhos"].cuda(), c["V"], c["unique"].cuda(), c["K"], c["Cb"].cuda(),
                          precision="fp32")
