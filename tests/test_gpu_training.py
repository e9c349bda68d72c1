"""Several optimizer steps of SlotTransformerLM on the HIP path beside the same steps of the
float64 model oracle (oracle/model.py), as train.py runs them (cross-entropy with padding
targets ignored, AdamW with weight decay 0.01, train.py:245, 313-326).

A single-step gradient test checks the kernels at the model's initialisation only; here
the weights move, so the attention, the scans, the gating and the fused norms run on the
states and weights that the previous steps produced.  The attention runs in its fp32 mode
(``attn_precision="fp32"``: 1e-4 against the exact oracle at one step), no autocast and no
dropout, so the two trajectories can be held to a fixed bar: the loss of every step within
1e-4 relative, and every weight after the last step within 1e-3 of the largest weight of
its tensor.  A wrong gradient anywhere moves the loss by far more within a few steps.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import model as omodel

pytestmark = pytest.mark.gpu


def norm_err(got, want):
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    return float((got - want).abs().max() / want.abs().max().clamp(min=1e-300))


@pytest.mark.parametrize("with_history", [True, False])
def test_adamw_steps_track_the_oracle(with_history):
    from mathbrain.model import SlotTransformerLM
    from mathbrain.synthetic import make_batch
    V, D, n_layers, H, N, B, L, steps = 300, 64, 2, 2, 16, 2, 64, 5
    torch.manual_seed(0)
    m = SlotTransformerLM(V, D, n_layers, H, N=N, dropout=0.0, max_hl=1024.0,
                          attn_precision="fp32").cuda()
    d = make_batch(B, L, V, N, 200, seed=11, max_hl=1024.0)
    x, uniq, cb = d["x"], d["unique"], d["c_base"]
    pm = uniq >= 0
    tgt = torch.full((B, L), -1, dtype=torch.int64)   # next token; the last step has none
    tgt[:, :-1] = x[:, 1:]
    rhos = m.ema_rhos.cpu()

    # the oracle's copy of every trainable tensor (lm_head.weight is embed.weight, tied)
    p = {k: v.detach().cpu().double().clone().requires_grad_() for k, v in m.state_dict().items()
         if k not in ("ema_rhos", "lm_head.weight")}
    named = dict(m.named_parameters())
    assert set(named) == set(p), sorted(set(named) ^ set(p))
    opt = torch.optim.AdamW(m.parameters(), lr=1e-3, weight_decay=0.01)
    opt_o = torch.optim.AdamW(list(p.values()), lr=1e-3, weight_decay=0.01, foreach=False)

    if with_history:
        args = (x.cuda(), uniq.cuda(), None, cb.cuda(), None, pm.cuda())
        okw = dict(unique_slots=uniq, c_base=cb.double(), pad_mask=pm)
    else:
        args = (x.cuda(),)
        okw = {}
    losses = []
    for s in range(steps):
        opt.zero_grad(set_to_none=True)
        loss = F.cross_entropy(m(*args).reshape(-1, V), tgt.cuda().reshape(-1), ignore_index=-1)
        loss.backward()
        opt.step()

        opt_o.zero_grad(set_to_none=True)
        lo = omodel.lm_forward(p, x, n_layers, H, rhos, V, **okw)
        loss_o = F.cross_entropy(lo.reshape(-1, V), tgt.reshape(-1), ignore_index=-1)
        loss_o.backward()
        opt_o.step()

        got, want = float(loss.detach()), float(loss_o.detach())
        losses.append((got, want))
        print(f"step {s}: loss {got:.6f} oracle {want:.6f} rel {abs(got - want) / abs(want):.2e}")
        assert abs(got - want) <= 1e-4 * abs(want), (s, got, want)
    assert losses[-1][1] < losses[0][1]   # the steps do train
    torch.cuda.synchronize()
    werr = {k: norm_err(named[k], v) for k, v in p.items()}
    worst = max(werr, key=werr.get)
    print(f"weights after {steps} steps: worst {worst} {werr[worst]:.2e}")
    assert werr[worst] < 1e-3, (worst, werr[worst])
