"""SlotTransformerLM on the HIP path against the model-level CPU oracle (oracle/model.py,
float64, the unique-slot device semantics with the absent-slot mass).

Logits and every parameter gradient are compared norm-wise (max|got - want| / max|want|)
at the task's bf16 bar, 2e-2, against the exact oracle at the model's own initialisation.
Against the oracle with the kernels' own gate rounding (the split gate; in the backward the
single fp16 product for slots whose probability stays below 2^-7) the logits must agree to
1e-4 and the gradients to TOL_ROUNDING_GRAD -- except pe_proj.weight, whose attention part
the kernel contracts from bf16 c_dec and bf16 dpre (as triton_flash_ema.py:463-465 does):
1e-2 there.
"""
import math

import pytest
import torch

from oracle import model as omodel

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
# the oracle rounding of the default attention mode at these models' shapes (head_dim <= 64,
# N <= 64: the split gate, and in the backward, which reads the forward's kept scores, the
# single product for slots whose probability stays below 2^-7; tests.test_gpu_flash.kernel_rounding)
SPLIT = "split_p"
# Gradients against that oracle (pe_proj.weight aside): measured up to 1.3e-4 (LayerNorm and
# RMSNorm weights and biases, whose gradients sum over every row and cancel; the all-split
# oracle gives 1.2e-4 on the same run), so the kernels' per-wave choice of gate product is
# resolved at 3e-4, well under the product of any single-product slot (3.6e-3 with every
# slot on it).
TOL_ROUNDING_GRAD = 3e-4


def norm_err(got, want):
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    return float((got - want).abs().max() / want.abs().max().clamp(min=1e-300))


def build(V=500, D=128, n_layers=2, H=4, N=16, seed=0, **kw):
    from mathbrain.model import SlotTransformerLM
    torch.manual_seed(seed)
    return SlotTransformerLM(V, D, n_layers, H, N=N, dropout=0.0, max_hl=1024.0, **kw)


def batch(B, L, V, N, seed, warmup=200):
    from mathbrain.synthetic import make_batch
    d = make_batch(B, L, V, N, warmup, seed=seed, max_hl=1024.0)
    return d["x"], d["unique"], d["c_base"], d["unique"] >= 0


@pytest.mark.parametrize("with_history", [True, False])
def test_model_forward_backward_vs_oracle(with_history):
    V, D, n_layers, H, N, B, L = 500, 128, 2, 4, 16, 2, 96
    m = build(V, D, n_layers, H, N).cuda()
    x, uniq, cb, pm = batch(B, L, V, N, seed=3)
    g = torch.Generator().manual_seed(4)
    R = torch.randn(B, L, V, generator=g)
    if with_history:
        logits = m(x.cuda(), uniq.cuda(), None, cb.cuda(), None, pm.cuda())
    else:
        logits = m(x.cuda())
    (logits * R.cuda()).sum().backward()
    torch.cuda.synchronize()

    rhos = m.ema_rhos.cpu()
    kw = dict(unique_slots=uniq, c_base=cb.double(), pad_mask=pm) if with_history else {}
    grads = dict(m.named_parameters())
    for gate_round, tol_logits in ((None, TOL_BF16), (SPLIT, 1e-4)):
        p = {k: v.detach().cpu().double().requires_grad_() for k, v in m.state_dict().items()
             if k != "ema_rhos" and k != "lm_head.weight"}
        want = omodel.lm_forward(p, x, n_layers, H, rhos, V, gate_round=gate_round, **kw)
        (want * R.double()).sum().backward()
        err = norm_err(logits, want)
        gerr = {k: norm_err(grads[k].grad, v.grad) for k, v in p.items()}
        worst = max(gerr, key=gerr.get)
        print(f"gate_round={gate_round}: logits {err:.2e}; worst grad {worst} {gerr[worst]:.2e}")
        assert err < tol_logits
        for k, e in gerr.items():
            tol = TOL_BF16 if gate_round is None else (1e-2 if k.endswith("pe_proj.weight") else TOL_ROUNDING_GRAD)
            assert e < tol, (gate_round, k, e)


def test_model_under_bf16_autocast_runs_and_tracks_fp32():
    V, D, n_layers, H, N, B, L = 800, 256, 1, 8, 16, 2, 64
    m = build(V, D, n_layers, H, N, seed=1).cuda()
    x, uniq, cb, pm = batch(B, L, V, N, seed=5)
    args = (x.cuda(), uniq.cuda(), None, cb.cuda(), None, pm.cuda())
    ref = m(*args)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = m(*args)
        out.float().sum().backward()
    assert torch.isfinite(out.float()).all()
    assert norm_err(out.float(), ref) < 5e-2
    for name, t in m.named_parameters():
        assert t.grad is not None and torch.isfinite(t.grad).all(), name


def test_model_few_slots_pads_to_sixteen():
    """Rows with fewer than 16 slots: the slot list is padded to 16 with -1 (the reference's
    K_max floor, model.py:170, which its .view would reject)."""
    V, D, H, N = 30, 128, 4, 16
    m = build(V, D, 1, H, N, seed=2).cuda()
    x = torch.tensor([[1, 2, 1, 3, 2, 1, 4, 5]])
    uniq = torch.tensor([[1, 2, 3, 4, 5, 6]])
    cb = torch.rand(1, 6, N)
    pm = torch.ones(1, 6, dtype=torch.bool)
    out = m(x.cuda(), uniq.cuda(), None, cb.cuda(), None, pm.cuda())
    p = {k: v.detach().cpu().double() for k, v in m.state_dict().items()
         if k != "ema_rhos" and k != "lm_head.weight"}
    want = omodel.lm_forward(p, x, 1, H, m.ema_rhos.cpu(), V, unique_slots=uniq, c_base=cb.double(),
                             pad_mask=pm)
    assert norm_err(out, want) < TOL_BF16


@pytest.mark.parametrize("kv_table", [None, True, False])
def test_model_vocab_table_path_vs_oracle(kv_table):
    """A vocabulary smaller than B * K_max: the layers project the embedding table and the
    attention reads slot rows by token id (kv_table None picks it here); forced either way
    the logits and every gradient match the float64 oracle with the kernel's gate rounding."""
    V, D, n_layers, H, N, B, L = 60, 128, 2, 4, 16, 3, 96
    m = build(V, D, n_layers, H, N, seed=6).cuda()
    m.kv_table = kv_table
    x, uniq, cb, pm = batch(B, L, V, N, seed=7)
    assert B * max(uniq.shape[1], 16) > V
    g = torch.Generator().manual_seed(8)
    R = torch.randn(B, L, V, generator=g)
    logits = m(x.cuda(), uniq.cuda(), None, cb.cuda(), None, pm.cuda())
    (logits * R.cuda()).sum().backward()
    torch.cuda.synchronize()
    p = {k: v.detach().cpu().double().requires_grad_() for k, v in m.state_dict().items()
         if k != "ema_rhos" and k != "lm_head.weight"}
    want = omodel.lm_forward(p, x, n_layers, H, m.ema_rhos.cpu(), V, gate_round=SPLIT,
                             unique_slots=uniq, c_base=cb.double(), pad_mask=pm)
    (want * R.double()).sum().backward()
    assert norm_err(logits, want) < 1e-4
    grads = dict(m.named_parameters())
    for k, v in p.items():
        tol = 1e-2 if k.endswith("pe_proj.weight") else TOL_ROUNDING_GRAD
        assert norm_err(grads[k].grad, v.grad) < tol, (kv_table, k)


@pytest.mark.parametrize("absent_mass", [True, False])
def test_model_absent_mass_switch_vs_oracle(absent_mass):
    """SlotTransformerLM(absent_mass=...) threads the softmax choice into every layer's
    attention: all V slots (the dense reference) or the valid slots only (the reference's
    Triton kernel); logits and gradients match the oracle under each, and the two differ."""
    V, D, n_layers, H, N, B, L = 400, 128, 2, 4, 16, 2, 64
    torch.manual_seed(11)
    from mathbrain.model import SlotTransformerLM
    m = SlotTransformerLM(V, D, n_layers, H, N=N, dropout=0.0, max_hl=1024.0,
                          absent_mass=absent_mass).cuda()
    x, uniq, cb, pm = batch(B, L, V, N, seed=12)
    g = torch.Generator().manual_seed(13)
    R = torch.randn(B, L, V, generator=g)
    logits = m(x.cuda(), uniq.cuda(), None, cb.cuda(), None, pm.cuda())
    (logits * R.cuda()).sum().backward()
    p = {k: v.detach().cpu().double().requires_grad_() for k, v in m.state_dict().items()
         if k != "ema_rhos" and k != "lm_head.weight"}
    kw = dict(unique_slots=uniq, c_base=cb.double(), pad_mask=pm)
    # every step evaluated through the closed-form backward, which takes the dW_pe product
    # from bf16 operands as the kernel does (without the absent mass p is ~V/K_b times
    # larger, so that rounding shows in pe_proj.weight's gradient)
    want = omodel.lm_forward(p, x, n_layers, H, m.ema_rhos.cpu(), V, gate_round=SPLIT,
                             absent_mass=absent_mass, t_eval=list(range(L)), **kw)
    (want * R.double()).sum().backward()
    assert norm_err(logits, want) < 1e-4
    grads = dict(m.named_parameters())
    for k, v in p.items():
        tol = 1e-2 if k.endswith("pe_proj.weight") else TOL_ROUNDING_GRAD
        assert norm_err(grads[k].grad, v.grad) < tol, (absent_mass, k)
    other = omodel.lm_forward({k: v.detach() for k, v in p.items()}, x, n_layers, H,
                              m.ema_rhos.cpu(), V, gate_round=SPLIT, absent_mass=not absent_mass, **kw)
    assert norm_err(other, want) > 1e-2


def test_model_collated_batch_with_token_zero_history():
    """A batch from the data pipeline (slot lists padded with id 0, as the reference's
    collate pads them) whose chunks carry token 0 in their history: the query side and the
    key side both keep token 0's carried c_base (the padding is masked to -1 before the
    query scan), and logits match the oracle with the same masking."""
    import numpy as np
    from mathbrain.data import WikiTextMMapDataset, preprocess_corpus
    import tempfile
    rng = np.random.default_rng(21)
    V = 50
    docs = []
    for _ in range(8):
        n = int(rng.integers(200, 320))
        d = rng.integers(1, V, n)
        d[rng.integers(0, 100, 6)] = 0             # token 0 in the history ...
        d[rng.integers(128, n, 6)] = 0             # ... and again inside later chunks
        docs.append(d.tolist())
    tmp = tempfile.mkdtemp(prefix="mb_h4_")
    preprocess_corpus(docs, tmp, N=16, min_hl=1.0, max_hl=1024.0)
    from mathbrain.synthetic import rhos_from_half_lives
    ds = WikiTextMMapDataset(tmp, 64, rhos_from_half_lives(16, 1.0, 1024.0))
    late = [i for i in range(len(ds)) if ds._cs[i] - ds._cds[i] >= 128][:6]
    chunks, us, pm, inv, cb, K, doc = ds.get_batch(late)
    pmc = pm.bool().cpu()
    usc = us.cpu()
    xc = chunks.cpu()
    inside = doc.cpu() != -1                       # chunk positions (the collate pads with 0)
    hit = [bool(((xc[b] == 0) & inside[b]).any() and not pmc[b].all()) for b in range(usc.shape[0])]
    assert any(hit), "a padded row must hold token 0 in its chunk and history"
    torch.manual_seed(22)
    from mathbrain.model import SlotTransformerLM
    m = SlotTransformerLM(V, 128, 1, 4, N=16, dropout=0.0, max_hl=1024.0).cuda()
    x = chunks[:, :-1]
    logits = m(x, unique_slots=us, inverse_indices=inv[:, :-1], c_base=cb, doc_ids=doc[:, :-1],
               pad_mask=pm)
    p = {k: v.detach().cpu().double() for k, v in m.state_dict().items()
         if k != "ema_rhos" and k != "lm_head.weight"}
    want = omodel.lm_forward(p, x.cpu(), 1, 4, m.ema_rhos.cpu(), V, unique_slots=usc,
                             c_base=cb.cpu().double(), pad_mask=pmc, gate_round=SPLIT)
    assert norm_err(logits, want) < 1e-4
    stale = omodel.lm_forward(p, x.cpu(), 1, 4, m.ema_rhos.cpu(), V, unique_slots=usc,
                              c_base=cb.cpu().double(), pad_mask=pmc, gate_round=SPLIT,
                              mask_query_keys=False)
    moved = norm_err(stale, want)
    print(f"0-padded query keys would move the logits by {moved:.2e}")
    assert moved > 1e-7


def test_model_traces_without_graph_breaks():
    """torch._dynamo sees every HIP entry point as a registered op (mathbrain::*), so the
    model's forward traces into one graph and a compiled step matches eager."""
    import torch._dynamo
    V, D, H, N, B, L = 300, 128, 4, 16, 2, 48
    m = build(V, D, 2, H, N, seed=31).cuda()
    x, uniq, cb, pm = batch(B, L, V, N, seed=32)
    args = (x.cuda(), uniq.cuda(), None, cb.cuda(), None, pm.cuda())
    torch._dynamo.reset()
    ex = torch._dynamo.explain(m)(*args)
    reasons = [str(r.reason)[:300] for r in ex.break_reasons]
    print(f"graphs {ex.graph_count}, breaks {ex.graph_break_count}: {reasons}")
    assert ex.graph_break_count == 0, reasons
    ops = {str(n.target) for g in ex.graphs for n in g.graph.nodes if n.op == "call_function"}
    assert any("mathbrain" in o for o in ops), ops
    ref = m(*args)
    (ref.float() ** 2).mean().backward()
    gref = {k: p.grad.clone() for k, p in m.named_parameters()}
    m.zero_grad()
    cm = torch.compile(m, backend="eager")
    out = cm(*args)
    (out.float() ** 2).mean().backward()
    assert norm_err(out, ref) < 1e-6
    # the traced graph recomputes the scores in the backward, which then takes the split gate
    # for every slot; eager keeps them and takes the single product where p < 2^-7
    for k, p in m.named_parameters():
        assert norm_err(p.grad, gref[k]) < 1e-4, k
