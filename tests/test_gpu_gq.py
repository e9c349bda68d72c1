"""The query gating folded into the attention (mb_flash_ema_fwd_gq, GatedQueryFlashEMAFunction):
the forward kernel computes Q = q_proj(LayerNorm(x_q * SiLU((C_seq + 1) W_pe))) itself, the
backward recomputes Q from the LayerNorm output.  Checked against the unfused composition on the same inputs (the gating
kernel, an fp32 q_proj GEMM, the attention kernels reading Q), which the model oracle pins
elsewhere: outputs and every gradient within 1e-4 norm-wise (the in-kernel q_proj takes fp16
hi + lo operand pairs, ~2^-22 relative per product), and SlotTransformerLM with
fold_query_gating=True against the same model with the separate gating kernel and q_proj GEMM."""
import pytest
import torch

from tests.test_gpu_flash import make_case, norm_err

pytestmark = pytest.mark.gpu

TOL = 1e-4
# The attention's own dW_pe term multiplies bf16-rounded dpre operands (in the default mode, as
# the reference does): a 1e-6 change of Q flips single bf16 roundings (2^-9 relative), so that
# gradient compares at the kernel-rounding bar of test_gpu_flash.py.
TOL_W_PE_BF16 = 2e-3


def gq_inputs(c, seed, table=False):
    B, H, L, hd = c["Q"].shape
    D = H * hd
    N = c["rhos"].shape[0]
    g = torch.Generator().manual_seed(seed)
    x_q = torch.randn(B, L, D, generator=g)
    C_seq = torch.rand(B, L, N, generator=g) * 3.0
    W_pe = c["W"] * 0.3
    ln_w = 1.0 + 0.2 * torch.randn(D, generator=g)
    ln_b = 0.1 * torch.randn(D, generator=g)
    W_q = torch.randn(D, D, generator=g) / D ** 0.5
    Ek, Ev = c["E_k"], c["E_v"]
    if table:
        tk = torch.randn(c["V"], D, generator=g) * 0.5
        tv = torch.randn(c["V"], D, generator=g) * 0.5
        Ek, Ev = tk, tv
    return dict(x_q=x_q, C_seq=C_seq, W_pe=W_pe, ln_w=ln_w, ln_b=ln_b, W_q=W_q, E_k=Ek, E_v=Ev)


def run_fused(c, p, use_silu=True, absent_mass=True, precision="bf16", dO=None):
    from mathbrain.triton_flash_ema import GatedQueryFlashEMAFunction
    H = c["Q"].shape[1]
    t = {k: v.cuda().requires_grad_(k not in ("C_seq",)) for k, v in p.items()}
    O = GatedQueryFlashEMAFunction.apply(t["x_q"], t["C_seq"], t["W_pe"], t["ln_w"], t["ln_b"], t["W_q"],
                                         c["x"].cuda(), t["E_k"], t["E_v"], c["rhos"].cuda(), c["V"],
                                         c["unique"].cuda(), c["K"], c["Cb"].cuda(), H, use_silu, c["Br"],
                                         absent_mass, precision, 1e-5)
    grads = {}
    if dO is not None:
        O.backward(dO.cuda())
        grads = {k: v.grad.detach().cpu() for k, v in t.items() if v.grad is not None}
    return O.detach().cpu(), grads


def run_unfused(c, p, use_silu=True, absent_mass=True, precision="bf16", dO=None):
    from mathbrain.triton_flash_ema import FlashEMAFunction
    from mathbrain.triton_fused_gating import GatedQueryFunction
    B, H, L, hd = c["Q"].shape
    t = {k: v.cuda().requires_grad_(k not in ("C_seq",)) for k, v in p.items()}
    x_ln = GatedQueryFunction.apply(t["x_q"], t["C_seq"], t["W_pe"], t["ln_w"], t["ln_b"], use_silu, 1e-5)
    Q = (x_ln @ t["W_q"].t()).view(B, L, H, hd).transpose(1, 2)
    O = FlashEMAFunction.apply(Q, c["x"].cuda(), t["E_k"], t["E_v"], t["W_pe"], c["rhos"].cuda(), c["V"],
                               c["unique"].cuda(), c["K"], c["Cb"].cuda(), use_silu, c["Br"], absent_mass,
                               precision)
    grads = {}
    if dO is not None:
        O.backward(dO.cuda())
        grads = {k: v.grad.detach().cpu() for k, v in t.items() if v.grad is not None}
    return O.detach().cpu(), grads


def check(c, p, seed=0, **kw):
    g = torch.Generator().manual_seed(seed + 9)
    dO = torch.randn(c["Q"].shape, generator=g)
    Of, gf = run_fused(c, p, dO=dO, **kw)
    Ou, gu = run_unfused(c, p, dO=dO, **kw)
    errs = {"O": norm_err(Of, Ou)}
    errs.update({k: norm_err(gf[k], gu[k]) for k in gu})
    assert set(gf) == set(gu), (sorted(gf), sorted(gu))
    msg = ", ".join(f"{k} {v:.2e}" for k, v in errs.items())
    print(msg)
    w_tol = TOL if kw.get("precision") == "fp32" else TOL_W_PE_BF16
    for k, e in errs.items():
        assert e < (w_tol if k == "W_pe" else TOL), msg


def test_gq_cfg_shape_h8_hd64():
    c = make_case(2, 96, 300, 8, 64, 64, warmup=100, seed=1, qs=0.5, es=0.3, ws=0.2)
    check(c, gq_inputs(c, 2))


@pytest.mark.parametrize("H,hd,N", [(1, 64, 16), (3, 32, 16), (12, 64, 16), (4, 32, 128), (16, 64, 33)])
def test_gq_head_groups_and_rates(H, hd, N):
    c = make_case(2, 70, 150, H, hd, N, warmup=60, seed=H + N, qs=0.5, es=0.3, ws=0.2)
    check(c, gq_inputs(c, H), seed=H)


@pytest.mark.parametrize("use_silu", [True, False])
@pytest.mark.parametrize("absent_mass", [True, False])
def test_gq_flags(use_silu, absent_mass):
    c = make_case(2, 45, 90, 4, 32, 16, warmup=50, seed=31, qs=0.5, es=0.3, ws=0.2)
    check(c, gq_inputs(c, 5), seed=3, use_silu=use_silu, absent_mass=absent_mass)


def test_gq_vocab_table_rows():
    c = make_case(2, 80, 70, 4, 64, 32, warmup=100, seed=51, qs=0.5, es=0.3, ws=0.2)
    check(c, gq_inputs(c, 6, table=True), seed=4)


def test_gq_fp32_mode():
    c = make_case(2, 64, 120, 8, 64, 64, warmup=80, seed=61, qs=0.5, es=0.3, ws=0.2)
    check(c, gq_inputs(c, 7), seed=5, precision="fp32")


def test_gq_rejects_wide_model():
    from mathbrain._lib import HipKernelError
    c = make_case(1, 16, 40, 17, 64, 16, warmup=0, seed=2)
    with pytest.raises(HipKernelError, match="d_model 1088"):
        run_fused(c, gq_inputs(c, 8))


@pytest.mark.parametrize("kv_table", [False, True])
def test_model_fold_matches_unfolded(kv_table):
    """SlotTransformerLM with the query gating folded into the attention against the same
    model with the separate gating kernel and q_proj GEMM: logits and every gradient."""
    from mathbrain.model import SlotTransformerLM
    from mathbrain.synthetic import make_batch
    V, D, H, N, B, L = 400, 256, 4, 16, 2, 80
    torch.manual_seed(3)
    m = SlotTransformerLM(V, D, 2, H, N=N, dropout=0.0, max_hl=1024.0).cuda()
    m.kv_table = kv_table
    d = make_batch(B, L, V, N, 150, seed=4, max_hl=1024.0)
    args = (d["x"].cuda(), d["unique"].cuda(), None, d["c_base"].cuda(), None, (d["unique"] >= 0).cuda())
    R = torch.randn(B, L, V, generator=torch.Generator().manual_seed(5)).cuda()
    out = {}
    for fold in (True, False):
        for layer in m.layers:
            layer.attn.fold_query_gating = fold
        m.zero_grad(set_to_none=True)
        logits = m(*args)
        (logits * R).sum().backward()
        out[fold] = (logits.detach().cpu(), {k: p.grad.detach().cpu() for k, p in m.named_parameters()})
    errs = {"logits": norm_err(out[True][0], out[False][0])}
    errs.update({k: norm_err(out[True][1][k], out[False][1][k]) for k in out[False][1]})
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:4]
    print(f"fold vs unfolded: logits {errs['logits']:.2e}; worst {worst}")
    for k, e in errs.items():
        assert e < (TOL_W_PE_BF16 if k.endswith("pe_proj.weight") else TOL), (k, e)
