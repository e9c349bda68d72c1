"""The forward's slot split (mb_flash_ema_fwd with a workspace): each workgroup's slot batches
run as ks parts whose partial softmax states flash_fwd_merge_kernel combines.  Checked through
the C ABI against the same launch without a workspace (unsplit) on the same inputs: O and LSE
agree to fp32 rounding of the reordered sums (1e-5 norm-wise; the unsplit path is pinned
against the oracle by test_gpu_flash.py), including rows whose parts hold no slot, padding
slots, both softmax modes, vocabulary rows, in all three precision modes.  Also the
planner: the configuration-2 shape splits in two on a 256-CU device, configuration 4's does
not."""
import pytest
import torch

from tests.test_gpu_flash import make_case, norm_err

pytestmark = pytest.mark.gpu

TOL = 1e-5


def run(c, ws_mode, use_silu=True, absent_mass=True, table=False, prec="fp16", scores=False):
    """mb_flash_ema_fwd on the case; ws_mode None (no workspace), "exact" (the planned bytes)
    or "short" (one byte less: the launch must then run unsplit)."""
    from mathbrain import _lib
    from mathbrain.triton_flash_ema import _flash_flags, _prec
    dev = torch.device("cuda", 0)
    B, H, L, hd = c["Q"].shape
    K, N = c["K"], c["rhos"].shape[0]
    D = H * hd
    Q = c["Q"].to(dev).contiguous()
    x = c["x"].to(dev)
    if table:   # vocabulary rows: the slots' rows scattered into a [V, D] table
        Ek = torch.zeros(c["V"], D)
        Ev = torch.zeros(c["V"], D)
        u = c["unique"]
        for b in range(B):
            ok = u[b] >= 0
            Ek[u[b][ok]] = c["E_k"][b][ok]
            Ev[u[b][ok]] = c["E_v"][b][ok]
        Ek, Ev = Ek.to(dev), Ev.to(dev)
    else:
        Ek, Ev = c["E_k"].to(dev).contiguous(), c["E_v"].to(dev).contiguous()
    W = c["W"].to(dev).contiguous()
    rh = c["rhos"].to(dev).float().contiguous()
    uniq = c["unique"].to(dev)
    Cb = c["Cb"].to(dev).float().contiguous()
    flags = _flash_flags(use_silu, absent_mass, table, _prec(prec))
    need = _lib.lib().mb_flash_ema_fwd_workspace(B, H, L, hd, K, N, flags)
    assert need >= 0
    ws, nws = None, 0
    if ws_mode is not None and need > 0:
        nws = need if ws_mode == "exact" else need - 1
        ws = torch.full((need,), 255, dtype=torch.uint8, device=dev)   # stale contents
    O = torch.full((B, H, L, hd), float("nan"), device=dev)
    LSE = torch.full((B, H, L), float("nan"), device=dev)
    S2 = torch.full((B, H, K, L), float("nan"), device=dev) if scores else None
    _lib.call("mb_flash_ema_fwd", _lib.ptr(Q), *Q.stride(), _lib.ptr(x), x.stride(0), x.stride(1),
              _lib.ptr(Ek), _lib.ptr(Ev), _lib.ptr(W), _lib.ptr(rh), _lib.ptr(uniq), _lib.ptr(Cb),
              B, H, L, hd, K, N, Cb.shape[3], Cb.shape[1], c["Br"], c["V"], flags, _lib.ptr(O),
              _lib.ptr(LSE), _lib.ptr(S2), _lib.ptr(ws), nws, _lib.stream(dev))
    torch.cuda.synchronize()
    return need, O.cpu(), LSE.cpu(), (S2.cpu() if scores else None)


def compare(c, tol=TOL, **kw):
    need, Os, Ls, Ss = run(c, "exact", **kw)
    assert need > 0, "the planner should split this small grid"
    _, Ou, Lu, Su = run(c, None, **kw)
    assert torch.isfinite(Os).all() and torch.isfinite(Ou).all()
    eo, el = norm_err(Os, Ou), norm_err(Ls, Lu)
    print(f"workspace {need} B: O {eo:.2e}, LSE {el:.2e}")
    assert eo < tol and el < tol
    if Ss is not None:   # the scores do not depend on the split: bit-identical
        valid = (c["unique"] >= 0)[:, None, :, None].expand_as(Ss)
        assert torch.equal(Ss[valid], Su[valid])


def test_split_matches_unsplit_cfg_like():
    c = make_case(2, 96, 300, 8, 64, 64, warmup=100, seed=1, qs=0.5, es=0.3, ws=0.2)
    compare(c)


def test_split_default_mode():
    """The default mode (the split gate in the forward) and its scores."""
    c = make_case(2, 70, 200, 4, 32, 16, warmup=60, seed=7, qs=0.5, es=0.3, ws=0.2)
    compare(c, prec="bf16", scores=True)
    c = make_case(2, 96, 300, 8, 64, 64, warmup=100, seed=1, qs=0.5, es=0.3, ws=0.2)
    compare(c, prec="bf16", scores=True)


@pytest.mark.parametrize("use_silu", [True, False])
@pytest.mark.parametrize("absent_mass", [True, False])
def test_split_softmax_modes(use_silu, absent_mass):
    c = make_case(2, 70, 200, 4, 32, 16, warmup=60, seed=7, qs=0.5, es=0.3, ws=0.2)
    compare(c, use_silu=use_silu, absent_mass=absent_mass)


def test_split_with_padding_slots_and_scores():
    c = make_case(2, 80, 150, 4, 64, 32, warmup=50, seed=11, qs=0.5, es=0.3, ws=0.2, pad_slots=37)
    compare(c, scores=True)


def test_split_vocab_rows():
    c = make_case(2, 64, 120, 8, 64, 64, warmup=80, seed=13, qs=0.5, es=0.3, ws=0.2)
    compare(c, table=True)


def test_split_fp32_mode():
    c = make_case(2, 64, 160, 8, 64, 64, warmup=80, seed=17, qs=0.5, es=0.3, ws=0.2)
    compare(c, prec="fp32", scores=True)


def test_split_empty_parts():
    # one sequence with a single valid slot among padding: most parts see no batch
    c = make_case(2, 60, 250, 4, 64, 16, warmup=40, seed=19, qs=0.5, es=0.3, ws=0.2)
    c["unique"][1, 1:] = -1
    compare(c, absent_mass=False)
    compare(c, absent_mass=True)


def test_short_workspace_runs_unsplit():
    c = make_case(2, 64, 150, 8, 64, 64, warmup=40, seed=23, qs=0.5, es=0.3, ws=0.2)
    need, Os, Ls, _ = run(c, "short", prec="bf16")
    _, Ou, Lu, _ = run(c, None, prec="bf16")
    assert need > 0
    assert torch.equal(Os, Ou) and torch.equal(Ls, Lu)


def test_planner_shapes():
    from mathbrain import _lib
    from mathbrain.triton_flash_ema import _flash_flags
    torch.cuda.init()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    f = _flash_flags(True, True, False, False)
    cfg2 = _lib.lib().mb_flash_ema_fwd_workspace(56, 8, 512, 64, 1638, 64, f)
    cfg4 = _lib.lib().mb_flash_ema_fwd_workspace(16, 8, 4096, 64, 6000, 128, f)
    print("CUs", cus, "cfg2 workspace", cfg2, "cfg4 workspace", cfg4)
    if cus == 256:
        assert cfg2 == 2 * 56 * 8 * 512 * (64 + 2) * 4
        assert cfg4 == 0
    assert _lib.lib().mb_flash_ema_fwd_workspace(1, 8, 64, 48, 10, 16, f) == -1   # head_dim 48
