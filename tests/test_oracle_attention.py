"""Pins the CPU oracle of flash-EMA attention (oracle/attention.py).

The reference has no test of attention values (its tests pin only the scans), so the
oracle is pinned by what the mathematics fixes:
  * the dense restatement of flash_ema_attention.flash_ema_forward equals the unique-slot
    form plus the (V - K_b) absent-slot mass, exactly (absent slots have zero counters,
    hence gate SiLU(0) = 0, score 0 and value 0);
  * with no decay and no occurrences the gate is constant in time, and the attention is
    torch's scaled_dot_product_attention on gated keys/values;
  * all-zero counters give a uniform softmax and a zero output;
  * a one-slot case evaluated by hand with the math module;
  * float64 gradcheck of the oracle, and autograd == the reference's closed-form
    gradients (mathbrain/triton_flash_ema.py:336-350, 446-465).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as att


def _problem(seed, B=2, L=10, V=24, H=2, hd=4, N=3, extra=3, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randint(0, V // 2, (B, L), generator=g)
    E_k_slots = torch.randn(V, H * hd, generator=g, dtype=dtype) * 0.5
    E_v_slots = torch.randn(V, H * hd, generator=g, dtype=dtype) * 0.5
    pe_weight = torch.randn(H * hd, N, generator=g, dtype=dtype) * 0.7
    rhos = torch.tensor([0.5, 0.9, 0.99][:N], dtype=dtype)
    Q = torch.randn(B, L, H * hd, generator=g, dtype=dtype)
    slots = []
    for b in range(B):
        s = torch.unique(x[b])
        hist = torch.arange(V // 2, V // 2 + extra)  # history-only slots
        slots.append(torch.cat([s, hist]))
    K = max(s.numel() for s in slots) + 2
    unique = torch.full((B, K), -1, dtype=torch.int64)
    c_init = torch.zeros(B, K, N, dtype=dtype)
    for b, s in enumerate(slots):
        unique[b, :s.numel()] = s
        c_init[b, :s.numel()] = torch.rand(s.numel(), N, generator=g, dtype=dtype) * 3
    E_k = E_k_slots[unique.clamp(min=0)]
    E_v = E_v_slots[unique.clamp(min=0)]
    return dict(x=x, E_k_slots=E_k_slots, E_v_slots=E_v_slots, pe_weight=pe_weight, rhos=rhos,
                Q=Q, unique=unique, c_init=c_init, E_k=E_k, E_v=E_v, V=V, H=H, hd=hd)


def _sparse(p, **kw):
    B, L, D = p["Q"].shape
    Qh = p["Q"].reshape(B, L, p["H"], p["hd"]).transpose(1, 2)
    return att.sparse(Qh, p["x"], p["E_k"], p["E_v"], p["pe_weight"].t(), p["rhos"], p["V"],
                      p["unique"], p["c_init"], **kw)


def _to_bld(O):
    B, H, L, hd = O.shape
    return O.transpose(1, 2).reshape(B, L, H * hd)


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("use_silu", [True, False])
def test_dense_equals_sparse_plus_absent_mass(seed, use_silu):
    p = _problem(seed)
    cg = att.scatter_c_global(p["unique"], p["c_init"], p["V"])
    dense = att.dense(p["Q"], p["x"], p["E_k_slots"], p["E_v_slots"], p["rhos"], p["pe_weight"],
                      p["H"], use_silu=use_silu, c_global=cg)
    sparse = _to_bld(_sparse(p, use_silu=use_silu))
    assert torch.allclose(dense, sparse, rtol=1e-12, atol=1e-14)
    # dropping the absent mass (the Triton kernel as executed) is a different function
    triton_like = _to_bld(_sparse(p, use_silu=use_silu, absent_mass=False))
    assert not torch.allclose(dense, triton_like, rtol=1e-3)


def test_dense_from_zero_state_is_the_reference_as_written():
    # flash_ema_attention.py:36 starts from C_global = 0; c_global=None must do the same
    p = _problem(4)
    a = att.dense(p["Q"], p["x"], p["E_k_slots"], p["E_v_slots"], p["rhos"], p["pe_weight"], p["H"])
    b = att.dense(p["Q"], p["x"], p["E_k_slots"], p["E_v_slots"], p["rhos"], p["pe_weight"], p["H"],
                  c_global=torch.zeros(2, p["V"], 3, dtype=torch.float64))
    assert torch.equal(a, b)


def test_no_absent_slots_when_all_tokens_are_slots():
    p = _problem(5)
    p["V"] = int(p["unique"].max()) + 1
    # every id < V is a slot of row 0? not necessarily; use a row whose slots cover 0..V-1
    V = p["V"]
    B, K = p["unique"].shape
    allslots = torch.arange(V)
    p["unique"] = torch.cat([allslots.expand(B, V), torch.full((B, 1), -1)], 1)
    g = torch.Generator().manual_seed(7)
    p["c_init"] = torch.rand(B, V + 1, 3, generator=g, dtype=torch.float64)
    p["c_init"][:, -1] = 0
    p["E_k"] = p["E_k_slots"][p["unique"].clamp(min=0)]
    p["E_v"] = p["E_v_slots"][p["unique"].clamp(min=0)]
    a = _sparse(p, absent_mass=True)
    b = _sparse(p, absent_mass=False)
    assert torch.allclose(a, b, rtol=1e-13)


@pytest.mark.parametrize("absent", [True, False])
def test_constant_gate_reduces_to_sdpa(absent):
    # rho = 1 and no slot token ever occurs in x: c_dec = c0 for all t, so the gate is
    # constant in time and the attention is plain softmax attention on gated keys/values.
    p = _problem(6, N=1)
    p["rhos"] = torch.ones(1, dtype=torch.float64)
    p["x"] = torch.full_like(p["x"], p["V"] + 5)  # never a slot
    B, L, D = p["Q"].shape
    H, hd = p["H"], p["hd"]
    O = _sparse(p, absent_mass=absent)
    valid = p["unique"] >= 0
    for b in range(B):
        k = int(valid[b].sum())
        g = F.silu(p["c_init"][b, :k] @ p["pe_weight"].t())           # [k, D]
        Kg = (p["E_k"][b, :k] * g).reshape(k, H, hd).transpose(0, 1)  # [H, k, hd]
        Vg = (p["E_v"][b, :k] * g).reshape(k, H, hd).transpose(0, 1)
        if absent:
            n_abs = p["V"] - k
            Kg = torch.cat([Kg, torch.zeros(H, n_abs, hd, dtype=Kg.dtype)], 1)
            Vg = torch.cat([Vg, torch.zeros(H, n_abs, hd, dtype=Vg.dtype)], 1)
        q = p["Q"][b].reshape(L, H, hd).transpose(0, 1)
        want = F.scaled_dot_product_attention(q, Kg, Vg)                # [H, L, hd]
        assert torch.allclose(O[b], want, rtol=1e-10, atol=1e-12)


def test_zero_counters_give_uniform_softmax_and_zero_output():
    p = _problem(8)
    p["c_init"].zero_()
    p["x"] = torch.full_like(p["x"], p["V"] + 1)
    O, LSE = _sparse(p, return_lse=True)
    assert torch.count_nonzero(O) == 0
    assert torch.allclose(LSE, torch.full_like(LSE, math.log(p["V"])))
    O2, LSE2 = _sparse(p, absent_mass=False, return_lse=True)
    kb = (p["unique"] >= 0).sum(1).to(torch.float64)
    assert torch.allclose(LSE2, torch.log(kb).reshape(-1, 1, 1).expand_as(LSE2))


def test_one_slot_by_hand():
    # B=H=hd=N=1, V=2 (one absent slot), slot u=5 with c0=1, rho=0.5, W=2, e_k=3, e_v=4,
    # x = [5, 7], q = [1, 2]
    def silu(z):
        return z / (1.0 + math.exp(-z))
    want = []
    c = 1.0
    for t, (xt, q) in enumerate([(5, 1.0), (7, 2.0)]):
        c_dec = c * 0.5
        g = silu(2.0 * c_dec)
        s = q * 3.0 * g
        p = math.exp(s) / (math.exp(s) + 1.0)
        want.append(p * 4.0 * g)
        c = c_dec + (1.0 if xt == 5 else 0.0)
    dt = torch.float64
    O = att.sparse(torch.tensor([1.0, 2.0], dtype=dt).reshape(1, 1, 2, 1), torch.tensor([[5, 7]]),
                   torch.tensor([[[3.0]]], dtype=dt), torch.tensor([[[4.0]]], dtype=dt),
                   torch.tensor([[2.0]], dtype=dt), torch.tensor([0.5], dtype=dt), 2,
                   torch.tensor([[5]]), torch.tensor([[[1.0]]], dtype=dt))
    assert torch.allclose(O.flatten(), torch.tensor(want, dtype=dt), rtol=1e-14)


def test_gate_rounding_modes_stay_close():
    p = _problem(9, dtype=torch.float64)
    exact = _sparse(p)
    errs = {}
    for mode in ("bf16", "f16", "f16c", "f16w", "split"):
        r = _sparse(p, gate_round=mode)
        errs[mode] = float((r - exact).abs().max() / exact.abs().max())
    # the split gate's forward is the exact one; each fp16 rounding moves the output, by less
    # than bf16's (3 more significand bits; measured 3.3x on this small problem), and rounding
    # both operands by more than rounding either alone
    assert errs["split"] == 0.0, errs
    assert 0.0 < errs["f16"] < errs["bf16"] / 2 < 2e-2, errs
    assert 0.0 < errs["f16c"] < 1.5 * errs["f16"] and 0.0 < errs["f16w"] < 1.5 * errs["f16"], errs


def test_gate_rounding_helpers_are_the_formats_roundings():
    """Each rounded operand is the nearest value of its format (torch's conversions), with W
    rounded after the kernels' log2 e pre-scaling."""
    g = torch.Generator().manual_seed(4)
    W = torch.randn(8, 16, generator=g, dtype=torch.float64) * 0.3
    c = torch.rand(5, 8, generator=g, dtype=torch.float64) * 900
    l2e = 1.0 / math.log(2.0)
    for mode in (None, "split", "f16c"):
        assert torch.equal(att._round_gate_operands(W, mode), W)
    for mode in (None, "split", "f16w"):
        assert torch.equal(att._round_gate_counter(c, mode), c)
    Wf = att._round_gate_operands(W, "f16") * l2e
    assert torch.allclose(Wf, Wf.to(torch.float16).double(), rtol=1e-12, atol=0)  # on the fp16 grid
    assert ((Wf - W * l2e).abs() <= (W * l2e).abs() * 2.0 ** -11 * (1 + 1e-9)).all()
    assert torch.equal(att._round_gate_operands(W, "bf16"), W.to(torch.bfloat16).double())
    assert torch.equal(att._round_gate_counter(c, "f16"), c.float().half().double())
    assert torch.equal(att._round_gate_counter(c, "bf16"), c.float().bfloat16().double())
    with pytest.raises(ValueError):
        att._round_gate_operands(W, "fp8")


@pytest.mark.parametrize("use_silu", [True, False])
@pytest.mark.parametrize("absent", [True, False])
def test_oracle_gradcheck(use_silu, absent):
    p = _problem(10, B=1, L=5, V=12, H=2, hd=2, N=2, extra=1)
    B, L, D = p["Q"].shape
    Qh = p["Q"].reshape(B, L, 2, 2).transpose(1, 2).contiguous().requires_grad_()
    Ek = p["E_k"].clone().requires_grad_()
    Ev = p["E_v"].clone().requires_grad_()
    W = p["pe_weight"].t().contiguous().requires_grad_()

    def f(q, ek, ev, w):
        return att.sparse(q, p["x"], ek, ev, w, p["rhos"], p["V"], p["unique"], p["c_init"],
                          use_silu=use_silu, absent_mass=absent)
    assert torch.autograd.gradcheck(f, (Qh, Ek, Ev, W), eps=1e-6, atol=1e-8, rtol=1e-6)


@pytest.mark.parametrize("seed", [0, 3])
@pytest.mark.parametrize("absent", [True, False])
def test_autograd_equals_reference_gradient_formulas(seed, absent):
    p = _problem(seed)
    B, L, D = p["Q"].shape
    H, hd = p["H"], p["hd"]
    Qh = p["Q"].reshape(B, L, H, hd).transpose(1, 2).contiguous().requires_grad_()
    Ek = p["E_k"].clone().requires_grad_()
    Ev = p["E_v"].clone().requires_grad_()
    W = p["pe_weight"].t().contiguous().requires_grad_()
    O = att.sparse(Qh, p["x"], Ek, Ev, W, p["rhos"], p["V"], p["unique"], p["c_init"],
                   absent_mass=absent)
    dO = torch.randn(O.shape, generator=torch.Generator().manual_seed(seed + 100), dtype=O.dtype)
    O.backward(dO)
    dQ, dEk, dEv, dW = att.sparse_backward_formulas(
        Qh.detach(), p["x"], p["E_k"], p["E_v"], W.detach(), p["rhos"], p["V"], p["unique"], dO,
        p["c_init"], absent_mass=absent)
    for got, want in ((Qh.grad, dQ), (Ek.grad, dEk), (Ev.grad, dEv), (W.grad, dW)):
        assert torch.allclose(got, want, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("seed", [1, 4])
def test_sampled_steps_equal_full_evaluation(seed):
    """t_eval only skips the evaluation at unlisted steps, not the state update there:
    forward rows and (with dO zero off the listed steps) every gradient equal the full
    loop's."""
    p = _problem(seed)
    B, L, D = p["Q"].shape
    H, hd = p["H"], p["hd"]
    Qh = p["Q"].reshape(B, L, H, hd).transpose(1, 2).contiguous()
    W = p["pe_weight"].t().contiguous()
    steps = [0, 3, L // 2, L - 1]
    args = (Qh, p["x"], p["E_k"], p["E_v"], W, p["rhos"], p["V"], p["unique"])
    O, LSE = att.sparse(*args, p["c_init"], return_lse=True)
    Os, LSEs = att.sparse(*args, p["c_init"], return_lse=True, t_eval=steps)
    assert torch.allclose(Os, O[:, :, steps], rtol=1e-13, atol=1e-15)
    assert torch.allclose(LSEs, LSE[:, :, steps], rtol=1e-13, atol=1e-15)
    dO = torch.zeros_like(O)
    dO[:, :, steps] = torch.randn(B, H, len(steps), hd, dtype=O.dtype,
                                  generator=torch.Generator().manual_seed(seed))
    full = att.sparse_backward_formulas(*args, dO, p["c_init"])
    sampled = att.sparse_backward_formulas(*args, dO, p["c_init"], t_eval=steps)
    for got, want in zip(sampled, full):
        assert torch.allclose(got, want, rtol=1e-12, atol=1e-15)


def _bwd(p, gate_round, seed=11):
    B, L, D = p["Q"].shape
    Qh = p["Q"].reshape(B, L, p["H"], p["hd"]).transpose(1, 2)
    g = torch.Generator().manual_seed(seed)
    dO = torch.randn(Qh.shape, generator=g, dtype=Qh.dtype)
    return att.sparse_backward_formulas(Qh, p["x"], p["E_k"], p["E_v"], p["pe_weight"].t(), p["rhos"],
                                        p["V"], p["unique"], dO, p["c_init"], gate_round=gate_round)


def test_split_p_takes_the_split_or_the_single_product_by_probability(monkeypatch):
    """"split_p" (the default kernels' backward with stored scores): its forward is the exact
    one; with a threshold of 0 its backward is "split"'s exactly; with every probability below
    the threshold the backward's gate takes the single fp16 product, which moves the gradients
    by about what "f16" moves them (not at all in dW_pe's counter operand); a threshold
    between the two gives a result between them."""
    p = _problem(12, L=40)
    assert torch.equal(_sparse(p, gate_round="split_p"), _sparse(p))
    split, f16 = _bwd(p, "split"), _bwd(p, "f16")
    dist = lambda a, b: float((a - b).abs().max() / b.abs().max())
    monkeypatch.setattr(att, "SPLIT_P", 0.0)
    for a, b in zip(_bwd(p, "split_p"), split):
        assert torch.equal(a, b)
    monkeypatch.setattr(att, "SPLIT_P", 2.0)
    lo = _bwd(p, "split_p")
    for k in range(3):
        d_lo, d_f16 = dist(lo[k], split[k]), dist(f16[k], split[k])
        assert 0.0 < d_lo < 3 * d_f16 and d_lo > d_f16 / 30, (k, d_lo, d_f16)
    _, _, P = _sparse(p, return_lse=True, return_probs=True)
    monkeypatch.setattr(att, "SPLIT_P", float(P[p["unique"] >= 0].median()))
    mid = _bwd(p, "split_p")
    assert 0.0 < dist(mid[0], split[0]) and 0.0 < dist(mid[0], lo[0])


def test_single_gate_halves_groups_16_steps():
    P = torch.zeros(1, 2, 1, 40, dtype=torch.float64)
    P[0, 0, 0, 17] = att.SPLIT_P          # at the threshold: the half [16, 32) splits
    P[0, 1, 0, 39] = att.SPLIT_P * 0.999  # below it everywhere: all single
    single = att.single_gate_halves(P)
    assert single.shape == (1, 2, 1, 3)
    assert single[0, 0, 0].tolist() == [True, False, True]
    assert single[0, 1, 0].tolist() == [True, True, True]


def test_return_probs_are_the_softmax_weights():
    p = _problem(13, L=12)
    O, LSE, P = _sparse(p, return_lse=True, return_probs=True)
    valid = (p["unique"] >= 0)
    # weights of the valid slots plus the absent mass sum to one at every (b, h, t)
    V, Kb = p["V"], valid.sum(1).to(torch.float64)
    absent = ((V - Kb).clamp(min=0).reshape(-1, 1, 1) * torch.exp(-LSE))  # score 0 each
    total = P.sum(1) + absent
    assert torch.allclose(total, torch.ones_like(total), rtol=1e-12)
    assert torch.count_nonzero(P[~valid]) == 0


def _cfg_rates(N=64, lo=1.0, hi=4096.0):
    """Rates of half-lives log-spaced from lo to hi, as SlotTransformerLM sets them."""
    hl = torch.logspace(math.log10(lo), math.log10(hi), N, dtype=torch.float64)
    return torch.exp(math.log(0.5) / hl).to(torch.float32)


def test_corrected_rates_rule():
    """The default forward's tile rule: with the model's rates (half-lives 1..4096) the first
    32-rate tile's largest bound B = 1/(1 - rho) is ~87 against ~5900 and is left to the
    single product; the comparison is 32 B_0 >= max B (at equality the tile is corrected);
    one tile, more than two, or the large rates first: every rate corrected."""
    r = _cfg_rates()
    B = 1.0 / (1.0 - r.double())
    assert 80 < float(B[:32].max()) < 95 and 5800 < float(B[32:].max()) < 6000
    m = att.corrected_rates(r)
    assert m.tolist() == [False] * 32 + [True] * 32
    assert att.corrected_rates(r.flip(0)).all()                  # large rates in tile 0
    assert att.corrected_rates(_cfg_rates(32)).all()              # one tile
    assert att.corrected_rates(_cfg_rates(96)).all()              # beyond the split's N
    assert att.corrected_rates(torch.full((64,), 0.9)).all()
    # B = 2^k exactly: 32 * 8 = 256 corrects tile 0, 512 does not
    eq = torch.tensor([1 - 2.0**-3] * 32 + [1 - 2.0**-8] * 32, dtype=torch.float32)
    assert att.corrected_rates(eq).all()
    gt = torch.tensor([1 - 2.0**-3] * 32 + [1 - 2.0**-9] * 32, dtype=torch.float32)
    assert att.corrected_rates(gt).tolist() == [False] * 32 + [True] * 32


def _problem64(seed, zero_tile=None, L=12):
    """_problem with N = 64 model rates; zero_tile t zeroes W_pe's rows of rate tile t."""
    p = _problem(seed, L=L)
    g = torch.Generator().manual_seed(seed + 100)
    D = p["pe_weight"].shape[0]
    p["rhos"] = _cfg_rates().double()
    p["pe_weight"] = torch.randn(D, 64, generator=g, dtype=torch.float64) * 0.05
    if zero_tile is not None:
        p["pe_weight"][:, 32 * zero_tile: 32 * zero_tile + 32] = 0.0
    K = p["unique"].shape[1]
    p["c_init"] = torch.rand(p["unique"].shape[0], K, 64, generator=g, dtype=torch.float64) / (1 - p["rhos"])
    p["c_init"] *= (p["unique"] >= 0).unsqueeze(-1)
    return p


def test_split_t_forward_rounds_only_the_uncorrected_tile():
    """"split_t" / "split_p" forward: the corrected tile's products exact, the other tile's
    the single fp16 product: with the uncorrected tile's W rows zero it is the exact forward,
    with the corrected tile's zero it is "f16"'s, and in general it sits between them."""
    p = _problem64(20, zero_tile=0)
    assert torch.equal(_sparse(p, gate_round="split_t"), _sparse(p))
    assert torch.equal(_sparse(p, gate_round="split_p"), _sparse(p))
    p = _problem64(20, zero_tile=1)
    assert torch.equal(_sparse(p, gate_round="split_t"), _sparse(p, gate_round="f16"))
    p = _problem64(21)
    exact = _sparse(p)
    d = lambda a: float((a - exact).abs().max() / exact.abs().max())
    dt, d16 = d(_sparse(p, gate_round="split_t")), d(_sparse(p, gate_round="f16"))
    assert 0.0 < dt < d16, (dt, d16)
    assert d(_sparse(p, gate_round="split")) == 0.0


def test_split_t_backward_takes_the_forwards_gate():
    """"split_t"'s backward gate is its forward's (the tile rule): with the uncorrected tile's
    W rows zero it is "split" exactly, otherwise close to it.  "split_p" takes p from the
    forward's scores (the stored ones) and the same gate where it splits: with a threshold of
    0 (every slot split) it is "split_t" up to the order of the score arithmetic."""
    p = _problem64(22, zero_tile=0)
    for a, b in zip(_bwd(p, "split_t"), _bwd(p, "split")):
        assert torch.equal(a, b)
    p = _problem64(23)
    st, sp = _bwd(p, "split_t"), _bwd(p, "split")
    assert any(not torch.equal(a, b) for a, b in zip(st, sp))
    for a, b in zip(st, sp):
        assert float((a - b).abs().max() / b.abs().max()) < 1e-2
    import oracle.attention as mod
    old = mod.SPLIT_P
    try:
        mod.SPLIT_P = 0.0
        for a, b in zip(_bwd(p, "split_p"), st):
            assert torch.allclose(a, b, rtol=1e-9, atol=1e-300)
    finally:
        mod.SPLIT_P = old
