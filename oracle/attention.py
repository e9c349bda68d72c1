"""TEST INFRASTRUCTURE ONLY: CPU restatement of flash-EMA gated attention (the checker).

Three forms of the same attention, all in torch on the CPU:

``dense``      flash_ema_attention.flash_ema_forward (mathbrain/flash_ema_attention.py
               :19-85): one loop over L with a dense [B, V, N] counter state, decay ->
               gate -> attend over all V slots -> count.  Two generalisations, both
               no-ops for the reference's own inputs: an optional key-side initial
               state ``c_global`` (the reference starts from zeros, :36), and an
               out-of-place count update so autograd can differentiate it (the
               reference's in-place ``C[...] += 1`` at :82 makes backward fail).
``sparse``     the same attention over the unique slots of each sequence only, with
               the (V - K_b) absent slots -- whose counters stay zero, so their gate
               is SiLU(0) = 0 and their score 0 -- folded into the softmax
               denominator as (V - K_b) * exp(0 - m).  ``absent_mass=False`` gives
               the Triton kernel as executed (triton_flash_ema.py:215-229 wipes the
               absent mass).  ``gate_round`` (GATE_ROUNDS) rounds the gate operands
               as the reference's Triton kernel ("bf16", triton_flash_ema.py:188-190)
               or the HIP kernels ("f16", "split") feed their matrix products.
``sparse_backward_formulas``
               the reference's closed-form gradients (triton_flash_ema.py:336-350
               and :446-465), evaluated loop by loop; autograd of ``sparse`` must
               agree with it.

``t_eval`` (both sparse forms) names the steps at which outputs and gradients are
evaluated; the counter state still advances over every step.  Steps are independent
given the state, so this is exact -- for the backward, provided dO is zero at every
other step (their terms are then identically zero).  It makes the checker affordable
on full-length sequences (T = 4096, thousands of slots).
"""
import math

import torch
import torch.nn.functional as F


def silu_grad(x):
    """SiLU'(x) = sig(x) * (1 + x * (1 - sig(x)))  (triton_flash_ema.py:458)."""
    s = torch.sigmoid(x)
    return s * (1 + x * (1 - s))


def dense(Q, x, E_k_slots, E_v_slots, rhos, pe_weight, n_heads, use_silu=True, c_global=None):
    """flash_ema_attention.flash_ema_forward (flash_ema_attention.py:19-85).

    Q [B, L, D], x [B, L] int64, E_k_slots / E_v_slots [V, D], rhos [N],
    pe_weight [D, N] (= pe_proj.weight), c_global [B, V, N] or None.
    Returns out [B, L, D].
    """
    B, L, D = Q.shape
    V = E_k_slots.shape[0]
    N = rhos.shape[0]
    H = n_heads
    hd = D // H
    C = torch.zeros(B, V, N, dtype=Q.dtype) if c_global is None else c_global.to(Q.dtype)
    E_k = E_k_slots.reshape(V, H, hd).unsqueeze(0)
    E_v = E_v_slots.reshape(V, H, hd).unsqueeze(0)
    rho = rhos.to(Q.dtype).reshape(1, 1, N)
    outs = []
    for t in range(L):
        C = C * rho                                                  # :48
        p_lin = (C @ pe_weight.t().to(Q.dtype)).reshape(B, V, H, hd)  # :51
        gate = F.silu(p_lin) if use_silu else p_lin                  # :52-55
        Kt = (E_k * gate).transpose(1, 2)                            # :58 [B,H,V,hd]
        Vt = (E_v * gate).transpose(1, 2)                            # :59
        q_t = Q[:, t].reshape(B, H, 1, hd)                           # :73
        attn = (q_t @ Kt.transpose(-2, -1)) / math.sqrt(hd)          # :76
        attn = torch.softmax(attn, dim=-1)                           # :77
        outs.append(attn @ Vt)                                       # :79 [B,H,1,hd]
        onehot = F.one_hot(x[:, t], V).to(Q.dtype).unsqueeze(-1)     # :82, out of place
        C = C + onehot
    O = torch.cat(outs, dim=2)                                       # [B,H,L,hd]
    return O.transpose(1, 2).reshape(B, L, D)                       # :84


# ``gate_round``: how the gate GEMM's operands are rounded and how the dW_pe product takes
# its operands.  None: exact everywhere.  "bf16": both gate operands bf16 (the reference's
# triton_flash_ema.py:188-190).  "f16": both fp16, W pre-scaled by log2 e (the HIP kernels'
# single-product gate).  "split": the gate exact (the HIP kernels' fp16 hi + lo split leaves
# ~2^-22, below what a float64 check resolves at these bars; the fp32 mode).  "split_t": the
# split only on the 32-rate tiles ``corrected_rates`` selects and the "f16" product on the
# others, in the forward and the backward (the default mode when the backward recomputes the
# scores).  "split_p": "split_t"'s forward; in the backward p from the forward's scores (as
# stored) and, per (sequence, slot, head, 16-step half of a 32-step block), the "f16" gate
# where the forward's probability stays below SPLIT_P at every step of the half, else
# "split_t"'s (the HIP default mode's backward reading stored scores).  "f16c" / "f16w": only
# the counter / only W_pe rounded to fp16 (for measuring which rounding matters).  Every mode
# but None takes the dW_pe product from bf16 c_dec and bf16 dpre (triton_flash_ema.py:463-465).
GATE_ROUNDS = (None, "bf16", "f16", "split", "split_t", "split_p", "f16c", "f16w")
TILE_ROUNDS = ("split_t", "split_p")  # forwards that correct only some rate tiles
SPLIT_P = 2.0 ** -7
PHALF = 16  # steps per decision: a wave of the HIP backward takes 16 steps of one head


def _round_gate_operands(W, gate_round):
    """W_pe as the gate GEMM sees it: exact, bf16-rounded, or f16(W * log2 e) / log2 e
    ("f16" and "f16w"; "f16c" and "split" leave W exact)."""
    if gate_round not in GATE_ROUNDS:
        raise ValueError(f"gate_round={gate_round!r}")
    if gate_round in (None, "f16c", "split", "split_t", "split_p"):
        return W
    if gate_round == "bf16":
        return W.to(torch.bfloat16).to(W.dtype)
    if gate_round in ("f16", "f16w"):
        l2e = 1.0 / math.log(2.0)
        return (W.float() * l2e).to(torch.float16).to(W.dtype) / l2e
    raise ValueError(f"gate_round={gate_round!r}")


def _round_gate_counter(c, gate_round):
    """c_dec as the gate GEMM sees it (rounded through float32, as computed on device):
    exact for None, "f16w" and "split", else fp16 ("f16", "f16c") or bf16 ("bf16")."""
    if gate_round not in GATE_ROUNDS:
        raise ValueError(f"gate_round={gate_round!r}")
    if gate_round in (None, "f16w", "split", "split_t", "split_p"):
        return c
    return c.float().to(torch.float16 if gate_round != "bf16" else torch.bfloat16).to(c.dtype)


def corrected_rates(rhos):
    """Bool [N]: the rates whose 32-rate tile the default mode's forward gate splits into
    hi + lo products (flash_fwd_kernel.h).  A counter stays near or below B = 1 / (1 - rho)
    (float32, as the kernel computes it), and a single fp16 product's rounding on a rate's
    term scales with its counter; with two tiles (32 < N <= 64) the first is left to the
    single product when its largest B is below 1/32 of the second's.  Every other case is
    corrected in full."""
    N = rhos.shape[0]
    mask = torch.ones(N, dtype=torch.bool)
    if not 32 < N <= 64:
        return mask
    r = rhos.detach().to(torch.float32)
    B = 1.0 / torch.clamp(1.0 - r, min=1e-30)
    b0, b1 = B[:32].max(), B[32:].max()
    if 32.0 * b0 < torch.maximum(b0, b1):
        mask[:32] = False
    return mask


def _tile_gate_operands(W, rhos, gate_round):
    """(rate mask, W operand) of the "split_t" / "split_p" forward gate: the corrected rates
    take W exact, the others W rounded as "f16" takes it; (None, W) for other modes."""
    if gate_round not in TILE_ROUNDS:
        return None, W
    mask = corrected_rates(rhos)
    return mask, torch.where(mask.unsqueeze(1), W, _round_gate_operands(W, "f16"))


def _tile_gate_counter(c, mask):
    """c_dec operand of the tile-corrected forward gate (mask None: c unchanged)."""
    if mask is None:
        return c
    return torch.where(mask, c, _round_gate_counter(c, "f16"))


def _gate_product(c, W):
    """The gate GEMM c_dec @ W_pe of both sparse forms (one place, so that a check can
    substitute another evaluation of it)."""
    return c @ W


def _steps(L, t_eval):
    return list(range(L)) if t_eval is None else sorted({int(t) for t in t_eval})


def sparse(Q, x, E_k, E_v, W_pe, rhos, V_total, unique, c_init=None, use_silu=True,
           absent_mass=True, gate_round=None, return_lse=False, t_eval=None, return_probs=False):
    """Unique-slot flash-EMA attention.

    Q [B, H, L, hd]; x [B, L]; E_k / E_v [B, K, D]; W_pe [N, D] (= pe_proj.weight.T);
    unique [B, K] int64 with -1 padding; c_init [B, K, N] key-side state at t=0
    (C_bounds[:, 0]).  Returns O [B, H, L, hd] (and LSE [B, H, L]); with ``t_eval``,
    O [B, H, len(t_eval), hd] and LSE [B, H, len(t_eval)] at those steps, in order.  With
    ``return_probs`` the softmax weights p [B, K, H, steps] of the valid slots come last.

    The per-step order is the reference's: c_dec = C * rho (triton_flash_ema.py:185),
    g = SiLU(c_dec @ W_pe[:, head]) (:188-196), s = q.(e_k*g)/sqrt(hd) over valid
    slots (:205-207), online softmax (:224-234), then C = c_dec + match (:241).
    """
    B, H, L, hd = Q.shape
    K = unique.shape[1]
    N = rhos.shape[0]
    D = H * hd
    dt = Q.dtype
    valid = unique != -1                                             # [B, K]
    Kb = valid.sum(1)                                                # [B]
    C = torch.zeros(B, K, N, dtype=dt) if c_init is None else c_init[:, :, :N].to(dt)
    C = C * valid.unsqueeze(-1).to(dt)
    rho = rhos.to(dt).reshape(1, 1, N)
    W = _round_gate_operands(W_pe[:N].to(dt), gate_round)
    tmask, W = _tile_gate_operands(W, rhos[:N], gate_round)
    Ek = E_k.reshape(B, K, H, hd).to(dt)
    Ev = E_v.reshape(B, K, H, hd).to(dt)
    log_absent = torch.log((V_total - Kb).clamp(min=0).to(dt))       # -inf if none absent
    outs, lses, probs = [], [], []
    evaluate = set(_steps(L, t_eval))
    for t in range(L):
        c_dec = C * rho
        if t not in evaluate:
            match = (x[:, t].unsqueeze(1) == unique) & valid
            C = c_dec + match.unsqueeze(-1).to(dt)
            continue
        cg = _tile_gate_counter(_round_gate_counter(c_dec, gate_round), tmask)
        pre = _gate_product(cg, W).reshape(B, K, H, hd)
        g = F.silu(pre) if use_silu else pre
        q_t = Q[:, :, t].unsqueeze(1)                                # [B,1,H,hd]
        s = (q_t * Ek * g).sum(-1) / math.sqrt(hd)                   # [B,K,H]
        s = s.masked_fill(~valid.unsqueeze(-1), float("-inf"))
        if absent_mass:
            extra = log_absent.reshape(B, 1, 1).expand(B, 1, H)
            lse = torch.logsumexp(torch.cat([s, extra], dim=1), dim=1)    # [B,H]
        else:
            lse = torch.logsumexp(s, dim=1)
        p = torch.exp(s - lse.unsqueeze(1))                          # [B,K,H]
        o = (p.unsqueeze(-1) * Ev * g).sum(1)                        # [B,H,hd]
        outs.append(o)
        lses.append(lse)
        if return_probs:
            probs.append(p)
        match = (x[:, t].unsqueeze(1) == unique) & valid
        C = c_dec + match.unsqueeze(-1).to(dt)
    O = torch.stack(outs, dim=2)                                     # [B,H,L,hd]
    LSE = torch.stack(lses, dim=2)                                   # [B,H,L]
    res = (O, LSE) if return_lse else (O,)
    if return_probs:
        res = res + (torch.stack(probs, dim=-1),)
    return res if len(res) > 1 else res[0]


@torch.no_grad()
def single_gate_halves(P):
    """[B, K, H, ceil(L / PHALF)]: True where the probabilities P [B, K, H, L] stay below
    SPLIT_P at every step of the half-block (steps past L count as 0)."""
    B, K, H, L = P.shape
    nh = (L + PHALF - 1) // PHALF
    P = F.pad(P, (0, nh * PHALF - L))
    return P.reshape(B, K, H, nh, PHALF).amax(-1) < SPLIT_P


def sparse_backward_formulas(Q, x, E_k, E_v, W_pe, rhos, V_total, unique, dO, c_init=None,
                             use_silu=True, absent_mass=True, gate_round=None, t_eval=None):
    """The reference's closed-form backward, loop by loop (float64 recommended).

    D = (dO*O).sum(-1) (triton_flash_ema.py:602); p = exp(s - LSE) (:336);
    ds = p (dO.v - D) (:339-340); dQ = sum_k ds k_dyn/sqrt(hd) (:343);
    dE_k = sum_t ds q*g/sqrt(hd) (:349); dE_v = sum_t p dO*g (:350);
    dpre = (ds q/sqrt(hd)*e_k + p dO*e_v) * SiLU'(pre) (:453-461);
    dW_pe[:, head] = sum c_dec^T dpre (:465).
    Returns dQ [B,H,L,hd], dE_k [B,K,D], dE_v [B,K,D], dW_pe [N,D].
    With ``gate_round`` the gate operands are rounded as in ``sparse`` (for "split_p" the
    backward's gate and p differ, see GATE_ROUNDS) and the dW_pe product takes bf16 c_dec (of
    the gate's rounded c_dec; of the float32 counter with the split modes) and bf16 dpre, as
    triton_flash_ema.py:463-465 does.
    With ``t_eval`` only those steps contribute (exact when dO is zero elsewhere); dQ
    is zero at the other steps.
    """
    B, H, L, hd = Q.shape
    K = unique.shape[1]
    N = rhos.shape[0]
    D = H * hd
    dt = Q.dtype
    steps = _steps(L, t_eval)
    O, LSE = sparse(Q, x, E_k, E_v, W_pe, rhos, V_total, unique, c_init, use_silu,
                    absent_mass, gate_round=gate_round, return_lse=True, t_eval=steps)
    Dv = (dO[:, :, steps] * O).sum(-1)                               # [B,H,len(steps)]
    slot = {t: i for i, t in enumerate(steps)}
    valid = unique != -1
    C = torch.zeros(B, K, N, dtype=dt) if c_init is None else c_init[:, :, :N].to(dt)
    C = C * valid.unsqueeze(-1).to(dt)
    rho = rhos.to(dt).reshape(1, 1, N)
    W = _round_gate_operands(W_pe[:N].to(dt), gate_round)
    tmask, W = _tile_gate_operands(W, rhos[:N], gate_round)
    Ek = E_k.reshape(B, K, H, hd).to(dt)
    Ev = E_v.reshape(B, K, H, hd).to(dt)
    bf = (lambda v: v.float().to(torch.bfloat16).to(dt)) if gate_round else (lambda v: v)
    if gate_round == "split_p":  # the forward's probabilities; per (b, k, h, half-block):
        # may the backward's gate be single fp16?
        _, _, P = sparse(Q, x, E_k, E_v, W_pe, rhos, V_total, unique, c_init, use_silu, absent_mass,
                         gate_round="split_t", return_lse=True, return_probs=True)
        single = single_gate_halves(P)                                # [B,K,H,nh]
        W16 = _round_gate_operands(W_pe[:N].to(dt), "f16")
    dQ = torch.zeros_like(Q)
    dEk = torch.zeros(B, K, H, hd, dtype=dt)
    dEv = torch.zeros(B, K, H, hd, dtype=dt)
    dW = torch.zeros(N, D, dtype=dt)
    scale = 1.0 / math.sqrt(hd)
    for t in range(L):
        c_dec = C * rho
        if t not in slot:
            match = (x[:, t].unsqueeze(1) == unique) & valid
            C = c_dec + match.unsqueeze(-1).to(dt)
            continue
        i = slot[t]
        cg = _tile_gate_counter(_round_gate_counter(c_dec, gate_round), tmask)
        pre = _gate_product(cg, W).reshape(B, K, H, hd)
        if gate_round == "split_p":
            pre16 = _gate_product(_round_gate_counter(c_dec, "f16"), W16).reshape(B, K, H, hd)
            pre = torch.where(single[..., t // PHALF].unsqueeze(-1), pre16, pre)
        g = F.silu(pre) if use_silu else pre
        gp = silu_grad(pre) if use_silu else torch.ones_like(pre)
        q_t = Q[:, :, t].unsqueeze(1)                                # [B,1,H,hd]
        do_t = dO[:, :, t].unsqueeze(1)
        if gate_round == "split_p":  # the forward's stored scores give p (its own gate)
            p = P[..., t] * valid.unsqueeze(-1).to(dt)
        else:
            s = (q_t * Ek * g).sum(-1) * scale
            p = torch.exp(s - LSE[:, :, i].unsqueeze(1)) * valid.unsqueeze(-1).to(dt)
        dp = (do_t * Ev * g).sum(-1)
        ds = p * (dp - Dv[:, :, i].unsqueeze(1))                     # [B,K,H]
        dQ[:, :, t] = (ds.unsqueeze(-1) * Ek * g).sum(1) * scale
        dEk += ds.unsqueeze(-1) * q_t * g * scale
        dEv += p.unsqueeze(-1) * do_t * g
        dpre = (ds.unsqueeze(-1) * q_t * scale * Ek + p.unsqueeze(-1) * do_t * Ev) * gp
        cw = c_dec.float().to(dt) if gate_round in ("split", "split_t", "split_p") else cg  # the kernel's float32 counter
        dW += torch.einsum("bkn,bkd->nd", bf(cw), bf(dpre.reshape(B, K, D)))
        match = (x[:, t].unsqueeze(1) == unique) & valid
        C = c_dec + match.unsqueeze(-1).to(dt)
    return dQ, dEk.reshape(B, K, D), dEv.reshape(B, K, D), dW


def scatter_c_global(unique, c_init, V):
    """Dense key-side initial state [B, V, N] from the unique-slot one (pads dropped)."""
    B, K, N = c_init.shape
    Cg = torch.zeros(B, V, N, dtype=c_init.dtype)
    for b in range(B):
        for k in range(K):
            u = int(unique[b, k])
            if u >= 0:
                Cg[b, u] = c_init[b, k]
    return Cg
