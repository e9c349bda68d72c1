"""TEST INFRASTRUCTURE ONLY: CPU restatement of SlotTransformerLM's forward (the checker).

``lm_forward`` evaluates mathbrain/model.py:144-186 from a parameter dict keyed like the
module's state_dict, in whatever dtype the parameters have (float64 in the tests), with
autograd intact so parameter gradients can be compared.  It composes the other oracle
pieces: the query scan (``scan.query_scan``), the gating (``gating.forward``) and the
attention, either

* ``attention="sparse"``: the device path of model.py:63-87 -- slot K/V projections of
  the sequence's unique slots and unique-slot attention with the absent-slot mass and the
  key-side c_base (``attention.sparse``), or
* ``attention="dense"``: the reference's CPU path of model.py:88-99 -- K/V projections of
  the whole vocabulary and the dense all-slot attention (``attention.dense``), which
  starts every key counter at zero.

Pinning: with no carried state (c_base None) the two must agree (dense == sparse + absent
mass at model level), which tests/test_oracle_model.py checks in float64.
"""
import torch
import torch.nn.functional as F

from . import attention as att
from . import gating
from . import scan


class _Rounded(torch.autograd.Function):
    """Rounds the value to ``dtype`` and back, and its gradient the same way: a tensor that
    torch.autocast keeps in bf16, forward and backward."""

    @staticmethod
    def forward(ctx, t, dtype):
        ctx.dt = dtype
        return t.to(dtype).to(t.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(ctx.dt).to(g.dtype), None


class _RoundedLinear(torch.autograd.Function):
    """a @ w.T as a Linear under torch.autocast computes it: both operands rounded to
    ``dtype``, the product accumulated wide and rounded to ``dtype``; in the backward the
    incoming gradient is rounded and both products rounded the same way."""

    @staticmethod
    def forward(ctx, a, w, dtype):
        r = lambda t: t.to(dtype).to(t.dtype)
        ar, wr = r(a), r(w)
        ctx.save_for_backward(ar, wr)
        ctx.dt = dtype
        return r(ar @ wr.t())

    @staticmethod
    def backward(ctx, g):
        ar, wr = ctx.saved_tensors
        r = lambda t: t.to(ctx.dt).to(t.dtype)
        gr = r(g)
        da = r(gr @ wr)
        dw = r(gr.reshape(-1, gr.shape[-1]).t() @ ar.reshape(-1, ar.shape[-1]))
        return da, dw, None


def linear(a, w, dtype=None):
    """nn.Linear without bias (w [out, in]); ``dtype`` (e.g. torch.bfloat16) evaluates it as
    torch.autocast does."""
    return a @ w.t() if dtype is None else _RoundedLinear.apply(a, w, dtype)


def rounded(t, dtype=None):
    return t if dtype is None else _Rounded.apply(t, dtype)


def rmsnorm(x, w, eps=1e-6):
    """model.py:17-19."""
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def swiglu(x, w1, w2, w3, amp=None, fused=False):
    """model.py:28-29 (nn.Linear weights are [out, in]); ``amp``: the autocast dtype, whose
    roundings the silu and the product of the bf16 projections then take too, each (torch's
    separate ops, the reference) or only the product (``fused``: a fused silu-product kernel)."""
    a = linear(x, w1, amp)
    h = rounded((F.silu(a) if fused else rounded(F.silu(a), amp)) * linear(x, w3, amp), amp)
    return linear(h, w2, amp)


def unique_index(x):
    """_build_unique_index (triton_flash_ema.py:475-507): sorted unique ids per row,
    -1 padded to K_max = max(max count, 16)."""
    rows = [torch.unique(r) for r in x]
    K = max(max(r.numel() for r in rows), 16)
    out = torch.full((x.shape[0], K), -1, dtype=torch.int64)
    for b, r in enumerate(rows):
        out[b, : r.numel()] = r
    return out


def lm_forward(p, x, n_layers, n_heads, rhos, vocab_size, unique_slots=None, c_base=None,
               pad_mask=None, use_silu=True, attention="sparse", gate_round=None,
               absent_mass=True, mask_query_keys=True, t_eval=None, amp=None, amp_pe_proj=False,
               amp_fused_swiglu=False):
    """Logits [B, L, V] of SlotTransformerLM.forward (model.py:144-186).

    ``absent_mass`` picks the attention's softmax (all V slots, or the valid slots only as
    the reference's Triton kernel computes it).  ``mask_query_keys=False`` reproduces the
    reference's query scan on the 0-padded slot list (model.py:157).  With ``t_eval`` the
    logits are [B, len(t_eval), V] at those positions only: K/V come from the embedding
    table and the counter states, not from other positions' hidden states, so every
    position's logits depend on its own row and the states alone (exact).

    ``amp`` (torch.bfloat16) evaluates the model as it runs under torch.autocast: every
    Linear's operands, product and gradients rounded to bf16 (``linear``), the SwiGLU silu and
    product too; norms, the gating and the attention (custom_fwd(cast_inputs=float32) in
    the reference, triton_flash_ema.py:573, triton_fused_gating.py) stay wide.  The query
    gate's pe_proj is a Linear in the reference's wrapper (triton_fused_gating.py:183), so
    under autocast its output is bf16 there; ``amp_pe_proj`` rounds it that way, where this
    implementation computes it inside the fp32 gating kernel.  ``amp_fused_swiglu`` rounds
    SwiGLU's silu-product once, as this implementation's fused kernel does (twice in torch's
    separate ops)."""
    B, L = x.shape
    E = p["embed.weight"]
    dt = E.dtype
    D = E.shape[1]
    H = n_heads
    hd = D // H
    x_q = E[x]                                                          # :149
    keys = unique_slots
    if unique_slots is not None and pad_mask is not None and mask_query_keys:
        # the collate padding masked to -1 on the query side too (the reference passes the
        # 0-padded list, model.py:157, which can overwrite token 0's carried row)
        keys = unique_slots.masked_fill(~pad_mask, -1)
    C_seq = torch.from_numpy(scan.query_scan(x, rhos, vocab_size, c_base, keys)).to(dt)  # :157
    steps = list(range(L)) if t_eval is None else [int(t) for t in t_eval]
    if t_eval is not None:
        if attention != "sparse":
            raise ValueError("t_eval needs the sparse attention")
        x_q = x_q[:, steps]
        C_seq = C_seq[:, steps]
    Le = len(steps)
    if unique_slots is not None and pad_mask is not None:               # :163-174
        unique = unique_slots.masked_fill(~pad_mask, -1)
        K_max = max(int(pad_mask.sum(1).max()), 16)
        unique = unique[:, :K_max]
        cb = c_base[:, :K_max].to(dt) if c_base is not None else None
        if unique.shape[1] < K_max:
            pad = K_max - unique.shape[1]
            unique = F.pad(unique, (0, pad), value=-1)
            cb = F.pad(cb, (0, 0, 0, pad)) if cb is not None else None
    else:
        unique = unique_index(x)                                        # :177
        cb = None
    for l in range(n_layers):
        pre = f"layers.{l}."
        g = lambda name: p[pre + name]
        a = rmsnorm(x_q, g("attn_norm.weight"))                         # :114
        Q_t = gating.forward(a, C_seq, g("attn.pe_proj.weight"), g("attn.ln_q.weight"),
                             g("attn.ln_q.bias"), g("attn.q_proj.weight"), use_silu,
                             linear=lambda u, w: linear(u, w, amp),
                             pe_linear=lambda u, w: linear(u, w, amp if amp_pe_proj else None))   # :75
        if attention == "sparse":
            E_active = E[unique.clamp(min=0)]                           # :64-65
            mem = F.layer_norm(E_active, (D,), g("attn.ln_kv.weight"), g("attn.ln_kv.bias"))
            Ek = linear(mem, g("attn.k_proj.weight"), amp)              # :67
            Ev = linear(mem, g("attn.v_proj.weight"), amp)              # :68
            Q_full = Q_t
            if t_eval is not None:   # rows of the other steps are never read
                Q_full = Q_t.new_zeros(B, L, D).index_copy(1, torch.tensor(steps), Q_t)
            Q_mha = Q_full.reshape(B, L, H, hd).transpose(1, 2)          # :81
            Wt = g("attn.pe_proj.weight").t()
            # "split_t" and "split_p" round the backward's gate differently from the forward's,
            # so their gradients come from the closed-form backward rather than from autograd
            if t_eval is None and gate_round not in att.TILE_ROUNDS:
                O = att.sparse(Q_mha, x, Ek, Ev, Wt, rhos.to(dt), vocab_size, unique, cb,
                               use_silu=use_silu, absent_mass=absent_mass, gate_round=gate_round)
            else:
                O = _SampledAttention.apply(Q_mha, Ek, Ev, Wt, x, rhos.to(dt), vocab_size, unique,
                                            cb, use_silu, absent_mass, gate_round, steps)
            out = O.transpose(1, 2).reshape(B, Le, D)                   # :87
        elif attention == "dense":
            mem = F.layer_norm(E, (D,), g("attn.ln_kv.weight"), g("attn.ln_kv.bias"))   # :92
            Eks = mem @ g("attn.k_proj.weight").t()                     # :93
            Evs = mem @ g("attn.v_proj.weight").t()                     # :94
            out = att.dense(Q_t, x, Eks, Evs, rhos.to(dt), g("attn.pe_proj.weight"), H, use_silu)
        else:
            raise ValueError(attention)
        out = linear(out, g("attn.o_proj.weight"), amp)                 # :101
        h = x_q + out                                                   # :114
        h = h + swiglu(rmsnorm(h, g("ffn_norm.weight")), g("ffn.w1.weight"), g("ffn.w2.weight"),
                       g("ffn.w3.weight"), amp, amp_fused_swiglu)       # :115
        x_q = h
    x_q = rmsnorm(x_q, p["final_norm.weight"])                          # :185
    return linear(x_q, E, amp)                                          # :186, tied lm_head


class _SampledAttention(torch.autograd.Function):
    """attention.sparse evaluated at ``steps`` only, with the reference's closed-form
    gradients (attention.sparse_backward_formulas, itself checked equal to autograd in
    float64) as its backward, so no per-step autograd graph is kept.  Q [B, H, L, hd] (rows
    of other steps unused); returns O [B, H, len(steps), hd]."""

    @staticmethod
    def forward(ctx, Q, Ek, Ev, Wt, x, rhos, V, unique, cb, use_silu, absent_mass, gate_round, steps):
        with torch.no_grad():
            O = att.sparse(Q, x, Ek, Ev, Wt, rhos, V, unique, cb, use_silu=use_silu,
                           absent_mass=absent_mass, gate_round=gate_round, t_eval=steps)
        ctx.save_for_backward(Q, Ek, Ev, Wt)
        ctx.rest = (x, rhos, V, unique, cb, use_silu, absent_mass, gate_round, steps)
        return O

    @staticmethod
    def backward(ctx, dO_e):
        Q, Ek, Ev, Wt = ctx.saved_tensors
        x, rhos, V, unique, cb, use_silu, absent_mass, gate_round, steps = ctx.rest
        dO = Q.new_zeros(Q.shape)
        dO[:, :, steps] = dO_e
        dQ, dEk, dEv, dW = att.sparse_backward_formulas(
            Q, x, Ek, Ev, Wt, rhos, V, unique, dO, cb, use_silu=use_silu, absent_mass=absent_mass,
            gate_round=gate_round, t_eval=steps)
        return (dQ, dEk.reshape(Ek.shape), dEv.reshape(Ev.shape), dW[: Wt.shape[0]]) + (None,) * 9
