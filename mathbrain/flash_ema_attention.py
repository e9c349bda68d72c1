"""The dense flash-EMA attention entry point, computed over each row's unique slots.

Drop-in for mathbrain/flash_ema_attention.py:19-85 (``flash_ema_forward``), the
reference's all-vocabulary PyTorch formulation: per step every one of the V vocabulary
slots is decayed, gated by SiLU(pe_proj(C)), scored and averaged, and the state starts
at zero.  A slot whose token has not occurred yet has C = 0, hence gate SiLU(0) = 0, score
0 and value 0: it adds exactly e^(0 - m) to the softmax denominator and nothing else.  So
the same output comes from the unique-slot kernels (``FlashEMAFunction`` with the
absent-slot mass) on the sorted unique tokens of each row, without the [B, V, N] state or
the O(L V N D) work, and it is differentiable (the reference's in-place state update
blocks autograd).  pe_proj must have no bias, as in the model (model.py:44): with a bias
absent slots would not gate to zero.
"""
from .triton_flash_ema import FlashEMAFunction, _build_unique_index, precompute_boundaries


def flash_ema_forward(Q, x, E_k_slots, E_v_slots, rhos, pe_proj, n_heads, use_silu=True):
    """flash_ema_attention.flash_ema_forward (flash_ema_attention.py:19): Q [B, L, D],
    x [B, L] token ids, E_k_slots / E_v_slots [V, D], rhos [N], pe_proj an
    nn.Linear(N, D) without bias.  Returns [B, L, D]."""
    if Q.device.type != "cuda":
        raise NotImplementedError("flash_ema_attention.flash_ema_forward: tensors must be on an "
                                  "MI355X GPU; this implementation has no CPU path")
    if getattr(pe_proj, "bias", None) is not None:
        raise NotImplementedError("flash_ema_forward: pe_proj with a bias is not supported "
                                  "(absent slots would not gate to zero)")
    B, L, D = Q.shape
    V = E_k_slots.shape[0]
    H = n_heads
    hd = D // H
    unique, K_max = _build_unique_index(x, Q.device)
    rows = unique.clamp(min=0)
    E_k = E_k_slots[rows]
    E_v = E_v_slots[rows]
    C_bounds = precompute_boundaries(x, unique, rhos, 64)
    Q_mha = Q.view(B, L, H, hd).transpose(1, 2)
    out = FlashEMAFunction.apply(Q_mha, x, E_k, E_v, pe_proj.weight.t(), rhos, V, unique, K_max,
                                 C_bounds, use_silu)
    return out.transpose(1, 2).reshape(B, L, D)
