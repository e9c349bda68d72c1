"""SlotTransformerLM over the gfx950 hot path.

Drop-in for mathbrain/model.py (:11-186): the same modules, parameter names, constructor
arguments and forward signatures, so checkpoints and train.py's calls carry over.  The
hot path runs in the HIP kernels: the query scan (``compute_query_ema_history``), the
key-side chunk states (``precompute_boundaries``), the gating with pe_proj folded in
(``fused_apply_symmetric_query_gating``), flash-EMA attention (``FlashEMAFunction``) and
RMSNorm (``rms_norm``), ln_kv (``layer_norm``) and SwiGLU's gate product
(``swiglu_product``), one fused pass per direction each.  The linear layers (the slot K/V projections, the FFN and the tied lm_head)
stay torch modules, as in the reference.  The reference's CPU branch (dense attention over the whole vocabulary,
model.py:88-99) is not a product path here: CPU tensors raise NotImplementedError.
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .triton_ema_query import compute_query_ema_history
from .triton_flash_ema import (FlashEMAFunction, GatedQueryFlashEMAFunction, _build_unique_index,
                               check_counter_range, precompute_boundaries)
from .triton_fused_gating import fused_apply_symmetric_query_gating
from .layernorm import layer_norm
from .rmsnorm import rms_norm
from .swiglu import swiglu_product


class RMSNorm(nn.Module):
    """model.py:11-19."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        # one fused HIP pass per direction (mb_rmsnorm_fwd / mb_rmsnorm_bwd) for
        # weight * (x * rsqrt(mean(x^2) + eps))
        return rms_norm(x, self.weight, self.eps)


class SwiGLU(nn.Module):
    """model.py:21-29."""

    def __init__(self, dim: int, hidden_dim: int):
        super().__init__()
        self.w1 = nn.Linear(dim, hidden_dim, bias=False)
        self.w2 = nn.Linear(hidden_dim, dim, bias=False)
        self.w3 = nn.Linear(dim, hidden_dim, bias=False)

    def forward(self, x):
        # silu(w1 x) * w3 x as one fused HIP pass per direction (mb_swiglu_fwd / _bwd)
        return self.w2(swiglu_product(self.w1(x), self.w3(x)))


class SlotAttentionLayer(nn.Module):
    """Multiplicative EMA cross-attention over the sequence's unique slots
    (model.py:32-102): memory = ln_kv(E[slots]), K = k_proj(memory), V = v_proj(memory),
    keys and values gated by SiLU(pe_proj(C)) inside the flash-EMA kernel."""

    def __init__(self, d_model: int, n_heads: int, dropout: float, n_scales: int, use_silu: bool = True,
                 absent_mass: bool = True, precision: str = "bf16"):
        super().__init__()
        assert d_model % n_heads == 0
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.q_proj = nn.Linear(d_model, d_model, bias=False)
        self.k_proj = nn.Linear(d_model, d_model, bias=False)
        self.v_proj = nn.Linear(d_model, d_model, bias=False)
        self.o_proj = nn.Linear(d_model, d_model, bias=False)
        self.pe_proj = nn.Linear(n_scales, d_model, bias=False)
        self.ln_kv = nn.LayerNorm(d_model)
        self.ln_q = nn.LayerNorm(d_model)
        self.resid_dropout = nn.Dropout(dropout)
        self.use_silu = use_silu
        # softmax over all V slots (the dense PyTorch reference) or over the valid slots only
        # (the reference's Triton kernel): see FlashEMAFunction
        self.absent_mass = absent_mass
        # the attention's gate arithmetic (triton_flash_ema.PRECISIONS): "bf16" (split fp16
        # gate operands, bf16 dW_pe), "fp16" (single fp16 gate operands) or "fp32"
        self.precision = precision
        # True: compute the queries (gating, ln_q, q_proj) inside the attention kernel
        # (GatedQueryFlashEMAFunction) when the shapes allow it.  Off by default: measured at
        # configuration 5 it costs more than it saves -- every 32-step workgroup streams all of
        # q_proj.weight, a training step's backward needs Q and the LayerNorm output anyway, and
        # even a forward without autograd took 35.7 ms against 35.3 ms with the separate gating
        # kernel and q_proj GEMM
        self.fold_query_gating = False

    def _folds_query_gating(self, D):
        return (bool(self.fold_query_gating) and self.pe_proj.bias is None and self.q_proj.bias is None
                and self.ln_q.weight is not None and self.ln_q.bias is not None and D % 32 == 0
                and D <= 1024 and self.head_dim <= 64)

    def forward(self, x_q, x, E_slots, rhos, C_seq, unique_tensor=None, K_max=None, C_bounds=None,
                E_active=None):
        """``E_active`` optionally carries the gather E_slots[max(unique, 0)] that every layer
        of the reference recomputes (model.py:63-64); SlotTransformerLM gathers once for all
        layers, so the embedding backward runs once on the layers' summed gradients.  A 2-D
        ``E_active`` [V, D] is the embedding table itself: the projections then cover the
        vocabulary and the attention reads each slot's row by its token id."""
        B, L, D = x_q.shape
        if unique_tensor is None or C_bounds is None:
            # model.py:88-99 runs the dense all-vocabulary reference here; it is the CPU
            # reference's path, not this implementation's.
            raise NotImplementedError(
                "SlotAttentionLayer: needs unique_tensor and C_bounds (the dense all-vocabulary "
                "path is the reference's CPU fallback, not part of this implementation)")
        # 1. slot K/V projections (model.py:63-68)
        if E_active is None:
            E_active = F.embedding(torch.clamp(unique_tensor, min=0), E_slots)
        memory_base = layer_norm(E_active, self.ln_kv.weight, self.ln_kv.bias, self.ln_kv.eps)
        E_k_active = self.k_proj(memory_base)
        E_v_active = self.v_proj(memory_base)
        H = self.n_heads
        hd = D // H
        W_pe_t = self.pe_proj.weight.t()
        if self._folds_query_gating(D):
            # 2 + 3. query gating, ln_q and q_proj inside the attention kernels
            out_mha = GatedQueryFlashEMAFunction.apply(
                x_q, C_seq, W_pe_t, self.ln_q.weight, self.ln_q.bias, self.q_proj.weight, x, E_k_active,
                E_v_active, rhos, E_slots.shape[0], unique_tensor, K_max, C_bounds, H, self.use_silu, 64,
                self.absent_mass, self.precision, self.ln_q.eps)
        else:
            # 2. query gating (model.py:75)
            Q_t = fused_apply_symmetric_query_gating(x_q, C_seq, self.pe_proj, self.ln_q, self.q_proj,
                                                     self.use_silu)
            # 3. gated cross-attention (model.py:79-87)
            Q_mha = Q_t.view(B, L, H, hd).transpose(1, 2)
            out_mha = FlashEMAFunction.apply(Q_mha, x, E_k_active, E_v_active, W_pe_t, rhos,
                                             E_slots.shape[0], unique_tensor, K_max, C_bounds, self.use_silu,
                                             64, self.absent_mass, self.precision)
        out = out_mha.transpose(1, 2).reshape(B, L, D)
        out = self.o_proj(out)
        return self.resid_dropout(out)


class SlotTransformerBlock(nn.Module):
    """model.py:105-116."""

    def __init__(self, d_model, n_heads, d_ff, dropout, n_scales, use_silu=True, absent_mass=True,
                 precision="bf16"):
        super().__init__()
        self.attn_norm = RMSNorm(d_model)
        self.attn = SlotAttentionLayer(d_model, n_heads, dropout, n_scales, use_silu, absent_mass, precision)
        self.ffn_norm = RMSNorm(d_model)
        self.ffn = SwiGLU(d_model, d_ff)

    def forward(self, x_q, x, E_slots, rhos, C_seq, unique_tensor=None, K_max=None, C_bounds=None,
                E_active=None):
        h = x_q + self.attn(self.attn_norm(x_q), x, E_slots, rhos, C_seq, unique_tensor, K_max, C_bounds,
                            E_active)
        h = h + self.ffn(self.ffn_norm(h))
        return h


class SlotTransformerLM(nn.Module):
    """model.py:119-186.  forward(x, unique_slots=None, inverse_indices=None, c_base=None,
    doc_ids=None, pad_mask=None) -> logits [B, L, vocab_size].

    With ``unique_slots`` and ``pad_mask`` (the data loader's history-expanded slots) the
    slots are those, padded with -1 where pad_mask is False; otherwise the sorted unique
    tokens of each row (``_build_unique_index``) with no carried state.  As in the
    reference, ``inverse_indices`` and ``doc_ids`` are accepted and unused (a chunk is one
    document).
    """

    def __init__(self, vocab_size, d_model, n_layers, n_heads, N=16, dropout=0.1, use_silu=True,
                 ema_dropout=0.0, min_hl=1.0, max_hl=2048.0, absent_mass=True, attn_precision="bf16"):
        super().__init__()
        self.vocab_size = vocab_size
        self.d_model = d_model
        self.n_scales = N
        self.ema_dropout = ema_dropout
        half_lives = torch.logspace(math.log10(min_hl), math.log10(max_hl), self.n_scales)
        rhos = torch.exp(-torch.log(torch.tensor(2.0)) / half_lives)
        # the attention's gate takes the key counters as fp16 operands: refuse half-lives
        # whose counters could leave that range, here rather than at the first step
        check_counter_range(rhos, "SlotTransformerLM")
        self.register_buffer("ema_rhos", rhos)
        self.embed = nn.Embedding(vocab_size, d_model)
        d_ff = 256 * ((int(8 * d_model / 3) + 255) // 256)
        self.layers = nn.ModuleList([
            SlotTransformerBlock(d_model, n_heads, d_ff, dropout, self.n_scales, use_silu, absent_mass,
                                 attn_precision)
            for _ in range(n_layers)
        ])
        self.final_norm = RMSNorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        self.lm_head.weight = self.embed.weight
        # K/V rows from the projected vocabulary table (True), from the per-row slot gather
        # (False), or whichever has fewer rows (None)
        self.kv_table = None

    def forward(self, x, unique_slots=None, inverse_indices=None, c_base=None, doc_ids=None, pad_mask=None):
        device = x.device
        if device.type != "cuda":
            raise NotImplementedError(
                "SlotTransformerLM: this implementation runs on an MI355X GPU only "
                "(the reference's CPU path is its dense PyTorch fallback)")
        E_slots = self.embed.weight
        x_q = self.embed(x)
        if unique_slots is not None and pad_mask is not None:
            # -1 marks the collate padding on both sides.  The reference passes the padded
            # list (pad id 0) to the query scan (model.py:157), where a padding entry can
            # overwrite a real token 0's carried row with zeros while the key side keeps it
            # (model.py:167-180); with the masked list the two sides agree.
            unique_tensor = unique_slots.masked_fill(~pad_mask, -1)
            # K_max: the slot list's width (at least 16).  The reference reads back the largest
            # valid count instead (model.py:169, a host sync every step) and cuts the list
            # there; with the data loader's prefix masks both are the width, and the kernels
            # skip a row's trailing padding slots either way.
            K_max = max(unique_tensor.shape[1], 16)
            c_base_kv = c_base[:, :K_max, :] if c_base is not None else None
            C_seq = compute_query_ema_history(x, self.ema_rhos, self.vocab_size, c_base, unique_tensor)
            if unique_tensor.shape[1] < K_max:
                # fewer than 16 slots in every row: pad the slot list to the 16 the
                # reference's K_max floor asks for (model.py:170), with -1
                pad = K_max - unique_tensor.shape[1]
                unique_tensor = F.pad(unique_tensor, (0, pad), value=-1)
                if c_base_kv is not None:
                    c_base_kv = F.pad(c_base_kv, (0, 0, 0, pad))
        else:
            C_seq = compute_query_ema_history(x, self.ema_rhos, self.vocab_size, c_base, unique_slots)
            # each row's distinct tokens padded to the row length (model.py:177 reads the
            # largest count back instead; the extra -1 slots are skipped by the kernels)
            unique_tensor, K_max = _build_unique_index(x, device, width=x.shape[1])
            c_base_kv = None
        if self.ema_dropout > 0 and self.training:
            C_seq = F.dropout(C_seq, p=self.ema_dropout, training=True)
        C_bounds = precompute_boundaries(x, unique_tensor, self.ema_rhos, 64, c_init=c_base_kv)
        # The slot rows every layer gathers (model.py:63-64) are the same: gather once, so that
        # autograd sums the layers' gradients first and runs one embedding backward.  When
        # the slot lists hold more rows than the vocabulary (B * K_max > V), the layers
        # instead project the embedding table itself (ln_kv, k_proj and v_proj act row by
        # row, so row u of the projected table is what every slot of token u would gather)
        # and the attention reads the slot rows from it by token id: fewer rows to
        # normalise, project and cast, and no gather or scatter.
        use_table = self.kv_table if self.kv_table is not None else x.shape[0] * K_max > E_slots.shape[0]
        if use_table:
            E_active = E_slots
        else:
            E_active = F.embedding(torch.clamp(unique_tensor, min=0), E_slots)
        for layer in self.layers:
            x_q = layer(x_q, x, E_slots, self.ema_rhos, C_seq, unique_tensor, K_max, C_bounds, E_active)
        x_q = self.final_norm(x_q)
        return self.lm_head(x_q)
