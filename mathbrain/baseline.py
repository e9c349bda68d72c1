"""RoPE transformer baseline (the comparison model train.py builds with --model rope).

Not on the Per-Slot EMA path: it exists so that train.py's ``from mathbrain.baseline
import RoPETransformerLM`` (train.py:43) resolves and a run can switch models.  The
module tree and parameter names follow mathbrain/baseline.py:31-129 (checkpoints load
by name); the blocks reuse this package's RMSNorm and SwiGLU (one HIP pass per
direction) and torch's scaled_dot_product_attention.  The rotary embedding rotates the
channel pairs (2i, 2i+1) of each head by t * theta^(-2i/hd), written with real cos/sin
tables instead of the reference's complex multiply (the same rotation).
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from .model import RMSNorm, SwiGLU


def rotary_tables(head_dim, max_len, theta=10000.0):
    """cos and sin [max_len, head_dim / 2] of the angles t * theta^(-2i/head_dim)."""
    inv = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)
    ang = torch.arange(max_len, dtype=torch.float32)[:, None] * inv[None, :]
    return ang.cos(), ang.sin()


def rotate(x, cos, sin):
    """Rotates the pairs (x[..., 2i], x[..., 2i+1]) of x [B, L, H, hd] by the step's angles
    (computed in fp32, returned in x's dtype)."""
    xf = x.float().unflatten(-1, (-1, 2))
    a, b = xf[..., 0], xf[..., 1]
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    return torch.stack((a * c - b * s, a * s + b * c), dim=-1).flatten(-2).type_as(x)


class CausalSelfAttention(nn.Module):
    """baseline.py:31-70."""

    def __init__(self, d_model: int, n_heads: int, dropout: float = 0.0):
        super().__init__()
        assert d_model % n_heads == 0
        self.d_model = d_model
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.wq = nn.Linear(d_model, d_model, bias=False)
        self.wk = nn.Linear(d_model, d_model, bias=False)
        self.wv = nn.Linear(d_model, d_model, bias=False)
        self.wo = nn.Linear(d_model, d_model, bias=False)
        self.resid_dropout = nn.Dropout(dropout)

    def forward(self, x, cos, sin):
        B, L, D = x.shape
        shape = (B, L, self.n_heads, self.head_dim)
        q = rotate(self.wq(x).view(shape), cos, sin).transpose(1, 2)
        k = rotate(self.wk(x).view(shape), cos, sin).transpose(1, 2)
        v = self.wv(x).view(shape).transpose(1, 2)
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True,
                                             dropout_p=self.resid_dropout.p if self.training else 0.0)
        return self.resid_dropout(self.wo(out.transpose(1, 2).reshape(B, L, D)))


class RoPETransformerBlock(nn.Module):
    """baseline.py:72-84."""

    def __init__(self, d_model: int, n_heads: int, d_ff: int, dropout: float = 0.0):
        super().__init__()
        self.attn_norm = RMSNorm(d_model)
        self.attn = CausalSelfAttention(d_model, n_heads, dropout)
        self.ffn_norm = RMSNorm(d_model)
        self.ffn = SwiGLU(d_model, d_ff)

    def forward(self, x, cos, sin):
        x = x + self.attn(self.attn_norm(x), cos, sin)
        return x + self.ffn(self.ffn_norm(x))


class RoPETransformerLM(nn.Module):
    """baseline.py:86-129: RoPETransformerLM(vocab_size, d_model, n_layers, n_heads,
    max_seq_len=4096, dropout=0.1); forward(x [B, L]) -> logits [B, L, vocab_size]."""

    def __init__(self, vocab_size: int, d_model: int, n_layers: int, n_heads: int,
                 max_seq_len: int = 4096, dropout: float = 0.1):
        super().__init__()
        self.vocab_size = vocab_size
        self.d_model = d_model
        self.embed = nn.Embedding(vocab_size, d_model)
        d_ff = 256 * ((int(8 * d_model / 3) + 255) // 256)
        self.layers = nn.ModuleList([RoPETransformerBlock(d_model, n_heads, d_ff, dropout)
                                     for _ in range(n_layers)])
        self.final_norm = RMSNorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        self.lm_head.weight = self.embed.weight
        cos, sin = rotary_tables(d_model // n_heads, max_seq_len)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)

    def forward(self, x):
        L = x.shape[1]
        cos, sin = self.rope_cos[:L], self.rope_sin[:L]
        h = self.embed(x)
        for layer in self.layers:
            h = layer(h, cos, sin)
        return self.lm_head(self.final_norm(h))
