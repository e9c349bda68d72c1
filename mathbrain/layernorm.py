"""LayerNorm on the gfx950 kernels of mb_layernorm_fwd / mb_layernorm_bwd.

``layer_norm(x, weight, bias, eps)`` is ``F.layer_norm(x, (D,), weight, bias, eps)`` over
the last dimension, in fp32 with one read of each row forward and backward; the model uses
it for ln_kv over the slot embeddings (mathbrain/model.py:63-64), where torch's LayerNorm
kernels and the fp32 output under autocast are the reference's.  CPU tensors raise
NotImplementedError: there is no CPU path.  Both directions are registered as torch ops
(mathbrain::layernorm_fwd / layernorm_bwd) for tracing.
"""
import torch

from . import _lib


def _rows_f32(x, D):
    return x.detach().to(torch.float32).contiguous().view(-1, D)


def _fwd_fake(x, weight, bias, eps):
    rows = x.numel() // x.shape[-1]
    stat = x.new_empty((rows,), dtype=torch.float32)
    return x.new_empty(x.shape, dtype=torch.float32), stat, stat.new_empty((rows,))


@_lib.traced_op("layernorm_fwd", _fwd_fake)
def layernorm_fwd(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                  eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y fp32, mean, rstd) of LayerNorm over the last dimension."""
    dev = _lib.require_gpu(x, weight, bias, what="LayerNorm")
    D = x.shape[-1]
    if weight.shape != (D,) or bias.shape != (D,):
        raise ValueError(f"LayerNorm: weight {tuple(weight.shape)} / bias {tuple(bias.shape)} "
                         f"do not match the last dim {D}")
    xf = _rows_f32(x, D)
    w = weight.detach().to(torch.float32).contiguous()
    b = bias.detach().to(torch.float32).contiguous()
    rows = xf.shape[0]
    y = torch.empty(x.shape, dtype=torch.float32, device=dev)
    mean = torch.empty(rows, dtype=torch.float32, device=dev)
    rstd = torch.empty(rows, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_layernorm_fwd", _lib.ptr(xf), _lib.ptr(w), _lib.ptr(b), rows, D,
                  float(eps), _lib.ptr(y), _lib.ptr(mean), _lib.ptr(rstd), _lib.stream(dev))
    return y, mean, rstd


def _bwd_fake(x, weight, bias, dy, mean, rstd):
    return x.new_empty(x.shape), weight.new_empty(weight.shape), bias.new_empty(bias.shape)


@_lib.traced_op("layernorm_bwd", _bwd_fake)
def layernorm_bwd(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, dy: torch.Tensor,
                  mean: torch.Tensor, rstd: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dx, dw, db) of layernorm_fwd for the output gradient dy."""
    dev = x.device
    D = x.shape[-1]
    xf = _rows_f32(x, D)
    w = weight.detach().to(torch.float32).contiguous()
    rows = xf.shape[0]
    g = dy.to(torch.float32).contiguous().view(rows, D)
    dx = torch.empty(x.shape, dtype=torch.float32, device=dev)
    dw = torch.empty(D, dtype=torch.float32, device=dev)
    db = torch.empty(D, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_layernorm_bwd", _lib.ptr(xf), _lib.ptr(w), _lib.ptr(g), _lib.ptr(mean),
                  _lib.ptr(rstd), rows, D, _lib.ptr(dx), _lib.ptr(dw), _lib.ptr(db),
                  _lib.stream(dev))
    return dx.to(x.dtype), dw.to(weight.dtype), db.to(bias.dtype)


class LayerNormFunction(torch.autograd.Function):
    """autograd for LayerNorm over the last dimension: gradients for x, weight and bias."""

    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        y, mean, rstd = layernorm_fwd(x, weight, bias, float(eps))
        ctx.save_for_backward(x, weight, bias, mean, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, bias, mean, rstd = ctx.saved_tensors
        dx, dw, db = layernorm_bwd(x, weight, bias, dy, mean, rstd)
        return dx, dw, db, None


def layer_norm(x, weight, bias, eps):
    """F.layer_norm over the last dimension on the GPU kernels (fp32 output)."""
    if x.device.type != "cuda":
        raise NotImplementedError("LayerNorm: tensors must be on an MI355X GPU; this "
                                  "implementation has no CPU path")
    D = x.shape[-1]
    if weight is None:
        weight = torch.ones(D, device=x.device)
    if bias is None:
        bias = torch.zeros(D, device=x.device)
    return LayerNormFunction.apply(x, weight, bias, eps)
