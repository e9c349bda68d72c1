"""LayerNorm on the gfx950 kernels of mb_layernorm_fwd / mb_layernorm_bwd.

``layer_norm(x, weight, bias, eps)`` is ``F.layer_norm(x, (D,), weight, bias, eps)`` over
the last dimension, in fp32 with one read of each row forward and backward; the model uses
it for ln_kv over the slot embeddings (mathbrain/model.py:63-64), where torch's LayerNorm
kernels and the fp32 output under autocast are the reference's.  CPU tensors raise
NotImplementedError: there is no CPU path.
"""
import torch

from . import _lib


class LayerNormFunction(torch.autograd.Function):
    """autograd for LayerNorm over the last dimension: gradients for x, weight and bias."""

    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        dev = _lib.require_gpu(x, weight, bias, what="LayerNorm")
        D = x.shape[-1]
        if weight.shape != (D,) or bias.shape != (D,):
            raise ValueError(f"LayerNorm: weight {tuple(weight.shape)} / bias {tuple(bias.shape)} "
                             f"do not match the last dim {D}")
        xf = x.detach().to(torch.float32).contiguous().view(-1, D)
        w = weight.detach().to(torch.float32).contiguous()
        b = bias.detach().to(torch.float32).contiguous()
        rows = xf.shape[0]
        y = torch.empty_like(xf)
        mean = torch.empty(rows, dtype=torch.float32, device=dev)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            _lib.call("mb_layernorm_fwd", _lib.ptr(xf), _lib.ptr(w), _lib.ptr(b), rows, D,
                      float(eps), _lib.ptr(y), _lib.ptr(mean), _lib.ptr(rstd), _lib.stream(dev))
        ctx.save_for_backward(xf, w, mean, rstd)
        ctx.shape = x.shape
        ctx.dtypes = (x.dtype, weight.dtype, bias.dtype)
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        xf, w, mean, rstd = ctx.saved_tensors
        rows, D = xf.shape
        dev = xf.device
        g = dy.to(torch.float32).contiguous().view(rows, D)
        dx = torch.empty_like(xf)
        dw = torch.empty(D, dtype=torch.float32, device=dev)
        db = torch.empty(D, dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            _lib.call("mb_layernorm_bwd", _lib.ptr(xf), _lib.ptr(w), _lib.ptr(g), _lib.ptr(mean),
                      _lib.ptr(rstd), rows, D, _lib.ptr(dx), _lib.ptr(dw), _lib.ptr(db),
                      _lib.stream(dev))
        xd, wd, bd = ctx.dtypes
        return dx.view(ctx.shape).to(xd), dw.to(wd), db.to(bd), None


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
