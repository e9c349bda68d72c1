"""RMSNorm on the gfx950 kernels of mb_rmsnorm_fwd / mb_rmsnorm_bwd.

``RMSNormFunction.apply(x, weight, eps)`` computes the reference's
``weight * (x * rsqrt(mean(x^2, -1) + eps))`` (mathbrain/model.py:11-19) in fp32 with one
read of each row forward and backward, in place of the pow / mean / rsqrt / multiply graph
torch builds from the reference's module.  The output has the dtype the reference's
expression would promote to (fp32 for an fp32 weight).  CPU tensors raise
NotImplementedError: there is no CPU path.
"""
import torch

from . import _lib


class RMSNormFunction(torch.autograd.Function):
    """autograd for RMSNorm: gradients for x and weight."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        dev = _lib.require_gpu(x, weight, what="RMSNorm")
        D = x.shape[-1]
        if weight.shape != (D,):
            raise ValueError(f"RMSNorm: weight {tuple(weight.shape)} does not match the last dim {D}")
        xf = x.detach().to(torch.float32).contiguous().view(-1, D)
        w = weight.detach().to(torch.float32).contiguous()
        rows = xf.shape[0]
        y = torch.empty_like(xf)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            _lib.call("mb_rmsnorm_fwd", _lib.ptr(xf), _lib.ptr(w), rows, D, float(eps),
                      _lib.ptr(y), _lib.ptr(rstd), _lib.stream(dev))
        ctx.save_for_backward(xf, w, rstd)
        ctx.shape = x.shape
        ctx.dtypes = (x.dtype, weight.dtype)
        return y.view(x.shape).to(torch.result_type(weight, x))

    @staticmethod
    def backward(ctx, dy):
        xf, w, rstd = ctx.saved_tensors
        rows, D = xf.shape
        dev = xf.device
        g = dy.to(torch.float32).contiguous().view(rows, D)
        dx = torch.empty_like(xf)
        dw = torch.empty(D, dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            _lib.call("mb_rmsnorm_bwd", _lib.ptr(xf), _lib.ptr(w), _lib.ptr(g), _lib.ptr(rstd),
                      rows, D, _lib.ptr(dx), _lib.ptr(dw), _lib.stream(dev))
        xd, wd = ctx.dtypes
        return dx.view(ctx.shape).to(xd), dw.to(wd), None


def rms_norm(x, weight, eps):
    """weight * (x * rsqrt(mean(x^2, -1) + eps)) on the GPU kernels (model.py:17-19)."""
    if x.device.type != "cuda":
        raise NotImplementedError("RMSNorm: tensors must be on an MI355X GPU; this "
                                  "implementation has no CPU path")
    return RMSNormFunction.apply(x, weight, eps)
