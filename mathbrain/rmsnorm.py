"""RMSNorm on the gfx950 kernels of mb_rmsnorm_fwd / mb_rmsnorm_bwd.

``RMSNormFunction.apply(x, weight, eps)`` computes the reference's
``weight * (x * rsqrt(mean(x^2, -1) + eps))`` (mathbrain/model.py:11-19) in fp32 with one
read of each row forward and backward, in place of the pow / mean / rsqrt / multiply graph
torch builds from the reference's module.  The output has the dtype the reference's
expression would promote to (fp32 for an fp32 weight).  CPU tensors raise
NotImplementedError: there is no CPU path.  Both directions are registered as torch ops
(mathbrain::rmsnorm_fwd / rmsnorm_bwd) for tracing.
"""
import torch

from . import _lib


def _rows_f32(x, D):
    return x.detach().to(torch.float32).contiguous().view(-1, D)


def _fwd_fake(x, weight, eps):
    rows = x.numel() // x.shape[-1]
    return (x.new_empty(x.shape, dtype=torch.result_type(weight, x)),
            x.new_empty((rows,), dtype=torch.float32))


@_lib.traced_op("rmsnorm_fwd", _fwd_fake)
def rmsnorm_fwd(x: torch.Tensor, weight: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(y, rstd): y = weight * x * rstd with rstd = rsqrt(mean(x^2) + eps) per row."""
    dev = _lib.require_gpu(x, weight, what="RMSNorm")
    D = x.shape[-1]
    if weight.shape != (D,):
        raise ValueError(f"RMSNorm: weight {tuple(weight.shape)} does not match the last dim {D}")
    xf = _rows_f32(x, D)
    w = weight.detach().to(torch.float32).contiguous()
    rows = xf.shape[0]
    y = torch.empty(x.shape, dtype=torch.float32, device=dev)
    rstd = torch.empty(rows, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_rmsnorm_fwd", _lib.ptr(xf), _lib.ptr(w), rows, D, float(eps),
                  _lib.ptr(y), _lib.ptr(rstd), _lib.stream(dev))
    return y.to(torch.result_type(weight, x)), rstd


def _bwd_fake(x, weight, dy, rstd):
    return x.new_empty(x.shape), weight.new_empty(weight.shape)


@_lib.traced_op("rmsnorm_bwd", _bwd_fake)
def rmsnorm_bwd(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor,
                rstd: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(dx, dw) of rmsnorm_fwd for the output gradient dy."""
    dev = x.device
    D = x.shape[-1]
    xf = _rows_f32(x, D)
    w = weight.detach().to(torch.float32).contiguous()
    rows = xf.shape[0]
    g = dy.to(torch.float32).contiguous().view(rows, D)
    dx = torch.empty(x.shape, dtype=torch.float32, device=dev)
    dw = torch.empty(D, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_rmsnorm_bwd", _lib.ptr(xf), _lib.ptr(w), _lib.ptr(g), _lib.ptr(rstd),
                  rows, D, _lib.ptr(dx), _lib.ptr(dw), _lib.stream(dev))
    return dx.to(x.dtype), dw.to(weight.dtype)


class RMSNormFunction(torch.autograd.Function):
    """autograd for RMSNorm: gradients for x and weight."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        y, rstd = rmsnorm_fwd(x, weight, float(eps))
        ctx.save_for_backward(x, weight, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, rstd = ctx.saved_tensors
        dx, dw = rmsnorm_bwd(x, weight, dy, rstd)
        return dx, dw, None


def rms_norm(x, weight, eps):
    """weight * (x * rsqrt(mean(x^2, -1) + eps)) on the GPU kernels (model.py:17-19)."""
    if x.device.type != "cuda":
        raise NotImplementedError("RMSNorm: tensors must be on an MI355X GPU; this "
                                  "implementation has no CPU path")
    return RMSNormFunction.apply(x, weight, eps)
