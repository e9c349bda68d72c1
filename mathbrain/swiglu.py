"""SwiGLU's gate product on the gfx950 kernels of mb_swiglu_fwd / mb_swiglu_bwd.

``swiglu_product(a, b)`` is ``F.silu(a) * b`` (mathbrain/model.py:21-29, with a = w1(x) and
b = w3(x)) in one pass forward and one backward, evaluated in fp32 and rounded once to the
inputs' dtype (fp32, or bf16 under autocast), in place of torch's separate SiLU and multiply
passes and their backwards.  CPU tensors raise NotImplementedError: there is no CPU path.
Both directions are registered as torch ops (mathbrain::swiglu_fwd / swiglu_bwd).
"""
import torch

from . import _lib

_DTYPES = {torch.float32: _lib.MB_DTYPE_F32, torch.bfloat16: _lib.MB_DTYPE_BF16}


def _aligned(t):
    """Contiguous, and 32-byte aligned for the kernels' vector loads (a contiguous view with
    a storage offset may not be)."""
    t = t.contiguous()
    return t if t.data_ptr() % 32 == 0 else t.clone()


def _common(a, b):
    dt = torch.promote_types(a.dtype, b.dtype)
    if dt not in _DTYPES:
        dt = torch.float32
    return dt


def _fwd_fake(a, b):
    return a.new_empty(a.shape, dtype=_common(a, b))


@_lib.traced_op("swiglu_fwd", _fwd_fake)
def swiglu_fwd(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """silu(a) * b in the promoted dtype of a and b (fp32 or bf16)."""
    dev = _lib.require_gpu(a, b, what="SwiGLU")
    if a.shape != b.shape:
        raise ValueError(f"SwiGLU: a {tuple(a.shape)} and b {tuple(b.shape)} differ")
    dt = _common(a, b)
    ac = _aligned(a.detach().to(dt))
    bc = _aligned(b.detach().to(dt))
    m = torch.empty_like(ac)
    with torch.cuda.device(dev):
        _lib.call("mb_swiglu_fwd", _lib.ptr(ac), _lib.ptr(bc), ac.numel(), _DTYPES[dt],
                  _lib.ptr(m), _lib.stream(dev))
    return m


def _bwd_fake(a, b, dm):
    return a.new_empty(a.shape), b.new_empty(b.shape)


@_lib.traced_op("swiglu_bwd", _bwd_fake)
def swiglu_bwd(a: torch.Tensor, b: torch.Tensor, dm: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(da, db) of swiglu_fwd for the output gradient dm, in the dtypes of a and b."""
    dev = a.device
    dt = _common(a, b)
    ac = _aligned(a.detach().to(dt))
    bc = _aligned(b.detach().to(dt))
    g = _aligned(dm.to(dt))
    da = torch.empty_like(ac)
    db = torch.empty_like(bc)
    with torch.cuda.device(dev):
        _lib.call("mb_swiglu_bwd", _lib.ptr(ac), _lib.ptr(bc), _lib.ptr(g), ac.numel(),
                  _DTYPES[dt], _lib.ptr(da), _lib.ptr(db), _lib.stream(dev))
    return da.to(a.dtype), db.to(b.dtype)


class SwiGLUProductFunction(torch.autograd.Function):
    """autograd for silu(a) * b: gradients for a and b."""

    @staticmethod
    def forward(ctx, a, b):
        m = swiglu_fwd(a, b)
        ctx.save_for_backward(a, b)
        return m

    @staticmethod
    def backward(ctx, dm):
        a, b = ctx.saved_tensors
        return swiglu_bwd(a, b, dm)


def swiglu_product(a, b):
    """F.silu(a) * b on the GPU kernels."""
    if a.device.type != "cuda":
        raise NotImplementedError("SwiGLU: tensors must be on an MI355X GPU; this "
                                  "implementation has no CPU path")
    return SwiGLUProductFunction.apply(a, b)
