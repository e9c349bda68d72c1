"""RMSNorm on the HIP kernels (mb_rmsnorm_fwd / mb_rmsnorm_bwd behind
mathbrain/rmsnorm.py) against the reference's expression
weight * (x * rsqrt(mean(x^2) + eps)) (mathbrain/model.py:17-19) evaluated by torch autograd
in float64: output, dx and dweight, norm-wise (max |diff| / max |ref|) within 1e-5 (fp32
kernels), at widths below, at and between the 64-lane tiles, ragged row counts and the
model's shape.  (At D = 1 the row is normalised to sign(x) and dx is a cancellation of two
O(1) terms down to ~1e-8, where a relative bar is meaningless; the smallest width is 3.)"""
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 1e-5


def rel(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / b.abs().max().clamp(min=1e-300))


def reference(x, w, eps):
    variance = x.pow(2).mean(-1, keepdim=True)
    return w * (x * torch.rsqrt(variance + eps))


@pytest.mark.parametrize("shape", [(5, 3), (3, 63), (7, 64), (2, 3, 100), (9, 128), (4, 7, 512),
                                   (6, 1000), (5, 1024), (56 * 16, 512)])
def test_rmsnorm_matches_reference_expression(shape):
    from mathbrain.rmsnorm import rms_norm
    g = torch.Generator().manual_seed(sum(shape))
    D = shape[-1]
    x = torch.randn(*shape, generator=g, dtype=torch.float64) * 3
    w = 1 + 0.5 * torch.randn(D, generator=g, dtype=torch.float64)
    dy = torch.randn(*shape, generator=g, dtype=torch.float64)
    eps = 1e-6
    xr, wr = x.clone().requires_grad_(), w.clone().requires_grad_()
    want = reference(xr, wr, eps)
    want.backward(dy)
    xg = x.float().cuda().requires_grad_()
    wg = w.float().cuda().requires_grad_()
    got = rms_norm(xg, wg, eps)
    got.backward(dy.float().cuda())
    print(f"rmsnorm {shape}", flush=True)
    assert got.dtype == torch.float32 and got.shape == x.shape
    assert rel(got, want) < TOL
    assert rel(xg.grad, xr.grad) < TOL
    assert rel(wg.grad, wr.grad) < TOL


def test_rmsnorm_tiny_values_use_eps():
    # rows of zeros: rstd = eps^-1/2, y = 0, dx = rstd * w * dy
    from mathbrain.rmsnorm import rms_norm
    x = torch.zeros(3, 128, device="cuda", requires_grad=True)
    w = torch.full((128,), 2.0, device="cuda", requires_grad=True)
    y = rms_norm(x, w, 1e-6)
    dy = torch.ones(3, 128, device="cuda")
    y.backward(dy)
    assert torch.count_nonzero(y) == 0
    assert torch.allclose(x.grad, torch.full_like(x, 2.0 * 1e3), rtol=1e-5)
    assert torch.count_nonzero(w.grad) == 0


def test_rmsnorm_rejects_wide_rows_and_cpu_tensors():
    from mathbrain import _lib
    from mathbrain.rmsnorm import rms_norm
    with pytest.raises(_lib.HipKernelError):
        rms_norm(torch.randn(2, 1025, device="cuda"), torch.ones(1025, device="cuda"), 1e-6)
    with pytest.raises(NotImplementedError):
        rms_norm(torch.randn(2, 8), torch.ones(8), 1e-6)
