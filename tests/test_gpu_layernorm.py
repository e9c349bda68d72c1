"""LayerNorm on the HIP kernels (mb_layernorm_fwd / mb_layernorm_bwd behind
mathbrain/layernorm.py, the model's ln_kv) against F.layer_norm evaluated by torch
autograd in float64: output, dx, dweight and dbias, norm-wise (max |diff| / max |ref|)
within 1e-5 (fp32 kernels), at widths around the 64-lane tiles, ragged row counts and the
model's vocabulary-table shape."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

TOL = 1e-5


def rel(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / b.abs().max().clamp(min=1e-300))


@pytest.mark.parametrize("shape", [(5, 3), (3, 63), (7, 64), (2, 3, 100), (9, 128), (6, 1000),
                                   (5, 1024), (50257, 512)])
def test_layernorm_matches_torch_float64(shape):
    from mathbrain.layernorm import layer_norm
    g = torch.Generator().manual_seed(sum(shape))
    D = shape[-1]
    x = torch.randn(*shape, generator=g, dtype=torch.float64) * 2 + 0.5
    w = 1 + 0.3 * torch.randn(D, generator=g, dtype=torch.float64)
    b = 0.1 * torch.randn(D, generator=g, dtype=torch.float64)
    dy = torch.randn(*shape, generator=g, dtype=torch.float64)
    xr, wr, br = (t.clone().requires_grad_() for t in (x, w, b))
    want = F.layer_norm(xr, (D,), wr, br, 1e-5)
    want.backward(dy)
    xg, wg, bg = (t.float().cuda().requires_grad_() for t in (x, w, b))
    got = layer_norm(xg, wg, bg, 1e-5)
    got.backward(dy.float().cuda())
    print(f"layernorm {shape}", flush=True)
    assert got.dtype == torch.float32 and got.shape == x.shape
    assert rel(got, want) < TOL
    assert rel(xg.grad, xr.grad) < TOL
    assert rel(wg.grad, wr.grad) < TOL
    assert rel(bg.grad, br.grad) < TOL


def test_layernorm_rejects_wide_rows_and_cpu_tensors():
    from mathbrain import _lib
    from mathbrain.layernorm import layer_norm
    with pytest.raises(_lib.HipKernelError):
        layer_norm(torch.randn(2, 1025, device="cuda"), torch.ones(1025, device="cuda"),
                   torch.zeros(1025, device="cuda"), 1e-5)
    with pytest.raises(NotImplementedError):
        layer_norm(torch.randn(2, 8), torch.ones(8), torch.zeros(8), 1e-5)
