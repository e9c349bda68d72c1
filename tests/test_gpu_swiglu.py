"""SwiGLU's gate product on the HIP kernels (mb_swiglu_fwd / mb_swiglu_bwd behind
mathbrain/swiglu.py) against the reference's F.silu(a) * b (mathbrain/model.py:21-29)
evaluated by torch autograd in float64 on the same input values: output and both input
gradients, norm-wise (max |diff| / max |ref|).  fp32 inputs: 1e-6.  bf16 inputs (autocast):
the kernels evaluate in fp32 and round once to bf16, so the bar is bf16's rounding, 8e-3
(2 ulp of the largest element).  Sizes cover the 8-element vector edge and a grid-stride
walk."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / b.abs().max().clamp(min=1e-300))


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.bfloat16, 8e-3)])
@pytest.mark.parametrize("shape", [(1,), (7,), (3, 9), (5, 1536), (4096, 1537)])
def test_swiglu_product_matches_reference(shape, dtype, tol):
    from mathbrain.swiglu import swiglu_product
    g = torch.Generator().manual_seed(len(shape) * 100 + shape[-1])
    a = (torch.randn(*shape, generator=g) * 3).to(dtype)
    b = torch.randn(*shape, generator=g).to(dtype)
    dm = torch.randn(*shape, generator=g).to(dtype)
    ar = a.double().requires_grad_()
    br = b.double().requires_grad_()
    want = F.silu(ar) * br
    want.backward(dm.double())
    ag = a.cuda().requires_grad_()
    bg = b.cuda().requires_grad_()
    got = swiglu_product(ag, bg)
    got.backward(dm.cuda())
    print(f"swiglu {shape} {dtype}", flush=True)
    assert got.dtype == dtype and ag.grad.dtype == dtype and bg.grad.dtype == dtype
    assert rel(got, want) < tol
    assert rel(ag.grad, ar.grad) < tol
    assert rel(bg.grad, br.grad) < tol


def test_swiglu_empty_and_cpu():
    from mathbrain.swiglu import swiglu_product
    e = torch.empty(0, 16, device="cuda")
    assert swiglu_product(e, e).shape == (0, 16)
    with pytest.raises(NotImplementedError):
        swiglu_product(torch.randn(4), torch.randn(4))


def test_swiglu_offset_views():
    # contiguous views that start 1 element into their storage (not 32-byte aligned)
    from mathbrain.swiglu import swiglu_product
    g = torch.Generator().manual_seed(5)
    base_a = torch.randn(1 + 40 * 24, generator=g).to(torch.bfloat16)
    base_b = torch.randn(1 + 40 * 24, generator=g).to(torch.bfloat16)
    a, b = base_a[1:].view(40, 24), base_b[1:].view(40, 24)
    want = F.silu(a.double()) * b.double()
    got = swiglu_product(a.cuda()[0:], b.cuda()[0:])
    ga = base_a.cuda()[1:].view(40, 24)
    gb = base_b.cuda()[1:].view(40, 24)
    got2 = swiglu_product(ga, gb)
    assert rel(got, want) < 8e-3 and rel(got2, want) < 8e-3
