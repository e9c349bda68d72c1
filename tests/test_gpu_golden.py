"""The HIP path against the committed fixtures of tests/golden/: the reference's scan known
answers, and the seeded scan and attention cases (expected outputs from the exact oracle).
Tolerances: scans 1e-5 relative per element; attention outputs and gradients 2e-2
norm-wise (max|d| / max|ref|) against the exact float64 oracle, as for the bf16 class."""
import os

import numpy as np
import pytest
import torch

from test_golden import GOLD, _normwise, check_kats, load_kats

pytestmark = pytest.mark.gpu


def _hip_scan(x, rhos, V, c_init=None, keys=None, doc=None):
    from mathbrain_amd.ema_query import compute_query_ema_history
    cu = lambda a: None if a is None else torch.as_tensor(a).cuda()
    return compute_query_ema_history(cu(x), cu(rhos), V, cu(c_init), cu(keys), cu(doc)).cpu().numpy()


def test_gpu_reference_kats():
    from test_golden import kat_scan
    for case in load_kats():
        check_kats(kat_scan(case, _hip_scan), case)


def test_gpu_scan_fixture():
    from mathbrain_amd.flash_ema import precompute_boundaries
    f = np.load(os.path.join(GOLD, "scan_small.npz"))
    C = _hip_scan(f["x"], f["rhos"], int(f["x"].max()) + 1, f["c_init"], f["keys"], f["doc"])
    np.testing.assert_allclose(C, f["C_seq"], rtol=1e-5, atol=1e-30)
    cu = lambda a: torch.as_tensor(a).cuda()
    Cb = precompute_boundaries(cu(f["x"]), cu(f["unique"]), cu(f["rhos"]), 64, cu(f["c_init"]))
    N = f["rhos"].shape[0]
    np.testing.assert_allclose(Cb.cpu().numpy()[..., :N], f["C_bounds"], rtol=1e-5, atol=1e-30)


def test_gpu_attention_fixture():
    from mathbrain_amd.flash_ema import flash_ema_backward, flash_ema_forward, precompute_boundaries
    f = {k: torch.from_numpy(v).cuda() for k, v in np.load(os.path.join(GOLD, "attention_small.npz")).items()}
    V = int(f["V"])
    K = f["unique"].shape[1]
    Cb = precompute_boundaries(f["x"], f["unique"], f["rhos"], 64, f["c_base"])
    O, LSE, *_ = flash_ema_forward(f["Q"], f["x"], f["E_k"], f["E_v"], f["W"], f["rhos"], V,
                                   f["unique"], K, Cb)
    assert _normwise(O.cpu(), f["O"].cpu()) < 2e-2
    assert _normwise(LSE.cpu(), f["LSE"].cpu()) < 2e-2
    grads = flash_ema_backward(f["Q"], f["x"], f["E_k"], f["E_v"], f["W"], f["rhos"], V, f["unique"],
                               Cb, O, LSE, f["dO"])
    for name, g in zip(("dQ", "dE_k", "dE_v", "dW"), grads):
        assert _normwise(g.cpu(), f[name].cpu()) < 2e-2, name
