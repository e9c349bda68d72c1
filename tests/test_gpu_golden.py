"""The HIP path against the committed fixtures of tests/golden/: the reference's scan known
answers, and the seeded scan, attention, data-pipeline and factored cases (expected outputs
from the exact oracle).  Tolerances: scans, states and c_base 1e-5 relative per element
(ids and masks exact); attention outputs and gradients 2e-2 norm-wise (max|d| / max|ref|)
against the exact float64 oracle, as for the bf16 class; the fp32 factored EMA 1e-4."""
import os

import numpy as np
import pytest
import torch

from test_golden import GOLD, _normwise, check_kats, load_kats

pytestmark = pytest.mark.gpu


def _hip_scan(x, rhos, V, c_init=None, keys=None, doc=None):
    from mathbrain.triton_ema_query import compute_query_ema_history
    cu = lambda a: None if a is None else torch.as_tensor(a).cuda()
    return compute_query_ema_history(cu(x), cu(rhos), V, cu(c_init), cu(keys), cu(doc)).cpu().numpy()


def test_gpu_reference_kats():
    from test_golden import kat_scan
    for case in load_kats():
        check_kats(kat_scan(case, _hip_scan), case)


def test_gpu_scan_fixture():
    from mathbrain.triton_flash_ema import precompute_boundaries
    f = np.load(os.path.join(GOLD, "scan_small.npz"))
    C = _hip_scan(f["x"], f["rhos"], int(f["x"].max()) + 1, f["c_init"], f["keys"], f["doc"])
    np.testing.assert_allclose(C, f["C_seq"], rtol=1e-5, atol=1e-30)
    cu = lambda a: torch.as_tensor(a).cuda()
    Cb = precompute_boundaries(cu(f["x"]), cu(f["unique"]), cu(f["rhos"]), 64, cu(f["c_init"]))
    N = f["rhos"].shape[0]
    np.testing.assert_allclose(Cb.cpu().numpy()[..., :N], f["C_bounds"], rtol=1e-5, atol=1e-30)


def test_gpu_attention_fixture():
    from mathbrain.triton_flash_ema import flash_ema_backward, flash_ema_forward, precompute_boundaries
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


def test_gpu_data_fixture():
    # the device data pipeline against the committed corpus: states, chunk list, one batch
    import tempfile

    from mathbrain.data import WikiTextMMapDataset, corpus_states
    f = np.load(os.path.join(GOLD, "data_small.npz"))
    st = corpus_states(torch.from_numpy(f["tokens"]).cuda(), torch.from_numpy(f["doc_ids"]).cuda(),
                       torch.from_numpy(f["rhos"]).cuda())
    np.testing.assert_allclose(st.cpu().numpy(), f["states"], rtol=1e-5, atol=1e-30)
    d = tempfile.mkdtemp(prefix="mb_gold_")
    f["tokens"].tofile(os.path.join(d, "tokens.bin"))
    f["doc_ids"].tofile(os.path.join(d, "doc_ids.bin"))
    f["states"].astype(np.float32).tofile(os.path.join(d, "states.bin"))
    ds = WikiTextMMapDataset(d, block_size=int(f["block"]), rhos=torch.from_numpy(f["rhos"]))
    assert np.array_equal(np.array(ds.chunks, np.int64), f["chunks_index"])
    ch, us, pm, inv, cb, K, dd = ds.get_batch(f["batch"].tolist())
    for name, got in (("chunks", ch), ("unique_slots", us), ("pad_mask", pm), ("inverse", inv),
                      ("doc_out", dd)):
        assert np.array_equal(got.cpu().numpy(), f[name]), name
    assert K == int(f["K_max"])
    np.testing.assert_allclose(cb.cpu().numpy(), f["c_base"], rtol=1e-5, atol=1e-30)


def test_gpu_factored_fixture():
    from mathbrain.factored_ema import factored_ema_forward
    f = {k: torch.from_numpy(v).cuda() for k, v in np.load(os.path.join(GOLD, "factored_small.npz")).items()}
    leaves = [f[k].clone().requires_grad_(True) for k in ("Q", "E_k", "E_v", "W")]
    O = factored_ema_forward(leaves[0], f["x"], leaves[1], leaves[2], f["rhos"], leaves[3], int(f["H"]),
                             c_base=f["c_base"], unique_slots=f["unique"], pad_mask=f["unique"] >= 0)
    O.backward(f["dO"])
    assert _normwise(O.detach().cpu(), f["O"].cpu()) < 1e-4
    for name, leaf in zip(("dQ", "dE_k", "dE_v", "dW"), leaves):
        assert _normwise(leaf.grad.cpu(), f[name].cpu()) < 1e-4, name
