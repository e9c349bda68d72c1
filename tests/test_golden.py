"""The oracle against the committed fixtures of tests/golden/ (written by
tests/golden/make_golden.py): the reference's own scan known answers, and seeded scan,
attention, data-pipeline and factored cases whose expected outputs pin the oracle against
regressions."""
import json
import os

import numpy as np
import torch

from oracle import attention as att
from oracle import scan as oscan

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_kats():
    with open(os.path.join(GOLD, "reference_kats.json")) as fh:
        return json.load(fh)


def kat_scan(case, fn):
    arr = lambda k, dt: None if k not in case else np.array(case[k], dtype=dt)
    return fn(arr("x", np.int64), np.array(case["rhos"], np.float32), case["V"],
              arr("c_init", np.float32), arr("keys", np.int64), arr("doc", np.int64))


def check_kats(C, case):
    for pos, want in case["expect"].items():
        b, t = (int(v) for v in pos.split(","))
        np.testing.assert_allclose(np.asarray(C)[b, t], want, rtol=1e-6, atol=1e-7,
                                   err_msg=f"{case['source']} at {pos}")


def test_oracle_reproduces_reference_kats():
    for case in load_kats():
        check_kats(kat_scan(case, oscan.query_scan), case)


def test_oracle_reproduces_scan_fixture():
    f = np.load(os.path.join(GOLD, "scan_small.npz"))
    C = oscan.query_scan(f["x"], f["rhos"], int(f["x"].max()) + 1, f["c_init"], f["keys"], f["doc"])
    np.testing.assert_allclose(C, f["C_seq"], rtol=1e-6, atol=1e-30)
    Cb = oscan.boundary_states(f["x"], f["unique"], f["rhos"], 64, f["c_init"])
    np.testing.assert_allclose(Cb, f["C_bounds"], rtol=1e-6, atol=1e-30)


def _normwise(a, b):
    a = torch.as_tensor(a, dtype=torch.float64)
    b = torch.as_tensor(b, dtype=torch.float64)
    return float((a - b).abs().max() / b.abs().max())


def test_oracle_reproduces_attention_fixture():
    f = {k: torch.from_numpy(v) for k, v in np.load(os.path.join(GOLD, "attention_small.npz")).items()}
    d = torch.float64
    V = int(f["V"])
    O, LSE = att.sparse(f["Q"].to(d), f["x"], f["E_k"].to(d), f["E_v"].to(d), f["W"].to(d),
                        f["rhos"].to(d), V, f["unique"], f["c_base"].to(d), return_lse=True)
    assert _normwise(O, f["O"]) < 1e-6 and _normwise(LSE, f["LSE"]) < 1e-6
    grads = att.sparse_backward_formulas(f["Q"].to(d), f["x"], f["E_k"].to(d), f["E_v"].to(d),
                                         f["W"].to(d), f["rhos"].to(d), V, f["unique"],
                                         f["dO"].to(d), f["c_base"].to(d))
    for name, g in zip(("dQ", "dE_k", "dE_v", "dW"), grads):
        assert _normwise(g, f[name]) < 1e-6, name


def test_oracle_reproduces_data_fixture():
    from oracle import data as od
    f = np.load(os.path.join(GOLD, "data_small.npz"))
    states, pos = od.corpus_states(f["tokens"], f["doc_ids"], f["rhos"])
    np.testing.assert_allclose(states, f["states"], rtol=1e-6, atol=1e-30)
    chunks, starts = od.chunk_index(f["doc_ids"], int(f["block"]))
    assert np.array_equal(np.array(chunks, np.int64), f["chunks_index"])
    items = [od.get_item(f["tokens"], f["doc_ids"], states, pos, starts, chunks[i], f["rhos"])
             for i in f["batch"]]
    ch, us, pm, inv, cb, K, dd = od.collate(items)
    for name, got in (("chunks", ch), ("unique_slots", us), ("pad_mask", pm), ("inverse", inv),
                      ("doc_out", dd)):
        assert np.array_equal(got, f[name]), name
    assert K == int(f["K_max"])
    np.testing.assert_allclose(cb, f["c_base"], rtol=1e-6, atol=1e-30)


def test_oracle_reproduces_factored_fixture():
    from oracle import factored as of
    f = {k: torch.from_numpy(v) for k, v in np.load(os.path.join(GOLD, "factored_small.npz")).items()}
    d = torch.float64
    leaves = [f[k].to(d).requires_grad_(True) for k in ("Q", "E_k", "E_v", "W")]
    O = of.closed_form(leaves[0], f["x"], leaves[1], leaves[2], f["rhos"].to(d), leaves[3],
                       int(f["H"]), c_base=f["c_base"].to(d), unique_slots=f["unique"],
                       pad_mask=f["unique"] >= 0)
    O.backward(f["dO"].to(d))
    assert _normwise(O, f["O"]) < 1e-6
    for name, leaf in zip(("dQ", "dE_k", "dE_v", "dW"), leaves):
        assert _normwise(leaf.grad, f[name]) < 1e-6, name
