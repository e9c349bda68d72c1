"""Writes the committed fixtures of tests/golden/ (run from the repository root:
``python tests/golden/make_golden.py``).

* reference_kats.json -- the known answers the reference's own scan tests hold, as data:
  inputs, the positions they check and the expected rows (the closed forms those tests
  assert, evaluated in float64 at their rates), each with the test file:line it comes from.
* scan_small.npz -- a seeded query-scan case (doc_ids, c_init with a duplicate key and
  pads) and the key-side chunk states, with the oracle's outputs.
* attention_small.npz -- a seeded flash-EMA case (absent-slot mass, SiLU gate) with the
  exact float64 oracle's O, LSE and the reference-formula gradients for a seeded dO
  (stored as float32).
* data_small.npz -- a six-document corpus (one of length 1, one of length 2) with the
  oracle's states, chunk list (block 7) and one collated batch of six chunks.
* factored_small.npz -- a seeded factored linear EMA case with c_base and padding slots,
  with the float64 step-by-step oracle's output and gradients for a seeded dO.

The outputs come from this repository's oracle (oracle/), never from the reference; the
fixtures pin the oracle against regressions and give the GPU tests fixed expected values.
"""
import json
import math
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))


def kats():
    r2 = [0.9, 0.5]
    r4 = [0.9, 0.8, 0.7, 0.6]
    p = lambda r, e: [float(np.float64(np.float32(v)) ** e) for v in r]
    return [
        dict(source="tests/test_doc_boundary.py:71-105", x=[[0, 1, 0, 2, 0, 1]],
             doc=[[0] * 6], rhos=r2, V=3,
             expect={"0,0": [0.0, 0.0], "0,2": p(r2, 2),
                     "0,4": [(a + 1.0) * a for a in p(r2, 2)]}),
        dict(source="tests/test_doc_boundary.py:108-134", x=[[0, 1, 0, 2]], rhos=r2, V=3,
             doc=[[0] * 4], c_init=[[[2.0, 1.5], [0.0, 0.0], [0.0, 0.0]]], keys=[[0, 1, 2]],
             expect={"0,0": [2.0, 1.5],
                     "0,2": [(c + 1.0) * a for c, a in zip([2.0, 1.5], p(r2, 2))]}),
        dict(source="tests/test_doc_boundary.py:22-68", x=[[0, 1, 2, 0, 1, 0, 1, 3, 0, 1]],
             doc=[[0, 0, 0, 0, 0, 1, 1, 1, 1, 1]], rhos=r4, V=5,
             expect={"0,5": [0.0] * 4, "0,8": p(r4, 3)}),
        dict(source="tests/test_doc_boundary.py:244-277",
             x=[[0, 1, 2, 0, 1, 2, 0, 1], [0, 1, 2, 0, 0, 1, 2, 0]],
             doc=[[0] * 8, [0, 0, 0, 0, 1, 1, 1, 1]], rhos=r2, V=5,
             expect={"1,4": [0.0, 0.0]}),
    ]


def scan_case():
    from oracle import scan as oscan
    rng = np.random.default_rng(2024)
    B, L, V, N, K = 3, 200, 37, 12, 20
    x = rng.integers(0, V, size=(B, L))
    rhos = np.exp(-np.log(2.0) / np.logspace(0, math.log10(300), N)).astype(np.float32)
    keys = np.stack([rng.permutation(V)[:K] for _ in range(B)])
    keys[0, 5] = keys[0, 2]   # duplicate key: the later one wins
    keys[2, -4:] = -1         # padding keys
    c_init = (rng.random((B, K, N)) * 4).astype(np.float32)
    doc = np.sort(rng.integers(0, 3, size=(B, L)), axis=1)
    C = oscan.query_scan(x, rhos, V, c_init, keys, doc)
    unique = np.where(keys >= 0, keys, -1)
    Cb = oscan.boundary_states(x, unique, rhos, 64, c_init)
    return dict(x=x, rhos=rhos, keys=keys, c_init=c_init, doc=doc, C_seq=C, unique=unique,
                C_bounds=Cb)


def attention_case():
    from mathbrain.synthetic import make_batch
    from oracle import attention as att
    B, L, V, H, hd, N = 2, 40, 120, 4, 32, 16
    d = make_batch(B, L, V, N, 48, seed=77, min_hl=2.0, max_hl=256.0)
    g = torch.Generator().manual_seed(78)
    K = d["unique"].shape[1]
    D = H * hd
    Q = torch.randn(B, H, L, hd, generator=g)
    E_k = torch.randn(B, K, D, generator=g) * 0.5
    E_v = torch.randn(B, K, D, generator=g) * 0.5
    W = torch.randn(N, D, generator=g) * 0.3
    dO = torch.randn(B, H, L, hd, generator=g)
    f = torch.float64
    O, LSE = att.sparse(Q.to(f), d["x"], E_k.to(f), E_v.to(f), W.to(f), d["rhos"].to(f), V,
                        d["unique"], d["c_base"].to(f), use_silu=True, absent_mass=True,
                        return_lse=True)
    dQ, dEk, dEv, dW = att.sparse_backward_formulas(
        Q.to(f), d["x"], E_k.to(f), E_v.to(f), W.to(f), d["rhos"].to(f), V, d["unique"],
        dO.to(f), d["c_base"].to(f), use_silu=True, absent_mass=True)
    t = lambda v: v.numpy().astype(np.float32) if v.is_floating_point() else v.numpy()
    return dict(x=t(d["x"]), unique=t(d["unique"]), c_base=t(d["c_base"]), rhos=t(d["rhos"]),
                Q=t(Q), E_k=t(E_k), E_v=t(E_v), W=t(W), dO=t(dO), V=np.array(V),
                O=t(O), LSE=t(LSE), dQ=t(dQ), dE_k=t(dEk), dE_v=t(dEv), dW=t(dW))


def data_case():
    from oracle import data as od
    rng = np.random.default_rng(31)
    lens = [60, 2, 1, 95, 40, 102]
    tokens = np.concatenate([rng.integers(0, 40, n) for n in lens]).astype(np.int32)
    doc_ids = np.repeat(np.arange(len(lens), dtype=np.int32), lens)
    rhos = od.rhos_for(6, 1.0, 128.0)
    states, pos = od.corpus_states(tokens, doc_ids, rhos)
    chunks, starts = od.chunk_index(doc_ids, 7)
    idx = np.array([0, 5, len(chunks) - 1, 9, 20, 31], np.int64)
    items = [od.get_item(tokens, doc_ids, states, pos, starts, chunks[i], rhos) for i in idx]
    ch, us, pm, inv, cb, K, dd = od.collate(items)
    return dict(tokens=tokens, doc_ids=doc_ids, rhos=rhos, block=np.array(7), states=states,
                chunks_index=np.array(chunks, np.int64), batch=idx, chunks=ch, unique_slots=us,
                pad_mask=pm, inverse=inv, c_base=cb, K_max=np.array(K), doc_out=dd)


def factored_case():
    from oracle import factored as of
    g = torch.Generator().manual_seed(41)
    B, L, V, H, hd, N, K = 2, 40, 30, 2, 32, 6, 8
    D = H * hd
    f = torch.float64
    Q = torch.randn(B, L, D, generator=g, dtype=f)
    x = torch.randint(0, V, (B, L), generator=g)
    Ek = torch.randn(V, D, generator=g, dtype=f) * 0.5
    Ev = torch.randn(V, D, generator=g, dtype=f) * 0.5
    rhos = torch.exp(-math.log(2.0) / torch.logspace(0, math.log10(64.0), N, dtype=f))
    W = torch.randn(N, D, generator=g, dtype=f) * 0.5
    u = torch.randint(-1, V, (B, K), generator=g)
    cb = torch.rand(B, K, N, generator=g, dtype=f) * 3
    leaves = [t.clone().requires_grad_(True) for t in (Q, Ek, Ev, W)]
    O = of.loop_forward(leaves[0], x, leaves[1], leaves[2], rhos, leaves[3], H, c_base=cb,
                        unique_slots=u, pad_mask=u >= 0)
    dO = torch.randn(B, L, D, generator=g, dtype=f)
    O.backward(dO)
    t = lambda v: v.detach().numpy().astype(np.float32)
    return dict(Q=t(Q), x=x.numpy(), E_k=t(Ek), E_v=t(Ev), rhos=t(rhos), W=t(W), unique=u.numpy(),
                c_base=t(cb), H=np.array(H), dO=t(dO), O=t(O), dQ=t(leaves[0].grad),
                dE_k=t(leaves[1].grad), dE_v=t(leaves[2].grad), dW=t(leaves[3].grad))


def main():
    with open(os.path.join(HERE, "reference_kats.json"), "w") as fh:
        json.dump(kats(), fh, indent=1)
    np.savez_compressed(os.path.join(HERE, "scan_small.npz"), **scan_case())
    np.savez_compressed(os.path.join(HERE, "attention_small.npz"), **attention_case())
    np.savez_compressed(os.path.join(HERE, "data_small.npz"), **data_case())
    np.savez_compressed(os.path.join(HERE, "factored_small.npz"), **factored_case())
    print("wrote", sorted(f for f in os.listdir(HERE) if not f.endswith(".py")))


if __name__ == "__main__":
    main()
