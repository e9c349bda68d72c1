"""Sequences longer than one on-chip pass (train.py's documented --seq_len 10000 gives chunks
of 10001 tokens, mathbrain/data.py:76-80; the reference's kernels loop over any L,
triton_ema_query.py:34, triton_flash_ema.py:56-78).

* query scan (mb_ema_query_scan_ws): beyond 8192 steps it runs in 2048-step pieces, each
  chain seeded from its token's last occurrence in an earlier piece; every C_seq element
  against the C oracle (1e-5 relative), the lazy final state and the stamps, with c_init
  keys (duplicates and pads) and document boundaries;
* boundary states: the tokens are staged 8192 at a time; every state against the float64
  oracle (oscan.boundary_states_f64: the fp32 step-by-step restatement carries one rounding
  per step, ~1e-5 by step 10000 itself);
* unique index: rows up to 16384 ids, bit-exact against torch.unique;
* a 2-layer SlotTransformerLM forward and backward on a 10001-token chunk without loader
  metadata (the unique-index path) against the model oracle at sampled positions.
"""
import numpy as np
import pytest
import torch

from oracle import model as omodel
from oracle import scan as oscan
from tests.test_gpu_scan import _close, _scan

pytestmark = pytest.mark.gpu


def zipf(rng, shape, V, alpha=1.1):
    r = np.arange(1, V + 1, dtype=np.float64)
    p = r ** -alpha
    p /= p.sum()
    perm = rng.permutation(V)
    return perm[rng.choice(V, size=shape, p=p)].astype(np.int64)


@pytest.mark.parametrize("L,N,docs", [(10001, 64, False), (16384, 32, False), (10001, 20, True),
                                       (8193, 16, True)])
def test_query_scan_long(L, N, docs):
    rng = np.random.default_rng(L + N)
    B, V, K = 2, 50257, 400
    x = zipf(rng, (B, L), V)
    rhos = np.exp(-np.log(2.0) / np.logspace(0, np.log10(8192), N)).astype(np.float32)
    # keys: tokens of the sequence (some first seen late) and others, duplicates and pads
    keys = np.stack([rng.choice(np.concatenate([x[b, ::13], rng.integers(0, V, 100)]), K, replace=False)
                     for b in range(B)])
    keys[0, -5:] = -1
    keys[1, 7] = keys[1, 3]
    c_init = (rng.random((B, K, N)) * 3).astype(np.float32)
    doc = np.sort(rng.integers(0, 6, size=(B, L)), axis=1) if docs else None
    print(f"L={L} N={N} docs={docs}", flush=True)
    got, st, sp = _scan(x, rhos, V, c_init, keys, doc, return_state=True)
    want = oscan.query_scan(x, rhos, V, c_init, keys, doc)
    _close(got.cpu().numpy(), want)
    sp = sp.cpu().numpy()
    st = st.cpu().numpy()
    for b in range(B):
        for k in range(K):
            if keys[b, k] < 0 or (keys[b, k + 1:] == keys[b, k]).any():
                continue  # pads and losing duplicates keep their rows
            occ = np.nonzero(x[b] == keys[b, k])[0]
            if occ.size:
                assert sp[b, k] == occ[-1]
                _close(st[b, k], want[b, occ[-1]].astype(np.float64) + 1.0)
            else:
                assert sp[b, k] == -1
                _close(st[b, k], c_init[b, k])


def test_query_scan_long_chunk_invariance():
    """The scan of a 12000-step sequence equals the scan of its first 4000 steps followed by
    the scan of the rest seeded with the first part's decayed lazy state (the data
    pipeline's carried c_base)."""
    rng = np.random.default_rng(5)
    B, L, V, N = 1, 12000, 3000, 16
    x = zipf(rng, (B, L), V)
    rhos = np.exp(-np.log(2.0) / np.logspace(0, 3, N)).astype(np.float32)
    full = _scan(x, rhos, V).cpu().numpy()
    a = 4000
    keys = np.unique(x[:, :a])[None, :]
    Ca = _scan(x[:, :a], rhos, V).cpu().numpy()
    c = np.zeros((1, keys.shape[1], N), np.float64)
    for i, u in enumerate(keys[0]):
        s = np.nonzero(x[0, :a] == u)[0][-1]
        c[0, i] = (Ca[0, s].astype(np.float64) + 1.0) * rhos.astype(np.float64) ** (a - s)
    rest = _scan(x[:, a:], rhos, V, c.astype(np.float32), keys).cpu().numpy()
    _close(full[:, :a], Ca)
    _close(full[:, a:], rest, rtol=3e-5)


@pytest.mark.parametrize("L,Br", [(10001, 64), (16384, 64), (12345, 50)])
def test_boundary_states_long(L, Br):
    from mathbrain.triton_flash_ema import precompute_boundaries
    rng = np.random.default_rng(L)
    B, V, N = 2, 50257, 64
    x = zipf(rng, (B, L), V)
    uniq = np.full((B, 300), -1, np.int64)
    for b in range(B):
        u = np.unique(x[b])
        sel = rng.choice(u, 290, replace=False)
        uniq[b, :290] = np.sort(sel)
    rhos = np.exp(-np.log(2.0) / np.logspace(0, np.log10(4096), N)).astype(np.float32)
    c0 = (rng.random((B, 300, N)) * 2).astype(np.float32)
    print(f"L={L} Br={Br}", flush=True)
    got = precompute_boundaries(torch.as_tensor(x).cuda(), torch.as_tensor(uniq).cuda(),
                                torch.as_tensor(rhos).cuda(), Br, torch.as_tensor(c0).cuda()).cpu().numpy()
    want = oscan.boundary_states_f64(x, uniq, rhos, Br, c0)
    _close(got[..., :N], want)


def test_boundary_states_long_doc_ids():
    from mathbrain.triton_flash_ema import precompute_boundaries
    rng = np.random.default_rng(7)
    B, L, V, N, Br = 2, 9000, 500, 16, 64
    x = rng.integers(0, V, size=(B, L)).astype(np.int64)
    uniq = np.stack([np.sort(rng.choice(V, 100, replace=False)) for _ in range(B)]).astype(np.int64)
    rhos = np.exp(-np.log(2.0) / np.logspace(0, 3, N)).astype(np.float32)
    doc = np.sort(rng.integers(0, 8, size=(B, L)), axis=1).astype(np.int64)
    got = precompute_boundaries(torch.as_tensor(x).cuda(), torch.as_tensor(uniq).cuda(),
                                torch.as_tensor(rhos).cuda(), Br, None, torch.as_tensor(doc).cuda()).cpu().numpy()
    want = oscan.boundary_states_f64(x, uniq, rhos, Br, None, doc)
    _close(got[..., :N], want)


@pytest.mark.parametrize("L,V", [(10001, 50257), (16384, 50257), (16384, 1 << 31), (9000, 20)])
def test_unique_rows_long(L, V):
    from mathbrain.triton_flash_ema import _build_unique_index
    rng = np.random.default_rng(L + V % 97)
    x = torch.as_tensor(zipf(rng, (3, L), V) if V < 100000 else rng.integers(-5, V, size=(3, L)))
    ids, K = _build_unique_index(x.cuda(), x.device)
    want = omodel.unique_index(x)
    assert K == want.shape[1]
    assert torch.equal(ids.cpu(), want)


def test_unique_rows_long_wide_range_is_flagged():
    """Beyond 8192 ids a row is sorted as 32-bit offsets: a row whose ids span 2^32 or more is
    refused (counts -1) rather than sorted wrongly."""
    from mathbrain._lib import HipKernelError
    from mathbrain.triton_flash_ema import _build_unique_index, unique_rows
    x = torch.zeros(2, 9000, dtype=torch.int64)
    x[1, 5] = 1 << 40
    ids, counts = unique_rows(x.cuda(), 9000)
    assert counts.cpu().tolist()[1] == -1 and counts.cpu().tolist()[0] == 1
    with pytest.raises(HipKernelError, match="2\\^32"):
        _build_unique_index(x.cuda(), x.device)


def test_model_long_chunk_sampled_positions():
    """SlotTransformerLM on one 10001-token chunk (the chunks train.py --seq_len 10000 makes)
    without loader metadata: logits and every parameter gradient at 48 sampled positions
    against the model oracle (exact float64 model, 2e-2; the attention's default split
    gate)."""
    from mathbrain.model import SlotTransformerLM
    rng = np.random.default_rng(11)
    V, D, NL, H, N, L = 2000, 128, 2, 4, 16, 10001
    torch.manual_seed(12)
    m = SlotTransformerLM(V, D, NL, H, N=N, dropout=0.0, max_hl=2048.0).cuda()
    x = torch.as_tensor(zipf(rng, (1, L), V))
    steps = sorted(rng.choice(L, 48, replace=False).tolist())
    R = torch.randn(1, len(steps), V, generator=torch.Generator().manual_seed(13))
    logits = m(x.cuda())
    sel = logits[:, torch.tensor(steps).cuda()]
    (sel * R.cuda()).sum().backward()
    torch.cuda.synchronize()
    p = {k: v.detach().cpu().double().requires_grad_() for k, v in m.state_dict().items()
         if k not in ("ema_rhos", "lm_head.weight")}
    want = omodel.lm_forward(p, x, NL, H, m.ema_rhos.cpu(), V, t_eval=steps)
    (want * R.double()).sum().backward()
    err = float((sel.detach().cpu().double() - want).abs().max() / want.abs().max())
    grads = dict(m.named_parameters())
    gerr = {k: float((grads[k].grad.cpu().double() - v.grad).abs().max() / v.grad.abs().max().clamp(min=1e-300))
            for k, v in p.items()}
    worst = max(gerr, key=gerr.get)
    print(f"L={L}: logits {err:.2e}, worst gradient {worst} {gerr[worst]:.2e}")
    assert err < 2e-2
    for k, e in gerr.items():
        assert e < 2e-2, (k, e)
