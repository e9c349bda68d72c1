"""Parity of the HIP EMA scans (mb_ema_query_scan, mb_ema_boundary_states) with the
CPU oracle, on the reference's known answers, seeded random and Zipf inputs, the
full-size scan configuration and the edge cases.  Tolerance: 1e-5 relative (fp32)."""
import numpy as np
import pytest
import torch

from oracle import scan as oscan

pytestmark = pytest.mark.gpu

RTOL = 1e-5
ATOL = 1e-30


def _close(got, want, rtol=RTOL):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    bad = err > rtol * np.abs(want) + ATOL
    assert not bad.any(), (f"{bad.sum()} / {bad.size} elements off; worst rel "
                           f"{(err / (np.abs(want) + 1e-30)).max():.3e}")


def _dev(t):
    return torch.as_tensor(t).cuda()


def _scan(x, rhos, V, c_init=None, keys=None, doc=None, **kw):
    from mathbrain.triton_ema_query import compute_query_ema_history
    return compute_query_ema_history(_dev(x), _dev(rhos), V,
                                     None if c_init is None else _dev(c_init),
                                     None if keys is None else _dev(keys),
                                     None if doc is None else _dev(doc), **kw)


def test_gpu_scan_reference_kats():
    # tests/test_doc_boundary.py:71-134 and :22-68 through the HIP path
    rh = np.array([0.9, 0.5], np.float32)
    C = _scan(np.array([[0, 1, 0, 2, 0, 1]]), rh, 3, doc=np.zeros((1, 6), np.int64)).cpu().numpy()
    _close(C[0, 2], rh.astype(np.float64) ** 2, 1e-6)
    _close(C[0, 4], (rh.astype(np.float64) ** 2 + 1) * rh.astype(np.float64) ** 2, 1e-6)
    assert np.all(C[0, 0] == 0)
    C = _scan(np.array([[0, 1, 0, 2]]), rh, 3, np.array([[[2.0, 1.5], [0, 0], [0, 0]]], np.float32),
              np.array([[0, 1, 2]])).cpu().numpy()
    assert np.allclose(C[0, 0], [2.0, 1.5])
    rh4 = np.array([0.9, 0.8, 0.7, 0.6], np.float32)
    x = np.array([[0, 1, 2, 0, 1, 0, 1, 3, 0, 1]])
    doc = np.array([[0, 0, 0, 0, 0, 1, 1, 1, 1, 1]])
    C = _scan(x, rh4, 5, doc=doc).cpu().numpy()
    assert np.all(C[0, 5] == 0)
    _close(C[0, 8], rh4.astype(np.float64) ** 3, 1e-6)


@pytest.mark.parametrize("N", [1, 4, 16, 20, 64, 128])
@pytest.mark.parametrize("with_init", [False, True])
def test_gpu_scan_random_vs_oracle(N, with_init):
    rng = np.random.default_rng(N * 7 + with_init)
    B, L, V = 3, 300, 40
    x = rng.integers(0, V, size=(B, L))
    rhos = np.exp(-np.log(2.0) / np.logspace(0, np.log10(512), N)).astype(np.float32)
    c_init = keys = None
    if with_init:
        K = 30
        keys = np.stack([rng.permutation(V)[:K] for _ in range(B)])
        keys[1, -5:] = -1
        c_init = (rng.random((B, K, N)) * 5).astype(np.float32)
    got = _scan(x, rhos, V, c_init, keys).cpu().numpy()
    want = oscan.query_scan(x, rhos, V, c_init, keys)
    _close(got, want)


def test_gpu_scan_doc_ids_and_strided_x():
    rng = np.random.default_rng(3)
    B, L, V, N = 4, 257, 17, 8
    full = rng.integers(0, V, size=(B, L + 1))
    doc = np.sort(rng.integers(0, 3, size=(B, L)), axis=1)
    rhos = np.linspace(0.3, 0.999, N).astype(np.float32)
    keys = np.stack([rng.permutation(V)[:10] for _ in range(B)])
    c_init = rng.random((B, 10, N)).astype(np.float32)
    xt = _dev(full)[:, :-1]  # non-contiguous view, as train.py passes tokens[:, :-1]
    from mathbrain.triton_ema_query import compute_query_ema_history
    got = compute_query_ema_history(xt, _dev(rhos), V, _dev(c_init), _dev(keys), _dev(doc)).cpu().numpy()
    want = oscan.query_scan(full[:, :-1], rhos, V, c_init, keys, doc)
    _close(got, want)


def test_gpu_scan_duplicate_and_padded_keys():
    x = np.array([[3, 3, 1, 0, 3]])
    rhos = np.array([0.5, 0.9, 0.99, 1.0], np.float32)
    keys = np.array([[3, 1, 3, -1, -1]])
    c_init = np.arange(20, dtype=np.float32).reshape(1, 5, 4)
    got = _scan(x, rhos, 5, c_init, keys).cpu().numpy()
    want = oscan.query_scan(x, rhos, 5, c_init, keys)
    _close(got, want)


def test_gpu_scan_wide_token_ids():
    # token ids beyond 2^(32 - log2 L) take the 64-bit sort-key path
    rng = np.random.default_rng(5)
    B, L, N = 2, 1000, 16
    V = 1 << 40
    base = rng.integers(0, 1 << 40, size=50)
    x = base[rng.integers(0, 50, size=(B, L))]
    rhos = np.linspace(0.5, 0.999, N).astype(np.float32)
    got = _scan(x, rhos, V).cpu().numpy()
    # relabel to a small vocabulary for the oracle's dense [V+1, N] state
    _, inv = np.unique(x, return_inverse=True)
    want = oscan.query_scan(inv.reshape(B, L), rhos, 50)
    _close(got, want)


@pytest.mark.parametrize("L", [1, 2, 63, 64, 1025, 8192])
def test_gpu_scan_lengths(L):
    rng = np.random.default_rng(L)
    V, N = 97, 8
    x = rng.integers(0, V, size=(2, L))
    rhos = np.linspace(0.2, 0.9999, N).astype(np.float32)
    _close(_scan(x, rhos, V).cpu().numpy(), oscan.query_scan(x, rhos, V))


@pytest.mark.parametrize("L,V,pattern", [(4096, 97, "uniform"), (2048, 3, "uniform"),
                                          (4096, 1, "uniform"), (4096, 1 << 19, "distinct"),
                                          (3000, 200, "zipf"), (2048, 50257, "zipf"),
                                          (100, 7, "uniform")])
def test_gpu_scan_hash_grouping_runs(L, V, pattern):
    """Grouping positions by token: the hash path (32-bit token keys and its tables in LDS,
    L <= 2048 at this N) with runs counted position by position, runs long enough for the
    position bitmaps (up to a few runs of ~700) and Zipf streams; the sort path for the longer
    sequences (one run of all 4096 positions, no repeats at all).  Every output element, the
    final state and the stamps against the oracle, with c_init keys."""
    rng = np.random.default_rng(L + V)
    B, N, K = 2, 8, 64
    if pattern == "uniform":
        x = rng.integers(0, V, size=(B, L))
    elif pattern == "distinct":
        x = np.stack([rng.permutation(V)[:L] for _ in range(B)])
    else:
        x = np.minimum(rng.zipf(1.1, size=(B, L)) - 1, V - 1)
    rhos = np.exp(-np.log(2.0) / np.logspace(0, np.log10(4096), N)).astype(np.float32)
    keys = np.stack([np.concatenate([rng.choice(x[b], K // 2), rng.integers(0, V, K - K // 2)])
                     for b in range(B)])
    keys[0, -3:] = -1
    c_init = (rng.random((B, K, N)) * 3).astype(np.float32)
    got, st, sp = _scan(x, rhos, V, c_init, keys, return_state=True)
    want = oscan.query_scan(x, rhos, V, c_init, keys)
    _close(got.cpu().numpy(), want)
    sp = sp.cpu().numpy()
    st = st.cpu().numpy()
    for b in range(B):
        for k in range(K):
            if keys[b, k] < 0 or (keys[b, k + 1:] == keys[b, k]).any():
                continue
            occ = np.nonzero(x[b] == keys[b, k])[0]
            if occ.size:
                assert sp[b, k] == occ[-1]
                _close(st[b, k], want[b, occ[-1]].astype(np.float64) + 1.0)
            else:
                assert sp[b, k] == -1


@pytest.mark.parametrize("L,V,N,docs", [(2048, 1 << 30, 128, False), (2048, 1 << 30, 20, True),
                                         (8192, 20000, 16, False), (4096, 1 << 30, 64, True)])
def test_gpu_scan_more_tokens_than_lds_state(L, V, N, docs):
    """Sequences with more distinct tokens than one pass's LDS state holds (up to all-distinct)
    take several passes over the sequence; every output element, the final state and the
    stamps against the oracle, with c_init keys (duplicates and pads included) and, for
    `docs`, document boundaries."""
    rng = np.random.default_rng(L + N)
    B = 2
    x = rng.integers(0, V, size=(B, L))
    x[1] = rng.permutation(V)[:L] if V >= L else x[1]  # row 1: all distinct when V allows
    rhos = np.exp(-np.log(2.0) / np.logspace(0, np.log10(4096), N)).astype(np.float32)
    K = 600
    keys = np.stack([np.concatenate([rng.choice(x[b], K // 2), rng.integers(0, V, K - K // 2)])
                     for b in range(B)])
    keys[0, -7:] = -1
    keys[1, 5] = keys[1, 3]
    c_init = (rng.random((B, K, N)) * 3).astype(np.float32)
    doc = np.sort(rng.integers(0, 5, size=(B, L)), axis=1) if docs else None
    got, st, sp = _scan(x, rhos, V, c_init, keys, doc, return_state=True)
    _, inv = np.unique(np.concatenate([x.ravel(), keys.ravel()]), return_inverse=True)
    xs = inv[:x.size].reshape(B, L)
    ks = np.where(keys >= 0, inv[x.size:].reshape(B, K), -1)
    Vs = int(inv.max()) + 1
    want = oscan.query_scan(xs, rhos, Vs, c_init, ks, doc)
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


def test_gpu_scan_long_without_vocab_raises():
    """Beyond 8192 steps the scan runs in pieces with a [B, vocab_size] table of last
    positions, so it needs the vocabulary size."""
    from mathbrain._lib import HipKernelError
    with pytest.raises(HipKernelError, match="vocab_size"):
        _scan(np.zeros((1, 8193), np.int64), np.array([0.5], np.float32), 0)


def test_gpu_scan_cfg3_full_size():
    """Config 3 at full size: B=56, T=2048, N=128, V=50257, c_base from an 8192-token
    Zipf(1.1) warm-up -- every output element against the oracle, plus the final state."""
    from mathbrain.synthetic import make_batch
    d = make_batch(56, 2048, 50257, 128, 8192, seed=3)
    C, state, stamps = _scan(d["x"].numpy(), d["rhos"].numpy(), 50257, d["c_base"].numpy(),
                             d["unique"].numpy(), return_state=True)
    want = oscan.query_scan(d["x"], d["rhos"], 50257, d["c_base"], d["unique"])
    _close(C.cpu().numpy(), want)
    # final lazy state of each key: C_seq at its last occurrence + 1
    stamps = stamps.cpu().numpy()
    st = state.cpu().numpy()
    x = d["x"].numpy()
    uniq = d["unique"].numpy()
    for b in (0, 17, 55):
        for k in range(0, int(d["counts"][b]), 97):
            occ = np.nonzero(x[b] == uniq[b, k])[0]
            if occ.size:
                assert stamps[b, k] == occ[-1]
                _close(st[b, k], want[b, occ[-1]].astype(np.float64) + 1.0)
            else:
                assert stamps[b, k] == -1
                assert np.array_equal(st[b, k], d["c_base"][b, k].numpy())


def test_gpu_scan_chained_chunks_equal_single_pass():
    """Carrying the returned state into the next chunk reproduces one long scan
    (the block-size invariance of tests/test_gold_standard.py:265-305)."""
    rng = np.random.default_rng(11)
    V, N, L = 60, 16, 600
    x = rng.integers(0, V, size=(1, L))
    rhos = np.exp(-np.log(2.0) / np.logspace(0, 3, N)).astype(np.float32)
    full = _scan(x, rhos, V).cpu().numpy()[0]
    keys = np.arange(V)[None]
    state = torch.zeros(1, V, N, device="cuda")
    stamps_abs = np.full(V, -10 ** 9)
    out = np.zeros_like(full)
    for cs in range(0, L, 128):
        ce = min(cs + 128, L)
        # c_base for this chunk: lazy state decayed to the chunk start
        d = np.where(stamps_abs >= 0, cs - stamps_abs, 0)
        cb = state.cpu().numpy()[0] * (rhos[None, :].astype(np.float64) ** d[:, None])
        cb = np.where((stamps_abs >= 0)[:, None], cb, 0).astype(np.float32)
        C, st, sp = _scan(x[:, cs:ce], rhos, V, cb[None], keys, return_state=True)
        out[cs:ce] = C.cpu().numpy()[0]
        sp = sp.cpu().numpy()[0]
        hit = sp >= 0
        stamps_abs[hit] = cs + sp[hit]
        state = torch.where(torch.as_tensor(hit).cuda()[None, :, None], st, state)
    _close(out, full, 2e-5)


@pytest.mark.parametrize("Br", [1, 16, 64, 100])
def test_gpu_boundary_vs_oracle(Br):
    from mathbrain.triton_flash_ema import precompute_boundaries
    rng = np.random.default_rng(Br)
    B, L, V, N, K = 3, 333, 50, 12, 40
    x = rng.integers(0, V, size=(B, L))
    unique = np.stack([rng.permutation(V)[:K] for _ in range(B)])
    unique[2, -7:] = -1
    rhos = np.exp(-np.log(2.0) / np.logspace(0, 3, N)).astype(np.float32)
    c_init = (rng.random((B, K, N)) * 4).astype(np.float32)
    got = precompute_boundaries(_dev(x), _dev(unique), _dev(rhos), Br, _dev(c_init)).cpu().numpy()
    want = oscan.boundary_states(x, unique, rhos, Br, c_init)
    assert got.shape == (B, want.shape[1], K, 16)
    assert np.all(got[..., N:] == 0)
    _close(got[..., :N], want, 2e-5)


def test_gpu_boundary_doc_ids_and_padded_c_init():
    from mathbrain.triton_flash_ema import precompute_boundaries
    rng = np.random.default_rng(9)
    B, L, V, N, K = 2, 200, 20, 4, 20
    x = rng.integers(0, V, size=(B, L))
    doc = np.sort(rng.integers(0, 4, size=(B, L)), axis=1)
    unique = np.stack([rng.permutation(V) for _ in range(B)])
    rhos = np.linspace(0.5, 0.99, N).astype(np.float32)
    c_init = rng.random((B, K, 16)).astype(np.float32)  # padded to 16 columns as the reference does
    got = precompute_boundaries(_dev(x), _dev(unique), _dev(rhos), 64, _dev(c_init), _dev(doc))
    want = oscan.boundary_states(x, unique, rhos, 64, c_init[:, :, :N], doc)
    _close(got.cpu().numpy()[..., :N], want, 2e-5)


@pytest.mark.parametrize("N,Br", [(100, 48), (200, 150), (128, 64), (33, 200)])
def test_gpu_boundary_wide_rates_ragged_slots(N, Br):
    """Two and four rates per lane, pieces shorter than 64 steps and chunks of several
    pieces, document resets, and a slot count that leaves part of the last 64-slot
    workgroup without slots."""
    from mathbrain.triton_flash_ema import precompute_boundaries
    rng = np.random.default_rng(N + Br)
    B, L, V, K = 2, 300, 90, 70
    x = rng.integers(0, V, size=(B, L))
    doc = np.sort(rng.integers(0, 3, size=(B, L)), axis=1)
    unique = np.stack([rng.permutation(V)[:K] for _ in range(B)])
    unique[1, -9:] = -1
    rhos = np.exp(-np.log(2.0) / np.logspace(0, 3, N)).astype(np.float32)
    c_init = (rng.random((B, K, N)) * 3).astype(np.float32)
    got = precompute_boundaries(_dev(x), _dev(unique), _dev(rhos), Br, _dev(c_init), _dev(doc)).cpu().numpy()
    want = oscan.boundary_states(x, unique, rhos, Br, c_init, doc)
    assert np.all(got[..., N:] == 0)
    _close(got[..., :N], want, 2e-5)


def test_gpu_boundary_cfg2_zipf():
    from mathbrain.triton_flash_ema import precompute_boundaries
    from mathbrain.synthetic import make_batch
    d = make_batch(4, 512, 50257, 64, 4096, seed=1)
    got = precompute_boundaries(d["x"].cuda(), d["unique"].cuda(), d["rhos"].cuda(), 64,
                                d["c_base"].cuda()).cpu().numpy()
    want = oscan.boundary_states(d["x"], d["unique"], d["rhos"], 64, d["c_base"])
    _close(got[..., :64], want, 2e-5)
