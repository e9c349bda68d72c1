"""mb_corpus_states_noalloc, the corpus-state entry point that allocates nothing (its
scratch is a device array inside the library), against mb_corpus_states with a caller
workspace, through the C ABI: two calls in a row, the second on a smaller corpus, each
bit-identical to the workspace entry point (same kernels, same order of operations) and
within 1e-5 of the CPU oracle; and the size limit rejected with MB_ERR_WORKSPACE."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import data as od

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _get_lib():
    from mathbrain import _lib
    L = _lib.lib()
    fn = L.mb_corpus_states_noalloc
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    return _lib, L


def _corpus(T, V, ndocs, N, seed):
    rng = np.random.default_rng(seed)
    ranks = np.arange(1, V + 1, dtype=np.float64)
    p = ranks ** -1.1
    tokens = rng.choice(V, size=T, p=p / p.sum()).astype(np.int32)
    cuts = np.sort(rng.choice(np.arange(1, T), size=ndocs - 1, replace=False))
    doc_ids = np.zeros(T, np.int32)
    doc_ids[cuts] = 1
    doc_ids = np.cumsum(doc_ids).astype(np.int32)
    rhos = od.rhos_for(N, 1.0, 4096.0)
    return tokens, doc_ids, rhos


def _run_both(tokens, doc_ids, rhos):
    _lib, L = _get_lib()
    from mathbrain.data import chain_order, corpus_states
    dev = torch.device("cuda:0")
    tk = torch.from_numpy(tokens).to(dev)
    dc = torch.from_numpy(doc_ids).to(dev)
    rh = torch.from_numpy(rhos).to(dev)
    want = corpus_states(tk, dc, rh)
    chain, order = chain_order(tk, dc)
    T, N = tokens.size, rhos.size
    got = torch.full((T, N), float("nan"), device=dev)
    torch.cuda.synchronize()
    rc = L.mb_corpus_states_noalloc(order.data_ptr(), chain.data_ptr(), T, rh.data_ptr(), N,
                                    got.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 0, L.mb_last_error()
    torch.cuda.synchronize()
    return got.cpu().numpy(), want.cpu().numpy()


def test_noalloc_matches_workspace_entry_on_two_calls():
    sizes = [(1_000_000, 50257, 400, 64, 1), (70_001, 5000, 30, 64, 2)]   # second call smaller
    for T, V, nd, N, seed in sizes:
        tokens, doc_ids, rhos = _corpus(T, V, nd, N, seed)
        print(f"noalloc corpus states T={T} N={N}", flush=True)
        got, want = _run_both(tokens, doc_ids, rhos)
        assert np.array_equal(got, want), float(np.nanmax(np.abs(got - want)))
        idx = np.random.default_rng(seed).choice(T, 2000, replace=False)
        ref, _ = od.corpus_states(tokens, doc_ids, rhos)
        err = np.abs(got[idx] - ref[idx]) / np.maximum(np.abs(ref[idx]), 1e-30)
        assert err.max() < 1e-5, err.max()


def test_noalloc_small_N_after_large():
    tokens, doc_ids, rhos = _corpus(20_000, 300, 5, 7, 3)
    got, want = _run_both(tokens, doc_ids, rhos)
    assert np.array_equal(got, want)


def test_noalloc_rejects_beyond_scratch():
    _lib, L = _get_lib()
    N = 128
    T = (SCRATCH_BYTES // (N * 12) + 1) * 1024
    assert L.mb_corpus_states_workspace(T, N) > SCRATCH_BYTES
    dummy = torch.empty(8, device="cuda:0")
    rc = L.mb_corpus_states_noalloc(dummy.data_ptr(), dummy.data_ptr(), T, dummy.data_ptr(), N,
                                    dummy.data_ptr(), None)
    assert rc == _lib.MB_ERR_WORKSPACE
    assert b"scratch" in L.mb_last_error()


def test_noalloc_calls_on_two_streams_do_not_race():
    """Two calls issued back to back on two streams (no host synchronisation between them)
    share the one scratch array: the library orders them through its per-device event, so
    both results equal the workspace entry point's, bit for bit."""
    _lib, L = _get_lib()
    from mathbrain.data import chain_order, corpus_states
    dev = torch.device("cuda:0")
    cases = []
    for T, V, nd, N, seed in [(600_000, 50257, 200, 64, 7), (300_000, 20000, 90, 64, 8)]:
        tokens, doc_ids, rhos = _corpus(T, V, nd, N, seed)
        tk = torch.from_numpy(tokens).to(dev)
        dc = torch.from_numpy(doc_ids).to(dev)
        rh = torch.from_numpy(rhos).to(dev)
        want = corpus_states(tk, dc, rh)
        chain, order = chain_order(tk, dc)
        got = torch.full((T, N), float("nan"), device=dev)
        cases.append((order, chain, T, rh, N, got, want))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    for (order, chain, T, rh, N, got, _), s in zip(cases, streams):
        rc = L.mb_corpus_states_noalloc(order.data_ptr(), chain.data_ptr(), T, rh.data_ptr(), N,
                                        got.data_ptr(), s.cuda_stream)
        assert rc == 0, L.mb_last_error()
    torch.cuda.synchronize()
    for (_, _, _, _, _, got, want) in cases:
        assert torch.equal(got, want)
