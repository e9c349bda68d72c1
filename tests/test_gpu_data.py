"""Parity of the device data pipeline (mb_corpus_states, mb_slot_lists, mb_slot_batch
behind mathbrain/data.py) with the CPU oracle of mathbrain/data.py: the corpus
states, the written files, every sample dict and collated batch, and the reference's
own scenarios run end to end.  Integers, ids and masks bit-exact; float32 states and
c_base to 1e-5 relative (each is a product or sum of powers of rho evaluated in another
order)."""
import os
import pickle
import tempfile

import numpy as np
import pytest
import torch

from oracle import data as od

pytestmark = pytest.mark.gpu

RTOL = 1e-5


def _close(got, want, rtol=RTOL, atol=1e-30):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want)
    bad = err > rtol * np.abs(want) + atol
    assert not bad.any(), (f"{bad.sum()} / {bad.size} off; worst rel "
                           f"{(err / (np.abs(want) + 1e-30)).max():.3e}")


def _states(tokens, doc_ids, rhos):
    from mathbrain.data import corpus_states
    return corpus_states(torch.from_numpy(np.asarray(tokens, np.int32)).cuda(),
                         torch.from_numpy(np.asarray(doc_ids, np.int32)).cuda(),
                         torch.from_numpy(np.asarray(rhos, np.float32)).cuda()).cpu().numpy()


def _corpus_dir(docs, N, lo, hi):
    from mathbrain.data import preprocess_corpus
    d = tempfile.mkdtemp(prefix="mb_data_")
    preprocess_corpus(docs, d, N=N, min_hl=lo, max_hl=hi)
    return d


def _docs_from(tokens, doc_ids):
    cuts = np.flatnonzero(np.diff(doc_ids)) + 1
    return [p.tolist() for p in np.split(tokens, cuts)]


def _oracle_for(ds):
    tokens = np.asarray(ds.tokens)
    doc_ids = np.asarray(ds.doc_ids)
    rhos = np.asarray(ds.rhos, np.float32)
    states, pos = od.corpus_states(tokens, doc_ids, rhos)
    chunks, starts = od.chunk_index(doc_ids, ds.block_size)
    assert chunks == ds.chunks and starts == ds.doc_starts
    return lambda i: od.get_item(tokens, doc_ids, states, pos, starts, chunks[i], rhos)


def _same_item(got, want):
    for k in ("chunk", "doc_ids", "unique_slots", "inverse_indices"):
        assert np.array_equal(got[k].cpu().numpy(), want[k]), k
    _close(got["c_base"].cpu().numpy(), want["c_base"])


def _same_batch(got, want):
    names = ("chunks", "unique_slots", "pad_mask", "inverse_indices", "c_bases", "K_max", "doc_ids")
    for name, g, w in zip(names, got, want):
        if name == "K_max":
            assert g == w
        elif name == "c_bases":
            _close(g.cpu().numpy(), w)
        else:
            assert np.array_equal(g.cpu().numpy(), w), name


# ---- corpus states ---------------------------------------------------------------------------

@pytest.mark.parametrize("N", [1, 4, 16, 64, 100, 128])
def test_gpu_corpus_states_match_oracle(N):
    from mathbrain.synthetic import zipf_corpus
    tokens, doc_ids = zipf_corpus(20000, 3000, median_len=700, seed=N)
    rhos = od.rhos_for(N, 1.0, 2048.0)
    print(f"corpus states T=20000 N={N}", flush=True)
    _close(_states(tokens, doc_ids, rhos), od.corpus_states(tokens, doc_ids, rhos)[0])


@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 1023, 1024, 1025, 4097])
def test_gpu_corpus_states_unit_edges(T):
    # one token repeated (one chain across every unit boundary) and a few others
    rng = np.random.default_rng(T)
    tokens = np.where(rng.random(T) < 0.7, 3, rng.integers(0, 6, T)).astype(np.int32)
    doc_ids = (np.arange(T) // 700).astype(np.int32)
    rhos = od.rhos_for(8, 1.0, 4096.0)
    print(f"corpus states unit edges T={T}", flush=True)
    _close(_states(tokens, doc_ids, rhos), od.corpus_states(tokens, doc_ids, rhos)[0])


def test_gpu_corpus_states_resets():
    # every position its own document: all states are 1; one document: the closed form
    T = 3000
    rhos = od.rhos_for(5, 1.0, 64.0)
    tokens = np.zeros(T, np.int32)
    assert np.array_equal(_states(tokens, np.arange(T, dtype=np.int32), rhos), np.ones((T, 5), np.float32))
    got = _states(tokens, np.zeros(T, np.int32), rhos)
    # states of a token at every step: s_t = rho s_{t-1} + 1 = (1 - rho^(t+1)) / (1 - rho)
    t = np.arange(T, dtype=np.float64)[:, None]
    r = rhos.astype(np.float64)[None]
    want = (1.0 - r ** (t + 1)) / (1.0 - r)
    _close(got, want, rtol=2e-5)


def test_gpu_corpus_states_large_spot_check():
    # 4 M tokens of a 50257-id Zipf corpus: 400 positions against the float64 closed form
    from mathbrain.synthetic import zipf_corpus
    T, N = (1 << 22) + 17, 64
    tokens, doc_ids = zipf_corpus(T, 50257, median_len=3000, seed=7)
    rhos = od.rhos_for(N, 1.0, 2048.0)
    print(f"corpus states T={T} N={N}", flush=True)
    got = _states(tokens, doc_ids, rhos)
    assert np.isfinite(got).all() and (got >= 1.0).all()
    rng = np.random.default_rng(0)
    seg = np.concatenate([[0], np.cumsum(doc_ids[1:] != doc_ids[:-1])])
    r = rhos.astype(np.float64)
    for t in rng.integers(0, T, 400):
        d0 = np.searchsorted(seg, seg[t])
        s = np.flatnonzero(tokens[d0:t + 1] == tokens[t]) + d0
        want = (r[None] ** (t - s)[:, None]).sum(0)
        _close(got[t], want, rtol=2e-5)


def test_gpu_preprocess_corpus_files():
    # the reference's file format (data.py:242-320) with the reference's content
    from mathbrain.synthetic import zipf_corpus
    tokens, doc_ids = zipf_corpus(6000, 500, median_len=400, seed=3)
    docs = _docs_from(tokens, doc_ids)
    d = _corpus_dir(docs, 16, 1.0, 1024.0)
    rhos = od.rhos_for(16, 1.0, 1024.0)
    want_s, want_p = od.corpus_states(tokens, doc_ids, rhos)
    assert np.array_equal(np.fromfile(os.path.join(d, "tokens.bin"), np.int32), tokens)
    assert np.array_equal(np.fromfile(os.path.join(d, "doc_ids.bin"), np.int32), doc_ids)
    _close(np.fromfile(os.path.join(d, "states.bin"), np.float32).reshape(-1, 16), want_s)
    with open(os.path.join(d, "pos_dict.pkl"), "rb") as f:   # written by this test's call
        pos = pickle.load(f)
    assert set(pos) == set(want_p)
    assert all(pos[v].dtype == np.int32 and np.array_equal(pos[v], want_p[v]) for v in want_p)


# ---- samples and batches ---------------------------------------------------------------------

def _dataset(docs, N, lo, hi, block):
    from mathbrain.data import WikiTextMMapDataset
    d = _corpus_dir(docs, N, lo, hi)
    return WikiTextMMapDataset(d, block_size=block, rhos=torch.from_numpy(od.rhos_for(N, lo, hi)))


@pytest.mark.parametrize("seed,block", [(0, 4), (1, 17), (2, 64)])
def test_gpu_dataset_items_match_oracle(seed, block):
    from mathbrain.synthetic import zipf_corpus
    tokens, doc_ids = zipf_corpus(3000, 200, median_len=300, seed=seed)
    ds = _dataset(_docs_from(tokens, doc_ids), 8, 1.0, 256.0, block)
    item = _oracle_for(ds)
    print(f"dataset items seed={seed} block={block} chunks={len(ds)}", flush=True)
    for i in range(len(ds)):
        _same_item(ds[i], item(i))


@pytest.mark.parametrize("B", [1, 5, 17])
def test_gpu_get_batch_matches_oracle_collate(B):
    from mathbrain.synthetic import zipf_corpus
    tokens, doc_ids = zipf_corpus(8000, 700, median_len=900, seed=10 + B)
    ds = _dataset(_docs_from(tokens, doc_ids), 12, 1.0, 512.0, 50)
    item = _oracle_for(ds)
    rng = np.random.default_rng(B)
    for rep in range(3):
        idx = rng.choice(len(ds), size=B, replace=False).tolist()
        print(f"get_batch B={B} rep={rep}", flush=True)
        _same_batch(ds.get_batch(idx), od.collate([item(i) for i in idx]))


def test_gpu_batch_zipf_full_vocab():
    # a configuration-2-like batch: 56 chunks of 512 + 1 tokens over 50257 ids, N = 64
    from mathbrain.synthetic import zipf_corpus
    tokens, doc_ids = zipf_corpus(300000, 50257, median_len=4000, seed=21)
    ds = _dataset(_docs_from(tokens, doc_ids), 64, 1.0, 4096.0, 512)
    item = _oracle_for(ds)
    idx = np.random.default_rng(1).choice(len(ds), size=56, replace=False).tolist()
    print(f"full-vocab batch chunks={len(ds)}", flush=True)
    got = ds.get_batch(idx)
    _same_batch(got, od.collate([item(i) for i in idx]))
    assert got[5] > 1000


def test_gpu_reference_scenarios():
    from torch.utils.data import DataLoader

    from mathbrain.data import dynamic_collate_fn
    # tests/test_data_pipeline.py:61-103: c_base of token 1 in the continuation chunk
    ds = _dataset([[1, 2, 3] * 5], 2, 1.0, 4.0, 8)
    r = od.rhos_for(2, 1.0, 4.0)
    it = ds[1]
    k = int((it["unique_slots"] == 1).nonzero()[0, 0])
    _close(it["c_base"][k].cpu().numpy(), (((r ** 3 + 1.0) * r ** 3) + 1.0) * r ** 2)
    # test_data_pipeline.py:171-223: a new document starts from zero
    ds = _dataset([[1, 2, 3, 1, 2], [1, 4, 5, 1, 4]], 2, 1.0, 4.0, 16)
    assert float(ds[1]["c_base"].abs().sum()) == 0.0
    # test_history_expansion.py:254-288: token 99 only in the history
    ds = _dataset([[10, 99, 10, 20, 10, 20, 10, 20]], 8, 1.0, 64.0, 3)
    r = od.rhos_for(8, 1.0, 64.0)
    s = ds.chunks[1][0]
    it = ds[1]
    k = it["unique_slots"].tolist().index(99)
    assert abs(float(it["c_base"][k, 0]) - r[0] ** (s - 1)) < 1e-5
    # test_history_expansion.py:360-372: a two-token document
    ds = _dataset([[5, 6]], 8, 1.0, 64.0, 3)
    assert len(ds) == 1 and set(ds[0]["unique_slots"].tolist()) == {5, 6}
    assert float(ds[0]["c_base"].abs().sum()) == 0.0
    # test_pipeline_thorough.py:469-510: a DataLoader over the dataset sees every target once
    docs = [list(range(i, i + 80)) for i in range(0, 500, 80)]
    ds = _dataset(docs, 4, 1.0, 64.0, 32)
    total = 0
    for chunks, us, pm, inv, cb, K, doc in DataLoader(ds, batch_size=4, collate_fn=dynamic_collate_fn):
        y, dx, dy = chunks[:, 1:].clone(), doc[:, :-1], doc[:, 1:]
        y[dy == -1] = -1
        y[dx != dy] = -1
        total += int((y != -1).sum())
    assert total == sum(len(d) - 1 for d in docs)


def test_gpu_slot_loader_matches_get_batch():
    from mathbrain.data import SlotBatchLoader, TokenBudgetSampler, dynamic_collate_fn
    from mathbrain.synthetic import zipf_corpus
    tokens, doc_ids = zipf_corpus(5000, 400, median_len=500, seed=5)
    ds = _dataset(_docs_from(tokens, doc_ids), 8, 1.0, 256.0, 40)
    sampler = TokenBudgetSampler(ds, token_budget=400, shuffle=False)
    n = 0
    for idx, got in zip(sampler, SlotBatchLoader(ds, sampler)):
        want = dynamic_collate_fn([ds[i] for i in idx])
        for g, w in zip(got, want):
            if isinstance(w, int):
                assert g == w
            else:
                assert torch.equal(g, w)
        n += 1
    assert n == len(sampler) > 3


def test_gpu_batch_feeds_the_model():
    # the collated batch goes straight into SlotTransformerLM as train.py passes it
    from mathbrain.model import SlotTransformerLM
    from mathbrain.synthetic import zipf_corpus
    tokens, doc_ids = zipf_corpus(4000, 300, median_len=600, seed=9)
    ds = _dataset(_docs_from(tokens, doc_ids), 16, 1.0, 1024.0, 64)
    chunks, us, pm, inv, cb, K, doc = ds.get_batch(list(range(min(6, len(ds)))))
    torch.manual_seed(0)
    model = SlotTransformerLM(vocab_size=300, d_model=128, n_layers=1, n_heads=4, N=16,
                              dropout=0.0, min_hl=1.0, max_hl=1024.0).cuda()
    logits = model(chunks[:, :-1], unique_slots=us, inverse_indices=inv[:, :-1], c_base=cb,
                   doc_ids=doc[:, :-1], pad_mask=pm)
    assert logits.shape == (chunks.shape[0], chunks.shape[1] - 1, 300)
    assert torch.isfinite(logits).all()
