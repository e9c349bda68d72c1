"""Pins the CPU oracle of the data pipeline (oracle/data.py) and checks the host-side
bookkeeping of mathbrain/data.py against it (no GPU needed).

Known answers are the reference's own (tests/test_pipeline_thorough.py,
tests/test_data_pipeline.py, tests/test_history_expansion.py); the rest are the closed
forms of the states and of c_base, evaluated by brute force in float64, and the
block-size invariance the reference tests (test_data_pipeline.py:106-168), which ties
c_base to the EMA query scan.
"""
import numpy as np
import pytest
import torch

from oracle import data as od
from oracle import scan


def corpus(docs):
    tokens = np.asarray([t for d in docs for t in d], np.int32)
    doc_ids = np.repeat(np.arange(len(docs), dtype=np.int32), [len(d) for d in docs])
    return tokens, doc_ids


def build(docs, N, lo, hi, block):
    tokens, doc_ids = corpus(docs)
    rhos = od.rhos_for(N, lo, hi)
    states, pos = od.corpus_states(tokens, doc_ids, rhos)
    chunks, starts = od.chunk_index(doc_ids, block)
    item = lambda i: od.get_item(tokens, doc_ids, states, pos, starts, chunks[i], rhos)
    return tokens, doc_ids, rhos, states, pos, chunks, starts, item


# ---- reference known answers -----------------------------------------------------------

def test_kat_preprocessing():
    # tests/test_pipeline_thorough.py:42-80
    docs = [[10, 20, 30, 10, 20], [10, 40, 50]]
    tokens, doc_ids, rhos, states, pos, *_ = build(docs, 2, 1.0, 4.0, 8)
    assert tokens.tolist() == [10, 20, 30, 10, 20, 10, 40, 50]
    assert doc_ids.tolist() == [0, 0, 0, 0, 0, 1, 1, 1]
    assert np.allclose(states[0], [1.0, 1.0])
    assert np.allclose(states[3], rhos ** 3 + 1.0, atol=1e-5)
    assert np.allclose(states[5], [1.0, 1.0])          # reset at the document change
    assert pos[10].tolist() == [0, 3, 5]


def test_kat_c_base_continuation_chunk():
    # tests/test_data_pipeline.py:61-103
    doc = [1, 2, 3] * 5
    *_, rhos, states, pos, chunks, starts, item = build([doc], 2, 1.0, 4.0, 8)
    assert len(chunks) == 2 and chunks[1][0] == 8
    it = item(1)
    k = int(np.flatnonzero(it["unique_slots"] == 1)[0])
    s6 = ((np.ones(2) * rhos ** 3 + 1.0) * rhos ** 3) + 1.0   # states at positions 0, 3, 6
    assert np.allclose(it["c_base"][k], s6 * rhos ** 2, atol=1e-5)


def test_kat_cross_doc_isolation():
    # tests/test_data_pipeline.py:171-223 and test_pipeline_thorough.py:129-186
    docs = [[1, 2, 3, 1, 2], [1, 4, 5, 1, 4]]
    *_, chunks, starts, item = build(docs, 2, 1.0, 4.0, 16)
    assert len(chunks) == 2 and chunks[1][2] == 1
    assert np.abs(item(1)["c_base"]).sum() == 0
    assert (item(1)["doc_ids"] == 1).all()


def test_kat_history_expansion():
    # tests/test_history_expansion.py:79-118: block 3, chunks [10,20,30,40], [40,50,10,20]
    tokens = [10, 20, 30, 40, 50, 10, 20]
    *_, chunks, starts, item = build([tokens], 8, 1.0, 64.0, 3)
    i0, i1 = item(0), item(1)
    assert set(i0["unique_slots"].tolist()) == set(i0["chunk"].tolist())
    assert np.abs(i0["c_base"]).sum() == 0
    hist = set(tokens[:chunks[1][0]]) - set(i1["chunk"].tolist())
    assert hist and hist <= set(i1["unique_slots"].tolist())
    # chunk tokens first, in id order, then history-only tokens in id order
    n_chunk = len(set(i1["chunk"].tolist()))
    assert i1["unique_slots"][:n_chunk].tolist() == sorted(set(i1["chunk"].tolist()))
    assert i1["unique_slots"][n_chunk:].tolist() == sorted(hist)
    assert (i1["unique_slots"][i1["inverse_indices"]] == i1["chunk"]).all()


def test_kat_history_only_token_decay():
    # tests/test_history_expansion.py:254-288: token 99 at position 1 only
    tokens = [10, 99, 10, 20, 10, 20, 10, 20]
    _, _, rhos, states, pos, chunks, starts, item = build([tokens], 8, 1.0, 64.0, 3)
    done = False
    for i, (s, e, _) in enumerate(chunks):
        it = item(i)
        if s > 1 and 99 not in it["chunk"].tolist():
            k = it["unique_slots"].tolist().index(99)
            assert abs(it["c_base"][k][0] - rhos[0] ** (s - 1)) < 1e-5
            done = True
            break
    assert done


def test_kat_cross_doc_history_excluded():
    # tests/test_history_expansion.py:190-211
    tokens = [10, 20, 30, 10, 40, 50, 10, 40]
    doc_ids = [0, 0, 0, 1, 1, 1, 1, 1]
    rhos = od.rhos_for(8, 1.0, 64.0)
    states, pos = od.corpus_states(tokens, doc_ids, rhos)
    chunks, starts = od.chunk_index(doc_ids, 3)
    seen = False
    for c in chunks:
        if c[2] == 1 and c[0] > starts[1]:
            slots = set(od.get_item(np.asarray(tokens), np.asarray(doc_ids), states, pos, starts, c,
                                    rhos)["unique_slots"].tolist())
            assert 20 not in slots and 30 not in slots
            seen = True
    assert seen


def test_kat_chunk_index():
    # tests/test_pipeline_thorough.py:84-126 and test_history_expansion.py:360-372
    docs = [list(range(100)), list(range(50)), list(range(200)), [1]]
    _, doc_ids = corpus(docs)
    chunks, starts = od.chunk_index(doc_ids, 64)
    assert 3 not in {d for _, _, d in chunks}
    assert all(e - s <= 65 for s, e, _ in chunks)
    assert len({p for s, e, d in chunks if d == 0 for p in range(s, e)}) == 100
    assert od.chunk_index(np.zeros(2, np.int32), 3)[0] == [(0, 2, 0)]


def test_kat_token_budget():
    # tests/test_pipeline_thorough.py:362-391
    docs = [list(range(i * 10, i * 10 + 50 + i * 20)) for i in range(10)]
    _, doc_ids = corpus(docs)
    chunks, _ = od.chunk_index(doc_ids, 128)
    lengths = [e - s for s, e, _ in chunks]
    batches = od.token_budget(lengths, 512, list(range(len(chunks))))
    assert sorted(i for b in batches for i in b) == list(range(len(chunks)))
    assert all(max(lengths[i] for i in b) * len(b) <= 512 or len(b) == 1 for b in batches)


# ---- closed forms --------------------------------------------------------------------------

def random_docs(rng, n_docs, max_len, V):
    return [rng.integers(0, V, size=int(rng.integers(1, max_len))).tolist() for _ in range(n_docs)]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_states_closed_form(seed):
    rng = np.random.default_rng(seed)
    tokens, doc_ids = corpus(random_docs(rng, 5, 30, 6))
    rhos = od.rhos_for(4, 1.0, 32.0)
    states, pos = od.corpus_states(tokens, doc_ids, rhos)
    want = od.states_closed_form(tokens, doc_ids, rhos)
    assert np.allclose(states, want, rtol=2e-6, atol=1e-6)
    for v, p in pos.items():
        assert p.tolist() == np.flatnonzero(tokens == v).tolist()


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_c_base_closed_form(seed):
    rng = np.random.default_rng(seed)
    docs = random_docs(rng, 4, 40, 8)
    tokens, doc_ids, rhos, states, pos, chunks, starts, item = build(docs, 3, 1.0, 16.0, 5)
    for i, c in enumerate(chunks):
        it = item(i)
        want = od.c_base_closed_form(tokens, doc_ids, c, it["unique_slots"], rhos)
        assert np.allclose(it["c_base"], want, rtol=2e-6, atol=1e-6)
        # the slots are exactly the tokens of the chunk and of its document history
        s, e, d = c
        assert set(it["unique_slots"].tolist()) == set(tokens[starts[d]:e].tolist())


def test_block_size_invariance():
    # tests/test_data_pipeline.py:106-168: the query scan over each chunk, started from
    # that chunk's c_base, gives states[t] - 1 at every position whatever the block size
    doc = [i % 5 for i in range(100)] + [7, 3, 7, 7, 1, 3]
    tokens, doc_ids = corpus([doc])
    rhos = od.rhos_for(4, 1.0, 32.0)
    states, pos = od.corpus_states(tokens, doc_ids, rhos)
    for block in (7, 16, 32, 64):
        chunks, starts = od.chunk_index(doc_ids, block)
        for c in chunks:
            it = od.get_item(tokens, doc_ids, states, pos, starts, c, rhos)
            C = scan.query_scan(it["chunk"][None], rhos, 8, it["c_base"][None],
                                it["unique_slots"][None])[0]
            assert np.allclose(C + 1.0, states[c[0]:c[1]], rtol=1e-5, atol=1e-5)


# ---- host bookkeeping of mathbrain.data against the oracle ------------------------------

@pytest.mark.parametrize("seed,block", [(0, 3), (1, 16), (2, 64), (3, 1)])
def test_chunk_index_matches_oracle(seed, block):
    from mathbrain import data as md
    rng = np.random.default_rng(seed)
    docs = random_docs(rng, 30, 150, 50) + [[5]] + random_docs(rng, 3, 4, 5)
    _, doc_ids = corpus(docs)
    cs, ce, cd, starts = md.chunk_index(doc_ids, block)
    want, want_starts = od.chunk_index(doc_ids, block)
    assert list(zip(cs.tolist(), ce.tolist(), cd.tolist())) == want
    assert starts == want_starts


def test_chunk_index_rejects_split_documents():
    from mathbrain import data as md
    with pytest.raises(ValueError):
        md.chunk_index(np.array([0, 0, 1, 1, 0, 0], np.int32), 4)


def test_token_budget_sampler_matches_oracle():
    from mathbrain import data as md

    class Lens:
        def __init__(self, n):
            self.n = n

        def __len__(self):
            return len(self.n)

        def chunk_len(self, i):
            return self.n[i]

    rng = np.random.default_rng(4)
    lengths = rng.integers(2, 130, size=200).tolist()
    s = md.TokenBudgetSampler(Lens(lengths), token_budget=700, shuffle=False)
    assert list(s) == od.token_budget(lengths, 700, list(range(200)))
    assert len(s) == len(s.batches)


def test_dynamic_collate_matches_oracle():
    from mathbrain import data as md
    rng = np.random.default_rng(5)
    docs = random_docs(rng, 6, 60, 12)
    tokens, doc_ids, rhos, states, pos, chunks, starts, item = build(docs, 4, 1.0, 32.0, 9)
    items = [item(i) for i in range(min(7, len(chunks)))]
    want = od.collate(items)
    got = md.dynamic_collate_fn([{k: torch.from_numpy(v) for k, v in it.items()} for it in items])
    for g, w in zip(got, want):
        if isinstance(w, int):
            assert g == w
        else:
            assert np.array_equal(g.numpy(), w)


def test_device_calls_need_a_gpu():
    from mathbrain import data as md
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(NotImplementedError):
        md.preprocess_corpus([[1, 2, 3]], "/tmp/mb_never_written")
    with pytest.raises(NotImplementedError):
        md.corpus_states(torch.zeros(3, dtype=torch.int32), torch.zeros(3, dtype=torch.int32),
                         torch.ones(2))
