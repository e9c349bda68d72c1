"""TEST INFRASTRUCTURE ONLY: CPU restatement of the data pipeline that produces the hot
path's inputs (the checker, never the product).

Each function restates one step of mathbrain/data.py in numpy, in the reference's own
order of operations and float32 arithmetic:

  rhos_for            data.py:268-270  (float64 logspace, cast to float32)
  corpus_states       data.py:276-303  per-token state after each occurrence, reset at
                                       every change of document id; plus pos_dict
  chunk_index         data.py:48-84    document ranges, chunks of block_size + 1 tokens
                                       overlapping by one, documents shorter than 2 skipped
  get_item            data.py:93-148   chunk, doc ids, history-expanded slot list,
                                       inverse indices and c_base of one chunk
  collate             data.py:207-232  padding to the batch maxima
  token_budget        data.py:167-192  greedy packing of a given index order under a
                                       padded-token budget

Closed forms that pin them (tests/test_oracle_data.py):
  states[t]  = sum_{s <= t, x_s = x_t, s in t's document segment} rho^(t-s)
  c_base[v]  = sum_{s < start, x_s = v, s in the chunk's document} rho^(start-s)
"""
import numpy as np


def rhos_for(N, min_hl=1.0, max_hl=2048.0):
    """Decay rates as preprocess_corpus computes them (data.py:268-270)."""
    scales = np.logspace(np.log10(min_hl), np.log10(max_hl), N)
    return np.exp(-np.log(2.0) / scales).astype(np.float32)


def corpus_states(tokens, doc_ids, rhos):
    """The preprocessing scan (data.py:276-303): returns (states [T, N] float32,
    pos_dict {token: int32 positions})."""
    tokens = np.asarray(tokens, dtype=np.int32)
    doc_ids = np.asarray(doc_ids, dtype=np.int32)
    rhos = np.asarray(rhos, dtype=np.float32)
    T, N = len(tokens), len(rhos)
    states = np.zeros((T, N), dtype=np.float32)
    V = int(tokens.max()) + 1 if T else 1
    cur = np.zeros((V, N), dtype=np.float32)
    last = np.full(V, -1, dtype=np.int64)
    pos = {}
    cur_doc = None
    for t in range(T):
        d = doc_ids[t]
        if cur_doc is None or d != cur_doc:                # data.py:287-290
            cur.fill(0.0)
            last.fill(-1)
            cur_doc = d
        v = tokens[t]
        pos.setdefault(int(v), []).append(t)
        if last[v] == -1:                                  # data.py:296-300
            cur[v] = 1.0
        else:
            cur[v] = cur[v] * (rhos ** np.float32(t - last[v])) + np.float32(1.0)
        last[v] = t
        states[t] = cur[v]
    return states, {v: np.asarray(p, dtype=np.int32) for v, p in pos.items()}


def chunk_index(doc_ids, block_size):
    """Chunk list [(start, end, doc_id)] and doc_starts {doc_id: start} (data.py:48-84)."""
    doc_ids = np.asarray(doc_ids)
    T = len(doc_ids)
    chunks, doc_starts = [], {}
    if T == 0:
        return chunks, doc_starts
    ranges = []
    s, cur = 0, int(doc_ids[0])
    for i in range(1, T):
        d = int(doc_ids[i])
        if d != cur:
            ranges.append((s, i, cur))
            s, cur = i, d
    ranges.append((s, T, cur))
    for s, e, d in ranges:
        n = e - s
        if n < 2:
            continue
        doc_starts[d] = s
        for c in range(max(1, (n - 1 + block_size - 1) // block_size)):
            cs = s + c * block_size
            ce = min(cs + block_size + 1, e)
            if ce - cs >= 2:
                chunks.append((cs, ce, d))
    return chunks, doc_starts


def get_item(tokens, doc_ids, states, pos_dict, doc_starts, chunk, rhos):
    """One sample (data.py:93-148): dict of chunk, doc_ids, unique_slots, inverse_indices,
    c_base as numpy arrays (int64 / float32)."""
    start, end, doc = chunk
    rhos = np.asarray(rhos, dtype=np.float32)
    ch = np.asarray(tokens[start:end], dtype=np.int64)
    chunk_unique, inverse = np.unique(ch, return_inverse=True)
    in_chunk = set(chunk_unique.tolist())
    ds = doc_starts[doc]
    extra = []
    if start > ds:
        extra = [int(t) for t in np.unique(tokens[ds:start]) if int(t) not in in_chunk]
    slots = np.concatenate([chunk_unique, np.asarray(extra, dtype=np.int64)])
    c_base = np.zeros((len(slots), len(rhos)), dtype=np.float32)
    for i, v in enumerate(slots.tolist()):
        hp = pos_dict.get(v)
        if hp is None:
            continue
        j = np.searchsorted(hp, start)
        if j > 0:
            lp = int(hp[j - 1])
            if int(doc_ids[lp]) == doc:
                c_base[i] = states[lp] * (rhos ** np.float32(start - lp))
    return {"chunk": ch, "doc_ids": np.asarray(doc_ids[start:end], dtype=np.int64),
            "unique_slots": slots.astype(np.int64), "inverse_indices": inverse.astype(np.int64),
            "c_base": c_base}


def collate(batch):
    """dynamic_collate_fn (data.py:207-232): (chunks, unique_slots, pad_mask,
    inverse_indices, c_bases, K_max, doc_ids)."""
    B = len(batch)
    L = max(len(it["chunk"]) for it in batch)
    N = batch[0]["c_base"].shape[1]
    K = max(len(it["unique_slots"]) for it in batch)
    chunks = np.zeros((B, L), np.int64)
    docs = np.full((B, L), -1, np.int64)
    slots = np.zeros((B, K), np.int64)
    mask = np.zeros((B, K), bool)
    cb = np.zeros((B, K, N), np.float32)
    inv = np.zeros((B, L), np.int64)
    for i, it in enumerate(batch):
        n, k = len(it["chunk"]), len(it["unique_slots"])
        chunks[i, :n] = it["chunk"]
        docs[i, :n] = it["doc_ids"]
        slots[i, :k] = it["unique_slots"]
        mask[i, :k] = True
        cb[i, :k] = it["c_base"]
        inv[i, :n] = it["inverse_indices"]
    return chunks, slots, mask, inv, cb, K, docs


def token_budget(lengths, token_budget, order, sort_within_batch=True):
    """TokenBudgetSampler._build_batches (data.py:167-192) over a given index order."""
    batches, cur, mx = [], [], 0
    for idx in order:
        n = lengths[idx]
        new_max = max(mx, n)
        if cur and new_max * (len(cur) + 1) > token_budget:
            if sort_within_batch:
                cur.sort(key=lambda i: lengths[i])
            batches.append(cur)
            cur, mx = [idx], n
        else:
            cur.append(idx)
            mx = new_max
    if cur:
        if sort_within_batch:
            cur.sort(key=lambda i: lengths[i])
        batches.append(cur)
    return batches


def states_closed_form(tokens, doc_ids, rhos):
    """float64 brute force of the closed form of corpus_states, for tiny corpora."""
    tokens = list(map(int, tokens))
    seg, s = [], 0
    for i, d in enumerate(doc_ids):
        if i and d != doc_ids[i - 1]:
            s += 1
        seg.append(s)
    rh = np.asarray(rhos, dtype=np.float64)
    out = np.zeros((len(tokens), len(rh)))
    for t in range(len(tokens)):
        for q in range(t + 1):
            if tokens[q] == tokens[t] and seg[q] == seg[t]:
                out[t] += rh ** (t - q)
    return out


def c_base_closed_form(tokens, doc_ids, chunk, slots, rhos):
    """float64 brute force of the closed form of get_item's c_base, for tiny corpora."""
    start, _, doc = chunk
    rh = np.asarray(rhos, dtype=np.float64)
    out = np.zeros((len(slots), len(rh)))
    s = start - 1
    while s >= 0 and int(doc_ids[s]) == doc:             # the chunk's document range
        for i, v in enumerate(slots):
            if int(tokens[s]) == int(v):
                out[i] += rh ** (start - s)
        s -= 1
    return out
