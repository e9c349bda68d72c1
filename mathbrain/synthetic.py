"""Seeded synthetic batches shaped like the reference's data pipeline output.

Tokens are drawn from a truncated Zipf(alpha) law over ranks 1..V (p ~ r^-alpha) and
mapped to ids through a seeded permutation, so id 0 is not special.  Each sequence gets
a warm-up history of W tokens; as in mathbrain/data.py:95-148 its slots are the sorted
unique chunk tokens followed by the sorted history-only tokens, and c_base is the
history's EMA state decayed to the chunk start,
    c_base[k] = sum_{s<W} rho^(W-s) I(h_s = u_k)
(the data.py convention: the state after the last occurrence, times rho^(start-last)).
Slot lists are padded with -1 and c_base with zeros, never with a real id.
"""
import math

import torch


def rhos_from_half_lives(N, min_hl, max_hl):
    """model.py:128-130: rho = exp(-ln 2 / logspace(log10 min_hl, log10 max_hl, N))."""
    hl = torch.logspace(math.log10(min_hl), math.log10(max_hl), N, dtype=torch.float64)
    return torch.exp(-math.log(2.0) / hl).to(torch.float32)


def zipf_tokens(shape, V, alpha, gen, perm):
    """Ids with P(rank r) ~ r^-alpha over r = 1..V, ranks mapped through `perm`."""
    r = torch.arange(1, V + 1, dtype=torch.float64)
    cdf = torch.cumsum(r.pow(-alpha), 0)
    cdf = cdf / cdf[-1]
    u = torch.rand(shape, generator=gen, dtype=torch.float64)
    rank = torch.searchsorted(cdf, u).clamp(max=V - 1)
    return perm[rank]


def make_batch(B, T, V, N, warmup, alpha=1.1, min_hl=1.0, max_hl=4096.0, seed=0,
               uniform=False, pad_frac=0.0):
    """Returns a dict with x [B,T] int64, unique [B,K_max] int64 (-1 padded), c_base
    [B,K_max,N] fp32, counts [B] (valid slots), rhos [N], pad_len [B] (tail positions
    holding token 0 for the padding-mask configuration, 0 otherwise).  CPU tensors."""
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(V, generator=gen)
    rhos = rhos_from_half_lives(N, min_hl, max_hl)
    if uniform:
        x = torch.randint(0, V, (B, T), generator=gen)
        hist = torch.randint(0, V, (B, warmup), generator=gen)
    else:
        x = zipf_tokens((B, T), V, alpha, gen, perm)
        hist = zipf_tokens((B, warmup), V, alpha, gen, perm)
    pad_len = torch.zeros(B, dtype=torch.int64)
    if pad_frac > 0:
        frac = torch.rand(B, generator=gen, dtype=torch.float64) * pad_frac
        pad_len = (frac * T).floor().to(torch.int64)
        for b in range(B):
            if pad_len[b] > 0:
                x[b, T - pad_len[b]:] = 0  # data.py:218 pads chunks with token 0
    slots, cbs = [], []
    w = rhos.double().unsqueeze(0).pow(torch.arange(warmup, 0, -1, dtype=torch.float64).unsqueeze(1))
    for b in range(B):
        cu = torch.unique(x[b])
        if warmup > 0:
            hu, inv = torch.unique(hist[b], return_inverse=True)
            state_h = torch.zeros(hu.numel(), N, dtype=torch.float64).index_add_(0, inv, w)
            extra = hu[~torch.isin(hu, cu)]
        else:
            hu = torch.empty(0, dtype=torch.int64)
            state_h = torch.zeros(0, N, dtype=torch.float64)
            extra = hu
        s = torch.cat([cu, extra])
        cb = torch.zeros(s.numel(), N, dtype=torch.float64)
        if hu.numel():
            idx = torch.searchsorted(hu, s).clamp(max=hu.numel() - 1)
            hit = hu[idx] == s
            cb[hit] = state_h[idx[hit]]
        slots.append(s)
        cbs.append(cb.to(torch.float32))
    counts = torch.tensor([s.numel() for s in slots], dtype=torch.int64)
    K_max = int(counts.max())
    unique = torch.full((B, K_max), -1, dtype=torch.int64)
    c_base = torch.zeros(B, K_max, N, dtype=torch.float32)
    for b in range(B):
        unique[b, :counts[b]] = slots[b]
        c_base[b, :counts[b]] = cbs[b]
    return dict(x=x, unique=unique, c_base=c_base, counts=counts, rhos=rhos, pad_len=pad_len,
                history=hist)


def make_doc_batch(B, T, V, N, alpha=1.1, median_len=1500, sigma=1.0, min_hl=1.0, max_hl=4096.0,
                   seed=0, max_history=8192):
    """Chunks of synthetic documents, shaped like the reference's training batches
    (mathbrain/data.py:95-148, collate :211-235).  Each row is one chunk of a document
    whose length is lognormal (median ``median_len``); the chunk starts at a random
    multiple of T inside the document, the tokens before it (at most ``max_history``)
    are its history, and a chunk that runs past the document end is padded with token 0
    and masked (``targets`` = -1, as train.py:320-323 masks padding).  Returns the
    make_batch dict plus ``targets`` [B, T] (next token or -1) and ``lengths`` [B]."""
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(V, generator=gen)
    rhos = rhos_from_half_lives(N, min_hl, max_hl)
    xs, hists, lens = [], [], []
    for b in range(B):
        Ld = int(math.exp(math.log(median_len) + sigma * float(torch.randn(1, generator=gen))))
        Ld = max(2, min(Ld, max_history + T))
        n_chunks = (Ld + T - 1) // T
        start = T * int(torch.randint(0, n_chunks, (1,), generator=gen))
        doc = zipf_tokens((Ld + 1,), V, alpha, gen, perm)
        chunk = doc[start:min(start + T + 1, Ld + 1)]
        hists.append(doc[max(0, start - max_history):start])
        xs.append(chunk)
        lens.append(min(T, chunk.numel() - 1))
    x = torch.zeros(B, T, dtype=torch.int64)
    targets = torch.full((B, T), -1, dtype=torch.int64)
    for b in range(B):
        n = lens[b]
        x[b, :n] = xs[b][:n]
        targets[b, :n] = xs[b][1:n + 1]
    slots, cbs = [], []
    for b in range(B):
        cu = torch.unique(x[b, :lens[b]])
        h = hists[b]
        W = h.numel()
        if W:
            w = rhos.double().unsqueeze(0).pow(torch.arange(W, 0, -1, dtype=torch.float64).unsqueeze(1))
            hu, inv = torch.unique(h, return_inverse=True)
            state_h = torch.zeros(hu.numel(), N, dtype=torch.float64).index_add_(0, inv, w)
            s = torch.cat([cu, hu[~torch.isin(hu, cu)]])
            cb = torch.zeros(s.numel(), N, dtype=torch.float64)
            idx = torch.searchsorted(hu, s).clamp(max=hu.numel() - 1)
            hit = hu[idx] == s
            cb[hit] = state_h[idx[hit]]
        else:
            s = cu
            cb = torch.zeros(s.numel(), N, dtype=torch.float64)
        slots.append(s)
        cbs.append(cb.to(torch.float32))
    counts = torch.tensor([s.numel() for s in slots], dtype=torch.int64)
    K_max = int(counts.max())
    unique = torch.full((B, K_max), -1, dtype=torch.int64)
    c_base = torch.zeros(B, K_max, N, dtype=torch.float32)
    for b in range(B):
        unique[b, :counts[b]] = slots[b]
        c_base[b, :counts[b]] = cbs[b]
    return dict(x=x, unique=unique, c_base=c_base, counts=counts, rhos=rhos, targets=targets,
                lengths=torch.tensor(lens, dtype=torch.int64))


def zipf_corpus(T, V, alpha=1.1, median_len=1500, sigma=1.0, seed=0):
    """A flat synthetic corpus shaped like preprocess_corpus's input (mathbrain/data.py:
    254-260): documents of lognormal length (median ``median_len``, at least 1 token)
    with Zipf(alpha) tokens, cut to T tokens in all.  Returns (tokens int32 [T], doc_ids
    int32 [T]) as numpy arrays, doc ids counting up from 0."""
    import numpy as np
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(V, generator=gen)
    tokens = zipf_tokens((T,), V, alpha, gen, perm).to(torch.int32).numpy()
    rng = np.random.default_rng(seed)
    lens = []
    total = 0
    while total < T:
        n = max(1, int(np.exp(np.log(median_len) + sigma * rng.standard_normal())))
        n = min(n, T - total)
        lens.append(n)
        total += n
    doc_ids = np.repeat(np.arange(len(lens), dtype=np.int32), lens)
    return tokens, doc_ids
