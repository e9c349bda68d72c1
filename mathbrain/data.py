"""Document-aware training data for the Per-Slot EMA model, kept on the GPU.

Drop-in for mathbrain/data.py: ``preprocess_corpus`` (:242-320), ``WikiTextMMapDataset``
(:24-148), ``TokenBudgetSampler`` (:151-202) and ``dynamic_collate_fn`` (:205-232), with
the same on-disk format (tokens.bin int32, doc_ids.bin int32, states.bin float32
[T, N], pos_dict.pkl) and the same sample and batch contents.

The MI355X form keeps the corpus resident in HBM (tokens, document ids, a
next-occurrence index and the [T, N] state rows: 4*(3 + N) bytes per token, about 31 GB
for a 120 M-token corpus at N = 64) and builds every sample or batch there:
``mb_slot_lists`` finds each chunk's slots (its own tokens, then the tokens of its
document's history, data.py:101-125) and ``mb_slot_batch`` writes the padded batch with
c_base (data.py:127-140, 207-232).  The corpus states themselves come from the
``mb_corpus_states`` scan (data.py:276-303).  There is no CPU path: the per-sample and
per-batch calls raise without a GPU.  Index building, chunking and batching (host
bookkeeping over chunk descriptors) run on the host as in the reference.
"""
import os
import pickle

import numpy as np
import torch
from torch.utils.data import Dataset, Sampler

from . import _lib

INT32_MAX = 2**31 - 1


def _rhos(N, min_hl, max_hl):
    """Decay rates written by the preprocessing step (data.py:268-270)."""
    scales = np.logspace(np.log10(min_hl), np.log10(max_hl), N)
    return np.exp(-np.log(2.0) / scales).astype(np.float32)


def _device(device):
    if device is None:
        if not torch.cuda.is_available():
            raise NotImplementedError(
                "mathbrain.data builds samples on an MI355X GPU; none is visible "
                "(this implementation has no CPU path)")
        return torch.device("cuda", torch.cuda.current_device())
    device = torch.device(device)
    if device.type != "cuda":
        raise NotImplementedError(f"mathbrain.data: device {device} is not a GPU; "
                                  "this implementation has no CPU path")
    return device


def _segments(doc_ids):
    """Document segment of each position: +1 wherever the document id changes."""
    seg = torch.zeros_like(doc_ids, dtype=torch.int32)
    if doc_ids.numel() > 1:
        seg[1:] = torch.cumsum((doc_ids[1:] != doc_ids[:-1]).to(torch.int32), 0, dtype=torch.int32)
    return seg


def sorted_occurrences(tokens):
    """(sorted tokens, positions sorted by token with ascending positions per token)."""
    srt, order = torch.sort(tokens, stable=True)
    return srt, order


def next_occurrence(tokens, srt=None, order=None):
    """Position of the next occurrence of each position's token (INT32_MAX if none)."""
    if order is None:
        srt, order = sorted_occurrences(tokens)
    nxt = torch.full_like(tokens, INT32_MAX, dtype=torch.int32)
    if tokens.numel() > 1:
        same = srt[1:] == srt[:-1]
        nxt[order[:-1][same]] = order[1:][same].to(torch.int32)
    return nxt


def chain_order(tokens, doc_ids):
    """(sorted keys, positions) of a stable sort by (document segment, token): the chains
    of one token inside one document that the state scan walks."""
    key = (_segments(doc_ids).to(torch.int64) << 32) | (tokens.to(torch.int64) & 0xFFFFFFFF)
    return torch.sort(key, stable=True)


def corpus_states(tokens, doc_ids, rhos):
    """EMA state of each position's token just after that occurrence, restarted at every
    change of document id (the preprocessing scan, data.py:276-303):

        states[t] = sum_{s <= t, tokens[s] = tokens[t], same document segment} rho^(t-s)

    tokens [T] int32 (ids >= 0), doc_ids [T] int32, rhos [N] float32, on the GPU.
    Returns [T, N] float32.
    """
    dev = _lib.require_gpu(tokens, doc_ids, rhos, what="corpus_states")
    T = tokens.numel()
    N = rhos.numel()
    rh = rhos.detach().to(torch.float32).contiguous()
    states = torch.empty(T, N, dtype=torch.float32, device=dev)
    if T == 0:
        return states
    chain, order = chain_order(tokens.reshape(-1), doc_ids.reshape(-1))
    ws = _lib.lib().mb_corpus_states_workspace(T, N)
    work = torch.empty(max(int(ws), 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.call("mb_corpus_states", _lib.ptr(order), _lib.ptr(chain), T, _lib.ptr(rh), N,
                  _lib.ptr(states), _lib.ptr(work), int(ws), _lib.stream(dev))
    return states


def preprocess_corpus(documents: list, data_dir: str, N: int = 64, min_hl: float = 1.0,
                      max_hl: float = 2048.0, device=None):
    """Flattens the documents and writes tokens.bin, doc_ids.bin, states.bin and
    pos_dict.pkl into data_dir, as mathbrain/data.py:242-320 does; the state scan runs on
    the GPU (``corpus_states``)."""
    dev = _device(device)
    os.makedirs(data_dir, exist_ok=True)
    lens = [len(d) for d in documents]
    tokens = np.fromiter((t for d in documents for t in d), dtype=np.int32, count=sum(lens))
    doc_ids = np.repeat(np.arange(len(documents), dtype=np.int32), lens)
    if len(tokens) and int(tokens.min()) < 0:
        raise ValueError("preprocess_corpus: negative token ids")
    tokens.tofile(os.path.join(data_dir, "tokens.bin"))
    doc_ids.tofile(os.path.join(data_dir, "doc_ids.bin"))
    rhos = _rhos(N, min_hl, max_hl)
    T = len(tokens)
    print(f"Preprocessing {T} tokens across {len(documents)} documents...")
    tok_d = torch.from_numpy(tokens).to(dev)
    states = corpus_states(tok_d, torch.from_numpy(doc_ids).to(dev), torch.from_numpy(rhos).to(dev))
    with open(os.path.join(data_dir, "states.bin"), "wb") as f:
        step = max(1, (1 << 28) // (4 * N))  # 256 MB of rows per host copy
        for s in range(0, T, step):
            f.write(states[s:s + step].cpu().numpy().tobytes())
    del states
    # pos_dict: token -> int32 array of its global positions (data.py:281, 293, 311-315)
    srt, order = sorted_occurrences(tok_d)
    srt_h = srt.cpu().numpy()
    order_h = order.to(torch.int32).cpu().numpy()
    cuts = np.flatnonzero(srt_h[1:] != srt_h[:-1]) + 1
    keys = srt_h[np.concatenate([[0], cuts])] if T else np.zeros(0, np.int32)
    pos_dict = {int(k): p for k, p in zip(keys, np.split(order_h, cuts))} if T else {}
    with open(os.path.join(data_dir, "pos_dict.pkl"), "wb") as f:
        pickle.dump(pos_dict, f)
    print(f"  tokens: {T} ({os.path.getsize(os.path.join(data_dir, 'tokens.bin')) / 1024**2:.2f} MB), "
          f"states: {os.path.getsize(os.path.join(data_dir, 'states.bin')) / 1024**3:.2f} GB")


def chunk_index(doc_ids, block_size):
    """Chunks of each document (data.py:48-84): (starts, ends, doc ids) int64 arrays and
    doc_starts {doc_id: first position}.  Documents shorter than two tokens are skipped;
    a chunk holds up to block_size + 1 tokens and overlaps the next by one."""
    d = np.asarray(doc_ids)
    T = len(d)
    empty = np.zeros(0, np.int64)
    if T == 0:
        return empty, empty, empty, {}
    brk = np.flatnonzero(d[1:] != d[:-1]) + 1
    rs = np.concatenate([[0], brk]).astype(np.int64)
    re_ = np.concatenate([brk, [T]]).astype(np.int64)
    ids = d[rs].astype(np.int64)
    if len(np.unique(ids)) != len(ids):
        raise ValueError("doc_ids must hold each document as one contiguous range "
                         "(as preprocess_corpus writes them)")
    lens = re_ - rs
    keep = lens >= 2
    rs, re_, ids, lens = rs[keep], re_[keep], ids[keep], lens[keep]
    doc_starts = {int(i): int(s) for i, s in zip(ids, rs)}
    nch = np.maximum(1, (lens - 1 + block_size - 1) // block_size)
    owner = np.repeat(np.arange(len(rs)), nch)
    first = np.repeat(np.cumsum(nch) - nch, nch)
    c = np.arange(int(nch.sum()), dtype=np.int64) - first
    cs = rs[owner] + c * block_size
    ce = np.minimum(cs + block_size + 1, re_[owner])
    ok = ce - cs >= 2
    return cs[ok], ce[ok], ids[owner][ok], doc_starts


class WikiTextMMapDataset(Dataset):
    """Chunks of a preprocessed corpus (mathbrain/data.py:24-148).

    ``ds[i]`` returns the reference's sample dict (chunk, doc_ids, unique_slots,
    inverse_indices, c_base) as tensors on the GPU; ``ds.get_batch(indices)`` returns
    ``dynamic_collate_fn`` of those samples in one device call.  ``device`` picks the GPU
    (default: the current one); the corpus is copied there on first use.
    """

    def __init__(self, cache_dir, block_size, rhos, in_memory=True, device=None):
        self.block_size = block_size
        self.N = rhos.shape[0]
        self.rhos = rhos
        self.tokens = np.memmap(os.path.join(cache_dir, "tokens.bin"), dtype=np.int32, mode="r")
        self.doc_ids = np.memmap(os.path.join(cache_dir, "doc_ids.bin"), dtype=np.int32, mode="r")
        states_path = os.path.join(cache_dir, "states.bin")
        if in_memory:
            self.states = np.fromfile(states_path, dtype=np.float32).reshape(len(self.tokens), self.N)
        else:
            self.states = np.memmap(states_path, dtype=np.float32, mode="r",
                                    shape=(len(self.tokens), self.N))
        T = len(self.tokens)
        if T and int(self.tokens.min()) < 0:
            raise ValueError("tokens.bin holds negative token ids")
        self.V = int(self.tokens.max()) + 1 if T else 1
        self._cs, self._ce, self._cd, self.doc_starts = chunk_index(self.doc_ids, block_size)
        self._cds = np.asarray([self.doc_starts[int(d)] for d in self._cd], dtype=np.int64)
        self.chunks = list(zip(self._cs.tolist(), self._ce.tolist(), self._cd.tolist()))
        self._device = device
        self._dev = None
        self._pos_dict = None
        print(f"Dataset: {len(self.doc_starts)} docs, {len(self.chunks)} chunks, "
              f"block_size={block_size}, {int((self._ce - self._cs).sum())} useful tokens")

    def __len__(self):
        return len(self.chunks)

    def chunk_len(self, idx):
        """Token length of chunk idx (for token-budget batching)."""
        return int(self._ce[idx] - self._cs[idx])

    @property
    def pos_dict(self):
        """token -> int32 array of its positions (pos_dict.pkl's content), built from
        tokens.bin on first use."""
        if self._pos_dict is None:
            tok = np.asarray(self.tokens)
            order = np.argsort(tok, kind="stable").astype(np.int32)
            srt = tok[order]
            cuts = np.flatnonzero(srt[1:] != srt[:-1]) + 1
            keys = srt[np.concatenate([[0], cuts])] if len(tok) else []
            self._pos_dict = {int(k): p for k, p in zip(keys, np.split(order, cuts))}
        return self._pos_dict

    def _resident(self):
        """The corpus in HBM: tokens, document ids, next-occurrence index, states, rates."""
        if self._dev is None:
            dev = _device(self._device)
            tok = torch.from_numpy(np.array(self.tokens)).to(dev)
            docs = torch.from_numpy(np.array(self.doc_ids)).to(dev)
            T = tok.numel()
            states = torch.empty(T, self.N, dtype=torch.float32, device=dev)
            step = max(1, (1 << 28) // (4 * self.N))
            for s in range(0, T, step):
                states[s:s + step].copy_(torch.from_numpy(np.ascontiguousarray(self.states[s:s + step])))
            rh = torch.as_tensor(self.rhos, dtype=torch.float32).detach().reshape(-1).to(dev)
            self._dev = dict(device=dev, tokens=tok, doc_ids=docs, next=next_occurrence(tok),
                             states=states, rhos=rh.contiguous())
        return self._dev

    def get_batch(self, indices):
        """dynamic_collate_fn([self[i] for i in indices]) built on the GPU:
        (chunks, unique_slots, pad_mask, inverse_indices, c_bases, K_max, doc_ids)."""
        r = self._resident()
        dev = r["device"]
        idx = np.asarray(indices, dtype=np.int64)
        B = len(idx)
        if B == 0:
            raise ValueError("get_batch: empty batch")
        desc = np.stack([self._cds[idx], self._cs[idx], self._ce[idx]])
        L = int((desc[2] - desc[1]).max())
        d = torch.from_numpy(desc).to(dev)
        T, V, N = r["tokens"].numel(), self.V, self.N
        last = torch.empty(B, V, dtype=torch.int32, device=dev)
        slot_of = torch.empty(B, V, dtype=torch.int32, device=dev)
        slot_tok = torch.empty(B, V, dtype=torch.int64, device=dev)
        counts = torch.empty(B, 2, dtype=torch.int32, device=dev)
        st = _lib.stream(dev)
        with torch.cuda.device(dev):
            _lib.call("mb_slot_lists", _lib.ptr(r["tokens"]), _lib.ptr(r["next"]), T, V,
                      _lib.ptr(d[0]), _lib.ptr(d[1]), _lib.ptr(d[2]), B, _lib.ptr(last),
                      _lib.ptr(slot_of), _lib.ptr(slot_tok), _lib.ptr(counts), st)
            K_max = int(counts[:, 1].max().item())
            chunks = torch.empty(B, L, dtype=torch.int64, device=dev)
            docs = torch.empty(B, L, dtype=torch.int64, device=dev)
            inv = torch.empty(B, L, dtype=torch.int64, device=dev)
            slots = torch.empty(B, K_max, dtype=torch.int64, device=dev)
            mask = torch.empty(B, K_max, dtype=torch.bool, device=dev)
            c_base = torch.empty(B, K_max, N, dtype=torch.float32, device=dev)
            _lib.call("mb_slot_batch", _lib.ptr(r["tokens"]), _lib.ptr(r["doc_ids"]),
                      _lib.ptr(r["states"]), _lib.ptr(r["rhos"]), N, T, V, _lib.ptr(d[0]),
                      _lib.ptr(d[1]), _lib.ptr(d[2]), B, _lib.ptr(last), _lib.ptr(slot_of),
                      _lib.ptr(slot_tok), _lib.ptr(counts), L, K_max, _lib.ptr(chunks),
                      _lib.ptr(docs), _lib.ptr(slots), _lib.ptr(mask), _lib.ptr(inv),
                      _lib.ptr(c_base), st)
        return chunks, slots, mask, inv, c_base, K_max, docs

    def __getitem__(self, idx):
        chunks, slots, mask, inv, c_base, K, docs = self.get_batch([idx])
        n = self.chunk_len(idx)
        return {"chunk": chunks[0, :n], "doc_ids": docs[0, :n], "unique_slots": slots[0, :K],
                "inverse_indices": inv[0, :n], "c_base": c_base[0, :K]}


class TokenBudgetSampler(Sampler):
    """Batches of chunk indices under a padded-token budget (data.py:151-202): greedy
    packing of a (shuffled) order, sorted by length within each batch."""

    def __init__(self, dataset, token_budget, shuffle=True, sort_within_batch=True):
        self.dataset = dataset
        self.token_budget = token_budget
        self.shuffle = shuffle
        self.sort_within_batch = sort_within_batch
        self.lengths = [dataset.chunk_len(i) for i in range(len(dataset))]
        self._build_batches()

    def _build_batches(self):
        indices = list(range(len(self.dataset)))
        if self.shuffle:
            import random
            random.shuffle(indices)
        self.batches = []
        cur, mx = [], 0
        for idx in indices:
            n = self.lengths[idx]
            new_max = max(mx, n)
            if cur and new_max * (len(cur) + 1) > self.token_budget:
                if self.sort_within_batch:
                    cur.sort(key=lambda i: self.lengths[i])
                self.batches.append(cur)
                cur, mx = [idx], n
            else:
                cur.append(idx)
                mx = new_max
        if cur:
            if self.sort_within_batch:
                cur.sort(key=lambda i: self.lengths[i])
            self.batches.append(cur)

    def __iter__(self):
        if self.shuffle:
            self._build_batches()
        yield from self.batches

    def __len__(self):
        return len(self.batches)


def dynamic_collate_fn(batch):
    """Pads samples to the batch maxima (data.py:205-232); the tensors stay on the
    samples' device.  Returns (chunks, unique_slots, pad_mask, inverse_indices, c_bases,
    K_max, doc_ids)."""
    B = len(batch)
    dev = batch[0]["chunk"].device
    L = max(it["chunk"].shape[0] for it in batch)
    N = batch[0]["c_base"].shape[1]
    K_max = max(it["unique_slots"].shape[0] for it in batch)
    chunks = torch.zeros(B, L, dtype=torch.long, device=dev)
    doc_ids = torch.full((B, L), -1, dtype=torch.long, device=dev)
    unique_slots = torch.zeros(B, K_max, dtype=torch.long, device=dev)
    pad_mask = torch.zeros(B, K_max, dtype=torch.bool, device=dev)
    c_bases = torch.zeros(B, K_max, N, dtype=torch.float32, device=dev)
    inverse_indices = torch.zeros(B, L, dtype=torch.long, device=dev)
    for i, it in enumerate(batch):
        n = it["chunk"].shape[0]
        k = it["unique_slots"].shape[0]
        chunks[i, :n] = it["chunk"]
        doc_ids[i, :n] = it["doc_ids"]
        unique_slots[i, :k] = it["unique_slots"]
        pad_mask[i, :k] = True
        c_bases[i, :k] = it["c_base"]
        inverse_indices[i, :n] = it["inverse_indices"]
    return chunks, unique_slots, pad_mask, inverse_indices, c_bases, K_max, doc_ids


class SlotBatchLoader:
    """Iterates a batch sampler (e.g. TokenBudgetSampler) and yields each batch from
    ``dataset.get_batch``: the device-side replacement of
    DataLoader(dataset, batch_sampler=sampler, collate_fn=dynamic_collate_fn)."""

    def __init__(self, dataset, batch_sampler):
        self.dataset = dataset
        self.batch_sampler = batch_sampler

    def __iter__(self):
        for indices in self.batch_sampler:
            yield self.dataset.get_batch(indices)

    def __len__(self):
        return len(self.batch_sampler)
