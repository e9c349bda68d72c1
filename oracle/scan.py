"""TEST INFRASTRUCTURE ONLY: CPU restatement of the EMA scans (the checker).

``query_scan`` and ``boundary_states`` call the plain-C restatement in
``oracle/ema_oracle.c`` (built by ``oracle/Makefile``); the ``*_closed_form``
functions evaluate the closed forms directly in float64 pure Python for tiny
inputs and are what pins the C restatement.  ``query_scan_dense_loop`` is the
reference's CPU algorithm itself (dense per-vocabulary state, one step at a time,
vectorised over the batch) in torch: the CPU baseline the benchmark times at full size,
pinned to the C restatement and the known answers in tests/test_oracle_scan.py.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libmbo_oracle.so")
_lib = None


def build():
    """Compile oracle/ema_oracle.c (gcc) into oracle/_build/libmbo_oracle.so."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        lib.mbo_query_scan.argtypes = [p, ctypes.c_int, ctypes.c_int, p, ctypes.c_int,
                                       ctypes.c_int64, p, p, ctypes.c_int, p, p]
        lib.mbo_query_scan.restype = ctypes.c_int
        lib.mbo_boundary_states.argtypes = [p, p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            p, ctypes.c_int, ctypes.c_int, p, p, p]
        lib.mbo_boundary_states.restype = None
        _lib = lib
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _as(a, dtype):
    if a is None:
        return None
    if hasattr(a, "detach"):  # torch tensor
        a = a.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(a), dtype=dtype)


def query_scan(x, rhos, vocab_size, c_init=None, c_init_keys=None, doc_ids=None):
    """C_seq [B, L, N] float32 -- compute_query_ema_history_pt
    (mathbrain/triton_ema_query.py:67-117) restated in C."""
    x = _as(x, np.int64)
    rhos = _as(rhos, np.float32)
    B, L = x.shape
    N = rhos.shape[0]
    if c_init is not None and c_init_keys is not None:
        c_init = _as(c_init, np.float32)
        c_init_keys = _as(c_init_keys, np.int64)
        K = c_init_keys.shape[1]
    else:
        c_init = c_init_keys = None
        K = 0
    doc_ids = _as(doc_ids, np.int64)
    out = np.zeros((B, L, N), dtype=np.float32)
    rc = _load().mbo_query_scan(_ptr(x), B, L, _ptr(rhos), N, int(vocab_size),
                                _ptr(c_init), _ptr(c_init_keys), K, _ptr(doc_ids), _ptr(out))
    if rc != 0:
        raise MemoryError("oracle query scan could not allocate its [V+1, N] state")
    return out


def boundary_states(x, unique, rhos, Br, c_init=None, doc_ids=None):
    """[B, ceil(L/Br), K, N] float32 -- _c_boundary_scan
    (mathbrain/triton_flash_ema.py:29-78) restated in C."""
    x = _as(x, np.int64)
    unique = _as(unique, np.int64)
    rhos = _as(rhos, np.float32)
    B, L = x.shape
    K = unique.shape[1]
    N = rhos.shape[0]
    nc = max(1, -(-L // Br))
    c_init = _as(c_init, np.float32)
    if c_init is not None:
        c_init = np.ascontiguousarray(c_init[:, :, :N])
    doc_ids = _as(doc_ids, np.int64)
    out = np.zeros((B, nc, K, N), dtype=np.float32)
    _load().mbo_boundary_states(_ptr(x), _ptr(unique), B, L, K, _ptr(rhos), N, int(Br),
                                _ptr(c_init), _ptr(doc_ids), _ptr(out))
    return out


def query_scan_closed_form(x, rhos, c_init=None, c_init_keys=None):
    """float64 closed form  C_seq[b,t] = c0[x_t] rho^t + sum_{s<t, x_s=x_t} rho^(t-s),
    where the c0 term is present only when x_t is a key (the last such key wins,
    as a sequential scatter leaves it).  Pure Python: tiny inputs only."""
    x = np.asarray(x, dtype=np.int64)
    rhos = np.asarray(rhos, dtype=np.float64)
    B, L = x.shape
    out = np.zeros((B, L, rhos.shape[0]))
    for b in range(B):
        c0 = {}
        if c_init is not None:
            for k, key in enumerate(np.asarray(c_init_keys)[b]):
                if key != -1:
                    c0[int(key)] = np.asarray(c_init, dtype=np.float64)[b, k]
        for t in range(L):
            v = int(x[b, t])
            acc = c0[v] * rhos ** t if v in c0 else np.zeros_like(rhos)
            for s in range(t):
                if x[b, s] == v:
                    acc = acc + rhos ** (t - s)
            out[b, t] = acc
    return out


def boundary_states_closed_form(x, unique, rhos, Br, c_init=None):
    """float64 closed form C_bound[b,j,k] = c0 rho^(jBr) + sum_{s<jBr, x_s=u_k} rho^(jBr-1-s)."""
    x = np.asarray(x, dtype=np.int64)
    unique = np.asarray(unique, dtype=np.int64)
    rhos = np.asarray(rhos, dtype=np.float64)
    B, L = x.shape
    K = unique.shape[1]
    nc = max(1, -(-L // Br))
    out = np.zeros((B, nc, K, rhos.shape[0]))
    for b in range(B):
        for k in range(K):
            c0 = np.zeros_like(rhos) if c_init is None else np.asarray(c_init, np.float64)[b, k, :rhos.shape[0]]
            for j in range(nc):
                T = j * Br
                acc = c0 * rhos ** T
                for s in range(min(T, L)):
                    if x[b, s] == unique[b, k] and unique[b, k] != -1:
                        acc = acc + rhos ** (T - 1 - s)
                out[b, j, k] = acc
    return out


def boundary_states_f64(x, unique, rhos, Br, c_init=None, doc_ids=None):
    """The same states as ``boundary_states`` in float64, chunk by chunk with numpy:
    S_{j+1} = S_j rho^Br + sum_{s in chunk j, x_s = u_k} rho^((j+1) Br - 1 - s), a document
    change at step s zeroing the state before that step's occurrence (triton_flash_ema.py:
    69-75).  For long sequences, where the fp32 step-by-step restatement accumulates its
    own rounding (one per step) and cannot check a kernel to 1e-5; pinned to the closed
    form and to the fp32 restatement on short inputs (tests/test_oracle_scan.py)."""
    x = np.asarray(_as(x, np.int64))
    unique = np.asarray(_as(unique, np.int64))
    rhos = np.asarray(_as(rhos, np.float32), dtype=np.float64)
    B, L = x.shape
    K = unique.shape[1]
    N = rhos.shape[0]
    nc = max(1, -(-L // Br))
    out = np.zeros((B, nc, K, N))
    logr = np.log(rhos)
    for b in range(B):
        S = np.zeros((K, N)) if c_init is None else np.asarray(_as(c_init, np.float64))[b, :, :N].copy()
        valid = unique[b] != -1
        doc = None if doc_ids is None else np.asarray(_as(doc_ids, np.int64))[b]
        for j in range(nc):
            out[b, j] = S
            t0, t1 = j * Br, min((j + 1) * Br, L)
            if t0 >= t1:
                continue
            n = t1 - t0
            steps = np.arange(t0, t1)
            keep_from = 0  # the last document change in the chunk drops what came before
            if doc is not None:
                chg = [s for s in steps if s > 0 and doc[s] != doc[s - 1]]
                if chg:
                    keep_from = chg[-1] - t0
                    S = np.zeros_like(S)
            hits = (x[b, t0:t1][None, :] == unique[b][:, None]) & valid[:, None]   # [K, n]
            hits[:, :keep_from] = False
            w = np.exp(np.outer(np.arange(n - 1, -1, -1), logr))                  # rho^(n-1-i) [n, N]
            S = S * np.exp(n * logr)[None, :] + hits.astype(np.float64) @ w
            if n < Br and j + 1 < nc:
                raise AssertionError("only the last chunk can be short")
    return out


def query_scan_dense_loop(x, rhos, vocab_size, c_init=None, c_init_keys=None, doc_ids=None):
    """C_seq [B, L, N] float32 by the algorithm of compute_query_ema_history_pt
    (mathbrain/triton_ema_query.py:67-117): per-vocabulary tables of the last position
    (-1e6 when unseen), the last counter row and the last document, a padding key -1 sent to
    the spare row V (:84-88); at each step the row of x_t is decayed by rho^(t - T_last),
    zeroed if its last occurrence was in another document, stored, and written back + 1
    (:94-115).  torch, float32, on the CPU."""
    import torch
    x = torch.as_tensor(x).long()
    rh = torch.as_tensor(rhos, dtype=torch.float32)
    B, L = x.shape
    N = rh.shape[0]
    C_seq = torch.zeros(B, L, N, dtype=torch.float32)
    T_last = torch.full((B, vocab_size + 1), -1000000.0, dtype=torch.float32)
    C_last = torch.zeros(B, vocab_size + 1, N, dtype=torch.float32)
    D_last = torch.full((B, vocab_size + 1), -1, dtype=torch.int32)
    if c_init is not None and c_init_keys is not None:
        keys = torch.as_tensor(c_init_keys).long()
        keys = torch.where(keys == -1, torch.full_like(keys, vocab_size), keys)
        T_last.scatter_(1, keys, 0.0)
        C_last.scatter_(1, keys.unsqueeze(-1).expand(-1, -1, N),
                        torch.as_tensor(c_init, dtype=torch.float32))
        if doc_ids is not None:
            first = torch.as_tensor(doc_ids)[:, :1].to(torch.int32).expand_as(keys)
            D_last.scatter_(1, keys, first)
    docs = None if doc_ids is None else torch.as_tensor(doc_ids).to(torch.int32)
    bi = torch.arange(B)
    for t in range(L):
        xt = x[:, t]
        tl = T_last[bi, xt]
        c = C_last[bi, xt] * rh.unsqueeze(0) ** (t - tl).unsqueeze(1)
        if docs is not None:
            same = (D_last[bi, xt] == docs[:, t]) | (tl < 0)
            c = c * same.unsqueeze(1).float()
            D_last[bi, xt] = docs[:, t]
        C_seq[:, t] = c
        T_last[bi, xt] = float(t)
        C_last[bi, xt] = c + 1.0
    return C_seq.numpy()
