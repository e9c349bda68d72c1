"""TEST INFRASTRUCTURE ONLY: CPU restatement of the EMA scans (the checker).

``query_scan`` and ``boundary_states`` call the plain-C restatement in
``oracle/ema_oracle.c`` (built by ``oracle/Makefile``); the ``*_closed_form``
functions evaluate the closed forms directly in float64 pure Python for tiny
inputs and are what pins the C restatement.
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
