"""Pins the CPU oracle of the EMA scans (oracle/scan.py, oracle/ema_oracle.c).

Known answers are the reference's own (tests/test_doc_boundary.py,
tests/test_pipeline_thorough.py, tests/test_gold_standard.py); the rest are
closed forms evaluated independently in float64.
"""
import math

import numpy as np
import pytest

from oracle import scan


def rhos_logspace(N, lo, hi):
    """model.py:128-130 / data.py:267-269: rho = exp(-ln2 / logspace(lo, hi, N))."""
    hl = np.logspace(math.log10(lo), math.log10(hi), N)
    return np.exp(-np.log(2.0) / hl).astype(np.float32)


# ---- reference known answers -------------------------------------------------

def test_kat_within_doc_continuity():
    # tests/test_doc_boundary.py:71-105
    x = np.array([[0, 1, 0, 2, 0, 1]])
    doc = np.zeros_like(x)
    rhos = np.array([0.9, 0.5], np.float32)
    C = scan.query_scan(x, rhos, 3, doc_ids=doc)
    assert np.allclose(C[0, 0], 0.0)
    assert np.allclose(C[0, 2], rhos ** 2, atol=1e-5)
    assert np.allclose(C[0, 4], (rhos ** 2 + 1.0) * rhos ** 2, atol=1e-5)


def test_kat_c_base_undecayed_at_t0():
    # tests/test_doc_boundary.py:108-134: c_base is used undecayed at t=0
    x = np.array([[0, 1, 0, 2]])
    rhos = np.array([0.9, 0.5], np.float32)
    c_init = np.array([[[2.0, 1.5], [0.0, 0.0], [0.0, 0.0]]], np.float32)
    keys = np.array([[0, 1, 2]])
    C = scan.query_scan(x, rhos, 3, c_init, keys, doc_ids=np.zeros_like(x))
    assert np.allclose(C[0, 0], [2.0, 1.5], atol=1e-5)
    # and the second occurrence carries (c0 + 1) decayed twice
    assert np.allclose(C[0, 2], (np.array([2.0, 1.5]) + 1.0) * rhos ** 2, atol=1e-5)


def test_kat_cross_doc_isolation():
    # tests/test_doc_boundary.py:22-68
    x = np.array([[0, 1, 2, 0, 1, 0, 1, 3, 0, 1]])
    doc = np.array([[0, 0, 0, 0, 0, 1, 1, 1, 1, 1]])
    rhos = np.array([0.9, 0.8, 0.7, 0.6], np.float32)
    Cw = scan.query_scan(x, rhos, 5, doc_ids=doc)
    Cwo = scan.query_scan(x, rhos, 5)
    assert np.allclose(Cw[0, 5], 0.0)
    assert np.abs(Cwo[0, 5]).sum() > 0
    assert np.allclose(Cw[0, 8], rhos ** 3, atol=1e-5)


def test_kat_batch_mixed_docs():
    # tests/test_doc_boundary.py:244-277
    x = np.array([[0, 1, 2, 0, 1, 2, 0, 1], [0, 1, 2, 0, 0, 1, 2, 0]])
    doc = np.array([[0] * 8, [0, 0, 0, 0, 1, 1, 1, 1]])
    C = scan.query_scan(x, np.array([0.9, 0.5], np.float32), 5, doc_ids=doc)
    assert np.abs(C[0, 6]).sum() > 0
    assert np.allclose(C[1, 4], 0.0, atol=1e-6)


def test_kat_manual_loop_and_same_recency():
    # tests/test_pipeline_thorough.py:191-271 (manual loop) and :394-463 (same
    # recency pattern gives the same value whichever token it is)
    rhos = rhos_logspace(4, 1.0, 16.0)
    tokens = [1, 2, 1, 3, 1, 2, 1]
    manual = np.zeros((7, 4), np.float32)
    state = np.zeros((4, 4), np.float32)
    last = np.full(4, -1000000)
    for t, v in enumerate(tokens):
        state[v] = state[v] * rhos ** (t - last[v]) if last[v] >= 0 else 0.0
        manual[t] = state[v]
        state[v] += 1.0
        last[v] = t
    C = scan.query_scan(np.array([tokens]), rhos, 4)
    assert np.abs(C[0] - manual).max() < 1e-4
    a = scan.query_scan(np.array([[1, 2, 3, 1, 2]]), rhos, 4)
    b = scan.query_scan(np.array([[2, 1, 3, 2, 1]]), rhos, 4)
    assert np.allclose(a[0, 3], b[0, 3], atol=1e-4)
    assert np.allclose(a[0, 1], 0.0) and np.allclose(b[0, 1], 0.0)


# ---- closed forms --------------------------------------------------------------

@pytest.mark.parametrize("seed", [0, 1, 2])
def test_query_scan_closed_form(seed):
    rng = np.random.default_rng(seed)
    B, L, V, N = 3, 40, 7, 5
    x = rng.integers(0, V, size=(B, L))
    rhos = rhos_logspace(N, 1.0, 64.0)
    keys = np.stack([rng.permutation(V)[:4] for _ in range(B)])
    keys[0, -1] = -1
    c_init = rng.random((B, 4, N)).astype(np.float32) * 3
    got = scan.query_scan(x, rhos, V, c_init, keys)
    want = scan.query_scan_closed_form(x, rhos, c_init, keys)
    assert np.allclose(got, want, rtol=2e-6, atol=1e-6)


def test_query_scan_repeated_key_last_wins():
    x = np.array([[3, 3, 1]])
    rhos = np.array([0.5, 0.9], np.float32)
    keys = np.array([[3, 1, 3]])
    c_init = np.array([[[1.0, 1.0], [0.0, 0.0], [4.0, 8.0]]], np.float32)
    C = scan.query_scan(x, rhos, 5, c_init, keys)
    assert np.allclose(C[0, 0], [4.0, 8.0])


@pytest.mark.parametrize("Br", [1, 3, 8, 64])
def test_boundary_closed_form(Br):
    rng = np.random.default_rng(Br)
    B, L, V, N, K = 2, 30, 9, 4, 6
    x = rng.integers(0, V, size=(B, L))
    unique = np.stack([rng.permutation(V)[:K] for _ in range(B)])
    unique[1, -2:] = -1
    rhos = rhos_logspace(N, 1.0, 32.0)
    c_init = rng.random((B, K, N)).astype(np.float32)
    got = scan.boundary_states(x, unique, rhos, Br, c_init)
    want = scan.boundary_states_closed_form(x, unique, rhos, Br, c_init)
    assert got.shape == (B, max(1, -(-L // Br)), K, N)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_boundary_doc_reset():
    # triton_flash_ema.py:69-75: the state is zeroed when the document changes
    x = np.array([[0, 1, 0, 1, 0, 1]])
    doc = np.array([[0, 0, 0, 1, 1, 1]])
    unique = np.array([[0, 1]])
    rhos = np.array([0.5], np.float32)
    got = scan.boundary_states(x, unique, rhos, 3, doc_ids=doc)
    # chunk 1 starts at t=3, after the last doc-0 step; doc reset happens at t=3
    assert np.allclose(got[0, 1, 0], [0.5 ** 2 + 1.0])  # 0 at t=0 and 2 -> rho^2 + 1 (before reset)


# ---- chunk invariance (tests/test_gold_standard.py:113-160, :265-305) ---------

def _states_after(tokens, rhos):
    """data.py:284-303 preprocess_corpus state after each occurrence (one document)."""
    V = max(tokens) + 1
    cur = np.zeros((V, len(rhos)), np.float32)
    last = np.full(V, -1)
    out = np.zeros((len(tokens), len(rhos)), np.float32)
    for t, v in enumerate(tokens):
        cur[v] = 1.0 if last[v] == -1 else cur[v] * rhos ** (t - last[v]) + 1.0
        last[v] = t
        out[t] = cur[v]
    return out


def _chunk_inputs(tokens, states, rhos, start, end):
    """data.py:95-148: chunk, expanded unique slots, c_base decayed to the chunk start."""
    chunk = tokens[start:end]
    cu = sorted(set(chunk))
    extra = sorted(set(tokens[:start]) - set(cu))
    slots = cu + extra
    c_base = np.zeros((len(slots), len(rhos)), np.float32)
    for i, v in enumerate(slots):
        prev = [p for p in range(start) if tokens[p] == v]
        if prev:
            c_base[i] = states[prev[-1]] * rhos ** (start - prev[-1])
    return np.array([chunk]), np.array([slots]), c_base[None]


@pytest.mark.parametrize("block", [8, 16, 32, 64, 128])
def test_chunked_equals_single_pass(block):
    rng = np.random.default_rng(42)
    common, rare = list(range(10, 20)), list(range(30, 50))
    tokens = [int(rng.choice(common)) if rng.random() < 0.7 else int(rng.choice(rare)) for _ in range(200)]
    rhos = rhos_logspace(16, 1.0, 512.0)
    truth = scan.query_scan(np.array([tokens]), rhos, 51)[0]
    states = _states_after(tokens, rhos)
    rebuilt = np.zeros_like(truth)
    for cs in range(0, len(tokens) - 1, block):
        ce = min(cs + block + 1, len(tokens))
        xc, keys, cb = _chunk_inputs(tokens, states, rhos, cs, ce)
        rebuilt[cs:ce] = scan.query_scan(xc, rhos, 51, cb, keys)[0]
    assert np.abs(truth - rebuilt).max() < 1e-5
    # the reference asserts mean < 1e-7 with torch's vectorised pow on both sides;
    # here the chunk states come from numpy's pow and the scan from glibc powf,
    # each within 1 ulp, so the mean of |diff| is allowed a second ulp's worth.
    assert np.abs(truth - rebuilt).mean() < 2e-7


# ---- the reference's dense-table CPU loop (the benchmark's CPU baseline) ------------

def test_dense_loop_known_answers():
    # tests/test_doc_boundary.py:71-105 and :108-134 through the dense-table loop
    rhos = np.array([0.9, 0.5], np.float32)
    x = np.array([[0, 1, 0, 2, 0, 1]])
    C = scan.query_scan_dense_loop(x, rhos, 3, doc_ids=np.zeros_like(x))
    assert np.allclose(C[0, 2], rhos ** 2, atol=1e-6)
    assert np.allclose(C[0, 4], (rhos ** 2 + 1.0) * rhos ** 2, atol=1e-6)
    x = np.array([[0, 1, 0, 2]])
    c_init = np.array([[[2.0, 1.5], [0.0, 0.0], [0.0, 0.0]]], np.float32)
    C = scan.query_scan_dense_loop(x, rhos, 3, c_init, np.array([[0, 1, 2]]), doc_ids=np.zeros_like(x))
    assert np.allclose(C[0, 0], [2.0, 1.5])
    x = np.array([[0, 1, 2, 0, 1, 0, 1, 3, 0, 1]])
    doc = np.array([[0, 0, 0, 0, 0, 1, 1, 1, 1, 1]])
    r4 = np.array([0.9, 0.8, 0.7, 0.6], np.float32)
    C = scan.query_scan_dense_loop(x, r4, 5, doc_ids=doc)
    assert np.allclose(C[0, 5], 0.0) and np.allclose(C[0, 8], r4 ** 3, atol=1e-6)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_dense_loop_equals_c_restatement(seed):
    """Two independent restatements of the same reference function: the dense per-vocabulary
    loop and the lazy C scan, with c_init, padding keys and document resets."""
    rng = np.random.default_rng(seed)
    B, L, V, N, K = 3, 200, 40, 8, 12
    x = rng.integers(0, V, (B, L))
    keys = np.stack([rng.permutation(V)[:K] for _ in range(B)])
    keys[:, -2:] = -1
    c_init = rng.random((B, K, N)).astype(np.float32) * 3
    docs = np.cumsum(rng.random((B, L)) < 0.02, axis=1)
    rhos = rhos_logspace(N, 1.0, 256.0)
    for d in (None, docs):
        a = scan.query_scan_dense_loop(x, rhos, V, c_init, keys, d)
        b = scan.query_scan(x, rhos, V, c_init, keys, d)
        assert np.allclose(a, b, rtol=1e-5, atol=1e-6), float(np.abs(a - b).max())


@pytest.mark.parametrize("docs", [False, True])
def test_boundary_states_f64_matches_closed_form_and_fp32_restatement(docs):
    """The float64 chunked boundary states (used to check long sequences, where the fp32
    step-by-step restatement carries one rounding per step) agree with the closed form in
    float64 and with the fp32 restatement to its rounding."""
    rng = np.random.default_rng(3 + docs)
    B, L, V, N, Br = 2, 150, 12, 5, 16
    x = rng.integers(0, V, (B, L))
    u = np.stack([np.sort(rng.choice(V, 8, replace=False)) for _ in range(B)])
    u[0, -1] = -1
    rh = rng.uniform(0.5, 0.99, N).astype(np.float32)
    c0 = rng.random((B, 8, N)).astype(np.float32)
    doc = np.sort(rng.integers(0, 4, (B, L)), axis=1) if docs else None
    a = scan.boundary_states_f64(x, u, rh, Br, c0, doc)
    b = scan.boundary_states(x, u, rh, Br, c0, doc)
    assert np.abs(a - b).max() / np.abs(a).max() < 1e-6
    if not docs:
        c = scan.boundary_states_closed_form(x, u, rh.astype(np.float64), Br, c0)
        assert np.abs(a - c).max() < 1e-12
