"""The C-ABI library builds for gfx950, loads, and exports exactly what include/*.h declares
(no GPU needed: nothing here launches a kernel)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(mb_[a-z0-9_]+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401  (the library binds to torch's HIP runtime)
    from mathbrain import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from mathbrain import build
        build.build()
    return ctypes.CDLL(_lib.LIB_PATH)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert {"mb_ema_query_scan", "mb_ema_boundary_states", "mb_last_error"} <= names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, f"declared in include/ but not exported: {missing}"


def test_binding_table_matches_header():
    from mathbrain import _lib
    assert set(_lib.SIGNATURES) == declared_symbols()


def test_abi_version_and_error_string(lib):
    lib.mb_abi_version.restype = ctypes.c_int
    assert lib.mb_abi_version() >= 1
    lib.mb_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.mb_last_error(), bytes)


def test_argument_errors_need_no_gpu(lib):
    """Argument checks run on the host before any launch and report through mb_last_error."""
    from mathbrain import _lib
    L = _lib.lib()
    rc = L.mb_ema_query_scan(None, 0, 1, 1, 4, None, 0, 10, None, None, 0, None, None, None, None, None)
    assert rc == _lib.MB_ERR_INVALID_ARGUMENT
    assert b"N=0" in L.mb_last_error()
    rc = L.mb_ema_boundary_states(None, 0, 1, 1, 4, None, 2, None, 4, 0, None, 0, None, None, 16, None)
    assert rc == _lib.MB_ERR_INVALID_ARGUMENT
    assert b"Br=0" in L.mb_last_error()
    # empty problems are accepted without touching the device
    assert L.mb_ema_query_scan(None, 0, 1, 0, 4, None, 4, 10, None, None, 0, None, None, None, None, None) == 0


def test_cpu_tensors_are_rejected():
    import torch
    from mathbrain.triton_ema_query import compute_query_ema_history
    with pytest.raises(NotImplementedError, match="no CPU path"):
        compute_query_ema_history(torch.zeros(1, 4, dtype=torch.long), torch.ones(2), 10)


def test_data_and_factored_argument_errors_need_no_gpu(lib):
    """The data-pipeline and factored entry points check sizes and workspace on the host."""
    from mathbrain import _lib
    L = _lib.lib()
    assert L.mb_corpus_states_workspace(0, 64) == 0
    assert L.mb_corpus_states_workspace(1024, 64) == 1024 // 1024 * 64 * 3 * 4
    rc = L.mb_corpus_states(None, None, 10, None, 200, None, None, 0, None)
    assert rc == _lib.MB_ERR_INVALID_ARGUMENT and b"N=200" in L.mb_last_error()
    rc = L.mb_corpus_states(1, 1, 10, 1, 4, 1, None, 0, None)   # no workspace
    assert rc == _lib.MB_ERR_WORKSPACE and b"workspace" in L.mb_last_error()
    assert L.mb_corpus_states(None, None, 0, None, 4, None, None, 0, None) == 0
    rc = L.mb_slot_lists(None, None, 10, 0, None, None, None, 2, None, None, None, None, None)
    assert rc == _lib.MB_ERR_INVALID_ARGUMENT and b"V=0" in L.mb_last_error()
    assert L.mb_slot_lists(None, None, 10, 5, None, None, None, 0, None, None, None, None, None) == 0
    rc = L.mb_slot_batch(None, None, None, None, 0, 10, 5, None, None, None, 1, None, None, None,
                         None, 4, 4, None, None, None, None, None, None, None)
    assert rc == _lib.MB_ERR_INVALID_ARGUMENT and b"N=0" in L.mb_last_error()
    rc = L.mb_factored_tok_fwd(None, None, 10, None, None, None, 1, 4, 2, 48, None, None)
    assert rc == _lib.MB_ERR_UNSUPPORTED and b"head_dim=48" in L.mb_last_error()
    rc = L.mb_factored_outer(None, None, None, None, 64, 10, None, 0, 0, 0, 1, 4, 2, 4, 64, None, None)
    assert rc == _lib.MB_ERR_INVALID_ARGUMENT and b"row stride" in L.mb_last_error()
    rc = L.mb_factored_apply(None, None, 0, None, None, 128, 10, None, 0, 0, 0, 1, 4, 2, 4, 16, 0,
                             None, 128, 0, None)
    assert rc == _lib.MB_ERR_UNSUPPORTED and b"head_dim=16" in L.mb_last_error()


def test_factored_and_data_cpu_tensors_are_rejected():
    import torch
    from mathbrain.factored_ema import factored_ema_forward
    with pytest.raises(NotImplementedError, match="no CPU path"):
        factored_ema_forward(torch.zeros(1, 4, 8), torch.zeros(1, 4, dtype=torch.long),
                             torch.zeros(5, 8), torch.zeros(5, 8), torch.ones(2), torch.zeros(2, 8), 2)


def test_scores_are_kept_up_to_the_memory_cap(monkeypatch):
    """FlashEMAFunction keeps the forward's scores for its backward only while the
    [B, H, K_max, L] fp32 tensor fits under SAVE_SCORES_MAX_BYTES, and never when switched off."""
    from mathbrain import triton_flash_ema as tfe
    assert tfe.keep_scores(56, 8, 1638, 512)                    # 1.47 GB
    cap_elems = tfe.SAVE_SCORES_MAX_BYTES // 4
    assert tfe.keep_scores(1, 1, cap_elems, 1)
    assert not tfe.keep_scores(1, 1, cap_elems + 1, 1)
    monkeypatch.setattr(tfe, "SAVE_SCORES", False)
    assert not tfe.keep_scores(56, 8, 1638, 512)


def test_score_budget_is_shared_by_the_tensors_still_alive(monkeypatch):
    """The saved-score limit is one budget per device for every score tensor still held:
    six cfg2-sized layers (1.47 GB each) fit 16 GiB, a twelfth does not while eleven are
    alive, and a freed tensor gives its bytes back."""
    import gc
    import torch
    from mathbrain import triton_flash_ema as tfe
    budget = tfe.ScoreBudget()
    monkeypatch.setattr(tfe, "score_budget", budget)
    Q = torch.empty(56, 8, 512, 0)      # the shape is all _reserve_scores reads
    held = []
    for _ in range(11):
        nb = tfe._reserve_scores(Q, 1638)
        assert nb == 4 * 56 * 8 * 1638 * 512
        t = torch.empty(1)
        budget.hold(t, nb)
        held.append(t)
    assert budget.held("cpu") == 11 * nb
    assert tfe._reserve_scores(Q, 1638) == 0            # 12 x 1.47 GB > 16 GiB
    del t
    held.pop()
    gc.collect()
    assert budget.held("cpu") == 10 * nb
    nb2 = tfe._reserve_scores(Q, 1638)
    assert nb2 == nb
    budget.release("cpu", nb2)
    held.clear()
    gc.collect()
    assert budget.held("cpu") == 0
    monkeypatch.setattr(tfe, "SAVE_SCORES", False)
    assert tfe._reserve_scores(Q, 1638) == 0


def test_counter_range_check_names_the_half_life_limit():
    """Rates whose key counters could leave the gate operands' fp16 range are refused on the
    host: the model with train.py's --max_hl 100000 raises at construction, and the
    functional check reads a rate tensor once per version."""
    import torch
    from mathbrain._lib import HipKernelError
    from mathbrain import triton_flash_ema as tfe
    from mathbrain.model import SlotTransformerLM
    assert 45000 < tfe.MAX_HALF_LIFE < 45500
    with pytest.raises(HipKernelError, match="half-lives up to 45359 steps"):
        SlotTransformerLM(100, 32, 1, 2, N=8, max_hl=100000.0)
    SlotTransformerLM(100, 32, 1, 2, N=8, max_hl=45000.0)
    SlotTransformerLM(100, 32, 1, 2, N=8)                     # train.py's default, 2048
    rhos = torch.exp(-torch.log(torch.tensor(2.0)) / torch.tensor([4.0, 4096.0]))
    tfe.check_counter_range(rhos)
    rhos[1] = 0.99999
    with pytest.raises(HipKernelError, match="half-life"):
        tfe.check_counter_range(rhos)
    with pytest.raises(HipKernelError, match="half-life inf"):
        tfe.check_counter_range([0.5, 1.0])
    tfe.check_counter_range([0.5, 0.999])
