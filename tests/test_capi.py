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
    from mathbrain_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from mathbrain_amd import build
        build.build()
    return ctypes.CDLL(_lib.LIB_PATH)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert {"mb_ema_query_scan", "mb_ema_boundary_states", "mb_last_error"} <= names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, f"declared in include/ but not exported: {missing}"


def test_binding_table_matches_header():
    from mathbrain_amd import _lib
    assert set(_lib.SIGNATURES) == declared_symbols()


def test_abi_version_and_error_string(lib):
    lib.mb_abi_version.restype = ctypes.c_int
    assert lib.mb_abi_version() >= 1
    lib.mb_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.mb_last_error(), bytes)


def test_argument_errors_need_no_gpu(lib):
    """Argument checks run on the host before any launch and report through mb_last_error."""
    from mathbrain_amd import _lib
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
    from mathbrain_amd.ema_query import compute_query_ema_history
    with pytest.raises(NotImplementedError, match="no CPU path"):
        compute_query_ema_history(torch.zeros(1, 4, dtype=torch.long), torch.ones(2), 10)
