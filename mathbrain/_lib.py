"""ctypes binding of libmathbrain_hip.so, the gfx950 C-ABI library.

The library is loaded after torch so that it binds to the HIP runtime torch has
already loaded (both carry the soname libamdhip64.so.7) and therefore shares
torch's devices, memory and streams.  There is no fallback: if the library is
missing every entry point raises, naming the build command.
"""
import ctypes
import functools
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmathbrain_hip.so")

MB_OK = 0
MB_ERR_INVALID_ARGUMENT = -1
MB_ERR_UNSUPPORTED = -2
MB_ERR_WORKSPACE = -3

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

# name -> argtypes; every entry is declared in include/mathbrain_hip.h
SIGNATURES = {
    "mb_last_error": ([], ctypes.c_char_p),
    "mb_abi_version": ([], _i),
    "mb_ema_query_scan": ([_p, _i64, _i64, _i, _i, _p, _i, _i64, _p, _p, _i, _p, _p, _p, _p, _p], _i),
    "mb_ema_query_scan_ws": ([_p, _i64, _i64, _i, _i, _p, _i, _i64, _p, _p, _i, _p, _p, _p, _p, _p, _i64,
                              _p], _i),
    "mb_ema_query_scan_workspace": ([_i, _i, _i64], _i64),
    "mb_ema_boundary_states": ([_p, _i64, _i64, _i, _i, _p, _i, _p, _i, _i, _p, _i64, _p, _p, _i, _p], _i),
    "mb_unique_rows": ([_p, _i64, _i64, _i, _i, _p, _i, _p, _p], _i),
    "mb_flash_ema_fwd": ([_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _p, _p, _p,
                          _i, _i, _i, _i, _i, _i, _i, _i, _i, _i64, _i, _p, _p, _p, _p, _i64, _p], _i),
    "mb_flash_ema_fwd_workspace": ([_i, _i, _i, _i, _i, _i, _i], _i64),
    "mb_flash_ema_bwd": ([_p, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p,
                          _p, _p, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i64, _i, _p, _p, _p, _p,
                          _p, _p], _i),
    "mb_flash_ema_fwd_gq": ([_p, _i64, _i64, _p, _i64, _i64, _p, _p, _f, _p, _p, _i64, _i64, _p, _p, _p,
                             _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i64, _i, _p, _p, _p], _i),
    "mb_gating_fwd": ([_p, _i64, _p, _i64, _p, _p, _i64, _p, _i, _p, _p, _i64, _i, _i, _f, _p, _p,
                       _p, _p, _p], _i),
    "mb_gating_bwd": ([_p, _p, _i64, _p, _i64, _p, _p, _i64, _p, _i, _p, _p, _p, _i64, _i, _i, _p,
                       _p, _p, _p, _p, _p], _i),
    "mb_corpus_states_workspace": ([_i64, _i], _i64),
    "mb_corpus_states": ([_p, _p, _i64, _p, _i, _p, _p, _i64, _p], _i),
    "mb_corpus_states_noalloc": ([_p, _p, _i64, _p, _i, _p, _p], _i),
    "mb_slot_lists": ([_p, _p, _i64, _i64, _p, _p, _p, _i, _p, _p, _p, _p, _p], _i),
    "mb_slot_batch": ([_p, _p, _p, _p, _i, _i64, _i64, _p, _p, _p, _i, _p, _p, _p, _p, _i, _i,
                       _p, _p, _p, _p, _p, _p, _p], _i),
    "mb_factored_outer": ([_p, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i, _i, _i, _i, _i,
                           _p, _p], _i),
    "mb_factored_apply": ([_p, _p, _i64, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i, _i, _i, _i,
                           _i, _i, _p, _i64, _i, _p], _i),
    "mb_factored_tok_fwd": ([_p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _p, _p], _i),
    "mb_factored_tok_bwd": ([_p, _p, _p, _i64, _p, _p, _p, _i, _i, _i, _i, _p, _p, _p, _p, _p], _i),
    "mb_rmsnorm_fwd": ([_p, _p, _i64, _i, _f, _p, _p, _p], _i),
    "mb_rmsnorm_bwd": ([_p, _p, _p, _p, _i64, _i, _p, _p, _p], _i),
    "mb_layernorm_fwd": ([_p, _p, _p, _i64, _i, _f, _p, _p, _p, _p], _i),
    "mb_layernorm_bwd": ([_p, _p, _p, _p, _p, _i64, _i, _p, _p, _p, _p], _i),
    "mb_swiglu_fwd": ([_p, _p, _i64, _i, _p, _p], _i),
    "mb_swiglu_bwd": ([_p, _p, _p, _i64, _i, _p, _p, _p], _i),
}

MB_FLASH_SILU = 1
MB_FLASH_ABSENT_MASS = 2
MB_FLASH_VOCAB_ROWS = 4
MB_FLASH_FP32 = 8
MB_FLASH_FAST_GATE = 16
MB_DTYPE_F32 = 0
MB_DTYPE_BF16 = 1

_lib = None


class HipKernelError(RuntimeError):
    """A C-ABI call rejected its arguments or its launch failed."""


class HipLibraryMissing(RuntimeError):
    """libmathbrain_hip.so is not built (python -m mathbrain.build)."""


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipLibraryMissing(
                f"{LIB_PATH} is missing; build it with `python -m mathbrain.build` "
                "(mathbrain has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def call(name, *args):
    """Calls C-ABI entry `name`; raises HipKernelError with the library's message on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != MB_OK:
        msg = lib().mb_last_error().decode(errors="replace")
        kind = {MB_ERR_INVALID_ARGUMENT: "invalid argument", MB_ERR_UNSUPPORTED: "unsupported",
                MB_ERR_WORKSPACE: "workspace too small"}.get(rc, f"HIP error {rc}")
        raise HipKernelError(f"{name}: {kind}: {msg}")


def ptr(t):
    """Device address of a tensor (None for None)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream(device):
    """The current torch stream of `device` as a raw hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def traced_op(name, fake):
    """Decorator: registers ``fn`` as the torch custom op ``mathbrain::<name>`` whose shape
    function (for fake / meta tensors) is ``fake``, and returns a callable that runs ``fn``
    directly in eager mode and the registered op while torch.compile traces.  A traced
    graph then holds the op instead of breaking at the ctypes call, and eager calls skip
    the dispatcher (about 50 us per call, measured).  ``fn`` takes tensors, optional
    tensors, ints, floats and bools (annotated) and returns new tensors."""
    def deco(fn):
        op = torch.library.custom_op(f"mathbrain::{name}", fn, mutates_args=())
        op.register_fake(fake)

        @functools.wraps(fn)
        def call(*args):
            if torch.compiler.is_compiling():
                return op(*args)
            return fn(*args)
        call.op = op
        return call
    return deco


def require_gpu(*tensors, what="mathbrain"):
    """Every tensor must live on one ROCm GPU: the product has no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise NotImplementedError(
                f"{what}: tensors must be on an MI355X GPU (got device {t.device}); "
                "this implementation has no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{what}: tensors on different devices ({dev} and {t.device})")
    return dev
