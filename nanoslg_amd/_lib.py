"""ctypes binding of libnslg_kv.so (declared in include/nslg_kv.h).

The library must be built in-tree (``python -m nanoslg_amd._build`` or
``__graft_entry__.build()``). There is no fallback: if the library is missing
or fails to load, every kernel call raises.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p, c_char_p, POINTER
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime first, so the library binds to it)

LIB_PATH = Path(__file__).resolve().parent / "libnslg_kv.so"

NSLG_F16, NSLG_BF16, NSLG_F32 = 0, 1, 2
NSLG_EWORKSPACE = -4
NSLG_ECAPTURE = -5  # a variant's first use on a device inside a stream capture
NSLG_NOALLOC_SCRATCH_BYTES = 16 << 20  # the static scratch of nslg_paged_decode_noalloc

_I32P = POINTER(c_int32)

# name -> (restype, argtypes); mirrors include/nslg_kv.h one to one.
SIGNATURES = {
    "nslg_version": (c_int32, []),
    "nslg_last_error": (c_char_p, []),
    "nslg_append_kv": (c_int32, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int32,
                                 c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p]),
    "nslg_zero_pages": (c_int32, [c_void_p, c_void_p, c_int32, c_int64, c_int32, c_int32, c_int32,
                                  c_int32, c_void_p, c_int32, c_void_p]),
    "nslg_copy_pages": (c_int32, [c_void_p, c_void_p, c_int32, c_int64, c_int32, c_int32, c_int32,
                                  c_int32, c_void_p, c_void_p, c_int32, c_void_p]),
    "nslg_gather_kv": (c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p,
                                 c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                 c_void_p]),
    "nslg_paged_decode_workspace_size": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int64, c_int32,
                                                    c_int32]),
    "nslg_paged_decode": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int32,
                                    c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32,
                                    c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p, c_size_t,
                                    c_int64, c_void_p]),
    "nslg_paged_decode_append": (c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                           c_void_p, c_void_p, c_int64, c_int32,
                                           c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32,
                                           c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p, c_size_t,
                                           c_int64, c_void_p]),
    "nslg_paged_decode_grouped_append": (c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                                   c_void_p, c_void_p, c_int64, c_int32,
                                                   c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32,
                                                   c_int32, c_int32, c_float, c_int32, c_void_p, c_int32,
                                                   c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_size_t,
                                                   c_int64, c_void_p]),
    "nslg_paged_decode_noalloc": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int32,
                                            c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32,
                                            c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p]),
    "nslg_paged_decode_grouped_workspace_size":(c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int64, c_int32,
                                                            c_int32, c_int32]),
    "nslg_paged_decode_grouped": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int32,
                                            c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32,
                                            c_int32, c_float, c_int32, c_void_p, c_int32, c_void_p, c_void_p,
                                            c_void_p, c_int64, c_void_p, c_size_t, c_int64, c_void_p]),
    "nslg_paged_decode_rope_append": (c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                                c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                                c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32,
                                                c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p,
                                                c_size_t, c_int64, c_void_p]),
    "nslg_paged_decode_grouped_rope_append": (c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                                        c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p,
                                                        c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p,
                                                        c_int64, c_int32, c_int32, c_int32, c_int32, c_float,
                                                        c_int32, c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                                        c_int64, c_void_p, c_size_t, c_int64, c_void_p]),
    "nslg_decode_plan_step": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p,
                                        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_int32, c_int64, c_int32, c_int32, c_int32, c_void_p]),
    "nslg_decode_plan_step_device": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
                                               c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                               c_void_p, c_void_p, c_int32, c_int64, c_int32, c_int32, c_int32,
                                               c_void_p]),
    "nslg_block_table_csr": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_int64, c_void_p, c_void_p, c_int64, c_int32, c_void_p]),
    "nslg_forward_plan": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                                    c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "nslg_forward_plan_csr": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
                                        c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_void_p]),
    "nslg_rope_append": (c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                   c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64,
                                   c_int32, c_int32, c_int32, c_void_p, c_void_p, c_int64, c_int32, c_void_p]),
    "nslg_paged_prefill_workspace_size": (c_size_t, [c_int32, c_int32, c_int32, c_int64, c_int32]),
    "nslg_paged_prefill": (c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_int32,
                                     c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p,
                                     c_void_p, c_int32, c_int32, c_int32, c_int32, c_float, c_int32,
                                     c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
    "nslg_paged_prefill_grid": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p, c_int32, c_int64, c_int32,
                                          c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p,
                                          c_void_p, c_int32, c_int32, c_int32, c_int32, c_float, c_int32,
                                          c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
    "nslg_paged_prefill_append": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p, c_int32, c_int64, c_int32,
                                            c_void_p, c_int64, c_void_p, c_int64,
                                            c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p,
                                            c_void_p, c_int32, c_int32, c_int32, c_int32, c_float, c_int32,
                                            c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
}

_lib = None
_fast = None
_lock = threading.Lock()


class KernelLibraryError(RuntimeError):
    """The HIP kernel library is missing, failed to load, or a call failed."""


def load() -> ctypes.CDLL:
    """Load the library once and attach the declared signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise KernelLibraryError(
                f"{LIB_PATH} is not built; run `python -m nanoslg_amd._build` "
                "(or __graft_entry__.build()) first — there is no CPU fallback")
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as e:
            raise KernelLibraryError(f"failed to load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def fast():
    """The CPython fast-call binding of the per-step entry points (built with the
    library): the same C functions as the ctypes ones of `load()`, called with the
    same Python arguments in a fraction of ctypes' conversion time."""
    global _fast
    if _fast is not None:
        return _fast
    load()
    try:
        from . import _nslg_fast
    except ImportError as e:
        raise KernelLibraryError(f"the fast-call binding of {LIB_PATH} is not built or does not load ({e}); "
                                 "run `python -m nanoslg_amd._build` (or __graft_entry__.build()) first") from e
    _fast = _nslg_fast
    return _fast


_host = None


def host():
    """The host-side forward planner (`_nslg_host`, plain C over the CPython API;
    built with the library, no GPU calls)."""
    global _host
    if _host is not None:
        return _host
    try:
        from . import _nslg_host
    except ImportError as e:
        raise KernelLibraryError(f"the host planner extension is not built or does not load ({e}); "
                                 "run `python -m nanoslg_amd._build` (or __graft_entry__.build()) first") from e
    _host = _nslg_host
    return _host


def last_error() -> str:
    msg = load().nslg_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise KernelLibraryError(f"{what} failed with status {rc}: {last_error()}")
