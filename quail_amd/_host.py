"""ctypes binding of libquail_host.so, the host half of the hot path.

The library (include/quail_host.h) holds the KV arena's page accounting,
filter and join admission and the chunk builder as native objects; the
Python classes in arena.py, pack.py and loop.py are thin faces over it.
Every call returns a status or a count; `check` turns a negative status
into the exception the reference raises for that failure: KeyError,
ValueError, AssertionError, or ArenaFullError (loop.py:30-31).

The library is built in-tree (quail_amd/libquail_host.so, see
__graft_entry__.build). There is no Python fallback: a missing library
raises.
"""

import ctypes
import os
import threading

import numpy as np

LIB_NAME = "libquail_host.so"
# QUAIL_HOST_LIB names another build of the same sources, e.g. the
# AddressSanitizer one (`make -C quail_amd/host asan`)
LIB_PATH = os.environ.get("QUAIL_HOST_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

QP_OK, QP_NONE = 0, 1
QP_E_KEY, QP_E_VALUE, QP_E_STATE, QP_E_ARENA_FULL = -1, -2, -3, -4
CHUNK_ARRAYS = 21

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_d = ctypes.c_void_p   # double* (numpy pointer)

BORROW_CHECK = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                ctypes.c_int32, ctypes.c_void_p)

# name -> (restype, argtypes), in the order include/quail_host.h declares them
SIGNATURES = {
    "qp_version": (ctypes.c_int, []),
    "qp_last_error": (ctypes.c_char_p, []),
    "qp_arena_new": (_p, [_i32, _i32]),
    "qp_arena_delete": (None, [_p]),
    "qp_arena_stats": (ctypes.c_int, [_p, _p]),
    "qp_arena_free_list": (_i64, [_p, _p, _i64]),
    "qp_arena_is_resident": (ctypes.c_int, [_p, _i64]),
    "qp_arena_key_info": (ctypes.c_int, [_p, _i64, _p]),
    "qp_arena_table": (_i64, [_p, _i64, _p, _i64]),
    "qp_arena_alloc": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _i32]),
    "qp_arena_shared_pages": (_i64, [_p, _i64, _i64, _i64, _p, _i64]),
    "qp_arena_release_pages": (_i64, [_p, _p, _i64]),
    "qp_arena_free_now": (_i64, [_p, _i64]),
    "qp_arena_drop_leading": (_i64, [_p, _i64, _i64]),
    "qp_arena_rewind": (_i64, [_p, _i64, _i64]),
    "qp_arena_grow": (ctypes.c_int, [_p, _i64, _i64, _p]),
    "qp_arena_pin": (ctypes.c_int, [_p, _i64]),
    "qp_arena_sole_pages": (_i64, [_p, _i64]),
    "qp_arena_retain": (ctypes.c_int, [_p, _i64, _d, _i32]),
    "qp_arena_pop_victim": (ctypes.c_int, [_p, _p, _i64, _p]),
    "qp_arena_clear_retention": (ctypes.c_int, [_p]),
    "qp_arena_retained_keys": (_i64, [_p, _p, _i64]),
    "qp_arena_resident_keys": (_i64, [_p, _p, _i64]),
    "qp_arena_set_retention_cap": (ctypes.c_int, [_p, _i64]),
    "qp_arena_activate": (ctypes.c_int, [_p, _i64, _i64, _i64, _i64, _i64]),
    "qp_arena_alloc_temporary": (ctypes.c_int, [_p, _i64, _p]),
    "qp_arena_hold": (ctypes.c_int, [_p, _i64, _i64]),
    "qp_arena_release": (ctypes.c_int, [_p, _i64]),
    "qp_arena_drop_holds": (ctypes.c_int, [_p, _p, _i64, _i32]),
    "qp_arena_held": (ctypes.c_int, [_p, _i64]),
    "qp_arena_free_key": (_i64, [_p, _i64]),
    "qp_arena_evict_key": (_i64, [_p, _i64]),
    "qp_arena_evict_retained": (_i64, [_p, _i64]),
    "qp_arena_drain_evictions": (_i64, [_p, _p, _p, _p, _i64]),
    "qp_tokens_new": (_p, []),
    "qp_tokens_delete": (None, [_p]),
    "qp_tokens_add": (_i64, [_p, _p, _p, _p, _i32]),
    "qp_tokens_add_flat": (_i64, [_p, _p, _i32, _i64, _p]),
    "qp_tokens_length": (_i64, [_p, _i64]),
    "qp_prefix_tree": (ctypes.c_int, [_p, _i32, _i64, _p, _i64, _p, _p, _p]),
    "qp_chunk_new": (_p, []),
    "qp_chunk_delete": (None, [_p]),
    "qp_chunk_reset": (ctypes.c_int, [_p]),
    "qp_chunk_add_group": (ctypes.c_int, [_p, _i64, _i64, _i32, _i32, _i64, _i64, _i64, _p,
                                          _i64, _i64, _p, _p, _i32]),
    "qp_chunk_build": (ctypes.c_int, [_p, _p, _i32]),
    "qp_chunk_summary": (ctypes.c_int, [_p, _p]),
    "qp_chunk_arrays": (ctypes.c_int, [_p, _p]),
    "qp_chunk_emit": (_i64, [_p, _p, _i64, _p]),
    "qp_chunk_temporaries": (_i64, [_p, _p, _i64]),
    "qp_chunk_fresh_keys": (_i64, [_p, _p, _i64]),
    "qp_filter_new": (_p, [_p, _i32, _p, _i32, _i64, _i64, _i32, _i64, _i64, _p, _p, _p]),
    "qp_filter_delete": (None, [_p]),
    "qp_filter_bind_arena": (ctypes.c_int, [_p, _p, _p, _i32]),
    "qp_filter_set_borrow_check": (ctypes.c_int, [_p, BORROW_CHECK, _p]),
    "qp_join_set_borrow_check": (ctypes.c_int, [_p, BORROW_CHECK, _p]),
    "qp_filter_next_chunk": (_i64, [_p, _i64, _p, _p, _p, _i64]),
    "qp_filter_stage_chunk": (ctypes.c_int, [_p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32]),
    "qp_filter_groups": (_i64, [_p, _p, _p, _p, _i64]),
    "qp_filter_report": (ctypes.c_int, [_p, _i32, _i32, _i32, _i32, _p]),
    "qp_filter_report_chunk": (_i64, [_p, _p, _i64, _p, _p, _p]),
    "qp_filter_state": (ctypes.c_int, [_p, _p]),
    "qp_filter_drain_ready": (_i64, [_p, _p, _i64]),
    "qp_filter_borrow": (ctypes.c_int, [_p, _i32, _p]),
    "qp_filter_borrowers": (_i64, [_p, _p, _i64]),
    "qp_join_new": (_p, [_i32, _p, _p, _p, _i64, _i64, _i32, _i32, _i64, _i32, _p, _p]),
    "qp_join_delete": (None, [_p]),
    "qp_join_register": (_i64, [_p, _i64, _i64, _p, _p]),
    "qp_join_seed": (ctypes.c_int, [_p, _p, _i32]),
    "qp_join_admit": (_i64, [_p, _i64, _i64, _p, _p]),
    "qp_join_bind_arena": (ctypes.c_int, [_p, _p]),
    "qp_join_set_key": (ctypes.c_int, [_p, _i32, _i64]),
    "qp_join_next_chunk": (_i64, [_p, _i64, _p, _p, _p, _p, _p, _i64]),
    "qp_join_report": (ctypes.c_int, [_p, _i32, _i32, _i64, _i64, _p, _i64]),
    "qp_join_events": (_i64, [_p, _i32, _p, _p, _i64]),
    "qp_join_state": (ctypes.c_int, [_p, _p]),
    "qp_join_partners": (_i64, [_p, _i32, _i32, _i64, _i64, _p]),
    "qp_join_borrow": (ctypes.c_int, [_p, _i32, _p]),
    "qp_join_borrowers": (_i64, [_p, _p, _i64]),
    "qp_join_prefix": (_i64, [_p, _i32]),
}

_lib = None
_lock = threading.Lock()


class HostLibraryMissing(RuntimeError):
    """libquail_host.so is not built: the host path has no other implementation."""


class ArenaFullError(RuntimeError):
    """A chunk's suffix pages do not fit the free KV arena (loop.py:30-31)."""


def load(path=LIB_PATH):
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise HostLibraryMissing(f"{path} is not built; run __graft_entry__.build() "
                                     f"(make -C quail_amd/host)")
        lib = ctypes.CDLL(path)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def exported_symbols():
    return tuple(SIGNATURES)


def last_error() -> str:
    return (load().qp_last_error() or b"").decode(errors="replace")


def raise_status(name, status):
    message = f"{name}: {last_error()}"
    if status == QP_E_KEY:
        raise KeyError(message)
    if status == QP_E_VALUE:
        raise ValueError(message)
    if status == QP_E_ARENA_FULL:
        raise ArenaFullError(message)
    raise AssertionError(message)


def check(name, value):
    """A status or count from `name`; negative values raise."""
    if value is not None and value < 0:
        raise_status(name, value)
    return value


def fn(name):
    return getattr(load(), name)


def call(name, *args):
    return check(name, getattr(load(), name)(*args))


def ptr(arr):
    """Data pointer of a contiguous numpy array (None for None)."""
    return None if arr is None else arr.ctypes.data


def i64(values):
    return np.ascontiguousarray(values, dtype=np.int64)


def i32(values):
    return np.ascontiguousarray(values, dtype=np.int32)


class Handle:
    """Owns one native object; deletes it with the matching *_delete."""

    __slots__ = ("ptr", "_delete")

    def __init__(self, ptr, delete):
        self.ptr = ptr or None
        self._delete = delete
        if not ptr:
            raise ValueError(last_error())

    def __del__(self):
        ptr, self.ptr = self.ptr, None
        if ptr and _lib is not None:
            getattr(_lib, self._delete)(ptr)
