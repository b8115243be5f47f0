"""ctypes binding of libquail_hip.so, the gfx950 kernels of the hot path.

Every C entry point (include/quail_hip.h) returns an int status; `call`
turns a non-zero status into the exception the reference raises for the
same kind of failure: ValueError for bad arguments or geometry
(attention.py:103-105, :796, :917-919), RuntimeError for a HIP failure.

The library is built in-tree (quail_amd/libquail_hip.so, see
__graft_entry__.build). There is no fallback: a missing library raises.
"""

import ctypes
import os
import threading

LIB_NAME = "libquail_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

QH_OK = 0
QH_E_ARGUMENT = -1
QH_E_UNSUPPORTED = -2
QH_E_WORKSPACE = -3
QH_E_HIP = -4

_p = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_long
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> argtypes, in the order include/quail_hip.h declares them
SIGNATURES = {
    "qh_version": [],
    "qh_last_error": [],
    "qh_add_rmsnorm_quant": [_p, _l, _p, _l, _p, _f, _i, _i, _p, _p, _i, _p],
    "qh_group_quant": [_p, _l, _i, _i, _p, _p, _i, _p],
    "qh_fp8_gemm_nt": [_p, _l, _p, _p, _l, _p, _p, _l, _i, _i, _i, _p],
    "qh_fp8_gemm_nt_ue8m0": [_p, _l, _p, _p, _l, _p, _p, _l, _i, _i, _i, _p],
    "qh_fp8_gemm_silu_quant": [_p, _l, _p, _p, _l, _p, _i, _i, _i, _p, _l, _p,
                               _i, _p],
    "qh_fp8_gemm_silu_quant_ue8m0": [_p, _l, _p, _p, _l, _p, _i, _i, _i, _p, _l, _p,
                                     _p],
    "qh_fp8_gemm_qkv_rope": [_p, _l, _p, _p, _l, _p, _i, _i, _i, _i, _p, _p, _i, _p, _p,
                             _f, _p, _l, _p, _p, _l, _i, _p],
    "qh_fp8_gemm_qkv_rope_kv": [_p, _l, _p, _p, _l, _p, _i, _i, _i, _i, _p, _p, _i, _p,
                                _p, _f, _p, _l, _p, _p, _p, _i, _i, _p],
    "qh_qk_norm_rope": [_p, _l, _p, _p, _i, _p, _p, _f, _i, _i, _i, _i,
                        _p, _p, _p, _p],
    "qh_qk_norm_rope_kv": [_p, _l, _p, _p, _i, _p, _p, _f, _i, _i, _i, _i,
                           _p, _p, _p, _p, _i, _p],
    "qh_kv_row_scatter": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "qh_kv_row_copy": [_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "qh_attention_workspace_bytes": [_i],
    "qh_attention": [_p, _l, _i, _p, _p, _p, _i, _p, _i, _i, _p, _p, _i, _p,
                     _p, _p, _i, _i, _i, _i, _i, _i, _f, _i, _p, _l, _p, _l,
                     _p, _sz, _p],
    "qh_attention_fp8": [_p, _l, _i, _p, _p, _p, _i, _p, _i, _i, _p, _p, _i, _i,
                         _i, _i, _i, _i, _f, _i, _p, _l, _p, _i, _p, _sz, _p],
    "qh_attention_fp8_noalloc": [_p, _l, _i, _p, _p, _p, _i, _p, _i, _i, _p, _p, _i,
                                 _i, _i, _i, _i, _i, _f, _i, _p, _l, _p, _i, _p],
    "qh_tree_attention": [_p, _l, _i, _p, _p, _l, _p, _p, _i, _p, _p, _i, _p, _i,
                          _p, _i, _i, _i, _i, _i, _f, _p, _l, _p, _l, _p, _i, _p,
                          _sz, _p],
    "qh_tree_attention_resident": [_p, _l, _i, _p, _p, _l, _p, _p, _i, _p, _p, _i, _p,
                                   _i, _p, _i, _i, _i, _i, _i, _f, _p, _l, _p, _l, _p,
                                   _i, _p, _sz, _p],
    "qh_merge_attn_quant": [_p, _p, _l, _p, _p, _l, _p, _i, _i, _p, _p, _i,
                            _p],
    "qh_silu_mul_quant": [_p, _l, _i, _i, _p, _p, _i, _p],
    "qh_gather_rows": [_p, _l, _p, _i, _i, _p, _p],
    "qh_gather_quant_rows": [_p, _l, _p, _i, _p, _i, _i, _p, _l, _p, _p],
    "qh_final_norm": [_p, _p, _p, _i, _i, _p, _f, _p, _p],
    "qh_fused_add_rms_norm": [_p, _p, _i, _i, _p, _f, _p],
    "qh_answer_bits": [_p, _i, _i, _p, _i, _p, _p, _p, _p],
    "qh_answer_logits": [_p, _i, _i, _p, _i, _p, _p, _p, _p],
    "qh_e4m3_encode": [_p, _l, _p, _p],
}

RESTYPES = {
    "qh_last_error": ctypes.c_char_p,
    "qh_attention_workspace_bytes": ctypes.c_size_t,
}

_lib = None
_lock = threading.Lock()


class KernelLibraryMissing(RuntimeError):
    """libquail_hip.so is not built: the hot path has no other implementation."""


def load(path=LIB_PATH):
    """Load the kernel library once; raise KernelLibraryMissing when absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise KernelLibraryMissing(
                f"{path} is not built; run __graft_entry__.build() "
                f"(make -C quail_amd/csrc)")
        lib = ctypes.CDLL(path)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        _lib = lib
        return lib


def exported_symbols():
    """The names the header declares, for the export check."""
    return tuple(SIGNATURES)


def last_error() -> str:
    return load().qh_last_error().decode(errors="replace")


def call(name, *args):
    """Call one entry point; raise on a non-zero status."""
    fn = getattr(load(), name)
    status = fn(*args)
    if status == QH_OK:
        return
    message = f"{name}: {last_error()}"
    if status in (QH_E_ARGUMENT, QH_E_UNSUPPORTED, QH_E_WORKSPACE):
        raise ValueError(message)
    raise RuntimeError(message)


def workspace_bytes(n_seqs: int) -> int:
    return int(load().qh_attention_workspace_bytes(int(n_seqs)))
