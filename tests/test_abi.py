"""The C-ABI library loads on the CPU and exports every declared symbol.

No compute call is made (there is no GPU here); qh_version and the
workspace-size query are host-only.
"""

import ctypes
import os
import re

import pytest

from quail_amd import _hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "quail_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qh_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_hip.exported_symbols())


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_hip.LIB_PATH):
        pytest.fail(f"{_hip.LIB_PATH} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_hip.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
    loaded = _hip.load()
    assert loaded.qh_version() == 1
    assert _hip.workspace_bytes(4096) >= 4097 * 4


def test_argument_errors_raise_value_error_without_a_gpu():
    # geometry checks run before any HIP call
    with pytest.raises(ValueError, match="multiple of 256"):
        _hip.call("qh_fp8_gemm_nt", None, 128, None, None, 128, None, None, 100,
                  4, 100, 128, None)
    with pytest.raises(ValueError, match="fp8_gemm_nt_ue8m0: N=100 must be a multiple of 256"):
        _hip.call("qh_fp8_gemm_nt_ue8m0", None, 128, None, None, 128, None, None, 100,
                  4, 100, 128, None)
    with pytest.raises(ValueError, match="fp8_gemm_silu_quant_ue8m0: I=100"):
        _hip.call("qh_fp8_gemm_silu_quant_ue8m0", None, 128, None, None, 128, None, 4, 100,
                  128, None, 100, None, None)
    with pytest.raises(ValueError, match="head_dim"):
        _hip.call("qh_attention", None, 0, 0, None, None, None, 0, None, 0, 16,
                  None, None, 0, None, None, None, 1, 1, 1, 32, 8, 64, 0.1, 1,
                  None, 0, None, 0, None, 0, None)


# (entry point, arguments, the error message's words): geometry the kernels
# cannot take, rejected before any pointer is read or HIP call made
REJECTED = [
    # a weight whose int32 element offsets would pass 2^31 (1,048,576 rows x 2,560)
    ("qh_fp8_gemm_nt", (None, 2560, None, None, 2560, None, None, 1 << 20, 16, 1 << 20, 2560,
                        None), "exceed 2 GiB"),
    ("qh_fp8_gemm_silu_quant", (None, 2560, None, None, 2560, None, 16, 1 << 19, 2560, None,
                                1 << 19, None, 0, None), "exceed 2 GiB"),
    ("qh_fp8_gemm_nt", (None, 2560, None, None, 2560, None, None, 19456, 16, 19456, 2500, None),
     "multiple of 128"),
    ("qh_group_quant", (None, 128, 4, 100, None, None, 0, None), "multiple of 128"),
    ("qh_e4m3_encode", (None, 6, None, None), "multiple of 4"),
    # more sequences than the no-allocation entry's static scratch holds
    ("qh_attention_fp8_noalloc", (None, 4096, 1, None, None, None, 1, None, 1, 16, None, None,
                                  10_000_000, 1, 1, 32, 8, 128, 0.1, 1, None, 4096, None, 0,
                                  None), "static scratch holds at most"),
    # a GQA group the tree kernel's head groups cannot tile (6 / 4 heads)
    ("qh_tree_attention", (None, 768, 1, None, None, 512, None, None, 1, None, None, 0, None, 0,
                           None, 0, 16, 6, 4, 128, 0.1, None, 0, None, 0, None, 0, None, 0,
                           None), "GQA group"),
    # more workgroups than the kernels' 32-bit workgroup index covers (2^31 - 1 queries,
    # 64 head groups)
    ("qh_attention", (None, 0, 0, None, None, None, 0, None, 0, 16, None, None, 0, None, None,
                      None, 1, (1 << 31) - 1, 1, 256, 64, 128, 0.1, 1, None, 0, None, 0, None,
                      0, None), "exceed 2\\^31 workgroups"),
    ("qh_tree_attention", (None, 32768, (1 << 31) - 1, None, None, 8192, None, None, 1, None,
                           None, 0, None, 0, None, 0, 16, 256, 64, 128, 0.1, None, 0, None, 0,
                           None, 0, None, 0, None), "exceed 2\\^31 workgroups"),
]


@pytest.mark.parametrize("name,args,words", REJECTED, ids=[f"{r[0]}-{r[2]}" for r in REJECTED])
def test_unsupported_geometry_is_rejected_before_any_launch(name, args, words):
    with pytest.raises(ValueError, match=words):
        _hip.call(name, *args)


HOST_HEADER = os.path.join(ROOT, "include", "quail_host.h")


def declared_host_functions():
    text = open(HOST_HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qp_[a-z0-9_]+)\s*\(", text)))


def test_host_header_and_binding_agree():
    from quail_amd import _host
    assert declared_host_functions() == sorted(_host.exported_symbols())


def test_host_library_exports_every_declared_symbol():
    from quail_amd import _host
    if not os.path.exists(_host.LIB_PATH):
        pytest.fail(f"{_host.LIB_PATH} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_host.LIB_PATH)
    for name in declared_host_functions():
        assert hasattr(lib, name), f"{name} not exported"
    assert _host.load().qp_version() == 1


def test_host_errors_map_to_the_reference_exceptions():
    from quail_amd import _host
    from quail_amd.arena import PageArena
    a = PageArena(4, 16)
    with pytest.raises(KeyError):
        a.table_pages("nobody")
    with pytest.raises(ValueError, match="capacity_tokens must cover"):
        a.alloc("x", 40, capacity_tokens=10)
    with pytest.raises(ValueError, match="arena of -1 pages"):
        PageArena(-1, 16)
    with pytest.raises(_host.ArenaFullError):
        _host.raise_status("probe", _host.QP_E_ARENA_FULL)
    with pytest.raises(AssertionError):
        _host.raise_status("probe", _host.QP_E_STATE)
