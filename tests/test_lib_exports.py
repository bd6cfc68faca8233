"""The C-ABI library builds, loads on the CPU and exports exactly what
include/compact_amd.h declares (no compute calls: there is no GPU here)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "compact_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cpt_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from compact_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from compact_amd import build
        build.build()
    return _lib.lib()


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "cpt_silu_mul_quant" in syms and "cpt_dequant_swiglu_backward" in syms
    assert len(syms) >= 9


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_python_binding_covers_header(lib):
    from compact_amd import _lib
    for name in declared_symbols():
        if name in ("cpt_status_string", "cpt_abi_version"):
            continue
        assert name in _lib.SIGNATURES or name in _lib.SIZE_QUERIES, \
            f"{name} has no ctypes signature"


def test_status_strings_and_version(lib):
    assert lib.cpt_abi_version() >= 1
    assert lib.cpt_status_string(0) == b"ok"
    assert b"group_size" in lib.cpt_status_string(2)


def test_argument_errors_need_no_gpu(lib):
    """Argument checks run before any HIP call, so they work on a CPU host and
    map to the reference's AssertionError contract."""
    from compact_amd import _lib
    rc = lib.cpt_silu_mul_quant(None, None, 4, 5664, 4, 64, None, None, None, None, None, None)
    assert rc == _lib.ERR_RAGGED
    rc = lib.cpt_silu_mul_quant(None, None, 4, 96, 4, 48, None, None, None, None, None, None)
    assert rc == _lib.ERR_GROUP_POW2
    rc = lib.cpt_v3_quantize_group_absmax(None, 2, 4, 96, 3, 48, None, None, None)
    assert rc == _lib.ERR_BITS
    with pytest.raises(AssertionError):
        _lib.check(rc, "probe")
    assert lib.cpt_dora_scale(None, None, None, 4, 8, 9, None, None) == _lib.ERR_DTYPE
    assert lib.cpt_dora_scale(None, None, None, -1, 8, 2, None, None) == _lib.ERR_SHAPE
    assert lib.cpt_col_dot_div(None, None, None, 4, 8, 2, None, None, None) == _lib.ERR_SHAPE
    assert lib.cpt_dora_col_norm(None, None, None, 4, 8, 2, 1.0, 2, None, None, 2,
                                 None) == _lib.ERR_SHAPE


def test_workspace_size_queries(lib):
    """Workspaces: fp32 partials per 128-row chunk for the column dot; ||W||^2,
    W A^T and A A^T for the DoRA norm."""
    assert lib.cpt_col_dot_workspace_bytes(1000, 24) == 8 * 24 * 4
    assert lib.cpt_col_dot_workspace_bytes(0, 24) == 24 * 4
    assert lib.cpt_dora_col_norm_workspace_bytes(100, 8) == (100 + 800 + 64) * 4
    assert lib.cpt_dora_col_norm_workspace_bytes(-1, 8) == -1


def test_product_refuses_cpu_tensors():
    import torch
    import compact_amd
    t = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        compact_amd.silu_mul_quant(t, t, 4, 64)
