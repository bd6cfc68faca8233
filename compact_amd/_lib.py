"""ctypes binding of libcompact_amd.so (the C ABI in include/compact_amd.h).

The library is built in-tree by `python -m compact_amd.build` into
compact_amd/_build/libcompact_amd.so.  There is no fallback: if the library is
missing, `lib()` raises, and so does every operator that needs it.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libcompact_amd.so")

F32, F16, BF16 = 0, 1, 2

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64

# name -> argument types (restype is int for every compute entry point)
SIGNATURES = {
    "cpt_v3_quantize_group_absmax": [_P, _I, _L, _L, _I, _L, _P, _P, _P],
    "cpt_v3_dequantize_group_absmax": [_P, _P, _L, _L, _I, _L, _P, _I, _P],
    "cpt_silu_mul": [_P, _P, _P, _L, _I, _P],
    "cpt_swiglu_backward": [_P, _P, _P, _P, _P, _L, _I, _P],
    "cpt_swiglu_backward_glu": [_P, _P, _P, _P, _P, _P, _L, _I, _P],
    "cpt_silu_mul_quant": [_P, _P, _L, _L, _I, _L, _P, _P, _P, _P, _P, _P],
    "cpt_dequant_swiglu_backward": [_P, _P, _P, _P, _P, _L, _L, _I, _L, _P, _P, _P, _P],
    "cpt_outlier_select": [_P, _I, _L, _L, _L, _P, _P, _P, _P, _P],
    "cpt_outlier_select_pair": [_P, _P, _I, _L, _L, _L, _P, _P, _P, _P, _P, _P, _P],
    "cpt_probe_mfma_rate": [_I, _I, _I, ctypes.c_float, _P, _P],
    "cpt_v3_quantize_outlier": [_P, _I, _L, _L, _I, _L, _P, _L, _P, _P, _P, _P],
    "cpt_v3_dequantize_outlier": [_P, _P, _P, _L, _P, _L, _L, _I, _L, _P, _P],
    "cpt_silu_mul_quant_outlier": [_P, _P, _L, _L, _I, _L, _P, _P, _L, _P, _P, _P, _P, _P, _P,
                                   _P, _P],
    "cpt_dequant_swiglu_backward_outlier": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _I,
                                            _L, _P, _P, _P, _P],
    "cpt_gemm_bf16": [_P, _L, _I, _P, _L, _I, _P, _L, _P, _L, _L, _P, _L, _L, _L, _L, _P],
    "cpt_gemm_bf16_ex": [_P, _L, _I, _P, _L, _I, _P, _L, _L, _L, _L, ctypes.c_float, _I, _I, _P, _P],
    "cpt_gemm_any": [_I, _P, _L, _L, _P, _L, _L, _P, _L, _L, _L, _L, _L, ctypes.c_float, _I, _P],
    "cpt_gemm_wgrad_glu": [_P, _L, _I, _L, _P, _P, _P, _P, _P, _L, _L, _L, _L, _P],
    "cpt_ffn_gate_up": [_P, _P, _P, _L, _L, _L, _I, _L, _P, _P, _P, _P, _P, _P, _P, _P],
    "cpt_ffn_down_dgrad": [_P, _P, _L, _L, _L, _I, _L, _P, _P, _P, _P, _P, _P, _P, _P],
    "cpt_gemm_bf16_lora": [_P, _L, _I, _P, _L, _I, _P, _L, _P, _L, _L, _P, _L, _L, _L, _L,
                           _L, _L, _I, _L, _P, _P, ctypes.c_float, _P, _P, ctypes.c_float, _P],
    "cpt_ffn_gate_up_lora": [_P, _P, _P, _L, _L, _L, _I, _L, _P, _P, _P, _P, _P, _P, _P,
                             _L, _L, _P, _P, ctypes.c_float, _P, _P, ctypes.c_float, _P],
    "cpt_ffn_gate_up_outlier": [_P, _P, _P, _L, _L, _L, _I, _L, _P, _P, _P, _P, _P, _P, _P, _P,
                                _P, _L, _L, _L, _P, _P, ctypes.c_float, _P, _P, ctypes.c_float,
                                _P],
    "cpt_ffn_down_dgrad_lora": [_P, _P, _L, _L, _L, _I, _L, _P, _P, _P, _P, _P, _P, _P,
                                _L, _L, _P, _P, ctypes.c_float, _P],
    "cpt_gemm_bf16_skinny": [_P, _L, _P, _L, _P, _L, _L, _L, _L, ctypes.c_float, _I, _P, _P],
    "cpt_gemm_bf16_skinny_t": [_P, _L, _P, _L, _P, _L, _I, _L, _L, _L, ctypes.c_float, _I, _P,
                               _P],
    "cpt_gemm_bf16_skinny_t_noalloc": [_P, _L, _P, _L, _P, _L, _I, _L, _L, _L, ctypes.c_float,
                                       _I, _P],
    "cpt_ffn_down_dgrad_outlier": [_P, _P, _L, _L, _L, _I, _L, _P, _P, _P, _P, _P, _P, _P, _P,
                                   _L, _P, _P, _P, _L, _L, _P, _P, ctypes.c_float, _P],
    "cpt_dora_scale": [_P, _P, _P, _L, _L, _I, _P, _P],
    "cpt_col_dot_div": [_P, _P, _P, _L, _L, _I, _P, _P, _P],
    "cpt_dora_col_norm": [_P, _P, _P, _L, _L, _L, ctypes.c_double, _I, _P, _P, _I, _P],
    "cpt_topk_abs": [_P, _I, _L, _L, _L, _P, _P, _P],
    "cpt_topk_scatter": [_P, _P, _I, _L, _L, _L, _P, _P],
    "cpt_gemm_stream_k_workspace": [_P, _L],
    "cpt_transpose_bf16": [_P, _L, _L, _L, _P, _L, _P],
    "cpt_gemm_bf16_skinny_dual": [_P, _L, _P, _L, _I, _P, _L, _P, _L, ctypes.c_float, _P, _L, _I,
                                  ctypes.c_float, _L, _L, _L, _I, _P, _P],
}

# size queries: name -> argument types (restype int64)
SIZE_QUERIES = {
    "cpt_col_dot_workspace_bytes": [_L, _L],
    "cpt_dora_col_norm_workspace_bytes": [_L, _L],
    "cpt_gemm_stream_k_bytes": [],
    "cpt_gemm_bf16_skinny_dual_workspace_bytes": [_L, _L, _L, _I],
}

CACHE_NONE, CACHE_BF16, CACHE_INT4, CACHE_INT8 = 0, 1, 4, 8

NOALLOC_SCRATCH_BYTES = 16 << 20    # CPT_NOALLOC_SCRATCH_BYTES

_lib = None


class LibraryMissing(RuntimeError):
    pass


def lib():
    """Load the HIP library once; raise LibraryMissing if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} not found: build it with `python -m compact_amd.build` "
            "(compact_amd has no CPU or eager fallback)")
    L = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    for name, argtypes in SIZE_QUERIES.items():
        fn = getattr(L, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int64
    L.cpt_status_string.argtypes = [ctypes.c_int]
    L.cpt_status_string.restype = ctypes.c_char_p
    L.cpt_abi_version.argtypes = []
    L.cpt_abi_version.restype = ctypes.c_int
    _lib = L
    return _lib


# status codes (include/compact_amd.h)
OK, ERR_BITS, ERR_RAGGED, ERR_GROUP_POW2, ERR_SHAPE, ERR_DTYPE, ERR_LAUNCH, ERR_ALIGN, \
    ERR_TOO_LARGE = range(9)


def check(status: int, what: str):
    """Map a C status to the reference's exception contract: argument
    violations are AssertionError (the reference asserts them,
    src/flashffn.py:1070-1072,1303-1311), launch failures RuntimeError."""
    if status == OK:
        return
    msg = f"{what}: {lib().cpt_status_string(status).decode()}"
    if status in (ERR_BITS, ERR_RAGGED, ERR_GROUP_POW2, ERR_SHAPE, ERR_DTYPE, ERR_ALIGN,
                  ERR_TOO_LARGE):
        raise AssertionError(msg)
    raise RuntimeError(msg)
