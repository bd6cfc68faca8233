"""ctypes binding of oracle/codec_ref.c (TEST INFRASTRUCTURE ONLY)."""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle_codec.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        L.oracle_quantize.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_void_p]
        L.oracle_quantize.restype = ctypes.c_int
        L.oracle_dequantize_bf16.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_void_p]
        L.oracle_dequantize_bf16.restype = ctypes.c_int
        L.oracle_f32_to_f16_bits.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16_bits.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16_bits.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16_bits.restype = ctypes.c_uint16
        _lib = L
    return _lib


def quantize(t: np.ndarray, bits: int, group: int):
    t = np.ascontiguousarray(t, dtype=np.float32)
    n, d = t.shape
    payload = np.zeros((n, d // 2) if bits == 4 else (n, d),
                       np.uint8 if bits == 4 else np.int8)
    scales = np.zeros((n, d // group), np.uint16)
    rc = lib().oracle_quantize(t.ctypes.data, n, d, bits, group,
                               payload.ctypes.data, scales.ctypes.data)
    assert rc == 0, "oracle_quantize rejected its arguments"
    return payload, scales.view(np.float16)


def dequantize_bf16(payload: np.ndarray, scales: np.ndarray, bits: int, group: int):
    payload = np.ascontiguousarray(payload)
    sc = np.ascontiguousarray(scales).view(np.uint16)
    n = payload.shape[0]
    d = payload.shape[1] * (2 if bits == 4 else 1)
    out = np.zeros((n, d), np.uint16)
    rc = lib().oracle_dequantize_bf16(payload.ctypes.data, sc.ctypes.data, n, d, bits,
                                      group, out.ctypes.data)
    assert rc == 0
    return out


def f32_to_f16_bits(x: float) -> int:
    return int(lib().oracle_f32_to_f16_bits(float(np.float32(x))))


def f32_to_bf16_bits(x: float) -> int:
    return int(lib().oracle_f32_to_bf16_bits(float(np.float32(x))))
