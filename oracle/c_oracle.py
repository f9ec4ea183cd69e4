"""ctypes binding of the C restatement (oracle/libqarr_oracle.so).

TEST INFRASTRUCTURE ONLY (tests/ and bench.py's cpu_baseline leg)."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libqarr_oracle.so"
_lib = None


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        lib = ctypes.CDLL(str(LIB))
        P, I = ctypes.c_void_p, ctypes.c_int64
        lib.oracle_quantize.argtypes = [P, I, I, I, I, I, P, P, P]
        lib.oracle_dequantize.argtypes = [P, P, P, I, I, I, I, I, P]
        lib.oracle_bf16_to_e4m3.argtypes = [ctypes.c_uint32]
        lib.oracle_bf16_to_e4m3.restype = ctypes.c_uint32
        lib.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_bf16.restype = ctypes.c_uint32
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def quantize(x: np.ndarray, tgrid):
    """Same contract as qarr_oracle.quantize_impl (f32 input)."""
    from oracle.qarr_oracle import as_2d_shape, group_layout
    x = np.ascontiguousarray(x, dtype=np.float32)
    S, H, W = as_2d_shape(x.shape)
    n_blk, K, M = group_layout(H, W, tgrid)
    lead = x.shape[:-2] if x.ndim >= 2 else ()
    x8 = np.empty(x.shape, np.uint8)
    sc8 = np.empty(lead + (M, K), np.uint8)
    sc32 = np.empty(lead + (M, 1, 1), np.float32)
    rc = load().oracle_quantize(_p(x), S, H, W, tgrid[0], tgrid[1], _p(x8), _p(sc8), _p(sc32))
    if rc:
        raise ValueError("tgrid does not divide the shape")
    return x8, sc8, sc32


def dequantize(x8: np.ndarray, sc8: np.ndarray, sc32: np.ndarray, tgrid) -> np.ndarray:
    from oracle.qarr_oracle import as_2d_shape
    x8 = np.ascontiguousarray(x8, dtype=np.uint8)
    sc8 = np.ascontiguousarray(sc8, dtype=np.uint8)
    sc32 = np.ascontiguousarray(sc32, dtype=np.float32)
    S, H, W = as_2d_shape(x8.shape)
    out = np.empty(x8.shape, np.float32)
    load().oracle_dequantize(_p(x8), _p(sc8), _p(sc32), S, H, W, tgrid[0], tgrid[1], _p(out))
    return out
