"""ctypes binding of ``libpratchya_fp8.so`` (the C ABI in include/pratchya_fp8.h).

The library is mandatory: every operator in this package runs on the gfx950
kernels and there is no CPU or PyTorch fallback.  A missing or stale library is
an ImportError-style failure at first use, never a silent slow path.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpratchya_fp8.so"
ABI_VERSION = 1

OK, EINVAL, EHIP, EUNSUPPORTED = 0, 1, 2, 3
DT_F32, DT_BF16, DT_E4M3 = 0, 1, 2

_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_int = ctypes.c_int

# (name, restype, argtypes) for every exported entry point.
SIGNATURES = {
    "pratchya_abi_version": (_c_int, []),
    "pratchya_last_error": (ctypes.c_char_p, []),
    "pratchya_quant_layout": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64,
                                       ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64),
                                       ctypes.POINTER(_c_i64)]),
    "pratchya_quantize_workspace_bytes": (ctypes.c_size_t, [_c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "pratchya_quantize": (_c_int, [_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                   _c_p, _c_p, _c_p, _c_p, ctypes.c_size_t, _c_p]),
    "pratchya_quantize_noalloc": (_c_int, [_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                           _c_p, _c_p, _c_p, _c_p]),
    "pratchya_quantize_noalloc_max_bytes": (ctypes.c_size_t, []),
    "pratchya_quantize_dequantize_workspace_bytes": (ctypes.c_size_t, [_c_int, _c_i64, _c_i64, _c_i64,
                                                                       _c_i64, _c_i64]),
    "pratchya_quantize_dequantize": (_c_int, [_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                              _c_p, _c_int, _c_int, _c_p, _c_p, _c_p, ctypes.c_size_t,
                                              _c_p]),
    "pratchya_requantize_cotangent": (_c_int, [_c_p, _c_int, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                               _c_p, _c_p, _c_p, _c_p]),
    "pratchya_gather_dequantize": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p,
                                            _c_i64, _c_p, _c_int, _c_p]),
    "pratchya_dequantize": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                     _c_p, _c_int, _c_p]),
    "pratchya_dequantize_bwd": (_c_int, [_c_p, _c_int, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _c_i64, _c_p, _c_p]),
    "pratchya_quantize_t128": (_c_int, [_c_p, _c_int, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                        _c_p, _c_p, _c_p, _c_p]),
    "pratchya_quantize_128x1": (_c_int, [_c_p, _c_int, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                         _c_p, _c_p, _c_p, _c_p]),
    "pratchya_gather_quantize": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64,
                                          _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, ctypes.c_size_t, _c_p]),
    "pratchya_elementwise_workspace_bytes": (ctypes.c_size_t, [_c_i64] * 9),
    "pratchya_elementwise": (_c_int, [_c_int, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i64,
                                      _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p,
                                      ctypes.c_size_t, _c_p]),
    "pratchya_momentum": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                   _c_i64, _c_i64, _c_int, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                   ctypes.c_float, _c_p, _c_p, _c_p]),
    "pratchya_ns_combine": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_int, _c_p]),
    "pratchya_ns_normalize_workspace_bytes": (_c_i64, []),
    "pratchya_ns_normalize": (_c_int, [_c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p]),
    "pratchya_ns_normalize_f32": (_c_int, [_c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p]),
    "pratchya_apply_update": (_c_int, [_c_p, _c_int, _c_int, ctypes.c_float, _c_p, _c_int, _c_p, _c_p,
                                       _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, ctypes.c_float,
                                       ctypes.c_float, _c_p, _c_int, _c_p]),
    "pratchya_quantize_t1x128": (_c_int, [_c_p, _c_int, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p,
                                          _c_p]),
    "pratchya_quantize_dual": (_c_int, [_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                        _c_p]),
    "pratchya_gemm_bs_nt": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                     _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                     _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_int, _c_p]),
    "pratchya_gemm_bs_nt_fq": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                        _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                        _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_int, _c_int, _c_p, _c_p,
                                        _c_p, _c_i64, _c_p]),
    "pratchya_gemm_bs_nt_fq_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "pratchya_gemm_bs_nt_q11": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_int, _c_p, _c_p, _c_p]),
    "pratchya_gemm_bs_blockmax": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                           _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                           _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_p, _c_p]),
    "pratchya_quantize_dequantize_premax": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p,
                                                     _c_int, _c_int, _c_p, _c_p, _c_p]),
    "pratchya_gemm_bs_nt_qa": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p,
                                        _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                        _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_int, _c_int, _c_p, _c_p,
                                        _c_p, _c_i64, _c_p]),
    "pratchya_gemm_bs_nt_qa_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_int]),
    "pratchya_gemm_bs_nt_qa_status_offset": (_c_i64, [_c_i64, _c_i64, _c_int]),
    "pratchya_gemm_bs_nt_fq_status_offset": (_c_i64, [_c_i64, _c_i64]),
    "pratchya_gemm_bs_kmajor": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_int, _c_p]),
    "pratchya_gemm_bf16_nt": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
                                       _c_int, _c_p]),
    "pratchya_gemm_bf16_nt_ns": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_int, _c_i64, _c_i64, _c_i64, _c_p,
                                          _c_i64, _c_p, _c_i64, _c_p]),
    "pratchya_gemm_bf16_gram_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "pratchya_gemm_bf16_gram_status_offset": (_c_i64, [_c_i64, _c_i64]),
    "pratchya_gemm_bf16_gram": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_p, _c_i64, _c_p]),
    "pratchya_transpose_b16": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "pratchya_split_pack_bf16": (_c_int, [_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                          ctypes.POINTER(_c_int), _c_p, _c_i64, _c_i64, _c_p]),
    "pratchya_gemm_span": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "pratchya_transpose_u8": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "pratchya_mfma_ceiling": (_c_int, [_c_p, _c_p, _c_i64, _c_int, _c_i64, _c_p, ctypes.POINTER(_c_i64), _c_p]),
    "pratchya_debug_bf16_to_e4m3": (_c_int, [_c_p, _c_p, _c_i64, _c_int, _c_p]),
    "pratchya_debug_f32_to_bf16": (_c_int, [_c_p, _c_p, _c_i64, _c_int, _c_p]),
}

_lock = threading.Lock()
_lib = None


class PratchyaError(RuntimeError):
    """A HIP launch failure or an unsupported request reported by the library."""


class PratchyaUnsupported(PratchyaError):
    """A valid request outside what the kernels cover (PRATCHYA_EUNSUPPORTED),
    e.g. a GEMM shape that is not a multiple of its tile."""


class PratchyaWaitTimeout(PratchyaError):
    """A kernel's bounded wait for other workgroups ran out (the status word
    of pratchya_gemm_bs_nt_fq or pratchya_gemm_bf16_gram): the outputs that
    depended on it hold NaN.  Never expected while the kernel has the device
    to itself; reported when wait checks are on (``_kernels.check_waits``)."""


def load() -> ctypes.CDLL:
    """Load the library once; raise if it is absent or has another ABI."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m pratchya_amd.build` "
                "(the gfx950 kernels are required, there is no fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.pratchya_abi_version()
        if ver != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI {ver}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Raise the Python error matching a library status code."""
    if rc == OK:
        return
    msg = load().pratchya_last_error().decode(errors="replace")
    if rc == EINVAL:
        raise ValueError(f"{what}: {msg}")
    if rc == EUNSUPPORTED:
        raise PratchyaUnsupported(f"{what}: {msg} (status {rc})")
    raise PratchyaError(f"{what}: {msg} (status {rc})")
