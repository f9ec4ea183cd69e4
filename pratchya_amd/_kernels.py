"""Torch-tensor wrappers over the C ABI (device memory and streams only).

Every function requires CUDA (ROCm) tensors and launches the gfx950 kernels on
the current stream of the tensor's device; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import os
from typing import Tuple

import torch

from . import _lib
from ._lib import PratchyaError, PratchyaUnsupported, PratchyaWaitTimeout  # noqa: F401  (re-exported)

E4M3 = torch.float8_e4m3fn
E8M0 = torch.float8_e8m0fnu


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("pratchya_amd runs on the GPU only; got a tensor on "
                               f"{t.device} (there is no CPU fallback)")


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return _lib.DT_F32
    if dt == torch.bfloat16:
        return _lib.DT_BF16
    raise TypeError(f"unsupported dtype {dt}; expected float32 or bfloat16")


def slices_hw(shape) -> Tuple[int, int, int]:
    """(slices, H, W) of a tensor shape: 0-d -> (1,1,1), 1-d -> (1,1,n)
    (pratchya/_qualia/_qarr.py:461-464); leading dims are independent slices."""
    shape = tuple(int(s) for s in shape)
    if len(shape) == 0:
        return 1, 1, 1
    if len(shape) == 1:
        return 1, 1, shape[0]
    s = 1
    for d in shape[:-2]:
        s *= d
    return s, shape[-2], shape[-1]


def group_layout(H: int, W: int, tgrid) -> Tuple[int, int, int]:
    """(n_blk, K, M) of one [H, W] slice (pratchya/_qualia/_qarr.py:474-480)."""
    lib = _lib.load()
    n_blk, K, M = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    _lib.check(lib.pratchya_quant_layout(H, W, int(tgrid[0]), int(tgrid[1]),
                                         ctypes.byref(n_blk), ctypes.byref(K), ctypes.byref(M)),
               "quantize layout")
    return n_blk.value, K.value, M.value


def _aligned(t: torch.Tensor, n: int) -> bool:
    return t.data_ptr() % n == 0


def _check_out(out, shapes, what):
    """Caller-provided output buffers: contiguous, on the device, of the right
    byte sizes (dtype views of uint8 / e4m3fn / e8m0 and f32 are accepted)."""
    if len(out) != len(shapes):
        raise ValueError(f"{what}: expected {len(shapes)} output buffers")
    for t, (shape, esz) in zip(out, shapes):
        n = 1
        for d in shape:
            n *= int(d)
        if not t.is_cuda or not t.is_contiguous() or t.numel() * t.element_size() != n * esz:
            raise ValueError(f"{what}: output buffer of {tuple(t.shape)} {t.dtype} does not fit {shape}")


def quantize(x: torch.Tensor, tgrid, out=None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Quantize ``x`` (bf16 or f32) with block grid ``tgrid``.

    Returns ``(x_fp8 [x.shape] e4m3fn, sc_fp8 [..., M, K] e8m0, sc_fp32
    [..., M, 1, 1] f32)`` exactly as pratchya/_qualia/_qarr.py:506.  ``out``
    may hold preallocated (payload, e8m0, f32) buffers to write instead.
    """
    _require_gpu(x)
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    a, b = int(tgrid[0]), int(tgrid[1])
    S, H, W = slices_hw(x.shape)
    n_blk, K, M = group_layout(H, W, (a, b))
    lead = tuple(x.shape[:-2]) if x.dim() >= 2 else ()
    if not x.is_contiguous() or not _aligned(x, 16):
        x = x.contiguous() if not x.is_contiguous() else x.clone()
    if out is None:
        x8 = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
        sc8 = torch.empty(lead + (M, K), dtype=torch.uint8, device=x.device)
        sc32 = torch.empty(lead + (M, 1, 1), dtype=torch.float32, device=x.device)
    else:
        _check_out(out, [(x.shape, 1), (lead + (M, K), 1), (lead + (M, 1, 1), 4)], "quantize")
        x8, sc8, sc32 = _u8(out[0]), _u8(out[1]), out[2]
    lib = _lib.load()
    code = _dtype_code(x.dtype)
    ws_bytes = lib.pratchya_quantize_workspace_bytes(code, S, H, W, a, b)
    if ws_bytes == 0 and not _aligned(x8, 8 if x.dtype == torch.bfloat16 else 4):
        ws_bytes = S * n_blk * 4      # a misaligned caller payload buffer: the general path runs
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device) if ws_bytes else None
    _lib.check(lib.pratchya_quantize(_ptr(x), code, S, H, W, a, b, _ptr(x8), _ptr(sc8), _ptr(sc32),
                                     _ptr(ws) if ws is not None else None, ws_bytes, _stream(x)), "quantize")
    return x8.view(E4M3), sc8.view(E8M0), sc32


def quantize_dequantize(x: torch.Tensor, tgrid, dtype: torch.dtype, fix_nan: bool = False, out=None):
    """Fake quantization in one pass: ``dequantize_impl(*quantize_impl(x, tgrid),
    dtype, tgrid)``, i.e. ``QArrayImpl(x, tgrid).astype(dtype)``
    (pratchya/_qualia/_qarr.py:339-342, 458-506, 541-569), without writing
    the payload.  ``fix_nan`` dequantizes NaN e8m0 scales as 1.0, as
    quantize_impl's backward does for a requantized cotangent (Q:512-526).

    Returns ``(y [x.shape] dtype, sc_fp8 [..., M, K] e8m0, sc_fp32 [..., M, 1, 1])``;
    the scales are quantize_impl's, unrepaired.  ``out`` may hold preallocated
    (y, e8m0, f32) buffers.
    """
    _require_gpu(x)
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"quantize_dequantize: output dtype {dtype} is not float32 or bfloat16")
    a, b = int(tgrid[0]), int(tgrid[1])
    S, H, W = slices_hw(x.shape)
    n_blk, K, M = group_layout(H, W, (a, b))
    lead = tuple(x.shape[:-2]) if x.dim() >= 2 else ()
    if not x.is_contiguous() or not _aligned(x, 16):
        x = x.contiguous() if not x.is_contiguous() else x.clone()
    if out is None:
        y = torch.empty(x.shape, dtype=dtype, device=x.device)
        sc8 = torch.empty(lead + (M, K), dtype=torch.uint8, device=x.device)
        sc32 = torch.empty(lead + (M, 1, 1), dtype=torch.float32, device=x.device)
    else:
        esz = 2 if dtype == torch.bfloat16 else 4
        _check_out(out, [(x.shape, esz), (lead + (M, K), 1), (lead + (M, 1, 1), 4)], "quantize_dequantize")
        y, sc8, sc32 = out[0], _u8(out[1]), out[2]
    lib = _lib.load()
    code = _dtype_code(x.dtype)
    ws_bytes = lib.pratchya_quantize_dequantize_workspace_bytes(code, S, H, W, a, b)
    if ws_bytes == 0 and not (_aligned(y, 16) and _aligned(sc8, 8)):
        ws_bytes = S * n_blk * 4      # misaligned caller buffers: the general path runs
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device) if ws_bytes else None
    _lib.check(lib.pratchya_quantize_dequantize(
        _ptr(x), code, S, H, W, a, b, _ptr(y), _dtype_code(dtype), 1 if fix_nan else 0, _ptr(sc8),
        _ptr(sc32), _ptr(ws) if ws is not None else None, ws_bytes, _stream(x)), "quantize_dequantize")
    return y, sc8.view(E8M0), sc32


def requantize_cotangent(g: torch.Tensor, g_sc8: torch.Tensor, g_sc32: torch.Tensor, out=None):
    """``quantize_impl(dequantize_impl_bwd(g, g_sc8, g_sc32, (1, 128)), (1, 128))``
    in one pass (pratchya/_qualia/_qarr.py:575-601 then 458-506): the cotangent
    of a Linear output requantized for the FP8 dgrad.  ``g`` bf16 / f32 with the
    (1, 128) scales of the tensor it is the cotangent of.  Returns
    ``(g_fp8, sc_fp8, sc_fp32)`` as ``quantize(g1, (1, 128))``; raises
    ``PratchyaUnsupported`` unless the layout has 8 blocks per group."""
    _require_gpu(g, g_sc8, g_sc32)
    if g.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"requantize_cotangent: dtype {g.dtype} is not float32 or bfloat16")
    S, H, W = slices_hw(g.shape)
    n_blk, K, M = group_layout(H, W, (1, 128))
    lead = tuple(g.shape[:-2]) if g.dim() >= 2 else ()
    if not g.is_contiguous() or not _aligned(g, 16):
        g = g.contiguous() if not g.is_contiguous() else g.clone()
    gs8, gs32 = _u8(g_sc8).contiguous(), g_sc32.contiguous().float()
    if gs8.numel() != S * n_blk or gs32.numel() != S * M:
        raise ValueError("requantize_cotangent: scales do not match a (1, 128) quantization of g's shape")
    if out is None:
        x8 = torch.empty(g.shape, dtype=torch.uint8, device=g.device)
        sc8 = torch.empty(lead + (M, K), dtype=torch.uint8, device=g.device)
        sc32 = torch.empty(lead + (M, 1, 1), dtype=torch.float32, device=g.device)
    else:
        _check_out(out, [(g.shape, 1), (lead + (M, K), 1), (lead + (M, 1, 1), 4)], "requantize_cotangent")
        x8, sc8, sc32 = _u8(out[0]), _u8(out[1]), out[2]
    lib = _lib.load()
    _lib.check(lib.pratchya_requantize_cotangent(_ptr(g), _dtype_code(g.dtype), _ptr(gs8), _ptr(gs32), S, H, W,
                                                 _ptr(x8), _ptr(sc8), _ptr(sc32), _stream(g)),
               "requantize_cotangent")
    return x8.view(E4M3), sc8.view(E8M0), sc32


def _u8(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8) if t.dtype != torch.uint8 else t


def quantize_t1x128(x: torch.Tensor, x_sc8: torch.Tensor = None, x_sc32: torch.Tensor = None):
    """``quantize_impl(x^T, (1, 128))`` (pratchya/_qualia/_qarr.py:458-506)
    of a [T, C] tensor, without materialising x^T: fp8_matmul's quantization
    of its transposed raw inputs (Q:786-788).  Blocks are 128 tokens of one
    channel, groups 8 consecutive blocks of one channel.  ``x`` and the input
    scales as for ``quantize_t128``.  Returns ``(xt_fp8 [C, T] e4m3fn,
    sc_fp8 [C*T/1024, 8] e8m0, sc_fp32 [C*T/1024, 1, 1] f32)``, the
    K-contiguous (1, 128) row operand of a GEMM that contracts over tokens.
    The kernel takes T a multiple of 1024; other token counts go through the
    general quantizer on the explicitly transposed (dequantized) tensor."""
    _require_gpu(x)
    if x.dim() != 2:
        raise ValueError("quantize_t1x128 needs a [T, C] tensor")
    T, C = int(x.shape[0]), int(x.shape[1])
    if x.dtype in (E4M3, torch.uint8):
        if x_sc8 is None or x_sc32 is None:
            raise ValueError("an fp8 input needs its (1, 128) scales")
        code, xin = _lib.DT_E4M3, _u8(x)
        xs8, xs32 = _u8(x_sc8).contiguous(), x_sc32.contiguous().float()
    elif x.dtype == torch.bfloat16 and x_sc8 is not None and x_sc32 is not None:
        code, xin = _lib.DT_BF16, x
        xs8, xs32 = _u8(x_sc8).contiguous(), x_sc32.contiguous().float()
    else:
        if x_sc8 is not None or x_sc32 is not None:
            raise ValueError("input scales apply to an fp8 payload or a bf16 cotangent only")
        xin = x if x.dtype in (torch.float32, torch.bfloat16) else x.float()
        code = _dtype_code(xin.dtype)
        xs8 = xs32 = None
    if T % 1024 or C % 8:
        # the reference's composition: the values (dequantized / taken through
        # dequantize_impl_bwd as the kernel does), transposed, quantized
        if code == _lib.DT_E4M3:
            v = dequantize(xin.view(E4M3), xs8.view(E8M0), xs32, torch.float32, (1, 128))
        elif xs8 is not None:
            v = dequantize_bwd(xin, xs8.view(E8M0), xs32, (1, 128))
        else:
            v = xin
        return quantize(v.t().contiguous(), (1, 128))
    if not xin.is_contiguous() or not _aligned(xin, 16):
        xin = xin.contiguous() if not xin.is_contiguous() else xin.clone()
    M = C * T // 1024
    xt8 = torch.empty((C, T), dtype=torch.uint8, device=x.device)
    sc8 = torch.empty((M, 8), dtype=torch.uint8, device=x.device)
    sc32 = torch.empty((M, 1, 1), dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().pratchya_quantize_t1x128(_ptr(xin), code,
                                                    _ptr(xs8) if xs8 is not None else None,
                                                    _ptr(xs32) if xs32 is not None else None,
                                                    1, T, C, _ptr(xt8), _ptr(sc8), _ptr(sc32), _stream(xin)),
               "quantize_t1x128")
    return xt8.view(E4M3), sc8.view(E8M0), sc32


def quantize_128x1(x: torch.Tensor, x_sc8: torch.Tensor = None, x_sc32: torch.Tensor = None, out=None):
    """``quantize_impl(x, (128, 1))`` (pratchya/_qualia/_qarr.py:458-506) with
    the payload in ``x``'s own [..., T, C] layout, from the same inputs as
    ``quantize_t128`` (bf16 / f32, an fp8 payload with its (1, 128) scales, or
    a bf16 cotangent with them).  Returns ``(q_fp8 [..., T, C] e4m3fn, sc_fp8
    [..., M, 8] e8m0, sc_fp32 [..., M, 1, 1] f32)``, exactly quantize_impl's.
    """
    return _quantize_128x1(x, x_sc8, x_sc32, out, rows=True)


def quantize_dual(x: torch.Tensor):
    """``quantize_impl(x, (1, 128))`` and, from the same pass,
    ``quantize_impl(dequantize_impl(that), (128, 1))`` with the second payload
    in ``x``'s own [..., T, C] layout (pratchya/_qualia/_qarr.py:458-506,
    :541-569): a quantized Linear's input and the FP8 weight gradient's
    token-axis requantization of it (Q:784-789).  ``x``: bf16 or f32
    [..., T, C] with T a multiple of 128 and C of 1024
    (``PratchyaUnsupported`` for other C).  Returns ``((q, sc8, sc32), (q2,
    sc8b, sc32b))``, bit-identical to ``quantize(x, (1, 128))`` and
    ``quantize_128x1`` of its payload."""
    _require_gpu(x)
    if x.dim() < 2:
        raise ValueError("quantize_dual needs a [..., T, C] tensor")
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    if not x.is_contiguous() or not _aligned(x, 16):
        x = x.contiguous() if not x.is_contiguous() else x.clone()
    lead = tuple(x.shape[:-2])
    T, C = int(x.shape[-2]), int(x.shape[-1])
    S = 1
    for d in lead:
        S *= int(d)
    _, K1, M1 = group_layout(T, C, (1, 128))
    _, K2, M2 = group_layout(T, C, (128, 1))
    dev = x.device
    q = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    sc8 = torch.empty(lead + (M1, K1), dtype=torch.uint8, device=dev)
    sc32 = torch.empty(lead + (M1, 1, 1), dtype=torch.float32, device=dev)
    q2 = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    sc8b = torch.empty(lead + (M2, K2), dtype=torch.uint8, device=dev)
    sc32b = torch.empty(lead + (M2, 1, 1), dtype=torch.float32, device=dev)
    _lib.check(_lib.load().pratchya_quantize_dual(_ptr(x), _dtype_code(x.dtype), S, T, C, _ptr(q), _ptr(sc8),
                                                  _ptr(sc32), _ptr(q2), _ptr(sc8b), _ptr(sc32b), _stream(x)),
               "quantize_dual")
    return (q.view(E4M3), sc8.view(E8M0), sc32), (q2.view(E4M3), sc8b.view(E8M0), sc32b)


def quantize_t128(x: torch.Tensor, x_sc8: torch.Tensor = None, x_sc32: torch.Tensor = None, out=None):
    """``quantize_impl(x, (128, 1))`` (pratchya/_qualia/_qarr.py:458-506) with
    the payload transposed per slice.

    ``x``: [..., T, C] bf16 or f32, or an e4m3fn payload quantized with tgrid
    (1, 128) whose scales are ``x_sc8`` / ``x_sc32`` (dequantized to f32 first,
    as ``dequantize_impl`` does).  A bf16 ``x`` given with scales is the
    cotangent of a tensor quantized (1, 128) with them: it goes through
    ``dequantize_impl_bwd`` (Q:575-601) first, in registers.  Returns ``(xt_fp8 [..., C, T] e4m3fn,
    sc_fp8 [..., M, 8] e8m0, sc_fp32 [..., M, 1, 1] f32)``: the scales are
    exactly ``quantize_impl(x, (128, 1))``'s, the payload is its payload with
    the last two axes swapped.  ``out`` may hold preallocated buffers.
    """
    return _quantize_128x1(x, x_sc8, x_sc32, out, rows=False)


def _quantize_128x1(x, x_sc8, x_sc32, out, rows):
    name = "quantize_128x1" if rows else "quantize_t128"
    _require_gpu(x)
    if x.dim() < 2:
        raise ValueError(f"{name} needs a [..., T, C] tensor")
    lead = tuple(x.shape[:-2])
    T, C = int(x.shape[-2]), int(x.shape[-1])
    S = 1
    for d in lead:
        S *= int(d)
    if x.dtype in (E4M3, torch.uint8):
        if x_sc8 is None or x_sc32 is None:
            raise ValueError("an fp8 input needs its (1, 128) scales")
        code = _lib.DT_E4M3
        xs8, xs32 = _u8(x_sc8).contiguous(), x_sc32.contiguous().float()
        xin = _u8(x)
    elif x.dtype == torch.bfloat16 and x_sc8 is not None and x_sc32 is not None:
        code = _lib.DT_BF16
        xs8, xs32 = _u8(x_sc8).contiguous(), x_sc32.contiguous().float()
        xin = x
    else:
        if x_sc8 is not None or x_sc32 is not None:
            raise ValueError("input scales apply to an fp8 payload or a bf16 cotangent only")
        code = _dtype_code(x.dtype if x.dtype in (torch.float32, torch.bfloat16) else torch.float32)
        xin = x if x.dtype in (torch.float32, torch.bfloat16) else x.float()
        xs8 = xs32 = None
    if not xin.is_contiguous() or not _aligned(xin, 16):
        xin = xin.contiguous() if not xin.is_contiguous() else xin.clone()
    _, K, M = group_layout(T, C, (128, 1))
    qshape = lead + ((T, C) if rows else (C, T))
    if out is None:
        xt = torch.empty(qshape, dtype=torch.uint8, device=x.device)
        sc8 = torch.empty(lead + (M, K), dtype=torch.uint8, device=x.device)
        sc32 = torch.empty(lead + (M, 1, 1), dtype=torch.float32, device=x.device)
    else:
        _check_out(out, [(qshape, 1), (lead + (M, K), 1), (lead + (M, 1, 1), 4)], name)
        xt, sc8, sc32 = _u8(out[0]), _u8(out[1]), out[2]
    lib = _lib.load()
    fn = lib.pratchya_quantize_128x1 if rows else lib.pratchya_quantize_t128
    _lib.check(fn(_ptr(xin), code, _ptr(xs8) if xs8 is not None else None,
                  _ptr(xs32) if xs32 is not None else None,
                  S, T, C, _ptr(xt), _ptr(sc8), _ptr(sc32), _stream(xin)), name)
    return xt.view(E4M3), sc8.view(E8M0), sc32


def dequantize(x_fp8: torch.Tensor, sc_fp8: torch.Tensor, sc_fp32: torch.Tensor,
               dtype: torch.dtype, tgrid) -> torch.Tensor:
    """``(f32(x8) * (f32(e<<23) * G)) / 128`` cast to ``dtype``
    (pratchya/_qualia/_qarr.py:541-569)."""
    _require_gpu(x_fp8, sc_fp8, sc_fp32)
    a, b = int(tgrid[0]), int(tgrid[1])
    S, H, W = slices_hw(x_fp8.shape)
    out_dtype = dtype if dtype in (torch.float32, torch.bfloat16) else torch.float32
    x8 = _u8(x_fp8).contiguous()
    sc8 = _u8(sc_fp8).contiguous()
    sc32 = sc_fp32.contiguous().float()
    out = torch.empty(x_fp8.shape, dtype=out_dtype, device=x_fp8.device)
    lib = _lib.load()
    _lib.check(lib.pratchya_dequantize(_ptr(x8), _ptr(sc8), _ptr(sc32), S, H, W, a, b, _ptr(out),
                                       _dtype_code(out_dtype), _stream(x8)), "dequantize")
    return out if out_dtype == dtype else out.to(dtype)


def gather_dequantize(x_fp8: torch.Tensor, sc_fp8: torch.Tensor, sc_fp32: torch.Tensor, tgrid,
                      idx: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``dequantize_impl(x)[idx]`` for a 2-D quantized table and an integer index
    array of any shape (pratchya/_qualia/_qarr.py:263-284 without the full
    dequantization): returns ``idx.shape + (W,)`` in ``dtype``.  Negative
    indices count from the end; indices are clamped to the table."""
    _require_gpu(x_fp8, sc_fp8, sc_fp32, idx)
    if x_fp8.dim() != 2:
        raise ValueError("gather_dequantize needs a 2-D table")
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"gather_dequantize: output dtype {dtype} is not float32 or bfloat16")
    H, W = int(x_fp8.shape[0]), int(x_fp8.shape[1])
    a, b = int(tgrid[0]), int(tgrid[1])
    ids = idx.reshape(-1).to(torch.int64).contiguous()
    out = torch.empty(tuple(idx.shape) + (W,), dtype=dtype, device=x_fp8.device)
    x8 = _u8(x_fp8).contiguous()
    sc8 = _u8(sc_fp8).contiguous()
    sc32 = sc_fp32.contiguous().float()
    lib = _lib.load()
    _lib.check(lib.pratchya_gather_dequantize(_ptr(x8), _ptr(sc8), _ptr(sc32), H, W, a, b, _ptr(ids),
                                              ids.numel(), _ptr(out), _dtype_code(dtype), _stream(x8)),
               "gather_dequantize")
    return out


ELEMENTWISE_OPS = ("add", "sub", "mul", "div", "floordiv", "mod")


def elementwise(op: str, x, grid_x, y, grid_y, tgrid, out=None):
    """``QArrayImpl(op(dequantize_impl(x, f32), dequantize_impl(y, f32)), tgrid)``
    in one fused pass (pratchya/_qualia/_qarr.py:121-261, 715-720): ``x`` and
    ``y`` are quantized (payload, e8m0, f32) triples of one shape with block
    grids ``grid_x`` / ``grid_y``; ``op`` one of ELEMENTWISE_OPS (jnp's add,
    subtract, multiply, divide, floor_divide, remainder).  Returns the result's
    ``(payload, sc_fp8, sc_fp32)`` as ``quantize`` lays them out; ``out`` may
    hold preallocated buffers."""
    if op not in ELEMENTWISE_OPS:
        raise ValueError(f"elementwise: operator {op!r} is not one of {ELEMENTWISE_OPS}")
    x8, xs8, xs32 = x
    y8, ys8, ys32 = y
    _require_gpu(x8, xs8, xs32, y8, ys8, ys32)
    if tuple(x8.shape) != tuple(y8.shape):
        raise ValueError(f"elementwise: operand shapes {tuple(x8.shape)} and {tuple(y8.shape)} differ")
    a, b = int(tgrid[0]), int(tgrid[1])
    S, H, W = slices_hw(x8.shape)
    n_blk, K, M = group_layout(H, W, (a, b))
    lead = tuple(x8.shape[:-2]) if x8.dim() >= 2 else ()
    xq, yq = _u8(x8).contiguous(), _u8(y8).contiguous()
    xs8c, ys8c = _u8(xs8).contiguous(), _u8(ys8).contiguous()
    xs32c, ys32c = xs32.contiguous().float(), ys32.contiguous().float()
    if out is None:
        q = torch.empty(x8.shape, dtype=torch.uint8, device=x8.device)
        sc8 = torch.empty(lead + (M, K), dtype=torch.uint8, device=x8.device)
        sc32 = torch.empty(lead + (M, 1, 1), dtype=torch.float32, device=x8.device)
    else:
        _check_out(out, [(x8.shape, 1), (lead + (M, K), 1), (lead + (M, 1, 1), 4)], "elementwise")
        q, sc8, sc32 = _u8(out[0]), _u8(out[1]), out[2]
    (xa, xb), (ya, yb) = (int(v) for v in grid_x), (int(v) for v in grid_y)
    lib = _lib.load()
    ws_bytes = lib.pratchya_elementwise_workspace_bytes(S, H, W, xa, xb, ya, yb, a, b)
    if ws_bytes == 0 and not (_aligned(xq, 16) and _aligned(yq, 16) and _aligned(q, 16)):
        ws_bytes = S * n_blk * 4          # unaligned payloads take the general path
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x8.device) if ws_bytes else None
    _lib.check(lib.pratchya_elementwise(ELEMENTWISE_OPS.index(op), _ptr(xq), _ptr(xs8c), _ptr(xs32c), xa, xb,
                                        _ptr(yq), _ptr(ys8c), _ptr(ys32c), ya, yb, S, H, W, a, b, _ptr(q),
                                        _ptr(sc8), _ptr(sc32), _ptr(ws) if ws is not None else None, ws_bytes,
                                        _stream(xq)), "elementwise")
    return q.view(E4M3), sc8.view(E8M0), sc32


def gather_quantize(x_fp8: torch.Tensor, sc_fp8: torch.Tensor, sc_fp32: torch.Tensor, tgrid, idx: torch.Tensor,
                    out_grid):
    """``quantize_impl(dequantize_impl(x)[idx], out_grid)`` for a 2-D quantized
    table and an integer index array of any shape, in one fused pass
    (pratchya/_qualia/_qarr.py:263-284 then 458-506): returns the
    ``(payload, sc_fp8, sc_fp32)`` of ``idx.shape + (W,)`` as ``quantize``
    lays them out."""
    _require_gpu(x_fp8, sc_fp8, sc_fp32, idx)
    if x_fp8.dim() != 2:
        raise ValueError("gather_quantize needs a 2-D table")
    H, W = int(x_fp8.shape[0]), int(x_fp8.shape[1])
    shape = tuple(idx.shape) + (W,)
    S, T, Wd = slices_hw(shape)
    a, b = int(out_grid[0]), int(out_grid[1])
    n_blk, K, M = group_layout(T, Wd, (a, b))
    lead = shape[:-2] if len(shape) >= 2 else ()
    ids = idx.reshape(-1).to(torch.int64).contiguous()
    q = torch.empty(shape, dtype=torch.uint8, device=x_fp8.device)
    sc8 = torch.empty(lead + (M, K), dtype=torch.uint8, device=x_fp8.device)
    sc32 = torch.empty(lead + (M, 1, 1), dtype=torch.float32, device=x_fp8.device)
    ws_bytes = S * n_blk * 4
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x_fp8.device)
    x8 = _u8(x_fp8).contiguous()
    lib = _lib.load()
    _lib.check(lib.pratchya_gather_quantize(_ptr(x8), _ptr(_u8(sc_fp8).contiguous()), _ptr(sc_fp32.contiguous().float()),
                                            H, W, int(tgrid[0]), int(tgrid[1]), _ptr(ids), S, T, a, b, _ptr(q),
                                            _ptr(sc8), _ptr(sc32), _ptr(ws), ws_bytes, _stream(x8)),
               "gather_quantize")
    return q.view(E4M3), sc8.view(E8M0), sc32


def dequantize_bwd(g: torch.Tensor, sc_fp8: torch.Tensor, sc_fp32: torch.Tensor, tgrid) -> torch.Tensor:
    """Cotangent of the payload: ``(g * (f32(e<<23) * G) / 128).astype(g.dtype)``
    (pratchya/_qualia/_qarr.py:575-601)."""
    _require_gpu(g, sc_fp8, sc_fp32)
    a, b = int(tgrid[0]), int(tgrid[1])
    S, H, W = slices_hw(g.shape)
    orig = g.dtype
    gg = g if g.dtype in (torch.float32, torch.bfloat16) else g.float()
    gg = gg.contiguous()
    sc8 = _u8(sc_fp8).contiguous()
    sc32 = sc_fp32.contiguous().float()
    out = torch.empty(gg.shape, dtype=gg.dtype, device=g.device)
    lib = _lib.load()
    _lib.check(lib.pratchya_dequantize_bwd(_ptr(gg), _dtype_code(gg.dtype), _ptr(sc8), _ptr(sc32),
                                           S, H, W, a, b, _ptr(out), _stream(gg)), "dequantize_bwd")
    return out if out.dtype == orig else out.to(orig)


def debug_bf16_to_e4m3(bits: torch.Tensor, mode: int) -> torch.Tensor:
    """Run the kernels' bf16 -> e4m3fn conversion (mode 0 software, 1 gfx950
    instructions) over uint16/int16 bf16 bit patterns."""
    _require_gpu(bits)
    bits = bits.contiguous()
    out = torch.empty(bits.shape, dtype=torch.uint8, device=bits.device)
    _lib.check(_lib.load().pratchya_debug_bf16_to_e4m3(_ptr(bits), _ptr(out), bits.numel(), mode,
                                                       _stream(bits)), "debug_bf16_to_e4m3")
    return out


def debug_f32_to_bf16(x: torch.Tensor, mode: int) -> torch.Tensor:
    """Run the kernels' f32 -> bf16 rounding (mode 0 software, 1 gfx950)."""
    _require_gpu(x)
    x = x.contiguous().float()
    out = torch.empty(x.shape, dtype=torch.int16, device=x.device)
    _lib.check(_lib.load().pratchya_debug_f32_to_bf16(_ptr(x), _ptr(out), x.numel(), mode,
                                                      _stream(x)), "debug_f32_to_bf16")
    return out


# --------------------------------------------------------------------------
# Block-scaled FP8 GEMM operands
# --------------------------------------------------------------------------
class Operand:
    """An FP8 GEMM operand in the K-contiguous layout the GEMM reads.

    ``payload``: e4m3fn/uint8 [rows, K]; ``sc8``/``sc32``: the quantizer's
    scale arrays; ``desc``: (rdiv, sr, sk, kg) addressing the block of
    (row, 128-wide K block kb) as (row // rdiv) * sr + kb * sk, its group as
    block // kg.
    """

    __slots__ = ("payload", "sc8", "sc32", "desc", "k_major")

    def __init__(self, payload, sc8, sc32, desc, k_major=False):
        self.payload = payload
        self.sc8 = sc8
        self.sc32 = sc32
        self.desc = tuple(int(v) for v in desc)
        self.k_major = bool(k_major)      # payload [K, rows] instead of [rows, K]

    @property
    def rows(self) -> int:
        return int(self.payload.shape[1 if self.k_major else 0])

    @property
    def k(self) -> int:
        return int(self.payload.shape[0 if self.k_major else 1])


def operand_rows(x8: torch.Tensor, sc8: torch.Tensor, sc32: torch.Tensor, tgrid) -> Operand:
    """Operand from a 2-D tensor quantized as [rows, K] with tgrid (a, 128)
    (activations (1,128), dY, weights used as W[k_out, n] in dgrad)."""
    a, b = int(tgrid[0]), int(tgrid[1])
    if b != 128 or x8.dim() != 2:
        raise ValueError(f"operand_rows needs a 2-D payload quantized with tgrid (a, 128), got {tgrid}")
    R, K = x8.shape
    _, kg, _ = group_layout(R, K, (a, b))
    return Operand(x8, sc8, sc32, (a, K // 128, 1, kg))


def operand_transposed(x8: torch.Tensor, sc8: torch.Tensor, sc32: torch.Tensor, tgrid,
                       payload_t: torch.Tensor = None) -> Operand:
    """Operand from a 2-D tensor quantized as [K, rows] with tgrid (128, b) and
    contracted over its first axis (weights W[K, N] in the forward; (128,1)
    token-axis quantized A and dY in wgrad).  The payload is transposed to
    [rows, K] (or ``payload_t`` is used if the caller already holds it)."""
    a, b = int(tgrid[0]), int(tgrid[1])
    if a != 128 or x8.dim() != 2:
        raise ValueError(f"operand_transposed needs a 2-D payload quantized with tgrid (128, b), got {tgrid}")
    K, R = x8.shape
    _, kg, _ = group_layout(K, R, (a, b))
    pt = transpose_u8(x8) if payload_t is None else payload_t
    return Operand(pt, sc8, sc32, (b, 1, R // b, kg))


def operand_t128(xt8: torch.Tensor, sc8: torch.Tensor, sc32: torch.Tensor) -> Operand:
    """Operand from ``quantize_t128`` of a 2-D [T, C] tensor: rows are the C
    channels, the contraction runs over the T tokens (wgrad)."""
    if xt8.dim() != 2:
        raise ValueError("operand_t128 needs the payload of a 2-D tensor")
    C, T = xt8.shape
    return Operand(xt8, sc8, sc32, (1, 1, C, 8))


def operand_k128(x8: torch.Tensor, sc8: torch.Tensor, sc32: torch.Tensor) -> Operand:
    """Operand from a 2-D [T, C] tensor quantized with tgrid (128, 1) in its own
    layout (``quantize(x, (128, 1))``): rows are the C channels, the
    contraction runs over the T tokens, and the payload is read K-major."""
    if x8.dim() != 2:
        raise ValueError("operand_k128 needs the payload of a 2-D tensor")
    T, C = x8.shape
    return Operand(x8, sc8, sc32, (1, 1, C, 8), k_major=True)


def transpose_u8(x8: torch.Tensor) -> torch.Tensor:
    """[rows, cols] fp8 payload -> [cols, rows] (same dtype)."""
    _require_gpu(x8)
    src = _u8(x8).contiguous()
    R, C = src.shape
    out = torch.empty((C, R), dtype=torch.uint8, device=src.device)
    _lib.check(_lib.load().pratchya_transpose_u8(_ptr(src), R, C, _ptr(out), _stream(src)), "transpose")
    return out.view(x8.dtype) if x8.dtype != torch.uint8 else out


GEMM_TILE_ROWS = 256


def _tile_readable(p: torch.Tensor) -> torch.Tensor:
    """A [rows, K] payload whose buffer is readable for at least
    GEMM_TILE_ROWS rows: the kernel reads an operand of fewer rows as one full
    tile (rows beyond ``rows`` feed only outputs that are not stored).  A
    payload whose storage already extends that far is used in place; a
    shorter one is copied into a zero-padded buffer."""
    rows, K = int(p.shape[0]), int(p.shape[1])
    if rows >= GEMM_TILE_ROWS:
        return p
    avail = p.untyped_storage().nbytes() - p.storage_offset() * p.element_size()
    if avail >= GEMM_TILE_ROWS * K * p.element_size():
        return p
    padded = torch.zeros((GEMM_TILE_ROWS, K), dtype=p.dtype, device=p.device)
    padded[:rows].copy_(p)
    return padded[:rows]


def _word_readable(e8: torch.Tensor) -> torch.Tensor:
    """An e8m0 array readable up to the next multiple of 4 bytes (the GEMM
    reads each byte as the aligned word that holds it): used in place when its
    storage extends that far, else copied into a padded buffer."""
    n = e8.numel()
    need = (n + 3) & ~3
    avail = e8.untyped_storage().nbytes() - e8.storage_offset()
    if avail >= need:
        return e8
    padded = torch.zeros(need, dtype=torch.uint8, device=e8.device)
    padded[:n].copy_(e8.reshape(-1))
    return padded[:n]


def gemm_nt(a: Operand, b: Operand, out_dtype: torch.dtype = torch.bfloat16,
            out: torch.Tensor = None) -> torch.Tensor:
    """C[M, N] = dequant(a) @ dequant(b)^T on the FP8 MFMA kernel (any M, N;
    K a multiple of 128)."""
    _require_gpu(a.payload, b.payload)
    if a.k != b.k:
        raise ValueError(f"contraction mismatch: {a.k} vs {b.k}")
    M, N, K = a.rows, b.rows, a.k
    if a.k_major or b.k_major:
        if not (a.k_major and b.k_major):
            raise PratchyaUnsupported("gemm_nt: K-major FP8 operands are supported as a pair")
        ap, bp = _u8(a.payload).contiguous(), _u8(b.payload).contiguous()
    else:
        ap, bp = _tile_readable(_u8(a.payload).contiguous()), _tile_readable(_u8(b.payload).contiguous())
    as8, bs8 = _word_readable(_u8(a.sc8).contiguous()), _word_readable(_u8(b.sc8).contiguous())
    as32, bs32 = a.sc32.contiguous().float(), b.sc32.contiguous().float()
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=ap.device)
    lib = _lib.load()
    if a.k_major:
        _lib.check(lib.pratchya_gemm_bs_kmajor(_ptr(ap), M, _ptr(as8), _ptr(as32), *a.desc,
                                               _ptr(bp), N, _ptr(bs8), _ptr(bs32), *b.desc,
                                               M, N, K, _ptr(out), out.stride(0), _dtype_code(out.dtype),
                                               _stream(ap)), "gemm_kmajor")
        return out
    _lib.check(lib.pratchya_gemm_bs_nt(_ptr(ap), K, _ptr(as8), _ptr(as32), *a.desc,
                                       _ptr(bp), K, _ptr(bs8), _ptr(bs32), *b.desc,
                                       M, N, K, _ptr(out), out.stride(0), _dtype_code(out.dtype),
                                       _stream(ap)), "gemm")
    return out


def gemm_nt_blockmax(a: Operand, b: Operand) -> Tuple[torch.Tensor, torch.Tensor]:
    """``gemm_nt(a, b, float32)`` plus the 128 x 128 block maxima of the
    product (max |c| as f32 bits, [M / 128, N / 128] int32) from the GEMM's
    epilogue: the first pass of the product's (128, 128) requantization.
    Operands K-contiguous or both K-major; M and N multiples of 128
    (``PratchyaUnsupported`` otherwise)."""
    _require_gpu(a.payload, b.payload)
    if a.k != b.k:
        raise ValueError(f"contraction mismatch: {a.k} vs {b.k}")
    M, N, K = a.rows, b.rows, a.k
    if a.k_major != b.k_major:
        raise PratchyaUnsupported("gemm_blockmax: K-major FP8 operands are supported as a pair")
    if a.k_major:
        ap, bp = _u8(a.payload).contiguous(), _u8(b.payload).contiguous()
    else:
        ap, bp = _tile_readable(_u8(a.payload).contiguous()), _tile_readable(_u8(b.payload).contiguous())
    as8, bs8 = _word_readable(_u8(a.sc8).contiguous()), _word_readable(_u8(b.sc8).contiguous())
    as32, bs32 = a.sc32.contiguous().float(), b.sc32.contiguous().float()
    out = torch.empty((M, N), dtype=torch.float32, device=ap.device)
    bmax = torch.empty((max(M // 128, 1), max(N // 128, 1)), dtype=torch.int32, device=ap.device)
    lda, ldb = (M, N) if a.k_major else (K, K)
    _lib.check(_lib.load().pratchya_gemm_bs_blockmax(_ptr(ap), lda, _ptr(as8), _ptr(as32), *a.desc,
                                                     _ptr(bp), ldb, _ptr(bs8), _ptr(bs32), *b.desc,
                                                     M, N, K, 1 if a.k_major else 0, _ptr(out), N, _ptr(bmax),
                                                     _stream(ap)), "gemm_blockmax")
    return out, bmax


def quantize_dequantize_premax(x: torch.Tensor, block_max: torch.Tensor, tgrid, dtype: torch.dtype,
                               fix_nan: bool = False):
    """``quantize_dequantize(x, tgrid, dtype, fix_nan)`` of an f32 ``x`` whose
    block maxima ``block_max`` (f32 bits of max |x| per block, as
    ``gemm_nt_blockmax`` returns them) are already known: only the group
    scales and the cast run.  Returns ``(y, sc_fp8, sc_fp32)``."""
    _require_gpu(x, block_max)
    if x.dtype != torch.float32:
        raise ValueError("quantize_dequantize_premax: x must be float32")
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"quantize_dequantize_premax: output dtype {dtype} is not float32 or bfloat16")
    a, b = int(tgrid[0]), int(tgrid[1])
    S, H, W = slices_hw(x.shape)
    n_blk, K, M = group_layout(H, W, (a, b))
    if block_max.numel() != S * n_blk or block_max.dtype not in (torch.int32, torch.uint32):
        raise ValueError(f"quantize_dequantize_premax: block_max must hold {S * n_blk} 32-bit maxima")
    lead = tuple(x.shape[:-2]) if x.dim() >= 2 else ()
    x = x.contiguous()
    bm = block_max.contiguous()
    y = torch.empty(x.shape, dtype=dtype, device=x.device)
    sc8 = torch.empty(lead + (M, K), dtype=torch.uint8, device=x.device)
    sc32 = torch.empty(lead + (M, 1, 1), dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().pratchya_quantize_dequantize_premax(
        _ptr(x), S, H, W, a, b, _ptr(bm), _ptr(y), _dtype_code(dtype), 1 if fix_nan else 0, _ptr(sc8), _ptr(sc32),
        _stream(x)), "quantize_dequantize_premax")
    return y, sc8.view(E8M0), sc32


def gemm_bf16_nt(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """C[M, N] = a @ b^T for bf16 ``a`` [M, K] and ``b`` [N, K] with f32
    accumulation, rounded once to ``out_dtype``: the bf16 dots of
    newton_schulz (pratchya/_nnx_impl/_optimizer.py:20-22) on the MFMA kernel.
    K must be a multiple of 64 (``PratchyaUnsupported`` otherwise)."""
    _require_gpu(a, b)
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16 or a.dim() != 2 or b.dim() != 2:
        raise ValueError("gemm_bf16_nt: a and b must be 2-D bfloat16")
    if a.shape[1] != b.shape[1]:
        raise ValueError(f"contraction mismatch: {a.shape[1]} vs {b.shape[1]}")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"gemm_bf16_nt: output dtype {out_dtype} is not float32 or bfloat16")
    M, N, Kd = int(a.shape[0]), int(b.shape[0]), int(a.shape[1])
    ap, bp = _tile_readable(a.contiguous()), _tile_readable(b.contiguous())
    out = torch.empty((M, N), dtype=out_dtype, device=ap.device)
    _lib.check(_lib.load().pratchya_gemm_bf16_nt(_ptr(ap), Kd, _ptr(bp), Kd, M, N, Kd, _ptr(out), N,
                                                 _dtype_code(out_dtype), _stream(ap)), "gemm_bf16")
    return out


# bf16 piece pairs of an f32 product (see pratchya_split_pack_bf16): the six
# pairs whose weight is at least 2^-24 of the leading product
_F32_PAIRS = ((0, 0), (0, 1), (1, 0), (0, 2), (1, 1), (2, 0))


def _split_pack(src: torch.Tensor, transpose: bool, planes, kp: int, out_rows_min: int = 0) -> torch.Tensor:
    """bf16 [max(out_rows, out_rows_min), len(planes) * kp] operand of the
    bf16 GEMM: segment s holds piece planes[s] of each source row (or column,
    ``transpose``); rows beyond the source's are zero."""
    src = src.contiguous()
    R, C = int(src.shape[0]), int(src.shape[1])
    out_rows = C if transpose else R
    rows = max(out_rows, out_rows_min)
    dst = (torch.zeros if rows > out_rows else torch.empty)((rows, len(planes) * kp), dtype=torch.bfloat16,
                                                             device=src.device)
    pl = (ctypes.c_int * len(planes))(*planes)
    _lib.check(_lib.load().pratchya_split_pack_bf16(_ptr(src), _dtype_code(src.dtype), R, C, C, 1 if transpose else 0,
                                                    len(planes), pl, _ptr(dst), len(planes) * kp, kp, _stream(src)),
               "split_pack")
    return dst


def matmul_f32(a: torch.Tensor, b: torch.Tensor, a_t: bool = False, b_t: bool = False) -> torch.Tensor:
    """f32 ``op(a) @ op(b)`` for 2-D f32 / bf16 tensors on the bf16 MFMA
    kernel: ``op(a)`` is ``a`` [M, K] (``a_t``: ``a`` is [K, M] and is used
    transposed), ``op(b)`` is ``b`` [K, N] (``b_t``: ``b`` is [N, K]).  Each
    f32 operand is split into three exact bf16 pieces and the piece products
    of weight >= 2^-24 run as one bf16 GEMM along a K six times as long (three
    times for a bf16 operand, once for two): f32 products to f32 accuracy, up
    to summation order (the f32 dots of pratchya/_qualia/_qarr.py:645-712,
    :618-622)."""
    _require_gpu(a, b)
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("matmul_f32: 2-D operands expected")
    for t in (a, b):
        if t.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"matmul_f32: unsupported dtype {t.dtype}")
    M, Kd = (int(a.shape[1]), int(a.shape[0])) if a_t else (int(a.shape[0]), int(a.shape[1]))
    Kb, N = (int(b.shape[1]), int(b.shape[0])) if b_t else (int(b.shape[0]), int(b.shape[1]))
    if Kd != Kb:
        raise ValueError(f"contraction mismatch: {Kd} vs {Kb}")
    if M == 0 or N == 0:
        return torch.empty((M, N), dtype=torch.float32, device=a.device)
    if Kd == 0:
        return torch.zeros((M, N), dtype=torch.float32, device=a.device)
    na = 1 if a.dtype == torch.bfloat16 else 3
    nb = 1 if b.dtype == torch.bfloat16 else 3
    pairs = [(i, j) for i, j in _F32_PAIRS if i < na and j < nb]
    # a non-finite value takes part only in the (0, 0) pair (plane 3: piece 0
    # with non-finite values as 0)
    a_planes = [3 if (i == 0 and j > 0) else i for i, j in pairs]
    b_planes = [3 if (j == 0 and i > 0) else j for i, j in pairs]
    kp = (Kd + 63) // 64 * 64
    # the GEMM's operand rows: A = op(a) rows, B = op(b) columns (N-major);
    # an N below one tile is padded to a multiple of 4 with zero rows
    n_rows = N if N >= GEMM_TILE_ROWS else (N + 3) // 4 * 4
    A = _split_pack(a, a_t, a_planes, kp)
    B = _split_pack(b, not b_t, b_planes, kp, n_rows)
    c = gemm_bf16_nt(A, B, torch.float32)
    return c if n_rows == N else c[:, :N]


def transpose_b16(x: torch.Tensor) -> torch.Tensor:
    """[rows, cols] 16-bit matrix -> its transpose [cols, rows], contiguous."""
    _require_gpu(x)
    if x.dim() != 2 or x.element_size() != 2:
        raise ValueError("transpose_b16: a 2-D 16-bit tensor is required")
    src = x.contiguous()
    R, C = int(src.shape[0]), int(src.shape[1])
    out = torch.empty((C, R), dtype=x.dtype, device=src.device)
    _lib.check(_lib.load().pratchya_transpose_b16(_ptr(src), R, C, _ptr(out), _stream(src)), "transpose_b16")
    return out


def ns_normalize(g: torch.Tensor) -> torch.Tensor:
    """``g / (||g||_F + 1e-7)`` (pratchya/_nnx_impl/_optimizer.py:17) in g's
    dtype.  bf16: the roundings of the bf16 jnp expression -- the squares,
    their sum, the square root, the sum with 1e-7 and every quotient rounded
    to bf16; f32: f32 squares, sum, square root and quotients.  The sum is
    accumulated in f32 in a fixed order.  Returns a new contiguous tensor of
    g's shape."""
    _require_gpu(g)
    if g.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("ns_normalize: g must be bfloat16 or float32")
    gc = g.contiguous()
    out = torch.empty_like(gc)
    lib = _lib.load()
    ws = torch.empty(int(lib.pratchya_ns_normalize_workspace_bytes()), dtype=torch.uint8, device=gc.device)
    fn = lib.pratchya_ns_normalize if g.dtype == torch.bfloat16 else lib.pratchya_ns_normalize_f32
    _lib.check(fn(_ptr(gc), _ptr(out), gc.numel(), _ptr(ws), ws.numel(), _stream(gc)), "ns_normalize")
    return out


# The Gram product and the requantizing GEMM exchange data between
# workgroups with bounded waits; a wait that runs out sets a status word in
# the call's workspace (and NaN in the outputs concerned) instead of hanging.
# With checks on (check_waits(True), or PRATCHYA_CHECK_WAITS=1 in the
# environment) each such call synchronizes its stream and raises
# PratchyaWaitTimeout when the word is set (not while the stream is being
# captured into a graph); either call also copies the word into a caller's
# ``status`` tensor (int32, on the device, no sync).
_CHECK_WAITS = os.environ.get("PRATCHYA_CHECK_WAITS", "0") not in ("", "0")


def check_waits(enable: bool = True) -> bool:
    """Turn the synchronous status check of the bounded waits on or off;
    returns the previous setting."""
    global _CHECK_WAITS
    prev, _CHECK_WAITS = _CHECK_WAITS, bool(enable)
    return prev


def _wait_status(ws: torch.Tensor, offset: int, status, what: str) -> None:
    word = ws[offset:offset + 4].view(torch.int32)
    if status is not None:
        if status.dtype != torch.int32 or status.device != ws.device or status.numel() < 1:
            raise ValueError(f"{what}: status must be an int32 tensor on {ws.device}")
        status.view(-1)[:1].copy_(word)
    if _CHECK_WAITS and not torch.cuda.is_current_stream_capturing() and int(word.item()) != 0:
        raise PratchyaWaitTimeout(f"{what}: a bounded wait between workgroups ran out (outputs hold NaN)")


_GRAM_WS = {}


def _gram_workspace(device: torch.device, stream) -> torch.Tensor:
    """The Gram product's workspace for ``stream``: sized once for the largest
    grid (one range per CU) and never replaced, so that a graph that captured
    a Gram call keeps a valid workspace whatever later calls need."""
    key = (device.index, stream.cuda_stream)
    ws = _GRAM_WS.get(key)
    if ws is None:
        # a shape whose grid is one range per CU: the largest workspace
        big = int(_lib.load().pratchya_gemm_bf16_gram_workspace_bytes(256 * 64, 64 * 4096))
        ws = torch.empty(big, dtype=torch.uint8, device=device)
        _GRAM_WS[key] = ws
    return ws


def gemm_bf16_gram(a: torch.Tensor, k_major: bool = False, status: torch.Tensor = None) -> torch.Tensor:
    """The symmetric bf16 product ``a @ a^T`` (f32 accumulation, rounded once
    to bf16) of a bf16 ``a`` [M, K], the Gram product of newton_schulz
    (pratchya/_nnx_impl/_optimizer.py:20-22): only the tiles on and above the
    diagonal are computed and the lower triangle is their transpose, so the
    result is exactly symmetric.  With ``k_major``, ``a`` is given as its
    [K, M] transpose and the result is ``a^T @ a`` [M, M] (the Gram product of
    a tall iterate, read without a transposed copy).  M must be a multiple of
    256 and K of 64 (``PratchyaUnsupported`` otherwise).  The partial-tile
    workspace is kept per device and stream; calls on one stream run in
    order.  ``status``: an int32 device tensor that receives the bounded
    wait's status word (0: every partial tile arrived)."""
    _require_gpu(a)
    if a.dtype != torch.bfloat16 or a.dim() != 2:
        raise ValueError("gemm_bf16_gram: a must be 2-D bfloat16")
    M, Kd = (int(a.shape[1]), int(a.shape[0])) if k_major else (int(a.shape[0]), int(a.shape[1]))
    lib = _lib.load()
    ws_bytes = int(lib.pratchya_gemm_bf16_gram_workspace_bytes(M, Kd))
    if ws_bytes <= 0:
        raise PratchyaUnsupported(f"gemm_bf16_gram: M must be a multiple of 256 and K of 64 (got {M}, {Kd})")
    ap = a.contiguous()
    ws = _gram_workspace(ap.device, torch.cuda.current_stream(ap.device))
    if ws.numel() < ws_bytes:
        raise PratchyaError(f"gemm_bf16_gram: workspace of {ws.numel()} bytes, {ws_bytes} needed")
    out = torch.empty((M, M), dtype=torch.bfloat16, device=ap.device)
    _lib.check(lib.pratchya_gemm_bf16_gram(_ptr(ap), int(ap.stride(0)), M, Kd, 1 if k_major else 0, _ptr(out), M,
                                           _ptr(ws), int(ws.numel()), _stream(ap)), "gemm_bf16_gram")
    _wait_status(ws, int(lib.pratchya_gemm_bf16_gram_status_offset(M, Kd)), status, "gemm_bf16_gram")
    return out


def gemm_bf16_nt_ns(a: torch.Tensor, b: torch.Tensor, x: torch.Tensor, out: torch.Tensor = None,
                    b_k_major: bool = False) -> torch.Tensor:
    """One Newton-Schulz step ``1.5 x - 0.5 (a @ b^T)`` (pratchya/_nnx_impl/
    _optimizer.py:20-27) with the combination in the bf16 GEMM's epilogue: the
    same bits as ``ns_combine(x, gemm_bf16_nt(a, b))``.  ``a`` [M, K], ``b``
    [N, K] (with ``b_k_major``: ``b`` given as its [K, N] transpose, read
    without a transposed copy), ``x`` [M, N], all bf16; ``out`` must not
    overlap ``x``."""
    _require_gpu(a, b, x)
    if any(t.dtype != torch.bfloat16 or t.dim() != 2 for t in (a, b, x)):
        raise ValueError("gemm_bf16_nt_ns: a, b and x must be 2-D bfloat16")
    bk = int(b.shape[0]) if b_k_major else int(b.shape[1])
    if a.shape[1] != bk:
        raise ValueError(f"contraction mismatch: {a.shape[1]} vs {bk}")
    M, N, Kd = int(a.shape[0]), int(b.shape[1] if b_k_major else b.shape[0]), int(a.shape[1])
    if tuple(x.shape) != (M, N):
        raise ValueError(f"gemm_bf16_nt_ns: x is {tuple(x.shape)}, the product is {(M, N)}")
    ap = _tile_readable(a.contiguous())
    bp = b.contiguous() if b_k_major else _tile_readable(b.contiguous())
    xc = x.contiguous()
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=ap.device)
    _lib.check(_lib.load().pratchya_gemm_bf16_nt_ns(_ptr(ap), Kd, _ptr(bp), int(bp.stride(0)), 1 if b_k_major else 0,
                                                    M, N, Kd, _ptr(xc), N, _ptr(out), out.stride(0), _stream(ap)),
               "gemm_bf16_ns")
    return out


def mfma_ceiling(a: torch.Tensor, b: torch.Tensor, bf16: bool, iters: int) -> int:
    """Launch the MFMA-rate probe (``pratchya_mfma_ceiling``, a measurement aid
    with no reference counterpart) on the bytes of ``a`` and ``b`` (2-D,
    contiguous, at least 256 rows of 128 bytes); returns the launch's FLOP count
    for the caller's timing."""
    _require_gpu(a, b)
    if a.dim() != 2 or b.dim() != 2 or a.shape[0] < 256 or b.shape[0] < 256:
        raise ValueError("mfma_ceiling: operands of at least 256 rows")
    ld = int(a.stride(0)) * a.element_size()
    if int(b.stride(0)) * b.element_size() != ld:
        raise ValueError("mfma_ceiling: a and b need the same row stride")
    sink = torch.empty(1, dtype=torch.float32, device=a.device)
    flop = ctypes.c_int64(0)
    _lib.check(_lib.load().pratchya_mfma_ceiling(_ptr(a), _ptr(b), ld, 1 if bf16 else 0, int(iters), _ptr(sink),
                                                 ctypes.byref(flop), _stream(a)), "mfma_ceiling")
    return int(flop.value)


def gemm_nt_fq(a: Operand, b: Operand, out_dtype: torch.dtype, fix_nan: bool = False, lead=None,
               status: torch.Tensor = None):
    """``QArrayImpl(dequant(a) @ dequant(b)^T, (1, 128)).astype(out_dtype)``
    with the requantization in the GEMM's epilogue: returns ``(y [M, N],
    sc_fp8, sc_fp32)`` bit-identical to ``quantize_dequantize(gemm_nt(a, b,
    float32), (1, 128), out_dtype, fix_nan)``.  ``lead``: leading dimensions
    of the product (its rows are ``prod(lead) * H`` flattened; the scales are
    shaped per slice as quantize_impl returns them).  Raises
    ``PratchyaUnsupported`` unless N is a multiple of 1024 and B's scale
    groups span at least 32 rows.  ``status``: an int32 device tensor that
    receives the strip exchange's status word (0: every wait completed)."""
    _require_gpu(a.payload, b.payload)
    if a.k != b.k:
        raise ValueError(f"contraction mismatch: {a.k} vs {b.k}")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"gemm_nt_fq: output dtype {out_dtype} is not float32 or bfloat16")
    M, N, K = a.rows, b.rows, a.k
    lib = _lib.load()
    ws_bytes = lib.pratchya_gemm_bs_nt_fq_workspace_bytes(M, N)
    if ws_bytes <= 0:
        raise PratchyaUnsupported(f"gemm_fq: N must be a multiple of 1024 (got {N})")
    ap, bp = _tile_readable(_u8(a.payload).contiguous()), _tile_readable(_u8(b.payload).contiguous())
    as8, bs8 = _word_readable(_u8(a.sc8).contiguous()), _word_readable(_u8(b.sc8).contiguous())
    as32, bs32 = a.sc32.contiguous().float(), b.sc32.contiguous().float()
    lead = tuple(lead) if lead else (1,)
    S = 1
    for d in lead[:-1]:
        S *= int(d)
    H = M // S
    y = torch.empty((M, N), dtype=out_dtype, device=ap.device)
    sc8 = torch.empty(tuple(lead[:-1]) + (H * N // 1024, 8), dtype=torch.uint8, device=ap.device)
    sc32 = torch.empty(tuple(lead[:-1]) + (H * N // 1024, 1, 1), dtype=torch.float32, device=ap.device)
    ws = torch.empty(int(ws_bytes), dtype=torch.uint8, device=ap.device)
    _lib.check(lib.pratchya_gemm_bs_nt_fq(_ptr(ap), K, _ptr(as8), _ptr(as32), *a.desc,
                                          _ptr(bp), K, _ptr(bs8), _ptr(bs32), *b.desc,
                                          M, N, K, _ptr(y), N, _dtype_code(out_dtype), 1 if fix_nan else 0,
                                          _ptr(sc8), _ptr(sc32), _ptr(ws), int(ws_bytes), _stream(ap)), "gemm_fq")
    _wait_status(ws, int(lib.pratchya_gemm_bs_nt_fq_status_offset(M, N)), status, "gemm_fq")
    return y, sc8.view(E8M0), sc32


def gemm_nt_q11(a: Operand, b: Operand, out_dtype: torch.dtype, lead=None):
    """``QArrayImpl(dequant(a) @ dequant(b)^T, (1, 1)).astype(out_dtype)``
    with the requantization in the GEMM's epilogue (the output grid of a
    weight quantized (a, 1): lm_head, LoRA): returns ``(y [M, N], sc_fp8,
    sc_fp32)`` bit-identical to ``quantize_dequantize(gemm_nt(a, b, float32),
    (1, 1), out_dtype)``, the scales shaped per slice of ``lead`` as there.
    Raises ``PratchyaUnsupported`` unless N is a multiple of 16."""
    _require_gpu(a.payload, b.payload)
    if a.k != b.k:
        raise ValueError(f"contraction mismatch: {a.k} vs {b.k}")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"gemm_nt_q11: output dtype {out_dtype} is not float32 or bfloat16")
    M, N, K = a.rows, b.rows, a.k
    if N % 16:
        raise PratchyaUnsupported(f"gemm_q11: N must be a multiple of 16 (got {N})")
    lib = _lib.load()
    ap, bp = _tile_readable(_u8(a.payload).contiguous()), _tile_readable(_u8(b.payload).contiguous())
    as8, bs8 = _word_readable(_u8(a.sc8).contiguous()), _word_readable(_u8(b.sc8).contiguous())
    as32, bs32 = a.sc32.contiguous().float(), b.sc32.contiguous().float()
    lead = tuple(lead) if lead else (1,)
    S = 1
    for d in lead[:-1]:
        S *= int(d)
    H = M // S
    y = torch.empty((M, N), dtype=out_dtype, device=ap.device)
    sc8 = torch.empty(tuple(lead[:-1]) + (H * N, 1), dtype=torch.uint8, device=ap.device)
    sc32 = torch.empty(tuple(lead[:-1]) + (H * N, 1, 1), dtype=torch.float32, device=ap.device)
    _lib.check(lib.pratchya_gemm_bs_nt_q11(_ptr(ap), K, _ptr(as8), _ptr(as32), *a.desc,
                                           _ptr(bp), K, _ptr(bs8), _ptr(bs32), *b.desc,
                                           M, N, K, _ptr(y), N, _dtype_code(out_dtype),
                                           _ptr(sc8), _ptr(sc32), _stream(ap)), "gemm_q11")
    return y, sc8.view(E8M0), sc32


def gemm_nt_qa(x: torch.Tensor, b: Operand, out_dtype: torch.dtype, fq: bool = False, lead=None,
               status: torch.Tensor = None):
    """``quantize_impl(x, (1, 128))`` of a bf16 activation ``x`` [..., K] and
    the GEMM ``dequant(x_q) @ dequant(b)^T`` in one launch (the quantize
    prologue, pratchya_gemm_bs_nt_qa): each row of ``x`` is quantized once,
    by the GEMM's workgroups before their first tiles.  Returns ``(y [M, N], (x8, sc8,
    sc32), out_scales)``: ``(x8, sc8, sc32)`` bit-identical to
    ``quantize(x, (1, 128))`` (what the backward keeps), ``y`` bit-identical to
    ``gemm_nt(operand_rows(*that), b, out_dtype)``, or with ``fq`` to
    ``gemm_nt_fq(..., out_dtype)``, whose output scales are ``out_scales``
    (else None).  ``lead`` shapes the output scales as in gemm_nt_fq.  Raises ``PratchyaUnsupported`` where the fused path does not
    apply (x not bf16, fewer than 256 rows, K not a multiple of 1024, B's scale
    groups narrower than 32 rows, N not a multiple of 1024 with ``fq``)."""
    _require_gpu(x, b.payload)
    if x.dtype != torch.bfloat16:
        raise PratchyaUnsupported(f"gemm_qa: the quantize prologue takes bf16 activations (got {x.dtype})")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"gemm_qa: output dtype {out_dtype} is not float32 or bfloat16")
    K = int(x.shape[-1])
    if b.k != K:
        raise ValueError(f"contraction mismatch: {K} vs {b.k}")
    if b.k_major:
        raise PratchyaUnsupported("gemm_qa: B must be K-contiguous")
    M, N = x.numel() // K, b.rows
    if not x.is_contiguous() or not _aligned(x, 16):
        x = x.contiguous() if not x.is_contiguous() else x.clone()
    S, H, W = slices_hw(x.shape)
    _, Kg, Mg = group_layout(H, W, (1, 128))
    xlead = tuple(x.shape[:-2]) if x.dim() >= 2 else ()
    x8 = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    xs8 = torch.empty(xlead + (Mg, Kg), dtype=torch.uint8, device=x.device)
    xs32 = torch.empty(xlead + (Mg, 1, 1), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    ws_bytes = lib.pratchya_gemm_bs_nt_qa_workspace_bytes(M, N, 1 if fq else 0)
    if ws_bytes <= 0:
        raise PratchyaUnsupported(f"gemm_qa: unsupported shape M={M} N={N} fq={fq}")
    bp = _tile_readable(_u8(b.payload).contiguous())
    bs8, bs32 = _word_readable(_u8(b.sc8).contiguous()), b.sc32.contiguous().float()
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if fq:
        lead = tuple(lead) if lead else (1,)
        Sl = 1
        for d in lead[:-1]:
            Sl *= int(d)
        Hl = M // Sl
        osc8 = torch.empty(tuple(lead[:-1]) + (Hl * N // 1024, 8), dtype=torch.uint8, device=x.device)
        osc32 = torch.empty(tuple(lead[:-1]) + (Hl * N // 1024, 1, 1), dtype=torch.float32, device=x.device)
    else:
        osc8 = osc32 = None
    ws = torch.empty(int(ws_bytes), dtype=torch.uint8, device=x.device)
    _lib.check(lib.pratchya_gemm_bs_nt_qa(_ptr(x), K, _ptr(x8), _ptr(xs8), _ptr(xs32),
                                          _ptr(bp), K, _ptr(bs8), _ptr(bs32), *b.desc,
                                          M, N, K, _ptr(y), N, _dtype_code(out_dtype), 1 if fq else 0,
                                          _ptr(osc8) if fq else None, _ptr(osc32) if fq else None,
                                          _ptr(ws), int(ws_bytes), _stream(x)), "gemm_qa")
    _wait_status(ws, int(lib.pratchya_gemm_bs_nt_qa_status_offset(M, N, 1 if fq else 0)), status, "gemm_qa")
    xq = (x8.view(E4M3), xs8.view(E8M0), xs32)
    return y, xq, ((osc8.view(E8M0), osc32) if fq else None)


def _as_operand(x, what):
    """(tensor, dtype code, sc8, sc32) of an optimizer operand: an fp8 payload
    given as a (payload, sc8, sc32) triple, or a bf16 / f32 tensor."""
    if isinstance(x, (tuple, list)):
        x8, s8, s32 = x
        _require_gpu(x8, s8, s32)
        return _u8(x8).contiguous(), _lib.DT_E4M3, _u8(s8).contiguous(), s32.contiguous().float()
    _require_gpu(x)
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"{what}: unsupported dtype {x.dtype}")
    return x.contiguous(), _dtype_code(x.dtype), None, None


def momentum(m, g, tgrid, arith: torch.dtype, beta1: float, beta1c: float, beta2: float, beta2c: float):
    """``c = beta1*m + beta1c*g`` and ``m_new = beta2*m + beta2c*g`` of the
    Miulion step (pratchya/_nnx_impl/_optimizer.py:124-135, :157-176), one
    rounding per operation in ``arith`` (float32 or bfloat16), in one pass.
    ``m``: the quantized momentum as a (payload, sc8, sc32) triple with tgrid
    ``tgrid``; ``g``: a triple in the same layout or a bf16 / f32 tensor.  The
    constants must be values of ``arith``.  Returns ``(c, m_new)`` in ``arith``."""
    m8, _, ms8, ms32 = _as_operand(m, "momentum")
    gt, gcode, gs8, gs32 = _as_operand(g, "momentum gradient")
    if tuple(gt.shape) != tuple(m8.shape):
        raise ValueError(f"momentum: gradient shape {tuple(gt.shape)} != momentum shape {tuple(m8.shape)}")
    S, H, W = slices_hw(m8.shape)
    c = torch.empty(m8.shape, dtype=arith, device=m8.device)
    nm = torch.empty(m8.shape, dtype=arith, device=m8.device)
    lib = _lib.load()
    _lib.check(lib.pratchya_momentum(_ptr(m8), _ptr(ms8), _ptr(ms32), _ptr(gt), gcode,
                                     _ptr(gs8) if gs8 is not None else None,
                                     _ptr(gs32) if gs32 is not None else None,
                                     S, H, W, int(tgrid[0]), int(tgrid[1]), _dtype_code(arith),
                                     beta1, beta1c, beta2, beta2c, _ptr(c), _ptr(nm), _stream(m8)), "momentum")
    return c, nm


def ns_combine(x: torch.Tensor, b: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
    """``1.5 * x - 0.5 * b`` with each operation rounded to ``x.dtype`` (bf16 or
    f32), one Newton-Schulz step's combination (pratchya/_nnx_impl/_optimizer.py:
    26-27), in one pass.  ``out`` may be ``x``."""
    _require_gpu(x, b)
    if x.dtype != b.dtype or tuple(x.shape) != tuple(b.shape):
        raise ValueError("ns_combine: x and b must share dtype and shape")
    xx, bb = x.contiguous(), b.contiguous()
    if out is None:
        out = torch.empty_like(xx)
    elif not out.is_contiguous() or tuple(out.shape) != tuple(xx.shape) or out.dtype != xx.dtype:
        raise ValueError("ns_combine: out must be a contiguous tensor like x")
    lib = _lib.load()
    _lib.check(lib.pratchya_ns_combine(_ptr(xx), _ptr(bb), _ptr(out), xx.numel(), _dtype_code(xx.dtype),
                                       _stream(xx)), "ns_combine")
    return out


def apply_update(u: torch.Tensor, use_sign: bool, scale: float, p, tgrid, arith: torch.dtype,
                 lr: float, lr_wd: float, out_dtype: torch.dtype) -> torch.Tensor:
    """``-(lr * u' + lr_wd * p)`` with ``u' = sign(u)`` (Lion) or ``u * scale``
    (Muon) (pratchya/_nnx_impl/_optimizer.py:147-153, :189-197): ``p`` and
    ``u * scale`` rounded to the leaf dtype ``arith``, the products and the sum
    in f32 (``lr``, ``lr_wd`` f32 values), one rounding to ``out_dtype``.
    ``p``: a (payload, sc8, sc32) triple with tgrid ``tgrid`` or a bf16 / f32
    tensor of ``u``'s shape."""
    _require_gpu(u)
    uu = u.contiguous()
    pt, pcode, ps8, ps32 = _as_operand(p, "update parameter")
    if tuple(pt.shape) != tuple(uu.shape):
        raise ValueError(f"apply_update: parameter shape {tuple(pt.shape)} != direction shape {tuple(uu.shape)}")
    S, H, W = slices_hw(uu.shape)
    a, b = (int(tgrid[0]), int(tgrid[1])) if pcode == _lib.DT_E4M3 else (1, 1)
    out = torch.empty(uu.shape, dtype=out_dtype, device=uu.device)
    lib = _lib.load()
    _lib.check(lib.pratchya_apply_update(_ptr(uu), _dtype_code(uu.dtype), 1 if use_sign else 0, scale,
                                         _ptr(pt), pcode, _ptr(ps8) if ps8 is not None else None,
                                         _ptr(ps32) if ps32 is not None else None, S, H, W, a, b,
                                         _dtype_code(arith), lr, lr_wd, _ptr(out), _dtype_code(out_dtype),
                                         _stream(uu)), "apply_update")
    return out
