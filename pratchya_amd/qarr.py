"""Quantized arrays on the gfx950 kernels: the operator API of
``pratchya/_qualia/_qarr.py`` (abbreviated ``Q``) over PyTorch tensors.

Same class name, private attribute names (``_QArrayImpl__value``,
``__sc_fp8``, ``__sc_fp32``, ``__tgrid``), methods, module functions,
argument meaning, output shapes and custom-vjp semantics as the reference.
Every quantize, dequantize, requantize and block-scaled GEMM runs on the
gfx950 kernels of ``libpratchya_fp8.so``; PyTorch provides device memory,
streams and autograd.

Differentiation.  The reference differentiates through ``jax.custom_vjp``
rules whose cotangents for an fp8 payload are bf16/f32 arrays (dequantize's
backward, Q:575-601) or fp8 triples (matmul_impl's backward, Q:637-640), and
quantize_impl's backward (Q:514-526) passes the former through and
dequantizes the latter.  PyTorch's engine would round a gradient to its
input's dtype (e4m3fn), so payloads here stay outside the autograd graph:
``quantize_impl`` tags its payload with the tensor it was quantized from, and
the autograd Functions below (dequantize, matmul, the mixed matmuls, the
elementwise ops) return the composed cotangent -- what the reference's
quantize backward would produce -- straight to that tensor.

GEMM backward.  ``matmul_impl``'s reference backward contracts the f32
cotangent with the dequantized operands in f32 (Q:621-622) and is the default
here ("f32": dequantize kernels plus the f32 product on the bf16 MFMA
kernel over exact bf16 pieces).  The "fp8" mode
(``set_matmul_backward("fp8")``) runs dgrad and wgrad on the FP8 MFMA kernel
instead, with the cotangent quantized (1, 128) for dgrad and both wgrad
operands requantized along the token axis (128, 1) -- the scheme of
``fp8_matmul``'s backward (Q:784-789); its results differ from the f32
backward by the quantization of the cotangent.
"""
from __future__ import annotations

import math
import operator
from typing import Optional, Tuple, Union

import torch
import torch.utils._pytree as pytree

from . import _kernels as K

E4M3 = K.E4M3
E8M0 = K.E8M0

_SRC = "_pratchya_src"        # payload attribute: the tensor it was quantized from
_PAYLOAD_T = "_pratchya_t"    # payload attribute: its byte transpose (weights)

_BACKWARD_MODES = ("f32", "fp8")
_backward_mode = "f32"
# fp8 weight gradient: both operands requantized (128, 1) in their own [tokens,
# channels] layout and read K-major, or with transposed payloads read
# K-contiguous; the two give identical bits.  True: K-major for weights of at
# most _WGRAD_K_MAJOR_ROWS rows (measured: config 4's [2048, 8192] gradient
# 377 vs 396 us for both requantizations and the GEMM; the [4096, *] and
# [16384, 4096] gradients of a d_model 4096 layer no faster, 22.4 vs
# 22.1-22.3 ms per layer step); False: never.
_wgrad_k_major = True
_WGRAD_K_MAJOR_ROWS = 2048


def set_matmul_backward(mode: str) -> None:
    """Select how matmul_impl's backward contracts: "f32" (the reference's
    f32 dots of the dequantized operands, default) or "fp8" (FP8 MFMA GEMMs
    on the requantized cotangent)."""
    global _backward_mode
    if mode not in _BACKWARD_MODES:
        raise ValueError(f"matmul backward mode must be one of {_BACKWARD_MODES}, got {mode!r}")
    _backward_mode = mode


def get_matmul_backward() -> str:
    return _backward_mode


# The quantized Linear's QArrayImpl(x, (1, 128)) @ kernel (pratchya/_nnx_impl/
# _module.py:46-50): the activation quantized by its own kernel before the
# GEMM (default), or inside the GEMM's launch as a prologue
# (pratchya_gemm_bs_nt_qa; same bytes).  Measured at d_model 4096 the
# prologue is 1-3% slower than the separate pass: it runs at the GEMM's two
# waves per SIMD, where the quantizer alone runs at full occupancy.
_quantize_prologue = False


def set_quantize_prologue(fused: bool) -> None:
    """Fuse the (1, 128) activation quantization of ``QArrayImpl(x, (1, 128))
    @ kernel`` into the GEMM's launch (True) or run it as its own pass
    (False, default).  With True, such an array of a bf16 activation is held
    unquantized until first use; a product with a quantized weight dequantized
    by ``astype`` / ``dequantize`` (the Linear's output) then runs the fused
    kernel, any other use quantizes it as before.  Results are bit-identical
    either way."""
    global _quantize_prologue
    _quantize_prologue = bool(fused)


def get_quantize_prologue() -> bool:
    return _quantize_prologue


def _prologue_eligible(value, tgrid, quant) -> bool:
    """A bf16 CUDA activation [..., K] with tgrid (1, 128), K a multiple of
    1024 and at least 256 rows: what pratchya_gemm_bs_nt_qa takes."""
    if not (_quantize_prologue and quant and torch.is_tensor(value) and tgrid is not None):
        return False
    if tuple(tgrid) != (1, 128) or value.dtype != torch.bfloat16 or not value.is_cuda or value.dim() < 2:
        return False
    K = int(value.shape[-1])
    return K % 1024 == 0 and value.numel() // K >= 256


def _grid_hw(shape) -> Tuple[int, int]:
    """(H, W) of the last two axes as the reference sees them (Q:461-464)."""
    if len(shape) == 0:
        return 1, 1
    if len(shape) == 1:
        return 1, int(shape[0])
    return int(shape[-2]), int(shape[-1])


def _src(x8) -> Optional[torch.Tensor]:
    src = getattr(x8, _SRC, None)
    return src if (src is not None and torch.is_grad_enabled()) else None


def _reduce_broadcast(g: torch.Tensor, target_shape) -> torch.Tensor:
    """Sum the broadcast axes of a cotangent (Q:624-632)."""
    target_shape = tuple(target_shape)
    if tuple(g.shape) == target_shape:
        return g
    axes = list(range(g.dim() - len(target_shape)))
    for i, (gs, ts) in enumerate(zip(g.shape[len(axes):], target_shape)):
        if ts == 1 and gs > 1:
            axes.append(len(axes) + i)
    g = g.sum(dim=tuple(axes))
    return g.reshape(target_shape)


# --------------------------------------------------------------------------
# quantize_impl / dequantize_impl  (Q:458-506, Q:541-569, vjps Q:508-528, Q:571-603)
# --------------------------------------------------------------------------
def quantize_impl(x: torch.Tensor, tgrid: Tuple = (128, 128)):
    """(x_fp8, sc_fp8, sc_fp32) of ``x`` with block grid ``tgrid`` (Q:458-506)."""
    x8, s8, s32 = K.quantize(x.detach(), tuple(tgrid))
    if x.requires_grad and torch.is_grad_enabled():
        setattr(x8, _SRC, x)
    return x8, s8, s32


def _grad_dtype(src: Optional[torch.Tensor]) -> torch.dtype:
    """dtype a cotangent is delivered in: the source tensor's when a kernel can
    write it (bf16 / f32), else f32 (autograd then casts, as it would anyway)."""
    if src is not None and src.dtype in (torch.float32, torch.bfloat16):
        return src.dtype
    return torch.float32


def _requant_cotangent(g32: torch.Tensor, tgrid, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """A matmul/elementwise f32 cotangent as it reaches the quantized input:
    requantized with the input's grid (Q:637-638) and dequantized by
    quantize_impl's backward with NaN e8m0 scales read as 1.0 (Q:521-526), in
    one pass.  ``dtype`` is the input's: the f32 result rounded to it is what
    autograd would deliver."""
    return K.quantize_dequantize(g32.contiguous(), tuple(tgrid), dtype, fix_nan=True)[0]


class _Dequantize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src, x8, sc8, sc32, dtype, tgrid):
        ctx.scales = (sc8, sc32)
        ctx.tgrid = tgrid
        return K.dequantize(x8, sc8, sc32, dtype, tgrid)

    @staticmethod
    def backward(ctx, g):
        sc8, sc32 = ctx.scales
        # dequantize_impl_bwd (Q:575-601), passed through quantize_impl_bwd (Q:518-519)
        return K.dequantize_bwd(g.contiguous(), sc8, sc32, ctx.tgrid), None, None, None, None, None


def dequantize_impl(x_fp8, sc_fp8, sc_fp32, dtype, tgrid):
    """``(f32(q) * (2^(e-127) * G)) / 128`` cast to ``dtype`` (Q:541-569)."""
    src = _src(x_fp8)
    if src is not None:
        return _Dequantize.apply(src, x_fp8, sc_fp8, sc_fp32, dtype, tuple(tgrid))
    return K.dequantize(x_fp8, sc_fp8, sc_fp32, dtype, tuple(tgrid))


class _GatherDequantize(torch.autograd.Function):
    """``dequantize_impl(x)[idx]`` (Q:263-284 for an integer index array) with
    the same vjp as that composition: the cotangent is scattered into the
    table's shape (summing repeated rows, as indexing's backward does) and
    taken through dequantize_impl_bwd (Q:575-601) to the table's source."""

    @staticmethod
    def forward(ctx, src, x8, sc8, sc32, tgrid, idx):
        ctx.saved = (sc8, sc32, idx)
        ctx.tgrid = tgrid
        ctx.H = int(x8.shape[0])
        return K.gather_dequantize(x8, sc8, sc32, tgrid, idx, torch.float32)

    @staticmethod
    def backward(ctx, g):
        sc8, sc32, idx = ctx.saved
        H, W = ctx.H, int(g.shape[-1])
        rows = idx.reshape(-1).to(torch.int64)
        rows = torch.where(rows < 0, rows + H, rows).clamp(0, H - 1)
        full = torch.zeros((H, W), dtype=torch.float32, device=g.device)
        full.index_put_((rows,), g.reshape(-1, W).float(), accumulate=True)
        return K.dequantize_bwd(full, sc8, sc32, ctx.tgrid), None, None, None, None, None


def _gather_dequantize(x8, sc8, sc32, tgrid, idx):
    src = _src(x8)
    if src is not None:
        return _GatherDequantize.apply(src, x8, sc8, sc32, tuple(tgrid), idx)
    return K.gather_dequantize(x8, sc8, sc32, tuple(tgrid), idx, torch.float32)


def _deq32(x8, s8, s32, tgrid) -> torch.Tensor:
    return K.dequantize(x8, s8, s32, torch.float32, tuple(tgrid))


def _mm_f32(a: torch.Tensor, b: torch.Tensor, a_t: bool = False, b_t: bool = False) -> torch.Tensor:
    """f32 ``op(a) @ op(b)`` with torch.matmul's batch broadcasting (``op``
    transposes the last two axes when ``a_t`` / ``b_t``), every 2-D product on
    the bf16 MFMA kernel over exact bf16 pieces (``K.matmul_f32``): the f32
    dots of the reference's mixed matmuls and matmul_impl backward.  Operands
    other than f32 / bf16 are converted to f32 first."""
    if a.dtype not in (torch.float32, torch.bfloat16):
        a = a.float()
    if b.dtype not in (torch.float32, torch.bfloat16):
        b = b.float()
    if a.dim() < 2 or b.dim() < 2:
        # vector operands: matmul's 1-D promotion, then drop the added axis
        if a.dim() == 1 and b.dim() == 1:
            return _mm_f32(a[None, :], b[:, None]).reshape(())
        if a.dim() == 1:
            return _mm_f32(a[None, :], b, False, b_t).squeeze(-2)
        return _mm_f32(a, b[:, None], a_t, False).squeeze(-1)
    if b.dim() == 2 and not a_t:
        lead = tuple(a.shape[:-2])
        out = K.matmul_f32(a.reshape(-1, a.shape[-1]), b, False, b_t)
        return out.reshape(lead + (a.shape[-2], out.shape[-1]))
    if a.dim() == 2 and b.dim() == 2:
        return K.matmul_f32(a, b, a_t, b_t)
    batch = torch.broadcast_shapes(tuple(a.shape[:-2]), tuple(b.shape[:-2]))
    ab = a.expand(batch + tuple(a.shape[-2:])).reshape((-1,) + tuple(a.shape[-2:]))
    bb = b.expand(batch + tuple(b.shape[-2:])).reshape((-1,) + tuple(b.shape[-2:]))
    outs = [K.matmul_f32(ab[i], bb[i], a_t, b_t) for i in range(ab.shape[0])]
    return torch.stack(outs).reshape(batch + tuple(outs[0].shape))


# --------------------------------------------------------------------------
# Block-scaled GEMM planning
# --------------------------------------------------------------------------
_GEMM_TILE_MN, _GEMM_TILE_K = 256, 128


def _lhs_operand(x8, s8, s32, grid):
    """x [..., M, K] quantized (a, 128) as a K-contiguous GEMM operand, or None
    (a grid whose blocks are not 128 wide along K)."""
    if x8.dim() < 2 or tuple(grid)[1] != 128:
        return None
    M, Kd = int(x8.shape[-2]), int(x8.shape[-1])
    lead = 1
    for d in x8.shape[:-2]:
        lead *= int(d)
    rows = lead * M
    a = int(grid[0])
    # leading slices flatten into rows when the group size does not depend on them
    if lead > 1 and K.group_layout(rows, Kd, grid)[1] != K.group_layout(M, Kd, grid)[1]:
        return None
    if Kd % _GEMM_TILE_K or a > M or M % a:
        return None
    return K.Operand(x8.reshape(rows, Kd), s8, s32, (a, Kd // 128, 1, K.group_layout(rows, Kd, grid)[1]))


def _rhs_operand(y8, s8, s32, grid):
    """y [K, N] quantized (128, b) as the transposed GEMM operand, or None.
    The byte transpose is made once per quantization and cached on the
    payload; a weight of fewer than 256 columns (a LoRA rank) is transposed
    into a buffer of 256 rows, which the kernel reads as one full tile."""
    if y8.dim() != 2 or tuple(grid)[0] != 128:
        return None
    Kd, N = int(y8.shape[0]), int(y8.shape[1])
    if Kd % _GEMM_TILE_K or N % 16:
        return None
    pt = getattr(y8, _PAYLOAD_T, None)
    if pt is None:
        if N < _GEMM_TILE_MN:
            full = torch.zeros((_GEMM_TILE_MN, Kd), dtype=torch.uint8, device=y8.device)
            _lib_transpose_into(y8, full)
            pt = full[:N]
        else:
            pt = K.transpose_u8(y8)
        setattr(y8, _PAYLOAD_T, pt)     # a weight is transposed once per quantization
    return K.operand_transposed(y8, s8, s32, grid, payload_t=pt)


def _lib_transpose_into(y8, dst):
    """Byte-transpose the [K, N] payload y8 into the first N rows of dst [>= N, K]."""
    Kd, N = int(y8.shape[0]), int(y8.shape[1])
    src = K._u8(y8).contiguous()
    K._lib.check(K._lib.load().pratchya_transpose_u8(K._ptr(src), Kd, N, K._ptr(dst), K._stream(src)), "transpose")


def _try_gemm(op_a, op_b) -> Optional[torch.Tensor]:
    """f32 C = dequant(op_a) . dequant(op_b)^T on the FP8 MFMA kernel, or None
    if the kernel does not cover the operands' layouts (it reports that before
    launching anything)."""
    if op_a is None or op_b is None:
        return None
    try:
        return K.gemm_nt(op_a, op_b, torch.float32)
    except K.PratchyaUnsupported:
        return None


def _matmul_forward(x8, xs8, xs32, y8, ys8, ys32, gx, gy) -> torch.Tensor:
    """f32 dequant(x) @ dequant(y) (Q:605-608): the FP8 MFMA GEMM for every
    (a, 128) x (128, b) pair of block grids (any M, N; K a multiple of 128);
    grids whose blocks are not 128 wide along K (blksize 16 / 32 presets)
    take the reference's own f32 dot of the operands dequantized by the
    kernels."""
    op_a = _lhs_operand(x8, xs8, xs32, gx)
    op_b = _rhs_operand(y8, ys8, ys32, gy) if op_a is not None else None
    out = _try_gemm(op_a, op_b)
    if out is not None:
        return out.reshape(tuple(x8.shape[:-1]) + (int(y8.shape[1]),))
    return _mm_f32(_deq32(x8, xs8, xs32, gx), _deq32(y8, ys8, ys32, gy))


def _fp8_backward(g, x8, xs8, xs32, y8, ys8, ys32, gx, gy, need_x, need_y, pre=None, x_dtype=None,
                  y_dtype=None):
    """dgrad / wgrad on the FP8 MFMA kernel (the "fp8" backward), or None
    when the layouts do not fit it.  ``pre``: the (1, 128) scales of the
    product's output quantization when ``g`` is the cotangent of that output
    before dequantize_impl_bwd (the quantizers apply it in registers).
    Returns ``(gxf, gyf, gx_final, gy_final)``: with ``x_dtype`` given and
    x's rows a multiple of 1024 wide, the dgrad GEMM's epilogue also
    requantizes x's cotangent with x's grid and dequantizes it to ``x_dtype``
    as ``_requant_cotangent`` would (``gx_final`` True), bit for bit; with
    ``y_dtype`` given, a (128, 128) weight grid and both weight dimensions
    multiples of 128, the wgrad GEMM's epilogue writes the gradient's block
    maxima and ``gyf`` is the weight's cotangent requantized and dequantized
    to ``y_dtype`` as ``_requant_cotangent`` would (``gy_final`` True), from
    the group scales and the cast alone."""
    if y8.dim() != 2 or tuple(gx) != (1, 128) or tuple(gy)[1] != 128:
        return None
    if _lhs_operand(x8, xs8, xs32, gx) is None:
        return None
    Kd, N = int(y8.shape[0]), int(y8.shape[1])
    rows = g.numel() // N
    # dgrad contracts over N (blocks of 128), wgrad over the tokens (blocks of 128)
    if rows % _GEMM_TILE_K or N % _GEMM_TILE_K or Kd % 16:
        return None
    g2 = g.reshape(rows, N)
    gxf = gyf = None
    gx_final = gy_final = False
    premax = y_dtype is not None and tuple(gy) == (128, 128) and Kd % 128 == 0 and N % 128 == 0
    try:
        if need_x:
            gq = K.requantize_cotangent(g2, *pre) if pre is not None else K.quantize(g2.contiguous(), (1, 128))
            op_g = K.operand_rows(*gq, (1, 128))
            op_w = K.operand_rows(y8, ys8, ys32, gy)          # W [K, N]: rows K, contraction N
            if x_dtype is not None and Kd % 1024 == 0:
                try:
                    gxf = K.gemm_nt_fq(op_g, op_w, x_dtype, fix_nan=True)[0]
                    gx_final = True
                except K.PratchyaUnsupported:
                    # the epilogue requantization takes B scale groups of 32
                    # rows or more; other weight grids keep the FP8 dgrad with
                    # the requantization as a separate pass
                    gxf = None
            if gxf is None:
                gxf = K.gemm_nt(op_g, op_w, torch.float32)
            gxf = gxf.reshape(tuple(g.shape[:-1]) + (Kd,))
        if need_y and _wgrad_k_major and Kd <= _WGRAD_K_MAJOR_ROWS:
            # both operands requantized (128, 1) in their own [tokens, channels]
            # layout and read K-major by the GEMM (no transposed payloads)
            xq = K.quantize_128x1(x8.reshape(rows, Kd), xs8, xs32)   # stored activation, requantized
            gq = K.quantize_128x1(g2.contiguous(), *(pre if pre is not None else ()))
            op_x, op_g = K.operand_k128(*xq), K.operand_k128(*gq)
        elif need_y:
            xt = K.quantize_t128(x8.reshape(rows, Kd), xs8, xs32)
            gt = K.quantize_t128(g2.contiguous(), *(pre if pre is not None else ()))
            op_x, op_g = K.operand_t128(*xt), K.operand_t128(*gt)
        if need_y and premax:
            # the (128, 128) requantization's block maxima come from the GEMM;
            # where that variant does not apply, the plain GEMM and the full
            # requantization below
            try:
                gw, bmax = K.gemm_nt_blockmax(op_x, op_g)
                gyf = K.quantize_dequantize_premax(gw, bmax, gy, y_dtype, fix_nan=True)[0]
                gy_final = True
            except K.PratchyaUnsupported:
                gyf = None
        if need_y and gyf is None:
            gyf = K.gemm_nt(op_x, op_g, torch.float32)
    except K.PratchyaUnsupported:
        return None
    return gxf, gyf, gx_final, gy_final


def _matmul_cotangents(g, saved, grids, need_x, need_y):
    """f32 cotangents of dequant(x) and dequant(y) from the product's cotangent
    ``g`` (f32, or bf16 holding exact values): the FP8 MFMA dgrad / wgrad in
    the "fp8" mode where the layouts fit, else the reference's f32 dots of the
    dequantized operands (Q:618-622)."""
    x8, xs8, xs32, y8, ys8, ys32 = saved
    gx, gy = grids
    res = _fp8_backward(g, x8, xs8, xs32, y8, ys8, ys32, gx, gy, need_x, need_y) \
        if _backward_mode == "fp8" else None
    if res is not None:
        return res[:2]
    if g.dtype != torch.bfloat16:
        g = g.float()
    gxf = _mm_f32(g, _deq32(y8, ys8, ys32, gy), b_t=True) if need_x else None
    gyf = _mm_f32(_deq32(x8, xs8, xs32, gx), g, a_t=True) if need_y else None
    return gxf, gyf


class _Matmul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src_x, src_y, x8, xs8, xs32, y8, ys8, ys32, gx, gy):
        ctx.saved = (x8, xs8, xs32, y8, ys8, ys32)
        ctx.grids = (gx, gy)
        ctx.dtypes = (_grad_dtype(src_x), _grad_dtype(src_y))
        return _matmul_forward(x8, xs8, xs32, y8, ys8, ys32, gx, gy)

    @staticmethod
    def backward(ctx, g):
        x8, y8 = ctx.saved[0], ctx.saved[3]
        gx, gy = ctx.grids
        need_x, need_y = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        gxf, gyf = _matmul_cotangents(g, ctx.saved, ctx.grids, need_x, need_y)
        grad_x = grad_y = None
        if need_x:
            grad_x = _requant_cotangent(_reduce_broadcast(gxf, x8.shape), gx, ctx.dtypes[0])
        if need_y:
            grad_y = _requant_cotangent(_reduce_broadcast(gyf, y8.shape), gy, ctx.dtypes[1])
        return grad_x, grad_y, None, None, None, None, None, None, None, None


def _linear_forward_fused(x8, xs8, xs32, y8, ys8, ys32, gx, gy, go, dtype):
    """``QArrayImpl(matmul_impl(x, y), go).astype(dtype)`` with the
    requantization in the GEMM's epilogue: ``(y, sc_fp8, sc_fp32)`` bit-identical
    to the f32 product followed by ``quantize_dequantize``, or None when the
    layouts do not fit.  ``go`` (1, 128), a quantized Linear's output, takes
    N a multiple of 1024 (its groups span four output tiles); (1, 1), the
    output of a weight quantized (a, 1) (lm_head, LoRA), N a multiple of 16."""
    go = tuple(go)
    if go not in ((1, 128), (1, 1)) or dtype not in (torch.float32, torch.bfloat16) or y8.dim() != 2:
        return None
    N = int(y8.shape[1])
    if N % (1024 if go == (1, 128) else 16):
        return None
    op_a = _lhs_operand(x8, xs8, xs32, gx)
    op_b = _rhs_operand(y8, ys8, ys32, gy) if op_a is not None else None
    if op_a is None or op_b is None:
        return None
    lead = tuple(x8.shape[:-1])
    try:
        if go == (1, 1):
            res, s8, s32 = K.gemm_nt_q11(op_a, op_b, dtype, lead=lead)
        else:
            res, s8, s32 = K.gemm_nt_fq(op_a, op_b, dtype, lead=lead)
    except K.PratchyaUnsupported:
        return None
    return res.reshape(lead + (N,)), s8, s32


class _QLinear(torch.autograd.Function):
    """``QArrayImpl(matmul_impl(x, y), go).astype(dtype)`` as one node: the
    composition a quantized Linear runs (pratchya/_nnx_impl/_module.py:46-50;
    Q:100-105, Q:339-342).

    Forward: the f32 product, then its requantization with grid ``go`` and
    dequantization to ``dtype`` in one pass (no payload is stored).
    Backward, the reference's chain: dequantize_impl_bwd of the cotangent
    with the output's scales (Q:575-601), passed through the output
    quantization's backward (Q:518-519), matmul_impl's backward (Q:615-640)
    and each input quantization's backward (Q:521-526).  The cotangent stays
    in its own dtype (its values are exact there) and each input cotangent is
    written once, requantized and dequantized, in its source's dtype."""

    @staticmethod
    def forward(ctx, src_x, src_y, x8, xs8, xs32, y8, ys8, ys32, gx, gy, go, dtype):
        fused = _linear_forward_fused(x8, xs8, xs32, y8, ys8, ys32, gx, gy, go, dtype)
        if fused is not None:
            res, os8, os32 = fused
        else:
            out = _matmul_forward(x8, xs8, xs32, y8, ys8, ys32, gx, gy)
            res, os8, os32 = K.quantize_dequantize(out, go, dtype)
        ctx.saved = (x8, xs8, xs32, y8, ys8, ys32)
        ctx.out_scales = (os8, os32)
        ctx.grids = (gx, gy, go)
        ctx.dtypes = (_grad_dtype(src_x), _grad_dtype(src_y))
        return res

    @staticmethod
    def backward(ctx, g):
        return _qlinear_grads(ctx, g) + (None,) * 10


def _qlinear_grads(ctx, g):
    """(grad_x, grad_y) of a quantized Linear's node (_QLinear, _QLinearQA):
    inputs 0 and 1 are the sources of x and y."""
    x8, y8 = ctx.saved[0], ctx.saved[3]
    gx, gy, go = ctx.grids
    os8, os32 = ctx.out_scales
    need_x, need_y = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    g = g.contiguous()
    res = None
    if (_backward_mode == "fp8" and tuple(go) == (1, 128) and g.dtype == torch.bfloat16
            and int(os8.shape[-1]) == 8):
        # the FP8 dgrad / wgrad quantizers take the cotangent through the
        # output's dequantize_impl_bwd themselves (8-block groups: the
        # output's scales index the same way for the flattened rows)
        res = _fp8_backward(g, *ctx.saved, gx, gy, need_x, need_y, pre=(os8, os32), x_dtype=ctx.dtypes[0],
                            y_dtype=ctx.dtypes[1] if y8.dim() == 2 else None)
    gx_final = gy_final = False
    if res is not None:
        gxf, gyf, gx_final, gy_final = res
    else:
        g1 = K.dequantize_bwd(g, os8, os32, go)
        gxf, gyf = _matmul_cotangents(g1, ctx.saved, (gx, gy), need_x, need_y)
    grad_x = grad_y = None
    if need_x:
        grad_x = gxf if gx_final else _requant_cotangent(_reduce_broadcast(gxf, x8.shape), gx, ctx.dtypes[0])
    if need_y:
        grad_y = gyf if gy_final else _requant_cotangent(_reduce_broadcast(gyf, y8.shape), gy, ctx.dtypes[1])
    return grad_x, grad_y


class _QLinearQA(torch.autograd.Function):
    """_QLinear with x given unquantized (a bf16 activation, grid (1, 128)):
    the activation's quantization runs inside the GEMM's launch
    (pratchya_gemm_bs_nt_qa, with the output's requantization in its
    epilogue), and the quantized activation it writes -- the bytes
    quantize_impl returns -- becomes x's fields (``xo``) and what the backward
    contracts.  Same values and gradients as quantize_impl followed by
    _QLinear."""

    @staticmethod
    def forward(ctx, src_x, src_y, x, xo, y8, ys8, ys32, gy, go, dtype):
        op_b = _rhs_operand(y8, ys8, ys32, gy)
        if op_b is None:
            raise K.PratchyaUnsupported("gemm_qa: the weight's layout does not fit the FP8 GEMM")
        lead, N = tuple(x.shape[:-1]), int(y8.shape[1])
        res, xq, (os8, os32) = K.gemm_nt_qa(x.detach(), op_b, dtype, fq=True, lead=lead)
        if src_x is not None:
            setattr(xq[0], _SRC, src_x)
        xo._materialize(xq)
        ctx.saved = xq + (y8, ys8, ys32)
        ctx.out_scales = (os8, os32)
        ctx.grids = ((1, 128), tuple(gy), tuple(go))
        ctx.dtypes = (_grad_dtype(src_x), _grad_dtype(src_y))
        return res.reshape(lead + (N,))

    @staticmethod
    def backward(ctx, g):
        return _qlinear_grads(ctx, g) + (None,) * 8


def matmul_impl(x_fp8, x_sc8, x_sc32, y_fp8, y_sc8, y_sc32, block_grid_x: Tuple, block_grid_y: Tuple):
    """f32 ``dequant(x) @ dequant(y)`` with the reference's vjp (Q:605-640)."""
    gx, gy = tuple(block_grid_x), tuple(block_grid_y)
    sx, sy = _src(x_fp8), _src(y_fp8)
    if sx is not None or sy is not None:
        return _Matmul.apply(sx, sy, x_fp8, x_sc8, x_sc32, y_fp8, y_sc8, y_sc32, gx, gy)
    return _matmul_forward(x_fp8, x_sc8, x_sc32, y_fp8, y_sc8, y_sc32, gx, gy)


class _MatmulMixed(torch.autograd.Function):
    """dequant(x) @ y with y a plain array (Q:645-676)."""

    @staticmethod
    def forward(ctx, src_x, y, x8, xs8, xs32, gx):
        ctx.saved = (x8, xs8, xs32, y.detach())
        ctx.gx = gx
        return _mm_f32(_deq32(x8, xs8, xs32, gx), y.detach())

    @staticmethod
    def backward(ctx, g):
        x8, xs8, xs32, y = ctx.saved
        g = g.float()
        grad_x = grad_y = None
        if ctx.needs_input_grad[0]:
            gxf = _reduce_broadcast(_mm_f32(g, y, b_t=True), x8.shape)
            grad_x = _requant_cotangent(gxf, ctx.gx)
        if ctx.needs_input_grad[1]:
            grad_y = _mm_f32(_deq32(x8, xs8, xs32, ctx.gx), g, a_t=True)
        return grad_x, grad_y, None, None, None, None


def matmul_mixed_impl(x_fp8, x_sc8, x_sc32, y_f32, block_grid_x: Tuple):
    gx = tuple(block_grid_x)
    sx = _src(x_fp8)
    if sx is not None or (torch.is_grad_enabled() and y_f32.requires_grad):
        return _MatmulMixed.apply(sx, y_f32, x_fp8, x_sc8, x_sc32, gx)
    return _mm_f32(_deq32(x_fp8, x_sc8, x_sc32, gx), y_f32)


class _RMatmulMixed(torch.autograd.Function):
    """x @ dequant(y) with x a plain array (Q:679-712)."""

    @staticmethod
    def forward(ctx, x, src_y, y8, ys8, ys32, gy):
        ctx.saved = (x.detach(), y8, ys8, ys32)
        ctx.gy = gy
        return _mm_f32(x.detach(), _deq32(y8, ys8, ys32, gy))

    @staticmethod
    def backward(ctx, g):
        x, y8, ys8, ys32 = ctx.saved
        g = g.float()
        grad_x = grad_y = None
        if ctx.needs_input_grad[0]:
            grad_x = _mm_f32(g, _deq32(y8, ys8, ys32, ctx.gy), b_t=True)
        if ctx.needs_input_grad[1]:
            gyf = _reduce_broadcast(_mm_f32(x, g, a_t=True), y8.shape)
            grad_y = _requant_cotangent(gyf, ctx.gy)
        return grad_x, grad_y, None, None, None, None


def rmatmul_mixed_impl(x_f32, y_fp8, y_sc8, y_sc32, block_grid_y: Tuple):
    gy = tuple(block_grid_y)
    sy = _src(y_fp8)
    if sy is not None or (torch.is_grad_enabled() and x_f32.requires_grad):
        return _RMatmulMixed.apply(x_f32, sy, y_fp8, y_sc8, y_sc32, gy)
    return _mm_f32(x_f32, _deq32(y_fp8, y_sc8, y_sc32, gy))


# --------------------------------------------------------------------------
# Elementwise ops on two quantized arrays (Q:715-763)
# --------------------------------------------------------------------------
def _floor_divide(x, y):
    """jnp.floor_divide on float tensors: the quotient of jnp's float divmod
    (CPython's float_divmod): mod = fmod(x, y), div = (x - mod) / y, minus one
    where mod != 0 and sign(y) != sign(mod), rounded half away from zero
    (lax.round).  Differs from torch.floor_divide for a zero divisor (NaN, not
    +-inf) and in the sign of some zero quotients."""
    if not torch.is_tensor(x):
        x = torch.as_tensor(x, dtype=y.dtype, device=y.device)
    if not torch.is_tensor(y):
        y = torch.as_tensor(y, dtype=x.dtype, device=x.device)
    mod = torch.fmod(x, y)
    div = (x - mod) / y
    # sign(y) != sign(mod) for a nonzero mod: a NaN mod (zero or NaN divisor), or opposite signs
    ind = (mod != 0) & (torch.isnan(mod) | ((y < 0) != (mod < 0)))
    div = torch.where(ind, div - 1, div)
    t = torch.trunc(div)
    return torch.where((div - t).abs() >= 0.5, t + torch.sign(div), t)


class _Elementwise(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src_x, src_y, x8, xs8, xs32, y8, ys8, ys32, op, tgrid):
        ctx.saved = (x8, xs8, xs32, y8, ys8, ys32)
        ctx.op, ctx.tgrid = op, tgrid
        return op(_deq32(x8, xs8, xs32, tgrid), _deq32(y8, ys8, ys32, tgrid))

    @staticmethod
    def backward(ctx, g):
        x8, xs8, xs32, y8, ys8, ys32 = ctx.saved
        xf = _deq32(x8, xs8, xs32, ctx.tgrid)
        yf = _deq32(y8, ys8, ys32, ctx.tgrid)
        if ctx.op is _floor_divide:
            gxf = gyf = None                 # piecewise constant: zero cotangents
        else:
            with torch.enable_grad():
                xf.requires_grad_(True)
                yf.requires_grad_(True)
                out = ctx.op(xf, yf)
                gxf, gyf = torch.autograd.grad(out, (xf, yf), g, allow_unused=True)
        gxf = torch.zeros_like(xf) if gxf is None else gxf
        gyf = torch.zeros_like(yf) if gyf is None else gyf
        grad_x = _requant_cotangent(_reduce_broadcast(gxf, x8.shape), ctx.tgrid) \
            if ctx.needs_input_grad[0] else None
        grad_y = _requant_cotangent(_reduce_broadcast(gyf, y8.shape), ctx.tgrid) \
            if ctx.needs_input_grad[1] else None
        return grad_x, grad_y, None, None, None, None, None, None, None, None


def make_elementwise_impl(op):
    def impl(x_fp8, x_sc8, x_sc32, y_fp8, y_sc8, y_sc32, tgrid):
        tgrid = tuple(tgrid)
        sx, sy = _src(x_fp8), _src(y_fp8)
        if sx is not None or sy is not None:
            return _Elementwise.apply(sx, sy, x_fp8, x_sc8, x_sc32, y_fp8, y_sc8, y_sc32, op, tgrid)
        return op(_deq32(x_fp8, x_sc8, x_sc32, tgrid), _deq32(y_fp8, y_sc8, y_sc32, tgrid))
    return impl


# Python's operators on float tensors are jnp's except floor division: % is
# torch.remainder (fmod, plus the divisor where the signs differ), as jnp.mod.
add_impl = make_elementwise_impl(operator.add)
mul_impl = make_elementwise_impl(operator.mul)
sub_impl = make_elementwise_impl(operator.sub)
truediv_impl = make_elementwise_impl(operator.truediv)
floordiv_impl = make_elementwise_impl(_floor_divide)
mod_impl = make_elementwise_impl(operator.mod)
pow_impl = make_elementwise_impl(operator.pow)


class _ElementwiseResult(_Elementwise):
    """Autograd node of an elementwise result computed by the fused kernel
    (pratchya_elementwise), which never stores the f32 result op(x, y).  The
    node's output stands in for that result as the source of the quantized
    payload: consumers of a quantized array compute from its payload and
    scales and use the source only to route the cotangent, so the output is a
    zero placeholder of the result's shape.  Backward is make_elementwise_impl's
    vjp (Q:722-750), as for _Elementwise."""

    @staticmethod
    def forward(ctx, src_x, src_y, x8, xs8, xs32, y8, ys8, ys32, op, tgrid):
        ctx.saved = (x8, xs8, xs32, y8, ys8, ys32)
        ctx.op, ctx.tgrid = op, tgrid
        return torch.zeros((), dtype=torch.float32, device=x8.device).expand(x8.shape)


# Operators the fused kernel computes (jnp.power is not among them: its f32
# results depend on the pow implementation).
_FUSED = {operator.add: "add", operator.sub: "sub", operator.mul: "mul", operator.truediv: "div",
          _floor_divide: "floordiv", operator.mod: "mod"}


def _fused_elementwise(op, x, grid_x, y, grid_y, tgrid):
    """QArrayImpl(op(dequant(x), dequant(y)), tgrid) for quantized triples of
    one shape, by the fused kernel, or None where it does not apply: another
    operator, broadcast shapes, or a gradient through operands quantized with
    different grids (that value is an f32 sum of two astype()s, Q:127-128, whose
    vjp is dequantize_impl's rather than the elementwise one)."""
    name = _FUSED.get(op)
    if name is None or tuple(x[0].shape) != tuple(y[0].shape) or not x[0].is_cuda:
        return None
    if x[0].dtype != E4M3 or y[0].dtype != E4M3:
        return None
    sx, sy = _src(x[0]), _src(y[0])
    grad = sx is not None or sy is not None
    if grad and (tuple(grid_x) != tuple(tgrid) or tuple(grid_y) != tuple(tgrid)):
        return None
    out8, s8, s32 = K.elementwise(name, x, grid_x, y, grid_y, tgrid)
    if grad:
        setattr(out8, _SRC, _ElementwiseResult.apply(sx, sy, *x, *y, op, tuple(tgrid)))
    return QArrayImpl._tree_unflatten((True, tuple(tgrid)), (out8, s8, s32))


# --------------------------------------------------------------------------
# QArrayImpl  (Q:15-425)
# --------------------------------------------------------------------------
_REFLECTED = {"__matmul__": "__rmatmul__", "__add__": "__radd__", "__sub__": "__rsub__",
              "__mul__": "__rmul__", "__truediv__": "__rtruediv__", "__div__": "__rtruediv__",
              "__floordiv__": "__rfloordiv__", "__mod__": "__rmod__", "__pow__": "__rpow__"}


def _value_of(other):
    return other.value if hasattr(other, "value") else other


def _adapted_grid(grid, shape) -> Tuple[int, int]:
    """Grid adapted to a new shape by gcd (Q:371-380)."""
    H, W = _grid_hw(shape)
    return math.gcd(int(grid[0]), H), math.gcd(int(grid[1]), W)


class QArrayImpl:
    """An FP8 block-quantized array: e4m3fn payload, per-block e8m0 scales and
    per-group f32 maxima (Q:15-425).  ``quant=False`` wraps a plain tensor."""

    def __new__(cls, value=None, tgrid=None, quant=True, **kwargs):
        # with the quantize prologue on, an activation the fused GEMM takes is
        # held unquantized (_PendingQuant) until its first use (subclasses
        # pass their own constructor arguments through)
        if cls is QArrayImpl and _prologue_eligible(value, tgrid, quant):
            return super().__new__(_PendingQuant)
        return super().__new__(cls)

    def __init__(self, value: Union["QArrayImpl", torch.Tensor], tgrid: Optional[Tuple[int, int]] = None,
                 quant: bool = True):
        if not quant:
            self.__value = value
        elif isinstance(value, QArrayImpl):
            self.__tgrid = value._QArrayImpl__tgrid
            self.__value = value._QArrayImpl__value
            self.__sc_fp8 = value._QArrayImpl__sc_fp8
            self.__sc_fp32 = value._QArrayImpl__sc_fp32
        else:
            assert tgrid is not None
            self.__tgrid = tuple(tgrid)
            if not torch.is_tensor(value):
                value = torch.as_tensor(value, dtype=torch.float32, device="cuda")
            # the reference upcasts to f32 (Q:29); bf16 and f32 inputs quantize
            # to identical bytes, so bf16 is passed through unconverted
            if value.dtype not in (torch.float32, torch.bfloat16):
                value = value.float()
            self.__value, self.__sc_fp8, self.__sc_fp32 = self.__quantize(value)

    def get_value(self):
        return self.__value

    def __quantize(self, value):
        # Q:35-44: 3-D arrays are quantized slice by slice; the kernels treat
        # leading axes as independent slices in one launch, with the same bytes.
        return quantize_impl(value, self.__tgrid)

    def dequantize(self, dtype):
        if self.__value.dtype != E4M3:
            return self.__value.to(dtype)
        return dequantize_impl(self.__value, self.__sc_fp8, self.__sc_fp32, dtype, self.__tgrid)

    def __jax_array__(self):
        return self.dequantize(torch.float32)

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        """Torch functions see a quantized array as its f32 dequantization
        (the role of ``__jax_array__`` for jnp functions, Q:58-59).  A tensor
        operator with the quantized array on its right (``t @ q``, ``t - q``)
        goes to the array's reflected method, as Python's operator protocol
        does for the reference's arrays."""
        kwargs = kwargs or {}
        name = getattr(func, "__name__", "")
        if (name in _REFLECTED and len(args) == 2 and not kwargs and isinstance(args[1], QArrayImpl)
                and not isinstance(args[0], QArrayImpl)):
            return getattr(args[1], _REFLECTED[name])(args[0])
        is_q = lambda v: isinstance(v, QArrayImpl)
        unwrap = lambda v: v.astype(torch.float32) if is_q(v) else v
        return func(*pytree.tree_map(unwrap, args, is_leaf=is_q), **pytree.tree_map(unwrap, kwargs, is_leaf=is_q))

    @property
    def shape(self):
        return tuple(self.__value.shape)

    @property
    def size(self):
        return self.__value.numel()

    @property
    def dtype(self):
        return self.__value.dtype

    @property
    def tgrid(self):
        return self.__tgrid

    def _promote(self, other, grid_idx=0):
        if isinstance(other, QArrayImpl):
            return other
        shape = tuple(other.shape) if hasattr(other, "shape") else tuple(torch.as_tensor(other).shape)
        H, W = _grid_hw(shape)
        target_a = self.__tgrid[0] if grid_idx == 0 else self.__tgrid[1]
        target_b = self.__tgrid[1]
        return QArrayImpl(other, tgrid=(math.gcd(target_a, H), math.gcd(target_b, W)))

    def __matmul__(self, other):
        other = _value_of(other)
        if "_pending" in self.__dict__ and isinstance(other, QArrayImpl):
            # x not quantized yet: the product keeps it so, for the fused GEMM
            return _LazyProduct(None, self.__tgrid, other.__tgrid, pending=(self, other))
        if isinstance(other, QArrayImpl):
            other = self._promote(other, 1)
            # QArrayImpl(matmul_impl(self, other), (self.tgrid[0], other.tgrid[1])) (Q:100-105)
            return _LazyProduct((self.__value, self.__sc_fp8, self.__sc_fp32, other.__value, other.__sc_fp8,
                                 other.__sc_fp32), self.__tgrid, other.__tgrid)
        return matmul_mixed_impl(self.__value, self.__sc_fp8, self.__sc_fp32, other, self.__tgrid)

    def __rmatmul__(self, other):
        other = _value_of(other)
        if isinstance(other, QArrayImpl):
            other = self._promote(other, 0)
            return _LazyProduct((other.__value, other.__sc_fp8, other.__sc_fp32, self.__value, self.__sc_fp8,
                                 self.__sc_fp32), other.__tgrid, self.__tgrid)
        return rmatmul_mixed_impl(other, self.__value, self.__sc_fp8, self.__sc_fp32, self.__tgrid)

    # -- elementwise arithmetic (Q:121-261) --------------------------------
    def _binary(self, other, impl, op, reverse=False):
        other = _value_of(other)
        if isinstance(other, QArrayImpl):
            other = self._promote(other)
            a, b = (other, self) if reverse else (self, other)
            fused = _fused_elementwise(op, (a.__value, a.__sc_fp8, a.__sc_fp32), a.__tgrid,
                                       (b.__value, b.__sc_fp8, b.__sc_fp32), b.__tgrid, self.__tgrid)
            if fused is not None:
                return fused
            if self.__tgrid != other.tgrid:
                return QArrayImpl(op(a.astype(torch.float32), b.astype(torch.float32)), self.__tgrid)
            x_out = impl(a.__value, a.__sc_fp8, a.__sc_fp32, b.__value, b.__sc_fp8, b.__sc_fp32, self.__tgrid)
            return QArrayImpl(x_out, self.__tgrid)
        dt = getattr(other, "dtype", torch.float32)
        mine = self.astype(dt if isinstance(dt, torch.dtype) else torch.float32)
        return op(other, mine) if reverse else op(mine, other)

    def __add__(self, other):
        return self._binary(other, add_impl, operator.add)

    def __radd__(self, other):
        return self.__add__(_value_of(other))

    def __sub__(self, other):
        return self._binary(other, sub_impl, operator.sub)

    def __rsub__(self, other):
        return self._binary(other, sub_impl, operator.sub, reverse=True)

    def __mul__(self, other):
        return self._binary(other, mul_impl, operator.mul)

    def __rmul__(self, other):
        return self.__mul__(_value_of(other))

    def __truediv__(self, other):
        return self._binary(other, truediv_impl, operator.truediv)

    def __rtruediv__(self, other):
        return self._binary(other, truediv_impl, operator.truediv, reverse=True)

    def __floordiv__(self, other):
        return self._binary(other, floordiv_impl, _floor_divide)

    def __rfloordiv__(self, other):
        return self._binary(other, floordiv_impl, _floor_divide, reverse=True)

    def __mod__(self, other):
        return self._binary(other, mod_impl, operator.mod)

    def __rmod__(self, other):
        return self._binary(other, mod_impl, operator.mod, reverse=True)

    def __pow__(self, other):
        return self._binary(other, pow_impl, operator.pow)

    def __rpow__(self, other):
        return self._binary(other, pow_impl, operator.pow, reverse=True)

    # -- views and restructuring (Q:263-402) --------------------------------
    def __getitem__(self, idx):
        if not hasattr(self, "_QArrayImpl__tgrid"):
            return QArrayImpl(self.get_value()[idx], quant=False)
        if (torch.is_tensor(idx) and not idx.is_floating_point() and idx.dtype != torch.bool
                and self.__value.dim() == 2 and self.__value.dtype == E4M3):
            # an embedding lookup: only the indexed rows are dequantized; without
            # a gradient to route, the rows are requantized in the same pass
            idx = idx.to(self.__value.device)
            if _src(self.__value) is None:
                grid = _adapted_grid(self.__tgrid, tuple(idx.shape) + (int(self.__value.shape[1]),))
                return QArrayImpl._tree_unflatten(
                    (True, grid), K.gather_quantize(self.__value, self.__sc_fp8, self.__sc_fp32, self.__tgrid,
                                                    idx, grid))
            sliced = _gather_dequantize(self.__value, self.__sc_fp8, self.__sc_fp32, self.__tgrid, idx)
        else:
            sliced = self.dequantize(torch.float32)[idx]
        return QArrayImpl(sliced, _adapted_grid(self.__tgrid, sliced.shape))

    def __neg__(self):
        new_obj = QArrayImpl.__new__(QArrayImpl)
        new_obj._QArrayImpl__tgrid = self.__tgrid
        new_obj._QArrayImpl__value = self.__value
        new_obj._QArrayImpl__sc_fp8 = self.__sc_fp8
        new_obj._QArrayImpl__sc_fp32 = -self.__sc_fp32
        return new_obj

    def apply(self, func):
        out_val = func(self.dequantize(torch.float32))
        return QArrayImpl(out_val, _adapted_grid(self.__tgrid, out_val.shape))

    def __abs__(self):
        new_obj = QArrayImpl.__new__(QArrayImpl)
        new_obj._QArrayImpl__tgrid = self.__tgrid
        # |q| of an e4m3fn byte clears its sign bit (NaN stays NaN)
        new_obj._QArrayImpl__value = (self.__value.view(torch.uint8) & 0x7F).view(E4M3)
        new_obj._QArrayImpl__sc_fp8 = self.__sc_fp8
        new_obj._QArrayImpl__sc_fp32 = self.__sc_fp32.abs()
        return new_obj

    def __repr__(self):
        return f"{self.__value}"

    @property
    def at(self):
        fp8_array = self

        class _Setter:
            def __init__(self, idx):
                self.idx = idx

            def set(self, val):
                val_f32 = val.astype(torch.float32) if isinstance(val, QArrayImpl) else val
                out = fp8_array.dequantize(torch.float32).clone()
                out[self.idx] = val_f32
                return QArrayImpl(out, fp8_array.tgrid)

        class _Helper:
            def __getitem__(self, idx):
                return _Setter(idx)

        return _Helper()

    def astype(self, dtype):
        if not hasattr(self, "_QArrayImpl__tgrid"):
            return self.get_value().to(dtype)
        return self.dequantize(dtype)

    @property
    def mT(self):
        return QArrayImpl(self.astype(torch.float32).transpose(-1, -2), (self.__tgrid[1], self.__tgrid[0]))

    @property
    def T(self):
        x = self.astype(torch.float32)
        return QArrayImpl(x.permute(*reversed(range(x.dim()))), (self.__tgrid[1], self.__tgrid[0]))

    def reshape(self, *args, **kwargs):
        shape = args[0] if len(args) == 1 and isinstance(args[0], (tuple, list)) else args
        return self._requantize(self.dequantize(torch.float32).reshape(*shape, **kwargs))

    def transpose(self, *axes):
        axes = axes[0] if len(axes) == 1 and isinstance(axes[0], (tuple, list)) else axes
        x = self.dequantize(torch.float32)
        return self._requantize(x.permute(*axes) if axes else x.permute(*reversed(range(x.dim()))))

    def sum(self, *args, **kwargs):
        if "axis" in kwargs:
            kwargs["dim"] = kwargs.pop("axis")
        if "keepdims" in kwargs:
            kwargs["keepdim"] = kwargs.pop("keepdims")
        return self._requantize(self.dequantize(torch.float32).sum(*args, **kwargs))

    def _requantize(self, out_val):
        return QArrayImpl(out_val, _adapted_grid(self.__tgrid, out_val.shape))

    @classmethod
    def concat(cls, arrays, axis=0):
        fp32 = [a.astype(torch.float32) if isinstance(a, QArrayImpl) else a for a in arrays]
        out = torch.cat(fp32, dim=axis)
        first = next((a for a in arrays if isinstance(a, QArrayImpl)), None)
        grid = first.tgrid if first else (1, 128)
        return cls(out, _adapted_grid(grid, out.shape))

    def _tree_flatten(self):
        if hasattr(self, "_QArrayImpl__tgrid"):
            return (self.__value, self.__sc_fp8, self.__sc_fp32), (True, self.__tgrid)
        return (self.__value,), (False, None)

    @classmethod
    def _tree_unflatten(cls, aux_data, children):
        is_quant, tgrid = aux_data
        obj = cls.__new__(cls)
        if is_quant:
            obj._QArrayImpl__tgrid = tgrid
            obj._QArrayImpl__value, obj._QArrayImpl__sc_fp8, obj._QArrayImpl__sc_fp32 = children
        else:
            obj._QArrayImpl__value = children[0]
        return obj


class _LazyProduct(QArrayImpl):
    """``QArrayImpl(matmul_impl(x, y), (x.tgrid[0], y.tgrid[1]))`` (Q:100-105,
    Q:111-116) held as its operands until first use.

    Dequantizing it to bf16 / f32 (``astype`` / ``dequantize``, how a Linear
    emits its output, pratchya/_nnx_impl/_module.py:50) runs the product, the
    requantization and the dequantization as one autograd node (_QLinear) and
    never stores the requantized payload; values and gradients are those of
    the step-by-step composition.  Any other use (payload, scales, slicing,
    arithmetic, pytree flattening) first materialises the quantized array
    exactly as the reference builds it, after which the object behaves as a
    plain QArrayImpl.  Repeated dequantizations to one dtype before that run
    the product once and return copies of its result; if the first result was
    changed in place (impossible on the reference's immutable arrays), the
    product is run again, so no returned tensor sees another's changes."""

    _FIELDS = ("_QArrayImpl__value", "_QArrayImpl__sc_fp8", "_QArrayImpl__sc_fp32")

    def __init__(self, operands, gx, gy, pending=None):
        self._QArrayImpl__tgrid = (int(gx[0]), int(gy[1]))
        self._operands = operands
        self._grids = (tuple(gx), tuple(gy))
        self._grad_enabled = torch.is_grad_enabled()
        self._dequantized = {}
        if pending is not None:
            # (x, y) with x a _PendingQuant not quantized yet: the Linear's
            # output (dequantize) takes x into the fused GEMM, anything else
            # quantizes it first (_resolve)
            self._pending_xy = pending
        else:
            self._srcs = (_src(operands[0]), _src(operands[3]))

    def _resolve(self):
        """The operands of a product whose x was pending, x quantized now."""
        if "_pending_xy" in self.__dict__:
            xo, yo = self.__dict__.pop("_pending_xy")
            with torch.set_grad_enabled(self._grad_enabled):
                self._operands = (xo._QArrayImpl__value, xo._QArrayImpl__sc_fp8, xo._QArrayImpl__sc_fp32,
                                  yo._QArrayImpl__value, yo._QArrayImpl__sc_fp8, yo._QArrayImpl__sc_fp32)
                self._srcs = (_src(self._operands[0]), _src(self._operands[3]))

    def _fused_dequantize(self, dtype):
        """The Linear's output with x's quantization in the GEMM's launch, or
        None where the fused kernel does not apply (x is then still pending)."""
        xo, yo = self._pending_xy
        go = self._QArrayImpl__tgrid
        gy = self._grids[1]
        if "_pending" not in xo.__dict__ or tuple(go) != (1, 128):
            return None
        y8, ys8, ys32 = yo._QArrayImpl__value, yo._QArrayImpl__sc_fp8, yo._QArrayImpl__sc_fp32
        if y8.dim() != 2 or int(y8.shape[1]) % 1024 or _rhs_operand(y8, ys8, ys32, gy) is None:
            return None
        x = xo._pending
        with torch.set_grad_enabled(self._grad_enabled):
            sx = x if (x.requires_grad and torch.is_grad_enabled()) else None
            sy = _src(y8)
            try:
                res = _QLinearQA.apply(sx, sy, x, xo, y8, ys8, ys32, gy, go, dtype)
            except K.PratchyaUnsupported:
                return None
        self._resolve()
        return res

    def __getattr__(self, name):
        # reached only for attributes not set yet: the quantized fields
        if name in _LazyProduct._FIELDS and "_operands" in self.__dict__:
            self._materialize()
            return self.__dict__[name]
        raise AttributeError(name)

    def _materialize(self):
        self._resolve()
        x8, xs8, xs32, y8, ys8, ys32 = self._operands
        gx, gy = self._grids
        sx, sy = self._srcs
        with torch.set_grad_enabled(self._grad_enabled):
            if sx is not None or sy is not None:
                out = _Matmul.apply(sx, sy, x8, xs8, xs32, y8, ys8, ys32, gx, gy)
            else:
                out = _matmul_forward(x8, xs8, xs32, y8, ys8, ys32, gx, gy)
            v, s8, s32 = quantize_impl(out, self._QArrayImpl__tgrid)
        self._QArrayImpl__value, self._QArrayImpl__sc_fp8, self._QArrayImpl__sc_fp32 = v, s8, s32
        del self._operands, self._srcs, self._dequantized

    def dequantize(self, dtype):
        if "_operands" not in self.__dict__ or dtype not in (torch.float32, torch.bfloat16):
            return super().dequantize(dtype)
        hit = self._dequantized.get(dtype)
        if hit is not None and hit[0]._version == hit[1]:
            return hit[0].clone()
        if "_pending_xy" in self.__dict__:
            res = self._fused_dequantize(dtype)
            if res is not None:
                self._dequantized[dtype] = (res, res._version)
                return res
            self._resolve()
        x8, xs8, xs32, y8, ys8, ys32 = self._operands
        gx, gy = self._grids
        go = self._QArrayImpl__tgrid
        sx, sy = self._srcs
        with torch.set_grad_enabled(self._grad_enabled):
            if sx is not None or sy is not None:
                res = _QLinear.apply(sx, sy, x8, xs8, xs32, y8, ys8, ys32, gx, gy, go, dtype)
            else:
                fused = _linear_forward_fused(x8, xs8, xs32, y8, ys8, ys32, gx, gy, go, dtype)
                if fused is not None:
                    res = fused[0]
                else:
                    out = _matmul_forward(x8, xs8, xs32, y8, ys8, ys32, gx, gy)
                    res = K.quantize_dequantize(out, go, dtype)[0]
        self._dequantized[dtype] = (res, res._version)   # recomputed if changed in place
        return res

    @property
    def shape(self):
        if "_pending_xy" in self.__dict__:
            xs, ys = self._pending_xy[0].shape, self._pending_xy[1].shape
            return tuple(torch.empty(xs, device="meta").matmul(torch.empty(ys, device="meta")).shape)
        if "_operands" in self.__dict__:
            x8, y8 = self._operands[0], self._operands[3]
            return tuple(torch.empty(x8.shape, device="meta").matmul(torch.empty(y8.shape, device="meta")).shape)
        return super().shape

    @property
    def size(self):
        return math.prod(self.shape)

    @property
    def dtype(self):
        return E4M3


class _PendingQuant(QArrayImpl):
    """``QArrayImpl(x, (1, 128))`` of a bf16 activation with the quantize
    prologue on (set_quantize_prologue): x held unquantized until first use.
    A product with a quantized weight that the Linear dequantizes quantizes x
    inside the GEMM's launch (_QLinearQA) and fills the fields with its bytes;
    any other use (payload, scales, arithmetic, slicing, pytree flattening)
    quantizes x first with quantize_impl.  Either way the fields hold
    quantize_impl(x, (1, 128)) bit for bit."""

    _FIELDS = ("_QArrayImpl__value", "_QArrayImpl__sc_fp8", "_QArrayImpl__sc_fp32")

    def __init__(self, value, tgrid=None, quant: bool = True):
        self._QArrayImpl__tgrid = (1, 128)
        self._pending = value
        self._grad_enabled = torch.is_grad_enabled()

    def __getattr__(self, name):
        # reached only for attributes not set yet: the quantized fields
        if name in _PendingQuant._FIELDS and "_pending" in self.__dict__:
            self._materialize()
            return self.__dict__[name]
        raise AttributeError(name)

    def _materialize(self, q=None):
        """Fill the fields: with ``q`` (the fused GEMM's quantized x) or by
        quantize_impl."""
        value = self.__dict__.pop("_pending")
        if q is None:
            with torch.set_grad_enabled(self._grad_enabled):
                q = quantize_impl(value, (1, 128))
        self._QArrayImpl__value, self._QArrayImpl__sc_fp8, self._QArrayImpl__sc_fp32 = q

    @property
    def shape(self):
        if "_pending" in self.__dict__:
            return tuple(self._pending.shape)
        return super().shape

    @property
    def size(self):
        return math.prod(self.shape)

    @property
    def dtype(self):
        return E4M3


for _cls in (QArrayImpl, _LazyProduct, _PendingQuant):   # lazy forms flatten to their materialised fields
    pytree.register_pytree_node(
        _cls,
        lambda q: q._tree_flatten(),
        lambda children, aux: QArrayImpl._tree_unflatten(aux, tuple(children)),
    )


# --------------------------------------------------------------------------
# fp8_matmul (Q:766-793)
# --------------------------------------------------------------------------
def _quantized_transpose(x, tgrid):
    """``QArrayImpl(x^T, tgrid)`` of a 2-D x [T, C] (the transposed operands
    of fp8_matmul's backward, Q:786-788).  With tgrid (1, 128), f32 / bf16
    values, T a multiple of 1024 and C of 8, quantize_t1x128 writes the same
    bytes without materialising x^T."""
    if (tuple(tgrid) == (1, 128) and x.dim() == 2 and x.dtype in (torch.float32, torch.bfloat16)
            and int(x.shape[0]) % 1024 == 0 and int(x.shape[1]) % 8 == 0):
        return QArrayImpl._tree_unflatten((True, (1, 128)), K.quantize_t1x128(x.contiguous()))
    return QArrayImpl(x.transpose(-1, -2), tgrid)


def _fp8_matmul_value(x, y, tgrid):
    with torch.no_grad():
        qx = x if isinstance(x, QArrayImpl) else QArrayImpl(x, tgrid)
        qy = y if isinstance(y, QArrayImpl) else QArrayImpl(y, tgrid)
        return (qx @ qy).dequantize(torch.float32)


class _FP8Matmul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, tgrid):
        ctx.save_for_backward(x, y)
        ctx.tgrid = tgrid
        return _fp8_matmul_value(x.detach(), y.detach(), tgrid)

    @staticmethod
    def backward(ctx, g):
        x, y = ctx.saved_tensors
        # Q:777-789: both gradients through the same quantized matmul, with the
        # raw inputs transposed in f32 and quantized along the transposed axis
        g_x = _fp8_matmul_value(g, _quantized_transpose(y, ctx.tgrid), ctx.tgrid) \
            if ctx.needs_input_grad[0] else None
        g_y = _fp8_matmul_value(_quantized_transpose(x, ctx.tgrid), g, ctx.tgrid) \
            if ctx.needs_input_grad[1] else None
        return g_x, g_y, None


def fp8_matmul(x_f32, y_f32, tgrid=(1, 16)):
    """End-to-end differentiable FP8 matrix multiplication (Q:766-793)."""
    return _FP8Matmul.apply(x_f32, y_f32, tuple(tgrid))
