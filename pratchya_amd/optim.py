"""Miulion, pratchya's quantized-momentum optimizer
(``pratchya/_nnx_impl/_optimizer.py:11-217``), for a PyTorch host on gfx950.

``miulion_optimizer(hyperparams, scheduler)`` returns a
``GradientTransformation(init, update)`` with optax's calling convention
(``_optimizer.py:62-217``): ``init(params)`` builds the momentum tree and
``update(updates, state, params)`` returns ``(updates, new_state)``.  Trees are
nested dicts / lists / tuples (``torch.utils._pytree``) whose leaves are
``QArrayImpl`` or tensors, like the reference's parameter trees.

Per quantized leaf the step is
  * the momentum pass on the GPU (``pratchya_momentum``): ``c`` and the new
    momentum from the quantized momentum and gradient in one kernel, the new
    momentum requantized with the parameter's block grid;
  * Muon for 2-D slices not named ``embed_tokens`` / ``lm_head``:
    ``newton_schulz(c)`` (5 iterations of two GEMMs on the hand-written MFMA
    kernel: bf16 directly, f32 over exact bf16 pieces), scaled by
    ``sqrt(max(N, M))``; Lion
    otherwise: ``sign(c)``;
  * the update pass on the GPU (``pratchya_apply_update``):
    ``-(lr * u + lr * wd * p)`` with the quantized parameter dequantized in
    registers.
A 3-D (layer-stacked) quantized leaf runs per layer in bf16 and returns a bf16
update (``_optimizer.py:117-145``); a 2-D one runs in f32 and returns an f32
update (``_optimizer.py:153-199``).  Unquantized leaves follow the same
formulas with torch operations.

Arithmetic follows the reference's dtype flow: Python-float constants take the
array's dtype (``beta1 * m`` is a bf16 product for a bf16 ``m``); the learning
rates are f32 values (optax schedules of the int32 step count), so the update
products are f32.
"""
from __future__ import annotations

import dataclasses
import math
from typing import Any, Callable, NamedTuple

import numpy as np
import torch
import torch.utils._pytree as pytree

from . import _kernels as K
from .qarr import QArrayImpl

__all__ = [
    "newton_schulz", "MiulionState", "MiulionHyperParams", "MiulionScheduler", "GradientTransformation",
    "miulion_optimizer",
]


def newton_schulz(G: torch.Tensor, steps: int = 5) -> torch.Tensor:
    """Orthogonalization by the cubic Newton-Schulz iteration
    (``_optimizer.py:11-29``): ``X = G / (||G||_F + 1e-7)`` (the transpose of a
    tall ``G``), then ``steps`` times ``X = 1.5 X - 0.5 (X X^T) X``, in ``G``'s
    dtype (bf16 for layer-stacked leaves, f32 for 2-D leaves, the two dtypes
    the optimizer passes; others are a ``TypeError``).  Everything runs on the
    hand-written kernels: the normalization on ``pratchya_ns_normalize``;
    bf16 products on the bf16 MFMA kernel (``pratchya_gemm_bf16_gram`` for
    the symmetric product where its side is a multiple of 256,
    ``pratchya_gemm_bf16_nt`` otherwise, ``pratchya_gemm_bf16_nt_ns`` for the
    second product with the combination in its epilogue); f32 products on the
    same kernel over exact bf16 pieces (``_kernels.matmul_f32``, f32
    accuracy) with ``pratchya_ns_combine``."""
    if G.dim() != 2:
        raise ValueError(f"newton_schulz: a 2-D array is required, got shape {tuple(G.shape)}")
    if G.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"newton_schulz: bfloat16 or float32 expected, got {G.dtype}")
    m, n = (int(d) for d in G.shape)
    transpose = m > n
    X = K.ns_normalize(G)                        # one fused two-pass kernel pair
    if m == 0 or n == 0:
        return X
    if X.dtype == torch.float32:
        # A tall G is iterated untransposed: with Y = X^T, X X^T = Y^T Y and
        # ((X X^T) X)^T = Y (Y^T Y), so Y <- 1.5 Y - 0.5 Y (Y^T Y) is the
        # transposed iteration without the transposes.
        for _ in range(steps):
            if transpose:
                A = K.matmul_f32(X, X, a_t=True)      # X^T X   [n, n]
                B = K.matmul_f32(X, A)                # X A     [m, n]
            else:
                A = K.matmul_f32(X, X, b_t=True)      # X X^T   [m, m]
                B = K.matmul_f32(A, X)                # A X     [m, n]
            X = K.ns_combine(X, B, out=X)
        return X
    # bf16: the kernel takes sides that are multiples of 64, so the iterate
    # is zero-padded to them; the pad rows and columns stay exactly zero
    # through every product and combination, and the products over the
    # original block are sums of the same bf16 products (plus exact zeros)
    mp, npad = -(-m // 64) * 64, -(-n // 64) * 64
    padded = (mp, npad) != (m, n)
    if padded:
        Xp = torch.zeros((mp, npad), dtype=X.dtype, device=X.device)
        Xp[:m, :n] = X
        X = Xp
    # the Gram product computes only its upper-triangle tiles (exactly
    # symmetric result) where its side is a multiple of 256; a tall iterate
    # is read K-major by it, with no transposed copy
    gram_side = npad if transpose else mp
    gram_ok = gram_side % 256 == 0
    for _ in range(steps):
        # the second product's epilogue also forms 1.5 X - 0.5 B (the bits
        # of ns_combine), into a new buffer
        if transpose:
            if gram_ok:
                A = K.gemm_bf16_gram(X, k_major=True)    # X^T X     [n, n]
            else:
                Xt = K.transpose_b16(X)                  # [n, m]
                A = K.gemm_bf16_nt(Xt, Xt)
            X = K.gemm_bf16_nt_ns(X, A, X)           # 1.5 X - 0.5 X A (A = A^T)
        else:
            A = K.gemm_bf16_gram(X) if gram_ok else K.gemm_bf16_nt(X, X)   # X X^T [m, m]
            # 1.5 X - 0.5 A X: a wide X is read K-major (no transposed copy);
            # for a square one the copy is cheaper than the K-major read
            # (measured: [4096, 4096] 1.08 vs 1.13 ms, [4096, 16384] 3.83 vs
            # 3.74 ms for 5 iterations)
            if npad > mp:
                X = K.gemm_bf16_nt_ns(A, X, X, b_k_major=True)
            else:
                X = K.gemm_bf16_nt_ns(A, K.transpose_b16(X), X)
    return X[:m, :n].contiguous() if padded else X


class MiulionState(NamedTuple):
    count: torch.Tensor          # int32 scalar
    momentum: Any


@dataclasses.dataclass
class MiulionHyperParams:
    lion_lr: float = 3e-4
    muon_lr: float = 0.02
    weight_decay: float = 0.1
    warmup_steps: int = 1000
    total_steps: int = 100000
    beta1: float = 0.9
    beta2: float = 0.99
    blksize: int = 128
    ns_steps: int = 5
    dtype: torch.dtype = torch.bfloat16


@dataclasses.dataclass
class MiulionScheduler:
    """Learning-rate schedules: callables of the step count (``_optimizer.py:47-58``)."""
    muon_schedule: Callable[[Any], Any]
    lion_schedule: Callable[[Any], Any]
    weight_decay: float

    def get_hyperparams(self, step):
        current_lion_lr = self.lion_schedule(step)
        current_muon_lr = self.muon_schedule(step)
        return current_lion_lr, current_muon_lr, self.weight_decay


class GradientTransformation(NamedTuple):
    init: Callable
    update: Callable


def _is_q(x) -> bool:
    return isinstance(x, QArrayImpl)


def _is_quantized(x) -> bool:
    return isinstance(x, QArrayImpl) and hasattr(x, "_QArrayImpl__tgrid")


def _triple(q: QArrayImpl):
    return q._tree_flatten()[0]


def _f32(x: float) -> float:
    return float(np.float32(x))


def _bf16(x: float) -> float:
    return float(torch.tensor(_f32(x), dtype=torch.float32).to(torch.bfloat16).float().item())


def _as_dtype(x: float, dtype: torch.dtype) -> float:
    """A Python-float constant converted to the array dtype it meets."""
    return _bf16(x) if dtype == torch.bfloat16 else _f32(x)


def _lr(v) -> float:
    """A schedule value as the f32 it is in the reference."""
    return _f32(float(v.item() if torch.is_tensor(v) else v))


def _should_use_muon(path, ndim: int) -> bool:
    """``_optimizer.py:96-109``: 2-D leaves whose key path names neither
    ``embed_tokens`` nor ``lm_head``."""
    if ndim != 2:
        return False
    path_str = "".join(str(p) for p in path).lower()
    return not any(k in path_str for k in ("embed_tokens", "lm_head"))


def _zero_momentum(p: QArrayImpl) -> QArrayImpl:
    """The quantized zero momentum of a quantized parameter: zero payload, e8m0
    bytes 0x00 (``FP8E8M0_MIN``, ``_optimizer.py:70-73``), zero group maxima."""
    x8, s8, s32 = _triple(p)
    z8 = torch.zeros_like(x8.view(torch.uint8)).view(x8.dtype)
    zs8 = torch.zeros_like(s8.view(torch.uint8)).view(s8.dtype)
    return QArrayImpl._tree_unflatten((True, p.tgrid), (z8, zs8, torch.zeros_like(s32)))


def _blocked_momentum(m: torch.Tensor, g: torch.Tensor, beta1: float, beta2: float):
    """``c`` and the new momentum for a gradient whose shape differs from the
    momentum's (``_optimizer.py:137-143``, :170-181): g is flattened, padded to
    the momentum's size and reshaped; c is cut back to g's shape."""
    flat_g = g.reshape(-1)
    pad = m.numel() - g.numel()
    if pad > 0:
        flat_g = torch.nn.functional.pad(flat_g, (0, pad))
    g_blocked = flat_g.reshape(m.shape)
    c_blocked, new_m = _momentum_torch(m, g_blocked, beta1, beta2)
    return c_blocked.reshape(-1)[:g.numel()].reshape(g.shape), new_m


def _momentum_torch(m: torch.Tensor, g: torch.Tensor, beta1: float, beta2: float):
    """``beta1*m + (1-beta1)*g`` and ``beta2*m + (1-beta2)*g`` with each
    Python-float constant rounded to the dtype of the array it multiplies
    (JAX's weak typing; torch would multiply by the f32 constant)."""
    c = _as_dtype(beta1, m.dtype) * m + _as_dtype(1.0 - beta1, g.dtype) * g
    new_m = _as_dtype(beta2, m.dtype) * m + _as_dtype(1.0 - beta2, g.dtype) * g
    return c, new_m


def _quantized_slice_step(path, g, m_t, p_t, tgrid, dtype, beta1, beta2, ns_steps, lion_lr, muon_lr, wd,
                          out_dtype):
    """One quantized 2-D slice in the leaf dtype ``dtype``: returns (update,
    new momentum triple).  ``g``: a triple or a tensor of the slice's shape."""
    shape = tuple(m_t[0].shape)
    g_shape = tuple(g[0].shape) if isinstance(g, tuple) else tuple(g.shape)
    if g_shape == shape:
        c, nm = K.momentum(m_t, g, tgrid, dtype, _as_dtype(beta1, dtype), _as_dtype(1.0 - beta1, dtype),
                           _as_dtype(beta2, dtype), _as_dtype(1.0 - beta2, dtype))
    else:
        mv = K.dequantize(*m_t, dtype, tgrid)
        gv = K.dequantize(*g, dtype, tgrid) if isinstance(g, tuple) else g.to(dtype)
        c, nm = _blocked_momentum(mv, gv, beta1, beta2)
    new_m = K.quantize(nm, tgrid)
    if _should_use_muon(path, len(g_shape)):
        u = newton_schulz(c, steps=ns_steps)
        scale = _as_dtype(math.sqrt(max(g_shape[0], g_shape[1])), dtype)
        lr = muon_lr
        upd = K.apply_update(u, False, scale, p_t, tgrid, dtype, lr, _f32(lr * np.float32(wd)), out_dtype)
    else:
        lr = lion_lr
        upd = K.apply_update(c, True, 0.0, p_t, tgrid, dtype, lr, _f32(lr * np.float32(wd)), out_dtype)
    return upd, new_m


def miulion_optimizer(hyperparams: MiulionHyperParams, scheduler: MiulionScheduler) -> GradientTransformation:
    """The quantized Miulion transformation (``_optimizer.py:62-217``)."""
    beta1 = hyperparams.beta1
    beta2 = hyperparams.beta2
    ns_steps = hyperparams.ns_steps

    def init_fn(params):
        def make_momentum_leaf(p):
            if _is_quantized(p):
                return _zero_momentum(p)
            if isinstance(p, QArrayImpl):
                p = p.get_value()
            if torch.is_floating_point(p):
                return torch.zeros_like(p, dtype=torch.float32)
            return torch.zeros_like(p)

        momentum = pytree.tree_map(make_momentum_leaf, params, is_leaf=_is_q)
        dev = next((l.get_value().device if _is_q(l) else l.device
                    for l in pytree.tree_leaves(params, is_leaf=_is_q)), None)
        return MiulionState(count=torch.zeros([], dtype=torch.int32, device=dev), momentum=momentum)

    def update_fn(updates, state: MiulionState, params=None):
        if params is None:
            raise ValueError("Miulion Optimizer requires 'params' to perform Weight Decay and precision mapping.")
        lion_lr, muon_lr, weight_decay = scheduler.get_hyperparams(state.count)
        lion_lr, muon_lr = _lr(lion_lr), _lr(muon_lr)
        wd = float(weight_decay)

        def update_leaf(path, g, m, param):
            if _is_quantized(param) and param.get_value().dim() == 3:
                # layer-stacked leaf: per layer in bf16 (_optimizer.py:117-145)
                tgrid = param.tgrid
                p8, ps8, ps32 = _triple(param)
                m8, ms8, ms32 = _triple(m)
                gq = _is_quantized(g)
                if gq:
                    g8, gs8, gs32 = _triple(g)
                else:
                    gv = g.get_value() if _is_q(g) else g
                ups, n8, ns8, ns32 = [], [], [], []
                for l in range(p8.shape[0]):
                    g_l = (g8[l], gs8[l], gs32[l]) if gq else gv[l].to(torch.bfloat16)
                    upd, (x8, s8, s32) = _quantized_slice_step(
                        path, g_l, (m8[l], ms8[l], ms32[l]), (p8[l], ps8[l], ps32[l]), tgrid, torch.bfloat16,
                        beta1, beta2, ns_steps, lion_lr, muon_lr, wd, torch.bfloat16)
                    ups.append(upd)
                    n8.append(x8)
                    ns8.append(s8)
                    ns32.append(s32)
                new_m = QArrayImpl._tree_unflatten(
                    (True, tgrid), (torch.stack(n8), torch.stack(ns8), torch.stack(ns32)))
                return torch.stack(ups), new_m

            if _is_quantized(param):
                # quantized leaf in f32 (_optimizer.py:155-199)
                tgrid = param.tgrid
                g_in = _triple(g) if _is_quantized(g) else (g.get_value() if _is_q(g) else g).float()
                upd, (x8, s8, s32) = _quantized_slice_step(
                    path, g_in, _triple(m), _triple(param), tgrid, torch.float32, beta1, beta2, ns_steps,
                    lion_lr, muon_lr, wd, torch.float32) if param.get_value().dim() == 2 else \
                    _quantized_nd_step(path, g_in, m, param, beta1, beta2, lion_lr, wd)
                return upd, QArrayImpl._tree_unflatten((True, tgrid), (x8, s8, s32))

            # unquantized parameter (_optimizer.py:162-199 without requantization)
            p = param.get_value() if _is_q(param) else param
            if _is_quantized(m):
                mv = m.astype(torch.bfloat16)
                gv = (g.astype(torch.bfloat16) if _is_q(g) else g.to(torch.bfloat16))
            else:
                mv = m
                gv = g.get_value() if _is_q(g) else g
            if tuple(mv.shape) == tuple(gv.shape):
                c, new_m = _momentum_torch(mv, gv, beta1, beta2)
            else:
                c, new_m = _blocked_momentum(mv, gv, beta1, beta2)
            lr = muon_lr if _should_use_muon(path, gv.dim()) else lion_lr
            if _should_use_muon(path, gv.dim()):
                u = newton_schulz(c, steps=ns_steps)
                u = u * _as_dtype(math.sqrt(max(gv.shape[0], gv.shape[1])), u.dtype)
            else:
                u = torch.sign(c)
            lr_wd = _f32(lr * np.float32(wd))
            update = -(u.float() * lr + p.float() * lr_wd)
            return update, new_m

        leaves_u, spec = pytree.tree_flatten_with_path(updates, is_leaf=_is_q)
        leaves_m = pytree.tree_leaves(state.momentum, is_leaf=_is_q)
        leaves_p = pytree.tree_leaves(params, is_leaf=_is_q)
        if not (len(leaves_u) == len(leaves_m) == len(leaves_p)):
            raise ValueError("updates, momentum and params must have the same tree structure")
        results = [update_leaf(path, g, m, p) for (path, g), m, p in zip(leaves_u, leaves_m, leaves_p)]
        new_updates = pytree.tree_unflatten([r[0] for r in results], spec)
        new_m = pytree.tree_unflatten([r[1] for r in results], spec)
        return new_updates, MiulionState(count=state.count + 1, momentum=new_m)

    return GradientTransformation(init_fn, update_fn)


def _quantized_nd_step(path, g_in, m: QArrayImpl, param: QArrayImpl, beta1, beta2, lion_lr, wd):
    """A quantized leaf that is neither 2-D nor 3-D (1-D, or 4-D and more): f32
    Lion step (``_optimizer.py:155-199`` with ``ndim != 2``)."""
    tgrid = param.tgrid
    c, nm = K.momentum(_triple(m), g_in, tgrid, torch.float32, _f32(beta1), _f32(1.0 - beta1),
                       _f32(beta2), _f32(1.0 - beta2))
    new_m = K.quantize(nm, tgrid)
    upd = K.apply_update(c, True, 0.0, _triple(param), tgrid, torch.float32, lion_lr,
                         _f32(lion_lr * np.float32(wd)), torch.float32)
    return upd, new_m
