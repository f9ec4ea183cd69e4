"""``qx``: any array function applied to quantized arrays, the mirror of
``pratchya/_qualia/_qual.py`` (exported as ``pratchya.qx``,
``pratchya/_qualia/__init__.py:2``) for a PyTorch host.

``qx.<name>(*args, **kwargs)`` resolves ``<name>`` in ``torch``, then
``torch.nn.functional``, then ``torch.special`` (the reference looks in
``jnp``, ``jax.nn``, ``jax.lax``, ``_qual.py:9-16``), calls it on the
arguments with every ``QArrayImpl`` replaced by its f32 dequantization
(``_qual.py:22-30``), and wraps the result (``_qual.py:38-55``):

* with a quantized argument, a result of that argument's shape is requantized
  with its block grid adapted by gcd (``QArrayImpl._requantize``, ``Q:371-380``);
  any other result becomes an unquantized ``QArrayImpl(r, quant=False)``;
  tuple results are wrapped element by element;
* without one, every result is wrapped unquantized.

Functions keep torch's semantics; the reference's keyword names ``axis`` and
``keepdims`` are accepted for ``dim`` / ``keepdim``, and a few jnp names that
torch spells differently are mapped (``_ALIASES``).  Dequantization and
requantization run on the gfx950 kernels and carry the reference's vjps
(``qarr.dequantize_impl`` / ``qarr.quantize_impl``), so ``qx`` results
differentiate like the reference's.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .qarr import QArrayImpl

_NAMESPACES = (torch, F, torch.special)

# jnp / jax.nn / jax.lax names with a different torch spelling
_ALIASES = {
    "concatenate": torch.cat,
    "power": torch.pow,
    "absolute": torch.abs,
    "divide": torch.div,
    "multiply": torch.mul,
    "subtract": torch.sub,
    "negative": torch.neg,
    "log_sigmoid": F.logsigmoid,
    "swish": F.silu,
    "expand_dims": torch.unsqueeze,
}

# functions whose axis defaults to the last one in jax (jax.nn.softmax & co.)
_LAST_AXIS_DEFAULT = ("softmax", "log_softmax")


def _resolve(name: str):
    if name in _ALIASES:
        return _ALIASES[name]
    for ns in _NAMESPACES:
        fn = getattr(ns, name, None)
        if callable(fn):
            return fn
    raise AttributeError(f"module '{__name__}' has no attribute '{name}'")


def _translate_kwargs(name: str, kwargs: dict) -> dict:
    out = dict(kwargs)
    if "axis" in out:
        out["dim"] = out.pop("axis")
    if "keepdims" in out:
        out["keepdim"] = out.pop("keepdims")
    if name in _LAST_AXIS_DEFAULT and "dim" not in out:
        out["dim"] = -1
    return out


def _unwrap(v):
    if isinstance(v, QArrayImpl):
        return v.astype(torch.float32)       # __jax_array__'s role (_qual.py:24-29)
    return v


def _shape(r):
    return tuple(r.shape) if hasattr(r, "shape") else ()


def __getattr__(name: str):
    if name.startswith("__"):
        raise AttributeError(name)
    fn = _resolve(name)

    def wrapper(*args, **kwargs):
        result = fn(*[_unwrap(a) for a in args],
                    **_translate_kwargs(name, {k: _unwrap(v) for k, v in kwargs.items()}))
        quant_arg = next((a for a in args
                          if isinstance(a, QArrayImpl) and hasattr(a, "_QArrayImpl__tgrid")), None)
        if quant_arg is not None:
            if isinstance(result, (tuple, list)):
                return tuple(quant_arg._requantize(r) if _shape(r) == quant_arg.shape
                             else QArrayImpl(r, quant=False) for r in result)
            if _shape(result) == quant_arg.shape:
                return quant_arg._requantize(result)
            return QArrayImpl(result, quant=False)
        if isinstance(result, (tuple, list)):
            return tuple(QArrayImpl(r, quant=False) for r in result)
        return QArrayImpl(result, quant=False)

    wrapper.__name__ = name
    wrapper.__qualname__ = name
    wrapper.__doc__ = f"qx.{name}: {getattr(fn, '__module__', '')}.{getattr(fn, '__name__', name)} on dequantized arguments"
    return wrapper
