"""Checkpoint format of trees with quantized-array leaves.

A quantized array is stored as its pytree children (pratchya/_qualia/_qarr.py:
404-425): the e4m3fn payload, the e8m0 block scales and the f32 group maxima,
byte for byte, with its tgrid as the auxiliary data.  That is the state a
JAX checkpointer writes for the reference's QArrayImpl leaves; here it goes
into one safetensors file (no pickling), with the tree structure and each
leaf's kind and tgrid in the file's metadata.  Loading rebuilds the same
tree with QArrayImpl leaves whose bytes equal the saved ones.
"""
from __future__ import annotations

import json
from typing import Any

import torch
import torch.utils._pytree as pytree
from safetensors import safe_open
from safetensors.torch import load_file, save_file

from .qarr import E4M3, QArrayImpl

E8M0 = torch.float8_e8m0fnu
_META = "pratchya_tree"


def _is_qarray(x) -> bool:
    return isinstance(x, QArrayImpl)


def _bytes(t: torch.Tensor) -> torch.Tensor:
    """A 1-byte tensor's storage as uint8 on the host (same shape)."""
    t = t.detach().contiguous()
    return (t.view(torch.uint8) if t.dtype != torch.uint8 else t).cpu()


def save_tree(path, tree: Any) -> None:
    """Write ``tree`` (dicts / lists / tuples of QArrayImpl, tensors and JSON
    values) to the safetensors file ``path``."""
    leaves, spec = pytree.tree_flatten(tree, is_leaf=_is_qarray)
    tensors, info = {}, []
    for i, leaf in enumerate(leaves):
        if isinstance(leaf, QArrayImpl):
            children, (is_quant, tgrid) = leaf._tree_flatten()
            if is_quant:
                value, sc8, sc32 = children
                tensors[f"{i}.value"] = _bytes(value)
                tensors[f"{i}.sc_fp8"] = _bytes(sc8)
                tensors[f"{i}.sc_fp32"] = sc32.detach().contiguous().float().cpu()
                info.append({"kind": "qarray", "tgrid": [int(tgrid[0]), int(tgrid[1])]})
            else:
                tensors[f"{i}.value"] = children[0].detach().contiguous().cpu()
                info.append({"kind": "qarray_raw"})
        elif torch.is_tensor(leaf):
            tensors[str(i)] = leaf.detach().contiguous().cpu()
            info.append({"kind": "tensor"})
        else:
            json.dumps(leaf)                     # raises for values the format cannot hold
            info.append({"kind": "value", "value": leaf})
    meta = {_META: json.dumps({"spec": pytree.treespec_dumps(spec), "leaves": info})}
    save_file(tensors, str(path), metadata=meta)


def load_tree(path, device: str = "cuda") -> Any:
    """Read a file written by ``save_tree``; tensors go to ``device``."""
    with safe_open(str(path), framework="pt") as f:
        meta = f.metadata() or {}
    if _META not in meta:
        raise ValueError(f"{path}: not a pratchya tree checkpoint")
    desc = json.loads(meta[_META])
    tensors = load_file(str(path))
    leaves = []
    for i, inf in enumerate(desc["leaves"]):
        kind = inf["kind"]
        if kind == "qarray":
            value = tensors[f"{i}.value"].to(device).view(E4M3)
            sc8 = tensors[f"{i}.sc_fp8"].to(device).view(E8M0)
            sc32 = tensors[f"{i}.sc_fp32"].to(device)
            leaves.append(QArrayImpl._tree_unflatten((True, tuple(inf["tgrid"])), (value, sc8, sc32)))
        elif kind == "qarray_raw":
            leaves.append(QArrayImpl._tree_unflatten((False, None), (tensors[f"{i}.value"].to(device),)))
        elif kind == "tensor":
            leaves.append(tensors[str(i)].to(device))
        else:
            leaves.append(inf["value"])
    return pytree.tree_unflatten(leaves, pytree.treespec_loads(desc["spec"]))
