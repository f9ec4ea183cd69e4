"""Checkpoint format of quantized-array trees (pratchya_amd.checkpoint): the
pytree children of every QArrayImpl leaf (pratchya/_qualia/_qarr.py:404-425)
round-trip byte for byte through a safetensors file, with the tree structure
and each leaf's tgrid.  The CPU test builds the arrays from oracle-quantized
bytes (no GPU); the GPU test quantizes on the device."""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O


def _qarray_from_oracle(x, tgrid, device="cpu"):
    from pratchya_amd.qarr import QArrayImpl
    v, s8, s32 = O.quantize_impl(x, tgrid)
    return QArrayImpl._tree_unflatten((True, tgrid), (
        torch.from_numpy(v).to(device).view(torch.float8_e4m3fn),
        torch.from_numpy(s8).to(device).view(torch.float8_e8m0fnu),
        torch.from_numpy(s32).to(device)))


def _assert_same_qarray(a, b):
    (av, as8, as32), (aq, ag) = a._tree_flatten()
    (bv, bs8, bs32), (bq, bg) = b._tree_flatten()
    assert aq and bq and tuple(ag) == tuple(bg)
    for x, y in ((av, bv), (as8, bs8), (as32, bs32)):
        assert x.dtype == y.dtype and tuple(x.shape) == tuple(y.shape)
        assert torch.equal(x.cpu().contiguous().view(torch.uint8), y.cpu().contiguous().view(torch.uint8))


def test_round_trip_on_cpu(tmp_path):
    from pratchya_amd.checkpoint import load_tree, save_tree
    from pratchya_amd.qarr import QArrayImpl
    rng = np.random.default_rng(12)
    w = _qarray_from_oracle(rng.standard_normal((256, 384)).astype(np.float32), (128, 128))
    x = _qarray_from_oracle(rng.standard_normal((2, 64, 256)).astype(np.float32) * 50, (1, 128))
    raw = QArrayImpl(torch.arange(6.0), quant=False)
    tree = {"blocks": {"w_r": w, "act": [x, torch.ones(3, dtype=torch.bfloat16)]}, "raw": raw, "step": 7,
            "name": "layer0", "tup": (1.5, None)}
    path = tmp_path / "ckpt.safetensors"
    save_tree(path, tree)
    back = load_tree(path, device="cpu")
    assert set(back) == set(tree) and back["step"] == 7 and back["name"] == "layer0" and back["tup"] == (1.5, None)
    _assert_same_qarray(back["blocks"]["w_r"], w)
    _assert_same_qarray(back["blocks"]["act"][0], x)
    assert torch.equal(back["blocks"]["act"][1], tree["blocks"]["act"][1])
    assert torch.equal(back["raw"].get_value(), raw.get_value())


def test_rejects_foreign_files(tmp_path):
    from safetensors.torch import save_file
    from pratchya_amd.checkpoint import load_tree
    path = tmp_path / "other.safetensors"
    save_file({"a": torch.zeros(2)}, str(path))
    with pytest.raises(ValueError, match="not a pratchya tree"):
        load_tree(path, device="cpu")


@pytest.mark.gpu
def test_round_trip_on_gpu(tmp_path):
    from pratchya_amd.checkpoint import load_tree, save_tree
    from pratchya_amd.qarr import QArrayImpl
    gen = torch.Generator(device="cuda").manual_seed(13)
    w = QArrayImpl(torch.randn((512, 256), generator=gen, device="cuda") * 0.02, (128, 128))
    m = QArrayImpl(torch.randn((1, 256, 512), generator=gen, device="cuda"), (128, 128))
    path = tmp_path / "gpu.safetensors"
    save_tree(path, {"w": w, "momentum": m})
    back = load_tree(path, device="cuda")
    _assert_same_qarray(back["w"], w)
    _assert_same_qarray(back["momentum"], m)
    assert back["w"]._tree_flatten()[0][0].is_cuda
    assert torch.equal(back["w"].dequantize(torch.float32), w.dequantize(torch.float32))
