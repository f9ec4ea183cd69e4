"""qx (mirror of pratchya/_qualia/_qual.py): name resolution, keyword
translation and the unquantized-argument path run on the CPU; the quantized
path (dequantize -> torch op -> requantize with the gcd-adapted grid) is
checked on the GPU bit-exactly against the oracle's quantizer applied to the
same torch op of the kernel-dequantized values."""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O


def _qx():
    from pratchya_amd import qx
    return qx


def test_resolution_order_and_aliases():
    qx = _qx()
    assert qx._resolve("tanh") is torch.tanh                 # torch first
    assert qx._resolve("silu") is torch.nn.functional.silu   # then torch.nn.functional
    assert qx._resolve("erfcx") is torch.special.erfcx       # then torch.special
    assert qx._resolve("concatenate") is torch.cat           # jnp spelling
    with pytest.raises(AttributeError):
        qx.definitely_not_a_function


def test_keyword_translation():
    qx = _qx()
    assert qx._translate_kwargs("sum", {"axis": 1, "keepdims": True}) == {"dim": 1, "keepdim": True}
    assert qx._translate_kwargs("softmax", {}) == {"dim": -1}
    assert qx._translate_kwargs("softmax", {"axis": 0}) == {"dim": 0}


def test_unquantized_arguments_wrap_unquantized():
    """Without a quantized argument every result is QArrayImpl(r, quant=False)
    (_qual.py:52-55), tuples element by element."""
    qx = _qx()
    x = torch.tensor([[-1.0, 2.0], [3.0, -4.0]])
    r = qx.relu(x)
    assert not hasattr(r, "_QArrayImpl__tgrid")
    assert torch.equal(r.get_value(), torch.relu(x))
    s = qx.sum(x, axis=0, keepdims=True)
    assert torch.equal(s.get_value(), x.sum(dim=0, keepdim=True))
    parts = qx.split(x, 1, axis=1)
    assert isinstance(parts, tuple) and len(parts) == 2
    assert all(not hasattr(p, "_QArrayImpl__tgrid") for p in parts)
    # an unquantized QArrayImpl argument is unwrapped to its value
    r2 = qx.abs(r)
    assert torch.equal(r2.get_value(), torch.relu(x))


@pytest.mark.gpu
def test_quantized_argument_requantized_bit_exact():
    from pratchya_amd import qarr as Q
    from pratchya_amd import _kernels as K
    from tests.helpers import assert_bytes_equal, assert_f32_bits_equal, assert_payload_equal, f32, u8
    qx = _qx()
    x = np.random.default_rng(3).standard_normal((256, 512)).astype(np.float32)
    q = Q.QArrayImpl(torch.from_numpy(x).cuda(), (1, 128))
    out = qx.silu(q)
    deq = K.dequantize(*q._tree_flatten()[0], torch.float32, (1, 128))
    want = O.quantize_impl(torch.nn.functional.silu(deq).cpu().numpy(), (1, 128))
    got = [t for t in out._tree_flatten()[0]]
    assert out.tgrid == (1, 128)
    assert_payload_equal(u8(got[0]), want[0], "qx.silu payload")
    assert_bytes_equal(u8(got[1]), want[1], "qx.silu e8m0")
    assert_f32_bits_equal(f32(got[2]), want[2], "qx.silu G")


@pytest.mark.gpu
def test_quantized_argument_shape_change_and_tuple():
    from pratchya_amd import qarr as Q
    qx = _qx()
    x = torch.randn((256, 512), device="cuda")
    q = Q.QArrayImpl(x, (1, 128))
    s = qx.sum(q, axis=-1)                              # shape changes: unquantized
    assert not hasattr(s, "_QArrayImpl__tgrid") and tuple(s.shape) == (256,)
    halves = qx.split(q, 256, axis=1)                   # tuple; same-shape elements only requantized
    assert len(halves) == 2 and all(not hasattr(h, "_QArrayImpl__tgrid") for h in halves)
    both = qx.sort(q, axis=-1)                          # (values, indices): both keep the shape
    assert all(hasattr(b, "_QArrayImpl__tgrid") for b in both)


@pytest.mark.gpu
def test_gradient_flows_through_qx():
    from pratchya_amd import qarr as Q
    qx = _qx()
    x = torch.randn((128, 256), device="cuda", requires_grad=True)
    y = qx.square(Q.QArrayImpl(x, (1, 128)))
    y.astype(torch.float32).sum().backward()
    assert x.grad is not None and x.grad.shape == x.shape
    # d/dx sum(requant(dequant(x)^2)): the cotangent 1 dequantized-bwd'ed, doubled, requantized
    assert torch.isfinite(x.grad).all()
