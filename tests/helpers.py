"""Shared helpers of the GPU parity tests (host <-> device conversions)."""
import numpy as np
import torch

from oracle import qarr_oracle as O


def to_dev_bf16(bits: np.ndarray) -> torch.Tensor:
    """bf16 bit patterns (uint16 ndarray) -> bfloat16 CUDA tensor (shape kept, 0-d included)."""
    arr = np.array(bits, dtype=np.uint16, copy=True, order="C")
    return torch.from_numpy(arr.view(np.int16)).view(torch.bfloat16).reshape(arr.shape).cuda()


def to_dev_f32(x: np.ndarray) -> torch.Tensor:
    arr = np.array(x, dtype=np.float32, copy=True, order="C")
    return torch.from_numpy(arr).reshape(arr.shape).cuda()


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().view(torch.uint8).cpu().numpy()


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_bytes_equal(got: np.ndarray, want: np.ndarray, what: str) -> None:
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    bad = np.nonzero(got.reshape(-1) != want.reshape(-1))[0]
    if bad.size:
        i = bad[:8]
        raise AssertionError(f"{what}: {bad.size} of {got.size} differ; first at {i.tolist()}: "
                             f"got {got.reshape(-1)[i].tolist()} want {want.reshape(-1)[i].tolist()}")


def assert_f32_bits_equal(got: np.ndarray, want: np.ndarray, what: str) -> None:
    got = np.ascontiguousarray(got, dtype=np.float32)
    want = np.ascontiguousarray(want, dtype=np.float32)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    assert_bytes_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32), what)


def assert_payload_equal(got: np.ndarray, want: np.ndarray, what: str) -> None:
    """Payload bytes equal; a NaN byte's sign (0x7F vs 0xFF) is not pinned by
    the reference (XLA's NaN propagation) and is compared as NaN-ness only."""
    got = np.asarray(got).copy()
    want = np.asarray(want).copy()
    gnan = (got & 0x7F) == 0x7F
    wnan = (want & 0x7F) == 0x7F
    assert np.array_equal(gnan, wnan), f"{what}: NaN payload positions differ"
    got[gnan] = 0x7F
    want[wnan] = 0x7F
    assert_bytes_equal(got, want, what)


def oracle_quant(x_f32: np.ndarray, tgrid):
    return O.quantize_impl(x_f32, tgrid)
