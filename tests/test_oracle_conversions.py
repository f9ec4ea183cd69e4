"""Pin the oracle's two rounding steps against torch's CPU casts.

pratchya/_qualia/_qarr.py:499 rounds f32 -> bf16 -> float8_e4m3fn.  torch's
CPU casts implement the same IEEE/OCP conversions (RNE, non-saturating e4m3fn),
so the oracle must agree with them on every bf16 pattern and on random and
edge f32 patterns.
"""
import numpy as np
import torch

from oracle import qarr_oracle as O


def test_bf16_to_e4m3fn_exhaustive():
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = O.bf16_bits_to_e4m3fn(b)
    ref = (torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
           .to(torch.float8_e4m3fn).view(torch.uint8).numpy())
    assert np.array_equal(ours, ref)


def test_bf16_to_e4m3fn_known_answers():
    f = lambda v: int(O.bf16_bits_to_e4m3fn(O.f32_to_bf16_bits(np.array([v], np.float32)))[0])
    assert f(448.0) == 0x7E
    assert f(464.0) == 0x7E          # tie rounds to even (448)
    assert f(466.0) == 0x7F          # above the tie: NaN (non-saturating)
    assert f(-466.0) == 0xFF
    assert f(2.0 ** -9) == 0x01      # smallest subnormal
    assert f(2.0 ** -10) == 0x00     # tie to even -> 0
    assert f(-0.0) == 0x80
    assert f(float("inf")) == 0x7F
    assert f(float("nan")) == 0x7F
    assert f(1.0) == 0x38
    assert f(256.0) == 0x78


def test_double_rounding_differs_from_single():
    v = np.float32(1.0625 + 2.0 ** -20)
    via_bf16 = O.bf16_bits_to_e4m3fn(O.f32_to_bf16_bits(np.array([v])))[0]
    direct = torch.tensor([v]).to(torch.float8_e4m3fn).view(torch.uint8).item()
    assert via_bf16 == 0x38 and direct == 0x39


def test_f32_to_bf16_random_and_edges():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    edges = np.array([0, 0x80000000, 0x00008000, 0x00018000, 0x3F808000, 0x3F818000, 0x7F7F8000,
                      0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x00000001, 0x807FFFFF, 0x3F80FFFF,
                      0x3F807FFF], dtype=np.uint32)
    u = np.concatenate([u, edges])
    x = u.view(np.float32)
    ours = O.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    # NaN stays NaN with its sign
    assert np.all((ours[nan] & 0x7FFF) > 0x7F80)
    assert np.array_equal(ours[nan] >> 15, (u[nan] >> 31).astype(np.uint16))


def test_e4m3fn_decode_all_bytes():
    q = np.arange(256, dtype=np.uint8)
    ours = O.e4m3fn_to_f32(q)
    ref = torch.from_numpy(q).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_e8m0_decode_bit_trick():
    e = np.arange(256, dtype=np.uint8)
    v = O.e8m0_to_f32(e)
    assert v[0] == 0.0                  # reference decodes 0x00 to 0.0 (not 2^-127)
    assert np.isinf(v[255])             # and 0xFF to +inf (not NaN)
    assert np.array_equal(v[1:255], np.exp2(np.arange(1, 255) - 127.0).astype(np.float32))
