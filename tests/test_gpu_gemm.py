"""GPU parity of the block-scaled FP8 GEMM against the oracle's
dequant-then-matmul (pratchya/_qualia/_qarr.py:605-608, 621-622).

Tolerance (the GEMM contract): relative Frobenius error <= 1e-2 for bf16
outputs.  f32 outputs are held to 1e-3: the FP8 MFMA's internal dot-product
accumulation is not a sequence of IEEE f32 additions (deviations of 1e-5 to
1e-4 relative on heavy-tailed data), while its arithmetic is exact whenever the
sums are exactly representable -- ``test_exact_integer_products`` pins that
case bit for bit, so the kernel's indexing and scale handling are checked
exactly and only the hardware accumulation is inside the tolerance.
"""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O
from tests.helpers import f32, to_dev_bf16, to_dev_f32, u8

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
F32_TOL = 1e-3


def _K():
    from pratchya_amd import _kernels
    return _kernels


def quant_dev(bits_or_f32, tgrid, bf16=True):
    K = _K()
    dev = to_dev_bf16(bits_or_f32) if bf16 else to_dev_f32(bits_or_f32)
    return K.quantize(dev, tgrid)


def deq_host(x8, s8, s32, tgrid):
    return O.dequantize_impl(u8(x8), u8(s8), f32(s32), "float32", tgrid).astype(np.float64)


def check(C, ref, tol, what):
    err = O.rel_fro(f32(C), ref)
    assert err <= tol, f"{what}: relative Frobenius error {err:.3e} > {tol}"
    return err


@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_forward_small(out):
    """x (1,128) @ W (128,128): the quantized Linear forward (M:46-50)."""
    K = _K()
    M_, K_, N_ = 512, 2048, 1024
    x = O.activation_input(M_, K_, seed=2)
    w = O.normal_input((K_, N_), 0.02, seed=3)
    xa = quant_dev(x, (1, 128))
    wq = quant_dev(w, (128, 128))
    a = K.operand_rows(*xa, (1, 128))
    b = K.operand_transposed(*wq, (128, 128))
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    C = K.gemm_nt(a, b, dt)
    torch.cuda.synchronize()
    ref = deq_host(*xa, (1, 128)) @ deq_host(*wq, (128, 128))
    check(C, ref, BF16_TOL if out == "bf16" else F32_TOL, f"fwd {out}")


def test_exact_integer_products():
    """Small-integer data whose quantized payloads, products and K-sums are all
    exact in f32: the GEMM must reproduce the exact product bit for bit
    (forward layout with two K spans and a two-group weight, f32 out)."""
    K = _K()
    M_, K_, N_ = 256, 2048, 512
    rng = np.random.default_rng(21)
    x = rng.integers(-8, 9, size=(M_, K_)).astype(np.float32)
    x[:, ::128] = 8.0                     # every block max 8 -> S = G = 8, q = 16 x
    x[3, 1024:] *= 0.5                    # a span with G = 4 in one row
    x[5, 1024:2048] = 0.0                 # an all-zero span
    w = rng.integers(-4, 5, size=(K_, N_)).astype(np.float32)
    w[::128, ::128] = 4.0
    w[1024:] *= 2.0
    xq = quant_dev(x, (1, 128), bf16=False)
    wq = quant_dev(w, (128, 128), bf16=False)
    xd, wd = deq_host(*xq, (1, 128)), deq_host(*wq, (128, 128))
    assert np.array_equal(xd, x) and np.array_equal(wd, w)   # lossless quantization
    C = K.gemm_nt(K.operand_rows(*xq, (1, 128)), K.operand_transposed(*wq, (128, 128)), torch.float32)
    torch.cuda.synchronize()
    # multiples of 1/2 with sums far below 2^24: float64 (and f32) exact
    exact = (x.astype(np.float64) @ w.astype(np.float64)).astype(np.float32)
    assert np.array_equal(f32(C), exact)


def test_transpose_u8():
    K = _K()
    rng = np.random.default_rng(0)
    x = rng.integers(0, 256, size=(384, 640), dtype=np.uint8)
    t = K.transpose_u8(torch.from_numpy(x).cuda())
    assert np.array_equal(t.cpu().numpy(), x.T)


def test_transpose_u8_tall():
    """More than 65535 row tiles: the tile index runs on one grid axis."""
    K = _K()
    rows = 65600 * 64
    x = torch.randint(0, 256, (rows, 64), dtype=torch.uint8, device="cuda")
    t = K.transpose_u8(x)
    torch.cuda.synchronize()
    assert torch.equal(t, x.t().contiguous())


@pytest.mark.parametrize("shape", [(4096 + 16, 16384 - 48), (1040, 4048), (2032, 2064)],
                         ids=lambda s: "x".join(map(str, s)))
def test_transpose_u8_ragged_large(shape):
    """128x128 tiles (from 2^22 bytes) with partial tiles on both edges, and
    sizes just around the switch from 64x64 tiles."""
    K = _K()
    g = torch.Generator(device="cuda").manual_seed(sum(shape))
    x = torch.randint(0, 256, shape, dtype=torch.uint8, device="cuda", generator=g)
    t = K.transpose_u8(x)
    torch.cuda.synchronize()
    assert torch.equal(t, x.t().contiguous())


def test_dgrad_shape():
    """g (1,128) @ W^T: W [K_out, N] read as B rows without a transpose."""
    K = _K()
    M_, N_, Ko = 512, 1024, 768
    g = O.normal_input((M_, N_), 1e-3, seed=4)
    w = O.normal_input((Ko, N_), 0.02, seed=3)
    gq = quant_dev(g, (1, 128))
    wq = quant_dev(w, (128, 128))
    a = K.operand_rows(*gq, (1, 128))
    b = K.operand_rows(*wq, (128, 128))
    C = K.gemm_nt(a, b, torch.float32)
    torch.cuda.synchronize()
    ref = deq_host(*gq, (1, 128)) @ deq_host(*wq, (128, 128)).T
    check(C, ref, F32_TOL, "dgrad")


def test_dgrad_groups_straddling_block_rows():
    """W [1024, 768] (128,128): 16-block groups start mid block-row, so rows'
    group maxima change at different K blocks (span 2)."""
    K = _K()
    M_, N_, Ko = 512, 768, 1024
    g = O.normal_input((M_, N_), 1e-3, seed=14)
    w = O.normal_input((Ko, N_), 0.02, seed=15)
    w_f = O.bf16_bits_to_f32(w)
    w_f[256:384] *= np.float32(64.0)          # a group max that differs from its neighbours'
    wq = quant_dev(w_f, (128, 128), bf16=False)
    gq = quant_dev(g, (1, 128))
    C = K.gemm_nt(K.operand_rows(*gq, (1, 128)), K.operand_rows(*wq, (128, 128)), torch.float32)
    torch.cuda.synchronize()
    ref = deq_host(*gq, (1, 128)) @ deq_host(*wq, (128, 128)).T
    check(C, ref, F32_TOL, "dgrad straddling groups")


def test_forward_weight_groups_straddling_block_rows():
    """x (1,128) @ W [1024, 768] (128,128) used transposed: the weight's
    16-block groups give its columns group changes at K blocks 3, 5, 6, ...
    (span 1)."""
    K = _K()
    M_, K_, N_ = 512, 1024, 768
    x = O.activation_input(M_, K_, seed=16)
    w_f = O.bf16_bits_to_f32(O.normal_input((K_, N_), 0.02, seed=17))
    w_f[384:512, 256:384] *= np.float32(64.0)
    xq = quant_dev(x, (1, 128))
    wq = quant_dev(w_f, (128, 128), bf16=False)
    C = K.gemm_nt(K.operand_rows(*xq, (1, 128)), K.operand_transposed(*wq, (128, 128)), torch.float32)
    torch.cuda.synchronize()
    ref = deq_host(*xq, (1, 128)) @ deq_host(*wq, (128, 128))
    check(C, ref, F32_TOL, "fwd straddling groups")


def test_wgrad_token_axis_groups():
    """A^T dY with both operands quantized (128,1) along tokens: group maxima
    change every K block and every 8 rows/columns."""
    K = _K()
    T, Cin, N_ = 1024, 512, 768
    a = O.activation_input(T, Cin, seed=5)
    dy = O.normal_input((T, N_), 1e-3, seed=6)
    aq = quant_dev(a, (128, 1))
    dq = quant_dev(dy, (128, 1))
    A_ = K.operand_transposed(*aq, (128, 1))
    B_ = K.operand_transposed(*dq, (128, 1))
    C = K.gemm_nt(A_, B_, torch.float32)
    torch.cuda.synchronize()
    ref = deq_host(*aq, (128, 1)).T @ deq_host(*dq, (128, 1))
    check(C, ref, F32_TOL, "wgrad")


def test_wgrad_from_transposed_requantize():
    """The config-4 wgrad chain: the stored (1,128) activation requantized to
    (128,1) from its fp8 payload, dY requantized (128,1) from bf16, both with
    token-contiguous payloads from quantize_t128, then A^T dY in f32."""
    K = _K()
    T, Cin, N_ = 1024, 512, 768
    a_bits = O.activation_input(T, Cin, seed=5)
    dy_bits = O.normal_input((T, N_), 1e-3, seed=6)
    a8 = K.quantize(to_dev_bf16(a_bits), (1, 128))                 # the forward's stored operand
    at = K.quantize_t128(*a8)
    dt = K.quantize_t128(to_dev_bf16(dy_bits))
    C = K.gemm_nt(K.operand_t128(*at), K.operand_t128(*dt), torch.float32)
    torch.cuda.synchronize()
    a_deq = O.dequantize_impl(u8(a8[0]), u8(a8[1]), f32(a8[2]), "float32", (1, 128))
    aq = O.quantize_impl(a_deq, (128, 1))
    dq = O.quantize_impl(O.bf16_bits_to_f32(dy_bits), (128, 1))
    ref = (O.dequantize_impl(*aq, "float32", (128, 1)).astype(np.float64).T
           @ O.dequantize_impl(*dq, "float32", (128, 1)).astype(np.float64))
    check(C, ref, F32_TOL, "wgrad via quantize_t128")


@pytest.mark.parametrize("shape", [(1024, 512, 768), (2048, 256, 4096), (16384, 2048, 8192)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_wgrad_k_major_operands_same_bits(shape, out):
    """The wgrad operands read K-major ([T, C], quantize_impl's own layout for
    tgrid (128, 1)) through the LDS transposing loads: each MFMA lane sums the
    same K values as with the transposed payloads, so the product is the same
    bit for bit (span-1 rescales, per-row B group maxima, config 4's shape)."""
    K = _K()
    T, Cin, N_ = shape
    a8 = K.quantize(to_dev_bf16(O.activation_input(T, Cin, seed=5)), (1, 128))
    at = K.quantize_t128(*a8)
    dt = K.quantize_t128(to_dev_bf16(O.normal_input((T, N_), 1e-3, seed=6)))
    nt = K.gemm_nt(K.operand_t128(*at), K.operand_t128(*dt), out)
    km = K.gemm_nt(K.operand_k128(K.transpose_u8(at[0]), at[1], at[2]),
                   K.operand_k128(K.transpose_u8(dt[0]), dt[1], dt[2]), out)
    torch.cuda.synchronize()
    assert torch.equal(km.view(torch.uint8), nt.view(torch.uint8))


def test_per_column_b_groups_exact():
    """B quantized (1, 128) as rows: every output column has its own group
    maxima, which change between the two 1024-wide K spans differently per
    column (the per-row B units).  Lossless small-integer data: the product
    must be exact bit for bit."""
    K = _K()
    M_, K_, N_ = 256, 2048, 384
    rng = np.random.default_rng(41)
    x = rng.integers(-8, 9, size=(M_, K_)).astype(np.float32)
    x[:, ::128] = 8.0
    y = rng.integers(-4, 5, size=(N_, K_)).astype(np.float32)
    y[:, ::128] = 4.0
    y *= np.exp2(np.arange(N_) % 5 - 2.0).astype(np.float32)[:, None]     # G = 4 * 2^p per column
    y[1::2, 1024:] *= 2.0                                                 # odd columns: second span 2x
    y[7, :1024] = 0.0                                                     # an all-zero span
    xq = quant_dev(x, (1, 128), bf16=False)
    yq = quant_dev(y, (1, 128), bf16=False)
    assert np.array_equal(deq_host(*xq, (1, 128)), x) and np.array_equal(deq_host(*yq, (1, 128)), y)
    C = K.gemm_nt(K.operand_rows(*xq, (1, 128)), K.operand_rows(*yq, (1, 128)), torch.float32)
    torch.cuda.synchronize()
    exact = (x.astype(np.float64) @ y.astype(np.float64).T).astype(np.float32)
    assert np.array_equal(f32(C), exact)


@pytest.mark.parametrize("shape", [(512, 4096, 300), (300, 2048, 1028)], ids=lambda s: "x".join(map(str, s)))
def test_per_column_b_groups_heavy_tailed(shape):
    """Rows of both operands scaled over 2^-20 .. 2^20 (each row its own
    group maxima), an N that is not a multiple of 8 or 32, edge tiles."""
    K = _K()
    M_, K_, N_ = shape
    rng = np.random.default_rng(42)
    x = (rng.standard_normal((M_, K_)) * np.exp2(rng.integers(-20, 21, (M_, 1)))).astype(np.float32)
    y = (rng.standard_normal((N_, K_)) * np.exp2(rng.integers(-20, 21, (N_, 1)))).astype(np.float32)
    y[:, K_ // 2:] *= np.exp2(rng.integers(-6, 7, (N_, 1))).astype(np.float32)
    xq = quant_dev(x, (1, 128), bf16=False)
    yq = quant_dev(y, (1, 128), bf16=False)
    C = K.gemm_nt(K.operand_rows(*xq, (1, 128)), K.operand_rows(*yq, (1, 128)), torch.float32)
    torch.cuda.synchronize()
    ref = deq_host(*xq, (1, 128)) @ deq_host(*yq, (1, 128)).T
    # per-element relative check as well: columns span 2^40 in magnitude
    scale = np.abs(deq_host(*xq, (1, 128))).max(1)[:, None] * np.abs(deq_host(*yq, (1, 128))).max(1)[None, :]
    assert np.all(np.abs(f32(C) - ref) <= 1e-3 * scale * np.sqrt(K_))
    check(C, ref, F32_TOL, "per-column groups")


def test_b_groups_straddling_rows():
    """B [N, 512] quantized (1, 128): a group of 8 blocks covers two rows, so
    B's group maxima change every 2 columns."""
    K = _K()
    M_, K_, N_ = 256, 512, 520
    rng = np.random.default_rng(43)
    x = rng.standard_normal((M_, K_)).astype(np.float32)
    y = (rng.standard_normal((N_, K_)) * np.exp2(rng.integers(-8, 9, (N_, 1)))).astype(np.float32)
    xq = quant_dev(x, (1, 128), bf16=False)
    yq = quant_dev(y, (1, 128), bf16=False)
    assert yq[2].numel() == N_ // 2
    C = K.gemm_nt(K.operand_rows(*xq, (1, 128)), K.operand_rows(*yq, (1, 128)), torch.float32)
    torch.cuda.synchronize()
    check(C, deq_host(*xq, (1, 128)) @ deq_host(*yq, (1, 128)).T, F32_TOL, "straddling B groups")


def test_wgrad_from_t1x128_requantize():
    """The fp8-mode wgrad chain: the stored (1,128) activation and dY, each
    transposed and quantized (1, 128) along the tokens (quantize_t1x128),
    then contracted over the tokens (span 8, per-row group maxima on both
    operands)."""
    K = _K()
    T, Cin, N_ = 2048, 512, 768
    a_bits = O.activation_input(T, Cin, seed=5)
    dy_bits = O.normal_input((T, N_), 1e-3, seed=6)
    a8 = K.quantize(to_dev_bf16(a_bits), (1, 128))
    at = K.quantize_t1x128(*a8)
    dt = K.quantize_t1x128(to_dev_bf16(dy_bits))
    C = K.gemm_nt(K.operand_rows(*at, (1, 128)), K.operand_rows(*dt, (1, 128)), torch.float32)
    torch.cuda.synchronize()
    a_deq = O.dequantize_impl(u8(a8[0]), u8(a8[1]), f32(a8[2]), "float32", (1, 128))
    aq = O.quantize_impl(np.ascontiguousarray(a_deq.T), (1, 128))
    dq = O.quantize_impl(np.ascontiguousarray(O.bf16_bits_to_f32(dy_bits).T), (1, 128))
    ref = (O.dequantize_impl(*aq, "float32", (1, 128)).astype(np.float64)
           @ O.dequantize_impl(*dq, "float32", (1, 128)).astype(np.float64).T)
    check(C, ref, F32_TOL, "wgrad via quantize_t1x128")


def test_group_maxima_change_across_spans():
    """Rows whose 1024-wide K spans differ by orders of magnitude, all-zero
    spans, and a weight with two groups (the accumulator rescaling path)."""
    K = _K()
    M_, K_, N_ = 256, 4096, 512
    rng = np.random.default_rng(9)
    x = rng.standard_normal((M_, K_)).astype(np.float32)
    scale = np.array([1.0, 1e4, 1e-4, 0.0], np.float32)
    x *= np.repeat(scale, 1024)[None, :]
    x[::7, 1024:2048] = 0.0
    w = (rng.standard_normal((K_, N_)) * 0.02).astype(np.float32)
    w[2048:] *= 300.0
    xq = quant_dev(x, (1, 128), bf16=False)
    wq = quant_dev(w, (128, 128), bf16=False)
    assert wq[2].numel() == 1  # one group max for this weight ([4096,512]: 128 blocks)
    a = K.operand_rows(*xq, (1, 128))
    b = K.operand_transposed(*wq, (128, 128))
    C = K.gemm_nt(a, b, torch.float32)
    torch.cuda.synchronize()
    ref = deq_host(*xq, (1, 128)) @ deq_host(*wq, (128, 128))
    check(C, ref, F32_TOL, "spans")


def test_weight_with_several_groups():
    """W [2048, 16384] (128,128): 2048 blocks, groups of 1024 -> two group
    maxima along K (config 5's FFN weights have four)."""
    K = _K()
    M_, K_, N_ = 256, 2048, 16384
    x = O.activation_input(M_, K_, seed=12)
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((K_, N_)) * 0.02).astype(np.float32)
    w[1024:] *= 8.0
    xq = quant_dev(x, (1, 128))
    wq = quant_dev(w, (128, 128), bf16=False)
    assert wq[2].numel() == 2
    a = K.operand_rows(*xq, (1, 128))
    b = K.operand_transposed(*wq, (128, 128))
    C = K.gemm_nt(a, b, torch.float32)
    torch.cuda.synchronize()
    ref = deq_host(*xq, (1, 128)).astype(np.float32) @ deq_host(*wq, (128, 128)).astype(np.float32)
    check(C, ref, F32_TOL, "w two groups")


def test_config3_full_shape_sampled_rows():
    """Config 3 at full size; the oracle is evaluated on 192 sampled rows."""
    K = _K()
    M_, K_, N_ = 16384, 2048, 8192
    x = O.activation_input(M_, K_, seed=2)
    w = O.normal_input((K_, N_), 0.02, seed=3)
    xq = quant_dev(x, (1, 128))
    wq = quant_dev(w, (128, 128))
    a = K.operand_rows(*xq, (1, 128))
    b = K.operand_transposed(*wq, (128, 128))
    C = K.gemm_nt(a, b, torch.bfloat16)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(1).choice(M_, 192, replace=False))
    xs = O.dequantize_impl(u8(xq[0])[rows], u8(xq[1]).reshape(M_, 2, 8)[rows].reshape(-1, 8),
                           f32(xq[2]).reshape(M_, 2)[rows].reshape(-1, 1, 1), "float32", (1, 128))
    wd = deq_host(*wq, (128, 128)).astype(np.float32)
    ref = xs.astype(np.float32) @ wd
    check(C[torch.from_numpy(rows).cuda()], ref, BF16_TOL, "config 3 sampled")


def _deq_t128_rows(xt8, s8, s32, T, C, rows):
    """Host dequantization of rows ``rows`` of a transposed (128,1) payload
    [C, T] (quantize_impl(x, (128,1)) of x [T, C], payload transposed)."""
    lut = O.e4m3fn_to_f32(np.arange(256, dtype=np.uint8))
    q = lut[u8(xt8)[rows]]                                            # [n, T]
    e = u8(s8).reshape(T // 128, C)[:, rows]                          # [T/128, n]
    G = f32(s32).reshape(-1)[(np.arange(T // 128)[:, None] * C + np.asarray(rows)[None, :]) // 8]
    sc = (O.e8m0_to_f32(e) * G).astype(np.float32)                   # [T/128, n]
    return ((q * np.repeat(sc.T, 128, axis=1)).astype(np.float32) / np.float32(128.0)).astype(np.float64)


def test_config4_full_shape_sampled_rows():
    """Config 4 at full size: dgrad dY [16384,8192] (1,128) x W [2048,8192]
    (128,128), and wgrad A^T . dY with both operands requantized along tokens
    by quantize_t128 (A from its stored fp8 payload), f32 outputs.  The
    oracle product is evaluated on sampled output rows from the GPU operands
    dequantized on the host (the quantizers' bytes are pinned separately)."""
    K = _K()
    T, Cin, N_ = 16384, 2048, 8192
    dy_bits = O.normal_input((T, N_), 1e-3, seed=4)
    w_bits = O.normal_input((Cin, N_), 0.02, seed=3)
    a_bits = O.activation_input(T, Cin, seed=2)
    dyq = quant_dev(dy_bits, (1, 128))
    wq = quant_dev(w_bits, (128, 128))
    dx = K.gemm_nt(K.operand_rows(*dyq, (1, 128)), K.operand_rows(*wq, (128, 128)), torch.float32)
    a8 = K.quantize(to_dev_bf16(a_bits), (1, 128))
    at = K.quantize_t128(*a8)
    dt = K.quantize_t128(to_dev_bf16(dy_bits))
    dw = K.gemm_nt(K.operand_t128(*at), K.operand_t128(*dt), torch.float32)
    torch.cuda.synchronize()
    rng = np.random.default_rng(4)
    # dgrad: 128 sampled rows of dY
    rows = np.sort(rng.choice(T, 128, replace=False))
    dys = O.dequantize_impl(u8(dyq[0])[rows], u8(dyq[1]).reshape(T, 8, 8)[rows].reshape(-1, 8),
                            f32(dyq[2]).reshape(T, 8)[rows].reshape(-1, 1, 1), "float32", (1, 128))
    ref = dys.astype(np.float64) @ deq_host(*wq, (128, 128)).T
    check(dx[torch.from_numpy(rows).cuda()], ref, F32_TOL, "config 4 dgrad sampled")
    # wgrad: 16 sampled channels of A against every channel of dY
    ch = np.sort(rng.choice(Cin, 16, replace=False))
    a_rows = _deq_t128_rows(*at, T, Cin, ch)
    g_all = _deq_t128_rows(*dt, T, N_, np.arange(N_))
    check(dw[torch.from_numpy(ch).cuda()], a_rows @ g_all.T, F32_TOL, "config 4 wgrad sampled")


EDGE_SHAPES = [
    # (M, K, N, weight grid): tiles that overhang M and / or N
    (300, 512, 384, (128, 128)),     # last tile row and column moved back into the matrix
    (100, 256, 128, (128, 128)),     # both dimensions below one tile
    (1, 128, 32, (128, 1)),          # a single token against a LoRA rank
    (257, 384, 1008, (128, 1)),      # lm_head-like vocabulary, one row past a tile
    (640, 1024, 48, (128, 1)),
]


@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("shape", EDGE_SHAPES, ids=lambda s: "x".join(map(str, s[:3])))
def test_edge_tiles(shape, out):
    """Shapes whose M or N is not a multiple of the 256x256 output tile:
    x (1,128) @ W, every output element against the oracle (rows and columns
    outside the matrix are never written: the output is filled with NaN
    first and must hold no NaN afterwards)."""
    K = _K()
    M_, K_, N_, wg = shape
    x = O.activation_input(M_, K_, seed=40 + M_)
    w = O.normal_input((K_, N_), 0.02, seed=41 + N_)
    xq = quant_dev(x, (1, 128))
    wq = quant_dev(w, wg)
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    C = torch.full((M_, N_), float("nan"), dtype=dt, device="cuda")
    K.gemm_nt(K.operand_rows(*xq, (1, 128)), K.operand_transposed(*wq, wg), dt, out=C)
    torch.cuda.synchronize()
    assert not torch.isnan(C).any()
    ref = deq_host(*xq, (1, 128)) @ deq_host(*wq, wg)
    check(C, ref, BF16_TOL if out == "bf16" else F32_TOL, f"edge {shape} {out}")


def test_edge_tile_output_stride():
    """An output written into the left part of a wider buffer (ldc > N) leaves
    the columns past N untouched."""
    K = _K()
    M_, K_, N_ = 300, 256, 96
    xq = quant_dev(O.activation_input(M_, K_, seed=3), (1, 128))
    wq = quant_dev(O.normal_input((K_, N_), 0.02, seed=4), (128, 1))
    wide = torch.full((M_, 160), -7.0, dtype=torch.float32, device="cuda")
    K.gemm_nt(K.operand_rows(*xq, (1, 128)), K.operand_transposed(*wq, (128, 1)), torch.float32,
              out=wide[:, :N_])
    torch.cuda.synchronize()
    assert torch.all(wide[:, N_:] == -7.0)
    check(wide[:, :N_], deq_host(*xq, (1, 128)) @ deq_host(*wq, (128, 1)), F32_TOL, "strided output")


def test_unsupported_shape_is_reported():
    """K must be a whole number of 128-wide blocks; a width below one tile must
    end on a 16-byte output chunk."""
    K = _K()
    xq = quant_dev(O.activation_input(128, 256, seed=1), (1, 128))
    wq = quant_dev(O.normal_input((256, 32), 0.02, seed=1), (128, 1))
    a = K.operand_rows(*xq, (1, 128))
    b = K.operand_transposed(*wq, (128, 1))
    with pytest.raises(Exception, match="multiple of 8"):
        K.gemm_nt(a, K.Operand(b.payload[:20], b.sc8, b.sc32, b.desc), torch.bfloat16)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp8", "bf16"])
def test_mfma_ceiling_probe_runs(bf16):
    """pratchya_mfma_ceiling (the bench's measurement aid) launches on real
    operand bytes, completes, and reports the FLOP count of its MFMA sequence:
    CUs (rounded down to a multiple of 8) x 8 waves x iters x 16 fragment pairs
    x 131072 (fp8 32x32x64) or 65536 (two bf16 32x32x16) FLOP."""
    K = _K()
    g = torch.Generator(device="cuda").manual_seed(3)
    a = torch.randint(0, 255, (256, 256), generator=g, device="cuda", dtype=torch.uint8)
    b = torch.randint(0, 255, (256, 256), generator=g, device="cuda", dtype=torch.uint8)
    if bf16:
        a = torch.randn((256, 128), generator=g, device="cuda").to(torch.bfloat16)
        b = torch.randn((256, 128), generator=g, device="cuda").to(torch.bfloat16)
    else:
        a[(a & 0x7F) == 0x7F] = 0           # no NaN bytes
        b[(b & 0x7F) == 0x7F] = 0
    flop = K.mfma_ceiling(a, b, bf16, 10)
    torch.cuda.synchronize()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert flop == (cus - cus % 8) * 8 * 10 * 16 * (65536 if bf16 else 131072)
