"""The C-ABI library loads and exports every entry point the headers declare.

CPU-only: no kernel is launched here (no GPU in the build container).
"""
import ctypes
import math
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(pratchya_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_headers_declare_entry_points():
    names = declared_symbols()
    assert "pratchya_quantize" in names and "pratchya_dequantize" in names
    assert len(names) >= 8


def test_library_exports_every_declared_symbol():
    from pratchya_amd import _lib
    lib = _lib.load()
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"missing exports: {missing}"


def test_python_binding_covers_every_declared_symbol():
    from pratchya_amd import _lib
    assert set(declared_symbols()) <= set(_lib.SIGNATURES), \
        set(declared_symbols()) - set(_lib.SIGNATURES)


def test_layout_and_argument_errors_without_gpu():
    from pratchya_amd import _kernels
    assert _kernels.group_layout(1024, 1024, (128, 128)) == (64, 64, 1)
    assert _kernels.group_layout(16384, 2048, (1, 128)) == (262144, 8, 32768)
    assert _kernels.group_layout(0, 128, (1, 128)) == (0, 8, 0)
    with pytest.raises(ValueError, match="does not divide"):
        _kernels.group_layout(10, 10, (3, 5))


def test_workspace_query():
    from pratchya_amd import _lib
    lib = _lib.load()
    # (1,128) bf16 takes the single-pass kernel: no workspace
    assert lib.pratchya_quantize_workspace_bytes(_lib.DT_BF16, 1, 16384, 2048, 1, 128) == 0
    # (128,128) needs one u32 per block
    assert lib.pratchya_quantize_workspace_bytes(_lib.DT_BF16, 1, 2048, 8192, 128, 128) == 1024 * 4


def test_transpose_arguments_without_gpu():
    """Argument checks of pratchya_transpose_u8 return before any launch."""
    from pratchya_amd import _lib
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)          # aligned, never dereferenced
    assert lib.pratchya_transpose_u8(fake, 0, 64, fake, None) == 0
    assert lib.pratchya_transpose_u8(fake, 100, 64, fake, None) == _lib.EUNSUPPORTED
    assert lib.pratchya_transpose_u8(None, 64, 64, None, None) == _lib.EINVAL
    # 128x128 tiles from 2^22 bytes: 2^31 tile rows of one tile each, and a
    # product of sides that would overflow 64 bits
    assert lib.pratchya_transpose_u8(fake, 128 << 31, 128, fake, None) == _lib.EUNSUPPORTED
    assert b"2^31" in lib.pratchya_last_error()
    assert lib.pratchya_transpose_u8(fake, 1 << 40, 1 << 40, fake, None) == _lib.EUNSUPPORTED
    assert b"2^31" in lib.pratchya_last_error()


def test_noalloc_quantize_arguments_without_gpu():
    """pratchya_quantize_noalloc rejects layouts beyond its scratch array and
    bad arguments before any HIP call."""
    from pratchya_amd import _lib
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)          # aligned, never dereferenced
    n = 2049 * 128                           # (128,128): 2049^2 blocks > 4 Mi
    assert lib.pratchya_quantize_noalloc(fake, _lib.DT_BF16, 1, n, n, 128, 128, fake, fake, fake,
                                         None) == _lib.EUNSUPPORTED
    assert b"maximum" in lib.pratchya_last_error()
    assert lib.pratchya_quantize_noalloc(None, _lib.DT_F32, 1, 10, 10, 3, 5, None, None, None, None) == _lib.EINVAL
    assert lib.pratchya_quantize_noalloc(None, 9, 1, 8, 8, 1, 8, None, None, None, None) == _lib.EINVAL
    assert lib.pratchya_quantize_noalloc(None, _lib.DT_F32, 1, 0, 128, 1, 128, None, None, None, None) == 0
    assert lib.pratchya_quantize_noalloc(None, _lib.DT_F32, 1, 128, 128, 128, 128, None, None, None,
                                         None) == _lib.EINVAL


def test_gemm_fq_arguments_without_gpu():
    """pratchya_gemm_bs_nt_fq: workspace query, and argument checks that
    return before any launch (N not a multiple of 1024, narrow B groups, null
    or short workspace)."""
    from pratchya_amd import _lib
    lib = _lib.load()
    # per 256-row x 1024-column strip: 256 maxima + one count, then a status word; 256-byte multiple
    assert lib.pratchya_gemm_bs_nt_fq_workspace_bytes(512, 2048) == ((2 * 2 * 257 + 1) * 4 + 255) // 256 * 256
    assert lib.pratchya_gemm_bs_nt_fq_workspace_bytes(300, 1024) == ((2 * 257 + 1) * 4 + 255) // 256 * 256
    assert lib.pratchya_gemm_bs_nt_fq_workspace_bytes(512, 768) == 0
    fake = ctypes.c_void_p(1 << 20)          # aligned, never dereferenced
    act = (1, 2, 1, 8)                       # (1,128) rows, K = 256
    wgt = (128, 1, 8, 1024)                  # (128,128) weight used transposed
    args = lambda N, bdesc, ws, ws_bytes: (fake, 256, fake, fake, *act, fake, 256, fake, fake, *bdesc,
                                           512, N, 256, fake, N, _lib.DT_BF16, 0, fake, fake, ws, ws_bytes, None)
    need = lib.pratchya_gemm_bs_nt_fq_workspace_bytes(512, 1024)
    assert lib.pratchya_gemm_bs_nt_fq(*args(768, wgt, fake, need)) == _lib.EUNSUPPORTED
    assert b"1024" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bs_nt_fq(*args(1024, (1, 1, 1024, 8), fake, need)) == _lib.EUNSUPPORTED
    assert lib.pratchya_gemm_bs_nt_fq(*args(1024, wgt, None, need)) == _lib.EINVAL
    assert lib.pratchya_gemm_bs_nt_fq(*args(1024, wgt, fake, need - 4)) == _lib.EINVAL
    assert b"workspace" in lib.pratchya_last_error()
    empty = (fake, 256, fake, fake, *act, fake, 256, fake, fake, *wgt, 0, 1024, 256, fake, 1024, _lib.DT_BF16, 0,
             fake, fake, fake, 0, None)
    assert lib.pratchya_gemm_bs_nt_fq(*empty) == 0


def test_bf16_gemm_and_transpose_arguments_without_gpu():
    """pratchya_gemm_bf16_nt and pratchya_transpose_b16 reject unsupported
    shapes and bad arguments before any launch."""
    from pratchya_amd import _lib
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)          # aligned, never dereferenced
    assert lib.pratchya_gemm_bf16_nt(fake, 96, fake, 96, 256, 256, 96, fake, 256, _lib.DT_BF16,
                                     None) == _lib.EUNSUPPORTED
    assert b"multiple of 64" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bf16_nt(fake, 128, fake, 128, 256, 100, 128, fake, 100, _lib.DT_BF16,
                                     None) == _lib.EUNSUPPORTED
    assert lib.pratchya_gemm_bf16_nt(None, 128, fake, 128, 256, 256, 128, fake, 256, _lib.DT_F32,
                                     None) == _lib.EINVAL
    assert lib.pratchya_gemm_bf16_nt(fake, 100, fake, 128, 256, 256, 64, fake, 256, _lib.DT_F32,
                                     None) == _lib.EINVAL
    assert lib.pratchya_gemm_bf16_nt(fake, 128, fake, 128, 0, 256, 128, fake, 256, _lib.DT_F32, None) == 0
    assert lib.pratchya_transpose_b16(fake, 12, 64, fake, None) == _lib.EUNSUPPORTED
    assert lib.pratchya_transpose_b16(None, 64, 64, None, None) == _lib.EINVAL
    assert lib.pratchya_transpose_b16(fake, 0, 64, fake, None) == 0


def test_invalid_tgrid_is_einval_without_launch():
    from pratchya_amd import _lib
    lib = _lib.load()
    rc = lib.pratchya_quantize(None, _lib.DT_F32, 1, 10, 10, 3, 5, None, None, None, None, 0, None)
    assert rc == _lib.EINVAL
    assert b"does not divide" in lib.pratchya_last_error()
    rc = lib.pratchya_quantize(None, 7, 1, 8, 8, 1, 8, None, None, None, None, 0, None)
    assert rc == _lib.EINVAL
    # empty tensors are valid no-ops
    assert lib.pratchya_quantize(None, _lib.DT_F32, 1, 0, 128, 1, 128, None, None, None, None, 0, None) == 0


@pytest.mark.parametrize("rows,K,desc,expect", [
    (16384, 2048, (1, 16, 1, 8), 8),          # (1,128) activation [16384, 2048]
    (8192, 2048, (128, 1, 64, 1024), 16),     # W [2048, 8192] (128,128) used transposed
    (2048, 8192, (128, 64, 1, 1024), 64),     # W [2048, 8192] (128,128) rows in dgrad
    (2048, 16384, (1, 1, 2048, 8), 1),        # (128,1) token-axis A [16384, 2048] transposed
    (4096, 16384, (128, 1, 32, 1024), 32),    # FFN down W [16384, 4096] used transposed
    (1024, 768, (128, 6, 1, 16), 2),          # W [1024, 768] (128,128): groups straddle block rows
])
def test_gemm_group_span(rows, K, desc, expect):
    from pratchya_amd import _lib
    assert _lib.load().pratchya_gemm_span(rows, K, *desc) == expect


def test_gemm_span_matches_brute_force():
    """The span the GEMM uses keeps every row's group index constant."""
    from pratchya_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(0)
    for _ in range(200):
        nk = int(rng.choice([1, 2, 4, 8, 16]))
        rdiv = int(rng.choice([1, 2, 4, 128]))
        rows = rdiv * int(rng.integers(1, 9))
        sr = int(rng.choice([0, 1, 2, 4, nk, 2 * nk]))
        sk = int(rng.choice([0, 1, 2, 8, rows // rdiv]))
        kg = int(rng.choice([1, 2, 4, 8, 16, 64]))
        P = lib.pratchya_gemm_span(rows, nk * 128, rdiv, sr, sk, kg)
        assert P >= 1
        changes = set()
        for rb in range(rows // rdiv):
            g = [(rb * sr + kb * sk) // kg for kb in range(nk)]
            for s0 in range(0, nk, P):
                assert len(set(g[s0:s0 + P])) == 1, (rows, nk, rdiv, sr, sk, kg, P)
            changes |= {kb for kb in range(1, nk) if g[kb] != g[kb - 1]}
        # maximal: the gcd of every position where some row's group changes
        want = 0
        for kb in changes:
            want = math.gcd(want, kb)
        assert P == (want or nk), (rows, nk, rdiv, sr, sk, kg, P, want)


@pytest.mark.parametrize("entry", ["pratchya_quantize_t128", "pratchya_quantize_128x1"])
def test_quantize_t128_argument_codes_without_gpu(entry):
    """Shape errors are reported before anything touches a buffer (both
    payload layouts share the checks)."""
    from pratchya_amd import _lib
    lib = _lib.load()
    f = getattr(lib, entry)
    # 100 tokens: tgrid (128, 1) does not divide -> the reference's reshape error
    assert f(None, _lib.DT_BF16, None, None, 1, 100, 64, None, None, None, None) == _lib.EINVAL
    # fp8 input whose (1, 128) grid does not divide the channels
    assert f(None, _lib.DT_E4M3, None, None, 1, 128, 64, None, None, None, None) == _lib.EINVAL
    # 12 channels: groups would straddle token blocks; not supported by this kernel
    assert f(None, _lib.DT_BF16, None, None, 1, 128, 12, None, None, None, None) == _lib.EUNSUPPORTED
    assert f(None, 7, None, None, 1, 128, 64, None, None, None, None) == _lib.EINVAL
    # empty tensors are a no-op
    assert f(None, _lib.DT_BF16, None, None, 0, 128, 64, None, None, None, None) == _lib.OK


def test_quantize_t1x128_argument_codes_without_gpu():
    """pratchya_quantize_t1x128 reports shape and argument errors before
    anything touches a buffer."""
    from pratchya_amd import _lib
    lib = _lib.load()
    f = lib.pratchya_quantize_t1x128
    fake = ctypes.c_void_p(1 << 20)
    assert f(None, _lib.DT_BF16, None, None, 1, -1, 64, None, None, None, None) == _lib.EINVAL
    # 100 tokens: tgrid (1, 128) of x^T does not divide them
    assert f(None, _lib.DT_BF16, None, None, 1, 100, 64, None, None, None, None) == _lib.EINVAL
    # fp8 input whose (1, 128) grid does not divide the channels
    assert f(None, _lib.DT_E4M3, None, None, 1, 1024, 64, None, None, None, None) == _lib.EINVAL
    # below 1024 tokens a group of 8 token blocks straddles channels
    assert f(None, _lib.DT_BF16, None, None, 1, 512, 64, None, None, None, None) == _lib.EUNSUPPORTED
    assert b"1024" in lib.pratchya_last_error()
    # 12 channels: not a multiple of 8
    assert f(None, _lib.DT_BF16, None, None, 1, 1024, 12, None, None, None, None) == _lib.EUNSUPPORTED
    assert f(None, 7, None, None, 1, 1024, 64, None, None, None, None) == _lib.EINVAL
    assert f(fake, _lib.DT_BF16, None, None, 1, 1024, 64, None, fake, fake, None) == _lib.EINVAL   # null output
    assert f(None, _lib.DT_BF16, None, None, 0, 1024, 64, None, None, None, None) == _lib.OK     # empty


def test_quantize_dequantize_codes_without_gpu():
    """Workspace query and argument errors of the one-pass fake quantization."""
    from pratchya_amd import _lib
    lib = _lib.load()
    ws = lib.pratchya_quantize_dequantize_workspace_bytes
    assert ws(_lib.DT_F32, 1, 32768, 4096, 1, 128) == 0           # single-pass kernel
    assert ws(_lib.DT_F32, 1, 4096, 16384, 128, 128) == 32 * 128 * 4
    assert ws(_lib.DT_F32, 1, 64, 256, 1, 32) == 64 * 8 * 4        # (1, 32): general path
    f = lib.pratchya_quantize_dequantize
    args = lambda xdt, H, W, a, b, odt: (None, xdt, 1, H, W, a, b, None, odt, 0, None, None, None, 0, None)
    assert f(*args(_lib.DT_F32, 10, 10, 3, 5, _lib.DT_BF16)) == _lib.EINVAL
    assert b"does not divide" in lib.pratchya_last_error()
    assert f(*args(7, 8, 128, 1, 128, _lib.DT_BF16)) == _lib.EINVAL
    assert f(*args(_lib.DT_F32, 8, 128, 1, 128, _lib.DT_E4M3)) == _lib.EINVAL
    assert f(*args(_lib.DT_F32, 0, 128, 1, 128, _lib.DT_F32)) == _lib.OK
    assert f(*args(_lib.DT_F32, 8, 128, 1, 128, _lib.DT_F32)) == _lib.EINVAL      # null buffers


def test_requantize_cotangent_codes_without_gpu():
    from pratchya_amd import _lib
    lib = _lib.load()
    f = lib.pratchya_requantize_cotangent
    assert f(None, _lib.DT_BF16, None, None, 1, 10, 100, None, None, None, None) == _lib.EINVAL   # 128 does not divide 100
    assert f(None, 7, None, None, 1, 8, 1024, None, None, None, None) == _lib.EINVAL
    assert f(None, _lib.DT_BF16, None, None, 1, 0, 1024, None, None, None, None) == _lib.OK
    assert f(None, _lib.DT_BF16, None, None, 1, 8, 1024, None, None, None, None) == _lib.EINVAL  # null buffers


def test_optimizer_entry_point_codes_without_gpu():
    """pratchya_momentum / pratchya_apply_update validate layouts, dtypes and
    buffers before any launch (empty tensors are a no-op)."""
    from pratchya_amd import _lib
    lib = _lib.load()
    m = lib.pratchya_momentum
    F32, BF16, E4M3 = _lib.DT_F32, _lib.DT_BF16, _lib.DT_E4M3
    # tgrid (96, 128) does not divide 256 x 256
    assert m(None, None, None, None, E4M3, None, None, 1, 256, 256, 96, 128, F32, 0.9, 0.1, 0.99, 0.01,
             None, None, None) == _lib.EINVAL
    assert b"does not fit" in lib.pratchya_last_error()
    # unsupported arithmetic and gradient dtypes
    assert m(None, None, None, None, E4M3, None, None, 1, 256, 256, 128, 128, E4M3, 0.9, 0.1, 0.99, 0.01,
             None, None, None) == _lib.EINVAL
    assert m(None, None, None, None, 7, None, None, 1, 256, 256, 128, 128, F32, 0.9, 0.1, 0.99, 0.01,
             None, None, None) == _lib.EINVAL
    # empty: nothing to do; non-empty with null buffers: an error
    assert m(None, None, None, None, BF16, None, None, 1, 0, 256, 128, 128, BF16, 0.9, 0.1, 0.99, 0.01,
             None, None, None) == _lib.OK
    assert m(None, None, None, None, BF16, None, None, 1, 256, 256, 128, 128, BF16, 0.9, 0.1, 0.99, 0.01,
             None, None, None) == _lib.EINVAL
    u = lib.pratchya_apply_update
    # an f32 direction with bf16 arithmetic is only valid for the sign (Lion) form
    assert u(None, F32, 0, 64.0, None, E4M3, None, None, 1, 256, 256, 128, 128, BF16, 0.05, 0.005,
             None, BF16, None) == _lib.EINVAL
    assert b"f32 direction" in lib.pratchya_last_error()
    assert u(None, E4M3, 1, 0.0, None, E4M3, None, None, 1, 256, 256, 128, 128, F32, 0.05, 0.005,
             None, F32, None) == _lib.EINVAL
    assert u(None, F32, 1, 0.0, None, F32, None, None, 1, 0, 256, 1, 1, F32, 0.05, 0.005,
             None, F32, None) == _lib.OK
    assert u(None, F32, 1, 0.0, None, F32, None, None, 1, 256, 256, 1, 1, F32, 0.05, 0.005,
             None, F32, None) == _lib.EINVAL


def test_elementwise_and_ns_combine_codes_without_gpu():
    """pratchya_elementwise / pratchya_ns_combine and the workspace query
    validate operators, grids, dtypes and buffers before any launch."""
    from pratchya_amd import _lib
    lib = _lib.load()
    e = lib.pratchya_elementwise
    # unknown operator, non-dividing result grid, non-dividing operand grid
    assert e(6, None, None, None, 1, 128, None, None, None, 1, 128, 1, 64, 256, 1, 128,
             None, None, None, None, 0, None) == _lib.EINVAL
    assert b"unknown operator" in lib.pratchya_last_error()
    assert e(0, None, None, None, 1, 128, None, None, None, 1, 128, 1, 64, 256, 3, 128,
             None, None, None, None, 0, None) == _lib.EINVAL
    assert b"result grid" in lib.pratchya_last_error()
    assert e(0, None, None, None, 1, 128, None, None, None, 1, 96, 1, 64, 256, 1, 128,
             None, None, None, None, 0, None) == _lib.EINVAL
    assert b"y grid" in lib.pratchya_last_error()
    # empty: nothing to do; non-empty with null buffers: an error
    assert e(0, None, None, None, 1, 128, None, None, None, 1, 128, 1, 0, 256, 1, 128,
             None, None, None, None, 0, None) == _lib.OK
    assert e(0, None, None, None, 1, 128, None, None, None, 1, 128, 1, 64, 256, 1, 128,
             None, None, None, None, 0, None) == _lib.EINVAL
    assert b"null buffer" in lib.pratchya_last_error()
    ws = lib.pratchya_elementwise_workspace_bytes
    assert ws(1, 64, 256, 1, 128, 1, 128, 1, 128) == 0                 # one-pass layout
    assert ws(1, 256, 256, 128, 128, 128, 128, 128, 128) == 4 * 4      # 2 x 2 blocks of (128, 128)
    assert ws(1, 64, 256, 1, 128, 1, 128, 3, 128) == 0                 # invalid: 0
    c = lib.pratchya_ns_combine
    assert c(None, None, None, 16, _lib.DT_E4M3, None) == _lib.EINVAL
    assert c(None, None, None, -1, _lib.DT_F32, None) == _lib.EINVAL
    assert c(None, None, None, 0, _lib.DT_BF16, None) == _lib.OK
    assert c(None, None, None, 16, _lib.DT_BF16, None) == _lib.EINVAL


def test_gather_quantize_codes_without_gpu():
    """pratchya_gather_quantize validates grids, the table and buffers before
    any launch."""
    from pratchya_amd import _lib
    lib = _lib.load()
    f = lib.pratchya_gather_quantize
    # table grid (96, 128) does not divide [512, 256]; result grid (3, 128) does not divide [40, 256]
    assert f(None, None, None, 512, 256, 96, 128, None, 1, 40, 8, 128, None, None, None, None, 0, None) == _lib.EINVAL
    assert f(None, None, None, 512, 256, 128, 128, None, 1, 40, 3, 128, None, None, None, None, 0, None) == _lib.EINVAL
    # nothing to look up; an empty table; null buffers; a missing workspace
    assert f(None, None, None, 512, 256, 128, 128, None, 1, 0, 1, 128, None, None, None, None, 0, None) == _lib.OK
    assert f(None, None, None, 0, 256, 1, 128, None, 1, 40, 8, 128, None, None, None, None, 0, None) == _lib.EINVAL
    assert f(None, None, None, 512, 256, 128, 128, None, 1, 40, 8, 128, None, None, None, None, 0, None) == _lib.EINVAL
    assert b"null buffer" in lib.pratchya_last_error()


def test_mfma_ceiling_argument_codes_without_gpu():
    """The MFMA-rate probe rejects null pointers and short rows before any launch."""
    from pratchya_amd import _lib
    lib = _lib.load()
    flop = ctypes.c_int64(0)
    p = ctypes.c_void_p(16)
    assert lib.pratchya_mfma_ceiling(None, p, 128, 0, 1, p, ctypes.byref(flop), None) == _lib.EINVAL
    assert lib.pratchya_mfma_ceiling(p, p, 64, 0, 1, p, ctypes.byref(flop), None) == _lib.EINVAL
    assert lib.pratchya_mfma_ceiling(p, p, 128, 0, 0, p, ctypes.byref(flop), None) == _lib.EINVAL
    assert lib.pratchya_mfma_ceiling(p, p, 128, 1, 1, p, None, None) == _lib.EINVAL


def test_gemm_bf16_gram_argument_codes_without_gpu():
    """The symmetric product sizes its workspace from M, K and the device's CUs
    (256 without a device), and rejects M not a multiple of 256, K not a
    multiple of 64 and a short workspace before any launch."""
    from pratchya_amd import _lib
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    other = ctypes.c_void_p(1 << 30)
    ws = lib.pratchya_gemm_bf16_gram_workspace_bytes(4096, 16384)
    # 256 ranges, 8 waves of 32 KB of partials each, then 2048 flags and a status word
    assert ws == 256 * 8 * 32768 + (256 * 8 + 1) * 4
    # one tile of one 64-wide step: a single range
    assert lib.pratchya_gemm_bf16_gram_workspace_bytes(256, 64) == 8 * 32768 + 9 * 4
    assert lib.pratchya_gemm_bf16_gram_workspace_bytes(300, 64) == 0
    assert lib.pratchya_gemm_bf16_gram_workspace_bytes(256, 96) == 0
    assert lib.pratchya_gemm_bf16_gram(fake, 128, 304, 128, 0, other, 304, other, 1 << 30, None) == _lib.EUNSUPPORTED
    assert lib.pratchya_gemm_bf16_gram(fake, 96, 256, 96, 0, other, 256, other, 1 << 30, None) == _lib.EUNSUPPORTED
    assert lib.pratchya_gemm_bf16_gram(fake, 128, 256, 128, 0, other, 256, other, 16, None) == _lib.EINVAL
    assert b"workspace" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bf16_gram(fake, 128, 256, 128, 0, other, 256, None, 1 << 30, None) == _lib.EINVAL
    assert lib.pratchya_gemm_bf16_gram(fake, 128, 0, 128, 0, other, 256, None, 0, None) == 0
    # K-major A: the row stride must cover M
    assert lib.pratchya_gemm_bf16_gram(fake, 128, 256, 128, 1, other, 256, other, 1 << 30, None) == _lib.EINVAL
    assert b"K-major" in lib.pratchya_last_error()


def test_ns_normalize_argument_codes_without_gpu():
    """The fused normalization rejects a null buffer, a short workspace and a
    misaligned operand before any launch; n = 0 is a no-op."""
    from pratchya_amd import _lib
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    ws_bytes = lib.pratchya_ns_normalize_workspace_bytes()
    assert ws_bytes == 1024 * 4
    assert lib.pratchya_ns_normalize(fake, fake, 0, None, 0, None) == 0
    assert lib.pratchya_ns_normalize(fake, None, 64, fake, ws_bytes, None) == _lib.EINVAL
    assert lib.pratchya_ns_normalize(fake, fake, 64, fake, ws_bytes - 4, None) == _lib.EINVAL
    assert b"workspace" in lib.pratchya_last_error()
    assert lib.pratchya_ns_normalize(ctypes.c_void_p((1 << 20) + 2), fake, 64, fake, ws_bytes, None) == _lib.EINVAL
    assert b"aligned" in lib.pratchya_last_error()
    # the f32 form: the same argument checks
    assert lib.pratchya_ns_normalize_f32(fake, fake, 0, None, 0, None) == 0
    assert lib.pratchya_ns_normalize_f32(fake, None, 64, fake, ws_bytes, None) == _lib.EINVAL
    assert lib.pratchya_ns_normalize_f32(fake, fake, 64, fake, ws_bytes - 4, None) == _lib.EINVAL
    assert b"workspace" in lib.pratchya_last_error()
    assert lib.pratchya_ns_normalize_f32(ctypes.c_void_p((1 << 20) + 8), fake, 64, fake, ws_bytes, None) == _lib.EINVAL
    assert b"aligned" in lib.pratchya_last_error()


def test_gemm_bf16_ns_argument_codes_without_gpu():
    """The fused Newton-Schulz GEMM rejects an output overlapping X, a bad X
    and K not a multiple of 64 before any launch."""
    from pratchya_amd import _lib
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    other = ctypes.c_void_p(1 << 30)
    assert lib.pratchya_gemm_bf16_nt_ns(fake, 128, fake, 128, 0, 256, 256, 128, other, 256, other, 256,
                                        None) == _lib.EINVAL
    assert b"overlaps" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bf16_nt_ns(fake, 128, fake, 128, 0, 256, 256, 128, None, 256, other, 256,
                                        None) == _lib.EINVAL
    assert lib.pratchya_gemm_bf16_nt_ns(fake, 96, fake, 96, 0, 256, 256, 96, fake, 256, other, 256,
                                        None) == _lib.EUNSUPPORTED
    assert lib.pratchya_gemm_bf16_nt_ns(fake, 128, fake, 128, 0, 0, 256, 128, fake, 256, other, 256, None) == 0
    # a K-major B with a row stride below N
    assert lib.pratchya_gemm_bf16_nt_ns(fake, 128, fake, 128, 1, 256, 256, 128, fake, 256, other, 256,
                                        None) == _lib.EINVAL
    assert b"K-major" in lib.pratchya_last_error()


def test_gemm_kmajor_argument_codes_without_gpu():
    """pratchya_gemm_bs_kmajor: M, N and the row strides must be multiples of
    16 with strides of at least M and N; checked before any launch."""
    from pratchya_amd import _lib
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)          # aligned, never dereferenced
    op = (1, 1, 256, 8)                      # (128, 1) groups of a [T, C] operand (K = T = 256)
    args = lambda M, N, lda, ldb: (fake, lda, fake, fake, *op, fake, ldb, fake, fake, *op, M, N, 256, fake, N,
                                   _lib.DT_F32, None)
    assert lib.pratchya_gemm_bs_kmajor(*args(264, 256, 264, 256)) == _lib.EINVAL
    assert b"multiples of 16" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bs_kmajor(*args(256, 256, 128, 256)) == _lib.EINVAL
    assert lib.pratchya_gemm_bs_kmajor(*args(256, 256, 256, 264)) == _lib.EINVAL
    assert lib.pratchya_gemm_bs_kmajor(*args(0, 256, 256, 256)) == _lib.OK
    assert lib.pratchya_gemm_bs_kmajor(*args(-1, 256, 256, 256)) == _lib.EINVAL


def test_status_offsets_without_gpu():
    """The bounded waits' status words: the last word of the requantizing
    GEMM's workspace layout (maxima, arrival counts, status) and the word
    after the Gram product's partial tiles and flags; -1 for shapes the
    calls reject."""
    from pratchya_amd import _lib
    lib = _lib.load()
    for M, N in ((2048, 2048), (32768, 16384), (300, 1024)):
        strips = -(-M // 256) * (N // 1024)
        assert lib.pratchya_gemm_bs_nt_fq_status_offset(M, N) == strips * 257 * 4
        assert lib.pratchya_gemm_bs_nt_fq_status_offset(M, N) + 4 <= lib.pratchya_gemm_bs_nt_fq_workspace_bytes(M, N)
    assert lib.pratchya_gemm_bs_nt_fq_status_offset(2048, 1000) == -1
    for M, Kd in ((4096, 16384), (256, 64), (1024, 2048)):
        off = lib.pratchya_gemm_bf16_gram_status_offset(M, Kd)
        assert off > 0 and off + 4 == lib.pratchya_gemm_bf16_gram_workspace_bytes(M, Kd)
    assert lib.pratchya_gemm_bf16_gram_status_offset(300, 64) == -1


def test_quantize_dual_argument_codes_without_gpu():
    """pratchya_quantize_dual rejects other dtypes, token counts and channel
    counts (EINVAL for grids that do not divide, EUNSUPPORTED for a width that
    is not a multiple of 1024), null and misaligned buffers, before any
    launch; an empty tensor is a no-op."""
    from pratchya_amd import _lib
    lib = _lib.load()
    f = ctypes.c_void_p(1 << 20)
    args = lambda q: (q, f, f, f, f, f, None)    # noqa: E731  (q: the payload, 16-byte aligned)
    assert lib.pratchya_quantize_dual(f, _lib.DT_BF16, 1, 0, 1024, *args(f)) == 0
    assert lib.pratchya_quantize_dual(f, _lib.DT_E4M3, 1, 128, 1024, *args(f)) == _lib.EINVAL
    assert lib.pratchya_quantize_dual(f, _lib.DT_BF16, 1, 100, 1024, *args(f)) == _lib.EINVAL
    assert lib.pratchya_quantize_dual(f, _lib.DT_BF16, 1, 128, 1000, *args(f)) == _lib.EINVAL
    assert lib.pratchya_quantize_dual(f, _lib.DT_BF16, 1, 128, 2560, *args(f)) == _lib.EUNSUPPORTED
    assert b"1024" in lib.pratchya_last_error()
    assert lib.pratchya_quantize_dual(f, _lib.DT_BF16, 1, 128, 1024, *args(None)) == _lib.EINVAL
    assert lib.pratchya_quantize_dual(f, _lib.DT_F32, 1, 128, 1024, *args(ctypes.c_void_p((1 << 20) + 8))) \
        == _lib.EUNSUPPORTED
    assert b"aligned" in lib.pratchya_last_error()


def test_gemm_qa_arguments_without_gpu():
    """pratchya_gemm_bs_nt_qa: workspace and status-word queries (the
    prologue's count, the status word, then the output requantization's
    layout with fq), and the argument checks that return before any launch:
    too few rows, K not a multiple of 1024, N not a multiple of 1024 with fq,
    narrow B groups, misaligned X or outputs, null or short workspace."""
    from pratchya_amd import _lib
    lib = _lib.load()
    for M, N, fq in ((512, 2048, 0), (32768, 16384, 1), (300, 1024, 1)):
        units = -(-M // 256)
        words = 2 + ((units * (N // 1024)) * 257 + 1 if fq else 0)
        assert lib.pratchya_gemm_bs_nt_qa_workspace_bytes(M, N, fq) == (words * 4 + 255) // 256 * 256
        assert lib.pratchya_gemm_bs_nt_qa_status_offset(M, N, fq) == 4
    assert lib.pratchya_gemm_bs_nt_qa_workspace_bytes(255, 1024, 0) == 0
    assert lib.pratchya_gemm_bs_nt_qa_workspace_bytes(512, 768, 1) == 0
    assert lib.pratchya_gemm_bs_nt_qa_status_offset(512, 768, 1) == -1
    fake = ctypes.c_void_p(1 << 20)          # aligned, never dereferenced
    wgt = (128, 1, 8, 1024)                  # (128,128) weight used transposed
    need = lib.pratchya_gemm_bs_nt_qa_workspace_bytes(512, 1024, 1)

    def args(M=512, N=1024, K=1024, bdesc=wgt, x=fake, A=fake, fq=1, ws=fake, ws_bytes=need):
        return (x, K, A, fake, fake, fake, K, fake, fake, *bdesc, M, N, K, fake, N, _lib.DT_BF16, fq,
                fake, fake, ws, ws_bytes, None)

    assert lib.pratchya_gemm_bs_nt_qa(*args(M=0)) == 0
    assert lib.pratchya_gemm_bs_nt_qa(*args(M=-1)) == _lib.EINVAL
    assert lib.pratchya_gemm_bs_nt_qa(*args(M=255)) == _lib.EUNSUPPORTED
    assert lib.pratchya_gemm_bs_nt_qa(*args(K=512)) == _lib.EUNSUPPORTED
    assert b"1024" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bs_nt_qa(*args(N=768)) == _lib.EUNSUPPORTED
    assert lib.pratchya_gemm_bs_nt_qa(*args(bdesc=(1, 1, 1024, 8))) == _lib.EUNSUPPORTED
    assert lib.pratchya_gemm_bs_nt_qa(*args(x=ctypes.c_void_p((1 << 20) + 8))) == _lib.EINVAL
    assert lib.pratchya_gemm_bs_nt_qa(*args(A=ctypes.c_void_p((1 << 20) + 128))) == _lib.EINVAL
    assert b"256-byte" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bs_nt_qa(*args(ws=None)) == _lib.EINVAL
    assert lib.pratchya_gemm_bs_nt_qa(*args(ws_bytes=need - 4)) == _lib.EINVAL
    assert b"workspace" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bs_nt_qa(*args(fq=2)) == _lib.EINVAL


def test_gemm_q11_arguments_without_gpu():
    """pratchya_gemm_bs_nt_q11: the checks that return before any launch --
    empty and negative sizes, N not a multiple of 16, null or misaligned
    scale arrays."""
    from pratchya_amd import _lib
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)          # aligned, never dereferenced
    wgt = (1, 1, 1024, 8)                    # (128,1) weight used transposed

    def args(M=512, N=1024, K=1024, sc8=fake, sc32=fake):
        return (fake, K, fake, fake, 1, 8, 1, 8, fake, K, fake, fake, *wgt, M, N, K, fake, N, _lib.DT_BF16,
                sc8, sc32, None)

    assert lib.pratchya_gemm_bs_nt_q11(*args(M=0)) == 0
    assert lib.pratchya_gemm_bs_nt_q11(*args(N=0)) == 0
    assert lib.pratchya_gemm_bs_nt_q11(*args(M=-1)) == _lib.EINVAL
    assert lib.pratchya_gemm_bs_nt_q11(*args(N=1000)) == _lib.EUNSUPPORTED
    assert b"multiple of 16" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bs_nt_q11(*args(sc8=None)) == _lib.EINVAL
    assert lib.pratchya_gemm_bs_nt_q11(*args(sc32=ctypes.c_void_p((1 << 20) + 4))) == _lib.EINVAL
    assert b"16-byte" in lib.pratchya_last_error()


def test_gemm_blockmax_and_premax_arguments_without_gpu():
    """pratchya_gemm_bs_blockmax rejects M or N not multiples of 128 and a
    null maxima buffer, pratchya_quantize_dequantize_premax a null buffer, an
    other output dtype and a non-dividing grid, before any launch; empty
    shapes are no-ops."""
    from pratchya_amd import _lib
    lib = _lib.load()
    f = ctypes.c_void_p(1 << 20)
    act = (1, 1, 2048, 8)                    # (128,1)-requantized operand read transposed
    args = lambda M, N, bm: (f, 256, f, f, *act, f, 256, f, f, *act, M, N, 256, 0, f, N, bm, None)  # noqa: E731
    assert lib.pratchya_gemm_bs_blockmax(*args(0, 256, f)) == 0
    assert lib.pratchya_gemm_bs_blockmax(*args(-1, 256, f)) == _lib.EINVAL
    assert lib.pratchya_gemm_bs_blockmax(*args(200, 256, f)) == _lib.EUNSUPPORTED
    assert b"128" in lib.pratchya_last_error()
    assert lib.pratchya_gemm_bs_blockmax(*args(256, 320, f)) == _lib.EUNSUPPORTED
    assert lib.pratchya_gemm_bs_blockmax(*args(256, 256, None)) == _lib.EINVAL
    q = lambda H, W, a, b, bm, dt: (f, 1, H, W, a, b, bm, f, dt, 1, f, f, None)  # noqa: E731
    assert lib.pratchya_quantize_dequantize_premax(*q(0, 256, 128, 128, f, _lib.DT_BF16)) == 0
    assert lib.pratchya_quantize_dequantize_premax(*q(256, 256, 128, 128, None, _lib.DT_BF16)) == _lib.EINVAL
    assert lib.pratchya_quantize_dequantize_premax(*q(256, 256, 128, 128, f, _lib.DT_E4M3)) == _lib.EINVAL
    assert lib.pratchya_quantize_dequantize_premax(*q(200, 256, 128, 128, f, _lib.DT_F32)) == _lib.EINVAL
