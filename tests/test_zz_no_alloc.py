"""pratchya_quantize_noalloc, the allocation-free quantize, against
pratchya_quantize with a caller workspace, through the C ABI: identical
payload, e8m0 and group-max bytes on two calls in a row (the second with a
smaller input, so stale scratch contents from the first would show), on
layouts that take the general path (block maxima in the library's scratch
array) and one that takes the single-pass kernel (no scratch); and captured
in a HIP graph, replayed with new inputs."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib():
    from pratchya_amd import _lib
    return _lib


def _layout(H, W, a, b):
    from pratchya_amd import _kernels
    return _kernels.group_layout(H, W, (a, b))


def _run(x, S, H, W, a, b, noalloc):
    L = _lib()
    lib = L.load()
    n_blk, K, M = _layout(H, W, a, b)
    q = torch.full((S * H * W,), 0xAB, dtype=torch.uint8, device="cuda")
    s8 = torch.full((S * n_blk,), 0xCD, dtype=torch.uint8, device="cuda")
    s32 = torch.full((S * M,), -1.0, dtype=torch.float32, device="cuda")
    code = L.DT_BF16 if x.dtype == torch.bfloat16 else L.DT_F32
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())     # noqa: E731
    if noalloc:
        rc = lib.pratchya_quantize_noalloc(P(x), code, S, H, W, a, b, P(q), P(s8), P(s32), st)
    else:
        nbytes = lib.pratchya_quantize_workspace_bytes(code, S, H, W, a, b)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
        rc = lib.pratchya_quantize(P(x), code, S, H, W, a, b, P(q), P(s8), P(s32), P(ws), nbytes, st)
    assert rc == 0, lib.pratchya_last_error().decode()
    torch.cuda.synchronize()
    return q, s8, s32


def _same(got, want, what):
    for g, w, name in zip(got, want, ("payload", "e8m0", "group max")):
        assert torch.equal(g.view(torch.uint8), w.view(torch.uint8)), f"{what}: {name} differs"


def test_noalloc_inside_graph_replays():
    """pratchya_quantize_noalloc captured in a HIP graph (the callers it is
    for), on the general path (block maxima in the shared scratch array,
    cleared by a fill kernel, no memset node).  Defined first in this file, so
    that run alone the capture is the process's first call (the scratch
    address is then resolved during the capture).  Three replays, each after
    copying a new input in and an eager call on another, smaller input (which
    leaves other contents in the scratch array), each compared with
    pratchya_quantize run eagerly on the same input, byte for byte."""
    L = _lib()
    lib = L.load()
    S, H, W, a, b = 1, 2048, 8192, 128, 128
    n_blk, K, M = _layout(H, W, a, b)
    g = torch.Generator(device="cuda").manual_seed(43)
    xs = [(torch.randn((S, H, W), generator=g, device="cuda") * std).to(torch.bfloat16) for std in (1.0, 0.02, 40.0)]
    x = torch.empty_like(xs[0])
    q = torch.empty((S * H * W,), dtype=torch.uint8, device="cuda")
    s8 = torch.empty((S * n_blk,), dtype=torch.uint8, device="cuda")
    s32 = torch.empty((S * M,), dtype=torch.float32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())     # noqa: E731
    x.copy_(xs[0])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.pratchya_quantize_noalloc(P(x), L.DT_BF16, S, H, W, a, b, P(q), P(s8), P(s32), st)
    assert rc == 0, lib.pratchya_last_error().decode()
    small = torch.randn((1, 512, 1024), generator=g, device="cuda").to(torch.bfloat16)
    for r, xr in enumerate(xs):
        x.copy_(xr)
        _run(small, 1, 512, 1024, 128, 128, noalloc=True)        # eager work on the shared scratch
        graph.replay()
        torch.cuda.synchronize()
        want = _run(xr, S, H, W, a, b, noalloc=False)
        _same((q, s8, s32), want, f"replay {r}")


@pytest.mark.parametrize("cases", [
    # general path twice, the second call smaller (and of another grid)
    [((1, 2048, 8192), (128, 128), torch.bfloat16, 1.0), ((1, 512, 1024), (128, 128), torch.float32, 3.0)],
    # slices, a grid whose groups straddle block rows, then a one-group matrix
    [((3, 1024, 768), (128, 128), torch.float32, 0.02), ((1, 256, 256), (128, 128), torch.bfloat16, 50.0)],
    # the single-pass (1, 128) kernel between two general-path calls
    [((1, 4096, 2048), (64, 128), torch.bfloat16, 1.0), ((1, 256, 2048), (1, 128), torch.bfloat16, 1.0),
     ((1, 128, 256), (128, 1), torch.float32, 7.0)],
])
def test_noalloc_matches_quantize(cases):
    g = torch.Generator(device="cuda").manual_seed(41)
    for (S, H, W), (a, b), dt, std in cases:
        x = (torch.randn((S, H, W), generator=g, device="cuda") * std).to(dt)
        x[..., 0, :] = 0.0                      # an all-zero block row
        want = _run(x, S, H, W, a, b, noalloc=False)
        got = _run(x, S, H, W, a, b, noalloc=True)
        _same(got, want, f"{(S, H, W)} {(a, b)} {dt}")


def test_noalloc_rejects_layouts_beyond_its_scratch():
    L = _lib()
    lib = L.load()
    assert lib.pratchya_quantize_noalloc_max_bytes() == 16 << 20
    x = torch.zeros(128, dtype=torch.float32, device="cuda")
    P = ctypes.c_void_p(x.data_ptr())
    n = 2049 * 128                                  # 2049^2 blocks of 128x128 > 4 Mi
    rc = lib.pratchya_quantize_noalloc(P, L.DT_F32, 1, n, n, 128, 128, P, P, P, None)
    assert rc == L.EUNSUPPORTED and b"maximum" in lib.pratchya_last_error()
