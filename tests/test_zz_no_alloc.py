"""The allocation-free forward entry point (mxs_nf4_linear_fwd_noalloc) against the workspace
one (mxs_nf4_linear_fwd): same bits, on two calls in a row that share the library's device array,
the second with fewer tokens; the size limit refused before anything launches."""

import pytest
import torch

from mindxsoup_amd import _lib, kernels
from mindxsoup_amd.quant import quantize_4bit

pytestmark = pytest.mark.gpu


def _weight(dev, n, k, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).half()
    return quantize_4bit(w)


def _inputs(dev, M, k, n, r, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn((M, k), device=dev, generator=g).half()
    h = (torch.randn((M, r), device=dev, generator=g) * 0.1).half()
    b = (torch.randn((n, r), device=dev, generator=g) * 0.01).half()
    bias = (torch.randn((n,), device=dev, generator=g) * 0.1).half()
    return x, h, b, bias


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_noalloc_matches_workspace_entry_twice(cuda):
    """down_proj's shape plans split-K 4: the partials go through the device array.  The second
    call has fewer tokens and must not see the first call's partials."""
    n, k, r = 1536, 8960, 16
    packed, st = _weight(cuda, n, k, 1)
    assert kernels.gemm_workspace_bytes(1024, n, k) > 0  # the plan splits: the array is used
    for M, seed in ((1024, 2), (300, 3)):
        x, h, b, bias = _inputs(cuda, M, k, n, r, seed)
        want = kernels.nf4_linear_fwd(x, packed, st, bias, h, b)
        got = torch.full((M, n), float("nan"), dtype=torch.float16, device=cuda)
        kernels.nf4_linear_fwd_noalloc(x, packed, st, got, bias, h, b)
        torch.cuda.synchronize()
        print(f"noalloc M={M} N={n} K={k}", flush=True)
        assert _same(got, want), f"M={M}"


def test_noalloc_unsplit_and_explicit_plans(cuda):
    """A plan without split-K (q_proj's shape) never touches the array; an explicit split plan
    on the same weight matches the workspace entry with the same plan."""
    n, k = 1536, 1536
    packed, st = _weight(cuda, n, k, 4)
    x, _, _, _ = _inputs(cuda, 512, k, n, 16, 5)
    for cfg, splits in ((-1, 1), (4, 4), (9, 2)):
        want = kernels.nf4_linear_fwd(x, packed, st, cfg=cfg, splits=splits)
        got = torch.empty_like(want)
        kernels.nf4_linear_fwd_noalloc(x, packed, st, got, cfg=cfg, splits=splits)
        torch.cuda.synchronize()
        assert _same(got, want), (cfg, splits)


def test_noalloc_refuses_plans_beyond_the_array(cuda):
    """4 splits x 2048 tokens x 1536 columns x 4 bytes = 48 MiB > 32 MiB: MXS_ERR_SIZE, and the
    output is left untouched."""
    n, k, M = 1536, 8960, 2048
    packed, st = _weight(cuda, n, k, 6)
    x = torch.zeros((M, k), dtype=torch.float16, device=cuda)
    y = torch.full((M, n), 7.0, dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="shape outside"):
        kernels.nf4_linear_fwd_noalloc(x, packed, st, y)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    assert _lib.lib().mxs_nf4_linear_fwd_noalloc(None, -1, k, n, None, None, None, None, None,
                                                 None, None, None, 0, None, -1, 1, None) == -1


def test_noalloc_replays_in_a_hip_graph(cuda):
    """Captured in a HIP graph (after one call outside the capture has looked up the array's
    address), the split-K down_proj forward replays to the workspace entry's bits, with eager
    calls that reuse the array between the replays."""
    n, k, r, M = 1536, 8960, 16, 1024
    packed, st = _weight(cuda, n, k, 7)
    x, h, b, bias = _inputs(cuda, M, k, n, r, 8)
    want = kernels.nf4_linear_fwd(x, packed, st, bias, h, b)
    y = torch.empty((M, n), dtype=torch.float16, device=cuda)
    kernels.nf4_linear_fwd_noalloc(x, packed, st, y, bias, h, b)  # the address lookup
    torch.cuda.synchronize()
    assert _same(y, want)
    y.fill_(float("nan"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.nf4_linear_fwd_noalloc(x, packed, st, y, bias, h, b)
    x2, h2, b2, bias2 = _inputs(cuda, 300, k, n, r, 9)
    other = torch.empty((300, n), dtype=torch.float16, device=cuda)
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        kernels.nf4_linear_fwd_noalloc(x2, packed, st, other, bias2, h2, b2)  # reuses the array
        torch.cuda.synchronize()
        y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert _same(y, want), rep
    assert _same(other, kernels.nf4_linear_fwd(x2, packed, st, bias2, h2, b2))
    del graph
