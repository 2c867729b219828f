"""The summed backward of projections over one input (mxs_nf4_linear_bwd_dx_grads_sum: q, k and
v's input gradients added in one tile loop over their three reductions, with every dA / dB in
the same launch) on the GPU.

Bars: dA and dB bit-equal to the separate launches'; dX against the float64 oracle's
dX_q + dX_k + dX_v within the north star's 1e-2 and no less accurate than the composition;
against the separate launches (each dX rounded to fp16, then added in fp16) within their
roundings (2^-9 of the largest value); the group backward (linear4bit.lora_backward_group with
sum_dx) taking it for q/k/v; graph replays equal to the eager result."""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

S, P = 2.0, 0.05
K = 1536


def _proj(dev, n, M, seed, x, masked=True):
    from mindxsoup_amd.quant import quantize_4bit

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = (torch.randn((n, K), device=dev, generator=g) * 0.02).half()
    packed, st = quantize_4bit(w)
    a = ((torch.rand((16, K), device=dev, generator=g) * 2 - 1) / K ** 0.5).half()
    b = (torch.randn((n, 16), device=dev, generator=g) * 0.01).half()
    dy = torch.randn((M, n), device=dev, generator=g).half()
    keep = (torch.rand((M, K), device=dev, generator=g) >= P).to(torch.uint8) if masked else None
    return dict(packed=packed, st=st, a=a, b=b, dy=dy, keep=keep, x=x, n=n)


def _w(p):
    st = p["st"]
    return O.dequant(O.NF4Weight(st.shape, p["packed"].view(-1).cpu().numpy(),
                                 st.absmax.cpu().numpy(), st.state2.code.cpu().numpy(),
                                 st.state2.absmax.cpu().numpy(), float(st.offset.item())))


def _np(t):
    return t.detach().float().cpu().numpy()


def _operands(ps, ms):
    """Per projection: Hs^T from the forward rows kernel, A^T, dHs finished (and transposed)."""
    from mindxsoup_amd import kernels

    ops = []
    for p in ps:
        h, ht = kernels.lora_h(p["x"], p["a"], S, p["keep"], ms)
        at = p["a"].t().contiguous()
        bt = p["b"].t().contiguous()
        ops.append(dict(ht=ht, at=at, bt=bt))
    dhs = kernels.lora_dh_group([p["dy"] for p in ps], [o["bt"] for o in ops], S)
    for o, (dh, dht) in zip(ops, dhs):
        o.update(dh=dh, dht=dht)
    return ops


@pytest.mark.parametrize("M", [1024, 512, 300, 37, 1200, 1430, 2048])
@pytest.mark.parametrize("shapes", [(1536, 256, 256), (256, 1536)])
def test_sum_equals_separate_and_oracle(cuda, M, shapes):
    """Up to 1152 tokens with the LoRA gradients in the same launch; past that the summed dX
    alone."""
    from mindxsoup_amd import kernels

    print(f"case dx sum M={M} N={shapes}", flush=True)
    ms = 1 / (1 - P)
    x = torch.randn((M, K), device=cuda).half()
    ps = [_proj(cuda, n, M, 70 + i, x) for i, n in enumerate(shapes)]
    grads_in = M <= 1152
    assert kernels.bwd_grads_sum_ok(M, list(shapes), K, 16) == grads_in
    assert kernels.bwd_grads_sum_ok(M, list(shapes), K, 16, grads=False)
    ops = _operands(ps, ms)
    dx, grads = kernels.nf4_linear_bwd_dx_grads_sum(
        [p["dy"] for p in ps], [p["packed"] for p in ps], [p["st"] for p in ps],
        [o["dh"] for o in ops], [o["at"] for o in ops], [o["dht"] for o in ops],
        [o["ht"] for o in ops], x, [p["keep"] for p in ps], ms, grads=grads_in)
    sep = [kernels.nf4_linear_bwd_dx_grads(p["dy"], p["packed"], p["st"], o["dh"], o["at"],
                                           o["dht"], o["ht"], x, p["keep"], ms)
           for p, o in zip(ps, ops)]
    torch.cuda.synchronize()
    if grads_in:
        for (da, db), (_, da1, db1) in zip(grads, sep):
            assert torch.equal(da, da1) and torch.equal(db, db1)
    else:
        assert grads is None
    two = sep[0][0]
    for r in sep[1:]:
        two = two + r[0]
    err_sep = ((dx.float() - two.float()).abs().max() / two.float().abs().max()).item()
    assert err_sep < 2 ** -9, err_sep
    x16 = _np(x).astype(np.float16)
    ref = 0.0
    for p in ps:
        ref = ref + O.lora_bwd(_np(p["dy"]).astype(np.float16), x16, _w(p),
                               _np(p["a"]).astype(np.float16), _np(p["b"]).astype(np.float16), S,
                               p["keep"].cpu().numpy(), P)[0]
    err = O.max_rel(_np(dx), ref)
    print(f"  max_rel vs oracle {err:.2e}, vs separate {err_sep:.2e}", flush=True)
    assert err < 1e-2
    assert err <= O.max_rel(_np(two), ref) * 1.05 + 1e-6


def test_sum_without_masks(cuda):
    """No dropout on any projection: the LoRA terms unmasked; equal to the separate launches'
    sum within their roundings, dA / dB bit-equal."""
    from mindxsoup_amd import kernels

    M = 700
    x = torch.randn((M, K), device=cuda).half()
    ps = [_proj(cuda, n, M, 90 + i, x, masked=False) for i, n in enumerate((1536, 256, 256))]
    ops = _operands(ps, 1.0)
    dx, grads = kernels.nf4_linear_bwd_dx_grads_sum(
        [p["dy"] for p in ps], [p["packed"] for p in ps], [p["st"] for p in ps],
        [o["dh"] for o in ops], [o["at"] for o in ops], [o["dht"] for o in ops],
        [o["ht"] for o in ops], x)
    sep = [kernels.nf4_linear_bwd_dx_grads(p["dy"], p["packed"], p["st"], o["dh"], o["at"],
                                           o["dht"], o["ht"], x) for p, o in zip(ps, ops)]
    torch.cuda.synchronize()
    two = sep[0][0] + sep[1][0] + sep[2][0]
    assert ((dx.float() - two.float()).abs().max() / two.float().abs().max()).item() < 2 ** -9
    for (da, db), (_, da1, db1) in zip(grads, sep):
        assert torch.equal(da, da1) and torch.equal(db, db1)


def test_sum_refuses_other_plans(cuda):
    """Plans the summed launch does not take are refused on the host: one problem, four, rank
    32, K below 1024, a weight height off the K-step, the gate/up shapes (their gradient
    workgroups take another column width), mixed keep masks."""
    from mindxsoup_amd import kernels

    assert not kernels.bwd_grads_sum_ok(1024, [1536], K, 16)
    assert not kernels.bwd_grads_sum_ok(1024, [1536, 256, 256, 256], K, 16)
    assert not kernels.bwd_grads_sum_ok(1024, [1536, 256, 256], K, 32)
    assert not kernels.bwd_grads_sum_ok(1024, [512, 512], 512, 16)
    assert not kernels.bwd_grads_sum_ok(1024, [1536, 200], K, 16)
    assert not kernels.bwd_grads_sum_ok(1024, [8960, 8960], K, 16)
    assert not kernels.bwd_grads_sum_ok(1024, [8960, 8960], K, 16, grads=False)
    assert not kernels.bwd_grads_sum_ok(0, [1536, 256, 256], K, 16)
    # past 1152 tokens the gradient workgroups want more waves than the tile kernel has
    assert not kernels.bwd_grads_sum_ok(1160, [1536, 256, 256], K, 16)
    assert kernels.bwd_grads_sum_ok(1160, [1536, 256, 256], K, 16, grads=False)
    M = 64
    x = torch.randn((M, K), device=cuda).half()
    ps = [_proj(cuda, n, M, 110 + i, x, masked=(i == 0)) for i, n in enumerate((1536, 256))]
    ops = _operands(ps, 1 / (1 - P))
    with pytest.raises(ValueError, match="keep mask"):
        kernels.nf4_linear_bwd_dx_grads_sum(
            [p["dy"] for p in ps], [p["packed"] for p in ps], [p["st"] for p in ps],
            [o["dh"] for o in ops], [o["at"] for o in ops], [o["dht"] for o in ops],
            [o["ht"] for o in ops], x, [p["keep"] for p in ps], 1 / (1 - P))


def _items(cuda, M, seed):
    from mindxsoup_amd import kernels

    ms = 1 / (1 - P)
    x = torch.randn((M, K), device=cuda).half()
    ps = [_proj(cuda, n, M, seed + i, x) for i, n in enumerate((1536, 256, 256))]
    items = []
    for p in ps:
        hp, at, bt = kernels.lora_h_partials(x, p["a"], S, p["keep"], ms, lora_b=p["b"])
        _, ht = kernels.nf4_linear_fwd_hp(x, p["packed"], p["st"], hp, p["b"])
        items.append(dict(dy=p["dy"], x2d=x, keep=p["keep"], ht=ht, at=at, bt=bt,
                          packed=p["packed"], state=p["st"], mask_scale=ms, s=S,
                          wants=(True, True, True)))
    return items


def test_group_backward_takes_the_sum(cuda):
    """lora_backward_group(sum_dx=True) on q/k/v: the summed launch's dx in the first item, None
    in the others, and the separate launches' dA / dB; without sum_dx, three dX."""
    from mindxsoup_amd import kernels
    from mindxsoup_amd.linear4bit import lora_backward_group

    items = _items(cuda, 1024, 130)
    summed = lora_backward_group(items, sum_dx=True)
    apart = lora_backward_group(items)
    dhs = kernels.lora_dh_group([it["dy"] for it in items], [it["bt"] for it in items], S)
    dx, _ = kernels.nf4_linear_bwd_dx_grads_sum(
        [it["dy"] for it in items], [it["packed"] for it in items],
        [it["state"] for it in items], [d[0] for d in dhs], [it["at"] for it in items],
        [d[1] for d in dhs], [it["ht"] for it in items], items[0]["x2d"],
        [it["keep"] for it in items], items[0]["mask_scale"])
    torch.cuda.synchronize()
    assert torch.equal(summed[0][0], dx)
    assert all(r[0] is None for r in summed[1:])
    assert all(r[0] is not None for r in apart)
    for r_s, r_a in zip(summed, apart):
        assert torch.equal(r_s[1], r_a[1]) and torch.equal(r_s[2], r_a[2])


def test_group_backward_past_the_fused_gradients(cuda):
    """At 1430 tokens lora_backward_group(sum_dx=True) takes the summed dX alone, then the
    gradients by weight height: dx within the roundings of the separate launches' sum; dB their
    bits; dA the bits of mxs_lora_grads over the finished dHs (the separate route at this size
    takes dHs from slice partials, added in another order: within 1e-3 of it)."""
    from mindxsoup_amd import kernels
    from mindxsoup_amd.linear4bit import lora_backward_group

    items = _items(cuda, 1430, 140)
    assert not kernels.bwd_grads_sum_ok(1430, [1536, 256, 256], K, 16)
    summed = lora_backward_group(items, sum_dx=True)
    apart = lora_backward_group(items)
    dhs = kernels.lora_dh_group([it["dy"] for it in items], [it["bt"] for it in items], S)
    torch.cuda.synchronize()
    two = apart[0][0] + apart[1][0] + apart[2][0]
    assert ((summed[0][0].float() - two.float()).abs().max()
            / two.float().abs().max()).item() < 2 ** -9
    assert all(r[0] is None for r in summed[1:])
    for it, (_, dht), r_s, r_a in zip(items, dhs, summed, apart):
        da, db = kernels.lora_grads(dht, it["ht"], it["x2d"], it["dy"], it["keep"],
                                    it["mask_scale"])
        assert torch.equal(r_s[1], da) and torch.equal(r_s[2], db)
        assert torch.equal(r_s[2], r_a[2])
        assert O.max_rel(_np(r_s[1]), _np(r_a[1]).astype(np.float64)) < 1e-3


def test_summed_backward_replays_in_a_graph(cuda):
    """The summed backward captured in a HIP graph: every replay, with eager work between them,
    equals the eager result bit for bit."""
    from mindxsoup_amd.linear4bit import lora_backward_group

    items = _items(cuda, 512, 150)
    eager = lora_backward_group(items, sum_dx=True)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        lora_backward_group(items, sum_dx=True)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = lora_backward_group(items, sum_dx=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0][0], eager[0][0])
        for r_o, r_e in zip(out, eager):
            assert torch.equal(r_o[1], r_e[1]) and torch.equal(r_o[2], r_e[2])
        lora_backward_group(items, sum_dx=True)  # eager work between the replays
        torch.cuda.synchronize()
