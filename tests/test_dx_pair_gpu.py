"""The summed input gradient of two projections over one input (mxs_nf4_linear_bwd_dx_hp_pair:
gate and up of the MLP in one split-K launch and one reduce) on the GPU.

Bars: against the float64 oracle's dX_gate + dX_up within the north star's 1e-2; against the two
separate launches (each dX rounded to fp16, then added in fp16) within their roundings (1.5 fp16
ulps of the largest value); the dHs^T side outputs bit-equal to the separate launches'; and the
group backward (linear4bit.lora_backward_group with sum_dx) taking it only where it applies."""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

S, P = 2.0, 0.05


def _proj(dev, n, k, M, seed, x):
    from mindxsoup_amd.quant import quantize_4bit

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).half()
    packed, st = quantize_4bit(w)
    a = ((torch.rand((16, k), device=dev, generator=g) * 2 - 1) / k ** 0.5).half()
    b = (torch.randn((n, 16), device=dev, generator=g) * 0.01).half()
    dy = torch.randn((M, n), device=dev, generator=g).half()
    keep = (torch.rand((M, k), device=dev, generator=g) >= P).to(torch.uint8)
    return dict(packed=packed, st=st, a=a, b=b, dy=dy, keep=keep, x=x, n=n, k=k)


def _w(p):
    st = p["st"]
    return O.dequant(O.NF4Weight(st.shape, p["packed"].view(-1).cpu().numpy(),
                                 st.absmax.cpu().numpy(), st.state2.code.cpu().numpy(),
                                 st.state2.absmax.cpu().numpy(), float(st.offset.item())))


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("M", [1024, 300, 37])
def test_pair_sums_the_two_input_gradients(cuda, M):
    from mindxsoup_amd import kernels

    print(f"case dx pair M={M}", flush=True)
    x = torch.randn((M, 1536), device=cuda).half()
    ps = [_proj(cuda, 8960, 1536, M, 30 + i, x) for i in range(2)]
    assert kernels.bwd_dx_pair_ok(M, 8960, 8960, 1536)
    dhps = [kernels.lora_dh_partials(p["dy"], p["b"].t().contiguous(), S) for p in ps]
    ats = [p["a"].t().contiguous() for p in ps]
    dx, dhts = kernels.nf4_linear_bwd_dx_hp_pair(
        [p["dy"] for p in ps], [p["packed"] for p in ps], [p["st"] for p in ps], dhps, ats,
        [p["keep"] for p in ps], 1 / (1 - P))
    sep = [kernels.nf4_linear_bwd_dx_hp(p["dy"], p["packed"], p["st"], dhp, at, p["keep"],
                                        1 / (1 - P)) for p, dhp, at in zip(ps, dhps, ats)]
    for (_, dht_sep), dht in zip(sep, dhts):
        assert torch.equal(dht, dht_sep)
    two = sep[0][0] + sep[1][0]
    err_sep = ((dx.float() - two.float()).abs().max() / two.float().abs().max()).item()
    assert 0 < err_sep < 2 ** -9, err_sep
    x16 = _np(x).astype(np.float16)
    ref = 0.0
    for p in ps:
        ref = ref + O.lora_bwd(_np(p["dy"]).astype(np.float16), x16, _w(p),
                               _np(p["a"]).astype(np.float16), _np(p["b"]).astype(np.float16), S,
                               p["keep"].cpu().numpy(), P)[0]
    err = O.max_rel(_np(dx), ref)
    print(f"  max_rel vs oracle {err:.2e}, vs separate {err_sep:.2e}", flush=True)
    assert err < 1e-2
    # the summed launch is no less accurate than the two rounded ones
    assert err <= O.max_rel(_np(two), ref) * 1.05 + 1e-6


def test_pair_refuses_other_plans(cuda):
    """Shapes whose own plan is not the narrow-output split kernel (q/o: 1536 x 1536) are
    refused on the host."""
    from mindxsoup_amd import kernels

    assert not kernels.bwd_dx_pair_ok(1024, 1536, 1536, 1536)
    assert not kernels.bwd_dx_pair_ok(1024, 8960, 8960, 1000)
    x = torch.randn((64, 1536), device=cuda).half()
    ps = [_proj(cuda, 1536, 1536, 64, 40 + i, x) for i in range(2)]
    dhps = [kernels.lora_dh_partials(p["dy"], p["b"].t().contiguous(), S) for p in ps]
    with pytest.raises(ValueError, match="does not take"):
        kernels.nf4_linear_bwd_dx_hp_pair([p["dy"] for p in ps], [p["packed"] for p in ps],
                                          [p["st"] for p in ps], dhps,
                                          [p["a"].t().contiguous() for p in ps])


def test_group_backward_sums(cuda):
    """lora_backward_group(sum_dx=True) gives one dx in the first item, the separate launches'
    sum within their roundings, and the separate launches' LoRA gradients: on gate and up from
    the pair, on q/k/v from the summed tile loop (tests/test_dx_sum_gpu.py)."""
    from mindxsoup_amd import kernels
    from mindxsoup_amd.linear4bit import lora_backward_group

    M = 512
    x = torch.randn((M, 1536), device=cuda).half()
    for shapes, paired in (([8960, 8960], True), ([1536, 256, 256], False)):
        ps = [_proj(cuda, n, 1536, M, 50 + i, x) for i, n in enumerate(shapes)]
        items = []
        for p in ps:
            hp, at, bt = kernels.lora_h_partials(x, p["a"], S, p["keep"], 1 / (1 - P),
                                                 lora_b=p["b"])
            _, ht = kernels.nf4_linear_fwd_hp(x, p["packed"], p["st"], hp, p["b"])
            items.append(dict(dy=p["dy"], x2d=x, keep=p["keep"], ht=ht, at=at, bt=bt,
                              packed=p["packed"], state=p["st"], mask_scale=1 / (1 - P), s=S,
                              wants=(True, True, True)))
        summed = lora_backward_group(items, sum_dx=True)
        apart = lora_backward_group(items)
        assert all(r[0] is None for r in summed[1:])
        for r_s, r_a in zip(summed, apart):
            assert torch.equal(r_s[1], r_a[1]) and torch.equal(r_s[2], r_a[2])
        two = apart[0][0]
        for r in apart[1:]:
            two = two + r[0]
        err = ((summed[0][0].float() - two.float()).abs().max() / two.float().abs().max()).item()
        assert 0 < err < 2 ** -9, (paired, err)



@pytest.mark.parametrize("M", [1024, 300, 768, 900])
def test_forward_pair_equals_two_launches(cuda, M):
    """gate and up forward in one launch (mxs_nf4_linear_fwd_hp_pair) give the bits of two
    nf4_linear_fwd_hp launches, y and the transposed LoRA operand, with a bias and without;
    within the north star's 1e-2 of the oracle.  300 tokens: one width (grid z selects the
    projection); 1024 and 900 (a partial last row band): 256x160 tiles up to column 3840 and
    256x128 tiles past it in one launch; 768: the split at column 640."""
    from mindxsoup_amd import kernels

    print(f"case fwd pair M={M}", flush=True)
    x = torch.randn((M, 1536), device=cuda).half()
    ps = [_proj(cuda, 8960, 1536, M, 40 + i, x) for i in range(2)]
    assert kernels.fwd_pair_ok(M, 8960, 8960, 1536)
    assert not kernels.fwd_pair_ok(M, 1536, 1536, 1536) and not kernels.fwd_pair_ok(M, 8960, 256, 1536)
    rows = kernels.lora_h_partials_group([x, x], [p["a"] for p in ps], S, [p["keep"] for p in ps],
                                         1 / (1 - P), [p["b"] for p in ps])
    bias = [torch.randn((8960,), device=cuda).half(), None]
    for biases in (None, bias):
        two = [kernels.nf4_linear_fwd_hp(x, p["packed"], p["st"], r[0], p["b"],
                                         None if biases is None else biases[i])
               for i, (p, r) in enumerate(zip(ps, rows))]
        pair = kernels.nf4_linear_fwd_hp_pair(x, [p["packed"] for p in ps], [p["st"] for p in ps],
                                              [r[0] for r in rows], [p["b"] for p in ps], biases)
        for (y2, t2), (y1, t1) in zip(two, pair):
            assert torch.equal(y1, y2) and torch.equal(t1, t2)
    x16 = _np(x).astype(np.float16)
    for p, (y, _) in zip(ps, pair):
        ref = O.lora_fwd(x16, _w(p), _np(p["a"]).astype(np.float16),
                         _np(p["b"]).astype(np.float16), S, p["keep"].cpu().numpy(), P)
        if p is ps[0]:
            ref = ref + _np(bias[0])
        assert O.max_rel(_np(y), ref) < 1e-2


@pytest.mark.parametrize("M", [1024, 300, 37])
def test_pair_with_gradients_equals_pair_then_grads(cuda, M):
    """mxs_nf4_linear_bwd_dx_hp_pair_grads (the pair GEMM, then its reduce and both projections'
    dA / dB in one launch) gives the bits of mxs_nf4_linear_bwd_dx_hp_pair followed by
    mxs_lora_grads_group: dX, the dHs^T side outputs and the four gradients; the gradients within
    the north star's 1e-2 of float64 products of the same operands."""
    from mindxsoup_amd import kernels

    print(f"case dx pair grads M={M}", flush=True)
    x = torch.randn((M, 1536), device=cuda).half()
    ps = [_proj(cuda, 8960, 1536, M, 60 + i, x) for i in range(2)]
    rows = kernels.lora_h_partials_group([x, x], [p["a"] for p in ps], S, [p["keep"] for p in ps],
                                         1 / (1 - P), [p["b"] for p in ps])
    hts = [kernels.nf4_linear_fwd_hp(x, p["packed"], p["st"], r[0], p["b"])[1]
           for p, r in zip(ps, rows)]
    dhps = [kernels.lora_dh_partials(p["dy"], p["b"].t().contiguous(), S) for p in ps]
    ats = [p["a"].t().contiguous() for p in ps]
    args = ([p["dy"] for p in ps], [p["packed"] for p in ps], [p["st"] for p in ps], dhps, ats)
    keeps = [p["keep"] for p in ps]
    dx, dhts, grads = kernels.nf4_linear_bwd_dx_hp_pair_grads(*args, hts, x, keeps, 1 / (1 - P))
    dx1, dhts1 = kernels.nf4_linear_bwd_dx_hp_pair(*args, keeps, 1 / (1 - P))
    grads1 = kernels.lora_grads_group(dhts1, hts, [x, x], [p["dy"] for p in ps], keeps,
                                      1 / (1 - P))
    torch.cuda.synchronize()
    assert torch.equal(dx, dx1)
    for t, t1 in zip(dhts, dhts1):
        assert torch.equal(t, t1)
    for (da, db), (da1, db1) in zip(grads, grads1):
        assert torch.equal(da, da1) and torch.equal(db, db1)
    for p, (da, db), dht, ht in zip(ps, grads, dhts, hts):
        xk = O.dropout_fp16(_np(x).astype(np.float16), p["keep"].cpu().numpy(), P)
        ref_a = _np(dht[:, :M]).astype(np.float64) @ xk.astype(np.float64)
        ref_b = _np(p["dy"]).astype(np.float64).T @ _np(ht[:, :M]).astype(np.float64).T
        assert O.max_rel(_np(da), ref_a) < 1e-2
        assert O.max_rel(_np(db), ref_b) < 1e-2


def test_pair_with_gradients_without_masks_and_refused_shapes(cuda):
    """No dropout (masks None): the pair with gradients still gives the bits of the pair then the
    gradient group; two projections whose gradients would take different columns per lane
    (8960 and 4096 outputs over 1536 inputs) are refused by the library, not computed."""
    from mindxsoup_amd import kernels

    M = 512
    x = torch.randn((M, 1536), device=cuda).half()
    ps = [_proj(cuda, 8960, 1536, M, 70 + i, x) for i in range(2)]
    rows = kernels.lora_h_partials_group([x, x], [p["a"] for p in ps], S, None, 1.0,
                                         [p["b"] for p in ps])
    hts = [kernels.nf4_linear_fwd_hp(x, p["packed"], p["st"], r[0], p["b"])[1]
           for p, r in zip(ps, rows)]
    dhps = [kernels.lora_dh_partials(p["dy"], p["b"].t().contiguous(), S) for p in ps]
    args = ([p["dy"] for p in ps], [p["packed"] for p in ps], [p["st"] for p in ps], dhps,
            [p["a"].t().contiguous() for p in ps])
    dx, dhts, grads = kernels.nf4_linear_bwd_dx_hp_pair_grads(*args, hts, x)
    dx1, dhts1 = kernels.nf4_linear_bwd_dx_hp_pair(*args)
    grads1 = kernels.lora_grads_group(dhts1, hts, [x, x], [p["dy"] for p in ps])
    torch.cuda.synchronize()
    assert torch.equal(dx, dx1)
    for (da, db), (da1, db1) in zip(grads, grads1):
        assert torch.equal(da, da1) and torch.equal(db, db1)
    q = [ps[0], _proj(cuda, 4096, 1536, M, 72, x)]
    if kernels.bwd_dx_pair_ok(M, 8960, 4096, 1536):
        dhq = [kernels.lora_dh_partials(p["dy"], p["b"].t().contiguous(), S) for p in q]
        htq = [torch.zeros_like(hts[0]) for _ in q]
        with pytest.raises(RuntimeError):
            kernels.nf4_linear_bwd_dx_hp_pair_grads(
                [p["dy"] for p in q], [p["packed"] for p in q], [p["st"] for p in q], dhq,
                [p["a"].t().contiguous() for p in q], htq, x)


@pytest.mark.parametrize("M,N,K", [(1024, 6144, 1536), (512, 11008, 4096), (1024, 14336, 4096)])
def test_forward_pair_mixed_widths_other_shapes(cuda, M, N, K):
    """Other MLP widths: where the launch cuts the columns into 256x160 and 256x128 tiles (at
    column 640, or 10240 for 14336 outputs at 1024 tokens) the results are still the bits of two
    one-projection launches."""
    from mindxsoup_amd import kernels

    print(f"case fwd pair mixed M={M} N={N} K={K}", flush=True)
    x = torch.randn((M, K), device=cuda).half()
    ps = [_proj(cuda, N, K, M, 80 + i, x) for i in range(2)]
    assert kernels.fwd_pair_ok(M, N, N, K)
    rows = kernels.lora_h_partials_group([x, x], [p["a"] for p in ps], S, [p["keep"] for p in ps],
                                         1 / (1 - P), [p["b"] for p in ps])
    two = [kernels.nf4_linear_fwd_hp(x, p["packed"], p["st"], r[0], p["b"])
           for p, r in zip(ps, rows)]
    pair = kernels.nf4_linear_fwd_hp_pair(x, [p["packed"] for p in ps], [p["st"] for p in ps],
                                          [r[0] for r in rows], [p["b"] for p in ps])
    for (y2, t2), (y1, t1) in zip(two, pair):
        assert torch.equal(y1, y2) and torch.equal(t1, t2)
