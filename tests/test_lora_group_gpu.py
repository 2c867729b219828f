"""The grouped LoRA row products (mxs_lora_h_partials_group, mxs_lora_dh_partials_group): several
projections over the same tokens in one launch give the bits of one launch each.  Groups mix
reduction lengths (1536 and 8960), so their problems run with different slice and wave counts
inside one launch."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, M, K, N, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn((M, K), device=dev, generator=g).half()
    a = ((torch.rand((16, K), device=dev, generator=g) * 2 - 1) / np.sqrt(K)).half()
    b = (torch.randn((N, 16), device=dev, generator=g) * 0.01).half()
    dy = torch.randn((M, N), device=dev, generator=g).half()
    keep = (torch.rand((M, K), device=dev, generator=g) >= 0.05).to(torch.uint8)
    return x, a, b, dy, keep


# (K, N) per projection: q/k/v of a layer, gate/up, and a mixed group with down's 8960
GROUPS = {
    "qkv": [(1536, 1536), (1536, 256), (1536, 256)],
    "gate_up": [(1536, 8960), (1536, 8960)],
    "mixed": [(8960, 1536), (1536, 256), (1536, 8960), (256, 1536)],
}


@pytest.mark.parametrize("group", sorted(GROUPS))
@pytest.mark.parametrize("M", [1024, 300, 37])
def test_grouped_rows_equal_separate_launches(cuda, group, M):
    from mindxsoup_amd import kernels

    print(f"case lora group {group} M={M}", flush=True)
    shapes = GROUPS[group]
    probs = [_inputs(cuda, M, K, N, 100 + i) for i, (K, N) in enumerate(shapes)]
    if group != "mixed":  # projections of one group share their input, as in the model
        probs = [(probs[0][0],) + p[1:] for p in probs]
    s, ms = 2.0, 1 / 0.95
    sep = [kernels.lora_h_partials(x, a, s, keep, ms, lora_b=b) for x, a, b, _, keep in probs]
    grp = kernels.lora_h_partials_group([p[0] for p in probs], [p[1] for p in probs], s,
                                        [p[4] for p in probs], ms, [p[2] for p in probs])
    bts = [o[2] for o in sep]
    dsep = [kernels.lora_dh_partials(p[3], bt, s) for p, bt in zip(probs, bts)]
    dgrp = kernels.lora_dh_partials_group([p[3] for p in probs], bts, s)
    torch.cuda.synchronize()
    for (hp1, at1, bt1), (hp2, at2, bt2) in zip(sep, grp):
        assert torch.equal(hp1, hp2) and torch.equal(at1, at2) and torch.equal(bt1, bt2)
    for d1, d2 in zip(dsep, dgrp):
        assert torch.equal(d1, d2)


def test_grouped_rows_without_masks_or_side_outputs(cuda):
    from mindxsoup_amd import kernels

    M = 256
    probs = [_inputs(cuda, M, K, 256, 7 + K) for K in (1536, 512)]
    s = 0.5
    sep = [kernels.lora_h_partials(x, a, s) for x, a, _, _, _ in probs]
    grp = kernels.lora_h_partials_group([p[0] for p in probs], [p[1] for p in probs], s)
    torch.cuda.synchronize()
    for (hp1, at1, _), (hp2, at2, bt2) in zip(sep, grp):
        assert torch.equal(hp1, hp2) and torch.equal(at1, at2) and bt2 is None


@pytest.mark.parametrize("M", [1024, 300])
def test_grouped_finished_dh_equals_one_launch_dh(cuda, M):
    """mxs_lora_dh_group against lora_dh(..., one_launch=True) per projection (the backward of
    the projections whose dX GEMM carries the weight gradients): dh and dht bit for bit."""
    from mindxsoup_amd import kernels

    probs = [_inputs(cuda, M, K, N, 40 + i) for i, (K, N) in enumerate(GROUPS["qkv"]
                                                                      + [(8960, 1536)])]
    bts = [b.t().contiguous() for _, _, b, _, _ in probs]
    sep = [kernels.lora_dh(p[3], None, 2.0, lora_bt=bt, one_launch=True)
           for p, bt in zip(probs, bts)]
    grp = kernels.lora_dh_group([p[3] for p in probs], bts, 2.0)
    torch.cuda.synchronize()
    for (d1, t1), (d2, t2) in zip(sep, grp):
        assert torch.equal(d1, d2) and torch.equal(t1, t2)


def _nf4(dev, n, k, seed, bias=False):
    from mindxsoup_amd.linear4bit import Linear4bit

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).half()
    b = (torch.randn((n,), device=dev, generator=g) * 0.1).half() if bias else None
    return Linear4bit.from_weight(w, b)


@pytest.mark.parametrize("M", [1024, 300, 37])
@pytest.mark.parametrize("lora", [True, False])
def test_grouped_qkv_gemm_equals_separate(cuda, M, lora):
    """mxs_nf4_linear_fwd_hp_group over q [1536], k [256], v [256] (K = 1536, one x) against
    each projection's own launch of the same tile configuration, bit for bit; and within 1e-2 of
    the planned single launches (k and v alone plan split-K tiles and a reduce)."""
    from mindxsoup_amd import kernels

    print(f"case qkv gemm group M={M} lora={lora}", flush=True)
    K = 1536
    layers = [_nf4(cuda, n, K, 300 + i, bias=(i == 0)) for i, n in enumerate((1536, 256, 256))]
    probs = [_inputs(cuda, M, K, L.out_features, 310 + i) for i, L in enumerate(layers)]
    x = probs[0][0]
    packeds = [L.weight.data.view(-1, 1) for L in layers]
    states = [L.weight.quant_state for L in layers]
    biases = [L.bias for L in layers]
    hps = bs = None
    if lora:
        outs = kernels.lora_h_partials_group([x] * 3, [p[1] for p in probs], 2.0,
                                             [p[4] for p in probs], 1 / 0.95,
                                             [p[2] for p in probs])
        hps, bs = [o[0] for o in outs], [p[2] for p in probs]
    grp = kernels.nf4_linear_fwd_hp_group([x] * 3, packeds, states, hps, bs, biases)
    for i in range(3):
        if lora:
            y1, ht1 = kernels.nf4_linear_fwd_hp(x, packeds[i], states[i], hps[i], bs[i],
                                                biases[i], cfg=10, splits=1)
            y0, _ = kernels.nf4_linear_fwd_hp(x, packeds[i], states[i], hps[i], bs[i],
                                              biases[i])
        else:
            y1 = kernels.nf4_linear_fwd(x, packeds[i], states[i], biases[i], cfg=10, splits=1)
            y0, ht1 = kernels.nf4_linear_fwd(x, packeds[i], states[i], biases[i]), None
        torch.cuda.synchronize()
        y2, ht2 = grp[i]
        assert torch.equal(y2, y1), i
        assert (ht2 is None) == (ht1 is None) and (ht1 is None or torch.equal(ht2, ht1))
        err = (y2.float() - y0.float()).abs().max() / y0.float().abs().max()
        assert err < 1e-2, (i, float(err))


@pytest.mark.parametrize("M", [1024, 512, 300])
def test_grouped_qkv_backward_equals_separate(cuda, M):
    """mxs_nf4_linear_bwd_dx_grads_group over v, k, q (K = 1536) against each projection's
    mxs_nf4_linear_bwd_dx_grads: dX, dA and dB bit for bit."""
    from mindxsoup_amd import kernels

    print(f"case qkv backward group M={M}", flush=True)
    K = 1536
    layers = [_nf4(cuda, n, K, 400 + i) for i, n in enumerate((256, 256, 1536))]
    Ns = [L.out_features for L in layers]
    assert kernels.bwd_grads_group_ok(M, Ns, K, 16)
    probs = [_inputs(cuda, M, K, n, 410 + i) for i, n in enumerate(Ns)]
    x = probs[0][0]
    s, ms = 2.0, 1 / 0.95
    packeds = [L.weight.data.view(-1, 1) for L in layers]
    states = [L.weight.quant_state for L in layers]
    saved = []
    for (_, a, b, _, keep), P, st in zip(probs, packeds, states):
        h, ht = kernels.lora_h(x, a, s, keep, ms)
        saved.append((ht, a.t().contiguous(), b.t().contiguous()))
    dhs = kernels.lora_dh_group([p[3] for p in probs], [sv[2] for sv in saved], s)
    sep = [kernels.nf4_linear_bwd_dx_grads(p[3], P, st, dh, sv[1], dht, sv[0], x, p[4], ms)
           for p, P, st, (dh, dht), sv in zip(probs, packeds, states, dhs, saved)]
    grp = kernels.nf4_linear_bwd_dx_grads_group(
        [p[3] for p in probs], packeds, states, [d[0] for d in dhs], [sv[1] for sv in saved],
        [d[1] for d in dhs], [sv[0] for sv in saved], [x] * 3, [p[4] for p in probs], ms)
    torch.cuda.synchronize()
    for (dx1, da1, db1), (dx2, da2, db2) in zip(sep, grp):
        assert torch.equal(dx1, dx2) and torch.equal(da1, da2) and torch.equal(db1, db2)


@pytest.mark.parametrize("M", [1024, 37])
def test_backward_group_equals_lora_backward(cuda, M):
    """linear4bit.lora_backward_group over gate and up (dX split-K GEMMs, dA / dB in one launch)
    and over v, k, q (the grouped dX + gradients launch) against lora_backward on each: dX, dA,
    dB bit for bit."""
    from mindxsoup_amd import kernels
    from mindxsoup_amd.linear4bit import lora_backward, lora_backward_group

    print(f"case backward group M={M}", flush=True)
    s, ms = 2.0, 1 / 0.95
    for shapes in ([(8960, 1536), (8960, 1536)], [(256, 1536), (256, 1536), (1536, 1536)]):
        layers = [_nf4(cuda, n, k, 500 + i) for i, (n, k) in enumerate(shapes)]
        probs = [_inputs(cuda, M, k, n, 510 + i) for i, (n, k) in enumerate(shapes)]
        x = probs[0][0]
        items = []
        for (n, k), L, (_, a, b, dy, keep) in zip(shapes, layers, probs):
            hp, at, bt = kernels.lora_h_partials(x, a, s, keep, ms, lora_b=b)
            _, ht = kernels.nf4_linear_fwd_hp(x, L.weight.data.view(-1, 1),
                                              L.weight.quant_state, hp, b)
            items.append(dict(dy=dy, x2d=x, keep=keep, ht=ht, at=at, bt=bt,
                              packed=L.weight.data.view(-1, 1), state=L.weight.quant_state,
                              mask_scale=ms, s=s, wants=(True, True, True)))
        want = [lora_backward(it["dy"], it["x2d"], it["keep"], it["ht"], it["at"], it["bt"],
                              it["packed"], it["state"], ms, s) for it in items]
        got = lora_backward_group(items)
        torch.cuda.synchronize()
        for w, g in zip(want, got):
            assert all(torch.equal(a_, b_) for a_, b_ in zip(w, g))


def test_grads_group_equals_separate(cuda):
    from mindxsoup_amd import kernels

    M, K, N = 700, 1536, 8960
    probs = [_inputs(cuda, M, K, N, 600 + i) for i in range(2)]
    dhts, hts = [], []
    for x, a, b, dy, keep in probs:
        _, ht = kernels.lora_h(x, a, 2.0, keep, 1 / 0.95)
        _, dht = kernels.lora_dh(dy, b, 2.0)
        dhts.append(dht)
        hts.append(ht)
    sep = [kernels.lora_grads(dht, ht, p[0], p[3], p[4], 1 / 0.95)
           for dht, ht, p in zip(dhts, hts, probs)]
    grp = kernels.lora_grads_group(dhts, hts, [p[0] for p in probs], [p[3] for p in probs],
                                   [p[4] for p in probs], 1 / 0.95)
    torch.cuda.synchronize()
    for (a1, b1), (a2, b2) in zip(sep, grp):
        assert torch.equal(a1, a2) and torch.equal(b1, b2)


def test_grouped_paths_without_tokens(cuda):
    """Zero tokens through every grouped entry: nothing computed, empty outputs, zero LoRA
    gradients (an empty reduction), as the single-projection entries give."""
    from mindxsoup_amd import kernels
    from mindxsoup_amd.linear4bit import lora_backward_group

    K = 1536
    layers = [_nf4(cuda, n, K, 700 + i) for i, n in enumerate((8960, 8960))]
    x = torch.empty((0, K), device=cuda, dtype=torch.float16)
    a = [(torch.rand((16, K), device=cuda) * 0.05).half() for _ in layers]
    b = [(torch.randn((L.out_features, 16), device=cuda) * 0.01).half() for L in layers]
    outs = kernels.lora_h_partials_group([x, x], a, 2.0, None, 1.0, b)
    ys = kernels.nf4_linear_fwd_hp_group([x, x], [L.weight.data.view(-1, 1) for L in layers],
                                         [L.weight.quant_state for L in layers],
                                         [o[0] for o in outs], b)
    assert all(y.shape == (0, L.out_features) for (y, _), L in zip(ys, layers))
    items = [dict(dy=torch.empty((0, L.out_features), device=cuda, dtype=torch.float16), x2d=x,
                  keep=None, ht=ht, at=o[1], bt=o[2], packed=L.weight.data.view(-1, 1),
                  state=L.weight.quant_state, mask_scale=1.0, s=2.0, wants=(True, True, True))
             for L, o, (_, ht) in zip(layers, outs, ys)]
    res = lora_backward_group(items)
    torch.cuda.synchronize()
    for (dx, da, db), L in zip(res, layers):
        assert dx.shape == (0, K)
        assert da.shape == (16, K) and not da.any()
        assert db.shape == (L.out_features, 16) and not db.any()


def test_dx_grads_without_tokens(cuda):
    """mxs_nf4_linear_bwd_dx_grads with zero tokens: empty dX, zero dA and dB."""
    from mindxsoup_amd import kernels

    L = _nf4(cuda, 1536, 1536, 720)
    e = lambda *shape: torch.empty(shape, device=cuda, dtype=torch.float16)  # noqa: E731
    dx, da, db = kernels.nf4_linear_bwd_dx_grads(e(0, 1536), L.weight.data.view(-1, 1),
                                                 L.weight.quant_state, e(0, 16), e(1536, 16),
                                                 e(16, 0), e(16, 0), e(0, 1536))
    torch.cuda.synchronize()
    assert dx.shape == (0, 1536) and not da.any() and not db.any()
