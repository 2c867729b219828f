"""The SwiGLU fused into the NF4 GEMM epilogues (mxs_nf4_linear_fwd_glu, mxs_nf4_linear_bwd_dx_glu)
and the fp16 MLP built on them (mindxsoup_amd/mlp.py, the interface of solution/mlp.py).

Bars: the fused epilogues give the bits of the unfused sequence (the GEMM, then mxs_silu_mul /
mxs_silu_mul_bwd: the epilogue rounds the product to fp16 before the SwiGLU reads it, as the
separate kernel does); the MLP block against a float64 composition of the oracle (NF4 decode,
peft LoRA products, the SwiGLU restatement) within max relative error 1e-2; the fused block
equal bit for bit to the three projections and silu_mul called one by one, forward and backward,
except the input gradient: the fused block adds gate's and up's parts in fp32 inside one launch
and rounds once, where the composition rounds each part and adds them in fp16.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _layer(dev, n, k, seed, bias=False):
    from mindxsoup_amd.linear4bit import Linear4bit

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).half()
    b = (torch.randn((n,), device=dev, generator=g) * 0.1).half() if bias else None
    return Linear4bit.from_weight(w, b)


def _w_oracle(layer):
    st = layer.weight.quant_state
    q = O.NF4Weight(st.shape, layer.weight.data.view(-1).cpu().numpy(), st.absmax.cpu().numpy(),
                    st.state2.code.cpu().numpy(), st.state2.absmax.cpu().numpy(),
                    float(st.offset.item()))
    return O.dequant(q)


def _np(t):
    return t.detach().cpu().numpy()


def _lora(dev, M, K, N, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn((M, K), device=dev, generator=g).half()
    a = ((torch.rand((16, K), device=dev, generator=g) * 2 - 1) / np.sqrt(K)).half()
    b = (torch.randn((N, 16), device=dev, generator=g) * 0.01).half()
    keep = (torch.rand((M, K), device=dev, generator=g) >= 0.05).to(torch.uint8)
    return x, a, b, keep


def _bits_equal(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


# up_proj shapes [N, K]: the model's (8960 x 1536, one 256x160 tile per CU), a partial last
# column tile (4224 = 26.4 x 160), a mid width (1536: 128x128 tiles, 8 producer waves), and a
# long reduction that plans split-K (the reduce kernel then applies the SwiGLU)
@pytest.mark.parametrize("n,k,M", [(8960, 1536, 1024), (8960, 1536, 300), (8960, 1536, 37),
                                   (4224, 1536, 200), (1536, 1536, 300), (1536, 8960, 512)])
@pytest.mark.parametrize("lora,bias", [(True, False), (False, True)])
def test_fwd_glu_equals_gemm_then_silu_mul(cuda, n, k, M, lora, bias):
    from mindxsoup_amd import kernels

    print(f"case fwd_glu n={n} k={k} M={M} lora={lora} bias={bias}", flush=True)
    assert kernels.glu_fused(M, n, k, False)
    layer = _layer(cuda, n, k, 61, bias)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    x, a, b, keep = _lora(cuda, M, k, n, 62)
    gate = (torch.randn((M, n), device=cuda) * 2).half()
    if lora:
        hp, _, _ = kernels.lora_h_partials(x, a, 2.0, keep, 1 / 0.95, lora_b=b)
        y1, ht1 = kernels.nf4_linear_fwd_hp(x, packed, st, hp, b, layer.bias)
        y2, h2, ht2 = kernels.nf4_linear_fwd_glu(x, packed, st, gate, hp, b, layer.bias)
    else:
        y1, ht1 = kernels.nf4_linear_fwd(x, packed, st, layer.bias), None
        y2, h2, ht2 = kernels.nf4_linear_fwd_glu(x, packed, st, gate, bias=layer.bias)
    h1 = kernels.silu_mul(gate, y1)
    torch.cuda.synchronize()
    assert _bits_equal(y2, y1) and _bits_equal(h2, h1)
    assert (ht2 is None) == (ht1 is None) and (ht1 is None or torch.equal(ht2, ht1))
    if not lora:  # the block's value against float64 decode-then-matmul and the oracle SwiGLU
        w = _w_oracle(layer)
        ref_y = O.linear_fwd(_np(x), w, _np(layer.bias) if bias else None)
        assert O.max_rel(_np(y2).astype(np.float64), ref_y) < TOL
        ref_h = O.silu_mul(_np(gate), ref_y.astype(np.float16))
        assert O.max_rel(_np(h2).astype(np.float64), ref_h.astype(np.float64)) < TOL


# down_proj shapes [N, K] (dX is [M, K]): the model's (1536 x 8960), a partial column tile, a
# mid width (128x128 tiles, 8 producer waves), and gate_proj's transpose (8960 x 1536), whose dX
# plans split-K
@pytest.mark.parametrize("n,k,M", [(1536, 8960, 1024), (1536, 8960, 300), (1536, 4224, 37),
                                   (1536, 1536, 300), (8960, 1536, 512)])
@pytest.mark.parametrize("lora", [True, False])
def test_bwd_dx_glu_equals_gemm_then_silu_mul_bwd(cuda, n, k, M, lora):
    from mindxsoup_amd import kernels

    print(f"case bwd_dx_glu n={n} k={k} M={M} lora={lora}", flush=True)
    assert kernels.glu_fused(M, n, k, True)
    layer = _layer(cuda, n, k, 71)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    h, a, b, keep = _lora(cuda, M, k, n, 72)
    dy = (torch.randn((M, n), device=cuda) * 0.5).half()
    gate = (torch.randn((M, k), device=cuda) * 2).half()
    up = (torch.randn((M, k), device=cuda) * 2).half()
    g1, u1, g2, u2 = gate.clone(), up.clone(), gate.clone(), up.clone()
    if lora:
        at, bt = a.t().contiguous(), b.t().contiguous()
        dhp = kernels.lora_dh_partials(dy, bt, 2.0)
        dh, dht1 = kernels.nf4_linear_bwd_dx_hp(dy, packed, st, dhp, at, keep, 1 / 0.95)
        dht2 = kernels.nf4_linear_bwd_dx_glu_(dy, packed, st, g2, u2, dhp, at, keep, 1 / 0.95)
    else:
        dh, dht1 = kernels.nf4_linear_bwd_dx(dy, packed, st), None
        dht2 = kernels.nf4_linear_bwd_dx_glu_(dy, packed, st, g2, u2)
    kernels.silu_mul_bwd_(dh, g1, u1)
    torch.cuda.synchronize()
    assert _bits_equal(g2, g1) and _bits_equal(u2, u1)
    assert (dht2 is None) == (dht1 is None) and (dht1 is None or torch.equal(dht2, dht1))
    if not lora:
        ref_dh = O.linear_bwd_dx(_np(dy), _w_oracle(layer))
        ref_dg, ref_du = O.silu_mul_bwd(ref_dh.astype(np.float16), _np(gate), _np(up))
        assert O.max_rel(_np(g2).astype(np.float64), ref_dg.astype(np.float64)) < TOL
        assert O.max_rel(_np(u2).astype(np.float64), ref_du.astype(np.float64)) < TOL


def test_glu_refused_where_the_plan_has_no_epilogue(cuda):
    """Narrow outputs plan the all-wave kernel, which has no SwiGLU epilogue: the query says so
    and the entries return an error instead of computing something else."""
    from mindxsoup_amd import kernels

    n, k, M = 256, 1536, 64
    assert not kernels.glu_fused(M, n, k, False)
    assert not kernels.glu_fused(M, k, n, True)
    layer = _layer(cuda, n, k, 81)
    x = torch.randn((M, k), device=cuda).half()
    gate = torch.randn((M, n), device=cuda).half()
    with pytest.raises(RuntimeError):
        kernels.nf4_linear_fwd_glu(x, layer.weight.data.view(-1, 1), layer.weight.quant_state,
                                   gate)
    torch.cuda.synchronize()


def _mlp(dev, hidden, inter, seed, dropout=0.05):
    from mindxsoup_amd.linear4bit import LoraLinear4bit
    from mindxsoup_amd.mlp import MLP

    layers = []
    for i, (n, k) in enumerate([(inter, hidden), (inter, hidden), (hidden, inter)]):
        m = LoraLinear4bit(_layer(dev, n, k, seed + i), r=16, lora_alpha=32,
                           lora_dropout=dropout)
        g = torch.Generator(device=dev)
        g.manual_seed(seed + 10 + i)
        with torch.no_grad():  # trained-looking B (peft starts it at zero)
            m.lora_B["default"].weight.copy_(
                torch.randn(m.lora_B["default"].weight.shape, device=dev, generator=g) * 0.01)
        layers.append(m)
    return MLP(*layers)


def _run(mlp, x, dy, fused, seed):
    from mindxsoup_amd import mlp as mlp_mod

    previous = mlp_mod.FUSED_SWIGLU
    mlp_mod.FUSED_SWIGLU = fused
    try:
        torch.manual_seed(seed)  # the same dropout draws, in the same order
        xg = x.clone().requires_grad_(True)
        for p in mlp.parameters():
            p.grad = None
        y = mlp(xg)
        y.backward(dy)
        torch.cuda.synchronize()
        grads = {n: p.grad.clone() for n, p in mlp.named_parameters() if p.grad is not None}
        return y.detach(), xg.grad, grads
    finally:
        mlp_mod.FUSED_SWIGLU = previous


@pytest.mark.parametrize("M", [1024, 300])
@pytest.mark.parametrize("fwd_tail", [False, True])
def test_mlp_fused_equals_projections_and_silu_mul(cuda, M, fwd_tail, monkeypatch):
    """NF4LoraMLPFunction against the reference's composition through the same modules
    (solution/mlp.py:42-44: down_proj(silu_mul(gate_proj(x16), up_proj(x16)))): output and all
    six LoRA gradients bit for bit, fp32 residual input as in the reference; the input gradient
    within the roundings of the composition's fp16 parts and their fp16 sum (at most 1.5 fp16
    ulps of the largest value: max relative error below 2^-9), since the fused block sums them in
    fp32 before its one rounding."""
    from mindxsoup_amd import mlp as mlp_mod

    print(f"case mlp fused/unfused M={M} fwd_tail={fwd_tail}", flush=True)
    monkeypatch.setattr(mlp_mod, "GLU_FORWARD_TAIL", fwd_tail)
    hidden, inter = 1536, 8960
    mlp = _mlp(cuda, hidden, inter, 90)
    mlp.train()
    x = torch.randn((1, M, hidden), device=cuda)  # fp32 residual stream
    dy = torch.randn((1, M, hidden), device=cuda)
    assert mlp_mod.fused_ok(mlp, x.half())
    y1, dx1, g1 = _run(mlp, x, dy, False, 5)
    y2, dx2, g2 = _run(mlp, x, dy, True, 5)
    assert y1.dtype == torch.float32 and dx1.dtype == torch.float32
    assert torch.equal(y2, y1)
    err = ((dx2 - dx1).abs().max() / dx1.abs().max()).item()
    assert 0 < err < 2 ** -9, err  # 0 would mean the summed launch did not run
    assert sorted(g1) == sorted(g2) and len(g1) == 6
    for name in g1:
        assert torch.equal(g2[name], g1[name]), name


def test_mlp_matches_oracle(cuda):
    """The fused block (dropout masks fixed) against a float64 composition of the oracle: Y, dX
    and the LoRA gradients of all three projections within max relative error 1e-2."""
    from mindxsoup_amd import mlp as mlp_mod

    M, hidden, inter, p, s = 200, 1536, 8960, 0.05, 2.0
    print(f"case mlp oracle M={M}", flush=True)
    mlp = _mlp(cuda, hidden, inter, 110)
    mlp.train()
    g = torch.Generator(device=cuda)
    g.manual_seed(111)
    keeps = [(torch.rand((M, k), device=cuda, generator=g) >= p).to(torch.uint8)
             for k in (hidden, hidden, inter)]
    for m, kp in zip((mlp.gate_proj, mlp.up_proj, mlp.down_proj), keeps):
        m.next_keep = kp
    x = torch.randn((M, hidden), device=cuda).half().requires_grad_(True)
    dy = torch.randn((M, hidden), device=cuda).half()
    assert mlp_mod.fused_ok(mlp, x)
    y = mlp(x)
    y.backward(dy)
    torch.cuda.synchronize()

    def parts(m):
        return (_w_oracle(m.base_layer), _np(m.lora_A["default"].weight).astype(np.float16),
                _np(m.lora_B["default"].weight).astype(np.float16))

    (wg, ag, bg), (wu, au, bu), (wd, ad, bd) = (parts(m) for m in
                                                 (mlp.gate_proj, mlp.up_proj, mlp.down_proj)
                                                 )
    kg, ku, kd = (_np(k) for k in keeps)
    xn, dyn = _np(x), _np(dy)
    gate = O.lora_fwd(xn, wg, ag, bg, s, kg, p).astype(np.float16)
    up = O.lora_fwd(xn, wu, au, bu, s, ku, p).astype(np.float16)
    h = O.silu_mul(gate, up)
    ref_y = O.lora_fwd(h, wd, ad, bd, s, kd, p)
    dh, dad, dbd = O.lora_bwd(dyn, h, wd, ad, bd, s, kd, p)
    dgate, dup = O.silu_mul_bwd(dh.astype(np.float16), gate, up)
    dxu, dau, dbu = O.lora_bwd(dup, xn, wu, au, bu, s, ku, p)
    dxg, dag, dbg = O.lora_bwd(dgate, xn, wg, ag, bg, s, kg, p)
    ref = dict(y=ref_y, dx=dxu + dxg, da_g=dag, db_g=dbg, da_u=dau, db_u=dbu, da_d=dad,
               db_d=dbd)
    got = dict(y=y, dx=x.grad, da_g=mlp.gate_proj.lora_A["default"].weight.grad,
               db_g=mlp.gate_proj.lora_B["default"].weight.grad,
               da_u=mlp.up_proj.lora_A["default"].weight.grad,
               db_u=mlp.up_proj.lora_B["default"].weight.grad,
               da_d=mlp.down_proj.lora_A["default"].weight.grad,
               db_d=mlp.down_proj.lora_B["default"].weight.grad)
    errs = {k: O.max_rel(_np(got[k]).astype(np.float64), ref[k]) for k in ref}
    print("  max_rel " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert all(v < TOL for v in errs.values()), errs


def test_mlp_without_grad_and_fallbacks(cuda):
    """Under no_grad the block runs without recording (direct path); eval mode draws no dropout;
    projections the fused path does not take (an adapter disabled) give the composition."""
    from mindxsoup_amd import mlp as mlp_mod

    print("case mlp no_grad/fallback", flush=True)
    mlp = _mlp(cuda, 1536, 8960, 130)
    mlp.eval()
    x = torch.randn((2, 64, 1536), device=cuda)
    with torch.no_grad():
        y1 = mlp(x)
        mlp_mod.FUSED_SWIGLU = False
        try:
            y2 = mlp(x)
        finally:
            mlp_mod.FUSED_SWIGLU = True
    assert y1.shape == x.shape and y1.dtype == torch.float32
    assert torch.equal(y1, y2)
    mlp.up_proj.disable_adapters = True
    assert not mlp_mod.fused_ok(mlp, x.half())
    with torch.no_grad():
        y3 = mlp(x)
    assert y3.shape == x.shape and not torch.equal(y3, y1)


def test_mlp_block_replays_in_a_graph(cuda):
    """The fused block (SwiGLU tails, grouped LoRA launches, grouped backward) captured in one
    HIP graph: three replays, with eager work and synchronisations between them, each equal bit
    for bit to the eager step."""
    from mindxsoup_amd import mlp as mlp_mod

    M = 512
    mlp = _mlp(cuda, 1536, 8960, 150, dropout=0.0)  # no random draws inside the graph
    mlp.train()
    x = torch.randn((M, 1536), device=cuda).half().requires_grad_(True)
    dy = torch.randn((M, 1536), device=cuda).half()
    assert mlp_mod.fused_ok(mlp, x)
    params = list(mlp.parameters())

    def step():
        for p in params + [x]:
            p.grad = None
        y = mlp(x)
        y.backward(dy)
        return y

    y0 = step().detach().clone()
    want = [x.grad.clone()] + [p.grad.clone() for p in params if p.grad is not None]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    for p in params + [x]:
        p.grad = None
    with torch.cuda.graph(graph):
        yg = mlp(x)
        yg.backward(dy)
    for rep in range(3):
        junk = torch.randn((M, 8960), device=cuda).half() * rep  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        got = [x.grad] + [p.grad for p in params if p.grad is not None]
        assert torch.equal(yg, y0), rep
        assert len(got) == len(want) and all(torch.equal(a, b) for a, b in zip(got, want)), rep
        del junk


def test_direct_nograd_gives_the_same_output(cuda):
    """solution/test_row_groups.py:57-71 on this build's functions: under no_grad, direct.run
    calls the forward without Function.apply (the Function's forward never sees autograd's
    context) and gives the same bits."""
    from mindxsoup_amd import direct, mlp as mlp_mod

    seen = []
    real = mlp_mod.NF4LoraMLPFunction.forward

    def spy(ctx, *args):
        seen.append(type(ctx).__name__)
        return real(ctx, *args)

    mlp = _mlp(cuda, 1536, 8960, 170)
    mlp.eval()
    x = torch.randn((1, 96, 1536), device=cuda)
    with torch.no_grad():
        ref = mlp(x)
        direct.enabled = True
        mlp_mod.NF4LoraMLPFunction.forward = staticmethod(spy)
        try:
            got = mlp(x)
        finally:
            direct.enabled = False
            mlp_mod.NF4LoraMLPFunction.forward = staticmethod(real)
    assert torch.equal(ref, got)
    assert seen == ["_Unrecorded"]
