"""Fused NF4 GEMMs and the LoRA branch on the GPU against the CPU oracle.

Bar (north star): GEMM outputs within max relative error 1e-2 (max|got - ref| / max|ref|, the
measure of solution/test_attention.py:91-92) of dequant-then-matmul; the in-GEMM decode itself
is checked bit for bit against the standalone dequant through one-hot inputs.  Shapes follow
solution/test_linear4bit.py:37-59 (out_features x tokens) and BASELINE configs 3-4.
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
    """The exact fp16 W the oracle decodes from the layer's packed bytes."""
    st = layer.weight.quant_state
    q = O.NF4Weight(st.shape, layer.weight.data.view(-1).cpu().numpy(), st.absmax.cpu().numpy(),
                    st.state2.code.cpu().numpy(), st.state2.absmax.cpu().numpy(),
                    float(st.offset.item()))
    return O.dequant(q)


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("n,k", [(256, 1536), (1536, 1536), (192, 128)])
@pytest.mark.parametrize("cfg,splits", [(-1, 1), (0, 1), (1, 2), (2, 1), (4, 3), (6, 2), (7, 1),
                                        (8, 1), (9, 1), (10, 1), (10, 2), (11, 1), (11, 3),
                                        (12, 1), (12, 2)])
def test_in_gemm_decode_is_bit_exact(cuda, n, k, cfg, splits):
    """One-hot rows: X = I gives Y = W^T and dY = I gives dX = W, each output a single exact
    product, so the fused kernels must reproduce the standalone dequant bit for bit (also with
    split-K, where the other splits add exact zeros)."""
    from mindxsoup_amd import kernels
    from mindxsoup_amd.linear4bit import _unpack

    print(f"case decode n={n} k={k} cfg={cfg} splits={splits}", flush=True)
    layer = _layer(cuda, n, k, 0)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    w = _unpack(packed, st, torch.float16)
    eye_k = torch.eye(k, dtype=torch.float16, device=cuda)
    y = kernels.nf4_linear_fwd(eye_k, packed, st, cfg=cfg, splits=splits)
    assert torch.equal(y.view(torch.int16), w.t().contiguous().view(torch.int16))
    eye_n = torch.eye(n, dtype=torch.float16, device=cuda)
    dx = kernels.nf4_linear_bwd_dx(eye_n, packed, st, cfg=cfg, splits=splits)
    assert torch.equal(dx.view(torch.int16), w.view(torch.int16))


@pytest.mark.parametrize("out_features,bias", [(1536, True), (256, True), (8960, False),
                                               (1536, False)])
@pytest.mark.parametrize("tokens", [37, 300, 512, 700, 1203, 2048])
def test_linear4bit_fwd_bwd_matches_oracle(cuda, out_features, bias, tokens):
    """solution/test_linear4bit.py:37-59 shapes: Y = x W^T + b and grad_x = grad W through the
    module and autograd, against float64 dequant-then-matmul."""
    print(f"case linear out={out_features} bias={bias} tokens={tokens}", flush=True)
    layer = _layer(cuda, out_features, 1536, 1, bias)
    torch.manual_seed(2)
    x = torch.randn(1, tokens, 1536, device=cuda, dtype=torch.float16, requires_grad=True)
    y = layer(x)
    g = torch.randn_like(y)
    y.backward(g)
    w = _w_oracle(layer)
    xb = _np(x)[0].astype(np.float16)
    ref_y = O.linear_fwd(xb, w, None if not bias else _np(layer.bias))
    ref_dx = O.linear_bwd_dx(_np(g)[0].astype(np.float16), w)
    ey, edx = O.max_rel(_np(y)[0], ref_y), O.max_rel(_np(x.grad)[0], ref_dx)
    print(f"  max_rel y={ey:.2e} dx={edx:.2e}", flush=True)
    assert y.shape == (1, tokens, out_features) and y.dtype == torch.float16
    assert ey < TOL and edx < TOL


@pytest.mark.parametrize("cfg,splits", [(0, 1), (0, 4), (1, 1), (1, 3), (2, 2), (4, 1), (6, 1),
                                        (6, 3), (7, 2), (8, 1), (9, 4), (10, 1), (10, 3),
                                        (11, 4), (12, 1), (12, 3)])
def test_tile_configs_agree_with_oracle(cuda, cfg, splits):
    from mindxsoup_amd import kernels

    print(f"case tiles cfg={cfg} splits={splits}", flush=True)
    layer = _layer(cuda, 1536, 1536, 3, bias=True)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    torch.manual_seed(4)
    x = torch.randn(300, 1536, device=cuda, dtype=torch.float16)
    dy = torch.randn(300, 1536, device=cuda, dtype=torch.float16)
    y = kernels.nf4_linear_fwd(x, packed, st, layer.bias, cfg=cfg, splits=splits)
    dx = kernels.nf4_linear_bwd_dx(dy, packed, st, cfg=cfg, splits=splits)
    w = _w_oracle(layer)
    assert O.max_rel(_np(y), O.linear_fwd(_np(x).astype(np.float16), w, _np(layer.bias))) < TOL
    assert O.max_rel(_np(dx), O.linear_bwd_dx(_np(dy).astype(np.float16), w)) < TOL


def _lora_inputs(dev, M, K, N, seed, x_kind="normal", dy_std=1.0):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    if x_kind == "silu_mul":  # saved activations silu(g) * u
        gg = torch.randn((M, K), device=dev, generator=g)
        uu = torch.randn((M, K), device=dev, generator=g)
        x = (torch.nn.functional.silu(gg) * uu).half()
    else:
        x = torch.randn((M, K), device=dev, generator=g).half()
    bound = 1.0 / np.sqrt(K)  # kaiming_uniform(a=sqrt(5)) bound for fan_in K
    a = ((torch.rand((16, K), device=dev, generator=g) * 2 - 1) * bound).half()
    b = (torch.randn((N, 16), device=dev, generator=g) * 0.01).half()
    dy = (torch.randn((M, N), device=dev, generator=g) * dy_std).half()
    keep = (torch.rand((M, K), device=dev, generator=g) >= 0.05).to(torch.uint8)
    return x, a, b, dy, keep


@pytest.mark.parametrize("name,n,k,m,x_kind,dy_std", [
    ("gate_proj (BASELINE config 3)", 8960, 1536, 1024, "normal", 1.0),
    ("down_proj (BASELINE config 4)", 1536, 8960, 1024, "silu_mul", 1e-3),
    ("k_proj ragged tokens", 256, 1536, 37, "normal", 1.0),
])
def test_fused_lora_fwd_bwd_matches_oracle(cuda, name, n, k, m, x_kind, dy_std):
    """peft LoRA (r=16, alpha=32, dropout 0.05 with an explicit mask) around the NF4 base:
    Y, dX, dA, dB against the float64 oracle (itself pinned against torch autograd)."""
    from mindxsoup_amd.linear4bit import NF4LoraFunction

    print(f"case lora {name} m={m}", flush=True)
    layer = _layer(cuda, n, k, 5)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    x, a, b, dy, keep = _lora_inputs(cuda, m, k, n, 6, x_kind, dy_std)
    p, s = 0.05, 2.0
    a_p = a.float().requires_grad_(True)  # fp32 LoRA params, as peft keeps them
    b_p = b.float().requires_grad_(True)
    xg = x.clone().requires_grad_(True)
    y = NF4LoraFunction.apply(xg, a_p, b_p, packed, st, None, keep, 1.0 / (1.0 - p), s)
    y.backward(dy)
    w = _w_oracle(layer)
    xn, an, bn, dyn, kn = (_np(x).astype(np.float16), _np(a).astype(np.float16),
                           _np(b).astype(np.float16), _np(dy).astype(np.float16),
                           keep.cpu().numpy())
    ref_y = O.lora_fwd(xn, w, an, bn, s, kn, p)
    ref_dx, ref_da, ref_db = O.lora_bwd(dyn, xn, w, an, bn, s, kn, p)
    errs = dict(y=O.max_rel(_np(y), ref_y), dx=O.max_rel(_np(xg.grad), ref_dx),
                da=O.max_rel(_np(a_p.grad), ref_da), db=O.max_rel(_np(b_p.grad), ref_db))
    print("  max_rel " + " ".join(f"{k_}={v:.2e}" for k_, v in errs.items()), flush=True)
    assert all(v < TOL for v in errs.values()), errs
    # the LoRA branch matters at this scale: dropping it moves Y beyond the tolerance's reach
    assert O.max_rel(ref_y, O.linear_fwd(xn, w)) > 1e-4


def test_lora_kernels_match_oracle(cuda):
    from mindxsoup_amd import kernels

    M, K, N = 300, 1536, 256
    x, a, b, dy, keep = _lora_inputs(cuda, M, K, N, 7)
    s, p = 2.0, 0.05
    h, ht = kernels.lora_h(x, a, s, keep, 1 / (1 - p))
    dh, dht = kernels.lora_dh(dy, b, s)
    da = kernels.lora_grad_a(dht, x, keep, 1 / (1 - p))
    db = kernels.lora_grad_b(ht, dy)
    xn, an, bn, dyn, kn = (_np(x).astype(np.float16), _np(a).astype(np.float16),
                           _np(b).astype(np.float16), _np(dy).astype(np.float16),
                           keep.cpu().numpy())
    ref_h = s * O.lora_h(xn, an, kn, p)
    assert O.max_rel(_np(h), ref_h) < TOL
    assert torch.equal(ht[:, :M].t(), h) and torch.all(ht[:, M:] == 0)
    ref_dh = s * (dyn.astype(np.float64) @ bn.astype(np.float64))
    assert O.max_rel(_np(dh), ref_dh) < TOL
    xd = O.dropout_fp16(xn, kn, p).astype(np.float64)
    assert O.max_rel(_np(da), _np(dh).astype(np.float64).T @ xd) < TOL
    assert O.max_rel(_np(db), dyn.astype(np.float64).T @ _np(h).astype(np.float64)) < TOL
    # the one-launch pair and the A^T side output agree with the separate calls bit for bit
    h2, ht2, at, bt = kernels.lora_h(x, a, s, keep, 1 / (1 - p), want_at=True, lora_b=b)
    assert torch.equal(h2, h) and torch.equal(ht2, ht)
    assert torch.equal(at, a.t().contiguous()) and torch.equal(bt, b.t().contiguous())
    dh2, _ = kernels.lora_dh(dy, None, s, lora_bt=bt)
    assert torch.equal(dh2, dh)
    da2, db2 = kernels.lora_grads(dht, ht, x, dy, keep, 1 / (1 - p))
    assert torch.equal(da2, da) and torch.equal(db2, db)
    da3, none = kernels.lora_grads(dht, ht, x, dy, keep, 1 / (1 - p), want_b=False)
    assert none is None and torch.equal(da3, da)


@pytest.mark.parametrize("M", [1, 64, 1000])
def test_lora_reductions_across_many_workgroups(cuda, M):
    """Reductions longer than one slice (K = 8960: 18 slices of H; M = 1000: 16 token blocks of
    dA/dB) are summed in a fixed order: repeated calls give the same bits."""
    from mindxsoup_amd import kernels

    K, N = 8960, 1536
    x, a, b, dy, keep = _lora_inputs(cuda, M, K, N, 11)
    s, p = 2.0, 0.1
    h, ht = kernels.lora_h(x, a, s, keep, 1 / (1 - p))
    dh, dht = kernels.lora_dh(dy, b, s)
    da, db = kernels.lora_grads(dht, ht, x, dy, keep, 1 / (1 - p))
    xn, an, bn, dyn, kn = (_np(x).astype(np.float16), _np(a).astype(np.float16),
                           _np(b).astype(np.float16), _np(dy).astype(np.float16),
                           keep.cpu().numpy())
    assert O.max_rel(_np(h), s * O.lora_h(xn, an, kn, p)) < TOL
    assert O.max_rel(_np(dh), s * (dyn.astype(np.float64) @ bn.astype(np.float64))) < TOL
    xd = O.dropout_fp16(xn, kn, p).astype(np.float64)
    assert O.max_rel(_np(da), _np(dh).astype(np.float64).T @ xd) < TOL
    assert O.max_rel(_np(db), dyn.astype(np.float64).T @ _np(h).astype(np.float64)) < TOL
    for _ in range(2):
        h2, _ = kernels.lora_h(x, a, s, keep, 1 / (1 - p))
        da2, db2 = kernels.lora_grads(dht, ht, x, dy, keep, 1 / (1 - p))
        assert torch.equal(h2, h) and torch.equal(da2, da) and torch.equal(db2, db)


def test_lora_sliced_and_single_launch_reductions_agree(cuda):
    """A 8960-long reduction runs over 4 slices of workgroups when given a workspace and in one
    launch without; both match the oracle (the summation order differs, the bound does not)."""
    from mindxsoup_amd import _lib, kernels

    M, K, N = 300, 8960, 8960
    x, a, b, dy, keep = _lora_inputs(cuda, M, K, N, 21)
    s, p = 2.0, 0.05
    assert kernels.lora_workspace_bytes(M, K, N, 16) > 0
    h, ht = kernels.lora_h(x, a, s, keep, 1 / (1 - p))            # sliced (workspace allocated)
    h1 = torch.empty_like(h)
    ht1 = torch.empty_like(ht)
    _lib.call("mxs_lora_h", _lib.ptr(x), M, K, _lib.ptr(a), 16,
              _lib.ptr(kernels.keep_bits(keep, M, K)), 1 / (1 - p), s,
              _lib.ptr(h1), _lib.ptr(ht1), ht1.shape[1], None, None, 0, None, None,
              _lib.stream_of(cuda))                                  # single launch
    bt = b.t().contiguous()
    dh, _ = kernels.lora_dh(dy, None, s, lora_bt=bt)                  # sliced
    dh1 = torch.empty_like(dh)
    dht1 = torch.empty((16, (M + 7) // 8 * 8), dtype=torch.float16, device=cuda)
    _lib.call("mxs_lora_dh", _lib.ptr(dy), M, N, _lib.ptr(bt), 16, s, _lib.ptr(dh1),
              _lib.ptr(dht1), dht1.shape[1], None, _lib.stream_of(cuda))
    xn, an, bn, dyn, kn = (_np(x).astype(np.float16), _np(a).astype(np.float16),
                           _np(b).astype(np.float16), _np(dy).astype(np.float16),
                           keep.cpu().numpy())
    ref_h = s * O.lora_h(xn, an, kn, p)
    ref_dh = s * (dyn.astype(np.float64) @ bn.astype(np.float64))
    for got, ref in ((h, ref_h), (h1, ref_h), (dh, ref_dh), (dh1, ref_dh)):
        assert O.max_rel(_np(got), ref) < TOL
    assert torch.equal(ht[:, :M].t(), h) and torch.all(ht[:, M:] == 0)
    assert torch.equal(ht1[:, :M].t(), h1) and torch.all(ht1[:, M:] == 0)


@pytest.mark.parametrize("n,k,M", [(1536, 1536, 300), (256, 1536, 37), (1536, 8960, 700),
                                   (8960, 1536, 64)])
def test_partial_sum_lora_path_equals_finished_path(cuda, n, k, M):
    """The GEMMs that finish the LoRA partial sums themselves (and write Hs^T / dHs^T) give the
    same bits as finishing them in a separate launch first."""
    from mindxsoup_amd import kernels

    print(f"case partials n={n} k={k} M={M}", flush=True)
    layer = _layer(cuda, n, k, 31, bias=True)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    x, a, b, dy, keep = _lora_inputs(cuda, M, k, n, 32)
    s, ms = 2.0, 1 / 0.95
    h, ht, at, bt = kernels.lora_h(x, a, s, keep, ms, n_out=n, want_at=True, lora_b=b)
    y = kernels.nf4_linear_fwd(x, packed, st, layer.bias, h, b)
    hp, at2, bt2 = kernels.lora_h_partials(x, a, s, keep, ms, lora_b=b)
    assert hp.shape[0] == kernels.lora_slices(M, k)
    y2, ht2 = kernels.nf4_linear_fwd_hp(x, packed, st, hp, b, layer.bias)
    assert torch.equal(y2, y) and torch.equal(ht2, ht)
    assert torch.equal(at2, at) and torch.equal(bt2, bt)
    dh, dht = kernels.lora_dh(dy, None, s, k_in=k, lora_bt=bt)
    dx = kernels.nf4_linear_bwd_dx(dy, packed, st, dh, None, keep, ms, lora_at=at)
    dhp = kernels.lora_dh_partials(dy, bt, s)
    dx2, dht2 = kernels.nf4_linear_bwd_dx_hp(dy, packed, st, dhp, at, keep, ms)
    assert torch.equal(dx2, dx) and torch.equal(dht2, dht)


@pytest.mark.parametrize("n,k,M", [(1536, 1536, 1024), (256, 1536, 1000), (8960, 1536, 700)])
def test_lora_finish_and_backward_sequence(cuda, n, k, M):
    """mxs_lora_finish gives the bits the fused dX GEMM writes as dHs^T from the same partials,
    and the shared backward sequence equals its kernels called one by one."""
    from mindxsoup_amd import kernels
    from mindxsoup_amd.linear4bit import lora_backward

    print(f"case finish/backward n={n} k={k} M={M}", flush=True)
    layer = _layer(cuda, n, k, 37)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    x, a, b, dy, keep = _lora_inputs(cuda, M, k, n, 38)
    s, ms = 2.0, 1 / 0.95
    hp, at, bt = kernels.lora_h_partials(x, a, s, keep, ms, lora_b=b)
    _, ht = kernels.nf4_linear_fwd_hp(x, packed, st, hp, b)
    dhp = kernels.lora_dh_partials(dy, bt, s)
    dx1, dht1 = kernels.nf4_linear_bwd_dx_hp(dy, packed, st, dhp, at, keep, ms)
    out, outT = kernels.lora_finish(dhp, M, want_out=True)
    assert torch.equal(outT, dht1)
    assert torch.equal(out, dht1[:, :M].t().contiguous())
    da1, db1 = kernels.lora_grads(dht1, ht, x, dy, keep, ms)
    if kernels.bwd_grads_fused(M, n, k, 16):
        # the one-launch backward: dHs finished in one launch, then dX and the gradients
        dh, dht1 = kernels.lora_dh(dy, None, s, lora_bt=bt, one_launch=True)
        dx1 = kernels.nf4_linear_bwd_dx(dy, packed, st, dh, None, keep, ms, lora_at=at)
        da1, db1 = kernels.lora_grads(dht1, ht, x, dy, keep, ms)
    dx2, da2, db2 = lora_backward(dy, x, keep, ht, at, bt, packed, st, ms, s)
    torch.cuda.synchronize()
    assert torch.equal(dx2, dx1) and torch.equal(da2, da1) and torch.equal(db2, db1)


@pytest.mark.parametrize("n,k,M", [(1536, 1536, 1024), (256, 1536, 1024), (1536, 1536, 300),
                                   (256, 1536, 37), (8960, 1536, 1024), (1536, 8960, 512),
                                   (1536, 1536, 1200), (1536, 1536, 1430), (1536, 1536, 2048)])
def test_bwd_dx_grads_one_launch(cuda, n, k, M):
    """mxs_nf4_linear_bwd_dx_grads equals mxs_nf4_linear_bwd_dx followed by mxs_lora_grads bit
    for bit, whether it fuses them (1536-wide projections) or not, and its gradients match the
    float64 products.  1200 tokens: 128x64 tiles with the gradient workgroups in a second round;
    1430: 128x128 tiles and gradient workgroups in one round; 2048: not fused."""
    from mindxsoup_amd import kernels

    print(f"case bwd_dx_grads n={n} k={k} M={M}", flush=True)
    layer = _layer(cuda, n, k, 51)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    x, a, b, dy, keep = _lora_inputs(cuda, M, k, n, 52)
    s, ms = 2.0, 1 / 0.95
    h, ht = kernels.lora_h(x, a, s, keep, ms)
    at = a.t().contiguous()
    bt = b.t().contiguous()
    dh, dht = kernels.lora_dh(dy, None, s, lora_bt=bt, one_launch=True)
    fused = kernels.bwd_grads_fused(M, n, k, 16)
    if (n, k, M) == (1536, 1536, 1024) or (n, k, M) == (256, 1536, 1024):
        assert fused, "the 1536-wide projections fuse at 1024 tokens"
    if n == 8960:
        assert not fused, "a split-K dX plan does not take the gradient workgroups"
    dx, da, db = kernels.nf4_linear_bwd_dx_grads(dy, packed, st, dh, at, dht, ht, x, keep, ms)
    dx1 = kernels.nf4_linear_bwd_dx(dy, packed, st, dh, None, keep, ms, lora_at=at)
    da1, db1 = kernels.lora_grads(dht, ht, x, dy, keep, ms)
    torch.cuda.synchronize()
    assert torch.equal(dx, dx1)
    assert torch.equal(da, da1) and torch.equal(db, db1)
    # dA = dHs^T drop(x), dB = dY^T Hs in float64 from the same fp16 operands (oracle dropout)
    xd = O.dropout_fp16(_np(x).astype(np.float16), keep.cpu().numpy(), 0.05).astype(np.float64)
    assert O.max_rel(_np(da), _np(dht[:, :M]).astype(np.float64) @ xd) < TOL
    assert O.max_rel(_np(db), _np(dy).astype(np.float64).T @ _np(h).astype(np.float64)) < TOL


def test_backward_sequence_replays_in_a_graph(cuda):
    """The backward sequence captured in a HIP graph: every replay, with eager work and
    synchronizations between replays, equals the eager result."""
    from mindxsoup_amd import kernels
    from mindxsoup_amd.linear4bit import lora_backward

    n, k, M = 1536, 1536, 1024
    print(f"case graph backward n={n} k={k} M={M}", flush=True)
    layer = _layer(cuda, n, k, 41)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    x, a, b, dy, keep = _lora_inputs(cuda, M, k, n, 42)
    s, ms = 2.0, 1 / 0.95
    hp, at, bt = kernels.lora_h_partials(x, a, s, keep, ms, lora_b=b)
    _, ht = kernels.nf4_linear_fwd_hp(x, packed, st, hp, b)
    ref = lora_backward(dy, x, keep, ht, at, bt, packed, st, ms, s)
    torch.cuda.synchronize()
    ref = [t.clone() for t in ref]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = lora_backward(dy, x, keep, ht, at, bt, packed, st, ms, s)
    for rep in range(4):
        for o in outs:
            o.zero_()
        _ = kernels.lora_dh_partials(dy, bt, s)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r), f"replay {rep} differs"


def test_lora_grads_without_tokens(cuda):
    from mindxsoup_amd import kernels

    r, K, N = 16, 1536, 256
    ht = torch.zeros((r, 0), dtype=torch.float16, device=cuda)
    x = torch.empty((0, K), dtype=torch.float16, device=cuda)
    dy = torch.empty((0, N), dtype=torch.float16, device=cuda)
    da, db = kernels.lora_grads(ht, ht, x, dy)
    assert torch.count_nonzero(da) == 0 and torch.count_nonzero(db) == 0
    assert da.shape == (r, K) and db.shape == (N, r)


@pytest.mark.parametrize("cfg,splits", [(-1, 1), (4, 4), (9, 4), (3, 2), (10, 2), (11, 4)])
def test_split_k_is_deterministic_on_a_reused_workspace(cuda, cfg, splits):
    """Split-K partials are summed in split order: repeated calls (and a call of another shape
    in between, on the same workspace) give identical bits."""
    from mindxsoup_amd import kernels

    layer = _layer(cuda, 1536, 8960, 12)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    g = torch.Generator(device=cuda)
    g.manual_seed(13)
    x = torch.randn((700, 8960), device=cuda, generator=g).half()
    dy = torch.randn((700, 1536), device=cuda, generator=g).half()
    ws = kernels.new_workspace(max(kernels.gemm_workspace_bytes(700, 1536, 8960, cfg, splits),
                                   kernels.gemm_workspace_bytes(700, 8960, 1536, cfg, splits)),
                               cuda)
    y0 = kernels.nf4_linear_fwd(x, packed, st, cfg=cfg, splits=splits, ws=ws)
    dx0 = kernels.nf4_linear_bwd_dx(dy, packed, st, cfg=cfg, splits=splits, ws=ws)
    for _ in range(2):
        y = kernels.nf4_linear_fwd(x, packed, st, cfg=cfg, splits=splits, ws=ws)
        dx = kernels.nf4_linear_bwd_dx(dy, packed, st, cfg=cfg, splits=splits, ws=ws)
        assert torch.equal(y, y0) and torch.equal(dx, dx0)
    w = _w_oracle(layer)
    assert O.max_rel(_np(y0), O.linear_fwd(_np(x).astype(np.float16), w)) < TOL


def test_lora_module_forward_backward(cuda):
    """LoraLinear4bit (peft layout) in training mode with a given mask equals the oracle; in
    eval mode (no dropout) it equals the merged-weight product x (W + s B A)^T."""
    from mindxsoup_amd.linear4bit import LoraLinear4bit

    base = _layer(cuda, 1536, 1536, 8, bias=True)
    mod = LoraLinear4bit(base, r=16, lora_alpha=32, lora_dropout=0.05)
    torch.nn.init.normal_(mod.lora_B["default"].weight, std=0.02)
    torch.manual_seed(9)
    x = torch.randn(2, 150, 1536, device=cuda, dtype=torch.float16)
    mod.eval()
    y = mod(x)
    w = _w_oracle(base).astype(np.float64)
    a = _np(mod.lora_A["default"].weight).astype(np.float16).astype(np.float64)
    b = _np(mod.lora_B["default"].weight).astype(np.float16).astype(np.float64)
    merged = w + 2.0 * b @ a
    ref = _np(x).reshape(-1, 1536).astype(np.float64) @ merged.T + _np(base.bias)
    assert O.max_rel(_np(y).reshape(-1, 1536), ref) < TOL
    mod.train()
    keep = (torch.rand(300, 1536, device=cuda) >= 0.05).to(torch.uint8)
    mod.next_keep = keep
    xg = x.clone().requires_grad_(True)
    y = mod(xg)
    dy = torch.randn_like(y)
    y.backward(dy)
    ga, gb = mod.lora_A["default"].weight.grad, mod.lora_B["default"].weight.grad
    assert ga.shape == (16, 1536) and gb.shape == (1536, 16) and xg.grad.shape == x.shape
    # training values against the oracle: y, dX, dA, dB of base + s * B(A(drop(x)))
    x2 = _np(x).reshape(-1, 1536).astype(np.float16)
    a16, b16 = a.astype(np.float16), b.astype(np.float16)
    w16, kp = _w_oracle(base), keep.cpu().numpy()
    ref_y = O.lora_fwd(x2, w16, a16, b16, 2.0, kp, 0.05, bias=_np(base.bias))
    ref_dx, ref_da, ref_db = O.lora_bwd(_np(dy).reshape(-1, 1536).astype(np.float16), x2, w16,
                                        a16, b16, 2.0, kp, 0.05)
    errs = [O.max_rel(_np(y).reshape(-1, 1536), ref_y),
            O.max_rel(_np(xg.grad).reshape(-1, 1536), ref_dx),
            O.max_rel(_np(ga), ref_da), O.max_rel(_np(gb), ref_db)]
    assert max(errs) < TOL, errs


def test_empty_tokens(cuda):
    from mindxsoup_amd import kernels

    layer = _layer(cuda, 256, 1536, 10)
    st = layer.weight.quant_state
    packed = layer.weight.data.view(-1, 1)
    x = torch.empty(0, 1536, device=cuda, dtype=torch.float16)
    assert kernels.nf4_linear_fwd(x, packed, st).shape == (0, 256)
    dy = torch.empty(0, 256, device=cuda, dtype=torch.float16)
    assert kernels.nf4_linear_bwd_dx(dy, packed, st).shape == (0, 1536)
