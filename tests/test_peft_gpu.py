"""LoRA layers with peft's layout routed to the fused kernels, the grouped q/k/v projections, and
the fp16 weight-cache branch of the patched Linear4bit, on the GPU against the CPU oracle
(max relative error 1e-2, the north star's GEMM bar)."""

import sys
import types

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _base(dev, n, k, seed, bias=False):
    from mindxsoup_amd.linear4bit import Linear4bit

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).half()
    b = (torch.randn((n,), device=dev, generator=g) * 0.1).half() if bias else None
    return Linear4bit.from_weight(w, b)


def _w16(layer):
    st = layer.weight.quant_state
    q = O.NF4Weight(st.shape, layer.weight.data.view(-1).cpu().numpy(), st.absmax.cpu().numpy(),
                    st.state2.code.cpu().numpy(), st.state2.absmax.cpu().numpy(),
                    float(st.offset.item()))
    return O.dequant(q)


def _np(t):
    return t.detach().float().cpu().numpy()


class PeftStyleLinear4bit(torch.nn.Module):
    """peft's lora.bnb.Linear4bit as peft writes it: base_layer plus lora_A / lora_B /
    lora_dropout ModuleDicts, scaling, active_adapters; its own forward is the unfused
    composition base(x) + lora_B(lora_A(dropout(x))) * scaling (solution/test_unpad.py:15-29)."""

    def __init__(self, base, r=16, alpha=32, p=0.05, name="default"):
        super().__init__()
        self.base_layer = base
        dev = base.weight.device
        self.lora_A = torch.nn.ModuleDict({name: torch.nn.Linear(base.in_features, r,
                                                                 bias=False, device=dev)})
        self.lora_B = torch.nn.ModuleDict({name: torch.nn.Linear(r, base.out_features,
                                                                 bias=False, device=dev)})
        torch.nn.init.normal_(self.lora_B[name].weight, std=0.02)
        self.lora_dropout = torch.nn.ModuleDict({name: torch.nn.Dropout(p)})
        self.scaling = {name: alpha / r}
        self.active_adapters = [name]
        self.merged = False
        self.disable_adapters = False
        self.unfused_calls = 0

    def forward(self, x, *args, **kwargs):
        self.unfused_calls += 1
        name = self.active_adapters[0]
        lora = self.lora_B[name](self.lora_A[name](self.lora_dropout[name](x.to(torch.float32))))
        return self.base_layer(x) + (lora * self.scaling[name]).to(x.dtype)


@pytest.fixture
def peft_patched(monkeypatch):
    """A `peft.tuners.lora.bnb` module whose Linear4bit is PeftStyleLinear4bit, patched by
    patch_peft_lora (restored after the test)."""
    from mindxsoup_amd import peft_lora

    class Linear4bit(PeftStyleLinear4bit):
        pass

    mods = {n: types.ModuleType(n) for n in ("peft", "peft.tuners", "peft.tuners.lora",
                                             "peft.tuners.lora.bnb")}
    mods["peft.tuners.lora.bnb"].Linear4bit = Linear4bit
    mods["peft"].tuners = mods["peft.tuners"]
    mods["peft.tuners"].lora = mods["peft.tuners.lora"]
    mods["peft.tuners.lora"].bnb = mods["peft.tuners.lora.bnb"]
    for n, m in mods.items():
        monkeypatch.setitem(sys.modules, n, m)
    assert peft_lora.patch_peft_lora()
    return Linear4bit


@pytest.mark.parametrize("n,k,M", [(1536, 1536, 300), (8960, 1536, 1024), (1536, 8960, 512)])
def test_peft_layer_runs_fused_and_matches_oracle(cuda, peft_patched, n, k, M):
    """A layer with peft's layout, after the patch: y, dX, dA and dB of one training step go
    through NF4LoraFunction and match the float64 oracle of base + s * B(A(drop(x)))."""
    print(f"case peft fused n={n} k={k} M={M}", flush=True)
    layer = peft_patched(_base(cuda, n, k, 1, bias=True)).train()
    torch.manual_seed(2)
    x = torch.randn(M, k, device=cuda).half().requires_grad_(True)
    keep = (torch.rand(M, k, device=cuda) >= 0.05).to(torch.uint8)
    layer.next_keep = keep
    y = layer(x)
    assert layer.unfused_calls == 0 and "NF4LoraFunction" in y.grad_fn.name()
    dy = torch.randn_like(y)
    y.backward(dy)
    a = _np(layer.lora_A["default"].weight).astype(np.float16)
    b = _np(layer.lora_B["default"].weight).astype(np.float16)
    w, kp, x16 = _w16(layer.base_layer), keep.cpu().numpy(), _np(x).astype(np.float16)
    ref_y = O.lora_fwd(x16, w, a, b, 2.0, kp, 0.05, bias=_np(layer.base_layer.bias))
    ref_dx, ref_da, ref_db = O.lora_bwd(_np(dy).astype(np.float16), x16, w, a, b, 2.0, kp, 0.05)
    errs = {"y": O.max_rel(_np(y), ref_y), "dx": O.max_rel(_np(x.grad), ref_dx),
            "dA": O.max_rel(_np(layer.lora_A["default"].weight.grad), ref_da),
            "dB": O.max_rel(_np(layer.lora_B["default"].weight.grad), ref_db)}
    print("  ", errs, flush=True)
    assert max(errs.values()) < TOL, errs


def test_peft_layer_fp32_input_under_autocast(cuda, peft_patched):
    """fp32 input under fp16 autocast (the residual stream of the reference's training loop):
    the fused path computes in fp16 and returns fp32, within the bar of peft's own result;
    without autocast an fp32 input runs peft's forward."""
    layer = peft_patched(_base(cuda, 1536, 1536, 3)).eval()
    x = torch.randn(2, 100, 1536, device=cuda)
    with torch.autocast("cuda", dtype=torch.float16):
        y = layer(x)
    assert layer.unfused_calls == 0 and y.dtype == torch.float32 and y.shape == (2, 100, 1536)
    with torch.no_grad():
        want = PeftStyleLinear4bit.forward(layer, x.half())
    assert O.max_rel(_np(y), _np(want)) < TOL
    layer(x)
    assert layer.unfused_calls == 2  # the direct call above, then the unpatched fallback


def test_peft_layer_declined_cases_run_peft(cuda, peft_patched):
    """Merged, disabled or rank-8 adapters, and CPU inputs, take peft's own forward."""
    for attr, value in (("merged", True), ("disable_adapters", True)):
        layer = peft_patched(_base(cuda, 256, 1536, 4))
        setattr(layer, attr, value)
        layer(torch.randn(8, 1536, device=cuda).half())
        assert layer.unfused_calls == 1, attr
    layer = peft_patched(_base(cuda, 256, 1536, 4), r=8)
    layer(torch.randn(8, 1536, device=cuda).half())
    assert layer.unfused_calls == 1


@pytest.mark.parametrize("M", [300, 1024])
def test_siblings_function_matches_oracle(cuda, M):
    """q, k, v over one input in shared launches (NF4LoraSiblingsFunction), training with
    dropout: each output, each LoRA gradient and the summed input gradient against the oracle."""
    from mindxsoup_amd.linear4bit import NF4LoraSiblingsFunction, Proj, siblings_ok

    print(f"case siblings M={M}", flush=True)
    shapes = [(1536, 1536), (256, 1536), (256, 1536)]
    bases = [_base(cuda, n, k, 10 + i, bias=True) for i, (n, k) in enumerate(shapes)]
    g = torch.Generator(device=cuda)
    g.manual_seed(7)
    x = torch.randn((M, 1536), device=cuda, generator=g).half().requires_grad_(True)
    projs, ab, keeps = [], [], []
    for base in bases:
        n, k = base.weight.quant_state.shape
        a = ((torch.rand((16, k), device=cuda, generator=g) * 2 - 1) / k ** 0.5) \
            .requires_grad_(True)
        b = (torch.randn((n, 16), device=cuda, generator=g) * 0.01).requires_grad_(True)
        keep = (torch.rand((M, k), device=cuda, generator=g) >= 0.05).to(torch.uint8)
        projs.append(Proj(base.weight.data.view(-1, 1), base.weight.quant_state, base.bias, keep,
                          1.0 / 0.95, 2.0))
        ab += [a, b]
        keeps.append(keep)
    projs = tuple(projs)
    assert siblings_ok(projs, 1536)
    ys = NF4LoraSiblingsFunction.apply(x, projs, True, None, *ab)
    dys = [torch.randn(y.shape, device=cuda, generator=g).half() for y in ys]
    torch.autograd.backward(ys, dys)
    x16 = _np(x).astype(np.float16)
    ref_dx = 0.0
    for i, base in enumerate(bases):
        a16 = _np(ab[2 * i]).astype(np.float16)
        b16 = _np(ab[2 * i + 1]).astype(np.float16)
        w, kp = _w16(base), keeps[i].cpu().numpy()
        ref_y = O.lora_fwd(x16, w, a16, b16, 2.0, kp, 0.05, bias=_np(base.bias))
        rdx, rda, rdb = O.lora_bwd(_np(dys[i]).astype(np.float16), x16, w, a16, b16, 2.0, kp,
                                   0.05)
        ref_dx = ref_dx + rdx
        errs = (O.max_rel(_np(ys[i]), ref_y), O.max_rel(_np(ab[2 * i].grad), rda),
                O.max_rel(_np(ab[2 * i + 1].grad), rdb))
        assert max(errs) < TOL, (i, errs)
        assert ab[2 * i].grad.dtype == torch.float32
    assert O.max_rel(_np(x.grad), ref_dx) < TOL


def test_cache_fp16_branch(cuda, monkeypatch):
    """FEATURES["nf4_cache_fp16"] (solution/linear4bit.py:132-148): the first call decodes the
    weight once and keeps it in fp16, bit-equal to the oracle's dequant; later calls reuse the
    same tensor; y and the input gradient match the oracle.  An input the direct path refuses
    leaves the cache empty."""
    from mindxsoup_amd import linear4bit

    monkeypatch.setattr(linear4bit, "cache_fp16", True)
    layer = _base(cuda, 1536, 1536, 21, bias=True)
    assert "_mindx_weight16" not in layer.__dict__
    x = torch.randn(512, 1536, device=cuda).half().requires_grad_(True)
    y = layer(x)
    cached = layer.__dict__["_mindx_weight16"]
    w = _w16(layer)
    assert np.array_equal(cached.cpu().numpy().view(np.int16), w.view(np.int16))
    dy = torch.randn_like(y)
    y.backward(dy)
    x16 = _np(x).astype(np.float16)
    assert O.max_rel(_np(y), O.linear_fwd(x16, w, _np(layer.bias))) < TOL
    assert O.max_rel(_np(x.grad), O.linear_bwd_dx(_np(dy).astype(np.float16), w)) < TOL
    layer(x[:37])
    assert layer.__dict__["_mindx_weight16"] is cached
    other = _base(cuda, 256, 1536, 22)
    other(torch.randn(4, 1536, device=cuda))  # fp32 input: not the direct path
    assert "_mindx_weight16" not in other.__dict__
