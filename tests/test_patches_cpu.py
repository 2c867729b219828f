"""The patches apply() installs on bitsandbytes and peft, against stand-in modules (neither library
is installed here): what gets installed, that it is idempotent, which calls it declines and hands
to the original unchanged, and what the taken branch calls.  The reference tests its hooks the
same way, with fakes (solution/test_stream.py:163-177).  No GPU: the taken branches are driven
with the HIP calls replaced by recorders."""

import sys
import types

import pytest
import torch

from tests.conftest import _Recorder


def _state(nested=True, shape=(64, 64)):
    n = shape[0] * shape[1]
    s2 = types.SimpleNamespace(absmax=torch.ones((n // 64 + 255) // 256),
                               code=torch.zeros(256), blocksize=256)
    return types.SimpleNamespace(shape=shape, blocksize=64, quant_type="nf4",
                                 dtype=torch.float16, nested=nested,
                                 absmax=torch.zeros(n // 64, dtype=torch.uint8),
                                 state2=s2 if nested else None,
                                 offset=torch.zeros(1))


def test_patch_bnb_nf4_installs_once(fake_bnb):
    from mindxsoup_amd import nf4

    originals = (fake_bnb.functional.dequantize_4bit, fake_bnb.ops._dequant_linear_fallback)
    assert nf4.patch_bnb_nf4()
    hooked = (fake_bnb.functional.dequantize_4bit, fake_bnb.ops._dequant_linear_fallback)
    assert hooked[0] is not originals[0] and hooked[1] is not originals[1]
    assert fake_bnb.functional._mindx_patched
    assert nf4.patch_bnb_nf4()  # a second call changes nothing
    assert (fake_bnb.functional.dequantize_4bit,
            fake_bnb.ops._dequant_linear_fallback) == hooked


def test_patch_bnb_nf4_without_bitsandbytes(monkeypatch):
    from mindxsoup_amd import nf4

    monkeypatch.setitem(sys.modules, "bitsandbytes", None)  # import fails
    monkeypatch.setitem(sys.modules, "bitsandbytes.functional", None)
    assert nf4.patch_bnb_nf4() is False


def test_dequantize_hook_declines_like_the_reference(fake_bnb):
    """solution/nf4.py:184-197: no state, `out` given, A not 2-D, a one-row A, or an input the
    HIP kernels do not take (here: CPU tensors) go to bitsandbytes' own function with the
    arguments unchanged."""
    from mindxsoup_amd import nf4

    original = fake_bnb.functional.dequantize_4bit
    nf4.patch_bnb_nf4()
    hook = fake_bnb.functional.dequantize_4bit
    st = _state()
    packed = torch.zeros(64 * 64 // 2, 1, dtype=torch.uint8)
    cases = [dict(A=packed, quant_state=None), dict(A=packed, quant_state=st, out=torch.empty(1)),
             dict(A=packed.view(-1), quant_state=st), dict(A=packed.view(1, -1), quant_state=st),
             dict(A=packed, quant_state=st)]  # CPU: _supported is False
    for kw in cases:
        before = len(original.calls)
        assert hook(**kw) == "dequantize_4bit"
        assert len(original.calls) == before + 1
        args, kwargs = original.calls[-1]
        assert kwargs["quant_state"] is kw["quant_state"] and kwargs.get("out") is kw.get("out")
        assert args[0] is kw["A"]


def test_dequantize_hook_takes_supported_inputs(fake_bnb, monkeypatch):
    """The taken branch: nested states hand absmax8 / code / absmax2 / offset to unpack_nf4;
    plain ones the fp32 absmax (solution/nf4.py:193-197)."""
    from mindxsoup_amd import nf4

    calls = _Recorder("unpacked")
    monkeypatch.setattr(nf4, "_supported", lambda *a, **k: True)
    monkeypatch.setattr(nf4, "unpack_nf4", calls)
    nf4.patch_bnb_nf4()
    hook = fake_bnb.functional.dequantize_4bit
    packed = torch.zeros(64 * 64 // 2, 1, dtype=torch.uint8)
    st = _state()
    assert hook(packed, quant_state=st) == "unpacked"
    args, kwargs = calls.calls[-1]
    assert args[0] is packed and args[1] == st.shape and args[2] is st.state2.absmax
    assert kwargs["absmax_8bit"] is st.absmax and kwargs["code"] is st.state2.code
    assert kwargs["offset"] is st.offset
    plain = _state(nested=False)
    plain.absmax = torch.ones(64, dtype=torch.float16)
    assert hook(packed, quant_state=plain) == "unpacked"
    args, kwargs = calls.calls[-1]
    assert args[2].dtype == torch.float32 and "absmax_8bit" not in kwargs


def test_linear_fallback_hook(fake_bnb, monkeypatch):
    """solution/nf4.py:199-207: declines unsupported weights (and an fp16 non-nested absmax);
    otherwise F.linear(A, unpack(B), bias)."""
    from mindxsoup_amd import nf4

    nf4.patch_bnb_nf4()
    hook = fake_bnb.ops._dequant_linear_fallback
    A = torch.randn(3, 64)
    B = torch.zeros(64 * 8 // 2, 1, dtype=torch.uint8)
    absmax = torch.ones(8)
    assert hook(A, B, (8, 64), absmax, 64, "nf4") == "fallback"  # CPU: declined
    w = torch.randn(8, 64)
    monkeypatch.setattr(nf4, "_supported", lambda *a, **k: True)
    monkeypatch.setattr(nf4, "unpack_nf4", lambda *a, **k: w)
    assert hook(A, B, (8, 64), absmax.half(), 64, "nf4") == "fallback"  # fp16 plain absmax
    bias = torch.randn(8)
    got = hook(A, B, (8, 64), absmax, 64, "nf4", bias)
    assert torch.equal(got, torch.nn.functional.linear(A, w, bias))


def test_patch_bnb_linear4bit(fake_bnb, monkeypatch):
    """solution/linear4bit.py:151-182: the HIP forward goes onto bitsandbytes.nn.Linear4bit once;
    a call the direct path does not take (a CPU input) runs bitsandbytes' own forward; with
    cache_weights the switch for the fp16 cache is set."""
    from mindxsoup_amd import linear4bit

    monkeypatch.setattr(linear4bit, "cache_fp16", linear4bit.cache_fp16)
    cls = fake_bnb.nn.Linear4bit
    assert linear4bit.patch_bnb_linear4bit(cache_weights=True)
    assert cls._mindx_direct and linear4bit.cache_fp16
    patched = cls.forward
    assert linear4bit.patch_bnb_linear4bit() and cls.forward is patched
    layer = cls()
    layer.weight = torch.nn.Parameter(torch.zeros(8, 1, dtype=torch.uint8), requires_grad=False)
    layer.bias = None
    assert layer(torch.randn(2, 16)) == "bnb forward"


def test_apply_installs_both_bnb_patches(fake_bnb, monkeypatch):
    import mindxsoup_amd
    from mindxsoup_amd import direct, linear4bit, mlp

    for key in ("mlp_fp16", "attention_fp16"):
        monkeypatch.setitem(mindxsoup_amd.FEATURES, key, False)
    for mod, name in ((direct, "enabled"), (linear4bit, "FUSED_GEMM"),
                      (linear4bit, "FUSED_LORA"), (linear4bit, "cache_fp16"),
                      (mlp, "FUSED_SWIGLU")):
        monkeypatch.setattr(mod, name, getattr(mod, name))
    mindxsoup_amd.apply()
    assert fake_bnb.functional._mindx_patched and fake_bnb.nn.Linear4bit._mindx_direct


# ---- peft's 4-bit LoRA layer ------------------------------------------------------------------

class _PeftLinear4bit(torch.nn.Module):
    """peft's lora.bnb.Linear4bit attribute layout with its own (unfused) forward."""

    def __init__(self, base, r=16, alpha=32, p=0.05, name="default"):
        super().__init__()
        self.base_layer = base
        self.lora_A = torch.nn.ModuleDict({name: torch.nn.Linear(base.in_features, r,
                                                                 bias=False)})
        self.lora_B = torch.nn.ModuleDict({name: torch.nn.Linear(r, base.out_features,
                                                                 bias=False)})
        self.lora_dropout = torch.nn.ModuleDict({name: torch.nn.Dropout(p)})
        self.scaling = {name: alpha / r}
        self.use_dora = {name: False}
        self.lora_bias = {name: False}
        self.active_adapters = [name]
        self.merged = False
        self.disable_adapters = False

    def forward(self, x, *args, **kwargs):
        return "peft forward"


@pytest.fixture
def fake_peft(monkeypatch):
    peft = types.ModuleType("peft")
    tuners = types.ModuleType("peft.tuners")
    lora = types.ModuleType("peft.tuners.lora")
    bnb = types.ModuleType("peft.tuners.lora.bnb")

    class Linear4bit(_PeftLinear4bit):
        pass

    bnb.Linear4bit = Linear4bit
    peft.tuners, tuners.lora, lora.bnb = tuners, lora, bnb
    for name, mod in (("peft", peft), ("peft.tuners", tuners), ("peft.tuners.lora", lora),
                      ("peft.tuners.lora.bnb", bnb)):
        monkeypatch.setitem(sys.modules, name, mod)
    monkeypatch.setattr(Linear4bit, "forward", Linear4bit.forward)
    return bnb


def _nf4_base(n=64, k=64):
    from mindxsoup_amd.linear4bit import Linear4bit

    base = Linear4bit(k, n, bias=False)
    base.set_quantized(torch.zeros(n * k // 2, dtype=torch.uint8), _state(shape=(n, k)))
    return base


def test_patch_peft_lora_installs_once(fake_peft):
    from mindxsoup_amd import peft_lora

    cls = fake_peft.Linear4bit
    original = cls.forward
    assert peft_lora.patch_peft_lora()
    assert cls._mindx_fused_lora and cls.forward._mindx_original is original
    patched = cls.forward
    assert peft_lora.patch_peft_lora() and cls.forward is patched
    layer = cls(_nf4_base())
    # a CPU input is not taken: peft's own forward runs, extra arguments passed through
    assert layer(torch.randn(2, 64)) == "peft forward"
    assert layer(torch.randn(2, 64), adapter_names=["default"]) == "peft forward"


def test_patch_peft_lora_without_peft(monkeypatch):
    from mindxsoup_amd import peft_lora

    monkeypatch.setitem(sys.modules, "peft", None)
    assert peft_lora.patch_peft_lora() is False


def test_adapter_resolution_declines_what_peft_composes_differently():
    """adapter_of reads peft's layout and refuses what the fused kernels do not compute:
    several or no active adapters, merged or disabled adapters, DoRA, a LoRA bias, another
    dropout module, a base that is not 4-bit."""
    from mindxsoup_amd import peft_lora

    layer = _PeftLinear4bit(_nf4_base(), r=16, alpha=32, p=0.05)
    ad = peft_lora.adapter_of(layer)
    assert ad is not None and ad.rank == 16 and ad.s == 2.0 and ad.p == 0.05
    assert ad.a is layer.lora_A["default"].weight and ad.b is layer.lora_B["default"].weight
    for attr, value in (("merged", True), ("disable_adapters", True),
                        ("active_adapters", ["default", "other"]), ("active_adapters", []),
                        ("use_dora", {"default": True}), ("lora_bias", {"default": True}),
                        ("_force_unfused", True)):
        bad = _PeftLinear4bit(_nf4_base())
        setattr(bad, attr, value)
        assert peft_lora.adapter_of(bad) is None, attr
    bad = _PeftLinear4bit(_nf4_base())
    bad.lora_dropout["default"] = torch.nn.ReLU()
    assert peft_lora.adapter_of(bad) is None
    bad = _PeftLinear4bit(torch.nn.Linear(64, 64))  # a dense base
    assert peft_lora.adapter_of(bad) is None
    plain = _PeftLinear4bit(_nf4_base(), p=0.0)
    plain.lora_dropout["default"] = torch.nn.Identity()
    assert peft_lora.adapter_of(plain).p == 0.0
    assert peft_lora.adapter_of(torch.nn.Linear(4, 4)) is None


def test_takes_refuses_ranks_the_row_kernels_do_not_hold(monkeypatch):
    """Ranks past 128 (the LoRA row kernels' eight 16-wide accumulator blocks) or not a multiple
    of 16 take the layer's own forward instead of raising inside the fused one."""
    from mindxsoup_amd import kernels, linear4bit, peft_lora

    monkeypatch.setattr(linear4bit, "_direct_ok", lambda *a, **k: True)
    monkeypatch.setattr(kernels, "fused_shape_ok", lambda *a, **k: True)
    monkeypatch.setattr(linear4bit, "FUSED_LORA", True)
    x16 = torch.zeros(4, 64, dtype=torch.float16)
    for r, want in ((16, True), (128, True), (24, False), (144, False), (256, False)):
        ad = peft_lora.adapter_of(_PeftLinear4bit(_nf4_base(), r=r, alpha=2 * r))
        assert ad is not None and ad.rank == r
        assert peft_lora.takes(ad, x16) is want, r


def test_keep_mask_and_dropout_flag():
    from mindxsoup_amd import peft_lora

    layer = _PeftLinear4bit(_nf4_base(), p=0.25)
    ad = peft_lora.adapter_of(layer)
    layer.train()
    assert ad.dropping()
    layer.eval()
    assert not ad.dropping()
    x2d = torch.zeros(7, 64)
    given = torch.ones(7, 64, dtype=torch.uint8)
    layer.next_keep = given
    assert ad.keep_mask(x2d) is given and layer.next_keep is None  # taken once
    torch.manual_seed(0)
    drawn = ad.keep_mask(torch.zeros(4000, 64))
    assert drawn.dtype == torch.uint8 and abs(drawn.float().mean().item() - 0.75) < 0.01


def test_apply_patches_peft(fake_peft, monkeypatch):
    import mindxsoup_amd
    from mindxsoup_amd import direct, linear4bit, mlp

    for key in ("nf4", "mlp_fp16", "attention_fp16"):
        monkeypatch.setitem(mindxsoup_amd.FEATURES, key, False)
    for mod, name in ((direct, "enabled"), (linear4bit, "FUSED_GEMM"),
                      (linear4bit, "FUSED_LORA"), (mlp, "FUSED_SWIGLU")):
        monkeypatch.setattr(mod, name, getattr(mod, name))
    mindxsoup_amd.apply()
    assert fake_peft.Linear4bit._mindx_fused_lora
