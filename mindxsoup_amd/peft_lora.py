"""LoRA layers with peft's attribute layout on the fused NF4 + LoRA kernels.

peft wraps a 4-bit projection as `lora.bnb.Linear4bit` and computes
base(x) + s * lora_B(lora_A(dropout(x))) with four launches of its own around the base (the
composition the reference restates at solution/test_unpad.py:15-29 and relies on at
solution/attention.py:193-201).  This module reads such a layer through its attributes only
(`base_layer`, `lora_A[name]`, `lora_B[name]`, `lora_dropout[name]`, `scaling[name]`,
`active_adapters`, `merged`, `disable_adapters`), so it serves peft's class, when peft is
installed, and this package's `LoraLinear4bit` alike, and sends the projection through
`NF4LoraFunction`: the LoRA row product in one launch, the base GEMM with the LoRA term added
in its accumulators, and the backward's dX / dA / dB in at most three launches.

A layer is taken when it has exactly one plain adapter (no DoRA or other variant, no LoRA bias),
is not merged or disabled, its base is an fp16 NF4 layer the fused kernels take, the rank is a
multiple of 16 no larger than 128, and the input is fp16 (or fp32 under fp16 autocast, where peft's branch
computes in fp16 as well).  Anything else runs the layer's own forward.
"""

import math

import torch

from . import kernels, linear4bit, stream


class Adapter:
    """The one active adapter of a LoRA layer, resolved: its base layer, the A [r, K] and
    B [N, r] weights, the dropout module and probability, and the scaling."""

    __slots__ = ("layer", "name", "base", "a", "b", "dropout", "p", "s")

    def __init__(self, layer, name, base, a, b, dropout, p, s):
        self.layer, self.name, self.base = layer, name, base
        self.a, self.b, self.dropout, self.p, self.s = a, b, dropout, p, s

    @property
    def rank(self):
        return self.a.shape[0]

    def dropping(self):
        """Whether a forward now applies dropout (the dropout module's own training flag)."""
        return self.p > 0 and self.dropout.training

    def keep_mask(self, x2d, shape=None):
        """u8 keep mask [M, K] for one training forward: the layer's `next_keep` when a caller
        set one (taken once), else a fresh Bernoulli(1 - p) draw on the current generator."""
        given = getattr(self.layer, "next_keep", None)
        if given is not None:
            self.layer.next_keep = None
            return given
        return torch.empty(x2d.shape if shape is None else shape, dtype=torch.uint8,
                           device=x2d.device).bernoulli_(1.0 - self.p)


def _entry(table, name):
    try:
        return table[name]
    except (KeyError, TypeError, IndexError):
        return None


def _scalar(v):
    if isinstance(v, torch.Tensor):
        if v.numel() != 1:
            return None
        v = v.item()
    if isinstance(v, (int, float)) and math.isfinite(v):
        return float(v)
    return None


def adapter_of(layer):
    """The Adapter of a layer with peft's LoRA layout, or None when the fused path must not take
    it: not exactly one active adapter, merged, disabled, a DoRA / variant adapter, a LoRA bias,
    a dropout other than nn.Dropout / nn.Identity, or a base that is not a 4-bit layer."""
    lora_a = getattr(layer, "lora_A", None)
    base = getattr(layer, "base_layer", None)
    if lora_a is None or base is None or getattr(layer, "_force_unfused", False):
        return None
    if getattr(layer, "disable_adapters", True) or getattr(layer, "merged", True):
        return None
    active = getattr(layer, "active_adapters", None)
    if isinstance(active, str):
        active = [active]
    active = list(active or [])
    if len(active) != 1:
        return None
    name = active[0]
    if _entry(getattr(layer, "use_dora", {}), name) or \
            name in (getattr(layer, "lora_variant", None) or {}) or \
            _entry(getattr(layer, "lora_bias", {}), name):
        return None
    a_mod, b_mod = _entry(lora_a, name), _entry(getattr(layer, "lora_B", None), name)
    drop = _entry(getattr(layer, "lora_dropout", None), name)
    if not (isinstance(a_mod, torch.nn.Linear) and isinstance(b_mod, torch.nn.Linear)):
        return None
    if a_mod.bias is not None or b_mod.bias is not None:
        return None
    if isinstance(drop, torch.nn.Dropout):
        p = float(drop.p)
    elif isinstance(drop, torch.nn.Identity) or drop is None:
        p = 0.0
    else:
        return None
    s = _scalar(_entry(getattr(layer, "scaling", None), name))
    if s is None or not 0.0 <= p < 1.0:
        return None
    state = getattr(getattr(base, "weight", None), "quant_state", None)
    if state is None or getattr(base, "compute_dtype", None) != torch.float16:
        return None
    a, b = a_mod.weight, b_mod.weight
    if a.dim() != 2 or b.dim() != 2 or b.shape[1] != a.shape[0]:
        return None
    return Adapter(layer, name, base, a, b, drop, p, s)


def _fp16_input(x):
    """x as the fp16 tensor the fused path multiplies, or None: fp16 as is; fp32 only under fp16
    autocast (peft's branch then runs its GEMMs in fp16 too)."""
    if not isinstance(x, torch.Tensor) or not x.is_cuda:
        return None
    if x.dtype == torch.float16:
        return x
    if x.dtype == torch.float32 and torch.is_autocast_enabled("cuda") and \
            torch.get_autocast_dtype("cuda") == torch.float16:
        return x.to(torch.float16)
    return None


MAX_RANK = 128


def takes(ad, x16):
    """Whether NF4LoraFunction takes this adapter on this fp16 input."""
    if ad is None or x16 is None or not linear4bit.FUSED_LORA:
        return False
    base = ad.base
    state = base.weight.quant_state
    # the LoRA row kernels hold r / 16 accumulator blocks, at most 8 (MXS_ERR_SIZE past r = 128)
    if ad.rank % 16 != 0 or ad.rank > MAX_RANK or ad.a.shape[1] != state.shape[1] or \
            ad.b.shape[0] != state.shape[0]:
        return False
    return linear4bit._direct_ok(base, x16, stream.offloaded(base)) and \
        kernels.fused_shape_ok(state)


def fused_project(ad, x16):
    """y = base(x16) + s * B(A(drop(x16))) through the fused kernels, fp16, x16's leading
    shape; the caller has checked takes(ad, x16)."""
    base = ad.base
    lead = x16.shape[:-1]
    x2d = x16.reshape(-1, x16.shape[-1]).contiguous()
    keep, mask_scale = None, 1.0
    if ad.dropping():
        keep = ad.keep_mask(x2d)
        mask_scale = 1.0 / (1.0 - ad.p)
    bias = linear4bit._cast_bias_once(base, x16)
    state = base.weight.quant_state
    if stream.offloaded(base):
        y = linear4bit.NF4LoraStreamFunction.apply(x2d, ad.a, ad.b, base, state, bias, keep,
                                                   mask_scale, ad.s)
    else:
        y = linear4bit.lora_project(x2d, ad.a, ad.b, base.weight.data.view(-1, 1), state, bias,
                                    keep, mask_scale, ad.s)
    return y if x16.dim() == 2 else y.view(*lead, y.shape[-1])


def lora_forward(layer, x, fallback, *args, **kwargs):
    """The forward of a peft-layout LoRA layer: the fused kernels when they take it (output in
    x's dtype, as the 4-bit base returns it), else fallback(layer, x, *args, **kwargs)."""
    if not args and not kwargs:
        ad = adapter_of(layer)
        x16 = _fp16_input(x) if ad is not None else None
        if takes(ad, x16):
            return fused_project(ad, x16).to(x.dtype)
    return fallback(layer, x, *args, **kwargs)


def patch_peft_lora():
    """Route peft's 4-bit LoRA layer (peft.tuners.lora.bnb.Linear4bit) through lora_forward;
    its own forward stays the fallback.  Returns whether peft's class was found (it is not
    installed in every environment; this package's LoraLinear4bit takes the same path)."""
    try:
        from peft.tuners.lora import bnb as peft_bnb
        cls = peft_bnb.Linear4bit
    except Exception:
        return False
    if getattr(cls, "_mindx_fused_lora", False):
        return True
    original = cls.forward

    def forward(self, x, *args, **kwargs):
        return lora_forward(self, x, original, *args, **kwargs)

    forward._mindx_original = original
    cls.forward = forward
    cls._mindx_fused_lora = True
    return True
