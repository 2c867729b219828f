"""Qwen2 MLP on fp16 activations (mirror of solution/mlp.py), with the SwiGLU fused into the NF4
GEMMs' epilogues when all three projections are LoRA-wrapped NF4 layers.

The reference casts the fp32 residual input to fp16 once, runs gate_proj and up_proj in fp16,
keeps fp16 gate/up for the SwiGLU backward and casts only the MLP output back
(solution/mlp.py:1-12, 33-44).  `fp16_forward` keeps that contract.  Where every projection is
a LoRA layer with peft's layout (this package's `LoraLinear4bit` or peft's own) that the fused
kernels take, `NF4LoraMLPFunction` runs the block as:

  forward:  gate = gate_proj(x16) and up = up_proj(x16) (fused GEMMs, LoRA included, their
            LoRA row products in one launch); hidden = silu(gate) * up, by the elementwise
            kernel or, with GLU_FORWARD_TAIL, from up's GEMM tile (mxs_nf4_linear_fwd_glu);
            out = down_proj(hidden).
  backward: down_proj's dX GEMM applies the SwiGLU adjoint in its epilogue and writes d(gate)
            and d(up) over gate's and up's memory (mxs_nf4_linear_bwd_dx_glu): d(hidden) is
            never stored; then down_proj's LoRA gradients, up_proj's and gate_proj's backward,
            and dx = dx_up + dx_gate (the order of solution/mlp_tail.py:42-46).

The values equal the unfused sequence (projection, silu_mul, projection, and autograd's
backward through them) bit for bit: the epilogue rounds each projection to fp16 before the
SwiGLU reads it, as the separate kernel does, and both evaluate the same fp32 formula.
"""

import torch

from . import direct, kernels, linear4bit, peft_lora, stream
from .linear4bit import Proj as _Proj, _cast_bias_once, lora_backward_group
from .silu_mul import silu_mul

FUSED_SWIGLU = True  # FEATURES["mlp_fused_swiglu"]
# The up projection's forward with the SwiGLU tail (mxs_nf4_linear_fwd_glu) measures break-even
# to 2 us slower than the GEMM followed by silu_mul at 1024 tokens on MI355X (its tail moves
# three tiles while the chip idles), so the block's forward composes them; the backward tail
# saves about 7 us and is used.  Both give the same bits.
GLU_FORWARD_TAIL = False

_NAMES = ("gate_proj", "up_proj", "down_proj")


class NF4LoraMLPFunction(torch.autograd.Function):
    """down(silu(gate(x)) * up(x)) for three NF4 + LoRA projections with the SwiGLU in the GEMM
    epilogues.  Inputs: x2d fp16 [M, hidden]; the LoRA A/B weights of gate, up and down (any
    float dtype; their gradients come back in it); `projs`, three `_Proj`.  Output fp16
    [M, hidden]."""

    @staticmethod
    def forward(ctx, x2d, ga, gb, ua, ub, da, db, projs):
        pg, pu, pd = projs
        M = x2d.shape[0]
        inter, hidden = pu.state.shape
        g_a, g_b, u_a, u_b, d_a, d_b = (t.to(torch.float16).contiguous()
                                        for t in (ga, gb, ua, ub, da, db))
        # gate's and up's LoRA row products read the same x: one launch when they can share it
        if pg.s == pu.s and pg.mask_scale == pu.mask_scale:
            (hp_g, at_g, bt_g), (hp, at_u, bt_u) = kernels.lora_h_partials_group(
                [x2d, x2d], [g_a, u_a], pg.s, [pg.keep, pu.keep], pg.mask_scale, [g_b, u_b])
        else:
            hp_g, at_g, bt_g = kernels.lora_h_partials(x2d, g_a, pg.s, pg.keep, pg.mask_scale,
                                                       lora_b=g_b)
            hp, at_u, bt_u = kernels.lora_h_partials(x2d, u_a, pu.s, pu.keep, pu.mask_scale,
                                                     lora_b=u_b)
        glu_tail = GLU_FORWARD_TAIL and kernels.glu_fused(M, inter, hidden, False)
        if not glu_tail and kernels.fwd_pair_ok(M, pg.state.shape[0], inter, hidden) and \
                hp_g.shape == hp.shape:
            # gate and up in one launch (grid z selects the projection; the bits of two)
            (gate, ht_g), (up, ht_u) = kernels.nf4_linear_fwd_hp_pair(
                x2d, [pg.packed, pu.packed], [pg.state, pu.state], [hp_g, hp], [g_b, u_b],
                [pg.bias, pu.bias])
            del hp_g
            h = kernels.silu_mul(gate, up)
        else:
            gate, ht_g = kernels.nf4_linear_fwd_hp(x2d, pg.packed, pg.state, hp_g, g_b, pg.bias)
            del hp_g
            if glu_tail:
                up, h, ht_u = kernels.nf4_linear_fwd_glu(x2d, pu.packed, pu.state, gate, hp, u_b,
                                                         pu.bias)
            else:
                up, ht_u = kernels.nf4_linear_fwd_hp(x2d, pu.packed, pu.state, hp, u_b, pu.bias)
                h = kernels.silu_mul(gate, up)
        hp, at_d, bt_d = kernels.lora_h_partials(h, d_a, pd.s, pd.keep, pd.mask_scale,
                                                 lora_b=d_b)
        y, ht_d = kernels.nf4_linear_fwd_hp(h, pd.packed, pd.state, hp, d_b, pd.bias)
        ctx.save_for_backward(x2d, gate, up, h, ht_g, at_g, bt_g, ht_u, at_u, bt_u, ht_d, at_d,
                              bt_d)
        ctx.projs = projs
        ctx.dtypes = tuple(t.dtype for t in (ga, gb, ua, ub, da, db))
        return y

    @staticmethod
    def backward(ctx, dy):
        (x2d, gate, up, h, ht_g, at_g, bt_g, ht_u, at_u, bt_u, ht_d, at_d,
         bt_d) = ctx.saved_tensors
        pg, pu, pd = ctx.projs
        need = ctx.needs_input_grad
        dy = dy.to(torch.float16).contiguous()
        M = dy.shape[0]
        hidden, inter = pd.state.shape
        # down_proj: dHs = s * dY B_down, then dX = dY W_down + keep/(1-p) * dHs A_down with the
        # SwiGLU adjoint applied in the epilogue (gate <- d(gate), up <- d(up))
        dhp = kernels.lora_dh_partials(dy, bt_d, pd.s)
        want_gd = need[5] or need[6]
        if kernels.glu_fused(M, hidden, inter, True):
            dht_d = kernels.nf4_linear_bwd_dx_glu_(dy, pd.packed, pd.state, gate, up, dhp, at_d,
                                                   pd.keep, pd.mask_scale, want_t=want_gd)
        else:
            dh, dht_d = kernels.nf4_linear_bwd_dx_hp(dy, pd.packed, pd.state, dhp, at_d, pd.keep,
                                                     pd.mask_scale, want_t=want_gd)
            kernels.silu_mul_bwd_(dh, gate, up)
            del dh
        del dhp
        grads_d = (None, None)
        if want_gd:
            grads_d = kernels.lora_grads(dht_d, ht_d, h, dy, pd.keep, pd.mask_scale,
                                         want_a=need[5], want_b=need[6])
        del h
        # up_proj and gate_proj with d(up) and d(gate) as their incoming gradients; their small
        # launches (dHs, dA / dB) shared, and their input gradients summed (in one launch where
        # the summed dX GEMM takes them)
        (dx, dua, dub), (_, dga, dgb) = lora_backward_group([
            dict(dy=up, x2d=x2d, keep=pu.keep, ht=ht_u, at=at_u, bt=bt_u, packed=pu.packed,
                 state=pu.state, mask_scale=pu.mask_scale, s=pu.s,
                 wants=(need[0], need[3], need[4])),
            dict(dy=gate, x2d=x2d, keep=pg.keep, ht=ht_g, at=at_g, bt=bt_g, packed=pg.packed,
                 state=pg.state, mask_scale=pg.mask_scale, s=pg.s,
                 wants=(need[0], need[1], need[2]))], sum_dx=True)
        grads = [dga, dgb, dua, dub, grads_d[0], grads_d[1]]
        grads = [None if g is None else g.to(t) for g, t in zip(grads, ctx.dtypes)]
        return (dx, *grads, None)


def _is_fp16_4bit(linear):
    """A 4-bit projection computing in fp16: bitsandbytes' or this package's Linear4bit, bare or
    LoRA-wrapped (solution/mlp.py:21-24)."""
    base = getattr(linear, "base_layer", linear)
    weight = getattr(base, "weight", None)
    return getattr(weight, "quant_state", None) is not None and \
        getattr(base, "compute_dtype", None) == torch.float16


def fused_ok(mlp, x16):
    """Whether NF4LoraMLPFunction takes this MLP and fp16 input: every projection a LoRA layer
    with peft's layout (peft_lora.adapter_of) over an NF4 base that the fused kernels take,
    shaped hidden -> inter -> hidden."""
    if not (FUSED_SWIGLU and linear4bit.FUSED_LORA and x16.dim() >= 2):
        return False
    ads = [peft_lora.adapter_of(getattr(mlp, n, None)) for n in _NAMES]
    if any(ad is None for ad in ads):
        return False
    states = [ad.base.weight.quant_state for ad in ads]
    inter, hidden = states[0].shape
    if tuple(states[1].shape) != (inter, hidden) or tuple(states[2].shape) != (hidden, inter):
        return False
    if any(stream.offloaded(ad.base) for ad in ads):
        return False  # offloaded bases take each projection's streamed path
    h_probe = x16.new_empty((1, inter))  # down_proj's input: fp16 on the same device
    return all(peft_lora.takes(ad, probe) for ad, probe in zip(ads, (x16, x16, h_probe)))


def fused_forward(mlp, x16):
    """NF4LoraMLPFunction on an MLP that fused_ok accepts (same dropout draws, in the same
    order, as calling the three projections)."""
    ads = [peft_lora.adapter_of(getattr(mlp, n)) for n in _NAMES]
    lead = x16.shape[:-1]
    x2d = x16.reshape(-1, x16.shape[-1]).contiguous()
    projs, tensors = [], []
    for ad in ads:
        base = ad.base
        keep, mask_scale = None, 1.0
        if ad.dropping():
            # gate and up read x; down reads hidden, [M, inter]
            keep = kernels.keep_bits(ad.keep_mask(x2d, (x2d.shape[0], base.in_features)),
                                     x2d.shape[0], base.in_features)
            mask_scale = 1.0 / (1.0 - ad.p)
        projs.append(_Proj(base.weight.data.view(-1, 1), base.weight.quant_state,
                           _cast_bias_once(base, x16), keep, mask_scale, ad.s))
        tensors += [ad.a, ad.b]
    y = direct.run(NF4LoraMLPFunction, x2d, *tensors, tuple(projs))
    return y.view(*lead, y.shape[-1])


def fp16_forward(mlp, x, previous=None):
    """Qwen2MLP.forward on fp16 activations (solution/mlp.py:33-44): x is cast to fp16 once,
    the block runs in fp16, and the output is cast back to x's dtype.  Inputs the reference's
    guard refuses (another activation, CPU, another dtype, projections that are not fp16 4-bit
    layers) go to `previous`; fp16 inputs are taken as they are."""
    act = getattr(getattr(mlp, "config", None), "hidden_act", "silu")
    if (act != "silu" or not isinstance(x, torch.Tensor) or not x.is_cuda
            or x.dtype not in (torch.float32, torch.float16)
            or not all(_is_fp16_4bit(getattr(mlp, n, None)) for n in _NAMES)):
        if previous is None:
            raise ValueError("input not supported by the fp16 MLP path")
        return previous(mlp, x)
    x16 = x.to(torch.float16)
    if fused_ok(mlp, x16):
        out = fused_forward(mlp, x16)
    else:
        out = mlp.down_proj(silu_mul(mlp.gate_proj(x16), mlp.up_proj(x16)))
    return out.to(x.dtype)


class MLP(torch.nn.Module):
    """Qwen2MLP's layout (gate_proj, up_proj, down_proj, SiLU) over NF4 projections, for when
    transformers' model is not used; forward is fp16_forward."""

    def __init__(self, gate_proj, up_proj, down_proj):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def forward(self, x):
        return fp16_forward(self, x)


def patch_qwen2_mlp_fp16():
    """Install fp16_forward on transformers' Qwen2MLP (solution/mlp.py:27-48); returns whether
    transformers' Qwen2 model is importable."""
    try:
        from transformers.models.qwen2 import modeling_qwen2
    except Exception:
        return False
    cls = modeling_qwen2.Qwen2MLP
    if getattr(cls, "_mindx_fp16", False):
        return True
    previous = cls.forward

    def forward(self, x):
        return fp16_forward(self, x, previous)

    cls.forward = forward
    cls._mindx_fp16 = True
    return True
