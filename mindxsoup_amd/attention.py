"""Qwen2 attention's q/k/v on the fused NF4 + LoRA kernels (the fp16 attention path of
solution/attention.py, rebuilt around this package's grouped launches).

The patched Qwen2Attention.forward keeps transformers' contract (same arguments, same
(output, weights) result, transformers' attention interface for the attention itself) and
changes how q, k and v are made:

  1. the input is cast to fp16 once;
  2. when q, k and v are LoRA layers of one rank, scaling and dropout over NF4 bases (peft's
     layout; peft_lora.adapter_of), all three run as one siblings projection: one launch
     of LoRA row products and one launch of fused GEMMs forward, shared launches backward; any
     other mix of fp16 NF4 projections (bare or LoRA) runs projection by projection, each on
     the fused kernels;
  3. q and k are rotated: in the siblings projection's grouped GEMM (FOLD_ROPE: the epilogue
     rotates before the fp16 store, the bits of a separate rotation launch; the backward's
     inverse rotation is one launch, rope.RotatedHeads), else by one launch over both
     (rope.qkv_rope); v goes to attention as a view, uncopied.

The call takes the original forward when the path cannot serve it (a reason from
`_refusal`): no GPU tensor, a KV cache or attention weights requested, no fp16 autocast (the
original then runs SDPA in fp32), another attention backend or head size, unusual cos / sin, or
a projection that is not an fp16 NF4 layer the fused kernels take.
"""

import torch

from . import linear4bit, peft_lora
from .rope import HEAD_DIM, _angles, as_heads, qkv_rope, rotated_heads

FOLD_ROPE = True  # rotate q and k in the siblings projection's GEMM when that path runs


def _refusal(module, hidden, position_embeddings, past_key_values, kwargs):
    """Why the fp16 path does not take this call, or None when it does."""
    if not isinstance(hidden, torch.Tensor) or not hidden.is_cuda or hidden.dim() != 3:
        return "input is not a [B, T, hidden] GPU tensor"
    if hidden.dtype not in (torch.float16, torch.float32):
        return f"input dtype {hidden.dtype}"
    if past_key_values is not None or kwargs.get("output_attentions", False):
        return "KV cache or attention weights requested"
    if not torch.is_autocast_enabled("cuda") or torch.get_autocast_dtype("cuda") != torch.float16:
        return "no fp16 autocast"
    if getattr(getattr(module, "config", None), "_attn_implementation", None) != "sdpa":
        return "attention backend is not sdpa"
    if getattr(module, "head_dim", None) != HEAD_DIM:
        return "head size is not 128"
    if not isinstance(position_embeddings, (tuple, list)) or len(position_embeddings) != 2:
        return "no (cos, sin) pair"
    b, t, _ = hidden.shape
    for x in position_embeddings:
        if not (isinstance(x, torch.Tensor) and x.is_cuda and x.dim() == 3
                and x.dtype in (torch.float16, torch.float32) and not x.requires_grad
                and x.shape[0] in (1, b) and tuple(x.shape[1:]) == (t, HEAD_DIM)):
            return "cos / sin shape or dtype"
    return None


def _route(proj, x16):
    """How one projection runs on x16: ("lora", Adapter) for a LoRA layer the fused kernels
    take, ("base", layer) for a bare fp16 NF4 layer on the HIP path, or None."""
    ad = peft_lora.adapter_of(proj)
    if ad is not None:
        return ("lora", ad) if peft_lora.takes(ad, x16) else None
    if getattr(proj, "lora_A", None) is not None:  # a LoRA layer this path does not take
        return None
    if getattr(getattr(proj, "weight", None), "quant_state", None) is None or \
            getattr(proj, "compute_dtype", None) != torch.float16:
        return None
    return ("base", proj) if linear4bit._direct_ok(proj, x16) else None


def _siblings(ads, x2d):
    """Proj records for linear4bit.siblings_project, or None when the three adapters differ in
    rank, scaling or dropout (their row products could not share a launch)."""
    if len({(ad.rank, ad.s, ad.p, ad.dropping()) for ad in ads}) != 1:
        return None
    projs = []
    for ad in ads:
        keep, mask_scale = None, 1.0
        if ad.dropping():
            keep = ad.keep_mask(x2d)
            mask_scale = 1.0 / (1.0 - ad.p)
        base = ad.base
        projs.append(linear4bit.Proj(base.weight.data.view(-1, 1), base.weight.quant_state,
                                     linear4bit._cast_bias_once(base, x2d), keep, mask_scale,
                                     ad.s))
    projs = tuple(projs)
    return projs if linear4bit.siblings_ok(projs, x2d.shape[1]) else None


def project_qkv(attn, x16, rope=None):
    """q, k, v fp16 [B, T, heads * 128] of the attention's projections on x16 [B, T, hidden],
    and whether q and k come rotated; None when one of them is not an fp16 NF4 projection the
    fused kernels take.  rope = (cos, sin) fp32 [1 or B, T, 128]: the siblings projection
    rotates q and k in its GEMM (the other paths return them unrotated)."""
    routes = [_route(getattr(attn, n, None), x16) for n in ("q_proj", "k_proj", "v_proj")]
    if any(r is None for r in routes):
        return None
    if all(kind == "lora" for kind, _ in routes) and \
            not any(linear4bit.stream.offloaded(ad.base) for _, ad in routes):
        x2d = x16.reshape(-1, x16.shape[-1]).contiguous()
        projs = _siblings([ad for _, ad in routes], x2d)
        if projs is not None:
            spec = None if rope is None else (2, *rope)
            outs = linear4bit.siblings_project(x2d, projs, [ad.a for _, ad in routes],
                                               [ad.b for _, ad in routes], rope=spec)
            return [y.view(*x16.shape[:-1], y.shape[-1]) for y in outs], rope is not None
    return [peft_lora.fused_project(obj, x16) if kind == "lora" else obj(x16)
            for kind, obj in routes], False


def patch_qwen2_attention_fp16():
    """Install the fp16 q/k/v path on transformers' Qwen2Attention; returns whether
    transformers' Qwen2 model is importable."""
    try:
        from transformers.models.qwen2 import modeling_qwen2
    except Exception:
        return False
    cls = modeling_qwen2.Qwen2Attention
    if getattr(cls, "_mindx_fp16", False):
        return True
    original = cls.forward

    def forward(self, hidden_states, position_embeddings, attention_mask, past_key_values=None,
                **kwargs):
        got = None
        if _refusal(self, hidden_states, position_embeddings, past_key_values, kwargs) is None:
            cos, sin = position_embeddings
            fold = _angles(cos, sin) if FOLD_ROPE else None
            got = project_qkv(self, hidden_states.to(torch.float16), fold)
        if got is None:
            return original(self, hidden_states, position_embeddings, attention_mask,
                            past_key_values, **kwargs)
        (q, k, v), rotated = got
        n_q, n_kv = q.shape[-1] // HEAD_DIM, k.shape[-1] // HEAD_DIM
        if rotated:
            query, key = rotated_heads(q, k, *fold, n_q, n_kv)
            value = as_heads(v, n_kv)
        else:
            query, key, value = qkv_rope(q, None, k, v, None, cos, sin, n_q, n_kv)
        attend = modeling_qwen2.ALL_ATTENTION_FUNCTIONS.get_interface(
            self.config._attn_implementation, modeling_qwen2.eager_attention_forward)
        out, weights = attend(self, query, key, value, attention_mask,
                              dropout=self.attention_dropout if self.training else 0.0,
                              scaling=self.scaling, sliding_window=self.sliding_window, **kwargs)
        # SDPA hands back [B, T, heads, D]; o_proj reads [B, T, heads * D] rows
        out = out.reshape(*hidden_states.shape[:-1], -1).contiguous()
        return self.o_proj(out), weights

    forward._mindx_original = original
    cls.forward = forward
    cls._mindx_fp16 = True
    return True

