"""Qwen2 attention with fp16 q/k/v (mirror of solution/attention.py:174-290): the input is cast to
fp16 once, the three projections run on the NF4 path and return fp16, and one launch
(rope.qkv_rope on csrc/rope.hip) adds any separate LoRA outputs, rotates q and k and writes the
fp16 q/k/v that SDPA reads.  With this package's LoraLinear4bit the LoRA term is already inside
each projection's GEMM, so qkv_rope only rotates.  Anything the fast path does not take (CPU, a
KV cache, another attention backend, no fp16 autocast, projections that are not fp16 4-bit
layers) goes to transformers' own forward.
"""

import math

import torch

from .linear4bit import LoraLinear4bit
from .rope import HEAD_DIM, qkv_rope


def _is_fp16_4bit(linear):
    base = getattr(linear, "base_layer", linear)
    return getattr(getattr(base, "weight", None), "quant_state", None) is not None and \
        getattr(base, "compute_dtype", None) == torch.float16


def _split_projection(proj):
    """(layer to call on the fp16 input, separate LoRA function or None, its scale), or None when
    the fast path does not take the projection (solution/attention.py:174-202).  This package's
    LoraLinear4bit and a bare fp16 4-bit layer are called whole; peft's LoRA wrapper around a
    4-bit layer gives its base and its LoRA branch, whose power-of-two scaling the kernel
    applies (exact in fp16 and fp32)."""
    if isinstance(proj, LoraLinear4bit) or getattr(proj, "lora_A", None) is None:
        return (proj, None, 1.0) if _is_fp16_4bit(proj) else None
    base = getattr(proj, "base_layer", None)
    if not _is_fp16_4bit(base):
        return None
    if getattr(proj, "disable_adapters", True) or getattr(proj, "merged", True):
        return None
    lora_a = proj.lora_A
    active = list(getattr(proj, "active_adapters", []))
    if len(active) != 1 or active[0] not in lora_a.keys() \
            or active[0] in getattr(proj, "lora_variant", {}):
        return None
    name = active[0]
    scaling = proj.scaling[name]
    exact = isinstance(scaling, (int, float)) and scaling > 0 and \
        math.frexp(scaling)[0] == 0.5 and 2.0 ** -8 <= scaling <= 2.0 ** 8

    def lora(x):  # peft's LoRA branch under autocast
        out = proj.lora_B[name](proj.lora_A[name](proj.lora_dropout[name](x)))
        return out if exact else out * scaling

    return base, lora, (float(scaling) if exact else 1.0)


def _fast_path_ok(module, hidden_states, position_embeddings, past_key_values, kwargs):
    """solution/attention.py:205-227."""
    if (not isinstance(hidden_states, torch.Tensor) or not hidden_states.is_cuda
            or hidden_states.dtype not in (torch.float32, torch.float16)
            or hidden_states.dim() != 3 or past_key_values is not None
            or kwargs.get("output_attentions", False)):
        return False
    if not (torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.float16):
        return False  # without fp16 autocast transformers runs SDPA in fp32: keep it
    config = getattr(module, "config", None)
    if getattr(config, "_attn_implementation", None) != "sdpa" or \
            getattr(module, "head_dim", None) != HEAD_DIM:
        return False
    if not isinstance(position_embeddings, (tuple, list)) or len(position_embeddings) != 2:
        return False
    cos, sin = position_embeddings
    batch, n_tokens, _ = hidden_states.shape
    return all(isinstance(x, torch.Tensor) and x.is_cuda and x.dim() == 3
               and x.dtype in (torch.float32, torch.float16) and not x.requires_grad
               and x.shape[0] in (1, batch) and tuple(x.shape[1:]) == (n_tokens, HEAD_DIM)
               for x in (cos, sin))


def patch_qwen2_attention_fp16():
    """Send Qwen2Attention.forward through the fp16 path (solution/attention.py:230-290); returns
    whether transformers' Qwen2 model is importable."""
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
        parts = None
        if _fast_path_ok(self, hidden_states, position_embeddings, past_key_values, kwargs):
            parts = [_split_projection(getattr(self, name, None))
                     for name in ("q_proj", "k_proj", "v_proj")]
        if parts is None or any(p is None for p in parts) or parts[1][1] is not None:
            return original(self, hidden_states, position_embeddings, attention_mask,
                            past_key_values, **kwargs)
        (q_layer, q_lora, q_scale), (k_layer, _, _), (v_layer, v_lora, v_scale) = parts
        input_shape = hidden_states.shape[:-1]
        x16 = hidden_states.to(torch.float16)
        # the order of the original forward: q (base, LoRA), k, v (base, LoRA)
        q_base = q_layer(x16)
        q_add = None if q_lora is None else q_lora(hidden_states)
        k = k_layer(x16)
        v_base = v_layer(x16)
        v_add = None if v_lora is None else v_lora(hidden_states)
        n_q, n_kv = q_base.shape[-1] // self.head_dim, k.shape[-1] // self.head_dim
        cos, sin = position_embeddings
        query, key, value = qkv_rope(q_base, q_add, k, v_base, v_add, cos, sin, n_q, n_kv,
                                     q_scale, v_scale)
        attention_interface = modeling_qwen2.ALL_ATTENTION_FUNCTIONS.get_interface(
            self.config._attn_implementation, modeling_qwen2.eager_attention_forward)
        attn_output, attn_weights = attention_interface(
            self, query, key, value, attention_mask,
            dropout=0.0 if not self.training else self.attention_dropout,
            scaling=self.scaling, sliding_window=self.sliding_window, **kwargs)
        attn_output = attn_output.reshape(*input_shape, -1).contiguous()
        return self.o_proj(attn_output), attn_weights

    forward._mindx_original = original
    cls.forward = forward
    cls._mindx_fp16 = True
    return True
