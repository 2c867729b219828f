"""Rotary position embedding of Qwen2's q and k on the projections' own memory, with the optional
LoRA add and fp16 cast of the reference's q/k/v kernel (solution/attention.py:28-82), on the HIP
kernel of csrc/rope.hip (mxs_qkv_rope).

The projections write [B, T, heads * 128] rows; attention reads [B, heads, T, 128].  The kernel
takes any (b, h, t) strides with a unit stride inside a head, so nothing is transposed or copied:
inputs are read where the projections put them and outputs are written in the projections'
layout, then handed to attention as [B, heads, T, 128] views.

    forward:   q' = rot(q_base + q_scale * q_lora),  k' = rot(k),  v' = v_base + v_scale * v_lora
    backward:  dq_base = rot^-1(dq'),  dk = rot^-1(dk'),  dq_lora = q_scale * dq_base,
               dv_base = dv',  dv_lora = v_scale * dv'

with rot(x) = x * cos + rotate_half(x) * sin (transformers' apply_rotary_pos_emb) in fp32 and one
rounding to the output dtype.  rot^-1 is the same kernel with the angle negated, so only cos and
sin are kept for the backward.  A v without a LoRA term never enters the kernel: attention gets a
view of v_base itself.
"""

import torch

from . import direct, kernels

HEAD_DIM = 128


def as_heads(x, n_heads):
    """[B, heads, T, D] view of a projection output [B, T, heads * D]; a 4-D tensor is taken as
    already [B, heads, T, D].  A copy is made only when the head dimension is not unit-stride."""
    if x.dim() == 3:
        b, t, width = x.shape
        x = x.unflatten(2, (n_heads, width // n_heads)).permute(0, 2, 1, 3)
    return x if x.stride(-1) == 1 else x.contiguous()


def as_rows(x):
    """[B, T, heads * D] from a [B, heads, T, D] tensor (a view when the memory already has the
    projections' layout, as every output of this module does)."""
    b, h, t, d = x.shape
    return x.permute(0, 2, 1, 3).reshape(b, t, h * d)


def _new_heads(like, n_heads, dtype):
    """An uninitialised [B, heads, T, D] tensor in the projections' memory layout."""
    b, _, t, d = like.shape
    return torch.empty((b, t, n_heads, d), dtype=dtype, device=like.device).permute(0, 2, 1, 3)


def _angles(cos, sin):
    """fp32 cos / sin rows [1 or B, T, D] sharing one layout with a unit last stride (fp16 rows
    widen exactly)."""
    cos = cos.float()
    sin = sin.float()
    if cos.dim() == 2:
        cos, sin = cos.unsqueeze(0), sin.unsqueeze(0)
    if cos.stride(-1) != 1 or cos.stride() != sin.stride():
        cos, sin = cos.contiguous(), sin.contiguous()
    return cos, sin


def _one_dtype(*tensors):
    """The kernel reads one input dtype: fp16 when all are fp16, else fp32 (exact widening)."""
    present = [t for t in tensors if t is not None]
    dt = torch.float16 if all(t.dtype == torch.float16 for t in present) else torch.float32
    return [None if t is None else t.to(dt) for t in tensors]


class QKVRotary(torch.autograd.Function):
    """The rotation of q and k (with the LoRA adds) as one kernel launch each way.  v_base may be
    None: then v is not part of the launch.  Outputs fp16 (q', k', and v' when v_base is given),
    [B, heads, T, D] views of [B, T, heads, D] memory."""

    @staticmethod
    def forward(ctx, n_q, n_kv, q_scale, v_scale, cos, sin, q_base, q_lora, k, v_base, v_lora):
        q_a, q_b, k_h = as_heads(q_base, n_q), None, as_heads(k, n_kv)
        if q_lora is not None:
            q_b = as_heads(q_lora, n_q)
        v_a = v_b = None
        if v_base is not None:
            v_a = as_heads(v_base, n_kv)
            v_b = None if v_lora is None else as_heads(v_lora, n_kv)
        q_a, q_b, k_h, v_a, v_b = _one_dtype(q_a, q_b, k_h, v_a, v_b)
        cos, sin = _angles(cos, sin)
        q_o = _new_heads(q_a, n_q, torch.float16)
        k_o = _new_heads(k_h, n_kv, torch.float16)
        v_o = None if v_a is None else _new_heads(v_a, n_kv, torch.float16)
        kernels.qkv_rope(q_a, q_b, k_h, v_a, v_b, cos, sin, q_o, k_o, v_o, backward=False,
                         q_scale=q_scale, v_scale=v_scale)
        ctx.save_for_backward(cos, sin)
        ctx.meta = (n_q, n_kv, q_scale, v_scale,
                    tuple(None if t is None else (t.dim(), t.dtype)
                          for t in (q_base, q_lora, k, v_base, v_lora)))
        return (q_o, k_o) if v_o is None else (q_o, k_o, v_o)

    @staticmethod
    def backward(ctx, dq, dk, dv=None):
        cos, sin = ctx.saved_tensors
        n_q, n_kv, q_scale, v_scale, kinds = ctx.meta
        need = ctx.needs_input_grad  # (autograd hands zeros, not None, for unused outputs)
        dq_h, dk_h = _one_dtype(as_heads(dq, n_q), as_heads(dk, n_kv))
        gq = _new_heads(dq_h, n_q, torch.float16)
        gk = _new_heads(dk_h, n_kv, torch.float16)
        kernels.qkv_rope(dq_h, None, dk_h, None, None, cos, sin, gq, gk, None, backward=True)

        def back(g, kind, scale=1.0):
            if kind is None:
                return None
            dim, dtype = kind
            g = g if dim == 4 else as_rows(g)
            g = g.to(dtype)
            return g * scale if scale != 1.0 else g

        grads = [back(gq, kinds[0]), back(gq, kinds[1], q_scale), back(gk, kinds[2]), None, None]
        if kinds[3] is not None and dv is not None:
            grads[3] = back(dv, kinds[3])
            grads[4] = back(dv, kinds[4], v_scale)
        grads = [g if need[6 + i] else None for i, g in enumerate(grads)]
        return (None, None, None, None, None, None, *grads)


class RotatedHeads(torch.autograd.Function):
    """q and k that a projection already returns rotated (the RoPE folded into the grouped q/k/v
    GEMM, kernels.nf4_linear_fwd_hp_group with rope): forward, the [B, heads, T, D] views of
    those outputs, no launch; backward, the inverse rotation of dq and dk in one launch (the
    backward half of QKVRotary), handed to the projection node, whose backward is that of the
    unrotated outputs.  Forward and backward together are QKVRotary's."""

    @staticmethod
    def forward(ctx, n_q, n_kv, cos, sin, q_rot, k_rot):
        cos, sin = _angles(cos, sin)
        ctx.save_for_backward(cos, sin)
        ctx.n = (n_q, n_kv)
        return as_heads(q_rot, n_q), as_heads(k_rot, n_kv)

    @staticmethod
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        n_q, n_kv = ctx.n
        dq_h, dk_h = _one_dtype(as_heads(dq, n_q), as_heads(dk, n_kv))
        gq = _new_heads(dq_h, n_q, torch.float16)
        gk = _new_heads(dk_h, n_kv, torch.float16)
        kernels.qkv_rope(dq_h, None, dk_h, None, None, cos, sin, gq, gk, None, backward=True)
        return None, None, None, None, as_rows(gq), as_rows(gk)


def rotated_heads(q_rot, k_rot, cos, sin, n_q, n_kv):
    """(q, k) [B, heads, T, 128] for attention from projection outputs [B, T, heads * 128] that
    are already rotated (RotatedHeads)."""
    return direct.run(RotatedHeads, n_q, n_kv, cos, sin, q_rot, k_rot)


def qkv_rope(q_base, q_lora, k, v_base, v_lora, cos, sin, n_q, n_kv, q_scale=1.0, v_scale=1.0):
    """(q, k, v) for attention, fp16 [B, heads, T, 128] (the reference's qkv_rope interface,
    solution/attention.py:169-171).  Inputs are the projections' [B, T, heads * 128] outputs (or
    [B, heads, T, 128] views); q_lora / v_lora (None for no LoRA term) are the LoRA branches'
    outputs, which the kernel multiplies by q_scale / v_scale in fp32 (a power of two gives the
    bits of a pre-scaled input).  An fp16 v without a LoRA term is returned as a view of
    v_base."""
    if v_lora is None and v_base.dtype == torch.float16:
        q, k = direct.run(QKVRotary, n_q, n_kv, q_scale, v_scale, cos, sin, q_base, q_lora, k,
                          None, None)
        return q, k, as_heads(v_base, n_kv)
    return direct.run(QKVRotary, n_q, n_kv, q_scale, v_scale, cos, sin, q_base, q_lora, k,
                      v_base, v_lora)
