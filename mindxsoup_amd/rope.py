"""Rotary position embedding for Qwen2 q/k, alone (mirror of solution/rope.py) and fused with the
LoRA add and the fp16 cast of q/k/v (mirror of solution/attention.py:28-171, qkv_rope), on the
HIP kernel of csrc/rope.hip (mxs_qkv_rope).

One launch per direction.  Forward: for each position and head, x = base (+ scale * LoRA) in
fp32, q and k rotated (x * cos + rotate_half(x) * sin, transformers' apply_rotary_pos_emb), v
only added, one rounding to the output dtype.  Backward is the same kernel rotating by the
opposite angle, so only cos and sin are saved.  q/k/v are [B, heads, T, 128] views of the
projections' [B, T, heads * 128] memory, read and written through their strides (no copies).
"""

import torch

from . import direct, kernels

HEAD_DIM = 128


def _heads(x, n_heads):
    """[B, T, heads * D] or [B, heads, T, D] -> [B, heads, T, D] view (no copy)
    (solution/attention.py:85-90)."""
    if x.dim() == 3:
        batch, tokens, width = x.shape
        x = x.view(batch, tokens, n_heads, width // n_heads).transpose(1, 2)  # also for T = 0
    return x if x.stride(-1) == 1 else x.contiguous()


def _empty_bhtd(batch, n_heads, n_tokens, dim, dtype, device):
    """[B, heads, T, D] tensor stored as [B, T, heads, D] (solution/attention.py:121-125)."""
    return torch.empty_strided((batch, n_heads, n_tokens, dim),
                               (n_tokens * n_heads * dim, dim, n_heads * dim, 1),
                               dtype=dtype, device=device)


def _cos_sin(cos, sin, batch, n_tokens):
    """fp32 cos / sin rows [1 or B, T, 128] with one layout and unit last stride (fp16 rows are
    widened exactly, as the reference's kernel loads them)."""
    cos, sin = cos.float(), sin.float()
    if cos.dim() == 2:
        cos, sin = cos[None], sin[None]
    if cos.stride() != sin.stride() or cos.stride(-1) != 1:
        cos, sin = cos.contiguous(), sin.contiguous()
    return cos, sin


def _common_dtype(tensors):
    """fp16 when every tensor is fp16, else fp32 (fp16 -> fp32 is exact)."""
    dts = {t.dtype for t in tensors if t is not None}
    return torch.float16 if dts == {torch.float16} else torch.float32


def _as(t, dtype):
    return None if t is None else (t if t.dtype == dtype else t.to(dtype))


def _launch(backward, q_a, q_b, k, v_a, v_b, cos, sin, outs, q_scale=1.0, v_scale=1.0):
    """q_a/k/v_a (+ q_b, v_b): [B, heads, T, D] views; outs: q, k, v destinations (v may be None
    with v_a)."""
    dt = _common_dtype((q_a, q_b, k, v_a, v_b))
    batch, _, n_tokens, _ = q_a.shape
    cos, sin = _cos_sin(cos, sin, batch, n_tokens)
    kernels.qkv_rope(_as(q_a, dt), _as(q_b, dt), _as(k, dt), _as(v_a, dt), _as(v_b, dt), cos,
                     sin, *outs, backward=backward, q_scale=q_scale, v_scale=v_scale)


class QKVRoPEFunction(torch.autograd.Function):
    """fp16 (q_base + q_lora) rotated, k rotated, (v_base + v_lora); inputs are the projections'
    [B, T, heads * D] outputs (LoRA parts may be None, and come times q_scale / v_scale: a power
    of two, so the product is exact either way).  Saves only cos and sin
    (solution/attention.py:127-166)."""

    @staticmethod
    def forward(ctx, q_base, q_lora, k, v_base, v_lora, cos, sin, n_q, n_kv, q_scale=1.0,
                v_scale=1.0):
        q_a, k_h, v_a = _heads(q_base, n_q), _heads(k, n_kv), _heads(v_base, n_kv)
        q_b = None if q_lora is None else _heads(q_lora, n_q)
        v_b = None if v_lora is None else _heads(v_lora, n_kv)
        batch, _, n_tokens, dim = q_a.shape
        outs = tuple(_empty_bhtd(batch, n, n_tokens, dim, torch.float16, q_a.device)
                     for n in (n_q, n_kv, n_kv))
        _launch(False, q_a, q_b, k_h, v_a, v_b, cos, sin, outs, q_scale, v_scale)
        ctx.save_for_backward(cos, sin)
        ctx.scales = (1.0, q_scale, 1.0, 1.0, v_scale)
        ctx.meta = (n_q, n_kv, [None if x is None else x.dtype
                                for x in (q_base, q_lora, k, v_base, v_lora)])
        return outs

    @staticmethod
    def backward(ctx, dq, dk, dv):
        cos, sin = ctx.saved_tensors
        n_q, n_kv, dtypes = ctx.meta
        dq, dk, dv = _heads(dq, n_q), _heads(dk, n_kv), _heads(dv, n_kv)
        batch, _, n_tokens, dim = dq.shape
        grads = tuple(_empty_bhtd(batch, n, n_tokens, dim, torch.float16, dq.device)
                      for n in (n_q, n_kv, n_kv))
        _launch(True, dq, None, dk, dv, None, cos, sin, grads)
        # back to the projections' [B, T, heads * D] shape; the storage already is that layout
        g_q, g_k, g_v = (g.transpose(1, 2).reshape(batch, n_tokens, -1) for g in grads)
        out = []
        for i, (grad, dtype) in enumerate(zip((g_q, g_q, g_k, g_v, g_v), dtypes)):
            if dtype is None or not ctx.needs_input_grad[i]:
                out.append(None)
                continue
            grad = grad.to(dtype)
            out.append(grad * ctx.scales[i] if ctx.scales[i] != 1.0 else grad)
        return (*out, None, None, None, None, None, None)


def qkv_rope(q_base, q_lora, k, v_base, v_lora, cos, sin, n_q, n_kv, q_scale=1.0, v_scale=1.0):
    """(q, k, v) fp16 [B, heads, T, 128] (solution/attention.py:169-171)."""
    return direct.run(QKVRoPEFunction, q_base, q_lora, k, v_base, v_lora, cos, sin, n_q, n_kv,
                      q_scale, v_scale)


def _rope_launch(backward, q, k, cos, sin, q_dtype, k_dtype):
    """Rotate (or rotate back) [B, heads, T, D] q and k (any strides with a unit last one);
    the outputs keep the layout of q and k (solution/rope.py:73-95)."""
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    q_out = torch.empty_like(q, dtype=q_dtype)
    k_out = torch.empty_like(k, dtype=k_dtype)
    if q_out.stride(-1) != 1 or k_out.stride(-1) != 1:
        q_out, k_out = q_out.contiguous(), k_out.contiguous()
    if q_dtype != k_dtype:  # one output dtype per launch
        tmp = torch.empty_like(k_out, dtype=q_dtype)
        _launch(backward, q, None, k, None, None, cos, sin, (q_out, tmp, None))
        k_out.copy_(tmp)
    else:
        _launch(backward, q, None, k, None, None, cos, sin, (q_out, k_out, None))
    return q_out, k_out


class RoPEFunction(torch.autograd.Function):
    """(q * cos + rotate_half(q) * sin, same for k), one launch each way; saves only cos, sin
    (solution/rope.py:98-115)."""

    @staticmethod
    def forward(ctx, q, k, cos, sin, out_dtype=None):
        q_out, k_out = _rope_launch(False, q, k, cos, sin,
                                    out_dtype or torch.result_type(q, cos),
                                    out_dtype or torch.result_type(k, cos))
        ctx.save_for_backward(cos, sin)
        ctx.dtypes = (q.dtype, k.dtype)
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        dq_in, dk_in = _rope_launch(True, dq, dk, cos, sin, *ctx.dtypes)
        return (dq_in if ctx.needs_input_grad[0] else None,
                dk_in if ctx.needs_input_grad[1] else None, None, None, None)


def apply_rope(q, k, cos, sin, unsqueeze_dim=1, out_dtype=None):
    """Same contract as transformers' apply_rotary_pos_emb for [B, heads, T, D] q/k
    (solution/rope.py:118-122); out_dtype writes the rotated q/k in that dtype (math in fp32)."""
    return RoPEFunction.apply(q, k, cos, sin, out_dtype)


_SUPPORTED = (torch.float16, torch.float32)


def _kernel_can_take(q, k, cos, sin, unsqueeze_dim):
    """solution/rope.py:128-140."""
    tensors = (q, k, cos, sin)
    if not all(isinstance(x, torch.Tensor) and x.is_cuda and x.dtype in _SUPPORTED
               for x in tensors):
        return False
    if unsqueeze_dim != 1 or q.dim() != 4 or k.dim() != 4 or cos.dim() != 3:
        return False
    batch, _, n_tokens, dim = q.shape
    return (dim == HEAD_DIM and k.shape[0] == batch and k.shape[2:] == q.shape[2:]
            and cos.shape == sin.shape and cos.shape[0] in (1, batch)
            and tuple(cos.shape[1:]) == (n_tokens, dim) and cos.dtype == sin.dtype
            and not cos.requires_grad and not sin.requires_grad and q.numel() > 0)


def patch_rope():
    """Send modeling_qwen2.apply_rotary_pos_emb through the kernel; anything unusual (CPU, other
    dtypes or shapes, trainable cos/sin) takes the original path (solution/rope.py:143-160).
    Returns whether transformers' Qwen2 model is importable."""
    try:
        from transformers.models.qwen2 import modeling_qwen2
    except Exception:
        return False
    original = modeling_qwen2.apply_rotary_pos_emb
    if getattr(original, "_mindx_patched", False):
        return True

    def apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1):
        if not _kernel_can_take(q, k, cos, sin, unsqueeze_dim):
            return original(q, k, cos, sin, unsqueeze_dim)
        return apply_rope(q, k, cos, sin)

    apply_rotary_pos_emb._mindx_patched = True
    modeling_qwen2.apply_rotary_pos_emb = apply_rotary_pos_emb
    return True
