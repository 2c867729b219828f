"""The q/k rotation and q/k/v LoRA-add + RoPE + cast of the fp16 attention path
(mindxsoup_amd/rope.py on csrc/rope.hip).

Bars: bit-exact against the oracle's restatement (oracle_qkv_rope) on the same inputs, forward
and backward, fp16 and fp32 in and out; and the reference's own comparisons against fp32 PyTorch
math with transformers' formula (solution/test_rope.py:48-62 and solution/test_attention.py
:190-246: 2e-3 for fp16 outputs, and a power-of-two LoRA scale bit-exact).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

HEAD_DIM, Q_HEADS, KV_HEADS = 128, 12, 2
TOLERANCE = {torch.float16: 2e-3, torch.float32: 1e-5}


def rotate_half(x):
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def reference(q, k, cos, sin, unsqueeze_dim=1):
    """transformers' apply_rotary_pos_emb math (modeling_qwen2.py)."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)


def model_like_cos_sin(dev, batch, n_tokens, dtype, theta=1e6):
    """Qwen2RotaryEmbedding: freqs = pos * inv_freq, emb = cat(freqs, freqs)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, HEAD_DIM, 2, device=dev).float() / HEAD_DIM))
    pos = torch.arange(n_tokens, device=dev).float()[None, :].expand(batch, -1)
    pos = pos + torch.arange(batch, device=dev)[:, None] * 3  # rows differ, like left padding
    freqs = pos[:, :, None] * inv_freq[None, None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _flat(x):
    """[B, heads, T, D] -> numpy [B, T, heads * D]."""
    b, h, t, d = x.shape
    return x.detach().transpose(1, 2).reshape(b, t, h * d).cpu().numpy()


def _rows(dev, batch, n_tokens, heads, dtype=torch.float16):
    """A projection's output as Qwen2Attention gets it: [B, T, heads * D]."""
    return torch.randn(batch, n_tokens, heads * HEAD_DIM, device=dev).to(dtype) \
        .requires_grad_(True)


def _heads(x, n):
    b, t, _ = x.shape
    return x.view(b, t, n, HEAD_DIM).transpose(1, 2)


def _rotate_both(q, k, v, cos, sin):
    """qkv_rope without LoRA terms and transformers' formula in fp32 (rounded to fp16), with
    gradients of both for the same incoming gradients."""
    from mindxsoup_amd.rope import qkv_rope

    ref_q, ref_k = reference(_heads(q.float(), Q_HEADS), _heads(k.float(), KV_HEADS), cos.float(),
                             sin.float())
    ref = (ref_q.half(), ref_k.half(), _heads(v, KV_HEADS))
    grads = [torch.randn_like(r) for r in ref]
    ref_grads = torch.autograd.grad(ref, (q, k, v), grads)
    ours = qkv_rope(q, None, k, v, None, cos, sin, Q_HEADS, KV_HEADS)
    our_grads = torch.autograd.grad(ours, (q, k, v), grads)
    return ours, ref, our_grads, ref_grads


@pytest.mark.parametrize("shape", [(4, 512), (3, 77)])
@pytest.mark.parametrize("cos_dtype", [torch.float32, torch.float16])
def test_rotation_matches_transformers_math(cuda, shape, cos_dtype):
    """The rotation of the attention path on model-like q/k (solution/test_rope.py:48-62's
    comparison, fp16 tolerance 2e-3): values, input gradients, and the layout promises (q', k'
    in the projections' [B, T, heads, D] memory; v' is v itself, no copy)."""
    print(f"case rope {shape} cos {cos_dtype}", flush=True)
    torch.manual_seed(0)
    batch, n_tokens = shape
    q, k, v = (_rows(cuda, batch, n_tokens, h) for h in (Q_HEADS, KV_HEADS, KV_HEADS))
    cos, sin = model_like_cos_sin(cuda, batch, n_tokens, cos_dtype)
    ours, ref, our_grads, ref_grads = _rotate_both(q, k, v, cos, sin)
    for name, a, b in zip(("q", "k", "v", "dq", "dk", "dv"), ours + our_grads, ref + ref_grads):
        assert a.dtype == b.dtype and a.shape == b.shape, name
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-3, atol=2e-3, msg=name)
    assert ours[0].stride() == _heads(q, Q_HEADS).stride()
    assert ours[1].stride() == _heads(k, KV_HEADS).stride()
    assert ours[2].data_ptr() == v.data_ptr()


def test_cos_sin_with_batch_one(cuda):
    """position_ids of shape [1, T] give cos/sin [1, T, D], broadcast over the batch."""
    torch.manual_seed(0)
    q, k, v = (_rows(cuda, 4, 100, h) for h in (Q_HEADS, KV_HEADS, KV_HEADS))
    cos, sin = model_like_cos_sin(cuda, 1, 100, torch.float32)
    ours, ref, our_grads, ref_grads = _rotate_both(q, k, v, cos, sin)
    for a, b in zip(ours + our_grads, ref + ref_grads):
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-3, atol=2e-3)


def _proj(dev, batch, n_tokens, heads):
    return (torch.randn(batch, n_tokens, heads * HEAD_DIM, device=dev) * 2).half() \
        .requires_grad_(True)


@pytest.mark.parametrize("n_tokens", [16, 300])
def test_qkv_rope_kernel_against_pytorch(cuda, n_tokens):
    """solution/test_attention.py:190-223: (base + LoRA) rotated -> fp16, against fp32 math."""
    from mindxsoup_amd.rope import qkv_rope

    print(f"case qkv_rope tokens={n_tokens}", flush=True)
    torch.manual_seed(0)
    batch = 3
    q_base, q_lora, k, v_base, v_lora = (_proj(cuda, batch, n_tokens, h) for h in
                                         (Q_HEADS, Q_HEADS, KV_HEADS, KV_HEADS, KV_HEADS))
    cos, sin = model_like_cos_sin(cuda, batch, n_tokens, torch.float32)

    def heads(x, n):
        return x.view(batch, n_tokens, n, HEAD_DIM).transpose(1, 2)

    inputs_ = (q_base, q_lora, k, v_base, v_lora)
    ref_q, ref_k = reference(heads(q_base.float() + q_lora.float(), Q_HEADS),
                             heads(k.float(), KV_HEADS), cos, sin)
    ref = (ref_q.half(), ref_k.half(), heads(v_base.float() + v_lora.float(), KV_HEADS).half())
    grads = [torch.randn_like(r) for r in ref]
    ref_grads = torch.autograd.grad(ref, inputs_, grads)
    ours = qkv_rope(q_base, q_lora, k, v_base, v_lora, cos, sin, Q_HEADS, KV_HEADS)
    our_grads = torch.autograd.grad(ours, inputs_, grads)
    for a, b in zip(ours, ref):
        assert a.dtype == torch.float16 and a.shape == b.shape
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-3, atol=2e-3)
    for a, b in zip(our_grads, ref_grads):
        assert a.dtype == b.dtype and a.shape == b.shape
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-3, atol=2e-3)


def test_power_of_two_lora_scale_in_the_kernel_is_bit_exact(cuda):
    """solution/test_attention.py:226-246."""
    from mindxsoup_amd.rope import qkv_rope

    torch.manual_seed(1)
    batch, n_tokens = 2, 37
    q_base, q_lora, k, v_base, v_lora = (_proj(cuda, batch, n_tokens, h) for h in
                                         (Q_HEADS, Q_HEADS, KV_HEADS, KV_HEADS, KV_HEADS))
    cos, sin = model_like_cos_sin(cuda, batch, n_tokens, torch.float32)
    inputs_ = (q_base, q_lora, k, v_base, v_lora)
    want = qkv_rope(q_base, q_lora * 2.0, k, v_base, v_lora * 2.0, cos, sin, Q_HEADS, KV_HEADS)
    got = qkv_rope(q_base, q_lora, k, v_base, v_lora, cos, sin, Q_HEADS, KV_HEADS, 2.0, 2.0)
    grads = [torch.randn_like(r) for r in want]
    want_grads = torch.autograd.grad(want, inputs_, grads)
    got_grads = torch.autograd.grad(got, inputs_, grads)
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    for a, b in zip(got_grads, want_grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize("in_dt,out_dt", [(torch.float16, torch.float16),
                                          (torch.float32, torch.float32),
                                          (torch.float32, torch.float16)])
@pytest.mark.parametrize("cos_batch", [1, 3])
@pytest.mark.parametrize("backward", [False, True])
def test_kernel_matches_oracle_bit_for_bit(cuda, in_dt, out_dt, cos_batch, backward):
    """mxs_qkv_rope against oracle_qkv_rope on the same inputs: q/k/v with LoRA terms, both
    directions, both dtypes, cos / sin per batch row or shared."""
    from mindxsoup_amd import kernels

    print(f"case rope oracle {in_dt}->{out_dt} cos_batch={cos_batch} bwd={backward}", flush=True)
    torch.manual_seed(5)
    B, T = 3, 45
    cos, sin = model_like_cos_sin(cuda, cos_batch, T, torch.float32)
    cos = cos + 0.01 * torch.randn_like(cos)  # halves that differ
    ins = [(torch.randn(B, T, h * HEAD_DIM, device=cuda) * 3).to(in_dt)
           for h in (Q_HEADS, Q_HEADS, KV_HEADS, KV_HEADS, KV_HEADS)]
    if backward:
        ins[1] = ins[4] = None  # the backward launch has no LoRA terms
    outs = [torch.empty(B, T, h * HEAD_DIM, device=cuda, dtype=out_dt)
            for h in (Q_HEADS, KV_HEADS, KV_HEADS)]

    def heads(x, n):
        return None if x is None else x.view(B, T, n, HEAD_DIM).transpose(1, 2)

    hn = (Q_HEADS, Q_HEADS, KV_HEADS, KV_HEADS, KV_HEADS)
    kernels.qkv_rope(*[heads(x, n) for x, n in zip(ins, hn)], cos, sin,
                     *[heads(x, n) for x, n in zip(outs, (Q_HEADS, KV_HEADS, KV_HEADS))],
                     backward=backward, q_scale=2.0, v_scale=0.5)
    torch.cuda.synchronize()
    npd = np.float16 if out_dt == torch.float16 else np.float32
    want = O.qkv_rope(*[None if x is None else x.cpu().numpy() for x in ins],
                      cos.cpu().numpy(), sin.cpu().numpy(), Q_HEADS, KV_HEADS, 2.0, 0.5,
                      backward=backward, out_dtype=npd)
    for got, ref in zip(outs, want):
        g = got.cpu().numpy()
        assert g.dtype == ref.dtype and np.array_equal(g.view(np.uint8), ref.view(np.uint8))


def test_strided_gradients_and_empty(cuda):
    """Gradients in attention's own layout ([B, heads, T, D] contiguous) go through the strides;
    zero tokens launch nothing."""
    from mindxsoup_amd.rope import qkv_rope

    torch.manual_seed(7)
    B, T = 2, 29
    q_base, k, v_base = (_proj(cuda, B, T, h) for h in (Q_HEADS, KV_HEADS, KV_HEADS))
    cos, sin = model_like_cos_sin(cuda, B, T, torch.float32)
    q, kk, v = qkv_rope(q_base, None, k, v_base, None, cos, sin, Q_HEADS, KV_HEADS)
    gq = torch.randn(B, Q_HEADS, T, HEAD_DIM, device=cuda).half()  # contiguous per head
    gk = torch.randn(B, KV_HEADS, T, HEAD_DIM, device=cuda).half()
    gv = torch.randn(B, KV_HEADS, T, HEAD_DIM, device=cuda).half()
    dq, dk, dv = torch.autograd.grad((q, kk, v), (q_base, k, v_base), (gq, gk, gv))
    want_q = O.qkv_rope(_flat(gq), None, _flat(gk), None, None, cos.cpu().numpy(),
                        sin.cpu().numpy(), Q_HEADS, KV_HEADS, backward=True)
    assert np.array_equal(dq.cpu().numpy(), want_q[0]) and np.array_equal(dk.cpu().numpy(),
                                                                          want_q[1])
    assert np.array_equal(dv.cpu().numpy(), _flat(gv))
    z = [torch.zeros(B, 0, h * HEAD_DIM, device=cuda, dtype=torch.float16)
         for h in (Q_HEADS, KV_HEADS, KV_HEADS)]
    c0, s0 = cos[:, :0], sin[:, :0]
    out = qkv_rope(z[0], None, z[1], z[2], None, c0, s0, Q_HEADS, KV_HEADS)
    assert [tuple(o.shape) for o in out] == [(B, Q_HEADS, 0, HEAD_DIM), (B, KV_HEADS, 0, HEAD_DIM),
                                             (B, KV_HEADS, 0, HEAD_DIM)]
    torch.cuda.synchronize()
