"""RoPE and the fused q/k/v LoRA-add + RoPE + cast (mindxsoup_amd/rope.py on csrc/rope.hip).

Bars: bit-exact against the oracle's restatement (oracle_qkv_rope) on the same inputs, forward
and backward, fp16 and fp32; and the reference's own tests' comparisons against fp32 PyTorch
math with transformers' formula (solution/test_rope.py:48-150: 1e-5 for fp32, 2e-3 for fp16;
solution/test_attention.py:190-246: 2e-3, and a power-of-two LoRA scale bit-exact).
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


def model_like_qk(dev, batch, n_q, n_k, n_tokens, dtype):
    """q and k as Qwen2Attention makes them: a [B, T, heads, D] buffer seen as [B, heads, T, D]."""
    q = torch.randn(batch, n_tokens, n_q * HEAD_DIM, device=dev).to(dtype)
    k = torch.randn(batch, n_tokens, n_k * HEAD_DIM, device=dev).to(dtype)
    q = q.view(batch, n_tokens, n_q, HEAD_DIM).transpose(1, 2).detach().requires_grad_(True)
    k = k.view(batch, n_tokens, n_k, HEAD_DIM).transpose(1, 2).detach().requires_grad_(True)
    assert not q.is_contiguous() and not k.is_contiguous()
    return q, k


def model_like_cos_sin(dev, batch, n_tokens, dtype, theta=1e6):
    """Qwen2RotaryEmbedding: freqs = pos * inv_freq, emb = cat(freqs, freqs)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, HEAD_DIM, 2, device=dev).float() / HEAD_DIM))
    pos = torch.arange(n_tokens, device=dev).float()[None, :].expand(batch, -1)
    pos = pos + torch.arange(batch, device=dev)[:, None] * 3  # rows differ, like left padding
    freqs = pos[:, :, None] * inv_freq[None, None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def run_both(q, k, cos, sin):
    from mindxsoup_amd.rope import apply_rope

    ref_q, ref_k = reference(q, k, cos, sin)
    grad_q, grad_k = torch.randn_like(ref_q), torch.randn_like(ref_k)
    ref_dq, ref_dk = torch.autograd.grad((ref_q, ref_k), (q, k), (grad_q, grad_k))
    out_q, out_k = apply_rope(q, k, cos, sin)
    dq, dk = torch.autograd.grad((out_q, out_k), (q, k), (grad_q, grad_k))
    return (out_q, out_k, dq, dk), (ref_q, ref_k, ref_dq, ref_dk)


def _flat(x):
    """[B, heads, T, D] -> numpy [B, T, heads * D]."""
    b, h, t, d = x.shape
    return x.detach().transpose(1, 2).reshape(b, t, h * d).cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("shape", [(4, 12, 2, 512), (3, 12, 2, 77)])
def test_rope_matches_reference(cuda, dtype, shape):
    """solution/test_rope.py:48-62."""
    print(f"case rope {dtype} {shape}", flush=True)
    torch.manual_seed(0)
    batch, n_q, n_k, n_tokens = shape
    q, k = model_like_qk(cuda, batch, n_q, n_k, n_tokens, dtype)
    cos, sin = model_like_cos_sin(cuda, batch, n_tokens, dtype)
    ours, ref = run_both(q, k, cos, sin)
    tol = TOLERANCE[dtype]
    for name, a, b in zip(("q", "k", "dq", "dk"), ours, ref):
        assert a.dtype == b.dtype and a.shape == b.shape, name
        torch.testing.assert_close(a.float(), b.float(), rtol=tol, atol=tol, msg=name)
    # no hidden copies: outputs keep the [B, T, heads, D] layout of q and k
    assert ours[0].stride() == q.stride() and ours[1].stride() == k.stride()


def test_cos_sin_with_batch_one(cuda):
    """position_ids of shape [1, T] give cos/sin [1, T, D], broadcast over the batch."""
    torch.manual_seed(0)
    q, k = model_like_qk(cuda, 4, 12, 2, 100, torch.float32)
    cos, sin = model_like_cos_sin(cuda, 1, 100, torch.float32)
    ours, ref = run_both(q, k, cos, sin)
    for a, b in zip(ours, ref):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_mixed_dtypes_promote_like_pytorch(cuda):
    """fp16 q/k with fp32 cos/sin: outputs fp32 as in the original, grads in the input dtype."""
    torch.manual_seed(0)
    q, k = model_like_qk(cuda, 2, 12, 2, 33, torch.float16)
    cos, sin = model_like_cos_sin(cuda, 2, 33, torch.float32)
    ours, ref = run_both(q, k, cos, sin)
    for a, b in zip(ours, ref):
        assert a.dtype == b.dtype
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-3, atol=2e-3)


def test_contiguous_inputs_and_out_dtype(cuda):
    from mindxsoup_amd.rope import apply_rope

    torch.manual_seed(0)
    q = torch.randn(2, 12, 50, HEAD_DIM, device=cuda, requires_grad=True)
    k = torch.randn(2, 2, 50, HEAD_DIM, device=cuda, requires_grad=True)
    cos, sin = model_like_cos_sin(cuda, 2, 50, torch.float32)
    ours, ref = run_both(q, k, cos, sin)
    for a, b in zip(ours, ref):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
    # fp32 q/k with out_dtype=fp16: the fp32 rotation rounded once; grads come back in fp32
    ref_q, ref_k = (x.half() for x in reference(q, k, cos, sin))
    grads = (torch.randn_like(ref_q), torch.randn_like(ref_k))
    ref_dq, ref_dk = torch.autograd.grad((ref_q, ref_k), (q, k), grads)
    out_q, out_k = apply_rope(q, k, cos, sin, out_dtype=torch.float16)
    dq, dk = torch.autograd.grad((out_q, out_k), (q, k), grads)
    for a, b in ((out_q, ref_q), (out_k, ref_k), (dq, ref_dq), (dk, ref_dk)):
        assert a.dtype == b.dtype
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-3, atol=2e-3)


def test_patch_routes_cuda_and_falls_back(cuda, monkeypatch):
    modeling_qwen2 = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")
    from mindxsoup_amd.rope import patch_rope

    monkeypatch.setattr(modeling_qwen2, "apply_rotary_pos_emb",
                        modeling_qwen2.apply_rotary_pos_emb)  # restored after the test
    assert patch_rope() and patch_rope()  # idempotent
    patched = modeling_qwen2.apply_rotary_pos_emb
    assert getattr(patched, "_mindx_patched", False)
    torch.manual_seed(0)
    q, k = model_like_qk(cuda, 2, 12, 2, 40, torch.float32)
    cos, sin = model_like_cos_sin(cuda, 2, 40, torch.float32)
    out_q, out_k = patched(q, k, cos, sin)
    assert out_q.grad_fn is not None and "RoPEFunction" in type(out_q.grad_fn).__name__
    ref_q, ref_k = reference(q, k, cos, sin)
    torch.testing.assert_close(out_q, ref_q, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(out_k, ref_k, rtol=1e-5, atol=1e-5)
    cpu = [x.detach().cpu() for x in (q, k, cos, sin)]  # CPU tensors take the original code
    cpu_q, cpu_k = patched(*cpu)
    ref_q, ref_k = reference(*cpu)
    torch.testing.assert_close(cpu_q, ref_q)
    torch.testing.assert_close(cpu_k, ref_k)


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
