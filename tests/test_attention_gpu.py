"""The fp16 attention path (mindxsoup_amd/attention.py) against transformers' own Qwen2Attention
forward on the same NF4 + LoRA projections, as solution/test_attention.py:117-137 checks it:
output, input gradient and LoRA gradients within max relative error 1e-2 under fp16 autocast, at
the model's sizes (hidden 1536, 12 / 2 heads of 128), with and without a padding mask."""

import pytest
import torch

pytestmark = pytest.mark.gpu

HIDDEN, Q_HEADS, KV_HEADS = 1536, 12, 2


def _attention(seed=0, targets=("q_proj", "v_proj")):
    transformers = pytest.importorskip("transformers")
    from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention

    from mindxsoup_amd.loader import replace_with_nf4

    cfg = transformers.Qwen2Config(hidden_size=HIDDEN, num_attention_heads=Q_HEADS,
                                   num_key_value_heads=KV_HEADS, intermediate_size=8960)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(seed)
    attn = Qwen2Attention(cfg, layer_idx=0).cuda()
    replace_with_nf4(attn, lora_targets=targets)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    for m in (getattr(attn, t) for t in targets):  # random B so the branch matters
        with torch.no_grad():
            w = m.lora_B["default"].weight
            w.copy_(torch.randn(w.shape, device="cuda", generator=g) * 0.02)
    return attn


def _padding_mask(batch, n_tokens, lengths):
    causal = torch.ones(n_tokens, n_tokens, dtype=torch.bool, device="cuda").tril()
    keys = torch.arange(n_tokens, device="cuda")[None, :] < \
        torch.tensor(lengths, device="cuda")[:, None]
    return (causal[None] & keys[:, None, :])[:, None]


def _cos_sin(n_tokens):
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, device="cuda").float() / 128))
    freqs = torch.arange(n_tokens, device="cuda").float()[None, :, None] * inv[None, None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def _run(attn, forward, hidden, cos, sin, mask):
    lora = [p for n, p in attn.named_parameters() if "lora_" in n]
    for p in lora:
        p.grad = None
    x = hidden.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.float16):
        out, _ = forward(attn, x, (cos, sin), mask)
    grad = torch.linspace(-1, 1, out.numel(), device="cuda").view_as(out).float()
    (out.float() * grad).sum().backward()
    return [out.detach().float(), x.grad.detach().clone()] + [p.grad.detach().clone() for p in lora]


def _max_rel(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-12)).item()


@pytest.mark.parametrize("batch,n_tokens,masked,targets", [
    (2, 64, False, ("q_proj", "v_proj")), (2, 77, True, ("q_proj", "v_proj")),
    (4, 512, True, ("q_proj", "v_proj")), (2, 77, True, ("q_proj", "k_proj", "v_proj")),
    (4, 512, True, ("q_proj", "k_proj", "v_proj"))])
def test_matches_original_without_dropout(cuda, monkeypatch, batch, n_tokens, masked, targets):
    """LoRA on q and v: each projection on its own fused kernels, then the rotation launch; on
    q, k and v: the three in shared launches (NF4LoraSiblingsFunction) with the rotation in
    their GEMM."""
    from transformers.models.qwen2 import modeling_qwen2

    from mindxsoup_amd import attention, linear4bit

    print(f"case attention batch={batch} tokens={n_tokens} masked={masked} lora={targets}",
          flush=True)
    cls = modeling_qwen2.Qwen2Attention
    original = getattr(cls.forward, "_mindx_original", cls.forward)
    monkeypatch.setattr(cls, "forward", original)
    monkeypatch.setattr(cls, "_mindx_fp16", False, raising=False)
    assert attention.patch_qwen2_attention_fp16() and attention.patch_qwen2_attention_fp16()
    calls, folded = [], []
    real = attention.qkv_rope
    monkeypatch.setattr(attention, "qkv_rope", lambda *a: calls.append(1) or real(*a))
    real_rot = attention.rotated_heads
    monkeypatch.setattr(attention, "rotated_heads",
                        lambda *a: folded.append(1) or real_rot(*a))
    attn = _attention(targets=targets).eval()  # LoRA dropout off
    sib = []
    real_sib = linear4bit.siblings_project
    monkeypatch.setattr(linear4bit, "siblings_project",
                        lambda *a, **k: sib.append(1) or real_sib(*a, **k))
    torch.manual_seed(3)
    hidden = torch.randn(batch, n_tokens, HIDDEN, device="cuda")
    cos, sin = _cos_sin(n_tokens)
    mask = _padding_mask(batch, n_tokens, [n_tokens - 9 * i for i in range(batch)]) \
        if masked else None
    ref = _run(attn, original, hidden, cos, sin, mask)
    ours = _run(attn, cls.forward, hidden, cos, sin, mask)
    assert calls or folded, "the fp16 path was not taken"
    assert bool(sib) == (len(targets) == 3), "q/k/v in shared launches exactly when all have LoRA"
    assert bool(folded) == bool(sib) and bool(calls) != bool(sib), "rotation in the GEMM"
    names = ["output", "grad input"] + [n for n, _ in attn.named_parameters() if "lora_" in n]
    assert len(ours) == len(ref) == 2 + 2 * len(targets)
    for name, a, b in zip(names, ours, ref):
        assert a.shape == b.shape and _max_rel(a, b) < 1e-2, f"{name}: {_max_rel(a, b):.2e}"


@pytest.mark.parametrize("batch,n_tokens,masked", [(1, 1024, False), (2, 77, True),
                                                   (4, 512, True)])
def test_rope_in_the_gemm_gives_the_bits_of_the_rotation_launch(cuda, monkeypatch, batch,
                                                                n_tokens, masked):
    """q, k, v all with LoRA: the rotation folded into the siblings GEMM (attention.FOLD_ROPE)
    against the same path with the rotation as its own launch: output, input gradient and
    LoRA gradients bit for bit (1024 tokens: the 128x64 plan; 2048: 128x128)."""
    from transformers.models.qwen2 import modeling_qwen2

    from mindxsoup_amd import attention

    print(f"case rope fold attention batch={batch} tokens={n_tokens}", flush=True)
    cls = modeling_qwen2.Qwen2Attention
    original = getattr(cls.forward, "_mindx_original", cls.forward)
    monkeypatch.setattr(cls, "forward", original)
    monkeypatch.setattr(cls, "_mindx_fp16", False, raising=False)
    assert attention.patch_qwen2_attention_fp16()
    attn = _attention(targets=("q_proj", "k_proj", "v_proj")).eval()
    torch.manual_seed(4)
    hidden = torch.randn(batch, n_tokens, HIDDEN, device="cuda")
    cos, sin = _cos_sin(n_tokens)
    mask = _padding_mask(batch, n_tokens, [n_tokens - 9 * i for i in range(batch)]) \
        if masked else None
    monkeypatch.setattr(attention, "FOLD_ROPE", False)
    apart = _run(attn, cls.forward, hidden, cos, sin, mask)
    monkeypatch.setattr(attention, "FOLD_ROPE", True)
    folded = _run(attn, cls.forward, hidden, cos, sin, mask)
    names = ["output", "grad input"] + [n for n, _ in attn.named_parameters() if "lora_" in n]
    assert len(folded) == len(apart) == 8
    for name, a, b in zip(names, folded, apart):
        assert torch.equal(a, b), name


def test_without_autocast_takes_original(cuda, monkeypatch):
    from transformers.models.qwen2 import modeling_qwen2

    from mindxsoup_amd import attention

    cls = modeling_qwen2.Qwen2Attention
    original = getattr(cls.forward, "_mindx_original", cls.forward)
    monkeypatch.setattr(cls, "forward", original)
    monkeypatch.setattr(cls, "_mindx_fp16", False, raising=False)
    attention.patch_qwen2_attention_fp16()
    calls = []
    real = attention.qkv_rope
    monkeypatch.setattr(attention, "qkv_rope", lambda *a: calls.append(1) or real(*a))
    attn = _attention().eval()
    hidden = torch.randn(1, 32, HIDDEN, device="cuda")
    cos, sin = _cos_sin(32)
    with torch.no_grad():
        a, _ = cls.forward(attn, hidden, (cos, sin), None)
        b, _ = original(attn, hidden, (cos, sin), None)
    assert not calls and torch.equal(a, b)
