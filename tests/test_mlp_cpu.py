"""The fp16 MLP's host side without a GPU: the SwiGLU-epilogue plan query of the C library, and
apply() installing the MLP forward on transformers' Qwen2MLP with the reference's guard
(solution/mlp.py:33-41: inputs it does not take keep the previous forward)."""

import pytest
import torch


def test_glu_plan_query():
    """The model's MLP shapes (Qwen2.5-1.5B: hidden 1536, intermediate 8960) take the SwiGLU
    epilogue in both directions; narrow outputs, which plan the all-wave kernel, do not."""
    from mindxsoup_amd import kernels

    for M in (1, 37, 1024, 2048):
        assert kernels.glu_fused(M, 8960, 1536, False)   # up_proj forward
        assert kernels.glu_fused(M, 1536, 8960, True)    # down_proj dX
    assert kernels.glu_fused(512, 1536, 8960, False)     # split-K plan: the reduce applies it
    assert not kernels.glu_fused(64, 256, 1536, False)   # all-wave 64x128 tiles
    assert not kernels.glu_fused(64, 1536, 256, True)
    assert not kernels.glu_fused(64, 8960, 1500, False)  # reduction not a multiple of 64
    assert not kernels.glu_fused(0, 8960, 1536, False)


def test_apply_patches_qwen2_mlp(monkeypatch):
    modeling_qwen2 = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")
    from transformers import Qwen2Config

    import mindxsoup_amd
    from mindxsoup_amd import direct, linear4bit, mlp

    cls = modeling_qwen2.Qwen2MLP
    monkeypatch.setattr(cls, "forward", cls.forward)
    monkeypatch.setattr(cls, "_mindx_fp16", False, raising=False)
    for mod, name in ((direct, "enabled"), (linear4bit, "FUSED_GEMM"),
                      (linear4bit, "FUSED_LORA"), (mlp, "FUSED_SWIGLU")):
        monkeypatch.setattr(mod, name, getattr(mod, name))
    cfg = Qwen2Config(hidden_size=64, intermediate_size=128, hidden_act="silu")
    torch.manual_seed(0)
    block = cls(cfg)
    x = torch.randn(2, 5, 64)
    before = block(x)
    original = cls.forward
    mindxsoup_amd.apply()
    assert cls._mindx_fp16 and cls.forward is not original
    assert mlp.FUSED_SWIGLU == mindxsoup_amd.FEATURES["mlp_fused_swiglu"]
    # nn.Linear projections on the CPU: the guard hands the call to the previous forward
    assert torch.equal(block(x), before)
    with pytest.raises(ValueError):
        mlp.fp16_forward(block, x)  # no previous forward to hand it to
