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


def _cpu_state(N=64, K=128, seed=0):
    import numpy as np

    from mindxsoup_amd.quant import QuantState, QuantState2, dynamic_map

    rng = np.random.default_rng(seed)
    nb = N * K // 64
    packed = torch.from_numpy(rng.integers(0, 256, N * K // 2, dtype=np.uint8)).view(-1, 1)
    state = QuantState(shape=(N, K),
                       absmax=torch.from_numpy(rng.integers(0, 256, nb, dtype=np.uint8)),
                       offset=torch.tensor(0.0123, dtype=torch.float32),
                       state2=QuantState2(torch.rand((nb + 255) // 256),
                                          torch.from_numpy(dynamic_map())))
    return packed, state


def test_quant_state_serialized_form():
    """QuantState.as_dict / from_dict in bitsandbytes' serialized form: the tensor keys, the
    packed JSON of the others, and a round trip (prefixes stripped, as from a state dict)."""
    from mindxsoup_amd.nf4 import NF4_VALUES
    from mindxsoup_amd.quant import QuantState, unpack_tensor_to_dict

    _, st = _cpu_state()
    d = st.as_dict(packed=True)
    assert sorted(d) == sorted(["absmax", "quant_map", "nested_absmax", "nested_quant_map",
                                "quant_state.bitsandbytes__nf4"])
    meta = unpack_tensor_to_dict(d["quant_state.bitsandbytes__nf4"])
    assert d["quant_state.bitsandbytes__nf4"].dtype == torch.uint8
    assert meta == {"quant_type": "nf4", "blocksize": 64, "dtype": "float16", "shape": [64, 128],
                    "nested_blocksize": 256, "nested_dtype": "float32",
                    "nested_offset": float(st.offset.item())}
    assert torch.equal(d["quant_map"], torch.from_numpy(NF4_VALUES.copy()))
    back = QuantState.from_dict({"weight." + k: v for k, v in d.items()}, "cpu")
    assert back.shape == st.shape and back.blocksize == 64 and back.nested
    assert torch.equal(back.absmax, st.absmax) and back.offset.item() == st.offset.item()
    assert torch.equal(back.state2.absmax, st.state2.absmax)
    assert torch.equal(back.state2.code, st.state2.code)
    assert torch.equal(QuantState.from_dict(st.as_dict(packed=False), "cpu").absmax, st.absmax)
    bad = dict(d)
    bad["quant_map"] = d["quant_map"] * 2
    with pytest.raises(NotImplementedError):
        QuantState.from_dict(bad, "cpu")


def test_linear4bit_state_dict_round_trip():
    """Linear4bit.state_dict writes bitsandbytes' keys; load_state_dict into a fresh layer
    restores the packed bytes, the quant state and the bias."""
    from mindxsoup_amd.linear4bit import Linear4bit

    packed, st = _cpu_state(seed=3)
    a = Linear4bit(128, 64, bias=True)
    a.set_quantized(packed, st)
    a.bias.data = torch.arange(64, dtype=torch.float16)
    sd = a.state_dict()
    assert sorted(sd) == sorted(["weight", "bias", "weight.absmax", "weight.quant_map",
                                 "weight.nested_absmax", "weight.nested_quant_map",
                                 "weight.quant_state.bitsandbytes__nf4"])
    b = Linear4bit(128, 64, bias=True)
    b.load_state_dict(sd)
    assert torch.equal(b.weight.data, a.weight.data) and torch.equal(b.bias, a.bias)
    qa, qb = a.weight.quant_state, b.weight.quant_state
    assert qb.shape == qa.shape and torch.equal(qb.absmax, qa.absmax)
    assert torch.equal(qb.state2.absmax, qa.state2.absmax)
    assert qb.offset.item() == qa.offset.item()


def test_apply_patches_qwen2_attention_and_rope(monkeypatch):
    modeling_qwen2 = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")

    import mindxsoup_amd
    from mindxsoup_amd import attention, direct, linear4bit, mlp

    cls = modeling_qwen2.Qwen2Attention
    monkeypatch.setattr(cls, "forward", cls.forward)
    monkeypatch.setattr(cls, "_mindx_fp16", False, raising=False)
    monkeypatch.setattr(modeling_qwen2, "apply_rotary_pos_emb", modeling_qwen2.apply_rotary_pos_emb)
    monkeypatch.setattr(modeling_qwen2.Qwen2MLP, "forward", modeling_qwen2.Qwen2MLP.forward)
    monkeypatch.setattr(modeling_qwen2.Qwen2MLP, "_mindx_fp16", False, raising=False)
    for mod, name in ((direct, "enabled"), (linear4bit, "FUSED_GEMM"),
                      (linear4bit, "FUSED_LORA"), (mlp, "FUSED_SWIGLU")):
        monkeypatch.setattr(mod, name, getattr(mod, name))
    original = cls.forward
    mindxsoup_amd.apply()
    assert cls._mindx_fp16 and cls.forward._mindx_original is original
    # the RoPE-only patch is not part of this build: apply_rotary_pos_emb stays transformers'
    assert not getattr(modeling_qwen2.apply_rotary_pos_emb, "_mindx_patched", False)
    # CPU inputs: the patched attention hands the call to the original
    from transformers import Qwen2Config

    cfg = Qwen2Config(hidden_size=256, num_attention_heads=2, num_key_value_heads=1)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    attn = cls(cfg, layer_idx=0)
    x = torch.randn(1, 8, 256)
    cos, sin = torch.ones(1, 8, 128), torch.zeros(1, 8, 128)
    a, _ = cls.forward(attn, x, (cos, sin), None)
    b, _ = original(attn, x, (cos, sin), None)
    assert torch.equal(a, b)
    assert attention._refusal(attn, x, (cos, sin), None, {}) is not None
    assert attention._route(torch.nn.Linear(4, 4), x) is None
