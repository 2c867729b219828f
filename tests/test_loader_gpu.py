"""A transformers Qwen2 model onto the NF4 path (mindxsoup_amd/loader.py), and its checkpoint in
bitsandbytes' serialized form back into a fresh model (Linear4bit state-dict hooks).  Shapes of
the reference's load test (solution/test_stream.py:180-211: vocab 512, hidden 256, intermediate
512, 2 layers, 4 / 2 heads)."""

import copy

import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _model(seed):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                                   num_hidden_layers=2, num_attention_heads=4,
                                   num_key_value_heads=2, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(seed)
    return transformers.Qwen2ForCausalLM(cfg).half().cuda().eval()


def test_replace_and_reload_qwen2(cuda):
    from mindxsoup_amd.linear4bit import _unpack
    from mindxsoup_amd.loader import replace_with_nf4

    model = _model(0)
    dense = copy.deepcopy(model)
    names = replace_with_nf4(model, lora_targets=("q_proj", "v_proj"))
    assert len(names) == 14 and not any(n.endswith("lm_head") for n in names)
    for name in names:  # the dense twin holds the weights the NF4 layers decode to
        mod = model.get_submodule(name)
        base = getattr(mod, "base_layer", mod)
        dense.get_submodule(name).weight.data = _unpack(base.weight.data,
                                                        base.weight.quant_state, torch.float16)
    ids = torch.randint(0, 512, (2, 40), device=cuda)
    with torch.no_grad():
        got = model(input_ids=ids).logits
        want = dense(input_ids=ids).logits
    # peft starts lora_B at zero: the LoRA layers equal their base here
    err = O.max_rel(got.float().cpu().numpy(), want.float().cpu().numpy())
    assert err < 1e-2, err
    # checkpoint in bitsandbytes' form -> a fresh model built the same way (other seed)
    sd = model.state_dict()
    key = "model.layers.0.self_attn.k_proj.weight"
    assert sd[key].dtype == torch.uint8 and key + ".quant_state.bitsandbytes__nf4" in sd
    assert "model.layers.0.self_attn.q_proj.base_layer.weight.absmax" in sd
    fresh = _model(1)
    replace_with_nf4(fresh, lora_targets=("q_proj", "v_proj"))
    missing, unexpected = fresh.load_state_dict(sd, strict=True)
    assert not missing and not unexpected
    with torch.no_grad():
        again = fresh(input_ids=ids).logits
    assert torch.equal(again, got)
    # and the quant state follows the module between devices
    fresh.cpu()
    st = fresh.model.layers[0].mlp.down_proj.weight.quant_state
    assert st.absmax.device.type == "cpu" and st.state2.absmax.device.type == "cpu"
    fresh.cuda()
    with torch.no_grad():
        assert torch.equal(fresh(input_ids=ids).logits, got)
