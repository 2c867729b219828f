"""Decoder NF4 weights in pinned host memory, streamed to the GPU a layer at a time
(mindxsoup_amd/stream.py, mirror of solution/stream.py).  The streamed bytes are the resident
bytes, so every output and input gradient must equal the resident model's bit for bit
(solution/stream.py:12-14; the reference's own check is solution/test_stream.py:120-177)."""

import pytest
import torch

pytestmark = pytest.mark.gpu

HIDDEN, KV, INTER = 256, 128, 512


class Block(torch.nn.Module):
    """The seven projections of a Qwen2 decoder layer at small sizes, all on one input."""

    def __init__(self, gen, device):
        super().__init__()
        from mindxsoup_amd.linear4bit import Linear4bit

        def lin(k, n):
            w = torch.randn(n, k, generator=gen, device=device) * k ** -0.5
            return Linear4bit.from_weight(w.half())

        self.q_proj = lin(HIDDEN, HIDDEN)
        self.k_proj, self.v_proj = lin(HIDDEN, KV), lin(HIDDEN, KV)
        self.o_proj = lin(HIDDEN, HIDDEN)
        self.gate_proj, self.up_proj = lin(HIDDEN, INTER), lin(HIDDEN, INTER)
        self.down_proj = lin(INTER, HIDDEN)

    def forward(self, x):
        kv = self.k_proj(x) + self.v_proj(x)
        a = self.o_proj(self.q_proj(x)) + torch.cat([kv, kv], dim=-1)
        return x + a + self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


class Toy(torch.nn.Module):
    def __init__(self, n_layers, seed, device):
        super().__init__()
        gen = torch.Generator(device=device).manual_seed(seed)
        self.model = torch.nn.Module()
        self.model.layers = torch.nn.ModuleList([Block(gen, device) for _ in range(n_layers)])

    def forward(self, x):
        for layer in self.model.layers:
            x = layer(x)
        return x


@pytest.fixture
def streaming(monkeypatch):
    from mindxsoup_amd import stream

    monkeypatch.setattr(stream, "enabled", True)
    stream.reset()
    yield stream
    stream.reset()


def _step(model, x, dy):
    x = x.detach().clone().requires_grad_(True)
    y = model(x)
    y.backward(dy)
    torch.cuda.synchronize()
    return y.detach(), x.grad


def _inputs(device, m=192, seed=5):
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(m, HIDDEN, generator=g, device=device).half()
    dy = (torch.randn(m, HIDDEN, generator=g, device=device) * 0.1).half()
    return x, dy


@pytest.mark.parametrize("slots", [1, 2, 3])
def test_streamed_equals_resident(cuda, streaming, slots):
    print(f"stream slots={slots}", flush=True)
    resident, streamed = Toy(4, 0, cuda), Toy(4, 0, cuda)
    x, dy = _inputs(cuda)
    want_y, want_g = _step(resident, x, dy)
    assert streaming.setup(streamed, slots=slots)
    w = streamed.model.layers[2].down_proj.weight
    assert w.data.stride()[0] == 0 and w._mindx_host.is_pinned()
    s = streaming.streamer()
    for _ in range(2):  # the second step starts with the last layers resident
        got_y, got_g = _step(streamed, x, dy)
        assert torch.equal(got_y, want_y) and torch.equal(got_g, want_g)
    if slots == 1:  # step 1: forward copies all 4 layers, backward the 3 below the last;
        # step 2 starts with layer 0 resident
        assert s.loads == 4 + 3 + 3 + 3, s.loads
    assert s.loads >= 4


def _lora_toy(cuda, seed):
    from mindxsoup_amd.linear4bit import LoraLinear4bit

    toy = Toy(3, seed, cuda)
    torch.manual_seed(seed)
    for layer in toy.model.layers:
        for name in ("q_proj", "gate_proj", "down_proj"):
            lora = LoraLinear4bit(getattr(layer, name), r=16, lora_alpha=32, lora_dropout=0.05)
            torch.nn.init.normal_(lora.lora_B["default"].weight, std=0.05)
            setattr(layer, name, lora)
    return toy.train()


def test_fused_lora_streamed_equals_resident(cuda, streaming):
    """peft-layout LoRA over offloaded bases keeps the fused kernels (NF4LoraStreamFunction):
    output, input gradient and the LoRA gradients equal the resident model's bit for bit."""
    from mindxsoup_amd import linear4bit

    resident, streamed = _lora_toy(cuda, 9), _lora_toy(cuda, 9)
    assert streaming.setup(streamed, slots=2)
    x, dy = _inputs(cuda, m=256)
    calls = []
    original = linear4bit.NF4LoraStreamFunction.apply

    def spy(*args):
        calls.append(1)
        return original(*args)

    linear4bit.NF4LoraStreamFunction.apply = spy
    try:
        for model in (resident, streamed):
            torch.manual_seed(21)  # the same dropout masks for both
            model.y, model.g = _step(model, x, dy)
    finally:
        linear4bit.NF4LoraStreamFunction.apply = original
    assert len(calls) == 9  # three LoRA projections in each of three layers, all fused
    assert torch.equal(streamed.y, resident.y) and torch.equal(streamed.g, resident.g)
    for (name, pr), (_, ps) in zip(resident.named_parameters(), streamed.named_parameters()):
        if pr.requires_grad:
            assert torch.equal(pr.grad, ps.grad), name


def test_prefetch_copies_ahead(cuda, streaming):
    streamed = Toy(4, 1, cuda)
    assert streaming.setup(streamed, slots=3, prefetch=2, hints=False)
    s = streaming.streamer()
    s.layer_begins(0, forward=True)
    assert set(s.table.slot_of) == {0, 1, 2} and s.loads == 3
    s.layer_begins(3, forward=False)  # backward order: 3, then 2 and 1 ahead
    assert set(s.table.slot_of) == {3, 2, 1}
    s.layer_begins(7, forward=True)  # outside the model: ignored
    x, dy = _inputs(cuda)
    _step(streamed, x, dy)  # demand copies without hints
    torch.cuda.synchronize()


def test_layer_unpack_equals_dequant_then_matmul(cuda, streaming, monkeypatch):
    from mindxsoup_amd import linear4bit

    resident, streamed = Toy(3, 2, cuda), Toy(3, 2, cuda)
    x, dy = _inputs(cuda, m=130)
    monkeypatch.setattr(linear4bit, "FUSED_GEMM", False)
    want_y, want_g = _step(resident, x, dy)
    assert streaming.setup(streamed, slots=2, layer_unpack=True)
    s = streaming.streamer()
    assert s.layer_tables is not None
    got_y, got_g = _step(streamed, x, dy)
    assert s.unpacked is not None
    assert torch.equal(got_y, want_y) and torch.equal(got_g, want_g)


def test_offloaded_without_streamer(cuda, streaming):
    from mindxsoup_amd.linear4bit import Linear4bit

    g = torch.Generator(device=cuda).manual_seed(3)
    w = (torch.randn(HIDDEN * 2, HIDDEN, generator=g, device=cuda) * 0.05).half()
    a, b = Linear4bit.from_weight(w), Linear4bit.from_weight(w)
    streaming.offload(b.weight)
    x, _ = _inputs(cuda, m=70)
    with torch.no_grad():
        assert torch.equal(b(x), a(x))
        assert torch.equal(b(x.float()), a(x.float()))  # the compute-dtype round trip


def test_reset_removes_hints(cuda, streaming):
    first, second = Toy(2, 6, cuda), Toy(3, 6, cuda)
    assert streaming.setup(first, slots=1)
    streaming.reset()
    assert all(not layer._forward_pre_hooks for layer in first.model.layers)
    assert streaming.setup(second, slots=1)
    x, dy = _inputs(cuda, m=64)
    _step(first, x, dy)  # one-off copies; no hint reaches the second model's streamer
    assert streaming.streamer().loads == 0


def test_reset_between_forward_and_backward(cuda, streaming):
    """A streamer retired by reset() after a forward gets no hints from that forward's backward
    (the input-gradient hooks check which streamer is current); the backward still runs on
    one-off copies and gives the resident gradients."""
    resident, streamed = Toy(3, 8, cuda), Toy(3, 8, cuda)
    x, dy = _inputs(cuda, m=64)
    _, want_g = _step(resident, x, dy)
    assert streaming.setup(streamed, slots=2)
    old = streaming.streamer()
    xg = x.detach().clone().requires_grad_(True)
    y = streamed(xg)
    loads = old.loads
    streaming.reset()
    y.backward(dy)
    torch.cuda.synchronize()
    assert old.loads == loads
    assert torch.equal(xg.grad, want_g)


def test_setup_declines(cuda, streaming, monkeypatch):
    toy = Toy(2, 4, cuda)
    monkeypatch.setattr(streaming, "enabled", False)
    assert not streaming.setup(toy)
    monkeypatch.setattr(streaming, "enabled", True)
    assert not streaming.setup(torch.nn.Linear(4, 4))  # no decoder layers
    assert not streaming.active()


def test_loader_offload_and_stream_qwen2(cuda, streaming):
    transformers = pytest.importorskip("transformers")
    from mindxsoup_amd.loader import replace_with_nf4

    cfg = transformers.Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                                   num_hidden_layers=3, num_attention_heads=4,
                                   num_key_value_heads=2, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    models = []
    for offload in (False, True):
        torch.manual_seed(0)
        m = transformers.Qwen2ForCausalLM(cfg).half().cuda().eval()
        replace_with_nf4(m, lora_targets=("q_proj", "v_proj"), offload=offload)
        models.append(m)
    resident, streamed = models
    k = streamed.model.layers[1].self_attn.k_proj.weight
    assert k.data.stride()[0] == 0 and not k._mindx_host.is_pinned()
    assert streaming.setup(streamed, slots=2)
    assert k._mindx_host.is_pinned()
    ids = torch.randint(0, 512, (2, 33), device=cuda)
    with torch.no_grad():
        want = resident(input_ids=ids).logits
        got = streamed(input_ids=ids).logits
    # both LoRA paths are fused (the streamed one on the slot's bytes)
    assert bool((got == want).all())
    # a checkpoint of the streamed model holds the weights, not the device placeholders
    sd_r, sd_s = resident.state_dict(), streamed.state_dict()
    assert sd_r.keys() == sd_s.keys()
    for key, v in sd_r.items():
        assert torch.equal(v.cpu(), sd_s[key].cpu()), key
    fresh = transformers.Qwen2ForCausalLM(cfg).half().cuda().eval()
    replace_with_nf4(fresh, lora_targets=("q_proj", "v_proj"))
    fresh.load_state_dict(sd_s, strict=True)
    with torch.no_grad():
        assert torch.equal(fresh(input_ids=ids).logits, want)
