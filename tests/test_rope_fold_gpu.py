"""RoPE folded into the grouped q/k/v forward GEMM (mxs_nf4_linear_fwd_hp_group_rope).

Bar: bit-exact.  The rotated q / k equal the grouped GEMM's unrotated outputs rotated by the
oracle's restatement of the reference's rotation (oracle_qkv_rope, solution/attention.py:28-82)
and by the rotation launch (mxs_qkv_rope); v and the LoRA side output are unchanged.  Both tile
plans run (128x64 tiles with 4 x 1 consumer waves when all tiles fit the CUs in one round, as at
1024 tokens; 128x128 otherwise), with and without LoRA, with the bias Qwen2's q/k/v carry, cos /
sin shared by the batch or per sequence, and halves of cos that differ (Qwen's are equal, which
would hide a swapped half or a wrong column order inside a head).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

K, HEAD_DIM, Q_HEADS, KV_HEADS = 1536, 128, 12, 2


def _nf4(dev, n, k, seed):
    from mindxsoup_amd.linear4bit import Linear4bit

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).half()
    b = (torch.randn((n,), device=dev, generator=g) * 0.1).half()
    return Linear4bit.from_weight(w, b)


def _cos_sin(dev, batch, n_tokens, seed):
    """Qwen2's rows (freqs = pos * inv_freq, cat(freqs, freqs)) with noise, so that the two
    halves of a row differ."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    inv = 1.0 / (1e6 ** (torch.arange(0, HEAD_DIM, 2, device=dev).float() / HEAD_DIM))
    pos = torch.arange(n_tokens, device=dev).float()[None, :] + \
        3 * torch.arange(batch, device=dev).float()[:, None]
    emb = torch.cat((pos[:, :, None] * inv, pos[:, :, None] * inv), dim=-1)
    cos = emb.cos() + 0.01 * torch.randn(emb.shape, device=dev, generator=g)
    sin = emb.sin() + 0.01 * torch.randn(emb.shape, device=dev, generator=g)
    return cos.contiguous(), sin.contiguous()


def _heads(y, B, T, n):
    return y.view(B, T, n, HEAD_DIM).transpose(1, 2)


@pytest.mark.parametrize("B,T,cos_batch,lora", [
    (1, 1024, 1, 16),    # 256 tiles of 128x64: the stack's shape
    (2, 1024, 2, 16),    # 512 tiles: the 128x128 plan
    (1, 1100, 1, 16),    # 128x128 with a partial row tile
    (3, 100, 1, 16),     # a partial row tile
    (3, 100, 1, 32),     # rank 32: the LoRA operands read from memory, not staged
    (3, 100, 3, 0),
    (1, 37, 1, 16),
])
def test_folded_rope_equals_the_rotation_of_the_projection(cuda, B, T, cos_batch, lora):
    from mindxsoup_amd import kernels

    print(f"case rope fold B={B} T={T} cos_batch={cos_batch} rank={lora}", flush=True)
    M = B * T
    layers = [_nf4(cuda, n, K, 400 + i) for i, n in enumerate((1536, 256, 256))]
    packeds = [L.weight.data.view(-1, 1) for L in layers]
    states = [L.weight.quant_state for L in layers]
    biases = [L.bias for L in layers]
    g = torch.Generator(device=cuda)
    g.manual_seed(17)
    x = torch.randn((M, K), device=cuda, generator=g).half()
    hps = bs = None
    if lora:
        As = [((torch.rand((lora, K), device=cuda, generator=g) * 2 - 1) / np.sqrt(K)).half()
              for _ in layers]
        bs = [(torch.randn((L.out_features, lora), device=cuda, generator=g) * 0.05).half()
              for L in layers]
        outs = kernels.lora_h_partials_group([x] * 3, As, 2.0, None, 1.0, bs)
        hps = [o[0] for o in outs]
    cos, sin = _cos_sin(cuda, cos_batch, T, 5)
    plain = kernels.nf4_linear_fwd_hp_group([x] * 3, packeds, states, hps, bs, biases)
    folded = kernels.nf4_linear_fwd_hp_group([x] * 3, packeds, states, hps, bs, biases,
                                             rope=(2, cos, sin))
    q_o = torch.empty(B, T, Q_HEADS * HEAD_DIM, device=cuda, dtype=torch.float16)
    k_o = torch.empty(B, T, KV_HEADS * HEAD_DIM, device=cuda, dtype=torch.float16)
    kernels.qkv_rope(_heads(plain[0][0], B, T, Q_HEADS), None,
                     _heads(plain[1][0], B, T, KV_HEADS), None, None, cos, sin,
                     _heads(q_o, B, T, Q_HEADS), _heads(k_o, B, T, KV_HEADS), None)
    torch.cuda.synchronize()
    assert torch.equal(folded[2][0], plain[2][0]), "v is not rotated"
    for (_, h1), (_, h2) in zip(plain, folded):
        assert (h1 is None) == (h2 is None) and (h1 is None or torch.equal(h1, h2))
    assert torch.equal(folded[0][0].view(B, T, -1), q_o), "q against the rotation launch"
    assert torch.equal(folded[1][0].view(B, T, -1), k_o), "k against the rotation launch"
    want_q, want_k, _ = O.qkv_rope(plain[0][0].view(B, T, -1).cpu().numpy(), None,
                                   plain[1][0].view(B, T, -1).cpu().numpy(), None, None,
                                   cos.cpu().numpy(), sin.cpu().numpy(), Q_HEADS, KV_HEADS)
    for got, want in ((folded[0][0], want_q), (folded[1][0], want_k)):
        g_ = got.view(B, T, -1).cpu().numpy()
        assert np.array_equal(g_.view(np.uint16), want.view(np.uint16))


def test_folded_rope_refuses_partial_heads(cuda):
    """Rotated outputs must be whole 128-column heads."""
    from mindxsoup_amd import kernels

    layers = [_nf4(cuda, n, 256, 450 + i) for i, n in enumerate((192, 128))]
    x = torch.randn((64, 256), device=cuda).half()
    cos, sin = _cos_sin(cuda, 1, 64, 1)
    with pytest.raises(ValueError, match="128-column heads"):
        kernels.nf4_linear_fwd_hp_group([x] * 2, [L.weight.data.view(-1, 1) for L in layers],
                                        [L.weight.quant_state for L in layers],
                                        rope=(2, cos, sin))
    with pytest.raises(ValueError, match="whole sequences"):
        kernels.nf4_linear_fwd_hp_group([x] * 2, [L.weight.data.view(-1, 1) for L in layers],
                                        [L.weight.quant_state for L in layers],
                                        rope=(1, cos[:, :48].contiguous(), sin[:, :48].contiguous()))


def test_folded_rope_replays_in_a_graph(cuda):
    """The grouped forward with the rotation captured in a HIP graph: every replay (eager work
    and synchronizations between them, new inputs copied in before each) equals the eager
    launch on the same inputs."""
    from mindxsoup_amd import kernels

    B, T = 1, 1024
    layers = [_nf4(cuda, n, K, 470 + i) for i, n in enumerate((1536, 256, 256))]
    packeds = [L.weight.data.view(-1, 1) for L in layers]
    states = [L.weight.quant_state for L in layers]
    biases = [L.bias for L in layers]
    g = torch.Generator(device=cuda)
    g.manual_seed(23)
    x = torch.randn((B * T, K), device=cuda, generator=g).half()
    cos, sin = _cos_sin(cuda, 1, T, 9)

    def run():
        return kernels.nf4_linear_fwd_hp_group([x] * 3, packeds, states, None, None, biases,
                                               rope=(2, cos, sin))

    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    for rep in range(3):
        x.copy_(torch.randn((B * T, K), device=cuda, generator=g).half())
        graph.replay()
        torch.cuda.synchronize()
        got = [y.clone() for y, _ in outs]
        want = [y for y, _ in run()]
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), rep
