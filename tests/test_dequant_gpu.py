"""NF4 dequant on the GPU against the CPU oracle, bit for bit (the reference's own tests:
solution/test_nf4.py:23-42 and :85-103, with bitsandbytes replaced by the oracle)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

QWEN_SHAPES = [(1536, 1536), (8960, 1536), (256, 1536), (1536, 8960)]


def _to_gpu(q, dev):
    return dict(packed=torch.from_numpy(q.packed).to(dev),
                absmax8=torch.from_numpy(q.absmax8).to(dev),
                code=torch.from_numpy(q.code).to(dev),
                absmax2=torch.from_numpy(q.absmax2).to(dev),
                offset=torch.tensor(q.offset, dtype=torch.float32, device=dev),
                absmax_f32=torch.from_numpy(q.absmax_f32).to(dev))


def _bits(t):
    return t.cpu().contiguous().view(torch.int16).numpy()


def _weights(shape, seed, std=0.02):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * std).astype(np.float16)


@pytest.mark.parametrize("shape", QWEN_SHAPES + [(100, 64)])
@pytest.mark.parametrize("nested", [True, False])
def test_unpack_matches_oracle(cuda, shape, nested):
    from mindxsoup_amd.nf4 import unpack_nf4

    print(f"case dequant shape={shape} nested={nested}", flush=True)
    q = O.quantize(_weights(shape, 0))
    g = _to_gpu(q, cuda)
    if nested:
        got = unpack_nf4(g["packed"], shape, g["absmax2"], 64, torch.float16,
                         absmax_8bit=g["absmax8"], code=g["code"], offset=g["offset"])
        want = O.dequant(q)
    else:
        got = unpack_nf4(g["packed"], shape, g["absmax_f32"], 64, torch.float16)
        want = O.dequant(packed=q.packed, absmax_f32=q.absmax_f32, shape=shape)
    torch.cuda.synchronize()
    assert got.shape == shape and got.dtype == torch.float16
    assert np.array_equal(_bits(got), want.view(np.int16))


@pytest.mark.parametrize("shape", QWEN_SHAPES + [(100, 64)])
@pytest.mark.parametrize("nested", [True, False])
def test_wide_kernel_is_bit_identical_to_the_one_byte_kernel(cuda, shape, nested):
    from mindxsoup_amd.nf4 import unpack_nf4, unpack_nf4_bytewise

    print(f"case wide-vs-bytes shape={shape} nested={nested}", flush=True)
    q = O.quantize(_weights(shape, 1, 0.05))
    g = _to_gpu(q, cuda)
    if nested:
        kw = dict(absmax_8bit=g["absmax8"], code=g["code"], offset=g["offset"])
        a = unpack_nf4(g["packed"], shape, g["absmax2"], 64, torch.float16, **kw)
        b = unpack_nf4_bytewise(g["packed"], shape, g["absmax2"], 64, torch.float16, **kw)
    else:
        a = unpack_nf4(g["packed"], shape, g["absmax_f32"], 64, torch.float16)
        b = unpack_nf4_bytewise(g["packed"], shape, g["absmax_f32"], 64, torch.float16)
    assert np.array_equal(_bits(a), _bits(b))


def test_fp32_output_matches_oracle(cuda):
    from mindxsoup_amd.nf4 import unpack_nf4

    shape = (256, 1536)
    q = O.quantize(_weights(shape, 2))
    g = _to_gpu(q, cuda)
    got = unpack_nf4(g["packed"], shape, g["absmax2"], 64, torch.float32,
                     absmax_8bit=g["absmax8"], code=g["code"], offset=g["offset"])
    want = O.dequant(q, out_dtype=np.float32)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_unaligned_and_odd_sizes_take_the_byte_kernel(cuda):
    """Packed bytes at an odd address and a size that is not whole 32-byte blocks."""
    from mindxsoup_amd.nf4 import unpack_nf4

    q = O.quantize(_weights((64, 128), 3))
    g = _to_gpu(q, cuda)
    buf = torch.empty(q.packed.size + 1, dtype=torch.uint8, device=cuda)
    buf[1:] = g["packed"]
    shifted = buf[1:]
    got = unpack_nf4(shifted, (64, 128), g["absmax2"], 64, torch.float16,
                     absmax_8bit=g["absmax8"], code=g["code"], offset=g["offset"])
    assert np.array_equal(_bits(got), O.dequant(q).view(np.int16))
    part = g["packed"][:1000]  # 31.25 blocks
    got = unpack_nf4(part, (2000,), g["absmax2"], 64, torch.float16,
                     absmax_8bit=g["absmax8"], code=g["code"], offset=g["offset"])
    want = O.dequant(packed=q.packed[:1000], absmax8=q.absmax8, code=q.code, absmax2=q.absmax2,
                     offset=q.offset)
    assert np.array_equal(_bits(got), want.view(np.int16))


def test_empty_input(cuda):
    from mindxsoup_amd.nf4 import unpack_nf4

    q = O.quantize(_weights((1, 64), 4))
    g = _to_gpu(q, cuda)
    got = unpack_nf4(g["packed"][:0], (0, 1536), g["absmax2"], 64, torch.float16,
                     absmax_8bit=g["absmax8"], code=g["code"], offset=g["offset"])
    assert got.shape == (0, 1536)


def test_golden_fixtures(cuda):
    from mindxsoup_amd.nf4 import unpack_nf4
    from tests.golden import load_dequant_fixtures

    for name, f in load_dequant_fixtures():
        print(f"case golden {name}", flush=True)
        dev = cuda
        got = unpack_nf4(torch.from_numpy(f["packed"]).to(dev), tuple(f["shape"]),
                         torch.from_numpy(f["absmax2"]).to(dev), 64, torch.float16,
                         absmax_8bit=torch.from_numpy(f["absmax8"]).to(dev),
                         code=torch.from_numpy(f["code"]).to(dev),
                         offset=torch.tensor(float(f["offset"]), dtype=torch.float32,
                                             device=dev))
        assert np.array_equal(_bits(got).reshape(-1), f["out_bits"].view(np.int16))


def _layer(dev, shapes, seed):
    """Weights quantized on the GPU and laid back to back, as the layer launch wants them."""
    from mindxsoup_amd.quant import quantize_4bit

    torch.manual_seed(seed)
    parts = []
    for shape in shapes:
        w = (torch.randn(shape, device=dev) * 0.02).half()
        parts.append(quantize_4bit(w))
    packed = torch.cat([p.view(-1) for p, _ in parts])
    absmax8 = torch.cat([s.absmax for _, s in parts])
    code = torch.cat([s.state2.code for _, s in parts])
    absmax2 = torch.cat([s.state2.absmax for _, s in parts])
    offset = torch.stack([s.offset for _, s in parts])
    nb = [s.absmax.numel() for _, s in parts]
    block0 = torch.tensor(np.concatenate([[0], np.cumsum(nb)]), dtype=torch.int64, device=dev)
    ng = [s.state2.absmax.numel() for _, s in parts]
    scale0 = torch.tensor(np.concatenate([[0], np.cumsum(ng)[:-1]]), dtype=torch.int64,
                          device=dev)
    return parts, packed, absmax8, code, absmax2, offset, block0, scale0


def test_layer_launch_equals_per_weight_unpack(cuda):
    """nf4_layer_kernel semantics (solution/nf4.py:89-110): one launch over a layer's 7 weights
    stored back to back gives each weight's own unpack, bit for bit."""
    from mindxsoup_amd.nf4 import launch_layer, unpack_state

    shapes = [(1536, 1536), (256, 1536), (256, 1536), (1536, 1536), (8960, 1536),
              (8960, 1536), (1536, 8960)]
    parts, packed, absmax8, code, absmax2, offset, block0, scale0 = _layer(cuda, shapes, 0)
    out = torch.empty(packed.numel() * 2, dtype=torch.float16, device=cuda)
    launch_layer(packed, out, absmax8, code, absmax2, offset, None, block0, scale0)
    pos = 0
    for (p, s), shape in zip(parts, shapes):
        n = shape[0] * shape[1]
        want = unpack_state(p, s)
        assert torch.equal(out[pos:pos + n].view(torch.int16), want.view(-1).view(torch.int16))
        pos += n


def test_layer_launch_with_weights_that_straddle_workgroups(cuda):
    """Weights whose block counts are not multiples of a workgroup's 128 blocks."""
    from mindxsoup_amd.nf4 import launch_layer, unpack_state

    shapes = [(3, 64), (100, 64), (7, 128), (300, 64), (1, 64)]
    parts, packed, absmax8, code, absmax2, offset, block0, scale0 = _layer(cuda, shapes, 1)
    out = torch.empty(packed.numel() * 2, dtype=torch.float16, device=cuda)
    launch_layer(packed, out, absmax8, code, absmax2, offset, None, block0, scale0)
    want = torch.cat([unpack_state(p, s).view(-1) for p, s in parts])
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


def test_layer_launch_layouts_of_equal_length(cuda):
    """Two layouts whose block0 tensors have the same length, built fresh for each call (the
    allocator may hand the second the first one's address): each launch decodes with its own
    layout's plan; a plan of another length is refused before launching."""
    from mindxsoup_amd.nf4 import launch_layer, layer_plan, unpack_state

    for shapes, seed in (([(512, 64), (100, 64), (300, 128)], 3),
                         ([(100, 64), (300, 128), (512, 64)], 4)):
        parts, packed, absmax8, code, absmax2, offset, block0, scale0 = _layer(cuda, shapes, seed)
        out = torch.empty(packed.numel() * 2, dtype=torch.float16, device=cuda)
        launch_layer(packed, out, absmax8, code, absmax2, offset, None, block0, scale0)
        want = torch.cat([unpack_state(p, s).view(-1) for p, s in parts])
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), shapes
        del block0
    wrong = layer_plan([0, 128], cuda)  # one workgroup; this layout has more
    with pytest.raises(RuntimeError, match="shape outside"):
        launch_layer(packed, out, absmax8, code, absmax2, offset, None,
                     torch.tensor([0, 512, 612, 1212], dtype=torch.int64, device=cuda), scale0,
                     wrong)


@pytest.mark.parametrize("shape", [(8960, 1536), (100, 64), (256, 1536)])
def test_gpu_quantizer_matches_oracle(cuda, shape):
    from mindxsoup_amd.quant import quantize_4bit

    w = _weights(shape, 5)
    packed, st = quantize_4bit(torch.from_numpy(w).to(cuda))
    q = O.quantize(w)
    assert np.array_equal(packed.view(-1).cpu().numpy(), q.packed)
    assert np.array_equal(st.absmax_f32.cpu().numpy().view(np.uint32), q.absmax_f32.view(np.uint32))
    assert np.float32(st.offset.item()) == np.float32(q.offset)
    assert np.array_equal(st.absmax.cpu().numpy(), q.absmax8)
    assert np.array_equal(st.state2.absmax.cpu().numpy().view(np.uint32), q.absmax2.view(np.uint32))
    assert np.array_equal(st.state2.code.cpu().numpy().view(np.uint32), q.code.view(np.uint32))


def test_full_model_grouped_dequant_properties(cuda):
    """BASELINE config 2 at full size (28 layers x 7 weights in one launch): every weight's
    slice of the output equal to its own unpack bit for bit (compared on the device) and, for
    one weight per layer kind, to the oracle."""
    from mindxsoup_amd.nf4 import launch_layer, unpack_state

    shapes = [(1536, 1536), (256, 1536), (256, 1536), (1536, 1536), (8960, 1536),
              (8960, 1536), (1536, 8960)]
    parts, packed, absmax8, code, absmax2, offset, block0, scale0 = _layer(cuda, shapes * 28, 2)
    out = torch.empty(packed.numel() * 2, dtype=torch.float16, device=cuda)
    launch_layer(packed, out, absmax8, code, absmax2, offset, None, block0, scale0)
    pos = 0
    for i, (p, s) in enumerate(parts):
        n = s.shape[0] * s.shape[1]
        assert torch.equal(out[pos:pos + n].view(torch.int16),
                           unpack_state(p, s).view(-1).view(torch.int16)), f"weight {i}"
        pos += n
    assert pos == out.numel()
    for i in (0, 1, 4, 6):
        p, s = parts[i]
        q = O.NF4Weight(s.shape, p.view(-1).cpu().numpy(), s.absmax.cpu().numpy(),
                        s.state2.code.cpu().numpy(), s.state2.absmax.cpu().numpy(),
                        float(s.offset.item()))
        n0 = int(block0[i].item()) * 64
        got = out[n0:n0 + s.shape[0] * s.shape[1]].cpu().view(torch.int16).numpy()
        assert np.array_equal(got, O.dequant(q).view(np.int16).reshape(-1))


def test_hbm_probe_streams_what_it_reports(cuda):
    """mxs_hbm_probe (bench.py's hbm_ceiling) moves the bytes it is timed on: the dequant's
    pattern writes each loaded dword four times at its chunk, the store stream writes every
    chunk, and the load stream reads every chunk (its per-wave XOR matches the host's), on a
    chunk count that leaves a partial workgroup."""
    from mindxsoup_amd import _lib

    n = 5000
    stream = _lib.stream_of(cuda)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, 4), dtype=torch.int32, device=cuda)
    dst = torch.zeros((n, 4), dtype=torch.int32, device=cuda)
    _lib.hbm_probe(0, _lib.ptr(src), _lib.ptr(dst), n, stream)
    torch.cuda.synchronize()
    words = src.view(-1)[:n]
    assert torch.equal(dst, words[:, None].expand(n, 4))
    _lib.hbm_probe(2, None, _lib.ptr(dst), n, stream)
    torch.cuda.synchronize()
    idx = torch.arange(n, dtype=torch.int32, device=cuda)
    assert torch.equal(dst, torch.stack([idx, idx ^ 1, idx ^ 2, idx ^ 3], 1))
    blocks = (n + 1023) // 1024
    sink = torch.zeros(blocks * 4, dtype=torch.int32, device=cuda)
    _lib.hbm_probe(1, _lib.ptr(src), _lib.ptr(sink), n, stream)
    torch.cuda.synchronize()
    x = src.cpu().numpy().view(np.uint32)
    want = np.zeros(blocks * 4, dtype=np.uint32)
    for b in range(blocks):
        for t in range(256):
            for u in range(4):
                c = b * 1024 + u * 256 + t
                if c < n:
                    want[b * 4 + t // 64] ^= np.bitwise_xor.reduce(x[c])
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), want)
