"""Keep bits: the dropout keep mask format every kernel takes (include/mxs_nf4.h).  The pack kernel
against numpy's little-endian bit packing of the reference's int8 `keep` (solution/dropout.py:64),
and the LoRA kernels fed byte masks and pre-packed bits giving the same bits."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _np_bits(keep):
    """Reference packing: row m -> ceil(K/32) little-endian u32 words, bit k%32 of word k//32."""
    M, K = keep.shape
    kw = (K + 31) // 32
    pad = np.zeros((M, 32 * kw), dtype=np.uint8)
    pad[:, :K] = keep != 0
    return np.packbits(pad, axis=1, bitorder="little").view("<u4").reshape(M, kw)


@pytest.mark.parametrize("M,K", [(1, 1), (3, 31), (5, 32), (7, 33), (64, 1536), (37, 8960),
                                 (2, 100)])
def test_pack_matches_numpy(cuda, M, K):
    from mindxsoup_amd import kernels

    rng = np.random.default_rng(M * 1000 + K)
    keep = (rng.random((M, K)) >= 0.3).astype(np.uint8) * rng.integers(1, 256, (M, K)).astype(np.uint8)
    got = kernels.keep_bits(torch.from_numpy(keep).to(cuda), M, K)
    assert got.dtype == torch.int32 and tuple(got.shape) == (M, (K + 31) // 32)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), _np_bits(keep))


def test_pack_takes_bool_int8_and_unaligned_rows(cuda):
    """bool and int8 masks pack like uint8; a row length that breaks the 16-byte fast path (K
    not a multiple of 16) and a view at an odd offset take the byte loop."""
    from mindxsoup_amd import kernels

    rng = np.random.default_rng(3)
    keep = rng.random((9, 200)) >= 0.5
    ref = _np_bits(keep.astype(np.uint8))
    t = torch.from_numpy(keep).to(cuda)
    for m in (t, t.to(torch.int8), t.to(torch.uint8)):
        assert np.array_equal(kernels.keep_bits(m, 9, 200).cpu().numpy().view(np.uint32), ref)
    big = torch.zeros(9 * 200 + 1, dtype=torch.uint8, device=cuda)
    big[1:] = t.to(torch.uint8).flatten()
    view = big[1:].view(9, 200)  # data at an odd address
    assert np.array_equal(kernels.keep_bits(view, 9, 200).cpu().numpy().view(np.uint32), ref)


def test_bits_pass_through_and_kernels_agree(cuda):
    """Pre-packed bits go straight to the kernels; the LoRA row product and the weight gradients
    give the same bits from a byte mask and from its packed form."""
    from mindxsoup_amd import kernels

    g = torch.Generator(device=cuda)
    g.manual_seed(5)
    M, K, N = 300, 1536, 8960
    x = torch.randn((M, K), device=cuda, generator=g).half()
    a = (torch.rand((16, K), device=cuda, generator=g) * 0.05).half()
    dy = torch.randn((M, N), device=cuda, generator=g).half()
    keep = (torch.rand((M, K), device=cuda, generator=g) >= 0.05).to(torch.uint8)
    bits = kernels.keep_bits(keep, M, K)
    assert kernels.keep_bits(bits, M, K).data_ptr() == bits.data_ptr()
    h8, ht8 = kernels.lora_h(x, a, 2.0, keep, 1 / 0.95)
    hb, htb = kernels.lora_h(x, a, 2.0, bits, 1 / 0.95)
    assert torch.equal(h8, hb) and torch.equal(ht8, htb)
    da8, db8 = kernels.lora_grads(ht8, ht8, x, dy, keep, 1 / 0.95)
    dab, dbb = kernels.lora_grads(ht8, ht8, x, dy, bits, 1 / 0.95)
    assert torch.equal(da8, dab) and torch.equal(db8, dbb)


def test_empty_mask(cuda):
    from mindxsoup_amd import kernels

    z = kernels.keep_bits(torch.zeros((0, 64), dtype=torch.uint8, device=cuda), 0, 64)
    assert tuple(z.shape) == (0, 2)
