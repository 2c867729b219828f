"""The kernels' dropout, bit for bit against the oracle's restatement of the reference
(solution/dropout.py:33-35: keep ? fp16(fp32(x) * fp32(1/(1-p))) : 0), over every finite fp16
input.  One-hot LoRA weights make each output a single dropped input: the row product
mxs_lora_h gives H = drop(x) A^T with A = [I 0] (s = 1), and mxs_lora_grads gives dA =
dHs^T drop(x) with dHs^T = [I 0].  The rates include ones where rounding the exact product once
to fp16 (a mixed-precision FMA) differs from the reference's two roundings for hundreds of
inputs (p = 0.04 and 0.4; none at p = 0.05: tests/test_oracle.py counts them)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _bits(a):
    """Bit patterns, with -0 as +0: a product's sum of signed zeros is +0 whatever the input's
    sign, so the one-hot outputs cannot show it."""
    b = a.view(np.uint16 if a.dtype == np.float16 else np.uint32).copy()
    b[a == 0] = 0
    return b


def _inputs(p, rows):
    """Every finite fp16 value whose dropped value is finite too (an infinite one would turn the
    one-hot products' zero terms into NaN), padded with zeros to whole rows of `rows`:
    [n / rows, rows]."""
    v = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    v = v[np.isfinite(v)]
    with np.errstate(over="ignore"):
        v = v[np.isfinite(O.dropout_fp16(v, np.ones(v.size, np.uint8), p))]
    pad = (-v.size) % rows
    return np.concatenate([v, np.zeros(pad, np.float16)]).reshape(-1, rows)


@pytest.mark.parametrize("p", [0.05, 0.04, 0.4])
def test_row_product_dropout_bits(cuda, p):
    from mindxsoup_amd import kernels

    print(f"case dropout rows p={p}", flush=True)
    vals = _inputs(p, 16)  # [~3900, 16]
    M = vals.shape[0]
    x = np.zeros((M, 32), np.float16)
    x[:, :16] = vals
    rng = np.random.default_rng(int(p * 1000))
    keep = (rng.random((M, 32)) < 0.75).astype(np.uint8)
    a = np.zeros((16, 32), np.float16)
    a[np.arange(16), np.arange(16)] = 1
    h, _ = kernels.lora_h(torch.from_numpy(x).to(cuda), torch.from_numpy(a).to(cuda), 1.0,
                          torch.from_numpy(keep).to(cuda), 1.0 / (1.0 - p))
    want = O.dropout_fp16(x, keep, p)[:, :16]
    got = h.cpu().numpy()
    bad = np.sum(_bits(got) != _bits(want))
    assert bad == 0, f"{bad} of {want.size} dropped values differ from the reference's rounding"


@pytest.mark.parametrize("p", [0.05, 0.04, 0.4])
def test_weight_gradient_dropout_bits(cuda, p):
    from mindxsoup_amd import kernels

    print(f"case dropout cols p={p}", flush=True)
    vals = np.ascontiguousarray(_inputs(p, 16).T)  # [16, ~3900]
    vals = np.concatenate([vals, np.zeros((16, (-vals.shape[1]) % 8), np.float16)], axis=1)
    M, K = vals.shape
    rng = np.random.default_rng(int(p * 1000) + 1)
    keep = (rng.random((M, K)) < 0.75).astype(np.uint8)
    ldt = 16
    dht = np.zeros((16, ldt), np.float16)
    dht[np.arange(16), np.arange(16)] = 1
    ht = np.zeros((16, ldt), np.float16)
    dy = np.zeros((M, 8), np.float16)
    da, _ = kernels.lora_grads(torch.from_numpy(dht).to(cuda), torch.from_numpy(ht).to(cuda),
                               torch.from_numpy(vals).to(cuda), torch.from_numpy(dy).to(cuda),
                               torch.from_numpy(keep).to(cuda), 1.0 / (1.0 - p))
    want = O.dropout_fp16(vals, keep, p).astype(np.float32)
    got = da.cpu().numpy()
    bad = np.sum(_bits(got) != _bits(want))
    assert bad == 0, f"{bad} of {want.size} dropped values differ from the reference's rounding"
