"""The grouped LoRA row products (mxs_lora_h_partials_group, mxs_lora_dh_partials_group): several
projections over the same tokens in one launch give the bits of one launch each.  Groups mix
reduction lengths (1536 and 8960), so their problems run with different slice and wave counts
inside one launch."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, M, K, N, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn((M, K), device=dev, generator=g).half()
    a = ((torch.rand((16, K), device=dev, generator=g) * 2 - 1) / np.sqrt(K)).half()
    b = (torch.randn((N, 16), device=dev, generator=g) * 0.01).half()
    dy = torch.randn((M, N), device=dev, generator=g).half()
    keep = (torch.rand((M, K), device=dev, generator=g) >= 0.05).to(torch.uint8)
    return x, a, b, dy, keep


# (K, N) per projection: q/k/v of a layer, gate/up, and a mixed group with down's 8960
GROUPS = {
    "qkv": [(1536, 1536), (1536, 256), (1536, 256)],
    "gate_up": [(1536, 8960), (1536, 8960)],
    "mixed": [(8960, 1536), (1536, 256), (1536, 8960), (256, 1536)],
}


@pytest.mark.parametrize("group", sorted(GROUPS))
@pytest.mark.parametrize("M", [1024, 300, 37])
def test_grouped_rows_equal_separate_launches(cuda, group, M):
    from mindxsoup_amd import kernels

    print(f"case lora group {group} M={M}", flush=True)
    shapes = GROUPS[group]
    probs = [_inputs(cuda, M, K, N, 100 + i) for i, (K, N) in enumerate(shapes)]
    if group != "mixed":  # projections of one group share their input, as in the model
        probs = [(probs[0][0],) + p[1:] for p in probs]
    s, ms = 2.0, 1 / 0.95
    sep = [kernels.lora_h_partials(x, a, s, keep, ms, lora_b=b) for x, a, b, _, keep in probs]
    grp = kernels.lora_h_partials_group([p[0] for p in probs], [p[1] for p in probs], s,
                                        [p[4] for p in probs], ms, [p[2] for p in probs])
    bts = [o[2] for o in sep]
    dsep = [kernels.lora_dh_partials(p[3], bt, s) for p, bt in zip(probs, bts)]
    dgrp = kernels.lora_dh_partials_group([p[3] for p in probs], bts, s)
    torch.cuda.synchronize()
    for (hp1, at1, bt1), (hp2, at2, bt2) in zip(sep, grp):
        assert torch.equal(hp1, hp2) and torch.equal(at1, at2) and torch.equal(bt1, bt2)
    for d1, d2 in zip(dsep, dgrp):
        assert torch.equal(d1, d2)


def test_grouped_rows_without_masks_or_side_outputs(cuda):
    from mindxsoup_amd import kernels

    M = 256
    probs = [_inputs(cuda, M, K, 256, 7 + K) for K in (1536, 512)]
    s = 0.5
    sep = [kernels.lora_h_partials(x, a, s) for x, a, _, _, _ in probs]
    grp = kernels.lora_h_partials_group([p[0] for p in probs], [p[1] for p in probs], s)
    torch.cuda.synchronize()
    for (hp1, at1, _), (hp2, at2, bt2) in zip(sep, grp):
        assert torch.equal(hp1, hp2) and torch.equal(at1, at2) and bt2 is None


@pytest.mark.parametrize("M", [1024, 300])
def test_grouped_finished_dh_equals_one_launch_dh(cuda, M):
    """mxs_lora_dh_group against lora_dh(..., one_launch=True) per projection (the backward of
    the projections whose dX GEMM carries the weight gradients): dh and dht bit for bit."""
    from mindxsoup_amd import kernels

    probs = [_inputs(cuda, M, K, N, 40 + i) for i, (K, N) in enumerate(GROUPS["qkv"]
                                                                      + [(8960, 1536)])]
    bts = [b.t().contiguous() for _, _, b, _, _ in probs]
    sep = [kernels.lora_dh(p[3], None, 2.0, lora_bt=bt, one_launch=True)
           for p, bt in zip(probs, bts)]
    grp = kernels.lora_dh_group([p[3] for p in probs], bts, 2.0)
    torch.cuda.synchronize()
    for (d1, t1), (d2, t2) in zip(sep, grp):
        assert torch.equal(d1, d2) and torch.equal(t1, t2)
