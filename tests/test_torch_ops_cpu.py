"""The compiled operator library (libmxs_nf4_torch.so) on the CPU: it loads, registers every
torch.ops.mxs_nf4 operator with its schema, and its Meta kernels and C++ autograd nodes give the
shapes, dtypes and gradient structure of the projection without a GPU (no kernel runs)."""

import pytest
import torch

from mindxsoup_amd import ops

M, K, N, R = 300, 1536, 256, 16


@pytest.fixture(scope="module")
def mx():
    return ops.load()


def _nf4(n=N, k=K, device="meta"):
    blocks = n * k // 64
    return (torch.empty(n * k // 2, 1, dtype=torch.uint8, device=device),
            torch.empty(blocks, dtype=torch.uint8, device=device),
            torch.empty(256, device=device), torch.empty((blocks + 255) // 256, device=device),
            torch.empty(1, device=device))


def test_every_op_registered_with_schema(mx):
    for name in ops.OPS:
        schema = str(getattr(mx, name).default._schema)
        assert schema.startswith(f"mxs_nf4::{name}("), schema
    assert "float mask_scale, float s" in str(mx.lora_linear.default._schema)
    assert str(mx.lora_bwd.default._schema).endswith("-> (Tensor, Tensor, Tensor)")
    assert "Tensor?[] keep" in str(mx.lora_siblings.default._schema)


def test_lora_linear_meta_shapes_and_grads(mx):
    """N-D input: y [..., N] fp16 from a node named NF4LoraFunction; its C++ backward gives dx in
    x's shape and dtype, dA / dB in the LoRA weights' dtype (fp32 here)."""
    x = torch.empty(2, 150, K, dtype=torch.float16, device="meta", requires_grad=True)
    a = torch.empty(R, K, device="meta", requires_grad=True)
    b = torch.empty(N, R, device="meta", requires_grad=True)
    keep = torch.empty(300, K, dtype=torch.uint8, device="meta")
    y = mx.lora_linear(x, a, b, *_nf4(), None, keep, 1 / 0.95, 2.0)
    assert y.shape == (2, 150, N) and y.dtype == torch.float16
    assert "NF4LoraFunction" in y.grad_fn.name()
    dx, da, db = torch.autograd.grad(y, (x, a, b), torch.empty_like(y))
    assert dx.shape == x.shape and dx.dtype == torch.float16
    assert da.shape == a.shape and da.dtype == torch.float32
    assert db.shape == b.shape and db.dtype == torch.float32


def test_lora_linear_partial_grads(mx):
    """Frozen LoRA weights: only dx; a frozen input: only dA and dB."""
    a = torch.empty(R, K, device="meta", dtype=torch.float16)
    b = torch.empty(N, R, device="meta", dtype=torch.float16)
    x = torch.empty(M, K, dtype=torch.float16, device="meta", requires_grad=True)
    y = mx.lora_linear(x, a, b, *_nf4(), None, None, 1.0, 2.0)
    (dx,) = torch.autograd.grad(y, (x,), torch.empty_like(y))
    assert dx.shape == (M, K)
    x = torch.empty(M, K, dtype=torch.float16, device="meta")
    a.requires_grad_(True)
    b.requires_grad_(True)
    y = mx.lora_linear(x, a, b, *_nf4(), None, None, 1.0, 2.0)
    da, db = torch.autograd.grad(y, (a, b), torch.empty_like(y))
    assert da.dtype == torch.float16 and db.dtype == torch.float16  # the weights' own dtype


def test_siblings_meta(mx):
    """q, k, v over one input: three outputs from one NF4LoraSiblingsFunction node; dx in x's
    shape, each LoRA weight's gradient in its shape."""
    shapes = [(1536, 1536), (256, 1536), (256, 1536)]
    x = torch.empty(M, K, dtype=torch.float16, device="meta", requires_grad=True)
    a_s = [torch.empty(R, k, device="meta", requires_grad=True) for _, k in shapes]
    b_s = [torch.empty(n, R, device="meta", requires_grad=True) for n, _ in shapes]
    ws = [_nf4(n, k) for n, k in shapes]
    ys = mx.lora_siblings(x, a_s, b_s, *[list(t) for t in zip(*ws)], [None] * 3, [None] * 3,
                          1.0, 2.0, True)
    assert [tuple(y.shape) for y in ys] == [(M, n) for n, _ in shapes]
    assert "NF4LoraSiblingsFunction" in ys[0].grad_fn.name()
    grads = torch.autograd.grad(ys, [x, *a_s, *b_s], [torch.empty_like(y) for y in ys])
    assert grads[0].shape == x.shape
    assert [tuple(g.shape) for g in grads[1:4]] == [(R, k) for _, k in shapes]
    assert [tuple(g.shape) for g in grads[4:]] == [(n, R) for n, _ in shapes]


def test_linear_and_dequant_meta(mx):
    x = torch.empty(4, 77, K, dtype=torch.float16, device="meta", requires_grad=True)
    y = mx.linear(x, *_nf4(), N, None)
    assert y.shape == (4, 77, N) and "NF4LinearFunction" in y.grad_fn.name()
    (dx,) = torch.autograd.grad(y, (x,), torch.empty_like(y))
    assert dx.shape == x.shape
    packed, a8, code, a2, off = _nf4()
    w = mx.dequant(packed, a8, code, a2, off, None, [N, K], torch.float16)
    assert w.shape == (N, K) and w.dtype == torch.float16


def test_inference_mode_runs_forward_only(mx):
    """Without autograd keys (inference mode) the autograd ops run their forward alone."""
    with torch.inference_mode():
        x = torch.empty(M, K, dtype=torch.float16, device="meta")
        a = torch.empty(R, K, device="meta")
        b = torch.empty(N, R, device="meta")
        y = mx.lora_linear(x, a, b, *_nf4(), None, None, 1.0, 2.0)
        assert y.shape == (M, N) and y.grad_fn is None
        assert mx.linear(x, *_nf4(), N, None).shape == (M, N)


def test_ops_refuse_another_c_abi_build(monkeypatch):
    """With MXS_NF4_LIB naming another build of libmxs_nf4.so, the operator library (which links
    the package's own copy) refuses to load instead of mixing the two builds."""
    monkeypatch.setenv("MXS_NF4_LIB", "/nonexistent/libmxs_nf4.so")
    monkeypatch.setattr(ops, "_ops", None)
    with pytest.raises(RuntimeError, match="MXS_NF4_LIB"):
        ops.load()
