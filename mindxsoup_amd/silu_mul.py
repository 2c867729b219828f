"""SwiGLU of the fp16 MLP on the HIP kernels of csrc/swiglu.hip: h = silu(gate) * up, whose
backward writes d(gate) and d(up) into gate's and up's own memory.

The MLP's gate and up outputs are read by nothing but this product's backward, so their buffers
can take their gradients (the memory argument of solution/silu_mul.py:1-13): the backward
allocates no [tokens, intermediate] buffers.  Arithmetic is fp32 on the fp16 inputs with one
rounding per output.  The interface (SiluMulInPlace, silu_mul and its guard) is the
reference's, so its callers and tests apply unchanged.
"""

import torch

from . import direct, kernels


def _kernel_takes(gate, up):
    """fp16 GPU tensors of one non-empty shape (solution/silu_mul.py:74-78's guard)."""
    return (isinstance(gate, torch.Tensor) and gate.is_cuda and gate.dtype == torch.float16
            and gate.shape == up.shape and gate.numel() > 0)


class SiluMulInPlace(torch.autograd.Function):
    """silu(gate) * up in fp16.  The saved gate and up are overwritten by the backward with
    d(gate) and d(up) and handed back as the gradients, so nothing else may read them after the
    backward (true of the MLP's projections, which keep no inputs of their own)."""

    @staticmethod
    def forward(ctx, gate, up):
        operands = (gate.contiguous(), up.to(torch.float16).contiguous())
        ctx.save_for_backward(*operands)
        return kernels.silu_mul(*operands)

    @staticmethod
    def backward(ctx, dh):
        gate, up = ctx.saved_tensors
        kernels.silu_mul_bwd_(dh.to(torch.float16), gate, up)  # gate <- d(gate), up <- d(up)
        return gate, up


def silu_mul(gate, up):
    """h = silu(gate) * up: the kernel for fp16 GPU tensors of one shape, else torch's own
    expression."""
    if not _kernel_takes(gate, up):
        return torch.nn.functional.silu(gate) * up
    return direct.run(SiluMulInPlace, gate, up)
