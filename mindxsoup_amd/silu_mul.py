"""silu(gate) * up for the fp16 MLP, with a backward that writes its gradients over gate and up
(the interface of solution/silu_mul.py, on the HIP kernels of csrc/swiglu.hip).

gate and up are read only by this backward and are dead right after it, so the backward stores
d(gate) into gate's memory and d(up) into up's (solution/silu_mul.py:1-13): no [N, 8960]
gradient buffers are allocated.  Values are computed in fp32 from the fp16 inputs and rounded to
fp16 once.
"""

import torch

from . import direct, kernels


class SiluMulInPlace(torch.autograd.Function):
    """silu(gate) * up in fp16; backward returns gate's and up's own memory holding their
    gradients (solution/silu_mul.py:52-71).  Only for gate/up that nothing else reads after this
    backward (the MLP's projections, whose 4-bit weights are frozen and keep no input)."""

    @staticmethod
    def forward(ctx, gate, up):
        gate = gate.contiguous()
        up = up.to(gate.dtype).contiguous()
        out = kernels.silu_mul(gate, up)
        ctx.save_for_backward(gate, up)
        return out

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        kernels.silu_mul_bwd_(grad.to(gate.dtype), gate, up)
        return gate, up


def silu_mul(gate, up):
    """The reference's guard (solution/silu_mul.py:74-78): fp16 CUDA tensors of one shape take
    the kernel; anything else is the plain expression, as in the reference."""
    if gate.dtype != torch.float16 or not gate.is_cuda or gate.shape != up.shape \
            or gate.numel() == 0:
        return torch.nn.functional.silu(gate) * up
    return direct.run(SiluMulInPlace, gate, up)
