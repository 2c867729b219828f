"""torch.ops.mxs_nf4: the compiled operator library (csrc/torch_ops.cpp, libmxs_nf4_torch.so).

The library registers the NF4 + LoRA projection's host side in C++ over the same C ABI the
ctypes binding (_lib.py) reaches: checks, allocation from torch's caching allocator, the launch
sequence on the current HIP stream, and autograd nodes whose backward runs in C++.  A projection
is one Python call forward and none backward, where the Python autograd Functions of
linear4bit make four or five ctypes calls per direction.  The ops give the same bits as those
Functions (same kernels, same order).

The device ops have Meta kernels, so fake-tensor tracing sees their shapes.  Nothing here falls
back: a missing library raises MxsLibraryError naming the build command.
"""

import os

import torch

from . import _lib

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmxs_nf4_torch.so")

OPS = ("dequant", "linear_fwd", "linear_bwd_dx", "lora_fwd", "lora_bwd", "lora_fwd_group",
       "lora_bwd_group", "linear", "lora_linear", "lora_siblings")

# set by apply() from FEATURES["torch_ops"]; False: the Python Functions.  Off when MXS_NF4_LIB
# names another build of the C-ABI library: this library links the package's own copy by file
# name, so its ops would run that copy instead of the named one.
ENABLED = not os.environ.get("MXS_NF4_LIB")

_ops = None


def load():
    """torch.ops.mxs_nf4 with the library loaded (once)."""
    global _ops
    if _ops is None:
        if os.environ.get("MXS_NF4_LIB"):
            raise _lib.MxsLibraryError(
                "MXS_NF4_LIB is set: the operator library links the package's own "
                "libmxs_nf4.so, not the named build; use the Python Functions "
                "(FEATURES['torch_ops'] = False) for A/B runs of another build")
        if not os.path.exists(PATH):
            raise _lib.MxsLibraryError(
                f"{PATH} is not built: run `python -m mindxsoup_amd.build` (hipcc, gfx950)")
        _lib.lib()  # the C-ABI library it links, loaded from the same file
        torch.ops.load_library(PATH)
        _ops = torch.ops.mxs_nf4
    return _ops


def nf4(packed, state):
    """The five NF4 operand tensors the ops take after the input: packed bytes, absmax (u8),
    the second-level code book, the second-level absmax and the offset."""
    return packed, state.absmax, state.state2.code, state.state2.absmax, state.offset


def linear(x, packed, state, bias=None):
    """Y = x W^T (+ bias), fp16 [..., N]; autograd: grad_x = grad W (NF4LinearFunction)."""
    return load().linear(x, *nf4(packed, state), int(state.shape[0]), bias)


def lora_linear(x, lora_a, lora_b, packed, state, bias, keep, mask_scale, s):
    """base(x) + s * B(A(drop(x))), fp16 [..., N] (NF4LoraFunction); keep: u8 [rows, K] or
    None; gradients for x, lora_a and lora_b (in their dtypes)."""
    return load().lora_linear(x, lora_a, lora_b, *nf4(packed, state), bias, keep,
                              float(mask_scale), float(s))


def lora_siblings(x2d, projs, lora_as, lora_bs, one_gemm=True, rope=None):
    """The projections `projs` (linear4bit.Proj, one scaling and dropout rate) over one input
    x2d fp16 [M, K], their launches shared (NF4LoraSiblingsFunction): a list of fp16 [M, N_i].
    one_gemm: the forward GEMMs in one grouped launch (128x128 tiles) rather than each on its
    own plan.  rope = (n_rope, cos, sin): the first n_rope outputs come rotated, their
    backward still that of the unrotated outputs (linear4bit.siblings_project)."""
    p0 = projs[0]
    n_rope, cos, sin = rope if rope is not None else (0, None, None)
    return load().lora_siblings(
        x2d, list(lora_as), list(lora_bs), [p.packed for p in projs],
        [p.state.absmax for p in projs], [p.state.state2.code for p in projs],
        [p.state.state2.absmax for p in projs], [p.state.offset for p in projs],
        [p.bias for p in projs], [p.keep for p in projs], float(p0.mask_scale), float(p0.s),
        bool(one_gemm), cos, sin, int(n_rope))


def dequant(packed, shape, dtype, absmax_8bit=None, code=None, absmax2=None, offset=None,
            absmax=None):
    """The dense `shape` matrix of packed NF4 (unpack_nf4): nested scales (absmax_8bit, code,
    absmax2, offset) or fp32 absmax."""
    return load().dequant(packed, absmax_8bit, code, absmax2, offset, absmax, list(shape),
                          dtype)
