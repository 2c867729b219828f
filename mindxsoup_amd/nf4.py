"""NF4 weight unpacking with fused double-dequant of absmax, on gfx950 HIP kernels.

Mirror of the reference's solution/nf4.py: the same host functions and arguments
(`unpack_nf4`, `launch_layer`, `_supported`, `patch_bnb_nf4`), with the Triton kernels replaced
by the C-ABI entry points mxs_nf4_dequant (wide kernel with one-byte fallback),
mxs_nf4_dequant_bytewise and mxs_nf4_dequant_layer.  The math is unchanged: block scale =
fma(code[absmax8], absmax2[blk >> 8], offset) in fp32, value = fp16(NF4[q] * scale), high nibble
first.
"""

import numpy as np
import torch

from . import _lib, ops

# NF4 code values (QLoRA, arXiv 2305.14314, App. E); the kernels hold the same constants.
NF4_VALUES = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)

_NF4_TABLE = {}


def _nf4_table(device):
    """The NF4 table as an fp32 tensor (solution/nf4.py:116-123)."""
    table = _NF4_TABLE.get(device)
    if table is None:
        table = torch.from_numpy(NF4_VALUES.copy()).to(device)
        _NF4_TABLE[device] = table
    return table


def _dtype_code(dtype):
    if dtype == torch.float16:
        return _lib.MXS_DTYPE_F16
    if dtype == torch.float32:
        return _lib.MXS_DTYPE_F32
    raise ValueError(f"unpack_nf4 writes fp16 or fp32, not {dtype}")


def _check_device(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("NF4 tensors must be on the GPU")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("NF4 tensors must be on one device")
    return dev


def unpack_nf4(packed, shape, absmax, blocksize, dtype, absmax_8bit=None, code=None,
               offset=None, out=None):
    """Dense `shape` matrix of `dtype` from packed NF4 bytes (solution/nf4.py:138-155).  With
    `absmax_8bit` the block scales are double-quantized: `absmax` is then the second-level scale
    (one per 256 blocks), `code` the 256-entry code book and `offset` the f32 scalar."""
    if blocksize != 64:
        raise ValueError("the HIP kernels take blocksize 64")
    n_bytes = packed.numel()
    nested = absmax_8bit is not None
    dev = _check_device(packed, absmax, absmax_8bit, code, offset)
    if out is None and ops.ENABLED:  # the compiled op: checks, allocation and launch in C++
        if nested:
            return ops.dequant(packed, shape, dtype, absmax_8bit=absmax_8bit, code=code,
                               absmax2=absmax, offset=offset)
        return ops.dequant(packed, shape, dtype, absmax=absmax)
    if out is None:
        out = torch.empty(shape, dtype=dtype, device=dev)
    elif out.dtype != dtype or not out.is_contiguous() or out.numel() != 2 * n_bytes:
        raise ValueError("out must be a contiguous tensor of the unpacked size and dtype")
    if packed.dtype != torch.uint8 or not packed.is_contiguous():
        raise ValueError("packed must be contiguous uint8")
    if nested:
        args = (_lib.ptr(absmax_8bit), _lib.ptr(code), _lib.ptr(absmax), _lib.ptr(offset), None)
    else:
        args = (None, None, None, None, _lib.ptr(absmax.float().contiguous()))
    _lib.call("mxs_nf4_dequant", _lib.ptr(packed), n_bytes, *args, _lib.ptr(out),
              _dtype_code(dtype), _lib.stream_of(dev))
    return out


def unpack_nf4_bytewise(packed, shape, absmax, blocksize, dtype, absmax_8bit=None, code=None,
                        offset=None):
    """The one-byte-per-lane kernel launched directly (as solution/test_nf4.py:68-82 does with
    nf4_unpack_kernel): the independent cross-check of the wide kernel."""
    if blocksize != 64:
        raise ValueError("the HIP kernels take blocksize 64")
    dev = _check_device(packed, absmax, absmax_8bit, code, offset)
    out = torch.empty(shape, dtype=dtype, device=dev)
    nested = absmax_8bit is not None
    if nested:
        args = (_lib.ptr(absmax_8bit), _lib.ptr(code), _lib.ptr(absmax), _lib.ptr(offset), None)
    else:
        args = (None, None, None, None, _lib.ptr(absmax.float().contiguous()))
    _lib.call("mxs_nf4_dequant_bytewise", _lib.ptr(packed.contiguous()), packed.numel(), *args,
              _lib.ptr(out), _dtype_code(dtype), _lib.stream_of(dev))
    return out


def launch_layer(packed, out, absmax_8bit, code, absmax2, offset, module_of, block0, scale0,
                 plan=None):
    """One launch: `out` (fp16) gets the values of all the weights packed one after the other
    (solution/nf4.py:158-162).  block0: int64 [n_modules + 1] (first block of each weight, then
    the total); scale0: int64 [n_modules] (first absmax2 index of each weight); code
    [n_modules * 256]; offset [n_modules].  `module_of` is accepted for the reference's signature
    and unused.  `plan`: the device workgroup -> weight map of layer_plan for this block0; without
    it, it is built here from block0's values (a host read of block0: callers in a loop build
    it once and pass it)."""
    del module_of
    dev = _check_device(packed, out, absmax_8bit, code, absmax2, offset, block0, scale0)
    n_modules = scale0.numel()
    if block0.numel() != n_modules + 1 or block0.dtype != torch.int64 or \
            scale0.dtype != torch.int64:
        raise ValueError("block0 must be int64 [n_modules + 1] and scale0 int64 [n_modules]")
    n_blocks = absmax_8bit.numel()
    if packed.numel() != 32 * n_blocks or out.numel() != 64 * n_blocks or \
            out.dtype != torch.float16:
        raise ValueError("packed/out sizes do not match the block count")
    if plan is None:
        plan = layer_plan(block0)
    elif plan.dtype != torch.int16 or plan.device != dev:
        raise ValueError("plan must be the int16 device map of layer_plan")
    _lib.call("mxs_nf4_dequant_layer", _lib.ptr(packed), n_blocks, _lib.ptr(absmax_8bit),
              _lib.ptr(code), _lib.ptr(absmax2), _lib.ptr(offset), _lib.ptr(block0),
              _lib.ptr(scale0), n_modules, _lib.ptr(plan), plan.numel(), _lib.ptr(out),
              _lib.stream_of(dev))
    return out


_PLANS = {}


def layer_plan(block0, device=None):
    """Device int16 map workgroup -> weight for the layer launch (the counterpart of the
    reference's per-program `module_of`, solution/stream.py:125-133), built on the host from
    block0's values (host or device tensor, or a sequence) and cached by those values: a
    different layout never gets another layout's plan."""
    if isinstance(block0, torch.Tensor):
        device = block0.device if device is None else device
        values = block0.detach().to("cpu", torch.int64).numpy()
    else:
        values = np.asarray(block0, np.int64)
    if device is None:
        raise ValueError("layer_plan needs a device for a host block0")
    b0 = np.ascontiguousarray(values, np.int64)
    key = (b0.tobytes(), str(torch.device(device)))
    plan = _PLANS.get(key)
    if plan is None:
        L = _lib.lib()
        n = L.mxs_nf4_dequant_layer_plan(b0.ctypes.data, b0.size - 1, None, 0)
        _lib.check(int(min(n, 0)), "mxs_nf4_dequant_layer_plan")
        host = np.empty(max(n, 1), np.int16)
        _lib.check(int(min(L.mxs_nf4_dequant_layer_plan(b0.ctypes.data, b0.size - 1,
                                                         host.ctypes.data, n), 0)),
                   "mxs_nf4_dequant_layer_plan")
        plan = torch.from_numpy(host[:max(n, 0)].copy()).to(device)
        if len(_PLANS) > 64:
            _PLANS.clear()
        _PLANS[key] = plan
    return plan


def _supported(packed, shape, blocksize, quant_type, dtype, nested_blocksize=256):
    """solution/nf4.py:165-172: what the HIP dequant takes."""
    numel = 1
    for dim in shape:
        numel *= int(dim)
    return (quant_type == "nf4" and blocksize == 64 and nested_blocksize == 256
            and dtype in (torch.float16, torch.float32) and packed.is_cuda
            and packed.dtype == torch.uint8 and packed.is_contiguous()
            and packed.numel() * 2 == numel)


def unpack_state(packed, state, dtype=None, absmax_8bit=None):
    """The dense weight of a QuantState (solution/linear4bit.py:36-40)."""
    return unpack_nf4(packed, state.shape, state.state2.absmax, state.blocksize,
                      dtype or state.dtype,
                      absmax_8bit=state.absmax if absmax_8bit is None else absmax_8bit,
                      code=state.state2.code, offset=state.offset)


def patch_bnb_nf4():
    """Hook bitsandbytes' dequant entry points (solution/nf4.py:175-211) when bitsandbytes is
    importable; returns False (no-op) when it is not."""
    try:
        import bitsandbytes.functional as bnb_functional
        from bitsandbytes.backends.cuda import ops as bnb_cuda_ops
    except Exception:
        return False

    if getattr(bnb_functional, "_mindx_patched", False):
        return True
    original_dequantize = bnb_functional.dequantize_4bit
    original_fallback = bnb_cuda_ops._dequant_linear_fallback

    def dequantize_4bit(A, quant_state=None, absmax=None, out=None, blocksize=None,
                        quant_type="fp4"):
        state = quant_state
        if (state is None or out is not None or A.dim() != 2 or A.shape[0] == 1
                or not _supported(A, state.shape, state.blocksize, state.quant_type,
                                  state.dtype,
                                  state.state2.blocksize if state.nested else 256)):
            return original_dequantize(A, quant_state=quant_state, absmax=absmax, out=out,
                                       blocksize=blocksize, quant_type=quant_type)
        if state.nested:
            return unpack_nf4(A, state.shape, state.state2.absmax, state.blocksize, state.dtype,
                              absmax_8bit=state.absmax, code=state.state2.code,
                              offset=state.offset)
        return unpack_nf4(A, state.shape, state.absmax.float(), state.blocksize, state.dtype)

    def dequant_linear_fallback(A, B, shapeB, absmax, blocksize, quant_type, bias=None,
                                absmax_8bit=None, absmax_code=None, absmax_offset=None):
        if not _supported(B, shapeB, blocksize, quant_type, A.dtype) or \
                (absmax_8bit is None and absmax.dtype != torch.float32):
            return original_fallback(A, B, shapeB, absmax, blocksize, quant_type, bias,
                                     absmax_8bit, absmax_code, absmax_offset)
        weight = unpack_nf4(B, shapeB, absmax, blocksize, A.dtype, absmax_8bit=absmax_8bit,
                            code=absmax_code, offset=absmax_offset)
        return torch.nn.functional.linear(A, weight, bias)

    bnb_functional.dequantize_4bit = dequantize_4bit
    bnb_cuda_ops._dequant_linear_fallback = dequant_linear_fallback
    bnb_functional._mindx_patched = True
    return True
