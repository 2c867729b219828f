"""NF4 weights on the GPU: bitsandbytes' QuantState fields and a quantizer.

`QuantState` keeps the attribute names the reference reads from `layer.weight.quant_state`
(solution/linear4bit.py:36-40, 112-129): shape, blocksize, quant_type, dtype, nested, absmax
(u8 codes when nested), offset, state2.absmax, state2.code, state2.blocksize.  `quantize_4bit`
produces them with the HIP quantizer (mxs_nf4_quantize), standing in for bitsandbytes'
quantize_4bit(..., compress_statistics=True) that the reference calls
(solution/test_nf4.py:33).
"""

from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib


@dataclass
class QuantState2:
    absmax: torch.Tensor          # f32 [ceil(n_blocks / 256)]
    code: torch.Tensor            # f32 [256]
    blocksize: int = 256


@dataclass
class QuantState:
    shape: tuple                  # (N, K) of the dense weight
    absmax: torch.Tensor          # u8 [n_blocks] when nested, else f32 [n_blocks]
    blocksize: int = 64
    quant_type: str = "nf4"
    dtype: torch.dtype = torch.float16
    offset: torch.Tensor = None   # f32 scalar tensor (nested)
    state2: QuantState2 = None
    nested: bool = True
    packing_format_for_cpu: bool = False
    absmax_f32: torch.Tensor = field(default=None, repr=False)  # first level, before nesting

    def to(self, device):
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        s2 = None if self.state2 is None else QuantState2(mv(self.state2.absmax),
                                                          mv(self.state2.code),
                                                          self.state2.blocksize)
        return QuantState(self.shape, mv(self.absmax), self.blocksize, self.quant_type,
                          self.dtype, mv(self.offset), s2, self.nested,
                          self.packing_format_for_cpu, mv(self.absmax_f32))


def dynamic_map():
    """Signed 8-bit dynamic-tree code book (Dettmers, arXiv 1511.04561), ascending, f32 [256]:
    for decade i = 0..6, the 2^i midpoints of an even fp32 split of [0.1, 1] scaled by 10^(i-6),
    both signs; plus 0 and 1.  The second-level code book of bitsandbytes' nested absmax."""
    vals = []
    for i in range(7):
        items = (1 << i) + 1
        scale = 10.0 ** (i - 6)
        b = np.array([np.float32(0.1 + 0.9 * j / (items - 1)) for j in range(items)], np.float32)
        mids = (b[:-1] + b[1:]) / np.float32(2.0)
        for m in mids:
            vals.append(np.float32(scale * float(m)))
            vals.append(np.float32(-scale * float(m)))
    vals += [np.float32(0.0), np.float32(1.0)]
    return np.sort(np.array(vals, np.float32))


_CODE = {}


def code_book(device):
    t = _CODE.get(device)
    if t is None:
        t = torch.from_numpy(dynamic_map()).to(device)
        _CODE[device] = t
    return t


def quantize_4bit(weight, blocksize=64, quant_type="nf4", compress_statistics=True):
    """(packed u8 [(N*K)//2, 1], QuantState) of an fp16 CUDA weight, on the GPU.
    Only the configuration the hot path takes is built: NF4, blocksize 64, nested absmax."""
    if quant_type != "nf4" or blocksize != 64 or not compress_statistics:
        raise NotImplementedError("the HIP quantizer builds NF4, blocksize 64, nested absmax")
    if not weight.is_cuda or weight.dtype != torch.float16:
        raise ValueError("quantize_4bit takes an fp16 CUDA tensor")
    w = weight.contiguous()
    n = w.numel()
    if n % 64:
        raise ValueError("the number of values must be a multiple of 64")
    dev = w.device
    nb = n // 64
    packed = torch.empty(n // 2, dtype=torch.uint8, device=dev)
    absmax_f32 = torch.empty(nb, dtype=torch.float32, device=dev)
    absmax8 = torch.empty(nb, dtype=torch.uint8, device=dev)
    absmax2 = torch.empty((nb + 255) // 256, dtype=torch.float32, device=dev)
    offset = torch.empty((), dtype=torch.float32, device=dev)
    L = _lib.lib()
    ws = torch.empty(L.mxs_nf4_quantize_workspace_bytes(n), dtype=torch.uint8, device=dev)
    code = code_book(dev)
    _lib.call("mxs_nf4_quantize", _lib.ptr(w), n, _lib.ptr(code), _lib.ptr(packed),
              _lib.ptr(absmax_f32), _lib.ptr(absmax8), _lib.ptr(absmax2), _lib.ptr(offset),
              _lib.ptr(ws), _lib.stream_of(dev))
    state = QuantState(shape=tuple(weight.shape), absmax=absmax8, offset=offset,
                       state2=QuantState2(absmax2, code), absmax_f32=absmax_f32,
                       dtype=weight.dtype)
    return packed.view(-1, 1), state
