"""NF4 weights on the GPU: bitsandbytes' QuantState fields and a quantizer.

`QuantState` keeps the attribute names the reference reads from `layer.weight.quant_state`
(solution/linear4bit.py:36-40, 112-129): shape, blocksize, quant_type, dtype, nested, absmax
(u8 codes when nested), offset, state2.absmax, state2.code, state2.blocksize.  `quantize_4bit`
produces them with the HIP quantizer (mxs_nf4_quantize), standing in for bitsandbytes'
quantize_4bit(..., compress_statistics=True) that the reference calls
(solution/test_nf4.py:33).
"""

import json
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib

# bitsandbytes' serialized QuantState (bitsandbytes 0.43-0.45, functional.py: QuantState.as_dict,
# from_dict, pack_dict_to_tensor; not part of the reference tree, which calls it through
# bitsandbytes): tensor fields under their own keys, the rest as the UTF-8 bytes of a JSON
# object in one u8 tensor under "quant_state.bitsandbytes__<quant_type>".
_QS_KEYS = ("absmax", "quant_map", "nested_absmax", "nested_quant_map", "quant_state",
            "quant_type", "blocksize", "dtype", "shape", "nested_blocksize", "nested_dtype",
            "nested_offset")


def pack_dict_to_tensor(d):
    """A JSON-serializable dict as a u8 tensor of its UTF-8 JSON text."""
    return torch.tensor(list(json.dumps(d).encode("utf-8")), dtype=torch.uint8)


def unpack_tensor_to_dict(t):
    return json.loads(bytes(t.cpu().numpy().tolist()).decode("utf-8"))


def _dtype_name(dt):
    return str(dt).replace("torch.", "")


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

    def as_dict(self, packed=False):
        """bitsandbytes' QuantState.as_dict: absmax, quant_map (the 16 NF4 values), and for the
        nested form nested_absmax, nested_quant_map, nested_blocksize, nested_dtype,
        nested_offset; with packed=True the non-tensor fields go into one u8 tensor under
        "quant_state.bitsandbytes__nf4" (the form Linear4bit writes into a state dict)."""
        from .nf4 import NF4_VALUES

        d = {"quant_type": self.quant_type, "absmax": self.absmax, "blocksize": self.blocksize,
             "quant_map": torch.from_numpy(NF4_VALUES.copy()).to(self.absmax.device),
             "dtype": _dtype_name(self.dtype), "shape": tuple(int(v) for v in self.shape)}
        if self.nested:
            d.update({"nested_absmax": self.state2.absmax,
                      "nested_blocksize": self.state2.blocksize,
                      "nested_quant_map": self.state2.code.clone(),
                      "nested_dtype": _dtype_name(self.state2.absmax.dtype),
                      "nested_offset": float(self.offset.item())})
        if not packed:
            return d
        out = {k: v for k, v in d.items() if isinstance(v, torch.Tensor)}
        out["quant_state.bitsandbytes__" + self.quant_type] = pack_dict_to_tensor(
            {k: v for k, v in d.items() if not isinstance(v, torch.Tensor)})
        return out

    @classmethod
    def from_dict(cls, qs_dict, device):
        """bitsandbytes' QuantState.from_dict over keys with any prefix (packed or unpacked).
        Only NF4 with a nested absmax at blocksizes 64 / 256 is built here."""
        qs_dict = dict(qs_dict)
        packed_keys = [k for k, v in qs_dict.items()
                       if "quant_state" in k and isinstance(v, torch.Tensor)]
        if not packed_keys and "quant_type" not in qs_dict:
            raise ValueError("expected packed or unpacked quant_state items, found neither")
        if len(packed_keys) > 1 or (packed_keys and
                                    packed_keys[0].split(".")[-1] != "bitsandbytes__nf4"):
            raise ValueError(f"unsupported quant_state items {packed_keys}")
        if packed_keys:
            qs_dict.update(unpack_tensor_to_dict(qs_dict.pop(packed_keys[0])))
        qs_dict = {k.split(".")[-1]: v for k, v in qs_dict.items()}
        unknown = set(qs_dict) - set(_QS_KEYS)
        if unknown:
            raise ValueError(f"unexpected quant_state keys {sorted(unknown)}")
        from .nf4 import NF4_VALUES

        qmap = qs_dict["quant_map"].detach().float().cpu().numpy()
        if (qs_dict["quant_type"] != "nf4" or "nested_absmax" not in qs_dict
                or int(qs_dict["blocksize"]) != 64 or int(qs_dict["nested_blocksize"]) != 256
                or not np.array_equal(qmap, NF4_VALUES.astype(np.float32))):
            raise NotImplementedError("the HIP path takes NF4, blocksize 64, nested absmax "
                                      "(blocksize 256)")
        state2 = QuantState2(qs_dict["nested_absmax"].to(device=device, dtype=torch.float32),
                             qs_dict["nested_quant_map"].to(device=device, dtype=torch.float32),
                             int(qs_dict["nested_blocksize"]))
        return cls(shape=tuple(int(v) for v in qs_dict["shape"]),
                   absmax=qs_dict["absmax"].to(device), blocksize=int(qs_dict["blocksize"]),
                   quant_type="nf4", dtype=getattr(torch, qs_dict["dtype"]),
                   offset=torch.tensor(float(qs_dict["nested_offset"]), dtype=torch.float32,
                                       device=device),
                   state2=state2, nested=True)

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
