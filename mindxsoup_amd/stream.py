"""Decoder layers' NF4 weights kept in pinned host memory and brought to the GPU one layer at a
time (mirror of solution/stream.py).

Each layer's packed NF4 bytes, then its 8-bit block scales, sit back to back in one pinned host
block (one host-to-device copy per layer); each module keeps a 1-byte device placeholder of the
same shape, so the module still looks like a GPU Linear4bit.  A ring of device slots holds the
layers in use.  While layer i runs, a second HIP stream (default priority) copies the next
layers (up to SLOTS - 1) in the order the layers run (forward, or backward).  A slot is
overwritten only after all work enqueued on the compute stream so far has finished, and the
compute stream waits for a slot's copy before reading it.

Correctness never depends on the prefetching.  Every NF4 product asks for its module's bytes
right before use (`bytes_for`), in forward and again in backward, and a layer that is not
resident is copied in then.  The bytes are the same bytes, so results are bit-identical to
keeping the weights on the GPU.  The product reads the slot directly: the fused NF4 GEMMs decode
the packed bytes in their main loop.  With LAYER_UNPACK the running layer is instead decoded
to fp16 by one launch (`nf4.launch_layer`) and multiplied by torch (the reference's structure).
"""

import copy
import threading

import torch

from . import nf4

SLOTS = 3          # device slots (layers resident at once): 24 MB each at Qwen2.5-1.5B's
                   # shapes, and with 3 a step copies ~2 of 4 layers instead of ~4
PREFETCH = 2       # layers copied ahead of the running one (at most SLOTS - 1)
LAYER_UNPACK = False  # FEATURES["layer_unpack"]: the running layer decoded to fp16 in one launch
_ALIGN = 256       # byte alignment of every module's span inside a slot

_streamer = None
enabled = False    # set by patch_stream_layers()


def _round_up(n, a=_ALIGN):
    return (n + a - 1) // a * a


def offload(param, pin=True):
    """Move a quantized weight's packed bytes and 8-bit block scales to host memory, once; 1-byte
    device placeholders of the same shapes stay behind (solution/stream.py:220-235)."""
    if hasattr(param, "_mindx_host"):
        return
    data = param.data
    state = param.quant_state
    host = torch.empty(data.numel(), dtype=torch.uint8, pin_memory=pin)
    host.copy_(data.reshape(-1))
    absmax = torch.empty(state.absmax.numel(), dtype=torch.uint8, pin_memory=pin)
    absmax.copy_(state.absmax.reshape(-1))
    param._mindx_host, param._mindx_shape, param._mindx_absmax = host, tuple(data.shape), absmax
    param.data = torch.empty(1, dtype=torch.uint8, device=data.device).expand(data.shape)
    state.absmax = torch.empty(1, dtype=torch.uint8,
                               device=state.absmax.device).expand(state.absmax.shape)


def offloaded(module):
    return hasattr(getattr(module, "weight", None), "_mindx_host")


class SlotTable:
    """Which layer each device slot holds, and the least-recently-used choice of the slot to
    overwrite (solution/stream.py:137-145).  Host bookkeeping only."""

    def __init__(self, n_slots):
        self.layer = [None] * n_slots
        self.used = [0] * n_slots
        self.slot_of = {}
        self.clock = 0

    def victim(self, keep):
        """A free slot, else the least recently used one whose layer is not in `keep`; None when
        every slot holds a layer in `keep`."""
        for i, layer in enumerate(self.layer):
            if layer is None:
                return i
        free = [i for i, layer in enumerate(self.layer) if layer not in keep]
        return min(free, key=lambda i: self.used[i]) if free else None

    def assign(self, slot, layer):
        old = self.layer[slot]
        if old is not None:
            del self.slot_of[old]
        self.layer[slot] = layer
        self.slot_of[layer] = slot

    def touch(self, slot):
        self.clock += 1
        self.used[slot] = self.clock


class LayerStreamer:
    """The host blocks, the device slots and the copy stream for a list of decoder layers (each
    a list of NF4 modules in call order)."""

    def __init__(self, groups, slots=None, prefetch=None, layer_unpack=None):
        self.groups = groups
        self.lock = threading.RLock()
        self.device = groups[0][0].weight.device
        self.copy_stream = torch.cuda.Stream(self.device)
        self.entries = {}  # id(module) -> (layer, offset, numel, shape, absmax offset, numel)
        self.host_layers = []
        sizes = []
        for layer, modules in enumerate(groups):
            spans, offset = [], 0
            for m in modules:
                offload(m.weight, pin=False)  # copied into the pinned layer block below
                n = m.weight._mindx_host.numel()
                spans.append([layer, offset, n, m.weight._mindx_shape])
                offset = _round_up(offset + n)
            for m, span in zip(modules, spans):
                n = m.weight._mindx_absmax.numel()
                span += [offset, n]
                offset = _round_up(offset + n)
            host = torch.empty(offset, dtype=torch.uint8, pin_memory=True)
            for m, span in zip(modules, spans):
                _, o, n, _, ao, an = span
                host[o:o + n].copy_(m.weight._mindx_host)
                host[ao:ao + an].copy_(m.weight._mindx_absmax)
                m.weight._mindx_host, m.weight._mindx_absmax = host[o:o + n], host[ao:ao + an]
                self.entries[id(m)] = tuple(span)
            self.host_layers.append(host)
            sizes.append(offset)
        n_slots = max(1, min(SLOTS if slots is None else slots, len(groups)))
        self.slots = [torch.empty(max(sizes), dtype=torch.uint8, device=self.device)
                      for _ in range(n_slots)]
        self.table = SlotTable(n_slots)
        self.ready = [None] * n_slots
        self.prefetch = PREFETCH if prefetch is None else prefetch
        self.current = None
        self.loads = 0          # layer copies issued
        self.unpacked = None    # the layer whose fp16 weights the buffer holds
        self.weights = {}       # id(module) -> [N, K] fp16 view of the buffer
        self.hooks = []         # handles of the layer hooks installed by setup()
        unpack = LAYER_UNPACK if layer_unpack is None else layer_unpack
        self.layer_tables = self._layer_tables() if unpack else None

    def _layer_tables(self):
        """Per layer, what the one-launch layer decode reads besides the slot (code books,
        second-level scales, offsets); None unless every layer has the same list of shapes and
        each layer's packed bytes and block scales are contiguous in its slot."""
        if len({tuple(tuple(m.weight.quant_state.shape) for m in g) for g in self.groups}) != 1:
            return None
        first = self.groups[0]
        abs_start = self.entries[id(first[0])][4]
        blocks = scales = 0
        block0, scale0 = [], []
        for m in first:
            _, off, n, _, ao, an = self.entries[id(m)]
            st = m.weight.quant_state
            if (off != blocks * 32 or ao != abs_start + blocks or an * 32 != n
                    or not getattr(st, "nested", False) or st.state2.code.numel() != 256
                    or st.offset.numel() != 1 or st.dtype != torch.float16):
                return None
            block0.append(blocks)
            scale0.append(scales)
            blocks += an
            scales += st.state2.absmax.numel()
        block0.append(blocks)
        dev = self.device
        tables = []
        for g in self.groups:
            sts = [m.weight.quant_state for m in g]
            tables.append((torch.cat([s.state2.code.reshape(-1).float() for s in sts]).to(dev),
                           torch.cat([s.state2.absmax.reshape(-1).float() for s in sts]).to(dev),
                           torch.cat([s.offset.reshape(-1).float() for s in sts]).to(dev)))
        self.block0 = torch.tensor(block0, dtype=torch.int64, device=dev)
        self.scale0 = torch.tensor(scale0, dtype=torch.int64, device=dev)
        self.plan = nf4.layer_plan(block0, dev)  # built once, from the host values
        self.packed_bytes, self.absmax_start = blocks * 32, abs_start
        self.buffer = torch.empty(blocks * 64, dtype=torch.float16, device=dev)
        for g in self.groups:
            at = 0
            for m in g:
                n = self.entries[id(m)][2]
                self.weights[id(m)] = self.buffer[at:at + 2 * n].view(
                    tuple(m.weight.quant_state.shape))
                at += 2 * n
        return tables

    def _load(self, layer, keep):
        slot = self.table.victim(keep)
        if slot is None:  # every slot holds a layer to keep: take the least recently used
            slot = min(range(len(self.slots)), key=lambda i: self.table.used[i])
        # the slot's old layer may still be read by work already on the compute stream
        done = torch.cuda.current_stream(self.device).record_event()
        self.copy_stream.wait_event(done)
        with torch.cuda.stream(self.copy_stream):
            host = self.host_layers[layer]
            self.slots[slot][:host.numel()].copy_(host, non_blocking=True)
            self.ready[slot] = self.copy_stream.record_event()
        # the allocator must not hand the slot's memory to anything else while this copy can
        # still be writing it (a streamer dropped by reset() with a prefetch in flight)
        self.slots[slot].record_stream(self.copy_stream)
        if self.unpacked == self.table.layer[slot]:
            self.unpacked = None
        self.table.assign(slot, layer)
        self.loads += 1
        return slot

    def _acquire(self, layer):
        slot = self.table.slot_of.get(layer)
        if slot is None:
            slot = self._load(layer, keep={layer, self.current})
        torch.cuda.current_stream(self.device).wait_event(self.ready[slot])
        self.table.touch(slot)
        return slot

    def _unpack_layer(self, layer, slot):
        if self.layer_tables is None or self.unpacked == layer:
            return
        data = self.slots[slot]
        code, absmax2, offset = self.layer_tables[layer]
        nf4.launch_layer(data[:self.packed_bytes], self.buffer,
                         data[self.absmax_start:self.absmax_start + self.packed_bytes // 32],
                         code, absmax2, offset, None, self.block0, self.scale0, self.plan)
        self.unpacked = layer

    def bytes_for(self, module):
        """The module's packed bytes ([shape] u8) and 8-bit block scales on the GPU, ready for
        the current stream (solution/stream.py:186-193)."""
        with self.lock:
            layer, off, n, shape, ao, an = self.entries[id(module)]
            data = self.slots[self._acquire(layer)]
            return data[off:off + n].view(shape), data[ao:ao + an]

    def weight_for(self, module):
        """The module's fp16 weight when its layer is the one decoded in the buffer, else
        None."""
        with self.lock:
            if self.entries[id(module)][0] != self.unpacked:
                return None
            return self.weights[id(module)]

    def layer_begins(self, layer, forward):
        """Hint: decoder layer `layer` is about to run (forward, or its backward); bring it in,
        decode it when LAYER_UNPACK, and copy the next layers in the order they will run
        (solution/stream.py:195-215)."""
        with self.lock:
            if not 0 <= layer < len(self.groups):
                return
            self.current = layer
            self._unpack_layer(layer, self._acquire(layer))
            step = 1 if forward else -1
            keep = {layer}
            for ahead in range(1, min(self.prefetch, len(self.slots) - 1) + 1):
                nxt = layer + step * ahead
                if not 0 <= nxt < len(self.groups):
                    break
                if nxt not in self.table.slot_of:
                    if self.table.victim(keep | {nxt}) is None:
                        break  # no slot to spare: the layer is copied when it is used
                    self._load(nxt, keep | {nxt})
                keep.add(nxt)

    def owns(self, module):
        return id(module) in self.entries


def bytes_for(module):
    """The module's packed bytes and block scales on the GPU: from the streamer's slots, or
    (before a streamer exists) a one-off synchronous copy."""
    if _streamer is not None and _streamer.owns(module):
        return _streamer.bytes_for(module)
    w = module.weight
    return (w._mindx_host.to(w.device).view(w._mindx_shape), w._mindx_absmax.to(w.device))


def weight_for(module):
    """The module's weight already decoded for the running layer, or None."""
    if _streamer is not None and _streamer.owns(module):
        return _streamer.weight_for(module)
    return None


def state_with(state, absmax):
    """A shallow copy of a quant state whose 8-bit block scales are `absmax` (a slot view)."""
    s = copy.copy(state)
    s.absmax = absmax
    return s


def active():
    return _streamer is not None


def streamer():
    return _streamer


def reset():
    """Forget the streamer and remove its layer hooks (its modules stay offloaded and use
    one-off copies)."""
    global _streamer
    if _streamer is not None:
        for h in _streamer.hooks:
            h.remove()
    _streamer = None


def _is_nf4(module):
    from .linear4bit import Linear4bit

    if isinstance(module, Linear4bit):
        return True
    try:
        import bitsandbytes as bnb
    except Exception:
        return False
    return isinstance(module, bnb.nn.Linear4bit)


def _streamable(module):
    """solution/stream.py:260-269."""
    w = module.weight
    state = getattr(w, "quant_state", None)
    return (w is not None and w.is_cuda and w.dtype == torch.uint8
            and (hasattr(w, "_mindx_host") or w.data.is_contiguous())
            and state is not None and getattr(state, "nested", False)
            and state.quant_type == "nf4" and state.blocksize == 64
            and getattr(state, "state2", None) is not None and state.state2.blocksize == 256
            and state.dtype == torch.float16 and module.compute_dtype == torch.float16
            and not getattr(state, "packing_format_for_cpu", False))


def setup(causal_lm, slots=None, prefetch=None, layer_unpack=None, hints=True):
    """Move the decoder layers' NF4 weights to the host, once, and start the streamer; only
    when every layer (`causal_lm.model.layers`) holds plain fp16-compute NF4 modules on one GPU
    (solution/stream.py:272-290).  With `hints`, each layer's forward pre-hook says that the
    layer begins, and a hook on its input's gradient says that the layer below begins its
    backward.  Returns whether the streamer runs."""
    global _streamer
    if _streamer is not None:
        return True
    if not enabled:
        return False
    layers = getattr(getattr(causal_lm, "model", None), "layers", None)
    if layers is None or not torch.cuda.is_available():
        return False
    groups = [[m for m in layer.modules() if _is_nf4(m)] for layer in layers]
    if not groups or any(not g for g in groups) or \
            not all(_streamable(m) for g in groups for m in g) or \
            len({m.weight.device for g in groups for m in g}) != 1:
        return False
    for g in groups:
        for m in g:
            m.compute_type_is_set = True
    _streamer = LayerStreamer(groups, slots, prefetch, layer_unpack)
    if hints:
        _streamer.hooks = [layer.register_forward_pre_hook(_hint_hook(index, _streamer))
                           for index, layer in enumerate(layers)]
    return True


def _hint_hook(index, s):
    def hook(module, args):
        if _streamer is not s:  # the streamer this hook was installed for is gone
            return None
        s.layer_begins(index, forward=True)
        x = args[0] if args else None
        if isinstance(x, torch.Tensor) and x.requires_grad and torch.is_grad_enabled():
            # fires when this layer's backward has produced its input gradient
            x.register_hook(lambda g: _backward_hint(s, index - 1))
        return None
    return hook


def _backward_hint(s, index):
    """The input-gradient hook's hint, dropped when reset() has retired its streamer between a
    forward and its backward."""
    if _streamer is s:
        s.layer_begins(index, forward=False)


def patch_stream_layers():
    """FEATURES["stream_weights"]: allow `setup` (solution/stream.py:349-352)."""
    global enabled
    enabled = True
