"""Models onto the NF4 path: a model's linear layers replaced by this package's Linear4bit
(quantized on the GPU, bitsandbytes' NF4 with nested absmax), optionally wrapped in peft-layout
LoRA layers, as transformers' load_in_4bit + peft build the model the reference trains
(solution/test_attention.py:27-54).  Checkpoints in bitsandbytes' serialized form load through
the modules' own load_state_dict (Linear4bit reads "weight" and "weight.<quant state key>").
"""

import torch

from . import stream
from .linear4bit import Linear4bit, LoraLinear4bit

QWEN2_TARGETS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def replace_with_nf4(model, skip=("lm_head",), lora_targets=(), r=16, lora_alpha=32,
                     lora_dropout=0.05, device=None, offload=False):
    """Replace every torch.nn.Linear of `model` (except modules whose name ends with a name in
    `skip`) by a Linear4bit quantized on `device` (default cuda:0) from its weight in fp16; those
    whose attribute name is in `lora_targets` are wrapped in LoraLinear4bit(r, lora_alpha,
    lora_dropout).  With `offload`, each decoder-layer weight (a name containing ".layers.")
    moves to host memory right after it is quantized, so the 4-bit layers never sit on the GPU
    all at once (solution/stream.py:293-330); stream.setup then streams them.  Returns the list
    of replaced module names."""
    dev = torch.device(device or "cuda:0")
    done = []
    for name, module in list(model.named_modules()):
        for child_name, child in list(module.named_children()):
            full = f"{name}.{child_name}" if name else child_name
            if type(child) is not torch.nn.Linear or any(full.endswith(s) for s in skip):
                continue
            w = child.weight.detach().to(device=dev, dtype=torch.float16)
            b = None if child.bias is None else child.bias.detach().to(dev, torch.float16)
            layer = Linear4bit.from_weight(w, b)
            if offload and ".layers." in f".{full}":
                stream.offload(layer.weight, pin=False)  # pinned per layer by the streamer
            if child_name in lora_targets:
                layer = LoraLinear4bit(layer, r=r, lora_alpha=lora_alpha,
                                       lora_dropout=lora_dropout)
            setattr(module, child_name, layer)
            done.append(full)
    return done
