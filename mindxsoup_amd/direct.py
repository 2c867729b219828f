"""Autograd Functions without the autograd wrapper when no graph is being recorded.

The reference calls each of its Functions through a helper that skips `Function.apply` under
no_grad (solution/direct.py:15-36): in a forward that records nothing, `apply` only adds Python
around `forward`, once per projection per layer.  `run(function, *args)` does the same here.
Its context stand-in is built fresh for each call and dropped when the call returns, so whatever
a forward stores on it (saved tensors, shapes) dies with the call instead of outliving it.
"""

import torch

enabled = False  # set by apply() from FEATURES["direct_nograd"]


class _Unrecorded:
    """What a Function's forward gets for `ctx` when nothing is recorded: attribute writes land
    on this throwaway object; saving and marking are no-ops."""

    needs_input_grad = ()
    materialize_grads = True

    def save_for_backward(self, *tensors):
        del tensors

    def mark_non_differentiable(self, *tensors):
        del tensors

    def mark_dirty(self, *tensors):
        del tensors

    def set_materialize_grads(self, value):
        self.materialize_grads = value


def run(function, *args):
    """function.apply(*args), or function.forward on a throwaway context when grad mode is off
    (and the switch is on): same outputs, no autograd node."""
    if enabled and not torch.is_grad_enabled():
        return function.forward(_Unrecorded(), *args)
    return function.apply(*args)
