"""Autograd functions called directly when no gradient is recorded (solution/direct.py:15-36).

Under no_grad, `Function.apply` only adds Python around `Function.forward`; `run` calls the
forward with a context object that drops whatever backward would have needed.
"""

import torch

enabled = False  # set by apply()


class _NoBackward:
    """The context a Function's forward sees when there will be no backward."""

    needs_input_grad = ()

    def __setattr__(self, _name, _value):
        pass  # one shared instance: it must not keep anything alive

    def save_for_backward(self, *_tensors):
        pass

    def mark_non_differentiable(self, *_tensors):
        pass


_context = _NoBackward()


def run(function, *args):
    if enabled and not torch.is_grad_enabled():
        return function.forward(_context, *args)
    return function.apply(*args)
