"""pytest setup: the `gpu` marker, import paths and shared fixtures."""

import os
import sys
import types

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mindxsoup_amd import _lib

    _lib.lib()  # raises if the HIP library is not built: GPU tests never run without it
    return torch.device("cuda:0")


class _Recorder:
    def __init__(self, result="original"):
        self.calls = []
        self.result = result

    def __call__(self, *args, **kwargs):
        self.calls.append((args, kwargs))
        return self.result


@pytest.fixture
def fake_bnb(monkeypatch):
    """A bitsandbytes package with the three entry points the reference patches."""
    import torch

    bnb = types.ModuleType("bitsandbytes")
    functional = types.ModuleType("bitsandbytes.functional")
    backends = types.ModuleType("bitsandbytes.backends")
    cuda = types.ModuleType("bitsandbytes.backends.cuda")
    ops = types.ModuleType("bitsandbytes.backends.cuda.ops")
    nn = types.ModuleType("bitsandbytes.nn")
    functional.dequantize_4bit = _Recorder("dequantize_4bit")
    ops._dequant_linear_fallback = _Recorder("fallback")

    class Linear4bit(torch.nn.Module):
        def forward(self, x):
            return "bnb forward"

    nn.Linear4bit = Linear4bit
    bnb.functional, bnb.backends, bnb.nn = functional, backends, nn
    backends.cuda, cuda.ops = cuda, ops
    for name, mod in (("bitsandbytes", bnb), ("bitsandbytes.functional", functional),
                      ("bitsandbytes.backends", backends), ("bitsandbytes.backends.cuda", cuda),
                      ("bitsandbytes.backends.cuda.ops", ops), ("bitsandbytes.nn", nn)):
        monkeypatch.setitem(sys.modules, name, mod)
    return types.SimpleNamespace(bnb=bnb, functional=functional, ops=ops, nn=nn)
