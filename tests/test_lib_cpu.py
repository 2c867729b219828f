"""The C-ABI library without a GPU: it loads, and exports every symbol include/mxs_nf4.h
declares (no compute calls here)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "mxs_nf4.h")).read()
    return sorted(set(re.findall(r"^(?:int|int64_t)\s+(mxs_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = _declared()
    assert "mxs_nf4_dequant" in names and "mxs_nf4_dequant_layer" in names
    assert len(names) >= 5


def test_library_exports_every_declared_symbol():
    from mindxsoup_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: build with `python -m mindxsoup_amd.build`")
    handle = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(handle, name), name
    # the Python binding knows every declared symbol, and nothing undeclared
    assert sorted(_lib.exported_symbols()) == _declared()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from mindxsoup_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(_lib.MxsLibraryError):
        _lib.lib()


def test_error_codes_raise():
    from mindxsoup_amd import _lib

    with pytest.raises(RuntimeError, match="alignment"):
        _lib.check(-3, "x")
    _lib.check(0, "x")


def test_layer_plan_marks_straddling_workgroups():
    """The host-side plan of the layer launch: 128 blocks per workgroup; -1 where one straddles."""
    import numpy as np

    from mindxsoup_amd import _lib

    L = _lib.lib()
    block0 = np.array([0, 128, 300, 300, 640], np.int64)  # includes an empty module
    n = L.mxs_nf4_dequant_layer_plan(block0.ctypes.data, 4, None, 0)
    assert n == 5
    out = np.zeros(n, np.int16)
    assert L.mxs_nf4_dequant_layer_plan(block0.ctypes.data, 4, out.ctypes.data, n) == n
    assert out.tolist() == [0, 1, -1, 3, 3]  # workgroup 2 spans blocks 256..383: modules 1 and 3
    assert L.mxs_nf4_dequant_layer_plan(block0.ctypes.data, 4, out.ctypes.data, 2) < 0
