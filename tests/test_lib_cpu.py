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


def test_probe_library_apart_from_the_product():
    """The HBM probes bench.py reports live in libmxs_probe.so (include/mxs_probe.h), not in
    the product library or its header."""
    from mindxsoup_amd import _lib

    text = open(os.path.join(ROOT, "include", "mxs_probe.h")).read()
    names = re.findall(r"^int\s+(mxs_\w+)\s*\(", text, flags=re.M)
    assert names == ["mxs_hbm_probe"]
    assert "mxs_hbm_probe" not in _declared()
    assert hasattr(_lib.probe_lib(), "mxs_hbm_probe")
    assert not hasattr(ctypes.CDLL(_lib.LIB_PATH), "mxs_hbm_probe")


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


def test_group_rope_entry_checks_its_rotation_operands_on_the_host():
    """mxs_nf4_linear_fwd_hp_group_rope refuses bad rotation operands before any device work:
    a rotated output that is not whole 128-column heads, n_rope outside 1..n, missing or
    misaligned cos / sin, and rows that are not whole sequences."""
    import ctypes

    from mindxsoup_amd import _lib

    f = _lib.lib().mxs_nf4_linear_fwd_hp_group_rope
    p = (ctypes.c_void_p * 2)(0x1000, 0x1000)  # stand-ins, never dereferenced on these paths

    def call(N, n_rope=1, cos=0x1000, cs_t=128, T=64, M=128):
        Ns = (ctypes.c_int * 2)(*N)
        return f(2, p, M, 256, Ns, p, p, p, p, p, None, None, 0, 0, None, 16, None, p, n_rope,
                 cos, 0x1000, 0, cs_t, T, None)

    assert call((192, 128)) == -4  # MXS_ERR_SIZE
    assert call((128, 128), n_rope=0) == -1  # MXS_ERR_ARG
    assert call((128, 128), n_rope=3) == -1
    assert call((128, 128), cos=None) == -1
    assert call((128, 128), T=48) == -1
    assert call((128, 128), cos=0x1004) == -3  # MXS_ERR_ALIGN
    assert call((128, 128), cs_t=130) == -3


def test_keep_bits_checks_shape_and_dtype():
    """keep_bits passes int32 [M, ceil(K/32)] through untouched and refuses other shapes and
    dtypes before anything is launched (no GPU needed)."""
    import pytest
    import torch

    from mindxsoup_amd import kernels

    assert kernels.keep_words(1) == 1 and kernels.keep_words(32) == 1 and kernels.keep_words(33) == 2
    bits = torch.zeros((4, 3), dtype=torch.int32)
    assert kernels.keep_bits(bits, 4, 96) is bits or kernels.keep_bits(bits, 4, 96).data_ptr() == bits.data_ptr()
    assert kernels.keep_bits(None, 4, 96) is None
    for bad in (torch.zeros((4, 4), dtype=torch.int32), torch.zeros((4, 95), dtype=torch.uint8),
                torch.zeros((4, 96), dtype=torch.float16)):
        with pytest.raises(ValueError):
            kernels.keep_bits(bad, 4, 96)
