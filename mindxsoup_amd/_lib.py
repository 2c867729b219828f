"""ctypes binding of libmxs_nf4.so (the C ABI declared in include/mxs_nf4.h).

This is the only way the Python side reaches the GPU kernels.  There is no fallback: if the
library is missing or fails to load, every call raises MxsLibraryError, naming the build command.
Tensors are passed as raw device pointers; launches go to torch's current HIP stream.
"""

import ctypes
import os

import torch

# MXS_NF4_LIB names another build of the same library (A/B timing of kernel variants).
LIB_PATH = os.environ.get("MXS_NF4_LIB") or \
    os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmxs_nf4.so")

MXS_DTYPE_F16 = 0
MXS_DTYPE_F32 = 1

_ERRORS = {-1: "bad argument (null pointer or negative size)", -2: "unsupported dtype",
           -3: "pointer alignment", -4: "shape outside what the kernels take"}


class MxsLibraryError(RuntimeError):
    pass


_lib = None

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float

# name -> argtypes (all return int)
_SIGNATURES = {
    "mxs_nf4_dequant": [P, I64, P, P, P, P, P, P, I32, P],
    "mxs_nf4_dequant_bytewise": [P, I64, P, P, P, P, P, P, I32, P],
    "mxs_nf4_dequant_layer": [P, I64, P, P, P, P, P, P, I32, P, I64, P, P],
    "mxs_nf4_dequant_layer_plan": [P, I32, P, I64],
    "mxs_nf4_quantize_workspace_bytes": [I64],
    "mxs_nf4_quantize": [P, I64, P, P, P, P, P, P, P, P],
    "mxs_nf4_gemm_workspace_bytes": [I32, I32, I32, I32, I32],
    "mxs_nf4_linear_fwd": [P, I32, I32, I32, P, P, P, P, P, P, P, P, I32, P, P, I32, I32, P],
    "mxs_nf4_linear_fwd_noalloc": [P, I32, I32, I32, P, P, P, P, P, P, P, P, I32, P, I32, I32, P],
    "mxs_nf4_linear_bwd_dx": [P, I32, I32, I32, P, P, P, P, P, P, P, I32, P, F32, P, P, I32, I32,
                              P],
    "mxs_lora_workspace_bytes": [I32, I32, I32, I32],
    "mxs_lora_h": [P, I32, I32, P, I32, P, F32, F32, P, P, I32, P, P, I32, P, P, P],
    "mxs_lora_dh": [P, I32, I32, P, I32, F32, P, P, I32, P, P],
    "mxs_lora_grad_a": [P, I32, P, I32, I32, I32, P, F32, P, P, P],
    "mxs_lora_grad_b": [P, I32, P, I32, I32, I32, P, P, P],
    "mxs_lora_grads": [P, P, I32, P, P, I32, I32, I32, I32, P, F32, P, P, P, P],
    "mxs_keep_pack": [P, I32, I32, P, P],
    "mxs_nf4_linear_fwd_hp_pair": [P, I32, I32, P, P, P, P, P, P, P, P, I32, I32, P, I32, P, P,
                                   P],
    "mxs_nf4_linear_fwd_pair_ok": [I32, I32, I32, I32],
    "mxs_nf4_linear_bwd_dx_grads": [P, I32, I32, I32, P, P, P, P, P, P, P, I32, P, F32, P, P, I32,
                                    P, P, P, P, P, P],
    "mxs_nf4_linear_bwd_grads_fused": [I32, I32, I32, I32],
    "mxs_silu_mul": [P, P, P, I64, P],
    "mxs_nf4_linear_fwd_glu": [P, I32, I32, I32, P, P, P, P, P, P, P, I32, I32, P, I32, P, P, P,
                               P, P, P],
    "mxs_nf4_linear_bwd_dx_glu": [P, I32, I32, I32, P, P, P, P, P, P, I32, I32, P, I32, P, F32, P,
                                  P, P, P, P],
    "mxs_nf4_linear_glu_fused": [I32, I32, I32, I32],
    "mxs_nf4_linear_bwd_dx_grads_group_ok": [I32, I32, P, I32, I32],
    "mxs_nf4_linear_bwd_dx_grads_group": [I32, P, I32, P, I32, P, P, P, P, P, P, P, I32, P, F32, P,
                                          P, I32, P, P, P, P, P],
    "mxs_nf4_linear_bwd_dx_grads_sum_ok": [I32, I32, P, I32, I32, I32],
    "mxs_nf4_linear_bwd_dx_grads_sum": [I32, P, I32, P, I32, P, P, P, P, P, P, P, I32, P, F32, P, P,
                                        I32, P, P, P, P, P],
    "mxs_nf4_linear_fwd_hp_group": [I32, P, I32, I32, P, P, P, P, P, P, P, P, I32, I32, P, I32, P,
                                    P, P],
    "mxs_nf4_linear_fwd_hp_group_rope": [I32, P, I32, I32, P, P, P, P, P, P, P, P, I32, I32, P,
                                         I32, P, P, I32, P, P, I64, I64, I32, P],
    "mxs_qkv_rope": [P, P, P, P, I64, I64, I32, I32, I32, I32, I32, I32, I32, F32, F32, P],
    "mxs_silu_mul_bwd": [P, P, P, I64, P],
    "mxs_lora_slices": [I32, I32],
    "mxs_lora_h_partials": [P, I32, I32, P, I32, P, F32, F32, I32, P, P, I32, P, P, P],
    "mxs_lora_dh_partials": [P, I32, I32, P, I32, F32, I32, P, P],
    "mxs_lora_h_partials_group": [I32, P, I32, P, P, I32, P, F32, F32, I32, P, P, P, P, P, P],
    "mxs_lora_h_partials_group_w32": [I32, P, I32, P, P, I32, P, F32, F32, I32, P, P, P, P, P, P,
                                      P],
    "mxs_lora_dh_partials_group": [I32, P, I32, P, P, I32, F32, I32, P, P],
    "mxs_lora_dh_group": [I32, P, I32, P, P, I32, F32, I32, P, P, P],
    "mxs_lora_grads_group": [I32, P, P, I32, P, P, I32, P, P, I32, P, F32, P, P, P],
    "mxs_lora_finish": [P, I32, I32, I32, I32, P, P, P],
    "mxs_nf4_linear_fwd_hp": [P, I32, I32, I32, P, P, P, P, P, P, P, I32, I32, P, I32, P, P, P,
                              I32, I32, P],
    "mxs_nf4_linear_bwd_dx_hp": [P, I32, I32, I32, P, P, P, P, P, P, I32, I32, P, I32, P, F32, P,
                                 P, P, I32, I32, P],
    "mxs_transpose_f16": [P, I32, I32, P, P],
    "mxs_nf4_linear_bwd_dx_hp_pair": [P, I32, P, I32, P, P, P, P, P, P, I32, I32, P, I32, P, F32,
                                      P, P, P, P],
    "mxs_nf4_linear_bwd_dx_hp_pair_grads": [P, I32, P, I32, P, P, P, P, P, P, I32, I32, P, I32,
                                            P, F32, P, P, P, P, P, P, P, P],
    "mxs_nf4_linear_bwd_dx_pair_ok": [I32, I32, I32, I32],
    "mxs_nf4_linear_bwd_dx_pair_workspace_bytes": [I32, I32, I32, I32],
}


_RESTYPES = {"mxs_nf4_dequant_layer_plan": ctypes.c_int64,
             "mxs_nf4_gemm_workspace_bytes": ctypes.c_int64,
             "mxs_lora_workspace_bytes": ctypes.c_int64,
             "mxs_nf4_linear_bwd_dx_pair_workspace_bytes": ctypes.c_int64}


def lib():
    """The loaded library; raises MxsLibraryError when it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MxsLibraryError(
                f"{LIB_PATH} is not built: run `python -m mindxsoup_amd.build` (hipcc, gfx950)")
        try:
            L = ctypes.CDLL(LIB_PATH)
        except OSError as e:
            raise MxsLibraryError(f"cannot load {LIB_PATH}: {e}") from e
        for name, args in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = L
    return _lib


def exported_symbols():
    return list(_SIGNATURES)


PROBE_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmxs_probe.so")
_probe = None


def probe_lib():
    """libmxs_probe.so (include/mxs_probe.h): the HBM rate probes bench.py reports beside the
    dequant.  Measurement only; the NF4 path never loads it."""
    global _probe
    if _probe is None:
        if not os.path.exists(PROBE_PATH):
            raise MxsLibraryError(
                f"{PROBE_PATH} is not built: run `python -m mindxsoup_amd.build` (hipcc, gfx950)")
        L = ctypes.CDLL(PROBE_PATH)
        L.mxs_hbm_probe.argtypes = [I32, P, P, I64, P]
        L.mxs_hbm_probe.restype = ctypes.c_int
        _probe = L
    return _probe


def hbm_probe(kind, src, dst, n_chunks, stream):
    check(probe_lib().mxs_hbm_probe(kind, src, dst, n_chunks, stream), "mxs_hbm_probe")


def ptr(t):
    """Raw device pointer of a tensor, or None."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_of(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def check(rc, name):
    if rc != 0:
        why = _ERRORS.get(rc, f"hipError_t {rc}")
        raise RuntimeError(f"{name} failed: {why}")


def call(name, *args):
    check(getattr(lib(), name)(*args), name)
