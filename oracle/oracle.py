"""CPU oracle for the NF4 quantized-linear hot path (TEST INFRASTRUCTURE ONLY).

Only tests/, the smoke check in __graft_entry__.py and the CPU-baseline leg of bench.py may
import this module, and only as the checker: the product (mindxsoup_amd) never imports it, and
fails loudly when its HIP library is missing instead of falling back to anything here.

Two layers:
  * liboracle_nf4.so (oracle/nf4_oracle.c): scalar C restatement of the reference's NF4 decode
    (solution/nf4.py:31-110) and of the bitsandbytes-style quantizer that makes test weights.
  * numpy references for the GEMMs around it: the dequant-then-matmul of NF4LinearFunction
    (solution/linear4bit.py:43-57) and peft's LoRA branch with the reference's dropout
    semantics (solution/dropout.py:18-37, solution/attention.py:193-201,
    solution/test_unpad.py:28-29), accumulated in float64 (a stricter bound than fp32).

Pinning: see the header of nf4_oracle.c for the decode; the GEMM/LoRA references here are
checked against float64 torch autograd and the merged-weight identity W + s*B*A in
tests/test_oracle.py.  Parity of the quantizer against bitsandbytes' own bit patterns is
unpinned (bitsandbytes is absent), and not needed: the path's contract starts at the packed
tensors.
"""

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle_nf4.so")

_lib = None


def build():
    """Compile liboracle_nf4.so with the committed Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.oracle_nf4_table.argtypes = [P]
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_dequant_nf4.argtypes = [P, i64, P, P, P, ctypes.c_float, P, ctypes.c_int,
                                         ctypes.c_int, P]
        L.oracle_dequant_nf4_f32.argtypes = L.oracle_dequant_nf4.argtypes
        L.oracle_dynamic_map.argtypes = [P]
        L.oracle_quantize_nf4.argtypes = [P, i64, P, P]
        L.oracle_absmax_mean.argtypes = [P, i64]
        L.oracle_absmax_mean.restype = ctypes.c_float
        L.oracle_quantize_absmax_256.argtypes = [P, i64, ctypes.c_float, P, P, P]
        L.oracle_num_threads.restype = ctypes.c_int
        L.oracle_set_num_threads.argtypes = [ctypes.c_int]
        L.oracle_silu_mul.argtypes = [P, P, P, i64]
        L.oracle_silu_mul_bwd.argtypes = [P, P, P, P, P, i64]
        L.oracle_qkv_rope.argtypes = [P, P, P, P, P, P, P, ctypes.c_int, P, P, P, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                      ctypes.c_float]
        _lib = L
    return _lib


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def nf4_table():
    out = np.zeros(16, np.float32)
    lib().oracle_nf4_table(_ptr(out))
    return out


def f32_to_f16_bits(x):
    """Scalar C conversion applied elementwise (slow; for pinning tests)."""
    L = lib()
    flat = np.asarray(x, np.float32).ravel()
    return np.array([L.oracle_f32_to_f16(float(v)) for v in flat], np.uint16).reshape(np.shape(x))


def num_threads():
    return lib().oracle_num_threads()


def set_num_threads(n):
    lib().oracle_set_num_threads(int(n))


@dataclass
class NF4Weight:
    """Packed NF4 weight with double-quantized absmax, in the field layout of bitsandbytes'
    QuantState as the reference reads it (solution/linear4bit.py:36-40): packed u8
    [(N*K)//2], absmax8 u8 [N*K/64], code f32 [256], absmax2 f32 [ceil(N*K/64/256)], offset."""
    shape: tuple
    packed: np.ndarray
    absmax8: np.ndarray
    code: np.ndarray
    absmax2: np.ndarray
    offset: float
    absmax_f32: np.ndarray = None  # first-level absmax before double quantization


def dynamic_map():
    out = np.zeros(256, np.float32)
    lib().oracle_dynamic_map(_ptr(out))
    return out


def quantize(w_f16):
    """NF4 + double-quant of an fp16 array (any shape with a multiple of 64 elements)."""
    w = np.ascontiguousarray(np.asarray(w_f16, np.float16)).view(np.uint16).ravel()
    n = w.size
    assert n % 64 == 0, "the oracle quantizer takes whole 64-value blocks"
    nb = n // 64
    packed = np.zeros(n // 2, np.uint8)
    absmax = np.zeros(nb, np.float32)
    L = lib()
    L.oracle_quantize_nf4(_ptr(w), n, _ptr(packed), _ptr(absmax))
    offset = float(L.oracle_absmax_mean(_ptr(absmax), nb))
    code = dynamic_map()
    ng = (nb + 255) // 256
    q8 = np.zeros(nb, np.uint8)
    absmax2 = np.zeros(ng, np.float32)
    L.oracle_quantize_absmax_256(_ptr(absmax), nb, ctypes.c_float(offset), _ptr(code), _ptr(q8),
                                 _ptr(absmax2))
    return NF4Weight(tuple(np.shape(w_f16)), packed, q8, code, absmax2, offset, absmax)


def quantize_absmax_256(absmax, offset, code):
    """Second-level quantization for a given offset (lets tests take the GPU's offset)."""
    absmax = np.ascontiguousarray(absmax, np.float32)
    nb = absmax.size
    q8 = np.zeros(nb, np.uint8)
    absmax2 = np.zeros((nb + 255) // 256, np.float32)
    lib().oracle_quantize_absmax_256(_ptr(absmax), nb, ctypes.c_float(offset),
                                     _ptr(np.ascontiguousarray(code, np.float32)), _ptr(q8),
                                     _ptr(absmax2))
    return q8, absmax2


def absmax_mean(absmax):
    absmax = np.ascontiguousarray(absmax, np.float32)
    return float(lib().oracle_absmax_mean(_ptr(absmax), absmax.size))


def quantize_blocks_nf4(w_f16):
    """First level only: (packed, absmax f32)."""
    w = np.ascontiguousarray(np.asarray(w_f16, np.float16)).view(np.uint16).ravel()
    packed = np.zeros(w.size // 2, np.uint8)
    absmax = np.zeros(w.size // 64, np.float32)
    lib().oracle_quantize_nf4(_ptr(w), w.size, _ptr(packed), _ptr(absmax))
    return packed, absmax


def dequant(wt: NF4Weight = None, *, packed=None, absmax8=None, code=None, absmax2=None,
            offset=0.0, absmax_f32=None, shape=None, fused=True, out_dtype=np.float16):
    """Decoded weight (fp16 array, or fp32 with out_dtype=np.float32).  Either an NF4Weight or
    the raw fields; absmax_f32 without absmax8 selects the non-nested form."""
    if wt is not None:
        packed, absmax8, code, absmax2, offset, shape = (wt.packed, wt.absmax8, wt.code,
                                                          wt.absmax2, wt.offset, wt.shape)
    packed = np.ascontiguousarray(packed, np.uint8).ravel()
    nested = absmax8 is not None
    n_bytes = packed.size
    if shape is None:
        shape = (2 * n_bytes,)
    args = [_ptr(packed), n_bytes,
            _ptr(np.ascontiguousarray(absmax8, np.uint8)) if nested else None,
            _ptr(np.ascontiguousarray(code, np.float32)) if nested else None,
            _ptr(np.ascontiguousarray(absmax2, np.float32)) if nested else None,
            ctypes.c_float(offset if nested else 0.0),
            None if nested else _ptr(np.ascontiguousarray(absmax_f32, np.float32)),
            int(nested), int(fused)]
    if out_dtype == np.float32:
        out = np.zeros(2 * n_bytes, np.float32)
        lib().oracle_dequant_nf4_f32(*args, _ptr(out))
        return out.reshape(shape)
    out = np.zeros(2 * n_bytes, np.uint16)
    lib().oracle_dequant_nf4(*args, _ptr(out))
    return out.view(np.float16).reshape(shape)


# ---------------------------------------------------------------------------------------------
# GEMM / LoRA references (float64 accumulation over the exact fp16 operands)
# ---------------------------------------------------------------------------------------------

def dropout_fp16(x_f16, keep_u8, p):
    """solution/dropout.py:33-35: keep ? fp16(fp32(x) * fp32(1/(1-p))) : 0.  Pinned in
    tests/test_oracle.py by closed forms (p = 0.5, 0.75 give exactly 2x, 4x; dropped elements
    +0.0) and by exact rational arithmetic over every finite fp16 value at p = 0.05."""
    x = np.asarray(x_f16, np.float16)
    if keep_u8 is None:
        return x
    scale = np.float32(1.0 / (1.0 - p))
    with np.errstate(over="ignore"):  # products past fp16's range become ±inf, as in the kernel
        kept = (x.astype(np.float32) * scale).astype(np.float16)
    return np.where(keep_u8 != 0, kept, np.float16(0))


def linear_fwd(x_f16, w_f16, bias=None):
    """NF4LinearFunction.forward (solution/linear4bit.py:47-49): x @ W^T + bias (float64)."""
    y = x_f16.astype(np.float64) @ w_f16.astype(np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


def linear_bwd_dx(dy_f16, w_f16):
    """NF4LinearFunction.backward (solution/linear4bit.py:51-57): grad @ W (float64)."""
    return dy_f16.astype(np.float64) @ w_f16.astype(np.float64)


def lora_h(x_f16, a_f16, keep_u8=None, p=0.0):
    """H = drop(x) @ A^T, lora_A of peft's branch (float64 of the fp16 dropped input)."""
    xd = dropout_fp16(x_f16, keep_u8, p).astype(np.float64)
    return xd @ np.asarray(a_f16, np.float64).T


def lora_fwd(x_f16, w_f16, a_f16, b_f16, s, keep_u8=None, p=0.0, bias=None):
    """peft Linear4bit with one adapter: base(x) + s * B(A(drop(x))) (solution/test_unpad.py:28-29,
    solution/attention.py:197-199), float64 over the fp16 operands."""
    h = lora_h(x_f16, a_f16, keep_u8, p)
    return linear_fwd(x_f16, w_f16, bias) + s * (h @ np.asarray(b_f16, np.float64).T)


def lora_bwd(dy_f16, x_f16, w_f16, a_f16, b_f16, s, keep_u8=None, p=0.0):
    """Gradients of lora_fwd: (dX, dA, dB), float64.
    dH = s * dY @ B; dX = dY @ W + drop'(dH @ A); dA = dH^T @ drop(x); dB = s * dY^T @ H."""
    dy = dy_f16.astype(np.float64)
    a = np.asarray(a_f16, np.float64)
    b = np.asarray(b_f16, np.float64)
    h = lora_h(x_f16, a_f16, keep_u8, p)
    xd = dropout_fp16(x_f16, keep_u8, p).astype(np.float64)
    dh = s * (dy @ b)
    g = dh @ a
    if keep_u8 is not None:
        g = np.where(keep_u8 != 0, g * float(np.float32(1.0 / (1.0 - p))), 0.0)
    dx = linear_bwd_dx(dy_f16, w_f16) + g
    da = dh.T @ xd
    db = s * (dy.T @ h)
    return dx, da, db


def max_rel(got, ref):
    """max|got - ref| / max|ref| (the measure of solution/test_attention.py:91-92)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-12))


def silu_mul(gate_f16, up_f16):
    """fp16 silu(gate) * up with the kernel's fp32 arithmetic (solution/silu_mul.py:26-44)."""
    g = np.ascontiguousarray(gate_f16, dtype=np.float16)
    u = np.ascontiguousarray(up_f16, dtype=np.float16)
    out = np.empty_like(g)
    lib().oracle_silu_mul(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out


def silu_mul_bwd(dh_f16, gate_f16, up_f16):
    """(d_gate, d_up) in fp16 for the incoming fp16 gradient dh (solution/silu_mul.py:35-41)."""
    d = np.ascontiguousarray(dh_f16, dtype=np.float16)
    g = np.ascontiguousarray(gate_f16, dtype=np.float16)
    u = np.ascontiguousarray(up_f16, dtype=np.float16)
    dg, du = np.empty_like(g), np.empty_like(g)
    lib().oracle_silu_mul_bwd(_ptr(d), _ptr(g), _ptr(u), _ptr(dg), _ptr(du), g.size)
    return dg, du


def qkv_rope(q_a, q_b, k, v_a, v_b, cos, sin, n_q, n_kv, q_scale=1.0, v_scale=1.0,
             backward=False, out_dtype=np.float16):
    """(q, k, v) of solution/attention.py:28-82 (qkv_rope_kernel) on [B, T, heads * 128] arrays
    (fp16 or fp32, all one dtype; q_b, v_a, v_b may be None), cos / sin [1 or B, T, 128]; the
    outputs are [B, T, heads * 128] of out_dtype (v None without v_a).  backward=True rotates
    back (the kernel's backward launch, attention.py:156-167)."""
    dt = np.asarray(q_a).dtype
    if dt not in (np.float16, np.float32):
        raise ValueError("fp16 or fp32 inputs")
    conv = [None if t is None else np.ascontiguousarray(t, dtype=dt) for t in (q_a, q_b, k, v_a, v_b)]
    q_a_, q_b_, k_, v_a_, v_b_ = conv
    batch, n_tokens, _ = q_a_.shape
    c = np.ascontiguousarray(cos, dtype=np.float32)
    s_ = np.ascontiguousarray(sin, dtype=np.float32)
    if c.shape != s_.shape or c.shape[1:] != (n_tokens, 128) or c.shape[0] not in (1, batch):
        raise ValueError("cos / sin must be [1 or B, T, 128]")
    q_o = np.empty((batch, n_tokens, n_q * 128), out_dtype)
    k_o = np.empty((batch, n_tokens, n_kv * 128), out_dtype)
    v_o = None if v_a_ is None else np.empty((batch, n_tokens, n_kv * 128), out_dtype)
    lib().oracle_qkv_rope(_ptr(q_a_), _ptr(q_b_) if q_b_ is not None else None, _ptr(k_),
                          _ptr(v_a_) if v_a_ is not None else None,
                          _ptr(v_b_) if v_b_ is not None else None, _ptr(c), _ptr(s_),
                          c.shape[0], _ptr(q_o), _ptr(k_o),
                          _ptr(v_o) if v_o is not None else None, batch, n_tokens, n_q, n_kv,
                          int(dt == np.float32), int(np.dtype(out_dtype) == np.float32),
                          int(backward), float(q_scale), float(v_scale))
    return q_o, k_o, v_o
