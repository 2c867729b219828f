"""Tensor-level calls of the fused NF4 GEMM and LoRA kernels (C ABI in include/mxs_nf4.h).

Every function checks shapes, dtypes and devices, allocates its outputs (and the split-K
workspace) with torch's caching allocator, and launches on the current HIP stream.  Nothing here
computes on the CPU or falls back to another implementation: an unsupported shape raises.
"""

import torch

from . import _lib


def _c(t):
    return None if t is None else t.contiguous()


def _nf4_args(packed, state):
    return (_lib.ptr(packed), _lib.ptr(state.absmax), _lib.ptr(state.state2.code),
            _lib.ptr(state.state2.absmax), _lib.ptr(state.offset))


def fused_shape_ok(state, M=None):
    """Whether the fused GEMMs take this weight: in_features and out_features multiples of 64
    (NF4 blocks along rows, 64-wide reduction steps), nested NF4 at blocksize 64."""
    n, k = state.shape
    return (state.quant_type == "nf4" and state.blocksize == 64 and state.nested
            and state.state2 is not None and state.state2.blocksize == 256
            and k % 64 == 0 and n % 64 == 0)


def _ws(M, Nc, Kr, dev, cfg, splits):
    nbytes = _lib.lib().mxs_nf4_gemm_workspace_bytes(M, Nc, Kr, cfg, splits)
    if nbytes <= 0:
        return None
    return torch.empty(nbytes // 4, dtype=torch.float32, device=dev)


def nf4_linear_fwd(x2d, packed, state, bias=None, lora_h=None, lora_b=None, cfg=-1, splits=1):
    """Y = x2d @ W^T (+ bias) (+ lora_h @ lora_b^T), fp16 [M, N]; W decoded inside the GEMM."""
    n, k = state.shape
    if x2d.dtype != torch.float16 or x2d.dim() != 2 or x2d.shape[1] != k:
        raise ValueError("x must be fp16 [M, in_features]")
    x2d = x2d.contiguous()
    M = x2d.shape[0]
    y = torch.empty((M, n), dtype=torch.float16, device=x2d.device)
    r = 0
    if lora_h is not None:
        r = lora_h.shape[1]
        if lora_b is None or lora_b.shape != (n, r) or lora_h.shape[0] != M:
            raise ValueError("lora_h [M, r] needs lora_b [N, r]")
        lora_h, lora_b = lora_h.contiguous(), lora_b.contiguous()
    if bias is not None:
        bias = bias.to(torch.float16).contiguous()
    ws = _ws(M, n, k, x2d.device, cfg, splits)
    _lib.call("mxs_nf4_linear_fwd", _lib.ptr(x2d), M, k, n, *_nf4_args(packed, state),
              _lib.ptr(bias), _lib.ptr(lora_h), _lib.ptr(lora_b), r, _lib.ptr(y), _lib.ptr(ws),
              cfg, splits, _lib.stream_of(x2d.device))
    return y


def nf4_linear_bwd_dx(dy2d, packed, state, lora_dh=None, lora_a=None, mask=None,
                      mask_scale=1.0, cfg=-1, splits=1):
    """dX = dy2d @ W (+ mask * mask_scale * (lora_dh @ lora_a)), fp16 [M, K]."""
    n, k = state.shape
    if dy2d.dtype != torch.float16 or dy2d.dim() != 2 or dy2d.shape[1] != n:
        raise ValueError("dy must be fp16 [M, out_features]")
    dy2d = dy2d.contiguous()
    M = dy2d.shape[0]
    dx = torch.empty((M, k), dtype=torch.float16, device=dy2d.device)
    r = 0
    if lora_dh is not None:
        r = lora_dh.shape[1]
        if lora_a is None or lora_a.shape != (r, k) or lora_dh.shape[0] != M:
            raise ValueError("lora_dh [M, r] needs lora_a [r, K]")
        lora_dh, lora_a = lora_dh.contiguous(), lora_a.contiguous()
    if mask is not None:
        if mask.dtype != torch.uint8 or mask.shape != (M, k):
            raise ValueError("mask must be uint8 [M, K]")
        mask = mask.contiguous()
    ws = _ws(M, k, n, dy2d.device, cfg, splits)
    _lib.call("mxs_nf4_linear_bwd_dx", _lib.ptr(dy2d), M, n, k, *_nf4_args(packed, state),
              _lib.ptr(lora_dh), _lib.ptr(lora_a), r, _lib.ptr(mask), float(mask_scale),
              _lib.ptr(dx), _lib.ptr(ws), cfg, splits, _lib.stream_of(dy2d.device))
    return dx


def _ldt(M):
    return (M + 7) // 8 * 8


def lora_h(x2d, lora_a, s, mask=None, mask_scale=1.0):
    """(h, ht): h = fp16(s * drop(x) @ A^T) [M, r] and its transpose [r, ldt]."""
    x2d = x2d.contiguous()
    lora_a = lora_a.to(torch.float16).contiguous()
    M, K = x2d.shape
    r = lora_a.shape[0]
    h = torch.empty((M, r), dtype=torch.float16, device=x2d.device)
    ht = torch.empty((r, _ldt(M)), dtype=torch.float16, device=x2d.device)
    _lib.call("mxs_lora_h", _lib.ptr(x2d), M, K, _lib.ptr(lora_a), r, _lib.ptr(_c(mask)),
              float(mask_scale), float(s), _lib.ptr(h), _lib.ptr(ht), ht.shape[1],
              _lib.stream_of(x2d.device))
    return h, ht


def lora_dh(dy2d, lora_b, s):
    """(dh, dht): dh = fp16(s * dY @ B) [M, r] and its transpose [r, ldt]."""
    dy2d = dy2d.contiguous()
    lora_b = lora_b.to(torch.float16).contiguous()
    M, N = dy2d.shape
    r = lora_b.shape[1]
    dh = torch.empty((M, r), dtype=torch.float16, device=dy2d.device)
    dht = torch.empty((r, _ldt(M)), dtype=torch.float16, device=dy2d.device)
    _lib.call("mxs_lora_dh", _lib.ptr(dy2d), M, N, _lib.ptr(lora_b), r, float(s), _lib.ptr(dh),
              _lib.ptr(dht), dht.shape[1], _lib.stream_of(dy2d.device))
    return dh, dht


def lora_grad_a(dht, x2d, mask=None, mask_scale=1.0):
    """dA = dh^T @ drop(x), fp32 [r, K]."""
    x2d = x2d.contiguous()
    M, K = x2d.shape
    r = dht.shape[0]
    da = torch.empty((r, K), dtype=torch.float32, device=x2d.device)
    _lib.call("mxs_lora_grad_a", _lib.ptr(dht), dht.shape[1], _lib.ptr(x2d), M, K, r,
              _lib.ptr(_c(mask)), float(mask_scale), _lib.ptr(da), _lib.stream_of(x2d.device))
    return da


def lora_grad_b(ht, dy2d):
    """dB = dY^T @ h, fp32 [N, r] (h already carries the scaling s)."""
    dy2d = dy2d.contiguous()
    M, N = dy2d.shape
    r = ht.shape[0]
    db = torch.empty((N, r), dtype=torch.float32, device=dy2d.device)
    _lib.call("mxs_lora_grad_b", _lib.ptr(ht), ht.shape[1], _lib.ptr(dy2d), M, N, r,
              _lib.ptr(db), _lib.stream_of(dy2d.device))
    return db
