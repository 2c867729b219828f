"""Tensor-level calls of the fused NF4 GEMM and LoRA kernels (C ABI in include/mxs_nf4.h).

Every function checks shapes, dtypes and devices, allocates its outputs with torch's caching
allocator, and launches on the current HIP stream.  Nothing here computes on the CPU or falls
back to another implementation: an unsupported shape raises.

Workspaces: the split-K GEMMs write fp32 partial sums to a workspace that a second small kernel
adds up in a fixed order; its contents need no initialisation and are dead after the call, so
one buffer serves any number of calls issued in order on one stream.  Calls take it as `ws` or
allocate it from torch's caching allocator.  The LoRA H / dH kernels use one the same way for
reductions of 1024 or more (split over workgroups); the dA / dB kernel needs none.
"""

import torch

from . import _lib


def new_workspace(nbytes, device):
    """A workspace of at least nbytes (u8 tensor; contents undefined)."""
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


def _workspace(nbytes, device, ws):
    if nbytes <= 0:
        return None
    if ws is None:
        return new_workspace(nbytes, device)
    if ws.numel() * ws.element_size() < nbytes:
        raise ValueError(f"workspace holds {ws.numel() * ws.element_size()} bytes, "
                         f"needs {nbytes}")
    return ws


def _c(t):
    return None if t is None else t.contiguous()


def keep_words(K):
    """32-bit words per row of a keep-bits mask over K columns."""
    return (K + 31) // 32


def keep_bits(mask, M, K):
    """The dropout keep mask as every kernel takes it: bits, int32 [M, ceil(K/32)], bit k % 32 of
    word k / 32 of row m set where element (m, k) is kept.  A byte mask [M, K] (uint8, int8 or
    bool; nonzero = kept, the reference's int8 `keep`, solution/dropout.py:64) is packed by one
    launch (mxs_keep_pack); a mask already in bits passes through; None stays None."""
    if mask is None:
        return None
    kw = keep_words(K)
    if mask.dtype == torch.int32 and tuple(mask.shape) == (M, kw):
        return mask.contiguous()
    if mask.dtype in (torch.uint8, torch.int8, torch.bool) and tuple(mask.shape) == (M, K):
        src = mask.contiguous().view(torch.uint8)
        bits = torch.empty((M, kw), dtype=torch.int32, device=mask.device)
        _lib.call("mxs_keep_pack", _lib.ptr(src), M, K, _lib.ptr(bits), _lib.stream_of(mask.device))
        return bits
    raise ValueError(f"mask must be a uint8 [{M}, {K}] keep mask or int32 [{M}, {kw}] keep bits, "
                     f"got {mask.dtype} {tuple(mask.shape)}")


def check_nf4_operands(packed, state, device=None):
    """Raise ValueError unless the NF4 operands the kernels read through raw pointers hold what
    state.shape [N, K] says: packed contiguous uint8 with N*K/2 bytes, absmax contiguous uint8
    with N*K/64 entries, state2.absmax contiguous fp32 with ceil(N*K/64/256) entries, the code
    book fp32 [256], offset fp32, all on `device` (default: packed's).  An offloaded weight's
    placeholder (a stride-0 expand of one byte, stream.offload) fails the contiguity test."""
    n, k = (int(d) for d in state.shape)
    blocks = n * k // 64
    device = packed.device if device is None else device
    if packed.dtype != torch.uint8 or not packed.is_contiguous() or 2 * packed.numel() != n * k:
        raise ValueError(f"packed must be contiguous uint8 with {n * k // 2} bytes for "
                         f"[{n}, {k}]")
    absmax = state.absmax
    if absmax.dtype != torch.uint8 or not absmax.is_contiguous() or absmax.numel() != blocks:
        raise ValueError(f"quant_state.absmax must be contiguous uint8 [{blocks}]")
    s2 = state.state2
    if s2 is None:
        raise ValueError("the fused kernels need a nested (double-quantized) absmax")
    a2, code, off = s2.absmax, s2.code, state.offset
    if a2.dtype != torch.float32 or not a2.is_contiguous() or \
            a2.numel() != (blocks + 255) // 256:
        raise ValueError(f"state2.absmax must be contiguous fp32 [{(blocks + 255) // 256}]")
    if code.dtype != torch.float32 or not code.is_contiguous() or code.numel() != 256:
        raise ValueError("state2.code must be contiguous fp32 [256]")
    if off is None or off.dtype != torch.float32 or off.numel() < 1:
        raise ValueError("quant_state.offset must be an fp32 tensor")
    for t in (packed, absmax, a2, code, off):
        if t.device != device:
            raise ValueError(f"NF4 operands must be on {device}, found {t.device}")


def _nf4_args(packed, state, device=None):
    check_nf4_operands(packed, state, device)
    return (_lib.ptr(packed), _lib.ptr(state.absmax), _lib.ptr(state.state2.code),
            _lib.ptr(state.state2.absmax), _lib.ptr(state.offset))


def fused_shape_ok(state, M=None):
    """Whether the fused GEMMs take this weight: in_features and out_features multiples of 64
    (NF4 blocks along rows, 64-wide reduction steps), nested NF4 at blocksize 64."""
    n, k = state.shape
    return (state.quant_type == "nf4" and state.blocksize == 64 and state.nested
            and state.state2 is not None and state.state2.blocksize == 256
            and k % 64 == 0 and n % 64 == 0)


def gemm_workspace_bytes(M, Nc, Kr, cfg=-1, splits=1):
    return int(_lib.lib().mxs_nf4_gemm_workspace_bytes(M, Nc, Kr, cfg, splits))


def lora_workspace_bytes(M, K, N, r):
    return int(_lib.lib().mxs_lora_workspace_bytes(M, K, N, r))


def projection_workspace_bytes(M, K, N, r=16):
    """Bytes one workspace needs for every call of a K -> N projection at M tokens."""
    return max(gemm_workspace_bytes(M, N, K), gemm_workspace_bytes(M, K, N),
               lora_workspace_bytes(M, K, N, r) if r else 0)


def _ws(M, Nc, Kr, dev, cfg, splits, ws=None):
    return _workspace(gemm_workspace_bytes(M, Nc, Kr, cfg, splits), dev, ws)


def nf4_linear_fwd(x2d, packed, state, bias=None, lora_h=None, lora_b=None, cfg=-1, splits=1,
                   ws=None):
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
    ws = _ws(M, n, k, x2d.device, cfg, splits, ws)
    _lib.call("mxs_nf4_linear_fwd", _lib.ptr(x2d), M, k, n, *_nf4_args(packed, state),
              _lib.ptr(bias), _lib.ptr(lora_h), _lib.ptr(lora_b), r, _lib.ptr(y), _lib.ptr(ws),
              cfg, splits, _lib.stream_of(x2d.device))
    return y


def nf4_linear_fwd_noalloc(x2d, packed, state, y, bias=None, lora_h=None, lora_b=None, cfg=-1,
                           splits=1):
    """nf4_linear_fwd into the caller's y [M, N] fp16 through mxs_nf4_linear_fwd_noalloc: the
    split-K partials live in the library's own device array (MXS_NF4_SCRATCH_BYTES), so the call
    allocates nothing.  Calls overlapping in time on one GPU share that array and race."""
    n, k = state.shape
    if x2d.dtype != torch.float16 or x2d.dim() != 2 or x2d.shape[1] != k or \
            not x2d.is_contiguous():
        raise ValueError("x must be contiguous fp16 [M, in_features]")
    M = x2d.shape[0]
    if y.dtype != torch.float16 or tuple(y.shape) != (M, n) or not y.is_contiguous() or \
            y.device != x2d.device:
        raise ValueError("y must be contiguous fp16 [M, out_features] on x's device")
    r = 0
    if lora_h is not None:
        r = lora_h.shape[1]
        if lora_b is None or tuple(lora_b.shape) != (n, r) or lora_h.shape[0] != M or \
                not (lora_h.is_contiguous() and lora_b.is_contiguous()):
            raise ValueError("lora_h [M, r] needs lora_b [N, r], both contiguous fp16")
    if bias is not None and (bias.dtype != torch.float16 or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous fp16")
    _lib.call("mxs_nf4_linear_fwd_noalloc", _lib.ptr(x2d), M, k, n,
              *_nf4_args(packed, state, x2d.device), _lib.ptr(bias), _lib.ptr(lora_h),
              _lib.ptr(lora_b), r, _lib.ptr(y), cfg, splits, _lib.stream_of(x2d.device))
    return y


def nf4_linear_bwd_dx(dy2d, packed, state, lora_dh=None, lora_a=None, mask=None,
                      mask_scale=1.0, cfg=-1, splits=1, lora_at=None, ws=None):
    """dX = dy2d @ W (+ mask * mask_scale * (lora_dh @ lora_a)), fp16 [M, K].  The kernel takes
    lora_A transposed ([K, r]); pass it as lora_at to skip the transpose."""
    n, k = state.shape
    if dy2d.dtype != torch.float16 or dy2d.dim() != 2 or dy2d.shape[1] != n:
        raise ValueError("dy must be fp16 [M, out_features]")
    dy2d = dy2d.contiguous()
    M = dy2d.shape[0]
    dx = torch.empty((M, k), dtype=torch.float16, device=dy2d.device)
    r = 0
    if lora_dh is not None:
        r = lora_dh.shape[1]
        if lora_at is None:
            if lora_a is None or lora_a.shape != (r, k):
                raise ValueError("lora_dh [M, r] needs lora_a [r, K]")
            lora_at = transpose(lora_a.to(torch.float16))
        if lora_at.shape != (k, r) or lora_dh.shape[0] != M:
            raise ValueError("lora_dh [M, r] needs lora_at [K, r]")
        lora_dh, lora_at = lora_dh.contiguous(), lora_at.contiguous()
    mask = keep_bits(mask, M, k)
    ws = _ws(M, k, n, dy2d.device, cfg, splits, ws)
    _lib.call("mxs_nf4_linear_bwd_dx", _lib.ptr(dy2d), M, n, k, *_nf4_args(packed, state),
              _lib.ptr(lora_dh), _lib.ptr(lora_at), r, _lib.ptr(mask), float(mask_scale),
              _lib.ptr(dx), _lib.ptr(ws), cfg, splits, _lib.stream_of(dy2d.device))
    return dx


def bwd_grads_fused(M, N, K, r):
    """True when nf4_linear_bwd_dx_grads computes dX and both LoRA gradients in one launch for a
    projection K -> N at M tokens (decided by the library's tile plan and the device's CUs)."""
    return bool(_lib.lib().mxs_nf4_linear_bwd_grads_fused(M, N, K, r))


def nf4_linear_bwd_dx_grads(dy2d, packed, state, lora_dh, lora_at, dht, ht, x2d, mask=None,
                            mask_scale=1.0, ws=None):
    """(dx, dA, dB): dX = dy2d @ W + mask * mask_scale * (lora_dh @ lora_at^T) fp16 [M, K],
    dA = dht @ drop(x2d) fp32 [r, K] and dB = dy2d^T @ ht^T fp32 [N, r] -- one launch where
    bwd_grads_fused says so.  lora_dh [M, r] and dht [r, ldt] come from one lora_dh call without
    a workspace; ht is the forward's Hs^T."""
    n, k = state.shape
    if dy2d.dtype != torch.float16 or dy2d.dim() != 2 or dy2d.shape[1] != n:
        raise ValueError("dy must be fp16 [M, out_features]")
    dy2d, x2d = dy2d.contiguous(), x2d.contiguous()
    M = dy2d.shape[0]
    r = lora_dh.shape[1]
    if x2d.shape != (M, k) or lora_dh.shape[0] != M or lora_at.shape != (k, r):
        raise ValueError("x [M, K], lora_dh [M, r] and lora_at [K, r] disagree")
    if dht.shape[0] != r or ht.shape != dht.shape or dht.shape[1] < M:
        raise ValueError("dht and ht must be [r, ldt] with ldt >= M")
    mask = keep_bits(mask, M, k)
    dev = dy2d.device
    dx = torch.empty((M, k), dtype=torch.float16, device=dev)
    da = torch.empty((r, k), dtype=torch.float32, device=dev)
    db = torch.empty((n, r), dtype=torch.float32, device=dev)
    ws = _ws(M, k, n, dev, -1, 1, ws)
    _lib.call("mxs_nf4_linear_bwd_dx_grads", _lib.ptr(dy2d), M, n, k, *_nf4_args(packed, state),
              _lib.ptr(lora_dh.contiguous()), _lib.ptr(lora_at.contiguous()), r, _lib.ptr(mask),
              float(mask_scale), _lib.ptr(dht.contiguous()), _lib.ptr(ht.contiguous()),
              dht.shape[1], _lib.ptr(x2d), _lib.ptr(da), _lib.ptr(db), _lib.ptr(dx),
              _lib.ptr(ws), _lib.stream_of(dev))
    return dx, da, db


def bwd_grads_group_ok(M, Ns, K, r):
    """True when nf4_linear_bwd_dx_grads_group takes projections [K -> N] for N in Ns."""
    return bool(_lib.lib().mxs_nf4_linear_bwd_dx_grads_group_ok(len(Ns), M, _int_array(Ns), K,
                                                               r))


def nf4_linear_bwd_dx_grads_group(dys, packeds, states, dhs, ats, dhts, hts, x2ds, masks=None,
                                  mask_scale=1.0):
    """nf4_linear_bwd_dx_grads for up to 4 projections of one input width in one launch: a list
    of (dx, dA, dB), the bits of the separate calls.  Only where bwd_grads_group_ok."""
    n = len(dys)
    masks = masks or [None] * n
    dys = [d.contiguous() for d in dys]
    x2ds = [x.contiguous() for x in x2ds]
    M, K = x2ds[0].shape
    r = dhs[0].shape[1]
    Ns = [st.shape[0] for st in states]
    for d, x, st, dh, at, dht, ht in zip(dys, x2ds, states, dhs, ats, dhts, hts):
        if d.shape != (M, st.shape[0]) or x.shape != (M, K) or st.shape[1] != K:
            raise ValueError("dy [M, N], x [M, K] and the weight [N, K] disagree")
        if dh.shape != (M, r) or at.shape != (K, r) or dht.shape[0] != r or ht.shape != dht.shape:
            raise ValueError("LoRA operands disagree")
    dev = dys[0].device
    for pk, st in zip(packeds, states):
        check_nf4_operands(pk, st, dev)
    dx = [torch.empty((M, K), dtype=torch.float16, device=dev) for _ in dys]
    da = [torch.empty((r, K), dtype=torch.float32, device=dev) for _ in dys]
    db = [torch.empty((nn_, r), dtype=torch.float32, device=dev) for nn_ in Ns]
    masks = [keep_bits(m, M, K) for m in masks]
    _lib.call("mxs_nf4_linear_bwd_dx_grads_group", n, _ptr_array(dys), M, _int_array(Ns), K,
              _ptr_array(packeds), _ptr_array([st.absmax for st in states]),
              _ptr_array([st.state2.code for st in states]),
              _ptr_array([st.state2.absmax for st in states]),
              _ptr_array([st.offset for st in states]), _ptr_array([_c(t) for t in dhs]),
              _ptr_array([_c(t) for t in ats]), r, _ptr_array(masks), float(mask_scale),
              _ptr_array([_c(t) for t in dhts]), _ptr_array([_c(t) for t in hts]),
              dhts[0].shape[1], _ptr_array(x2ds), _ptr_array(da), _ptr_array(db),
              _ptr_array(dx), _lib.stream_of(dev))
    return list(zip(dx, da, db))


def bwd_grads_sum_ok(M, Ns, K, r, grads=True):
    """True when nf4_linear_bwd_dx_grads_sum takes projections [K -> N] for N in Ns (with their
    LoRA gradients in the same launch, or, grads=False, the summed dX alone)."""
    return bool(_lib.lib().mxs_nf4_linear_bwd_dx_grads_sum_ok(len(Ns), M, _int_array(Ns), K, r,
                                                             int(bool(grads))))


def nf4_linear_bwd_dx_grads_sum(dys, packeds, states, dhs, ats, dhts, hts, x2d, masks=None,
                                mask_scale=1.0, grads=True):
    """The backward of 2..3 projections over one input x2d in one launch: (dx, [(dA, dB), ..]),
    dx = the sum of their input gradients (one fp32 accumulator, rounded once), dA / dB the bits
    of nf4_linear_bwd_dx_grads (grads=False: (dx, None), the summed dX alone).  Only where
    bwd_grads_sum_ok(..., grads); every projection has a keep mask or none does."""
    n = len(dys)
    masks = masks or [None] * n
    if any(m is None for m in masks) and any(m is not None for m in masks):
        raise ValueError("every projection has a keep mask, or none does")
    dys = [d.contiguous() for d in dys]
    x2d = x2d.contiguous()
    M, K = x2d.shape
    r = dhs[0].shape[1]
    Ns = [st.shape[0] for st in states]
    for d, st, dh, at, dht, ht in zip(dys, states, dhs, ats, dhts, hts):
        if d.shape != (M, st.shape[0]) or st.shape[1] != K:
            raise ValueError("dy [M, N], x [M, K] and the weight [N, K] disagree")
        if dh.shape != (M, r) or at.shape != (K, r) or dht.shape[0] != r or ht.shape != dht.shape:
            raise ValueError("LoRA operands disagree")
    dev = x2d.device
    for pk, st in zip(packeds, states):
        check_nf4_operands(pk, st, dev)
    dx = torch.empty((M, K), dtype=torch.float16, device=dev)
    da = [torch.empty((r, K), dtype=torch.float32, device=dev) for _ in dys] if grads else None
    db = [torch.empty((nn_, r), dtype=torch.float32, device=dev) for nn_ in Ns] if grads else None
    masks = [keep_bits(m, M, K) for m in masks]
    _lib.call("mxs_nf4_linear_bwd_dx_grads_sum", n, _ptr_array(dys), M, _int_array(Ns), K,
              _ptr_array(packeds), _ptr_array([st.absmax for st in states]),
              _ptr_array([st.state2.code for st in states]),
              _ptr_array([st.state2.absmax for st in states]),
              _ptr_array([st.offset for st in states]), _ptr_array([_c(t) for t in dhs]),
              _ptr_array([_c(t) for t in ats]), r, _ptr_array(masks), float(mask_scale),
              _ptr_array([_c(t) for t in dhts]), _ptr_array([_c(t) for t in hts]),
              dhts[0].shape[1], _lib.ptr(x2d), _ptr_array(da) if grads else None,
              _ptr_array(db) if grads else None, _lib.ptr(dx), _lib.stream_of(dev))
    return dx, list(zip(da, db)) if grads else None


def lora_slices(M, Kr):
    """Reduction slices the partial-sum LoRA kernels use (1..4)."""
    return int(_lib.lib().mxs_lora_slices(M, Kr))


def lora_h_partials(x2d, lora_a, s, mask=None, mask_scale=1.0, lora_b=None):
    """(hp, at, bt): s * drop(x) @ A^T as fp32 partial sums [slices, ldt, r] (the fused forward
    GEMM finishes them), lora_A^T [K, r] and, given lora_b [N, r], lora_B^T [r, N]."""
    x2d = x2d.contiguous()
    lora_a = lora_a.to(torch.float16).contiguous()
    M, K = x2d.shape
    r = lora_a.shape[0]
    dev = x2d.device
    hp = torch.empty((lora_slices(M, K), _ldt(M), r), dtype=torch.float32, device=dev)
    at = torch.empty((K, r), dtype=torch.float16, device=dev)
    bt, N = None, 0
    if lora_b is not None:
        lora_b = lora_b.to(torch.float16).contiguous()
        N = lora_b.shape[0]
        if lora_b.shape != (N, r):
            raise ValueError("lora_b must be [N, r]")
        bt = torch.empty((r, N), dtype=torch.float16, device=dev)
    _lib.call("mxs_lora_h_partials", _lib.ptr(x2d), M, K, _lib.ptr(lora_a), r,
              _lib.ptr(keep_bits(mask, M, K)),
              float(mask_scale), float(s), hp.shape[1], _lib.ptr(at), _lib.ptr(lora_b), N,
              _lib.ptr(bt), _lib.ptr(hp), _lib.stream_of(dev))
    return hp, at, bt


def lora_dh_partials(dy2d, lora_bt, s):
    """s * dY @ B as fp32 partial sums [slices, ldt, r] (the fused dX GEMM finishes them);
    lora_bt = lora_B^T [r, N]."""
    dy2d = dy2d.contiguous()
    M, N = dy2d.shape
    r = lora_bt.shape[0]
    if lora_bt.shape != (r, N):
        raise ValueError("lora_bt must be [r, N]")
    dhp = torch.empty((lora_slices(M, N), _ldt(M), r), dtype=torch.float32, device=dy2d.device)
    _lib.call("mxs_lora_dh_partials", _lib.ptr(dy2d), M, N, _lib.ptr(lora_bt.contiguous()), r,
              float(s), dhp.shape[1], _lib.ptr(dhp), _lib.stream_of(dy2d.device))
    return dhp


def _ptr_array(ts):
    import ctypes

    return (ctypes.c_void_p * len(ts))(*[None if t is None else t.data_ptr() for t in ts])


def _int_array(vals):
    import ctypes

    return (ctypes.c_int * len(vals))(*vals)


def lora_h_partials_group(xs, lora_as, s, masks=None, mask_scale=1.0, lora_bs=None):
    """lora_h_partials for up to 4 projections over the same tokens in one launch: a list of
    (hp, at, bt) as lora_h_partials returns them, the same bits.  xs may repeat one tensor (the
    q/k/v or gate/up projections share their input)."""
    n = len(xs)
    masks = masks or [None] * n
    lora_bs = lora_bs or [None] * n
    xs = [x.contiguous() for x in xs]
    M = xs[0].shape[0]
    if any(x.shape[0] != M for x in xs) or not 1 <= n <= 4:
        raise ValueError("1..4 problems over the same number of tokens")
    a16 = [a.to(torch.float16).contiguous() for a in lora_as]
    r = a16[0].shape[0]
    dev = xs[0].device
    outs, bts, b16 = [], [], []
    for x, a, b in zip(xs, a16, lora_bs):
        K = x.shape[1]
        if a.shape != (r, K):
            raise ValueError("lora_a must be [r, K] with one r")
        hp = torch.empty((lora_slices(M, K), _ldt(M), r), dtype=torch.float32, device=dev)
        at = torch.empty((K, r), dtype=torch.float16, device=dev)
        bt = None
        if b is not None:
            b = b.to(torch.float16).contiguous()
            if b.shape[1] != r:
                raise ValueError("lora_b must be [N, r]")
            bt = torch.empty((r, b.shape[0]), dtype=torch.float16, device=dev)
        outs.append((hp, at, bt))
        bts.append(bt)
        b16.append(b)
    masks = [keep_bits(m, M, x.shape[1]) for m, x in zip(masks, xs)]
    _lib.call("mxs_lora_h_partials_group", n, _ptr_array(xs), M,
              _int_array([x.shape[1] for x in xs]), _ptr_array(a16), r, _ptr_array(masks),
              float(mask_scale), float(s), _ldt(M), _ptr_array([o[1] for o in outs]),
              _ptr_array(b16), _int_array([0 if b is None else b.shape[0] for b in b16]),
              _ptr_array(bts), _ptr_array([o[0] for o in outs]), _lib.stream_of(dev))
    return outs


def lora_dh_partials_group(dys, lora_bts, s):
    """lora_dh_partials for up to 4 projections in one launch: a list of partials, the same bits
    as separate calls."""
    n = len(dys)
    dys = [d.contiguous() for d in dys]
    M = dys[0].shape[0]
    if any(d.shape[0] != M for d in dys) or not 1 <= n <= 4 or len(lora_bts) != n:
        raise ValueError("1..4 problems over the same number of tokens")
    bts = [b.contiguous() for b in lora_bts]
    r = bts[0].shape[0]
    for d, b in zip(dys, bts):
        if b.shape != (r, d.shape[1]):
            raise ValueError("lora_bt must be [r, N] with one r")
    dev = dys[0].device
    outs = [torch.empty((lora_slices(M, d.shape[1]), _ldt(M), r), dtype=torch.float32,
                        device=dev) for d in dys]
    _lib.call("mxs_lora_dh_partials_group", n, _ptr_array(dys), M,
              _int_array([d.shape[1] for d in dys]), _ptr_array(bts), r, float(s), _ldt(M),
              _ptr_array(outs), _lib.stream_of(dev))
    return outs


def lora_dh_group(dys, lora_bts, s):
    """lora_dh(dy, None, s, lora_bt=bt, one_launch=True) for up to 4 projections in one launch:
    a list of (dh [M, r], dht [r, ldt]), the same bits as separate calls."""
    n = len(dys)
    dys = [d.contiguous() for d in dys]
    M = dys[0].shape[0]
    if any(d.shape[0] != M for d in dys) or not 1 <= n <= 4 or len(lora_bts) != n:
        raise ValueError("1..4 problems over the same number of tokens")
    bts = [b.contiguous() for b in lora_bts]
    r = bts[0].shape[0]
    for d, b in zip(dys, bts):
        if b.shape != (r, d.shape[1]):
            raise ValueError("lora_bt must be [r, N] with one r")
    dev = dys[0].device
    dh = [torch.empty((M, r), dtype=torch.float16, device=dev) for _ in dys]
    dht = [torch.empty((r, _ldt(M)), dtype=torch.float16, device=dev) for _ in dys]
    _lib.call("mxs_lora_dh_group", n, _ptr_array(dys), M, _int_array([d.shape[1] for d in dys]),
              _ptr_array(bts), r, float(s), _ldt(M), _ptr_array(dh), _ptr_array(dht),
              _lib.stream_of(dev))
    return list(zip(dh, dht))


def nf4_linear_fwd_hp(x2d, packed, state, lora_hp, lora_b, bias=None, cfg=-1, splits=1, ws=None):
    """(y, ht): Y = x2d @ W^T (+ bias) + fp16(sum of lora_hp) @ lora_b^T, and that fp16 LoRA
    operand transposed [r, ldt] (zeros past M)."""
    n, k = state.shape
    if x2d.dtype != torch.float16 or x2d.dim() != 2 or x2d.shape[1] != k:
        raise ValueError("x must be fp16 [M, in_features]")
    x2d = x2d.contiguous()
    M = x2d.shape[0]
    S, ldt, r = lora_hp.shape
    if ldt != _ldt(M) or lora_b.shape != (n, r) or lora_hp.dtype != torch.float32:
        raise ValueError("lora_hp [slices, ldt, r] fp32 needs lora_b [N, r]")
    lora_b = lora_b.to(torch.float16).contiguous()
    if bias is not None:
        bias = bias.to(torch.float16).contiguous()
    y = torch.empty((M, n), dtype=torch.float16, device=x2d.device)
    ht = torch.empty((r, ldt), dtype=torch.float16, device=x2d.device)
    ws = _ws(M, n, k, x2d.device, cfg, splits, ws)
    _lib.call("mxs_nf4_linear_fwd_hp", _lib.ptr(x2d), M, k, n, *_nf4_args(packed, state),
              _lib.ptr(bias), _lib.ptr(lora_hp.contiguous()), S, ldt, _lib.ptr(lora_b), r,
              _lib.ptr(ht), _lib.ptr(y), _lib.ptr(ws), cfg, splits, _lib.stream_of(x2d.device))
    return y, ht


def rope_spec(n_rope, cos, sin, M):
    """(cos stride b, cos stride t, tokens per sequence) for the RoPE of the grouped forward's
    first n_rope outputs over M rows: cos / sin fp32 [1 or B, T, 128] of one layout with a unit
    last stride, M = B * T."""
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.dim() != 3 \
            or cos.shape != sin.shape or cos.stride() != sin.stride() or cos.stride(-1) != 1 \
            or cos.shape[2] != 128:
        raise ValueError("cos / sin must be fp32 [1 or B, T, 128] with one layout")
    T = cos.shape[1]
    if n_rope < 1 or T < 1 or M % T != 0 or cos.shape[0] not in (1, M // T):
        raise ValueError("the rows must be B whole sequences of cos / sin's T tokens")
    return (cos.stride(0) if cos.shape[0] > 1 else 0), cos.stride(1), T


def nf4_linear_fwd_hp_group(x2ds, packeds, states, lora_hps=None, lora_bs=None, biases=None,
                            rope=None):
    """nf4_linear_fwd_hp for up to 4 projections of one input width over the same tokens in one
    launch (128x64 tiles when they fit the CUs in one round, else 128x128; unsplit): a list of
    (y, ht) (ht None without LoRA), the bits of nf4_linear_fwd_hp(..., cfg=10, splits=1) for
    each.  rope = (n_rope, cos, sin): the first n_rope outputs (attention's q and k, widths
    multiples of 128) come rotated (mxs_nf4_linear_fwd_hp_group_rope), the bits of qkv_rope's
    forward on the unrotated outputs; cos / sin as rope_spec takes them."""
    n = len(x2ds)
    lora_hps = lora_hps or [None] * n
    lora_bs = lora_bs or [None] * n
    biases = biases or [None] * n
    x2ds = [x.contiguous() for x in x2ds]
    M, K = x2ds[0].shape
    if not 1 <= n <= 4 or any(x.shape != (M, K) or x.dtype != torch.float16 for x in x2ds):
        raise ValueError("1..4 fp16 inputs [M, K] of one shape")
    dev = x2ds[0].device
    S = ldt = r = 0
    ys, hts, b16, bias16 = [], [], [], []
    for pk, st, hp, b, bias in zip(packeds, states, lora_hps, lora_bs, biases):
        nn_, k = st.shape
        if k != K:
            raise ValueError("every weight must take K inputs")
        check_nf4_operands(pk, st, dev)
        ys.append(torch.empty((M, nn_), dtype=torch.float16, device=dev))
        ht = None
        if hp is not None:
            S, ldt, r = hp.shape
            if ldt != _ldt(M) or b is None or b.shape != (nn_, r) or hp.dtype != torch.float32:
                raise ValueError("lora_hp [slices, ldt, r] fp32 needs lora_b [N, r]")
            b = b.to(torch.float16).contiguous()
            ht = torch.empty((r, ldt), dtype=torch.float16, device=dev)
        hts.append(ht)
        b16.append(b)
        bias16.append(None if bias is None else bias.to(torch.float16).contiguous())
    hps = [None if hp is None else hp.contiguous() for hp in lora_hps]
    if any(hp is not None and hp.shape != (S, ldt, r) for hp in hps):
        raise ValueError("LoRA partials of one shape")
    args = (n, _ptr_array(x2ds), M, K, _int_array([st.shape[0] for st in states]),
            _ptr_array(packeds), _ptr_array([st.absmax for st in states]),
            _ptr_array([st.state2.code for st in states]),
            _ptr_array([st.state2.absmax for st in states]),
            _ptr_array([st.offset for st in states]), _ptr_array(bias16), _ptr_array(hps), S,
            ldt, _ptr_array(b16), r, _ptr_array(hts), _ptr_array(ys))
    if rope is None:
        _lib.call("mxs_nf4_linear_fwd_hp_group", *args, _lib.stream_of(dev))
    else:
        n_rope, cos, sin = rope
        cs_b, cs_t, T = rope_spec(n_rope, cos, sin, M)
        if n_rope > n or any(st.shape[0] % 128 for st in states[:n_rope]) \
                or cos.device != dev or sin.device != dev:
            raise ValueError("rotated outputs: whole 128-column heads on the input's device")
        _lib.call("mxs_nf4_linear_fwd_hp_group_rope", *args, n_rope, _lib.ptr(cos),
                  _lib.ptr(sin), cs_b, cs_t, T, _lib.stream_of(dev))
    return list(zip(ys, hts))


def nf4_linear_bwd_dx_hp(dy2d, packed, state, lora_dhp, lora_at, mask=None, mask_scale=1.0,
                         cfg=-1, splits=1, ws=None, want_t=True):
    """(dx, dht): dX = dy2d @ W + mask * mask_scale * (fp16(sum of lora_dhp) @ lora_at^T), and
    that fp16 operand transposed [r, ldt] (None unless want_t)."""
    n, k = state.shape
    if dy2d.dtype != torch.float16 or dy2d.dim() != 2 or dy2d.shape[1] != n:
        raise ValueError("dy must be fp16 [M, out_features]")
    dy2d = dy2d.contiguous()
    M = dy2d.shape[0]
    S, ldt, r = lora_dhp.shape
    if ldt != _ldt(M) or lora_at.shape != (k, r) or lora_dhp.dtype != torch.float32:
        raise ValueError("lora_dhp [slices, ldt, r] fp32 needs lora_at [K, r]")
    mask = keep_bits(mask, M, k)
    dx = torch.empty((M, k), dtype=torch.float16, device=dy2d.device)
    dht = torch.empty((r, ldt), dtype=torch.float16, device=dy2d.device) if want_t else None
    ws = _ws(M, k, n, dy2d.device, cfg, splits, ws)
    _lib.call("mxs_nf4_linear_bwd_dx_hp", _lib.ptr(dy2d), M, n, k, *_nf4_args(packed, state),
              _lib.ptr(lora_dhp.contiguous()), S, ldt, _lib.ptr(lora_at.contiguous()), r,
              _lib.ptr(mask), float(mask_scale), _lib.ptr(dht), _lib.ptr(dx), _lib.ptr(ws), cfg,
              splits, _lib.stream_of(dy2d.device))
    return dx, dht


def fwd_pair_ok(M, N0, N1, K):
    """Whether nf4_linear_fwd_hp_pair takes two projections [K -> N0], [K -> N1] at M tokens."""
    return bool(_lib.lib().mxs_nf4_linear_fwd_pair_ok(M, N0, N1, K))


def nf4_linear_fwd_hp_pair(x2d, packeds, states, lora_hps, lora_bs, biases=None):
    """nf4_linear_fwd_hp for two projections over the same x2d in one launch (grid z selects the
    projection; the same bits as two calls): [(y, ht), (y, ht)].  Only where fwd_pair_ok."""
    (n0, k), (n1, k1) = states[0].shape, states[1].shape
    if x2d.dtype != torch.float16 or x2d.dim() != 2 or x2d.shape[1] != k or k1 != k:
        raise ValueError("x must be fp16 [M, in_features] of two weights [N_i, K]")
    x2d = x2d.contiguous()
    M = x2d.shape[0]
    if not fwd_pair_ok(M, n0, n1, k):
        raise ValueError(f"the forward pair does not take [{k} -> {n0}], [{k} -> {n1}] at {M} "
                         "tokens")
    S, ldt, r = lora_hps[0].shape
    for hp, b, n in zip(lora_hps, lora_bs, (n0, n1)):
        if hp.shape != (S, ldt, r) or hp.dtype != torch.float32 or ldt != _ldt(M) or \
                b.shape != (n, r):
            raise ValueError("lora_hp [slices, ldt, r] fp32 (one shape) and lora_b [N, r]")
    biases = biases or [None, None]
    biases = [None if b is None else b.to(torch.float16).contiguous() for b in biases]
    dev = x2d.device
    for pk, st in zip(packeds, states):
        check_nf4_operands(pk, st, dev)
    ys = [torch.empty((M, n), dtype=torch.float16, device=dev) for n in (n0, n1)]
    hts = [torch.empty((r, ldt), dtype=torch.float16, device=dev) for _ in range(2)]
    _lib.call("mxs_nf4_linear_fwd_hp_pair", _lib.ptr(x2d), M, k, _int_array([n0, n1]),
              _ptr_array(packeds), _ptr_array([st.absmax for st in states]),
              _ptr_array([st.state2.code for st in states]),
              _ptr_array([st.state2.absmax for st in states]),
              _ptr_array([st.offset for st in states]), _ptr_array(biases),
              _ptr_array([h.contiguous() for h in lora_hps]), S, ldt,
              _ptr_array([b.contiguous() for b in lora_bs]), r, _ptr_array(hts), _ptr_array(ys),
              _lib.stream_of(dev))
    return list(zip(ys, hts))


def bwd_dx_pair_ok(M, N0, N1, K):
    """True when nf4_linear_bwd_dx_hp_pair takes projections [K -> N0] and [K -> N1] at M tokens
    (both plan the narrow-output split-K kernel on their own)."""
    return bool(_lib.lib().mxs_nf4_linear_bwd_dx_pair_ok(M, N0, N1, K))


def _dx_pair_operands(dys, packeds, states, lora_dhps, lora_ats, masks):
    """The checked operands of the summed dX pair: (dys, M, N0, N1, K, slices, ldt, r, keep bits,
    device)."""
    masks = masks or [None, None]
    (n0, k), (n1, k1) = states[0].shape, states[1].shape
    dys = [d.contiguous() for d in dys]
    M = dys[0].shape[0]
    if k1 != k or dys[0].shape != (M, n0) or dys[1].shape != (M, n1) or \
            any(d.dtype != torch.float16 for d in dys):
        raise ValueError("dy_i must be fp16 [M, N_i] of two weights [N_i, K]")
    if not bwd_dx_pair_ok(M, n0, n1, k):
        raise ValueError(f"the pair does not take [{k} -> {n0}], [{k} -> {n1}] at {M} tokens")
    S, ldt, r = lora_dhps[0].shape
    for hp, at in zip(lora_dhps, lora_ats):
        if hp.shape != (S, ldt, r) or hp.dtype != torch.float32 or ldt != _ldt(M) or \
                at.shape != (k, r):
            raise ValueError("lora_dhp [slices, ldt, r] fp32 (one shape) and lora_at [K, r]")
    masks = [keep_bits(mk, M, k) for mk in masks]
    dev = dys[0].device
    for pk, st in zip(packeds, states):
        check_nf4_operands(pk, st, dev)
    return dys, M, n0, n1, k, S, ldt, r, masks, dev


def _dx_pair_args(dys, M, n0, n1, k, packeds, states, lora_dhps, S, ldt, lora_ats, r, masks,
                  mask_scale, dhts):
    return (_ptr_array(dys), M, _int_array([n0, n1]), k,
            _ptr_array(packeds), _ptr_array([st.absmax for st in states]),
            _ptr_array([st.state2.code for st in states]),
            _ptr_array([st.state2.absmax for st in states]),
            _ptr_array([st.offset for st in states]),
            _ptr_array([h.contiguous() for h in lora_dhps]), S, ldt,
            _ptr_array([a.contiguous() for a in lora_ats]), r,
            _ptr_array(masks), float(mask_scale), _ptr_array(dhts))


def nf4_linear_bwd_dx_hp_pair(dys, packeds, states, lora_dhps, lora_ats, masks=None,
                              mask_scale=1.0, want_t=True, ws=None):
    """(dx, [dht0, dht1]): dX = the sum of nf4_linear_bwd_dx_hp's two input gradients, from ONE
    split-K launch over both reductions and one reduce (each projection's part is never rounded
    to fp16 on its own), and each projection's fp16 dHs^T (None unless want_t).  Only where
    bwd_dx_pair_ok."""
    dys, M, n0, n1, k, S, ldt, r, masks, dev = _dx_pair_operands(dys, packeds, states, lora_dhps,
                                                                 lora_ats, masks)
    dx = torch.empty((M, k), dtype=torch.float16, device=dev)
    dhts = [torch.empty((r, ldt), dtype=torch.float16, device=dev) if want_t else None
            for _ in range(2)]
    ws = _workspace(int(_lib.lib().mxs_nf4_linear_bwd_dx_pair_workspace_bytes(M, n0, n1, k)),
                    dev, ws)
    _lib.call("mxs_nf4_linear_bwd_dx_hp_pair",
              *_dx_pair_args(dys, M, n0, n1, k, packeds, states, lora_dhps, S, ldt, lora_ats, r,
                             masks, mask_scale, dhts),
              _lib.ptr(dx), _lib.ptr(ws), _lib.stream_of(dev))
    return dx, dhts


def nf4_linear_bwd_dx_hp_pair_grads(dys, packeds, states, lora_dhps, lora_ats, hts, x2d,
                                    masks=None, mask_scale=1.0, ws=None):
    """(dx, [dht0, dht1], [(dA0, dB0), (dA1, dB1)]): nf4_linear_bwd_dx_hp_pair and then both
    projections' lora_grads_group from its dHs^T, the shared input x2d [M, K] and their Hs^T
    (hts), in two launches (the pair GEMM; its reduce and the gradients together); the bits of
    those two calls."""
    dys, M, n0, n1, k, S, ldt, r, masks, dev = _dx_pair_operands(dys, packeds, states, lora_dhps,
                                                                 lora_ats, masks)
    x2d = x2d.contiguous()
    if x2d.shape != (M, k) or any(tuple(ht.shape) != (r, ldt) for ht in hts):
        raise ValueError("x [M, K] and ht [r, ldt] disagree with the pair")
    dx = torch.empty((M, k), dtype=torch.float16, device=dev)
    dhts = [torch.empty((r, ldt), dtype=torch.float16, device=dev) for _ in range(2)]
    da = [torch.empty((r, k), dtype=torch.float32, device=dev) for _ in range(2)]
    db = [torch.empty((n, r), dtype=torch.float32, device=dev) for n in (n0, n1)]
    ws = _workspace(int(_lib.lib().mxs_nf4_linear_bwd_dx_pair_workspace_bytes(M, n0, n1, k)),
                    dev, ws)
    _lib.call("mxs_nf4_linear_bwd_dx_hp_pair_grads",
              *_dx_pair_args(dys, M, n0, n1, k, packeds, states, lora_dhps, S, ldt, lora_ats, r,
                             masks, mask_scale, dhts),
              _ptr_array([_c(t) for t in hts]), _lib.ptr(x2d), _ptr_array(da), _ptr_array(db),
              _lib.ptr(dx), _lib.ptr(ws), _lib.stream_of(dev))
    return dx, dhts, list(zip(da, db))


def glu_fused(M, N, K, bwd):
    """True when the projection K -> N at M tokens takes the SwiGLU epilogue on its planned
    kernel: nf4_linear_fwd_glu (bwd False) or nf4_linear_bwd_dx_glu (bwd True)."""
    return bool(_lib.lib().mxs_nf4_linear_glu_fused(M, N, K, int(bool(bwd))))


def _glu_operand(t, M, n, name):
    if t.dtype != torch.float16 or t.shape != (M, n) or not t.is_contiguous() \
            or t.data_ptr() % 16:
        raise ValueError(f"{name} must be a contiguous, 16-byte aligned fp16 [M, {n}] tensor")
    return t


def nf4_linear_fwd_glu(x2d, packed, state, gate, lora_hp=None, lora_b=None, bias=None, ws=None):
    """(y, h, ht): the up projection Y = x2d @ W^T (+ bias) (+ fp16(sum of lora_hp) @ lora_b^T)
    and H = silu(gate) * Y, both fp16 [M, N], from one launch; ht is the LoRA operand transposed
    [r, ldt] (None without LoRA).  Only where glu_fused(M, N, K, False)."""
    n, k = state.shape
    if x2d.dtype != torch.float16 or x2d.dim() != 2 or x2d.shape[1] != k:
        raise ValueError("x must be fp16 [M, in_features]")
    x2d = x2d.contiguous()
    M = x2d.shape[0]
    _glu_operand(gate, M, n, "gate")
    dev = x2d.device
    S = ldt = r = 0
    ht = None
    if lora_hp is not None:
        S, ldt, r = lora_hp.shape
        if ldt != _ldt(M) or lora_b is None or lora_b.shape != (n, r) \
                or lora_hp.dtype != torch.float32:
            raise ValueError("lora_hp [slices, ldt, r] fp32 needs lora_b [N, r]")
        lora_b = lora_b.to(torch.float16).contiguous()
        lora_hp = lora_hp.contiguous()
        ht = torch.empty((r, ldt), dtype=torch.float16, device=dev)
    if bias is not None:
        bias = bias.to(torch.float16).contiguous()
    y = torch.empty((M, n), dtype=torch.float16, device=dev)
    h = torch.empty((M, n), dtype=torch.float16, device=dev)
    ws = _ws(M, n, k, dev, -1, 1, ws)
    _lib.call("mxs_nf4_linear_fwd_glu", _lib.ptr(x2d), M, k, n, *_nf4_args(packed, state),
              _lib.ptr(bias), _lib.ptr(lora_hp), S, ldt, _lib.ptr(lora_b), r, _lib.ptr(ht),
              _lib.ptr(gate), _lib.ptr(y), _lib.ptr(h), _lib.ptr(ws), _lib.stream_of(dev))
    return y, h, ht


def nf4_linear_bwd_dx_glu_(dy2d, packed, state, gate, up, lora_dhp=None, lora_at=None,
                           mask=None, mask_scale=1.0, ws=None, want_t=True):
    """In place: the down projection's dH = dy2d @ W (+ mask * mask_scale * (fp16(sum of
    lora_dhp) @ lora_at^T)) goes through the SwiGLU backward in the GEMM's epilogue: gate <-
    d(gate), up <- d(up) (fp16 [M, K]); dH itself is not stored.  Returns dht, the LoRA operand
    transposed [r, ldt] (None without LoRA or unless want_t).  Only where
    glu_fused(M, N, K, True)."""
    n, k = state.shape
    if dy2d.dtype != torch.float16 or dy2d.dim() != 2 or dy2d.shape[1] != n:
        raise ValueError("dy must be fp16 [M, out_features]")
    dy2d = dy2d.contiguous()
    M = dy2d.shape[0]
    _glu_operand(gate, M, k, "gate")
    _glu_operand(up, M, k, "up")
    dev = dy2d.device
    S = ldt = r = 0
    dht = None
    if lora_dhp is not None:
        S, ldt, r = lora_dhp.shape
        if ldt != _ldt(M) or lora_at is None or lora_at.shape != (k, r) \
                or lora_dhp.dtype != torch.float32:
            raise ValueError("lora_dhp [slices, ldt, r] fp32 needs lora_at [K, r]")
        lora_dhp, lora_at = lora_dhp.contiguous(), lora_at.contiguous()
        mask = keep_bits(mask, M, k)
        if want_t:
            dht = torch.empty((r, ldt), dtype=torch.float16, device=dev)
    ws = _ws(M, k, n, dev, -1, 1, ws)
    _lib.call("mxs_nf4_linear_bwd_dx_glu", _lib.ptr(dy2d), M, n, k, *_nf4_args(packed, state),
              _lib.ptr(lora_dhp), S, ldt, _lib.ptr(lora_at), r, _lib.ptr(mask),
              float(mask_scale), _lib.ptr(dht), _lib.ptr(gate), _lib.ptr(up), _lib.ptr(ws),
              _lib.stream_of(dev))
    return dht


def lora_finish(partials, M, want_out=False):
    """(out, outT): the fp16 operand from LoRA partial sums [slices, ldt, r] fp32 (added in slice
    order, as the fused GEMMs do): out [M, r] (None unless want_out) and outT [r, ldt]."""
    S, ldt, r = partials.shape
    if partials.dtype != torch.float32 or ldt != _ldt(M):
        raise ValueError("partials must be fp32 [slices, ldt, r]")
    dev = partials.device
    out = torch.empty((M, r), dtype=torch.float16, device=dev) if want_out else None
    outT = torch.empty((r, ldt), dtype=torch.float16, device=dev)
    _lib.call("mxs_lora_finish", _lib.ptr(partials.contiguous()), S, M, r, ldt, _lib.ptr(out),
              _lib.ptr(outT), _lib.stream_of(dev))
    return out, outT


def transpose(t2d):
    """[rows, cols] fp16 -> [cols, rows] fp16 on the GPU (mxs_transpose_f16)."""
    t2d = t2d.contiguous()
    rows, cols = t2d.shape
    out = torch.empty((cols, rows), dtype=torch.float16, device=t2d.device)
    _lib.call("mxs_transpose_f16", _lib.ptr(t2d), rows, cols, _lib.ptr(out),
              _lib.stream_of(t2d.device))
    return out


def _ldt(M):
    return (M + 7) // 8 * 8


def lora_h(x2d, lora_a, s, mask=None, mask_scale=1.0, ws=None, n_out=None, want_at=False,
           lora_b=None):
    """(h, ht): h = fp16(s * drop(x) @ A^T) [M, r] and its transpose [r, ldt]; with want_at also
    (at, bt): lora_A^T [K, r] and, given lora_b [N, r], lora_B^T [r, N] (else None) -- the
    backward's operands, written by the same launch."""
    x2d = x2d.contiguous()
    lora_a = lora_a.to(torch.float16).contiguous()
    M, K = x2d.shape
    r = lora_a.shape[0]
    dev = x2d.device
    h = torch.empty((M, r), dtype=torch.float16, device=dev)
    ht = torch.empty((r, _ldt(M)), dtype=torch.float16, device=dev)
    ws = _workspace(lora_workspace_bytes(M, K, n_out or K, r), dev, ws)
    at = bt = None
    N = 0
    if want_at:
        at = torch.empty((K, r), dtype=torch.float16, device=dev)
        if lora_b is not None:
            lora_b = lora_b.to(torch.float16).contiguous()
            N = lora_b.shape[0]
            if lora_b.shape != (N, r):
                raise ValueError("lora_b must be [N, r]")
            bt = torch.empty((r, N), dtype=torch.float16, device=dev)
    _lib.call("mxs_lora_h", _lib.ptr(x2d), M, K, _lib.ptr(lora_a), r,
              _lib.ptr(keep_bits(mask, M, K)),
              float(mask_scale), float(s), _lib.ptr(h), _lib.ptr(ht), ht.shape[1], _lib.ptr(at),
              _lib.ptr(lora_b if bt is not None else None), N, _lib.ptr(bt), _lib.ptr(ws),
              _lib.stream_of(dev))
    return (h, ht, at, bt) if want_at else (h, ht)


def lora_dh(dy2d, lora_b, s, ws=None, k_in=None, lora_bt=None, one_launch=False):
    """(dh, dht): dh = fp16(s * dY @ B) [M, r] and its transpose [r, ldt].  The kernel takes
    lora_B transposed ([r, N], the bt output of lora_h); given only lora_b it is transposed here.
    one_launch: no workspace, so the whole reduction stays in one launch (long reductions are
    otherwise split over slices of workgroups and finished by a second launch)."""
    dy2d = dy2d.contiguous()
    M, N = dy2d.shape
    if lora_bt is None:
        lora_bt = lora_b.to(torch.float16).t().contiguous()
    r = lora_bt.shape[0]
    if lora_bt.shape != (r, N):
        raise ValueError("lora_bt must be [r, N]")
    ws = None if one_launch else _workspace(lora_workspace_bytes(M, k_in or N, N, r),
                                            dy2d.device, ws)
    dh = torch.empty((M, r), dtype=torch.float16, device=dy2d.device)
    dht = torch.empty((r, _ldt(M)), dtype=torch.float16, device=dy2d.device)
    _lib.call("mxs_lora_dh", _lib.ptr(dy2d), M, N, _lib.ptr(lora_bt.contiguous()), r, float(s),
              _lib.ptr(dh), _lib.ptr(dht), dht.shape[1], _lib.ptr(ws), _lib.stream_of(dy2d.device))
    return dh, dht


def lora_grads(dht, ht, x2d, dy2d, mask=None, mask_scale=1.0, want_a=True, want_b=True,
               ws=None):
    """(dA, dB) in one launch: dA = dh^T @ drop(x) fp32 [r, K], dB = dY^T @ h fp32 [N, r]
    (None where not wanted)."""
    x2d, dy2d = x2d.contiguous(), dy2d.contiguous()
    M, K = x2d.shape
    N = dy2d.shape[1]
    r = dht.shape[0]
    if dy2d.shape[0] != M or ht.shape != dht.shape:
        raise ValueError("x, dy and the transposed LoRA activations disagree")
    da = torch.empty((r, K), dtype=torch.float32, device=x2d.device) if want_a else None
    db = torch.empty((N, r), dtype=torch.float32, device=x2d.device) if want_b else None
    if da is None and db is None:
        return None, None
    _lib.call("mxs_lora_grads", _lib.ptr(dht), _lib.ptr(ht), dht.shape[1], _lib.ptr(x2d),
              _lib.ptr(dy2d), M, K, N, r, _lib.ptr(keep_bits(mask, M, K)), float(mask_scale),
              _lib.ptr(da),
              _lib.ptr(db), _lib.ptr(ws), _lib.stream_of(x2d.device))
    return da, db


def lora_grads_group(dhts, hts, x2ds, dy2ds, masks=None, mask_scale=1.0):
    """lora_grads (dA and dB) for up to 4 projections of equal shapes in one launch: a list of
    (dA [r, K] fp32, dB [N, r] fp32), the bits of separate calls."""
    n = len(dhts)
    masks = masks or [None] * n
    x2ds = [x.contiguous() for x in x2ds]
    dy2ds = [d.contiguous() for d in dy2ds]
    M = x2ds[0].shape[0]
    r, ldt = dhts[0].shape
    dev = x2ds[0].device
    for dht, ht, x, dy in zip(dhts, hts, x2ds, dy2ds):
        if dht.shape != (r, ldt) or ht.shape != (r, ldt) or x.shape[0] != M or dy.shape[0] != M:
            raise ValueError("dht / ht [r, ldt], x [M, K], dy [M, N] disagree")
    da = [torch.empty((r, x.shape[1]), dtype=torch.float32, device=dev) for x in x2ds]
    db = [torch.empty((d.shape[1], r), dtype=torch.float32, device=dev) for d in dy2ds]
    _lib.call("mxs_lora_grads_group", n, _ptr_array([_c(t) for t in dhts]),
              _ptr_array([_c(t) for t in hts]), ldt, _ptr_array(x2ds), _ptr_array(dy2ds), M,
              _int_array([x.shape[1] for x in x2ds]), _int_array([d.shape[1] for d in dy2ds]), r,
              _ptr_array([keep_bits(m, M, x.shape[1]) for m, x in zip(masks, x2ds)]),
              float(mask_scale), _ptr_array(da),
              _ptr_array(db), _lib.stream_of(dev))
    return list(zip(da, db))


def lora_grad_a(dht, x2d, mask=None, mask_scale=1.0, ws=None):
    """dA = dh^T @ drop(x), fp32 [r, K]."""
    x2d = x2d.contiguous()
    M, K = x2d.shape
    r = dht.shape[0]
    da = torch.empty((r, K), dtype=torch.float32, device=x2d.device)
    _lib.call("mxs_lora_grad_a", _lib.ptr(dht), dht.shape[1], _lib.ptr(x2d), M, K, r,
              _lib.ptr(keep_bits(mask, M, K)), float(mask_scale), _lib.ptr(da), _lib.ptr(ws),
              _lib.stream_of(x2d.device))
    return da


def lora_grad_b(ht, dy2d, ws=None):
    """dB = dY^T @ h, fp32 [N, r] (h already carries the scaling s)."""
    dy2d = dy2d.contiguous()
    M, N = dy2d.shape
    r = ht.shape[0]
    db = torch.empty((N, r), dtype=torch.float32, device=dy2d.device)
    _lib.call("mxs_lora_grad_b", _lib.ptr(ht), ht.shape[1], _lib.ptr(dy2d), M, N, r,
              _lib.ptr(db), _lib.ptr(ws), _lib.stream_of(dy2d.device))
    return db


def silu_mul(gate, up):
    """fp16 silu(gate) * up (contiguous, same shape); one HIP launch."""
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate)
    _lib.call("mxs_silu_mul", _lib.ptr(gate), _lib.ptr(up), _lib.ptr(out), gate.numel(),
              _lib.stream_of(gate.device))
    return out


def silu_mul_bwd_(grad, gate, up):
    """In place: gate <- d(gate), up <- d(up) for the incoming fp16 gradient (gate and up must
    be contiguous)."""
    grad = grad.contiguous()
    if not (gate.is_contiguous() and up.is_contiguous()):
        raise ValueError("gate and up must be contiguous (their memory takes the gradients)")
    _lib.call("mxs_silu_mul_bwd", _lib.ptr(grad), _lib.ptr(gate), _lib.ptr(up), gate.numel(),
              _lib.stream_of(gate.device))


def qkv_rope(q_a, q_b, k, v_a, v_b, cos, sin, q_o, k_o, v_o, backward=False, q_scale=1.0,
             v_scale=1.0):
    """mxs_qkv_rope on [B, H, T, 128] views with unit stride along the head (any other strides):
    q_o = rot(q_a + q_scale * q_b), k_o = rot(k), v_o = v_a + v_scale * v_b (q_b, v_a, v_b may
    be None; v_o with v_a); rot the forward rotation, or its inverse with backward.  Inputs all
    fp16 or all fp32, outputs all fp16 or all fp32; cos / sin fp32 [1 or B, T, 128] rows with
    unit last stride."""
    ins = [q_a, q_b, k, v_a, v_b]
    outs = [q_o, k_o, v_o]
    in_dt = {t.dtype for t in ins if t is not None}
    out_dt = {t.dtype for t in outs if t is not None}
    if len(in_dt) != 1 or len(out_dt) != 1 or not in_dt <= {torch.float16, torch.float32} \
            or not out_dt <= {torch.float16, torch.float32}:
        raise ValueError("inputs of one dtype and outputs of one dtype, each fp16 or fp32")
    batch, n_q, n_tokens, dim = q_a.shape
    n_kv = k.shape[1]
    if dim != 128 or k.shape != (batch, n_kv, n_tokens, 128):
        raise ValueError("q and k must be [B, H, T, 128]")
    for t, n in ((q_b, n_q), (v_a, n_kv), (v_b, n_kv), (q_o, n_q), (k_o, n_kv), (v_o, n_kv)):
        if t is not None and t.shape != (batch, n, n_tokens, 128):
            raise ValueError("operand shapes disagree")
    if (v_a is None) != (v_o is None) or (v_b is not None and v_a is None):
        raise ValueError("v_o goes with v_a, v_b needs v_a")
    for t in ins + outs:
        if t is not None and t.stride(-1) != 1:
            raise ValueError("unit stride along the head required")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape \
            or cos.stride() != sin.stride() or cos.stride(-1) != 1 \
            or tuple(cos.shape[1:]) != (n_tokens, 128) or cos.shape[0] not in (1, batch):
        raise ValueError("cos / sin must be fp32 [1 or B, T, 128] with one layout")
    import ctypes

    tens = (ctypes.c_void_p * 8)(*[None if t is None else t.data_ptr() for t in ins + outs])
    strides = (ctypes.c_int64 * 24)(*[s for t in ins + outs
                                      for s in ((0, 0, 0) if t is None else
                                                (t.stride(0), t.stride(1), t.stride(2)))])
    cs_b = cos.stride(0) if cos.shape[0] == batch else 0
    _lib.call("mxs_qkv_rope", tens, strides, _lib.ptr(cos), _lib.ptr(sin), cs_b, cos.stride(1),
              batch, n_tokens, n_q, n_kv, int(torch.float32 in in_dt),
              int(torch.float32 in out_dt), int(bool(backward)), float(q_scale),
              float(v_scale), _lib.stream_of(q_a.device))
