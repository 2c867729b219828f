"""Linear4bit forward/backward on the HIP NF4 path (mirror of solution/linear4bit.py), and the
LoRA-wrapped projection with its branch fused into the same kernels.

`NF4LinearFunction` keeps the reference's contract (solution/linear4bit.py:43-57): forward
Y = x @ W^T + bias, backward grad_x = grad @ W, no gradient for the frozen W or bias.  With
FUSED_GEMM the two products run as the fused dequant-GEMM kernels; otherwise W is decoded by the
HIP dequant kernel and multiplied by torch (the reference's own structure).

`Linear4bit` is a bitsandbytes-compatible module for when bitsandbytes is absent (same
`forward(self, x)`, same `weight.quant_state` fields); `patch_bnb_linear4bit` installs the same
forward on `bitsandbytes.nn.Linear4bit` when it is importable.  `LoraLinear4bit` has peft's
attribute layout (base_layer, lora_A/lora_B/lora_dropout dicts, scaling, active_adapters,
merged, disable_adapters) and computes base(x) + s * B(A(drop(x))) with `NF4LoraFunction`.
"""

import contextlib
import math

import torch

from . import direct, kernels, ops, stream
from .nf4 import _supported, unpack_nf4
from .quant import QuantState, quantize_4bit

_enabled = True
cache_fp16 = False   # set by patch_bnb_linear4bit(cache_weights=...)
FUSED_GEMM = True    # FEATURES["nf4_fused_gemm"]
FUSED_LORA = True    # FEATURES["nf4_fused_lora"]


@contextlib.contextmanager
def disabled():
    """Run the unpatched path inside the block (solution/linear4bit.py:25-33)."""
    global _enabled
    previous, _enabled = _enabled, False
    try:
        yield
    finally:
        _enabled = previous


def _unpack(packed, state, dtype, absmax_8bit=None):
    """The dense [N, K] weight (solution/linear4bit.py:36-40)."""
    return unpack_nf4(packed, state.shape, state.state2.absmax, state.blocksize, dtype,
                      absmax_8bit=state.absmax if absmax_8bit is None else absmax_8bit,
                      code=state.state2.code, offset=state.offset)


def _fused(state, x):
    return FUSED_GEMM and x.dtype == torch.float16 and kernels.fused_shape_ok(state)


class NF4LinearFunction(torch.autograd.Function):
    """F.linear(x, unpack(W), bias); backward grad_x = grad @ unpack(W).  W and bias frozen."""

    @staticmethod
    def forward(ctx, x, packed, state, bias):
        ctx.packed, ctx.state = packed, state
        if _fused(state, x):
            lead = x.shape[:-1]
            y = kernels.nf4_linear_fwd(x.reshape(-1, x.shape[-1]), packed, state, bias)
            return y.view(*lead, y.shape[-1])
        return torch.nn.functional.linear(x, _unpack(packed, state, x.dtype), bias)

    @staticmethod
    def backward(ctx, grad):
        grad_x = None
        if ctx.needs_input_grad[0]:
            state = ctx.state
            if _fused(state, grad):
                lead = grad.shape[:-1]
                g = kernels.nf4_linear_bwd_dx(grad.reshape(-1, grad.shape[-1]), ctx.packed,
                                              state)
                grad_x = g.view(*lead, g.shape[-1])
            else:
                grad_x = torch.matmul(grad, _unpack(ctx.packed, state, state.dtype)
                                      .to(grad.dtype))
        return grad_x, None, None, None


def _stream_product(module, state, x, bias, backward):
    """x @ W^T + bias (forward) or x @ W (backward) for a module whose bytes live in host
    memory: the decoded layer buffer when its layer is decoded, else the fused GEMM (or the
    dequant and torch) on the slot's bytes, asked for right before this use."""
    w16 = stream.weight_for(module)
    if w16 is None:
        packed, absmax = stream.bytes_for(module)
        packed = packed.view(-1, 1)
        if _fused(state, x):
            st = stream.state_with(state, absmax)
            lead = x.shape[:-1]
            x2d = x.reshape(-1, x.shape[-1])
            y = (kernels.nf4_linear_bwd_dx(x2d, packed, st) if backward
                 else kernels.nf4_linear_fwd(x2d, packed, st, bias))
            return y.view(*lead, y.shape[-1])
        w16 = _unpack(packed, state, state.dtype, absmax)
    w = w16.to(x.dtype)
    return torch.matmul(x, w) if backward else torch.nn.functional.linear(x, w, bias)


class NF4StreamFunction(torch.autograd.Function):
    """NF4LinearFunction for a module whose bytes live in host memory (stream.py): the bytes are
    asked for right before each use, in forward and again in backward
    (solution/linear4bit.py:68-84)."""

    @staticmethod
    def forward(ctx, x, module, state, bias):
        ctx.module, ctx.state = module, state
        return _stream_product(module, state, x, bias, backward=False)

    @staticmethod
    def backward(ctx, grad):
        grad_x = None
        if ctx.needs_input_grad[0]:
            grad_x = _stream_product(ctx.module, ctx.state, grad, None, backward=True)
        return grad_x, None, None, None


def _streamed_forward(layer, x):
    """Linear4bit.forward's own steps (input to the compute dtype, bias cast, output back to the
    input dtype) around the streamed product (solution/linear4bit.py:87-97)."""
    inp_dtype = x.dtype
    if layer.compute_dtype is not None:
        x = x.to(layer.compute_dtype)
    bias = _cast_bias_once(layer, x)
    if bias is not None:
        bias = bias.to(layer.compute_dtype)
    return direct.run(NF4StreamFunction, x, layer, layer.weight.quant_state, bias).to(inp_dtype)


def _dh_kind(M, N, K, r, want_x, want_a, want_b):
    """How lora_backward takes dHs for this projection: "finished" (one launch, for the dX GEMM
    that also computes dA and dB) or "partials" (finished by the dX GEMM)."""
    fused = want_x and want_a and want_b and kernels.bwd_grads_fused(M, N, K, r)
    return "finished" if fused else "partials"


def prepare_dh(items):
    """dHs for several projections at once, grouped into one launch per kind (and LoRA scaling):
    items are (dy [M, N], lora_bt [r, N], K, s, (want_x, want_a, want_b)); returns for each the
    keyword arguments (dh= or dhp=) of lora_backward.  The q/k/v projections' output gradients
    arrive together from attention's backward, gate/up's from the SwiGLU's."""
    out = [None] * len(items)
    groups = {}
    for i, (dy, bt, K, s, wants) in enumerate(items):
        M, N = dy.shape
        kind = _dh_kind(M, N, K, bt.shape[0], *wants)
        groups.setdefault((kind, float(s)), []).append(i)
    for (kind, s), idx in groups.items():
        for j in range(0, len(idx), 4):
            part = idx[j:j + 4]
            dys = [items[i][0] for i in part]
            bts = [items[i][1] for i in part]
            if kind == "finished":
                for i, r in zip(part, kernels.lora_dh_group(dys, bts, s)):
                    out[i] = {"dh": r}
            else:
                for i, r in zip(part, kernels.lora_dh_partials_group(dys, bts, s)):
                    out[i] = {"dhp": r}
    return out


def lora_backward(dy, x2d, keep, ht, at, bt, packed, state, mask_scale, s, want_x=True,
                  want_a=True, want_b=True, ws=None, dh=None, dhp=None):
    """(dX, dA, dB) of one NF4 + LoRA projection (None where not wanted), on the current stream.
    Where the dX GEMM leaves CUs idle (kernels.bwd_grads_fused: 1536-wide projections at 1024
    tokens) and all three are wanted: dHs = s * dY B finished in one launch, then one launch for
    dX and both weight gradients (their workgroups run beside the dX tiles).  Otherwise dHs as
    slice partials, the fused dX GEMM (which finishes dHs and writes dHs^T), then dA and dB in
    one launch.  (A variant that ran the weight gradients on a second stream beside the GEMM
    lost more to the cross-queue waits of the graph, 5-10 us per fork and join, than it
    gained.)  `ws`: an optional workspace for every call of this projection
    (kernels.projection_workspace_bytes).  `dh` = (dh, dht) or `dhp` (partials): dHs already
    computed, of the kind this projection's plan takes (prepare_dh)."""
    M, N = dy.shape
    K, r = x2d.shape[1], bt.shape[0]
    if _dh_kind(M, N, K, r, want_x, want_a, want_b) == "finished":
        if dh is None:
            dh = kernels.lora_dh(dy, None, s, lora_bt=bt, one_launch=True)
        return kernels.nf4_linear_bwd_dx_grads(dy, packed, state, dh[0], at, dh[1], ht, x2d,
                                               keep, mask_scale, ws=ws)
    if dhp is None:
        dhp = kernels.lora_dh_partials(dy, bt, s)
    want_g = want_a or want_b
    dx = dht = None
    if want_x or want_g:
        dx, dht = kernels.nf4_linear_bwd_dx_hp(dy, packed, state, dhp, at, keep, mask_scale,
                                               ws=ws, want_t=want_g)
    if not want_x:
        dx = None
    da = db = None
    if want_g:
        da, db = kernels.lora_grads(dht, ht, x2d, dy, keep, mask_scale, want_a=want_a,
                                    want_b=want_b, ws=ws)
    return dx, da, db


def _pair_takes(items, pre):
    """Whether the two projections' input gradients go through one summed dX launch
    (kernels.nf4_linear_bwd_dx_hp_pair): both take dHs partials, both want dX, one input
    tensor, one dropout scale, and shapes the pair's plan takes."""
    if len(items) != 2 or any("dhp" not in p for p in pre):
        return False
    a, b = items
    x0, x1 = a["x2d"], b["x2d"]
    return (a["wants"][0] and b["wants"][0] and a["mask_scale"] == b["mask_scale"]
            and x0.shape == x1.shape and x0.data_ptr() == x1.data_ptr()
            and pre[0]["dhp"].shape == pre[1]["dhp"].shape
            and kernels.bwd_dx_pair_ok(x0.shape[0], a["dy"].shape[1], b["dy"].shape[1],
                                       x0.shape[1]))


def _sum_takes(items):
    """The summed launch (kernels.nf4_linear_bwd_dx_grads_sum) takes these projections: 2..3 over
    one input, every gradient wanted, one LoRA scaling and dropout scale, a keep mask for every
    one or none, and a plan the library takes (q, k and v)."""
    if not 2 <= len(items) <= 3:
        return False
    a = items[0]
    x = a["x2d"]
    masked = a["keep"] is not None
    for it in items:
        if (tuple(it["wants"]) != (True, True, True) or it["x2d"].data_ptr() != x.data_ptr()
                or it["x2d"].shape != x.shape or it["s"] != a["s"]
                or it["mask_scale"] != a["mask_scale"] or (it["keep"] is not None) != masked):
            return False
    return kernels.bwd_grads_sum_ok(x.shape[0], [it["state"].shape[0] for it in items],
                                    x.shape[1], a["bt"].shape[0], grads=False)


def _backward_summed(items):
    """dHs of all items in one launch, then one launch for their summed dX and (up to 1152
    tokens) every dA / dB; past that the summed dX alone, then dA / dB in one launch per
    weight height (k and v share one)."""
    a = items[0]
    x = a["x2d"]
    dhs = kernels.lora_dh_group([it["dy"] for it in items], [it["bt"] for it in items], a["s"])
    Ns = [it["state"].shape[0] for it in items]
    fused = kernels.bwd_grads_sum_ok(x.shape[0], Ns, x.shape[1], a["bt"].shape[0])
    dx, grads = kernels.nf4_linear_bwd_dx_grads_sum(
        [it["dy"] for it in items], [it["packed"] for it in items],
        [it["state"] for it in items], [d[0] for d in dhs], [it["at"] for it in items],
        [d[1] for d in dhs], [it["ht"] for it in items], x,
        [it["keep"] for it in items], a["mask_scale"], grads=fused)
    if grads is None:
        grads = [None] * len(items)
        for n_ in dict.fromkeys(Ns):
            idx = [i for i, n2 in enumerate(Ns) if n2 == n_]
            if len(idx) > 1:
                res = kernels.lora_grads_group([dhs[i][1] for i in idx],
                                               [items[i]["ht"] for i in idx], [x] * len(idx),
                                               [items[i]["dy"] for i in idx],
                                               [items[i]["keep"] for i in idx], a["mask_scale"])
            else:
                i = idx[0]
                res = [kernels.lora_grads(dhs[i][1], items[i]["ht"], x, items[i]["dy"],
                                          items[i]["keep"], a["mask_scale"])]
            for i, r in zip(idx, res):
                grads[i] = r
    return [(dx if i == 0 else None, da, db) for i, (da, db) in enumerate(grads)]


def lora_backward_group(items, ws=None, sum_dx=False):
    """lora_backward for up to 4 projections over the same tokens whose output gradients arrive
    together (q/k/v from attention's backward, gate/up from the SwiGLU's), with their small
    launches shared: dHs in one launch per kind (prepare_dh); the dX GEMMs that carry the weight
    gradients in one launch where kernels.bwd_grads_group_ok allows; otherwise each dX GEMM,
    then dA and dB of all of them in one launch (equal shapes).  items: dicts with dy, x2d,
    keep, ht, at, bt, packed, state, mask_scale, s and wants = (want_x, want_a, want_b).
    Returns [(dx, dA, dB)], the bits of lora_backward on each.
    sum_dx (projections over one input, whose input gradients autograd adds): the first item's
    dx is the sum of all the items' (added in item order), the others' None; projections a
    summed launch takes get their sum from that one launch, the fp32 sum rounded once instead
    of each part rounded and added: q, k and v (_sum_takes: one tile loop over their three
    reductions, with every dA / dB in the same launch), gate and up (_pair_takes: split-K
    planes of both reductions, then one launch for their reduce and, where every weight
    gradient is wanted, both projections' dA / dB)."""
    n = len(items)
    if sum_dx and _sum_takes(items):
        return _backward_summed(items)
    pre = prepare_dh([(it["dy"], it["bt"], it["x2d"].shape[1], it["s"], it["wants"])
                      for it in items])
    out = [None] * n
    M = items[0]["dy"].shape[0]
    fused = [i for i in range(n) if "dh" in pre[i]]
    if len(fused) > 1:
        its = [items[i] for i in fused]
        K, r = its[0]["x2d"].shape[1], its[0]["bt"].shape[0]
        if (all(it["x2d"].shape[1] == K and it["mask_scale"] == its[0]["mask_scale"]
                for it in its)
                and kernels.bwd_grads_group_ok(M, [it["state"].shape[0] for it in its], K, r)):
            res = kernels.nf4_linear_bwd_dx_grads_group(
                [it["dy"] for it in its], [it["packed"] for it in its],
                [it["state"] for it in its], [pre[i]["dh"][0] for i in fused],
                [it["at"] for it in its], [pre[i]["dh"][1] for i in fused],
                [it["ht"] for it in its], [it["x2d"] for it in its],
                [it["keep"] for it in its], its[0]["mask_scale"])
            for i, r_ in zip(fused, res):
                out[i] = r_
    for i in fused:
        if out[i] is None:
            it = items[i]
            out[i] = lora_backward(it["dy"], it["x2d"], it["keep"], it["ht"], it["at"], it["bt"],
                                   it["packed"], it["state"], it["mask_scale"], it["s"],
                                   *it["wants"], ws=ws, **pre[i])
    pending = []
    if sum_dx and not fused and _pair_takes(items, pre):
        want_t = [it["wants"][1] or it["wants"][2] for it in items]
        pair_args = ([it["dy"] for it in items], [it["packed"] for it in items],
                     [it["state"] for it in items], [p["dhp"] for p in pre],
                     [it["at"] for it in items])
        if all(it["wants"][1] and it["wants"][2] for it in items) and \
                items[0]["dy"].shape == items[1]["dy"].shape:
            # the pair's reduce and both projections' dA / dB in one launch
            dx, _, grads = kernels.nf4_linear_bwd_dx_hp_pair_grads(
                *pair_args, [it["ht"] for it in items], items[0]["x2d"],
                [it["keep"] for it in items], items[0]["mask_scale"], ws=ws)
            out = [[dx, *grads[0]], [None, *grads[1]]]
        else:
            dx, dhts = kernels.nf4_linear_bwd_dx_hp_pair(
                *pair_args, [it["keep"] for it in items], items[0]["mask_scale"],
                want_t=any(want_t), ws=ws)
            out = [[dx, None, None], [None, None, None]]
            pending = [(i, dhts[i]) for i in range(2) if want_t[i]]
        sum_dx = False  # summed
    for i in range(n):
        if out[i] is not None:
            continue
        it = items[i]
        want_x, want_a, want_b = it["wants"]
        want_g = want_a or want_b
        dx, dht = None, None
        if want_x or want_g:
            dx, dht = kernels.nf4_linear_bwd_dx_hp(it["dy"], it["packed"], it["state"],
                                                   pre[i]["dhp"], it["at"], it["keep"],
                                                   it["mask_scale"], ws=ws, want_t=want_g)
        out[i] = [dx if want_x else None, None, None]
        if want_g:
            pending.append((i, dht))
    both = [(i, d) for i, d in pending if items[i]["wants"][1] and items[i]["wants"][2]]
    shapes = {(items[i]["x2d"].shape[1], items[i]["dy"].shape[1], items[i]["mask_scale"])
              for i, _ in both}
    if len(both) > 1 and len(shapes) == 1:
        res = kernels.lora_grads_group([d for _, d in both], [items[i]["ht"] for i, _ in both],
                                       [items[i]["x2d"] for i, _ in both],
                                       [items[i]["dy"] for i, _ in both],
                                       [items[i]["keep"] for i, _ in both],
                                       items[both[0][0]]["mask_scale"])
        for (i, _), (da, db) in zip(both, res):
            out[i][1], out[i][2] = da, db
        pending = [(i, d) for i, d in pending if (i, d) not in both]
    for i, dht in pending:
        it = items[i]
        da, db = kernels.lora_grads(dht, it["ht"], it["x2d"], it["dy"], it["keep"],
                                    it["mask_scale"], want_a=it["wants"][1],
                                    want_b=it["wants"][2], ws=ws)
        out[i][1], out[i][2] = da, db
    out = [list(o) for o in out]
    if sum_dx:
        dx = None
        for o in out:
            if o[0] is not None:
                dx = o[0] if dx is None else dx + o[0]
            o[0] = None
        out[0][0] = dx
    return [tuple(o) for o in out]


class NF4LoraFunction(torch.autograd.Function):
    """base(x) + s * B(A(drop(x))) for a frozen NF4 base, fused:
    forward:  Hs = s * drop(x) A^T as slice partials (mxs_lora_h_partials), then one fused GEMM
              that finishes Hs and computes Y = x W^T + bias + Hs B^T (and writes Hs^T);
    backward: dHs = s * dY B as slice partials (mxs_lora_dh_partials), then one fused GEMM
              that finishes dHs and computes dX = dY W + keep/(1-p) * dHs A (and writes dHs^T);
              dA = dHs^T drop(x) and dB = dY^T Hs in one launch.
    `keep` is the dropout keep mask: u8 [M, K] or keep bits (kernels.keep_bits; packed once in
    the forward and saved so), None without dropout; mask_scale = 1/(1-p)."""

    @staticmethod
    def forward(ctx, x2d, lora_a, lora_b, packed, state, bias, keep, mask_scale, s):
        a16 = lora_a.to(torch.float16).contiguous()
        b16 = lora_b.to(torch.float16).contiguous()
        n, k = state.shape
        keep = kernels.keep_bits(keep, x2d.shape[0], k)  # packed once, kept for the backward
        hp, at, bt = kernels.lora_h_partials(x2d, a16, s, keep, mask_scale, lora_b=b16)
        y, ht = kernels.nf4_linear_fwd_hp(x2d, packed, state, hp, b16, bias)
        ctx.save_for_backward(x2d, keep, ht, at, bt)
        ctx.packed, ctx.state, ctx.mask_scale, ctx.s = packed, state, mask_scale, s
        ctx.dtypes = (lora_a.dtype, lora_b.dtype)
        return y

    @staticmethod
    def backward(ctx, dy):
        x2d, keep, ht, at, bt = ctx.saved_tensors
        dy = dy.to(torch.float16).contiguous()
        dx, da, db = lora_backward(dy, x2d, keep, ht, at, bt, ctx.packed, ctx.state,
                                   ctx.mask_scale, ctx.s, want_x=ctx.needs_input_grad[0],
                                   want_a=ctx.needs_input_grad[1],
                                   want_b=ctx.needs_input_grad[2])
        if da is not None:
            da = da.to(ctx.dtypes[0])
        if db is not None:
            db = db.to(ctx.dtypes[1])
        return dx, da, db, None, None, None, None, None, None


class Proj:
    """What one projection's kernels need besides its LoRA tensors: the packed NF4 weight and its
    state, the fp16 bias, the u8 dropout keep mask (None without dropout), 1/(1-p) and the LoRA
    scaling."""

    __slots__ = ("packed", "state", "bias", "keep", "mask_scale", "s")

    def __init__(self, packed, state, bias, keep, mask_scale, s):
        self.packed, self.state, self.bias = packed, state, bias
        self.keep, self.mask_scale, self.s = keep, mask_scale, s


def siblings_ok(projs, K):
    """Whether NF4LoraSiblingsFunction takes these projections of one input width K: 2 to 4 of
    them, one LoRA scaling and one dropout rate (their row products share one launch), every
    weight within the grouped GEMM's 32-bit offsets."""
    return (2 <= len(projs) <= 4
            and len({(p.s, p.mask_scale) for p in projs}) == 1
            and all(p.state.shape[1] == K and p.state.shape[0] * K < 2 ** 32 for p in projs)
            and 128 * K * 2 < 2 ** 32)


class NF4LoraSiblingsFunction(torch.autograd.Function):
    """NF4 + LoRA projections that read the same input (a layer's q, k and v), computed with
    their launches shared: forward, one launch of LoRA row products (s * drop(x) A^T for each)
    and one launch of the fused GEMMs; backward, lora_backward_group (the dHs launches, the dX
    GEMMs with their dA / dB, shared where the plans allow) and dx = the sum of the projections'
    input gradients.  Each output equals NF4LoraFunction on its projection to within the GEMM
    tolerance (the grouped GEMM runs every problem on one tile plan).
    Inputs: x2d fp16 [M, K], `projs` (a tuple of Proj that siblings_ok accepts), one_gemm (the
    forward GEMMs in one grouped launch, else each on its own plan), rope (None, or
    (n_rope, cos, sin): the first n_rope outputs come rotated by the grouped GEMM, which needs
    one_gemm), then each projection's lora_A [r, K] and lora_B [N, r] (their gradients come
    back in their dtypes).
    Outputs: one fp16 [M, N_i] per projection.  The backward is that of the unrotated outputs
    whatever rope is: a rotated output's gradient must reach it rotated back (rope.RotatedHeads
    does that between this node and attention)."""

    @staticmethod
    def forward(ctx, x2d, projs, one_gemm, rope, *ab):
        n = len(projs)
        a16 = [t.to(torch.float16).contiguous() for t in ab[0::2]]
        b16 = [t.to(torch.float16).contiguous() for t in ab[1::2]]
        s, mask_scale = projs[0].s, projs[0].mask_scale
        keeps = [kernels.keep_bits(p.keep, x2d.shape[0], x2d.shape[1]) for p in projs]
        rows = kernels.lora_h_partials_group([x2d] * n, a16, s, keeps, mask_scale, b16)
        if rope is not None and not one_gemm:
            raise ValueError("the RoPE rides on the grouped GEMM (one_gemm)")
        if one_gemm:
            outs = kernels.nf4_linear_fwd_hp_group([x2d] * n, [p.packed for p in projs],
                                                   [p.state for p in projs],
                                                   [r[0] for r in rows], b16,
                                                   [p.bias for p in projs], rope=rope)
        elif n == 2 and kernels.fwd_pair_ok(x2d.shape[0], projs[0].state.shape[0],
                                            projs[1].state.shape[0], x2d.shape[1]):
            # gate and up: one launch (grid z selects the projection), the bits of two
            outs = kernels.nf4_linear_fwd_hp_pair(x2d, [p.packed for p in projs],
                                                  [p.state for p in projs], [r[0] for r in rows],
                                                  b16, [p.bias for p in projs])
        else:
            outs = [kernels.nf4_linear_fwd_hp(x2d, p.packed, p.state, r[0], b, p.bias)
                    for p, r, b in zip(projs, rows, b16)]
        ctx.save_for_backward(x2d, *keeps, *[o[1] for o in outs],
                              *[r[1] for r in rows], *[r[2] for r in rows])
        ctx.projs = projs
        ctx.dtypes = [t.dtype for t in ab]
        return tuple(o[0] for o in outs)

    @staticmethod
    def backward(ctx, *dys):
        projs = ctx.projs
        n = len(projs)
        saved = ctx.saved_tensors
        x2d = saved[0]
        keeps, hts, ats, bts = (saved[1 + i * n:1 + (i + 1) * n] for i in range(4))
        need = ctx.needs_input_grad
        items = []
        for i, p in enumerate(projs):
            dy = dys[i]
            if dy is None:
                dy = torch.zeros((x2d.shape[0], p.state.shape[0]), dtype=torch.float16,
                                 device=x2d.device)
            items.append(dict(dy=dy.to(torch.float16).contiguous(), x2d=x2d, keep=keeps[i],
                              ht=hts[i], at=ats[i], bt=bts[i], packed=p.packed, state=p.state,
                              mask_scale=p.mask_scale, s=p.s,
                              wants=(need[0], need[4 + 2 * i], need[5 + 2 * i])))
        res = lora_backward_group(items, sum_dx=True)
        dx = res[0][0] if need[0] else None
        grads = []
        for i, (_, da, db) in enumerate(res):
            grads += [None if da is None else da.to(ctx.dtypes[2 * i]),
                      None if db is None else db.to(ctx.dtypes[2 * i + 1])]
        return (dx, None, None, None, *grads)


class NF4LoraStreamFunction(NF4LoraFunction):
    """NF4LoraFunction for a base whose bytes live in host memory (stream.py): the slot's bytes
    are asked for right before the forward GEMM and again before the backward one, so the same
    kernels run on the same bytes as for a resident base."""

    @staticmethod
    def forward(ctx, x2d, lora_a, lora_b, module, state, bias, keep, mask_scale, s):
        packed, absmax = stream.bytes_for(module)
        y = NF4LoraFunction.forward(ctx, x2d, lora_a, lora_b, packed.view(-1, 1),
                                    stream.state_with(state, absmax), bias, keep, mask_scale, s)
        ctx.module, ctx.base_state = module, state
        ctx.packed = ctx.state = None  # the slot may hold another layer by the backward
        return y

    @staticmethod
    def backward(ctx, dy):
        packed, absmax = stream.bytes_for(ctx.module)
        ctx.packed, ctx.state = packed.view(-1, 1), stream.state_with(ctx.base_state, absmax)
        return NF4LoraFunction.backward(ctx, dy)


def linear_project(x, packed, state, bias):
    """NF4LinearFunction on a resident weight: the compiled op (torch.ops.mxs_nf4.linear, its
    backward in C++) when ops.ENABLED and the fused GEMM takes the shape, else the Python
    Function (which also holds the unpack-then-F.linear branch)."""
    if ops.ENABLED and _fused(state, x):
        return ops.linear(x, packed, state, bias)
    return direct.run(NF4LinearFunction, x, packed, state, bias)


def lora_project(x2d, lora_a, lora_b, packed, state, bias, keep, mask_scale, s):
    """NF4LoraFunction on a resident weight: torch.ops.mxs_nf4.lora_linear when ops.ENABLED,
    else the Python Function; the same kernels in the same order, so the same bits."""
    if ops.ENABLED:
        return ops.lora_linear(x2d, lora_a, lora_b, packed, state, bias, keep, mask_scale, s)
    return NF4LoraFunction.apply(x2d, lora_a, lora_b, packed, state, bias, keep, mask_scale, s)


def siblings_project(x2d, projs, lora_as, lora_bs, one_gemm=True, rope=None):
    """NF4LoraSiblingsFunction: torch.ops.mxs_nf4.lora_siblings when ops.ENABLED, else the
    Python Function.  Returns one fp16 [M, N_i] per projection.  rope = (n_rope, cos, sin):
    the first n_rope outputs come rotated (RoPE folded into the grouped GEMM), with the
    backward of the unrotated outputs (see NF4LoraSiblingsFunction)."""
    if ops.ENABLED:
        return ops.lora_siblings(x2d, projs, lora_as, lora_bs, one_gemm, rope)
    ab = [t for pair in zip(lora_as, lora_bs) for t in pair]
    return NF4LoraSiblingsFunction.apply(x2d, projs, bool(one_gemm), rope, *ab)


# ---------------------------------------------------------------------------------------------
# Modules
# ---------------------------------------------------------------------------------------------

def _direct_ok(layer, x, streamed=False):
    """When the HIP path takes a call (solution/linear4bit.py:112-129, without bitsandbytes'
    small-M kernel heuristic: the HIP path takes every token count).  With `streamed`, the same
    test for a weight whose bytes live in host memory (stream.offload), its size checked on the
    host copy; without it such a weight is refused (it takes the streamed branch)."""
    if not _enabled:
        return False
    weight = layer.weight
    if hasattr(weight, "_mindx_host") != streamed:
        return False
    state = getattr(weight, "quant_state", None)
    return (isinstance(x, torch.Tensor) and x.is_cuda and x.dtype == torch.float16
            and getattr(layer, "compute_type_is_set", False)
            and layer.compute_dtype == torch.float16
            and state is not None and getattr(state, "nested", False)
            and getattr(state, "state2", None) is not None
            and state.state2.blocksize == 256 and state.dtype == torch.float16
            and not getattr(state, "packing_format_for_cpu", False)
            and len(state.shape) == 2 and x.shape[-1] == state.shape[1] and x.numel() > 0
            and not weight.requires_grad
            and (layer.bias is None or not layer.bias.requires_grad)
            and (_host_size_ok(weight, state) if streamed else
                 _supported(weight.data, state.shape, state.blocksize, state.quant_type,
                            x.dtype, state.state2.blocksize)))


def _host_size_ok(weight, state):
    n, k = state.shape
    return (state.quant_type == "nf4" and state.blocksize == 64
            and weight._mindx_host.numel() * 2 == n * k)


def _cached_weight(layer, x):
    """The weight unpacked once to fp16 and kept (solution/linear4bit.py:132-148); None unless
    this call would take the direct path."""
    weight16 = layer.__dict__.get("_mindx_weight16")
    if weight16 is None:
        if not _direct_ok(layer, x):
            return None
        packed = layer.weight.data.view(-1, 1)
        weight16 = _unpack(packed, layer.weight.quant_state, torch.float16)
        layer.__dict__["_mindx_weight16"] = weight16
        return weight16
    if not (_enabled and isinstance(x, torch.Tensor) and x.is_cuda and x.dtype == torch.float16
            and x.numel() > 0 and x.shape[-1] == weight16.shape[1]):
        return None
    return weight16


def _cast_bias_once(layer, x):
    bias = layer.bias
    if bias is not None and bias.dtype != x.dtype:  # what Linear4bit.forward does, once
        bias.data = bias.data.to(x.dtype)
    return bias


def hip_forward(layer, x, original=None):
    """The patched Linear4bit.forward (solution/linear4bit.py:161-179): fp16 cache, then the
    streamed branch for offloaded weights, then the direct HIP path, else `original` (bitsandbytes' forward when patched onto it)."""
    if cache_fp16:
        weight16 = _cached_weight(layer, x)
        if weight16 is not None:
            return torch.nn.functional.linear(x, weight16, _cast_bias_once(layer, x))
    if isinstance(x, torch.Tensor) and x.is_cuda and stream.offloaded(layer):
        return _streamed_forward(layer, x)
    if not _direct_ok(layer, x):
        if original is None:
            raise ValueError("input not supported by the HIP NF4 path")
        return original(layer, x)
    bias = _cast_bias_once(layer, x)
    if bias is not None:
        bias = bias.to(layer.compute_dtype)
    packed = layer.weight.data.view(-1, 1)  # canonical [(N*K+1)//2, 1]
    return linear_project(x, packed, layer.weight.quant_state, bias)


class Linear4bit(torch.nn.Module):
    """Frozen NF4 linear layer with bitsandbytes' Linear4bit fields (weight.data = packed u8,
    weight.quant_state, bias, compute_dtype, compute_type_is_set) for when bitsandbytes is not
    installed.  Inputs the HIP path does not take (another dtype, CPU) are cast to the compute
    dtype and back, like bitsandbytes' own forward; CPU inputs raise."""

    def __init__(self, input_features, output_features, bias=True, compute_dtype=torch.float16,
                 device=None):
        super().__init__()
        self.in_features = input_features
        self.out_features = output_features
        self.compute_dtype = compute_dtype
        self.compute_type_is_set = True
        self.weight = None
        if bias:
            self.bias = torch.nn.Parameter(torch.zeros(output_features, dtype=torch.float16,
                                                       device=device), requires_grad=False)
        else:
            self.register_parameter("bias", None)

    @classmethod
    def from_weight(cls, weight, bias=None):
        """Quantize an fp16 CUDA weight [N, K] (NF4, blocksize 64, nested absmax)."""
        n, k = weight.shape
        layer = cls(k, n, bias=bias is not None, device=weight.device)
        packed, state = quantize_4bit(weight.to(torch.float16))
        layer.set_quantized(packed, state)
        if bias is not None:
            layer.bias.data = bias.detach().to(device=weight.device).clone()
        return layer

    def set_quantized(self, packed, state):
        w = torch.nn.Parameter(packed.view(-1, 1), requires_grad=False)
        w.quant_state = state
        self.weight = w

    def _apply(self, fn, recurse=True):
        """Module.to / .cuda move the packed bytes; the quant state (an attribute of the weight
        parameter) follows them."""
        super()._apply(fn, recurse)
        state = getattr(self.weight, "quant_state", None)
        if state is not None and state.absmax.device != self.weight.device:
            self.weight.quant_state = state.to(self.weight.device)
        return self

    # bitsandbytes' state-dict form (nn/modules.py Linear4bit._save_to_state_dict): the packed
    # bytes under "weight", the quant state's as_dict(packed=True) under "weight.<key>", bias.
    # An offloaded weight (stream.offload) writes its host copies, not the device placeholders.
    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        w = self.weight
        state = getattr(w, "quant_state", None)
        if state is None:
            return
        qs = state.as_dict(packed=True)
        if hasattr(w, "_mindx_host"):
            destination[prefix + "weight"] = w._mindx_host.view(w._mindx_shape)
            qs["absmax"] = w._mindx_absmax.view(state.absmax.shape)
        for k, v in qs.items():
            destination[prefix + "weight." + k] = v if keep_vars else v.detach()

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        key = prefix + "weight"
        qs = {k: v for k, v in state_dict.items() if k.startswith(key + ".")}
        if key not in state_dict:
            if strict:
                missing_keys.append(key)
            return
        dev = self.weight.device if self.weight is not None else state_dict[key].device
        try:
            state = QuantState.from_dict({k[len(key) + 1:]: v for k, v in qs.items()}, dev)
        except (ValueError, NotImplementedError, KeyError) as e:
            error_msgs.append(f"{key}: {e}")
            return
        self.set_quantized(state_dict[key].to(dev).view(-1, 1), state)
        b = prefix + "bias"
        if self.bias is not None:
            if b in state_dict:
                self.bias.data = state_dict[b].to(device=dev, dtype=self.bias.dtype).clone()
            elif strict:
                missing_keys.append(b)
        elif b in state_dict and strict:
            unexpected_keys.append(b)

    def forward(self, x):
        if isinstance(x, torch.Tensor) and x.is_cuda and stream.offloaded(self):
            return _streamed_forward(self, x)
        if _direct_ok(self, x):
            return hip_forward(self, x)
        return _generic_forward(self, x)


def _generic_forward(layer, x):
    """Any other input on the GPU: to the compute dtype, the HIP path, back to the input dtype."""
    if not x.is_cuda:
        raise ValueError("the NF4 HIP path needs a GPU tensor")
    inp_dtype = x.dtype
    x16 = x.to(layer.compute_dtype)
    state = layer.weight.quant_state
    bias = layer.bias.to(layer.compute_dtype) if layer.bias is not None else None
    packed = layer.weight.data.view(-1, 1)
    return linear_project(x16, packed, state, bias).to(inp_dtype)


class LoraLinear4bit(torch.nn.Module):
    """peft's lora.bnb.Linear4bit layout around a 4-bit base: base_layer, lora_A / lora_B /
    lora_dropout as ModuleDicts keyed by adapter name, scaling dict, active_adapters, merged,
    disable_adapters.  forward = base(x) + s * B(A(drop(x))) (solution/test_unpad.py:28-29),
    fused into the NF4 kernels when FUSED_LORA and the shapes allow it."""

    def __init__(self, base_layer, r=16, lora_alpha=32, lora_dropout=0.05, adapter="default"):
        super().__init__()
        self.base_layer = base_layer
        k, n = base_layer.in_features, base_layer.out_features
        dev = base_layer.weight.device
        self.r = {adapter: r}
        self.lora_alpha = {adapter: lora_alpha}
        self.scaling = {adapter: lora_alpha / r}
        self.lora_A = torch.nn.ModuleDict(
            {adapter: torch.nn.Linear(k, r, bias=False, device=dev)})
        self.lora_B = torch.nn.ModuleDict(
            {adapter: torch.nn.Linear(r, n, bias=False, device=dev)})
        self.lora_dropout = torch.nn.ModuleDict(
            {adapter: torch.nn.Dropout(lora_dropout) if lora_dropout > 0 else torch.nn.Identity()})
        torch.nn.init.kaiming_uniform_(self.lora_A[adapter].weight, a=math.sqrt(5))
        torch.nn.init.zeros_(self.lora_B[adapter].weight)
        self.active_adapters = [adapter]
        self.merged = False
        self.disable_adapters = False
        self.next_keep = None  # optional u8 keep mask for the next training forward (tests)

    def _adapter(self):
        if self.disable_adapters or self.merged or len(self.active_adapters) != 1:
            return None
        return self.active_adapters[0]

    def forward(self, x):
        from . import peft_lora

        return peft_lora.lora_forward(self, x, _composed_lora)


def _composed_lora(layer, x):
    """base(x) + s * B(A(drop(x))) as separate torch operations (peft's own composition), for
    inputs or layers the fused path does not take."""
    name = layer._adapter()
    base = layer.base_layer
    if name is None:
        return base(x)
    a = layer.lora_A[name].weight.to(x.dtype)
    b = layer.lora_B[name].weight.to(x.dtype)
    h = layer.lora_dropout[name](x)
    return base(x) + (h @ a.t() @ b.t()) * layer.scaling[name]


def patch_bnb_linear4bit(cache_weights=False):
    """Install the HIP forward on bitsandbytes.nn.Linear4bit (solution/linear4bit.py:151-182)
    when bitsandbytes is importable; returns whether it did."""
    global cache_fp16
    cache_fp16 = cache_weights
    try:
        import bitsandbytes as bnb
    except Exception:
        return False
    cls = bnb.nn.Linear4bit
    if getattr(cls, "_mindx_direct", False):
        return True
    original = cls.forward

    def forward(self, x):
        return hip_forward(self, x, original)

    cls.forward = forward
    cls._mindx_direct = True
    return True
