"""Benchmark of the NF4 hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Headline: standalone NF4 dequant of all 28 layers x 7 projections
of Qwen2.5-1.5B (q/o [1536,1536], k/v [256,1536], gate/up [8960,1536], down [1536,8960]), NF4
at blocksize 64 with double-quantized absmax, decoded to fp16 by one launch over the whole model
(the weights back to back in HBM, as the reference's layer unpack stores them).  A step is that
one launch; `value` is GB/s over the algorithmic bytes: packed + absmax8 + absmax2 + fp16 out =
3 296 280 960 B per step.  Inputs are resident in HBM before timing.

Also reported under "fused_stack" (not the headline): the fused NF4+LoRA projections of BASELINE
configs[2] (gate+up forward), configs[3] (down_proj backward) and configs[4] (all 196
projections forward + backward at M = 1024, captured as one HIP graph per step), in TFLOP/s
against the dense fp16 MFMA peak; and CPU baselines timed on this host (the oracle's C decode
with OpenMP; for the GEMMs, one layer with torch CPU fp32 GEMMs).  Prints ONE JSON line.
"""

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

LAYERS = 28
# (name, out_features N, in_features K) of one Qwen2.5-1.5B decoder layer
PROJ = [("q", 1536, 1536), ("k", 256, 1536), ("v", 256, 1536), ("o", 1536, 1536),
        ("gate", 8960, 1536), ("up", 8960, 1536), ("down", 1536, 8960)]
HBM_PEAK_GBS = 8000.0


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "nf4_dequant_model_traffic.txt")


def measured_traffic(path=TRAFFIC_FILE):
    """HBM bytes per launch of the dequant kernel, from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel calibration); None without it."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def calibrate(dev, nbytes=1 << 30, reps=5):
    """A plain device-to-device copy of known size, for scaling the PMC byte counters: each of
    the `reps` copy launches reads nbytes and writes nbytes."""
    src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / reps * 1e3
    print(json.dumps({"calibration": "copy", "bytes_read_per_launch": nbytes,
                      "bytes_written_per_launch": nbytes, "launches": reps,
                      "ms_per_launch": round(ms, 4),
                      "gbs": round(2 * nbytes / ms / 1e6, 1)}), flush=True)


def model_weights(dev, seed=0):
    """All 196 NF4 weights back to back: N(0, 0.02) fp16 quantized on the GPU."""
    from mindxsoup_amd.quant import quantize_4bit

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    parts = []
    for _ in range(LAYERS):
        for _, n, k in PROJ:
            w = (torch.randn((n, k), device=dev, generator=g) * 0.02).half()
            packed, st = quantize_4bit(w)
            st.absmax_f32 = None
            parts.append((packed.view(-1), st))
            del w
    packed = torch.cat([p for p, _ in parts])
    absmax8 = torch.cat([s.absmax for _, s in parts])
    code = torch.cat([s.state2.code for _, s in parts])
    absmax2 = torch.cat([s.state2.absmax for _, s in parts])
    offset = torch.stack([s.offset for _, s in parts])
    nb = np.array([s.absmax.numel() for _, s in parts])
    ng = np.array([s.state2.absmax.numel() for _, s in parts])
    block0 = torch.tensor(np.concatenate([[0], np.cumsum(nb)]), dtype=torch.int64, device=dev)
    scale0 = torch.tensor(np.concatenate([[0], np.cumsum(ng)[:-1]]), dtype=torch.int64,
                          device=dev)
    del parts
    return dict(packed=packed, absmax8=absmax8, code=code, absmax2=absmax2, offset=offset,
                block0=block0, scale0=scale0, nb=nb, ng=ng)


def dequant_bytes(m):
    return (m["packed"].numel() + m["absmax8"].numel() + 4 * m["absmax2"].numel()
            + 2 * 64 * m["absmax8"].numel())


def bench_dequant(m, steps, warmup):
    from mindxsoup_amd.nf4 import launch_layer, layer_plan

    out = torch.empty(m["packed"].numel() * 2, dtype=torch.float16, device=m["packed"].device)
    plan = layer_plan(m["block0"])  # once, outside the timed steps

    def step():
        launch_layer(m["packed"], out, m["absmax8"], m["code"], m["absmax2"], m["offset"], None,
                     m["block0"], m["scale0"], plan)

    for _ in range(warmup):
        step()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in ev:
        a.record(stream)
        step()
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_launch = [a.elapsed_time(b) for a, b in ev]
    return wall / steps * 1e3, float(np.mean(per_launch)), out


def hbm_ceiling(packed, out, steps, warmup):
    """What HBM delivers on this part (mxs_hbm_probe in libmxs_probe.so), timed like the
    dequant: pure 16-byte load and store streams over the output's bytes, and the dequant's
    access pattern without its arithmetic (4-byte non-temporal loads of the packed bytes,
    16-byte non-temporal stores over the fp16 output: 20 % reads, 80 % writes).  GB/s over the bytes each launch moves."""
    from mindxsoup_amd import _lib

    n = packed.numel() // 4             # dword chunks of the packed bytes
    m = out.numel() * out.element_size() // 16  # 16-byte chunks of the output
    sink = torch.empty(((m + 1023) // 1024) * 4, dtype=torch.int32, device=out.device)
    cases = {"pattern": (0, packed, out, n, 20 * n),
             "load_only": (1, out, sink, m, 16 * m),
             "store_only": (2, None, out, m, 16 * m)}
    stream = torch.cuda.current_stream()
    res = {}
    for name, (kind, src, dst, chunks, nbytes) in cases.items():
        def launch():
            _lib.hbm_probe(kind, _lib.ptr(src), _lib.ptr(dst), chunks,
                           _lib.stream_of(dst.device))

        for _ in range(warmup):
            launch()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(steps):
            launch()
        b.record(stream)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / steps
        res[name] = {"GBps": round(nbytes / ms / 1e6, 1), "bytes": nbytes,
                     "ms": round(ms, 4)}
    return res


# The GPU box gives one GPU's job a share of 16 host cores (its OMP_NUM_THREADS), whatever its
# affinity set shows; more threads would only oversubscribe that share.
CPU_SHARE = 16


def host_cores():
    """Threads for the CPU baselines: the cores this process may run on, at most the job's
    share (both counts are reported with the baseline)."""
    return min(len(os.sched_getaffinity(0)), CPU_SHARE)


def cpu_baseline_dequant(m, budget_s=20.0):
    """The oracle's C decode (OpenMP) over the same packed weights, on this host: whole-model
    passes, repeated within the time budget; median."""
    from oracle import oracle as O

    cores = host_cores()
    O.set_num_threads(cores)
    packed = m["packed"].cpu().numpy()
    absmax8 = m["absmax8"].cpu().numpy()
    code = m["code"].cpu().numpy().reshape(-1, 256)
    absmax2 = m["absmax2"].cpu().numpy()
    offset = m["offset"].cpu().numpy()
    nb, ng = m["nb"], m["ng"]
    b0 = np.concatenate([[0], np.cumsum(nb)])
    g0 = np.concatenate([[0], np.cumsum(ng)])
    n_w = len(nb)

    def one_pass(n_weights):
        for i in range(n_weights):
            O.dequant(packed=packed[32 * b0[i]:32 * b0[i + 1]], absmax8=absmax8[b0[i]:b0[i + 1]],
                      code=code[i], absmax2=absmax2[g0[i]:g0[i + 1]], offset=float(offset[i]))

    one_pass(7)  # warm-up: one layer
    times = []
    start = time.perf_counter()
    while True:
        t = time.perf_counter()
        one_pass(n_w)
        times.append(time.perf_counter() - t)
        if time.perf_counter() - start > budget_s or len(times) >= 5:
            break
    sec = float(np.median(times))
    return dict(value=round(dequant_bytes(m) / sec / 1e9, 3), unit="GB/s", cores=cores,
                cores_available=len(os.sched_getaffinity(0)), cpu_count=os.cpu_count(),
                kind="port",
                sample=f"whole model (196 weights) decoded by oracle/nf4_oracle.c, "
                       f"median of {len(times)} passes, {sec:.3f} s/pass, "
                       f"torch threads {torch.get_num_threads()}")


# ---------------------------------------------------------------------------------------------
# Fused NF4 + LoRA projections (BASELINE configs[2..4])
# ---------------------------------------------------------------------------------------------
M_TOKENS, RANK, ALPHA, P_DROP = 1024, 16, 32, 0.05
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, MI355X spec


def proj_flops(n, k, m=M_TOKENS, r=RANK, fwd=True, bwd=True):
    """Algorithmic FLOPs of one NF4+LoRA projection: base 2MNK per direction; LoRA forward
    2Mr(K+N) (H and its product with B), backward 4Mr(K+N) (dH, dX_lora, dA, dB)."""
    f = 0
    if fwd:
        f += 2 * m * n * k + 2 * m * r * (k + n)
    if bwd:
        f += 2 * m * n * k + 4 * m * r * (k + n)
    return f


def make_proj(dev, g, n, k, x=None, x_kind="normal", dy_std=1.0):
    """One projection's synthetic inputs: NF4 weight N(0,0.02), LoRA A Kaiming-uniform, B
    N(0,0.01), fp16; X [M,K] ~ N(0,1) (or silu(g)*u), dY ~ N(0, dy_std); keep mask Bernoulli(0.95)."""
    from mindxsoup_amd import kernels
    from mindxsoup_amd.quant import quantize_4bit

    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).half()
    packed, st = quantize_4bit(w)
    st.absmax_f32 = None
    del w
    if x is None:
        if x_kind == "silu_mul":
            a_ = torch.randn((M_TOKENS, k), device=dev, generator=g)
            b_ = torch.randn((M_TOKENS, k), device=dev, generator=g)
            x = (torch.nn.functional.silu(a_) * b_).half()
        else:
            x = torch.randn((M_TOKENS, k), device=dev, generator=g).half()
    bound = 1.0 / np.sqrt(k)
    la = ((torch.rand((RANK, k), device=dev, generator=g) * 2 - 1) * bound).half()
    lb = (torch.randn((n, RANK), device=dev, generator=g) * 0.01).half()
    dy = (torch.randn((M_TOKENS, n), device=dev, generator=g) * dy_std).half()
    keep8 = (torch.rand((M_TOKENS, k), device=dev, generator=g) >= P_DROP).to(torch.uint8)
    # the kernels' mask format: keep bits, drawn (packed) before any timing like x and dy
    keep = kernels.keep_bits(keep8, M_TOKENS, k)
    return dict(packed=packed, st=st, x=x, a=la, b=lb, dy=dy, keep=keep, keep8=keep8, n=n, k=k,
                ws=shared_workspace(dev))


_WS = {}


def shared_workspace(dev):
    """One workspace for every projection's kernels (they run in stream order), allocated before
    any graph capture."""
    from mindxsoup_amd import kernels

    if dev not in _WS:
        need = max(kernels.projection_workspace_bytes(M_TOKENS, k, n, RANK) for _, n, k in PROJ)
        _WS[dev] = kernels.new_workspace(need, dev)
    return _WS[dev]


def proj_fwd(p, s=ALPHA / RANK):
    from mindxsoup_amd import kernels

    hp, at, bt = kernels.lora_h_partials(p["x"], p["a"], s, p["keep"], 1.0 / (1.0 - P_DROP),
                                         lora_b=p["b"])
    y, ht = kernels.nf4_linear_fwd_hp(p["x"], p["packed"], p["st"], hp, p["b"], ws=p["ws"])
    return y, (ht, at, bt)


def proj_bwd(p, saved, s=ALPHA / RANK):
    from mindxsoup_amd.linear4bit import lora_backward

    ht, at, bt = saved
    return lora_backward(p["dy"], p["x"], p["keep"], ht, at, bt, p["packed"], p["st"],
                         1.0 / (1.0 - P_DROP), s, ws=p["ws"])


# Projections of one layer whose LoRA row products share a launch (indices into PROJ): forward,
# those reading the same activations (q/k/v; gate/up); backward, those whose output gradients
# the model produces together (q/k/v from attention's backward, gate/up from the SwiGLU's).
FWD_GROUPS = [(0, 1, 2), (3,), (4, 5), (6,)]
BWD_GROUPS = [(6,), (5, 4), (3,), (2, 1, 0)]
# Projections over one input, whose input gradients a model adds: each group's sum comes from
# one summed launch (q/k/v: one tile loop over the three reductions, their dA / dB in the same
# launch; gate/up: split-K planes of both reductions and one reduce)
SUM_DX_GROUPS = [(5, 4), (2, 1, 0)]


def layer_fwd(projs, s=ALPHA / RANK):
    """Forward of one layer's 7 projections: grouped LoRA row products, then each fused GEMM.
    Returns (ys, saved): each projection's output and what its backward needs."""
    from mindxsoup_amd import kernels

    ys = [None] * len(projs)
    saved = [None] * len(projs)
    for grp in FWD_GROUPS:
        ps = [projs[i] for i in grp]
        if len(ps) == 1:
            ys[grp[0]], saved[grp[0]] = proj_fwd(ps[0], s)
            continue
        outs = kernels.lora_h_partials_group([p["x"] for p in ps], [p["a"] for p in ps], s,
                                             [p["keep"] for p in ps], 1.0 / (1.0 - P_DROP),
                                             [p["b"] for p in ps])
        if grp == (0, 1, 2):  # q, k, v: one GEMM launch (k and v alone would plan split-K)
            res = kernels.nf4_linear_fwd_hp_group([p["x"] for p in ps],
                                                  [p["packed"] for p in ps],
                                                  [p["st"] for p in ps], [o[0] for o in outs],
                                                  [p["b"] for p in ps])
            for i, (_, at, bt), (y, ht) in zip(grp, outs, res):
                ys[i], saved[i] = y, (ht, at, bt)
            continue
        if len(ps) == 2 and kernels.fwd_pair_ok(M_TOKENS, ps[0]["n"], ps[1]["n"], ps[0]["k"]):
            # gate and up over one input: one launch (grid z selects the projection)
            res = kernels.nf4_linear_fwd_hp_pair(ps[0]["x"], [p["packed"] for p in ps],
                                                 [p["st"] for p in ps], [o[0] for o in outs],
                                                 [p["b"] for p in ps])
            for i, (_, at, bt), (y, ht) in zip(grp, outs, res):
                ys[i], saved[i] = y, (ht, at, bt)
            continue
        for i, p, (hp, at, bt) in zip(grp, ps, outs):
            ys[i], ht = kernels.nf4_linear_fwd_hp(p["x"], p["packed"], p["st"], hp, p["b"],
                                                  ws=p["ws"])
            saved[i] = (ht, at, bt)
    return ys, saved


def layer_bwd(projs, saved, s=ALPHA / RANK):
    """Backward of one layer's 7 projections in reverse order; each group's small launches
    (dHs, dA / dB) and the v/k/q dX GEMMs shared, gate's and up's dX summed by one launch
    (linear4bit.lora_backward_group).  Returns each projection's (dX, dA, dB) (up's dX is the
    sum, gate's None)."""
    from mindxsoup_amd.linear4bit import lora_backward_group

    grads = [None] * len(projs)
    for grp in BWD_GROUPS:
        res = lora_backward_group([dict(dy=projs[i]["dy"], x2d=projs[i]["x"],
                                        keep=projs[i]["keep"], ht=saved[i][0], at=saved[i][1],
                                        bt=saved[i][2], packed=projs[i]["packed"],
                                        state=projs[i]["st"], mask_scale=1.0 / (1.0 - P_DROP),
                                        s=s, wants=(True, True, True)) for i in grp],
                                  ws=projs[grp[0]]["ws"], sum_dx=grp in SUM_DX_GROUPS)
        for i, r in zip(grp, res):
            grads[i] = r
    return grads


class AutogradLayer:
    """One layer's projections as a training step sees them: the four activations (q/k/v's,
    o's, gate/up's, down's) as leaves that need their gradient, fp32 LoRA weights (peft keeps
    them in fp32) and each projection's Proj record (packed weight, state, keep mask)."""

    def __init__(self, projs, s=ALPHA / RANK):
        from mindxsoup_amd.linear4bit import Proj

        self.projs = projs
        self.x = {i: projs[i]["x"].detach().requires_grad_(True) for i in (0, 3, 4, 6)}
        self.a = [p["a"].float().requires_grad_(True) for p in projs]
        self.b = [p["b"].float().requires_grad_(True) for p in projs]
        self.rec = [Proj(p["packed"], p["st"], None, p["keep"], 1.0 / (1.0 - P_DROP), s)
                    for p in projs]
        self.dys = [p["dy"] for p in projs]
        self.leaves = [*self.x.values(), *self.a, *self.b]

    def forward(self):
        """The 7 outputs in PROJ order: q/k/v in one siblings node (one grouped GEMM launch),
        o, gate/up in one siblings node (each GEMM on its own plan), down."""
        from mindxsoup_amd import linear4bit

        r, a, b = self.rec, self.a, self.b
        qkv = linear4bit.siblings_project(self.x[0], r[0:3], a[0:3], b[0:3], one_gemm=True)
        o = linear4bit.lora_project(self.x[3], a[3], b[3], r[3].packed, r[3].state, None,
                                    r[3].keep, r[3].mask_scale, r[3].s)
        gu = linear4bit.siblings_project(self.x[4], r[4:6], a[4:6], b[4:6], one_gemm=False)
        down = linear4bit.lora_project(self.x[6], a[6], b[6], r[6].packed, r[6].state, None,
                                       r[6].keep, r[6].mask_scale, r[6].s)
        return [*qkv, o, *gu, down]


def autograd_step(alayers):
    """Forward of every layer through the autograd ops, then one torch.autograd.grad over all
    outputs: every input and LoRA weight gradient, as a training step's backward makes them."""
    outs, dys, leaves = [], [], []
    for L in alayers:
        outs += L.forward()
        dys += L.dys
        leaves += L.leaves
    return torch.autograd.grad(outs, leaves, dys)


def stack_layers(dev, g):
    """The 28 layers' projections: q/k/v share one activation, gate/up
    another, o and down have their own; inputs resident before any timing."""
    layers = []
    for _ in range(LAYERS):
        x_attn = torch.randn((M_TOKENS, 1536), device=dev, generator=g).half()
        x_mlp = torch.randn((M_TOKENS, 1536), device=dev, generator=g).half()
        projs = []
        for name, n, k in PROJ:
            x = x_attn if name in ("q", "k", "v") else x_mlp if name in ("gate", "up") else None
            projs.append(make_proj(dev, g, n, k, x=x))
        layers.append(projs)
    torch.cuda.synchronize()
    print("bench: projection stack inputs resident", file=sys.stderr, flush=True)
    return layers


def stack_step(layers):
    """One step of the stack: every layer's forward, then every layer's backward in reverse."""
    def step():
        saved = []
        for projs in layers:
            saved.append(layer_fwd(projs)[1])
        for projs, hts in zip(reversed(layers), reversed(saved)):
            layer_bwd(projs, hts)
    return step


def graph_time(fn, steps, warmup):
    """Capture fn() in a HIP graph, replay: mean ms per replay (events on the capture stream's
    replay stream) and the wall-clock mean."""
    fn()  # eager warm-up (first launches set kernel attributes)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record(stream)
    for _ in range(steps):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps * 1e3
    return a.elapsed_time(b) / steps, wall


def eager_time(fn, steps, warmup):
    """fn() launched eagerly (no graph): mean ms per call between HIP events on the current
    stream, and the host's own ms per call (wall time of the Python calls alone, before the
    final synchronize: the cost of argument checks, allocations and launches)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    host = (time.perf_counter() - t0) / steps * 1e3
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps, host


def bench_mlp(dev, g, steps, warmup):
    """One Qwen2 MLP block (gate, up, down with LoRA r=16, dropout 0.05; SwiGLU) forward +
    backward through autograd at M = 1024, one HIP graph per step: the SwiGLU fused into the
    up/down GEMM epilogues (mlp.NF4LoraMLPFunction) against the reference's composition of the
    three projections and silu_mul (solution/mlp.py:42-44) over the same kernels."""
    from mindxsoup_amd import mlp as mlp_mod
    from mindxsoup_amd.linear4bit import Linear4bit, LoraLinear4bit

    layers = []
    for n, k in ((8960, 1536), (8960, 1536), (1536, 8960)):
        w = (torch.randn((n, k), device=dev, generator=g) * 0.02).half()
        m = LoraLinear4bit(Linear4bit.from_weight(w, None), r=RANK, lora_alpha=ALPHA,
                           lora_dropout=P_DROP)
        del w
        with torch.no_grad():
            m.lora_B["default"].weight.normal_(0.0, 0.01, generator=g)
        layers.append(m)
    block = mlp_mod.MLP(*layers).train()
    x = torch.randn((M_TOKENS, 1536), device=dev, generator=g).half().requires_grad_(True)
    dy = torch.randn((M_TOKENS, 1536), device=dev, generator=g).half()
    if not mlp_mod.fused_ok(block, x):
        raise RuntimeError("the fused MLP path does not take the model's shapes")

    def step():
        block(x).backward(dy)

    res = {}
    previous = mlp_mod.FUSED_SWIGLU
    try:
        for key, fused in (("unfused_ms", False), ("fused_ms", True)):
            mlp_mod.FUSED_SWIGLU = fused
            ms, _ = graph_time(step, steps, warmup)
            res[key] = round(ms, 4)
    finally:
        mlp_mod.FUSED_SWIGLU = previous
    fl = 2 * proj_flops(8960, 1536) + proj_flops(1536, 8960)
    res["gflop"] = round(fl / 1e9, 3)
    res["tflops"] = round(fl / res["fused_ms"] / 1e9, 1)
    res["saved_ms"] = round(res["unfused_ms"] - res["fused_ms"], 4)
    res["kernels_us"] = swiglu_kernel_times(block, x, dy, steps, warmup)
    del block, layers, x, dy
    return res


def swiglu_kernel_times(block, x, dy, steps, warmup):
    """The SwiGLU's kernels alone at the block's shapes (us per launch, 20 launches per graph
    replay): up_proj's forward GEMM plain and with the SwiGLU tail, and the elementwise kernel;
    down_proj's dX GEMM plain and with the adjoint tail, and the elementwise backward."""
    from mindxsoup_amd import kernels

    s, ms_ = ALPHA / RANK, 1.0 / (1.0 - P_DROP)
    up, down = block.up_proj, block.down_proj
    pu, su = up.base_layer.weight.data.view(-1, 1), up.base_layer.weight.quant_state
    pd, sd = down.base_layer.weight.data.view(-1, 1), down.base_layer.weight.quant_state
    a_u = up.lora_A["default"].weight.half()
    b_u = up.lora_B["default"].weight.half()
    b_d = down.lora_B["default"].weight.half()
    a_d = down.lora_A["default"].weight.half()
    xs = x.detach()
    M = xs.shape[0]
    gate = torch.randn((M, 8960), device=xs.device).half()
    upv = torch.randn((M, 8960), device=xs.device).half()
    keep = kernels.keep_bits((torch.rand((M, 8960), device=xs.device) >= P_DROP).to(torch.uint8),
                             M, 8960)
    hp, _, _ = kernels.lora_h_partials(xs, a_u, s, None, 1.0, lora_b=b_u)
    at_d, bt_d = a_d.t().contiguous(), b_d.t().contiguous()
    dhp = kernels.lora_dh_partials(dy, bt_d, s)
    y0, _ = kernels.nf4_linear_fwd_hp(xs, pu, su, hp, b_u)
    dh0, _ = kernels.nf4_linear_bwd_dx_hp(dy, pd, sd, dhp, at_d, keep, ms_)
    g2, u2 = gate.clone(), upv.clone()
    cases = {
        "up_fwd_gemm": lambda: kernels.nf4_linear_fwd_hp(xs, pu, su, hp, b_u),
        "up_fwd_gemm_swiglu": lambda: kernels.nf4_linear_fwd_glu(xs, pu, su, gate, hp, b_u),
        "silu_mul": lambda: kernels.silu_mul(gate, y0),
        "down_dx_gemm": lambda: kernels.nf4_linear_bwd_dx_hp(dy, pd, sd, dhp, at_d, keep, ms_),
        "down_dx_gemm_swiglu": lambda: kernels.nf4_linear_bwd_dx_glu_(dy, pd, sd, g2, u2, dhp,
                                                                      at_d, keep, ms_),
        "silu_mul_bwd": lambda: kernels.silu_mul_bwd_(dh0, g2, u2),
    }
    reps = 20
    out = {}
    for name, fn in cases.items():
        ms, _ = graph_time(lambda: [fn() for _ in range(reps)], max(3, steps // 10),
                           max(2, warmup // 5))
        out[name] = round(ms * 1e3 / reps, 2)
    return out


def bench_qkv_rope(dev, g, steps, warmup):
    """The q/k/v LoRA-add + RoPE + cast kernel (mxs_qkv_rope) at one layer of the model, 1024
    tokens (12 q heads, 2 k/v heads of 128): forward with the projections' LoRA outputs added
    (the reference's call, solution/attention.py:271-276) and without (LoRA already inside the
    fused projections: q and k rotated, v passed through), and the backward (dq, dk rotated
    back, dv copied).  HBM-bound: GB/s over the bytes each launch must move."""
    from mindxsoup_amd import kernels

    T, nq, nkv, D = M_TOKENS, 12, 2, 128

    def t(h):
        return torch.randn((1, T, h * D), device=dev, generator=g).half()

    def heads(x, h):
        return x.view(1, T, h, D).transpose(1, 2)

    qa, qb, k, va, vb = t(nq), t(nq), t(nkv), t(nkv), t(nkv)
    pos = torch.arange(T, device=dev, dtype=torch.float32)
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    emb = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], dim=-1)[None]
    cos, sin = emb.cos().contiguous(), emb.sin().contiguous()
    qo, ko, vo = t(nq), t(nkv), t(nkv)
    cs = 2 * T * D * 4  # cos + sin rows read per launch
    cases = {
        "fwd_lora_add": ((heads(qa, nq), heads(qb, nq), heads(k, nkv), heads(va, nkv),
                          heads(vb, nkv)), False, T * D * 2 * (2 * nq + nkv + 2 * nkv) + cs
                         + T * D * 2 * (nq + 2 * nkv)),
        "fwd_fused_lora": ((heads(qa, nq), None, heads(k, nkv), None, None), False,
                           T * D * 2 * 2 * (nq + nkv) + cs),
        "bwd": ((heads(qa, nq), None, heads(k, nkv), heads(va, nkv), None), True,
                T * D * 2 * 2 * (nq + 2 * nkv) + cs),
    }
    reps = 20
    res = {}
    for name, (ins, bwd, nbytes) in cases.items():
        outs = (heads(qo, nq), heads(ko, nkv), heads(vo, nkv) if ins[3] is not None else None)

        def fn():
            for _ in range(reps):
                kernels.qkv_rope(*ins, cos, sin, *outs, backward=bwd, q_scale=2.0, v_scale=2.0)

        ms, _ = graph_time(fn, max(3, steps // 10), max(2, warmup // 5))
        us = ms * 1e3 / reps
        res[name] = {"us": round(us, 2), "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1),
                     "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 3)}
    res["qkv_proj"] = bench_qkv_fold(dev, g, steps, warmup, cos, sin)
    return res


def bench_qkv_fold(dev, g, steps, warmup, cos, sin):
    """The attention path's q/k/v forward at 1024 tokens (q 1536, k and v 256 over K = 1536,
    LoRA partials and bias): the grouped GEMM followed by the rotation launch, against the
    grouped GEMM with the rotation in its epilogue (the same bits).  Four weight sets rotated
    so the weights come from HBM; us per layer."""
    from mindxsoup_amd import kernels

    s, T = ALPHA / RANK, M_TOKENS
    sets = []
    for _ in range(4):
        ps = [make_proj(dev, g, n, 1536) for n in (1536, 256, 256)]
        x = ps[0]["x"]
        hps = [o[0] for o in kernels.lora_h_partials_group([x] * 3, [p["a"] for p in ps], s,
                                                           None, 1.0, [p["b"] for p in ps])]
        bias = [(torch.randn((p["n"],), device=dev, generator=g) * 0.1).half() for p in ps]
        qo = torch.empty((1, T, 1536), device=dev, dtype=torch.float16)
        ko = torch.empty((1, T, 256), device=dev, dtype=torch.float16)
        sets.append((x, ps, hps, bias, qo, ko))

    def heads(y, h):
        return y.view(1, T, h, 128).transpose(1, 2)

    def apart():
        for x, ps, hps, bias, qo, ko in sets:
            out = kernels.nf4_linear_fwd_hp_group([x] * 3, [p["packed"] for p in ps],
                                                  [p["st"] for p in ps], hps,
                                                  [p["b"] for p in ps], bias)
            kernels.qkv_rope(heads(out[0][0], 12), None, heads(out[1][0], 2), None, None, cos,
                             sin, heads(qo, 12), heads(ko, 2), None)

    def folded():
        for x, ps, hps, bias, _, _ in sets:
            kernels.nf4_linear_fwd_hp_group([x] * 3, [p["packed"] for p in ps],
                                            [p["st"] for p in ps], hps, [p["b"] for p in ps],
                                            bias, rope=(2, cos, sin))

    res = {}
    for name, fn in (("gemm_then_rope_us", apart), ("gemm_rope_fused_us", folded)):
        ms, _ = graph_time(fn, max(3, steps // 10), max(2, warmup // 5))
        res[name] = round(ms * 1e3 / len(sets), 2)
    return res


PCIE_PEAK_GBS = 63.0  # PCIe Gen5 x16, one direction, after 128b/130b encoding


def bench_stream(dev, g, steps, warmup, n_layers=4):
    """Host-streamed decoder weights (mindxsoup_amd/stream.py): a stack of n_layers decoder
    layers of the model's seven NF4 projections, X [1024, 1536] fp16, forward + backward
    (input gradients), with the weights resident in HBM, streamed through 2 device slots (the
    fused GEMMs read the slot), and streamed with the running layer decoded by one launch.
    Wall clock per step (the streamer's host logic and copies included), and one layer's
    pinned host -> device copy on the copy stream against PCIe's peak."""
    from mindxsoup_amd import stream
    from mindxsoup_amd.linear4bit import Linear4bit

    shapes = {"q_proj": (1536, 1536), "k_proj": (256, 1536), "v_proj": (256, 1536),
              "o_proj": (1536, 1536), "gate_proj": (8960, 1536), "up_proj": (8960, 1536),
              "down_proj": (1536, 8960)}

    class Layer(torch.nn.Module):
        def __init__(self):
            super().__init__()
            for name, (n, k) in shapes.items():
                w = torch.randn(n, k, device=dev, generator=g) * k ** -0.5
                setattr(self, name, Linear4bit.from_weight(w.half()))

        def forward(self, x):
            kv = (self.k_proj(x) + self.v_proj(x)).repeat(1, 6)
            mlp = self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))
            return x + self.o_proj(self.q_proj(x)) + kv + mlp

    class Stack(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.model = torch.nn.Module()
            self.model.layers = torch.nn.ModuleList([Layer() for _ in range(n_layers)])

        def forward(self, x):
            for layer in self.model.layers:
                x = layer(x)
            return x

    x0 = (torch.randn(M_TOKENS, 1536, device=dev, generator=g) * 0.5).half()
    dy = (torch.randn(M_TOKENS, 1536, device=dev, generator=g) * 0.01).half()

    def timed(model):
        def step():
            x = x0.detach().requires_grad_(True)
            model(x).backward(dy)
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    out = {"layers": n_layers, "tokens": M_TOKENS}
    out["resident_ms_per_step"] = round(timed(Stack()), 3)
    was = stream.enabled
    stream.enabled = True
    try:
        for key, unpack, slots in (("streamed", False, 2), ("streamed_3_slots", False, 3),
                                   ("streamed_layer_unpack", True, 2)):
            stream.reset()
            model = Stack()
            assert stream.setup(model, slots=slots, layer_unpack=unpack)
            s = stream.streamer()
            ms = timed(model)
            out[key + "_ms_per_step"] = round(ms, 3)
            out[key + "_copies_per_step"] = round(s.loads / (steps + warmup), 2)
        host = s.host_layers[0]
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        reps = 20
        with torch.cuda.stream(s.copy_stream):
            s.slots[0][:host.numel()].copy_(host, non_blocking=True)
            start.record()
            for _ in range(reps):
                s.slots[0][:host.numel()].copy_(host, non_blocking=True)
            end.record()
        end.synchronize()
        ms = start.elapsed_time(end) / reps
        gbs = host.numel() / ms / 1e6
        out["layer_copy"] = {"bytes": host.numel(), "ms": round(ms, 4), "GBps": round(gbs, 1),
                             "pcie_frac": round(gbs / PCIE_PEAK_GBS, 3)}
    finally:
        stream.reset()
        stream.enabled = was
    return out


def bench_fused(dev, steps, warmup):
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    out = {}
    # config 3: forward of gate_proj and up_proj on one X [1024, 1536] (they share the input)
    gate = make_proj(dev, g, 8960, 1536)
    up = make_proj(dev, g, 8960, 1536, x=gate["x"])
    ms, _ = graph_time(lambda: (proj_fwd(gate), proj_fwd(up)), steps, warmup)
    fl = 2 * proj_flops(8960, 1536, bwd=False)
    out["config3_fwd_gate_up"] = {"ms": round(ms, 4), "gflop": round(fl / 1e9, 3),
                                  "tflops": round(fl / ms / 1e9, 1)}
    # the dominant kernel alone: the fused forward GEMM with its LoRA epilogue (gate, up)
    from mindxsoup_amd import kernels
    hg, _ = kernels.lora_h(gate["x"], gate["a"], 2.0, gate["keep"], 1 / (1 - P_DROP))
    hu, _ = kernels.lora_h(up["x"], up["a"], 2.0, up["keep"], 1 / (1 - P_DROP))
    ms_k, _ = graph_time(lambda: (kernels.nf4_linear_fwd(gate["x"], gate["packed"], gate["st"],
                                                         None, hg, gate["b"], ws=gate["ws"]),
                                  kernels.nf4_linear_fwd(up["x"], up["packed"], up["st"], None,
                                                         hu, up["b"], ws=up["ws"])),
                         steps, warmup)
    fl_k = 2 * (2 * M_TOKENS * 8960 * 1536 + 2 * M_TOKENS * RANK * 8960)
    out["gemm_fwd_kernel"] = {"ms_per_launch": round(ms_k / 2, 4),
                              "tflops": round(fl_k / ms_k / 1e9, 1)}
    del gate, up, hg, hu
    # config 4: backward through down_proj (X = silu(g) * u saved, dY ~ N(0, 1e-3))
    down = make_proj(dev, g, 1536, 8960, x_kind="silu_mul", dy_std=1e-3)
    _, ht = proj_fwd(down)
    ms, _ = graph_time(lambda: proj_bwd(down, ht), steps, warmup)
    fl = proj_flops(1536, 8960, fwd=False)
    out["config4_bwd_down"] = {"ms": round(ms, 4), "gflop": round(fl / 1e9, 3),
                               "tflops": round(fl / ms / 1e9, 1)}
    del down, ht
    out["mlp_block"] = bench_mlp(dev, g, steps, warmup)
    out["qkv_rope"] = bench_qkv_rope(dev, g, steps, warmup)
    out["stream_weights"] = bench_stream(dev, g, max(5, steps // 4), max(2, warmup // 4))
    # config 5: forward + backward of all 28 layers x 7 projections, M = 1024
    layers = stack_layers(dev, g)
    step = stack_step(layers)

    def step_ungrouped():  # each projection's LoRA row products in launches of their own
        saved = []
        for projs in layers:
            saved.append([proj_fwd(p)[1] for p in projs])
        for projs, hts in zip(reversed(layers), reversed(saved)):
            for p, ht in zip(reversed(projs), reversed(hts)):
                proj_bwd(p, ht)

    from mindxsoup_amd import ops

    st_steps, st_warm = max(3, steps // 5), max(2, warmup // 5)
    ms, wall = graph_time(step, st_steps, st_warm)
    ms_u, _ = graph_time(step_ungrouped, st_steps, st_warm)
    raw_eager, raw_host = eager_time(step, st_steps, st_warm)
    # the same step as a training loop runs it: autograd nodes, eager launches
    alayers = [AutogradLayer(projs) for projs in layers]
    torch.cuda.synchronize()
    print("bench: autograd step (torch.ops.mxs_nf4)", file=sys.stderr, flush=True)
    prev = ops.ENABLED
    try:
        ops.ENABLED = True
        eager, host = eager_time(lambda: autograd_step(alayers), st_steps, st_warm)
        ag_ms, _ = graph_time(lambda: autograd_step(alayers), st_steps, st_warm)
        ops.ENABLED = False  # the Python Functions over ctypes, for comparison
        print("bench: autograd step (Python Functions)", file=sys.stderr, flush=True)
        py_eager, py_host = eager_time(lambda: autograd_step(alayers), st_steps, st_warm)
    finally:
        ops.ENABLED = prev
    per_dir = 2 * LAYERS * len(PROJ)
    fl = LAYERS * sum(proj_flops(n, k) for _, n, k in PROJ)
    tf = fl / ms / 1e9
    out["config5_stack"] = {"ms_per_step": round(ms, 4), "wall_ms_per_step": round(wall, 4),
                            "tflop_per_step": round(fl / 1e12, 4), "tflops": round(tf, 1),
                            "mfma_frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                            "launches": "one HIP graph per step",
                            "lora_rows": "q/k/v and gate/up grouped per launch",
                            "ungrouped_ms_per_step": round(ms_u, 4),
                            "eager_ms_per_step": round(eager, 4),
                            "eager_over_graph": round(eager / ms, 3),
                            "eager_host_ms_per_step": round(host, 4),
                            "eager_host_us_per_projection_direction": round(
                                host * 1e3 / per_dir, 2),
                            "eager_path": "autograd step through torch.ops.mxs_nf4 (C++ nodes)",
                            "autograd_graph_ms_per_step": round(ag_ms, 4),
                            "eager_python_ms_per_step": round(py_eager, 4),
                            "eager_python_host_us_per_projection_direction": round(
                                py_host * 1e3 / per_dir, 2),
                            "eager_raw_kernel_calls_ms_per_step": round(raw_eager, 4),
                            "eager_raw_kernel_calls_host_us_per_projection_direction": round(
                                raw_host * 1e3 / per_dir, 2)}
    del layers, alayers
    return out


def cpu_baseline_layer(dev):
    """One layer's 7 NF4+LoRA projections forward + backward on the host: the oracle's C decode,
    then torch CPU fp32 GEMMs (x28 extrapolated to the step, labelled as such)."""
    from oracle import oracle as O

    cores = host_cores()
    torch.set_num_threads(cores)
    O.set_num_threads(cores)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    projs = [make_proj(dev, g, n, k) for _, n, k in PROJ]
    host = []
    for p in projs:
        st = p["st"]
        host.append(dict(
            packed=p["packed"].view(-1).cpu().numpy(), absmax8=st.absmax.cpu().numpy(),
            code=st.state2.code.cpu().numpy(), absmax2=st.state2.absmax.cpu().numpy(),
            offset=float(st.offset.item()), shape=st.shape,
            x=p["x"].float().cpu(), a=p["a"].float().cpu(), b=p["b"].float().cpu(),
            dy=p["dy"].float().cpu(), keep=p["keep8"].cpu().bool()))
    del projs

    def layer_pass():
        for h in host:
            w = torch.from_numpy(O.dequant(packed=h["packed"], absmax8=h["absmax8"],
                                           code=h["code"], absmax2=h["absmax2"],
                                           offset=h["offset"], shape=h["shape"])
                                 .astype(np.float32))
            xd = torch.where(h["keep"], h["x"] * (1 / (1 - P_DROP)), 0.0)
            hh = xd @ h["a"].T * 2.0
            _ = h["x"] @ w.T + hh @ h["b"].T
            dh = h["dy"] @ h["b"] * 2.0
            _ = h["dy"] @ w + torch.where(h["keep"], (dh @ h["a"]) * (1 / (1 - P_DROP)), 0.0)
            _ = dh.T @ xd
            _ = h["dy"].T @ hh

    layer_pass()
    times = []
    start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < 10 and len(times) < 10):
        t = time.perf_counter()
        layer_pass()
        times.append(time.perf_counter() - t)
    sec = float(np.median(times))
    fl = sum(proj_flops(n, k) for _, n, k in PROJ)
    return {"value": round(fl / sec / 1e12, 4), "unit": "TFLOP/s", "cores": cores,
            "cores_available": len(os.sched_getaffinity(0)), "cpu_count": os.cpu_count(),
            "kind": "port",
            "sample": f"one layer (7 projections) fwd+bwd, M=1024: oracle decode + torch CPU fp32 "
                      f"GEMMs, median {sec * 1e3:.1f} ms/layer; x28 extrapolated step "
                      f"{sec * LAYERS * 1e3:.0f} ms"}


# One GEMM of the stack alone (for rocprofv3 counter passes and tile-plan sweeps):
# name -> (out_features N, in_features K, direction)
KERNELS = {"gate_fwd": (8960, 1536, "fwd"), "gateup_dx": (8960, 1536, "bwd"),
           "down_fwd": (1536, 8960, "fwd"), "down_dx": (1536, 8960, "bwd"),
           "qo_fwd": (1536, 1536, "fwd"), "qo_dx": (1536, 1536, "bwd")}


def bench_kernel(dev, name, tokens, steps, warmup, cfg=-1, splits=1):
    """One projection GEMM with its LoRA term (the partial sums of the row product already
    made), launched `steps` times after `warmup`, eagerly on the current stream: mean us per
    launch from HIP events on that stream, TFLOP/s over 2*M*N*K + 2*M*r*(output columns)."""
    from mindxsoup_amd import kernels

    n, k, direction = KERNELS[name]
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    p = make_proj(dev, g, n, k)
    x = torch.randn((tokens, k), device=dev, generator=g).half()
    dy = torch.randn((tokens, n), device=dev, generator=g).half()
    keep = kernels.keep_bits((torch.rand((tokens, k), device=dev, generator=g) >= P_DROP)
                             .to(torch.uint8), tokens, k)
    s, ms_ = ALPHA / RANK, 1.0 / (1.0 - P_DROP)
    nc, kr = (n, k) if direction == "fwd" else (k, n)
    ws = kernels.new_workspace(max(kernels.projection_workspace_bytes(tokens, k, n, RANK),
                                   kernels.gemm_workspace_bytes(tokens, nc, kr, cfg, splits)), dev)
    if direction == "fwd":
        hp, at, bt = kernels.lora_h_partials(x, p["a"], s, keep, ms_, lora_b=p["b"])

        def launch():
            kernels.nf4_linear_fwd_hp(x, p["packed"], p["st"], hp, p["b"], cfg=cfg,
                                      splits=splits, ws=ws)
        cols = n
    else:
        bt = p["b"].t().contiguous()
        at = p["a"].t().contiguous()
        dhp = kernels.lora_dh_partials(dy, bt, s)

        def launch():
            kernels.nf4_linear_bwd_dx_hp(dy, p["packed"], p["st"], dhp, at, keep, ms_, cfg=cfg,
                                         splits=splits, ws=ws)
        cols = k
    for _ in range(warmup):
        launch()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(steps):
        launch()
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / steps * 1e3
    fl = 2 * tokens * n * k + 2 * tokens * RANK * cols
    return {"kernel": name, "tokens": tokens, "N": n, "K": k, "direction": direction,
            "cfg": cfg, "splits": splits, "us_per_launch": round(us, 2),
            "tflops": round(fl / us / 1e6, 1),
            "mfma_frac": round(fl / us / 1e6 / MFMA_PEAK_TFLOPS, 4),
            "timing": "HIP events around the launches (GEMM + its split-K reduce, if any)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemm", action="store_true", help="dequant only")
    ap.add_argument("--stream", action="store_true",
                    help="only the host-streamed weights section (its JSON on stdout)")
    ap.add_argument("--qkv", action="store_true",
                    help="only the q/k/v RoPE section: the rotation kernel and the q/k/v "
                         "projection with the rotation apart or folded (its JSON on stdout)")
    ap.add_argument("--calibrate", action="store_true",
                    help="only run a 1 GiB device copy (reference for the PMC byte counters)")
    ap.add_argument("--kernel", choices=sorted(KERNELS),
                    help="only one projection GEMM, launched --steps times (its JSON on stdout)")
    ap.add_argument("--tokens", type=int, default=M_TOKENS, help="M for --kernel")
    ap.add_argument("--cfg", type=int, default=-1, help="tile configuration for --kernel")
    ap.add_argument("--splits", type=int, default=1, help="split-K for --kernel with --cfg")
    ap.add_argument("--stack", action="store_true",
                    help="only the 28-layer projection stack as one HIP graph: one eager step, "
                         "then --warmup and --steps replays (its JSON on stdout)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the hot path is "
              "data-parallel: forward and dX need no exchange, the LoRA gradients one "
              "all-reduce per layer). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate:
        calibrate(dev)
        return
    if args.kernel:
        print(json.dumps(bench_kernel(dev, args.kernel, args.tokens, args.steps, args.warmup,
                                      args.cfg, args.splits)), flush=True)
        return
    if args.stack:
        g = torch.Generator(device=dev)
        g.manual_seed(1)
        ms, wall = graph_time(stack_step(stack_layers(dev, g)), args.steps, args.warmup)
        fl = LAYERS * sum(proj_flops(n, k) for _, n, k in PROJ)
        print(json.dumps({"config5_stack": {"ms_per_step": round(ms, 4),
                                            "wall_ms_per_step": round(wall, 4),
                                            "tflops": round(fl / ms / 1e9, 1)}}), flush=True)
        return
    if args.stream:
        g = torch.Generator(device=dev)
        g.manual_seed(1)
        print(json.dumps(bench_stream(dev, g, args.steps, args.warmup)), flush=True)
        return
    if args.qkv:
        g = torch.Generator(device=dev)
        g.manual_seed(1)
        print(json.dumps({"qkv_rope": bench_qkv_rope(dev, g, args.steps, args.warmup)}),
              flush=True)
        return
    m = model_weights(dev)
    torch.cuda.synchronize()
    print(f"bench: {len(m['nb'])} NF4 weights resident ({m['packed'].numel() / 1e9:.3f} GB packed)",
          file=sys.stderr, flush=True)
    ms_step, ms_kernel, dq_out = bench_dequant(m, args.steps, args.warmup)
    print(f"bench: dequant timed, {ms_step:.4f} ms/step", file=sys.stderr, flush=True)
    ceiling = hbm_ceiling(m["packed"], dq_out, args.steps, args.warmup)
    del dq_out
    nblocks = m["absmax8"].numel()
    cpu_baseline_dequant_cached = None
    if not args.no_cpu:
        print("bench: CPU baseline (oracle decode)", file=sys.stderr, flush=True)
        cpu_baseline_dequant_cached = cpu_baseline_dequant(m)
    nbytes = dequant_bytes(m)
    value = nbytes / (ms_step / 1e3) / 1e9
    achieved = nbytes / (ms_kernel / 1e3) / 1e9
    result = {
        "metric": "NF4 dequant GB/s (Qwen2.5-1.5B, 28 layers x 7 projections, one launch)",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u8->f16 (fp32 decode)",
        "data": "synthetic: N(0,0.02) fp16 weights quantized to NF4 on the GPU (seed 0)",
        "config": {"workload": "BASELINE configs[1]: standalone NF4 dequant, all 196 weights",
                   "bytes_per_step": nbytes, "weights": LAYERS * len(PROJ),
                   "packed_bytes": m["packed"].numel(), "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "k_dequant_wide<nested, multi, f16>",
                     "kernel_ms": round(ms_kernel, 4)},
        "hbm_ceiling": ceiling,
    }
    # the dequant's own read / write mix at the pure streams' rates: the rate its bytes could
    # move at if reads ran at load_only's and writes at store_only's
    wbytes = 2 * 64 * nblocks
    mix = nbytes / ((nbytes - wbytes) / ceiling["load_only"]["GBps"]
                    + wbytes / ceiling["store_only"]["GBps"])
    ceiling["mix_GBps"] = round(mix, 1)
    ceiling["dequant_over_mix"] = round(achieved / mix, 4)
    del m
    torch.cuda.empty_cache()
    if not args.no_gemm:
        print("bench: fused NF4+LoRA projections", file=sys.stderr, flush=True)
        fused = bench_fused(dev, args.steps, args.warmup)
        st = fused["config5_stack"]
        fused["roofline"] = {"bound": "mfma", "achieved": fused["gemm_fwd_kernel"]["tflops"],
                             "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(fused["gemm_fwd_kernel"]["tflops"] / MFMA_PEAK_TFLOPS, 4),
                             "kernel": "k_nf4_gemm forward (gate/up, LoRA epilogue)"}
        result["fused_stack"] = fused
        print(f"bench: stack {st['ms_per_step']} ms/step, {st['tflops']} TFLOP/s",
              file=sys.stderr, flush=True)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_dequant_cached
        if not args.no_gemm:
            print("bench: CPU baseline (one layer of projections)", file=sys.stderr, flush=True)
            result["fused_stack"]["cpu_baseline"] = cpu_baseline_layer(dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
