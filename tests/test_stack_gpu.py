"""The step bench.py times for BASELINE configs[4] (one decoder layer's 7 NF4 + LoRA projections,
forward then backward, with the grouped launches the timed stack uses), checked projection by
projection against the float64 oracle at M = 1024 tokens: y, dX, dA and dB within the north
star's max relative error 1e-2 (the summed dX of q/k/v and of gate/up against the oracle's
sums)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def test_timed_layer_step_matches_oracle(cuda):
    import bench

    g = torch.Generator(device=cuda)
    g.manual_seed(11)
    x_attn = torch.randn((bench.M_TOKENS, 1536), device=cuda, generator=g).half()
    x_mlp = torch.randn((bench.M_TOKENS, 1536), device=cuda, generator=g).half()
    projs = []
    for name, n, k in bench.PROJ:
        x = x_attn if name in ("q", "k", "v") else x_mlp if name in ("gate", "up") else None
        projs.append(bench.make_proj(cuda, g, n, k, x=x, x_kind="silu_mul" if name == "down"
                                     else "normal", dy_std=1e-3 if name == "down" else 1.0))
    ys, saved = bench.layer_fwd(projs)
    grads = bench.layer_bwd(projs, saved)
    torch.cuda.synchronize()
    s, p = bench.ALPHA / bench.RANK, bench.P_DROP
    names = [name for name, _, _ in bench.PROJ]
    ig, iu = names.index("gate"), names.index("up")
    assert grads[ig][0] is None and grads[iu][0] is not None
    iq, ik, iv = names.index("q"), names.index("k"), names.index("v")
    assert grads[iq][0] is None and grads[ik][0] is None and grads[iv][0] is not None
    ref_dx_sum = 0.0
    ref_qkv = 0.0
    for (name, n, k), pr, y, (dx, da, db) in zip(bench.PROJ, projs, ys, grads):
        st = pr["st"]
        w = O.dequant(O.NF4Weight(st.shape, pr["packed"].view(-1).cpu().numpy(),
                                  st.absmax.cpu().numpy(), st.state2.code.cpu().numpy(),
                                  st.state2.absmax.cpu().numpy(), float(st.offset.item())))
        x16, a16, b16 = (_np(pr[key]).astype(np.float16) for key in ("x", "a", "b"))
        kp, dy16 = pr["keep8"].cpu().numpy(), _np(pr["dy"]).astype(np.float16)
        ref_y = O.lora_fwd(x16, w, a16, b16, s, kp, p)
        ref_dx, ref_da, ref_db = O.lora_bwd(dy16, x16, w, a16, b16, s, kp, p)
        errs = {"y": O.max_rel(_np(y), ref_y), "dA": O.max_rel(_np(da), ref_da),
                "dB": O.max_rel(_np(db), ref_db)}
        if name in ("gate", "up"):
            ref_dx_sum = ref_dx_sum + ref_dx
            if name == "up":
                errs["dx(gate+up)"] = O.max_rel(_np(dx), ref_dx_sum)
        elif name in ("q", "k", "v"):
            ref_qkv = ref_qkv + ref_dx
            if name == "v":
                errs["dx(q+k+v)"] = O.max_rel(_np(dx), ref_qkv)
        else:
            errs["dx"] = O.max_rel(_np(dx), ref_dx)
        print(f"case stack layer {name}: " + " ".join(f"{k_}={v:.1e}" for k_, v in errs.items()),
              flush=True)
        assert max(errs.values()) < 1e-2, (name, errs)


def _flat(ys, grads):
    out = []
    for y in ys:
        out.append(y)
    for grad in grads:
        out.extend(t for t in grad if t is not None)
    return out


def test_graph_replayed_stack_step_equals_eager(cuda):
    """The step as bench.py times it: layers sharing one workspace, forward of each then
    backward in reverse, captured in one HIP graph.  Every replay's outputs (y, the summed and
    single dX, dA, dB of every projection) equal the eager run's bit for bit, with eager steps
    that overwrite the shared workspace run between the replays."""
    import bench

    g = torch.Generator(device=cuda)
    g.manual_seed(12)
    layers = []
    for _ in range(2):
        x_attn = torch.randn((bench.M_TOKENS, 1536), device=cuda, generator=g).half()
        x_mlp = torch.randn((bench.M_TOKENS, 1536), device=cuda, generator=g).half()
        projs = []
        for name, n, k in bench.PROJ:
            x = x_attn if name in ("q", "k", "v") else x_mlp if name in ("gate", "up") else None
            projs.append(bench.make_proj(cuda, g, n, k, x=x))
        layers.append(projs)

    def step():
        ys, saved = [], []
        for projs in layers:
            y, sv = bench.layer_fwd(projs)
            ys += y
            saved.append(sv)
        grads = []
        for projs, sv in zip(reversed(layers), reversed(saved)):
            grads += bench.layer_bwd(projs, sv)
        return _flat(ys, grads)

    print("case stack graph replay: eager reference", flush=True)
    eager = [t.clone() for t in step()]
    torch.cuda.synchronize()
    assert len(eager) == 2 * (7 + 7 * 2 + 4)  # dX of o, down and the two sums
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    assert len(static) == len(eager)
    for rep in range(3):
        print(f"case stack graph replay {rep}", flush=True)
        again = step()  # eager work on the same workspace between replays
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(again, eager))
        graph.replay()
        torch.cuda.synchronize()
        bad = [i for i, (a, b) in enumerate(zip(static, eager)) if not torch.equal(a, b)]
        assert not bad, (rep, bad)
    del graph
