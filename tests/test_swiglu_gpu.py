"""SwiGLU of the fp16 MLP (mindxsoup_amd/silu_mul.py on csrc/swiglu.hip) against the oracle's
restatement of solution/silu_mul.py, with the reference test's shapes and tolerance
(solution/test_silu_mul.py:22-40: atol = rtol = 1e-3, i.e. about one fp16 ulp)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _np(t):
    return t.detach().cpu().numpy()


def _close(got, want):
    g = got.astype(np.float32)
    w = want.astype(np.float32)
    assert np.all(np.abs(g - w) <= 1e-3 + 1e-3 * np.abs(w))
    return float(np.mean(got.view(np.uint16) == want.view(np.uint16)))


@pytest.mark.parametrize("shape", [(1, 8960), (37, 8960), (1, 1430, 8960), (5, 1000), (3, 2049)])
def test_silu_mul_matches_oracle(cuda, shape):
    from mindxsoup_amd.silu_mul import silu_mul

    print(f"case silu_mul shape={shape}", flush=True)
    torch.manual_seed(0)
    gate = (torch.randn(shape, device=cuda) * 3).half().requires_grad_(True)
    up = (torch.randn(shape, device=cuda) * 3).half().requires_grad_(True)
    grad = torch.randn(shape, device=cuda).half()
    want_out = O.silu_mul(_np(gate), _np(up))
    want_dg, want_du = O.silu_mul_bwd(_np(grad), _np(gate), _np(up))
    g, u = gate * 1, up * 1  # not leaves, as in the MLP: their memory becomes the gradients
    out = silu_mul(g, u)
    assert out.dtype == torch.float16 and out.shape == gate.shape
    exact = _close(_np(out), want_out)
    out.backward(grad)
    exact_g = _close(_np(gate.grad), want_dg)
    exact_u = _close(_np(up.grad), want_du)
    # same fp32 formula; the kernel's hardware exp2 and reciprocal (about 1 ulp each) against
    # libm's expf and an IEEE division move an fp16 result only near a rounding boundary
    assert min(exact, exact_g, exact_u) > 0.99, (exact, exact_g, exact_u)


def test_backward_writes_over_gate_and_up(cuda):
    """The in-place backward: the gradients autograd hands on live in gate's and up's memory."""
    from mindxsoup_amd.silu_mul import SiluMulInPlace

    torch.manual_seed(2)
    n, inter = 300, 8960
    gate = torch.randn(n, inter, device=cuda).half()
    up = torch.randn(n, inter, device=cuda).half()
    grad = torch.randn(n, inter, device=cuda).half()
    want_dg, want_du = O.silu_mul_bwd(_np(grad), _np(gate), _np(up))
    g = gate.clone().requires_grad_(True)
    u = up.clone().requires_grad_(True)
    gi, ui = g * 1, u * 1
    ptr_g, ptr_u = gi.data_ptr(), ui.data_ptr()
    seen = {}
    gi.register_hook(lambda t: seen.__setitem__("g", t.data_ptr()))
    ui.register_hook(lambda t: seen.__setitem__("u", t.data_ptr()))
    SiluMulInPlace.apply(gi, ui).backward(grad)
    assert seen == {"g": ptr_g, "u": ptr_u}
    _close(_np(g.grad), want_dg)
    _close(_np(u.grad), want_du)


@pytest.mark.parametrize("n,offset", [(7, 0), (1001, 1), (8 * 4096 + 5, 3), (0, 0)])
def test_silu_mul_unaligned_and_tails(cuda, n, offset):
    from mindxsoup_amd import kernels

    print(f"case silu_mul tail n={n} offset={offset}", flush=True)
    torch.manual_seed(3)
    buf_g = (torch.randn(n + offset, device=cuda) * 4).half()
    buf_u = (torch.randn(n + offset, device=cuda) * 4).half()
    buf_d = torch.randn(n + offset, device=cuda).half()
    g, u, d = buf_g[offset:], buf_u[offset:], buf_d[offset:]
    out = kernels.silu_mul(g, u)
    want = O.silu_mul(_np(g), _np(u))
    want_dg, want_du = O.silu_mul_bwd(_np(d), _np(g), _np(u))
    kernels.silu_mul_bwd_(d, g, u)
    torch.cuda.synchronize()
    if n:
        _close(_np(out), want)
        _close(_np(g), want_dg)
        _close(_np(u), want_du)


def test_special_values_match_oracle_exactly(cuda):
    """Where exp over- or underflows (|gate| large, infinities) and at gate = 0, the hardware
    exp2 and reciprocal give the oracle's values (libm expf, IEEE division).  Values are equal;
    a zero's sign may differ where sigmoid(gate) falls into fp32's subnormal range (gate near
    -88: the hardware reciprocal returns 0 there, so d(gate) is +0 where libm's subnormal
    sigmoid leaves -0)."""
    from mindxsoup_amd import kernels

    gv = np.array([0.0, -0.0, 1e-7, -1e-7, 20, -20, 88, -88, 100, -100, 1000, -1000, 65504,
                   -65504, np.inf, -np.inf], np.float16)
    uv = np.array([1, -3, 2, 0.5, 1, 1, -2, 2, 1, 1, 0.25, 4, 1, 1, 1, 1], np.float16)
    dv = np.array([1, 2, -1, 4, 1, -1, 0.5, 2, 1, 1, 1, 1, 0.5, 0.5, 1, 1], np.float16)
    g = torch.from_numpy(gv).to(cuda)
    u = torch.from_numpy(uv).to(cuda)
    d = torch.from_numpy(dv).to(cuda)
    out = kernels.silu_mul(g, u)
    kernels.silu_mul_bwd_(d, g, u)
    torch.cuda.synchronize()
    want = O.silu_mul(gv, uv)
    want_dg, want_du = O.silu_mul_bwd(dv, gv, uv)
    for got, ref in ((out, want), (g, want_dg), (u, want_du)):
        got = _np(got)
        same = (got == ref) | (np.isnan(got) & np.isnan(ref))
        assert same.all(), (got, ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(4, 512, 8960), (3, 77, 1001)])
def test_swiglu_matches_pytorch(cuda, dtype, shape):
    """solution/test_kernels.py:14-35 on silu_mul: forward and backward against fp32 PyTorch
    (2e-3 for fp16, 1e-4 for fp32; fp32 inputs take the plain expression, as the reference's
    guard sends them)."""
    from mindxsoup_amd.silu_mul import silu_mul

    tol = {torch.float16: 2e-3, torch.float32: 1e-4}[dtype]
    torch.manual_seed(0)
    gate = torch.randn(shape, device=cuda, dtype=dtype, requires_grad=True)
    up = torch.randn(shape, device=cuda, dtype=dtype, requires_grad=True)
    grad = torch.randn(shape, device=cuda, dtype=dtype)
    ref = torch.nn.functional.silu(gate.float()) * up.float()
    ref.backward(grad.float())
    ref_dgate, ref_dup = gate.grad.float(), up.grad.float()
    gate.grad = up.grad = None
    out = silu_mul(gate * 1, up * 1)  # not leaves: their memory takes the gradients
    out.backward(grad)
    torch.testing.assert_close(out.float(), ref, rtol=tol, atol=tol)
    torch.testing.assert_close(gate.grad.float(), ref_dgate, rtol=tol, atol=tol)
    torch.testing.assert_close(up.grad.float(), ref_dup, rtol=tol, atol=tol)
