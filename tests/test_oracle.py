"""Pins of the CPU oracle (no GPU): each check is independent of the oracle's own code, chosen
so that a plausible mistake (wrong table value, swapped nibbles, wrong block index, a missing or
extra rounding, a sign or transposition error in the LoRA gradients) fails one of them."""

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import oracle as O


# --- NF4 table ----------------------------------------------------------------------------

def test_nf4_table_is_the_normal_quantile_code():
    """NF4 = normalised quantiles of N(0,1): 8 positive from linspace(0.9677083, 0.5, 9), 7
    negative from linspace(0.9677083, 0.5, 8), plus 0 (QLoRA, arXiv 2305.14314, Sec. 3 / App. E;
    the offset 0.9677083 = (1 - 1/(2*15) + 1 - 1/(2*16)) / 2)."""
    from scipy.stats import norm

    off = 0.9677083
    pos = norm.ppf(np.linspace(off, 0.5, 9)[:-1])
    neg = -norm.ppf(np.linspace(off, 0.5, 8)[:-1])
    vals = np.sort(np.concatenate([pos, neg, [0.0]]))
    vals = vals / vals.max()
    table = O.nf4_table()
    assert table.dtype == np.float32 and table.shape == (16,)
    np.testing.assert_allclose(table, vals, rtol=0, atol=2e-7)
    assert table[7] == 0.0 and table[0] == -1.0 and table[15] == 1.0
    assert np.all(np.diff(table) > 0)


def test_product_table_matches_oracle_table():
    from mindxsoup_amd.nf4 import NF4_VALUES

    assert np.array_equal(NF4_VALUES.view(np.uint32), O.nf4_table().view(np.uint32))


# --- fp16 rounding ------------------------------------------------------------------------

def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000)).astype(np.float32)
    bits = rng.integers(0, 2 ** 32, 5000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    bits = bits[np.isfinite(bits)]
    edge = np.array([0.0, -0.0, 65504, 65519.996, 65520, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                     2 ** -14, 2 ** -14 - 2 ** -25, 1 + 2 ** -11, 1 + 3 * 2 ** -11, np.inf,
                     -np.inf, 1e-30], np.float32)
    allx = np.concatenate([x, bits, edge]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = allx.astype(np.float16).view(np.uint16)
    got = O.f32_to_f16_bits(allx)
    assert np.array_equal(got, want)


# --- dequant: closed forms ----------------------------------------------------------------

def _one_block_case(code_val, absmax2_val, offset, byte_values):
    packed = np.asarray(byte_values, np.uint8)
    n_blocks = (packed.size + 31) // 32
    code = np.zeros(256, np.float32)
    code[3] = code_val
    absmax8 = np.full(n_blocks, 3, np.uint8)
    absmax2 = np.full((n_blocks + 255) // 256, absmax2_val, np.float32)
    return O.dequant(packed=packed, absmax8=absmax8, code=code, absmax2=absmax2, offset=offset)


def test_dequant_zero_code_and_unit_code():
    # scale = 0.5 * 2 + 0.25 = 1.25 exactly; byte 0x7F -> (NF4[7] = 0, NF4[15] = 1) * 1.25
    out = _one_block_case(0.5, 2.0, 0.25, [0x7F] * 32)
    assert out.dtype == np.float16
    assert np.all(out[0::2] == 0.0) and np.all(out[1::2] == np.float16(1.25))
    # 0xF0 -> high nibble first: (1.25, -1.25)
    out = _one_block_case(0.5, 2.0, 0.25, [0xF0] * 32)
    assert np.all(out[0::2] == np.float16(1.25)) and np.all(out[1::2] == np.float16(-1.25))
    # code[q8] = 0: the scale is the offset alone
    out = _one_block_case(0.0, 123.0, 0.5, [0xF0] * 32)
    assert np.all(out[0::2] == np.float16(0.5))


def test_dequant_all_bytes_brute_force():
    """Every byte value: value 2i from the high nibble, 2i+1 from the low, times the scale, one
    rounding to fp16 (numpy's own float32 -> float16 conversion)."""
    table = O.nf4_table()
    for scale_parts in [(0.75, 0.03125, 0.0), (-0.3, 0.07, 0.051), (1.0, 1e-3, 2e-4)]:
        packed = np.arange(256, dtype=np.uint8)
        out = _one_block_case(*scale_parts, packed)
        c, a2, off = (np.float32(v) for v in scale_parts)
        s = np.float32(Fraction(float(c)) * Fraction(float(a2)) + Fraction(float(off)))
        hi = (table[packed >> 4] * s).astype(np.float16)
        lo = (table[packed & 15] * s).astype(np.float16)
        assert np.array_equal(out[0::2].view(np.uint16), hi.view(np.uint16))
        assert np.array_equal(out[1::2].view(np.uint16), lo.view(np.uint16))


def test_dequant_block_and_group_indexing():
    """Block b (32 bytes) takes absmax8[b]; absmax2 advances every 256 blocks.  With distinct
    powers of two per block and per group the output names its own block and group."""
    n_blocks = 600
    packed = np.full(32 * n_blocks, 0xFF, np.uint8)  # every value NF4[15] = 1.0
    code = (2.0 ** -np.arange(256)).astype(np.float32)[::-1].copy()  # ascending, exact
    absmax8 = (np.arange(n_blocks) % 200 + 40).astype(np.uint8)
    absmax2 = np.array([1.0, 4.0, 16.0], np.float32)
    out = O.dequant(packed=packed, absmax8=absmax8, code=code, absmax2=absmax2, offset=0.0)
    want_block = code[absmax8] * absmax2[np.arange(n_blocks) // 256]
    want = np.repeat(want_block, 64).astype(np.float16)
    assert np.array_equal(out.view(np.uint16), want.view(np.uint16))


def _fma32(a, b, c):
    return np.float32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_dequant_scale_is_one_fused_multiply_add():
    """Against exact rational arithmetic: the fused scale is RN(c*a2 + off); the unfused one is
    RN(RN(c*a2) + off).  Cases are picked where the two differ, so a dropped FMA shows."""
    rng = np.random.default_rng(3)
    found = 0
    for _ in range(4000):
        c, a2, off = (np.float32(v) for v in rng.uniform(-1, 1, 3))
        fused = _fma32(c, a2, off)
        unfused = np.float32(np.float32(c * a2) + off)
        if fused == unfused:
            continue
        found += 1
        code = np.zeros(256, np.float32)
        code[9] = c
        packed = np.full(32, 0xF7, np.uint8)  # values (1.0, 0.0) * scale
        got_f = O.dequant(packed=packed, absmax8=np.array([9], np.uint8), code=code,
                          absmax2=np.array([a2], np.float32), offset=float(off),
                          out_dtype=np.float32)
        got_u = O.dequant(packed=packed, absmax8=np.array([9], np.uint8), code=code,
                          absmax2=np.array([a2], np.float32), offset=float(off),
                          out_dtype=np.float32, fused=False)
        assert got_f[0] == fused and got_u[0] == unfused
        if found > 40:
            break
    assert found > 10


def test_fused_and_unfused_differ_by_at_most_one_ulp():
    """solution/test_nf4.py:41-42: the two absmax decodes give fp16 values at most one ulp apart."""
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((256, 512)) * 0.05).astype(np.float16)
    q = O.quantize(w)
    a = O.dequant(q).view(np.uint16).astype(np.int32)
    b = O.dequant(q, fused=False).view(np.uint16).astype(np.int32)
    assert np.abs(a - b).max() <= 1


def test_dequant_numpy_restatement():
    """An independent vectorised numpy decode (whole arrays, no per-byte loop) agrees bit for
    bit with the scalar C oracle on a random double-quantized weight."""
    rng = np.random.default_rng(11)
    n_blocks = 1000
    packed = rng.integers(0, 256, 32 * n_blocks, dtype=np.uint8)
    absmax8 = rng.integers(0, 256, n_blocks, dtype=np.uint8)
    code = np.sort(rng.uniform(-1, 1, 256).astype(np.float32))
    absmax2 = rng.uniform(0.01, 0.1, (n_blocks + 255) // 256).astype(np.float32)
    offset = np.float32(0.031)
    got = O.dequant(packed=packed, absmax8=absmax8, code=code, absmax2=absmax2,
                    offset=float(offset))
    blk = np.arange(n_blocks)
    scale = np.array([_fma32(c, a, offset) for c, a in zip(code[absmax8], absmax2[blk // 256])],
                     np.float32)
    nib = np.stack([packed >> 4, packed & 15], axis=1).reshape(-1)
    want = (O.nf4_table()[nib] * np.repeat(scale, 64)).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


# --- quantizer ----------------------------------------------------------------------------

def test_quantize_roundtrip_error_bound():
    """|w - deq(quant(w))| <= absmax_b * (largest half-gap of NF4) + second-level error: fails
    for a swapped nibble order or a wrong block index on either side."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((512, 256)) * 0.02).astype(np.float16)
    q = O.quantize(w)
    d = O.dequant(q).astype(np.float32).reshape(-1)
    table = O.nf4_table().astype(np.float64)
    half_gap = np.max(np.diff(table)) / 2
    blk_absmax = np.repeat(q.absmax_f32, 64)
    scale = np.repeat(q.code[q.absmax8] * q.absmax2[np.arange(q.absmax8.size) // 256] + q.offset,
                      64)
    err = np.abs(d - w.reshape(-1).astype(np.float32))
    bound = blk_absmax * half_gap + np.abs(scale - blk_absmax) + 1e-3 * np.abs(d) + 1e-7
    assert np.all(err <= bound)
    # and much better than chance: relative RMS error of NF4 on Gaussian data is ~10 %
    rel = np.sqrt(np.mean(err ** 2)) / np.sqrt(np.mean(w.astype(np.float32) ** 2))
    assert rel < 0.15


def test_quantize_picks_nearest_codes():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((64, 128)) * 0.02).astype(np.float16)
    q = O.quantize(w)
    table = O.nf4_table()
    x = w.reshape(-1, 64).astype(np.float32) / q.absmax_f32[:, None]
    nib = np.stack([q.packed >> 4, q.packed & 15], 1).reshape(-1, 64)
    d_got = np.abs(x - table[nib])
    d_best = np.abs(x[..., None] - table[None, None, :]).min(-1)
    assert np.all(d_got <= d_best + 1e-6)
    v = (q.absmax_f32 - q.offset) / q.absmax2[np.arange(q.absmax8.size) // 256]
    assert np.all(np.abs(v - q.code[q.absmax8]) <= np.abs(v[:, None] - q.code[None]).min(1) + 1e-7)


def test_dynamic_map_properties_and_product_copy():
    from mindxsoup_amd.quant import dynamic_map

    code = O.dynamic_map()
    assert code.shape == (256,) and np.all(np.diff(code) >= 0)
    assert code[-1] == 1.0 and 0.0 in code and (code < 0).sum() == 127
    assert np.isclose(code.min(), -0.99296875, atol=1e-7)
    assert np.array_equal(dynamic_map().view(np.uint32), code.view(np.uint32))


def test_absmax_mean_close_to_exact_mean():
    rng = np.random.default_rng(2)
    a = rng.uniform(0, 0.1, 300000).astype(np.float32)
    exact = math.fsum(float(v) for v in a) / a.size
    assert abs(O.absmax_mean(a) - exact) <= 1e-7 * exact


# --- LoRA dropout -------------------------------------------------------------------------

def _round_binary(q, man_bits, emin, emax):
    """Round the rational q to nearest even in a binary format with man_bits fraction bits,
    smallest normal exponent emin and largest exponent emax (subnormals kept, overflow to an
    infinity).  Returns a Fraction or ±math.inf; exact, independent of any float hardware."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    quantum = Fraction(2) ** (max(e, emin) - man_bits)
    n = a / quantum
    whole = n.numerator // n.denominator
    rest = n - whole
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and whole % 2 == 1):
        whole += 1
    r = whole * quantum
    if r >= Fraction(2) ** (emax + 1):
        return sign * math.inf
    return sign * r


def _rn_f64(q):
    return _round_binary(q, 52, -1022, 1023)


def _rn_f32(q):
    return _round_binary(q, 23, -126, 127)


def _rn_f16(q):
    return _round_binary(q, 10, -14, 15)


def _all_finite_f16():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = bits.view(np.float16)
    return x[np.isfinite(x)]


def test_dropout_closed_forms():
    """solution/dropout.py:33-35 with a scale of exactly 2 (p = 0.5) or 4 (p = 0.75): every kept
    finite fp16 x becomes exactly 2x or 4x (±inf where that leaves fp16's range, sign of zero
    kept); a dropped element is +0.0 whatever x is, -0.0 and negatives included."""
    x = _all_finite_f16()
    assert x.size == 63488
    ones = np.ones(x.size, np.uint8)
    for p, factor in ((0.5, 2), (0.75, 4)):
        got = O.dropout_fp16(x, ones, p)
        for xi, gi in zip(x.tolist(), got.tolist()):
            want = Fraction(xi) * factor
            if abs(want) > 65504:
                assert gi == math.copysign(math.inf, xi), (p, xi, gi)
            else:
                assert Fraction(gi) == want, (p, xi, gi)
                assert math.copysign(1.0, gi) == math.copysign(1.0, xi)
        dropped = O.dropout_fp16(x, np.zeros(x.size, np.uint8), p)
        assert np.all(dropped.view(np.uint16) == 0)


def test_dropout_p005_is_two_roundings_of_the_exact_product():
    """p = 0.05 (the BASELINE configs): the scale is the Python double 1/(1 - p) narrowed to the
    fp32 kernel argument; each kept x is fp16_RN(fp32_RN(x * scale)), computed here in exact
    rational arithmetic over all 63,488 finite fp16 values.  A missing fp32 step, a scale of
    1 - p, or an fp16 scale fails it."""
    p = 0.05
    scale = _rn_f32(_rn_f64(1 / _rn_f64(1 - Fraction(p))))
    assert float(scale) == float(np.float32(1.0 / (1.0 - p)))
    assert scale != Fraction(20, 19)  # the narrowing is visible: not the exact 1/0.95
    x = _all_finite_f16()
    got = O.dropout_fp16(x, np.ones(x.size, np.uint8), p)
    for xi, gi in zip(x.tolist(), got.tolist()):
        want = _rn_f16(_rn_f32(Fraction(xi) * scale))
        if want in (math.inf, -math.inf):
            assert gi == want, (xi, gi)
        else:
            assert Fraction(gi) == want, (xi, gi)
            if want == 0:
                assert math.copysign(1.0, gi) == math.copysign(1.0, xi)
    # a scale rounded to fp16 first (a plausible slip) gives other bits somewhere
    s16 = _rn_f16(scale)
    assert any(Fraction(g) != _rn_f16(_rn_f32(Fraction(xi) * s16))
               for xi, g in zip(x.tolist(), got.tolist()) if abs(xi) < 30000)
    # mixed mask: dropped elements are +0, kept ones as above
    rng = np.random.default_rng(5)
    keep = (rng.uniform(size=x.size) >= p).astype(np.uint8)
    mixed = O.dropout_fp16(x, keep, p)
    assert np.all(mixed.view(np.uint16)[keep == 0] == 0)
    assert np.array_equal(mixed.view(np.uint16)[keep != 0], got.view(np.uint16)[keep != 0])


def test_round_binary_pins():
    """The exact rounding helper against known values: fp16's largest finite, the first value
    that overflows, ties to even, the smallest subnormals."""
    assert _rn_f16(Fraction(65504)) == 65504
    assert _rn_f16(Fraction(65519)) == 65504
    assert _rn_f16(Fraction(65520)) == math.inf
    assert _rn_f16(1 + Fraction(1, 2 ** 11)) == 1  # tie, even stays
    assert _rn_f16(1 + Fraction(3, 2 ** 11)) == 1 + Fraction(2, 2 ** 10)  # tie, rounds up
    assert _rn_f16(Fraction(1, 2 ** 25)) == 0  # half the smallest subnormal: tie to even 0
    assert _rn_f16(Fraction(3, 2 ** 26)) == Fraction(1, 2 ** 24)
    assert _rn_f32(Fraction(1, 3)) == Fraction(float(np.float32(1 / 3)))
    assert _rn_f64(Fraction(1, 10)) == Fraction(0.1)


# --- GEMM / LoRA references ---------------------------------------------------------------

def _lora_case(seed, m=24, k=64, n=40, r=16, p=0.25):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
    a = (rng.standard_normal((r, k)) * 0.1).astype(np.float16)
    b = (rng.standard_normal((n, r)) * 0.1).astype(np.float16)
    dy = rng.standard_normal((m, n)).astype(np.float16)
    keep = (rng.uniform(size=(m, k)) > p).astype(np.uint8)
    return x, w, a, b, dy, keep, p


def test_lora_reference_matches_torch_autograd():
    """The hand-written backward (dX, dA, dB) against float64 torch autograd of the forward."""
    x, w, a, b, dy, keep, p = _lora_case(0)
    s = 2.0
    xt = torch.tensor(x.astype(np.float64), requires_grad=True)
    at = torch.tensor(a.astype(np.float64), requires_grad=True)
    bt = torch.tensor(b.astype(np.float64), requires_grad=True)
    # dropout on the fp16 input as the reference rounds it (the mask and scale are constants)
    xd = torch.tensor(O.dropout_fp16(x, keep, p).astype(np.float64))
    mask_scale = torch.tensor(np.where(keep != 0, float(np.float32(1 / (1 - p))), 0.0))
    # forward with the dropped input expressed through x so autograd sees d(xd)/dx
    xd_graph = xt * mask_scale + (xd - (torch.tensor(x.astype(np.float64)) * mask_scale))
    y = xt @ torch.tensor(w.astype(np.float64)).T + s * (xd_graph @ at.T) @ bt.T
    y.backward(torch.tensor(dy.astype(np.float64)))
    y_ref = O.lora_fwd(x, w, a, b, s, keep, p)
    dx, da, db = O.lora_bwd(dy, x, w, a, b, s, keep, p)
    np.testing.assert_allclose(y_ref, y.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(da, at.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, bt.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_lora_forward_merged_weight_identity():
    """Without dropout, base + s*B(A(x)) equals x @ (W + s*B@A)^T (peft's merge formula)."""
    x, w, a, b, _, _, _ = _lora_case(1)
    s = 2.0
    merged = w.astype(np.float64) + s * b.astype(np.float64) @ a.astype(np.float64)
    np.testing.assert_allclose(O.lora_fwd(x, w, a, b, s),
                               x.astype(np.float64) @ merged.T, rtol=1e-10, atol=1e-10)


def test_max_rel_definition():
    assert O.max_rel([1.0, 2.0], [1.0, 4.0]) == pytest.approx(0.5)


def _ulp_diff_f16(a, b):
    """Distance in fp16 ulps (finite values, same-sign ordering by bit pattern)."""
    ia = a.astype(np.float16).view(np.int16).astype(np.int64)
    ib = b.astype(np.float16).view(np.int16).astype(np.int64)
    ia = np.where(ia < 0, -32768 - ia, ia)
    ib = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ia - ib)


def test_silu_mul_oracle_against_float64_and_closed_forms():
    rng = np.random.default_rng(11)
    n = 50000
    g = (rng.standard_normal(n) * 3).astype(np.float16)
    u = (rng.standard_normal(n) * 3).astype(np.float16)
    d = rng.standard_normal(n).astype(np.float16)
    out = O.silu_mul(g, u)
    dg, du = O.silu_mul_bwd(d, g, u)
    g64, u64, d64 = g.astype(np.float64), u.astype(np.float64), d.astype(np.float64)
    s = 1.0 / (1.0 + np.exp(-g64))
    silu = g64 * s
    # the kernel's fp32 arithmetic lands within one fp16 ulp of the exact value
    assert _ulp_diff_f16(out, (u64 * silu).astype(np.float16)).max() <= 1
    assert _ulp_diff_f16(dg, (d64 * u64 * (s + silu * (1 - s))).astype(np.float16)).max() <= 1
    assert _ulp_diff_f16(du, (d64 * silu).astype(np.float16)).max() <= 1
    # gate = 0: sigmoid = 1/2, silu = 0
    z = np.zeros(8, np.float16)
    uu = np.array([1, -2, 3.5, 0.25, 100, -7, 2048, 1e-3], np.float16)
    dd = np.array([2, 2, -1, 4, 0.5, 1, 1, 8], np.float16)
    assert np.all(O.silu_mul(z, uu) == 0)
    dgz, duz = O.silu_mul_bwd(dd, z, uu)
    assert np.all(duz == 0)
    assert np.array_equal(dgz, (dd.astype(np.float32) * uu.astype(np.float32) * 0.5).astype(np.float16))
    # large |gate|: silu -> gate (sigmoid -> 1) and -> 0 (sigmoid -> 0)
    big = np.array([30, 60, 1000], np.float16)
    one = np.ones(3, np.float16)
    assert np.array_equal(O.silu_mul(big, one), big)
    assert np.all(np.abs(O.silu_mul(-big, one).astype(np.float32)) < 1e-6)
    # the derivative in the order of solution/test_silu_mul.py:13-19 (d*u*s*(1 + g*(1-s)))
    g32, u32, d32 = g.astype(np.float32), u.astype(np.float32), d.astype(np.float32)
    s32 = (1.0 / (1.0 + np.exp(-g32))).astype(np.float32)
    alt_dg = (d32 * u32 * s32 * (1 + g32 * (1 - s32))).astype(np.float16).astype(np.float32)
    assert np.allclose(dg.astype(np.float32), alt_dg, atol=1e-3, rtol=1e-3)


def _qwen_cos_sin(batch, n_tokens, offsets=True):
    """cos / sin as Qwen2RotaryEmbedding makes them (theta 1e6, head_dim 128), fp32 [B, T, 128]."""
    import torch
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    cfg = Qwen2Config(hidden_size=1536, num_attention_heads=12, num_key_value_heads=2,
                      rope_theta=1e6)
    rot = Qwen2RotaryEmbedding(cfg)
    pos = torch.arange(n_tokens)[None, :].expand(batch, -1)
    if offsets:  # rows differ, like left padding
        pos = pos + torch.arange(batch)[:, None] * 3
    cos, sin = rot(torch.zeros(1, dtype=torch.float32), pos)
    return cos.float().numpy(), sin.float().numpy()


def test_qkv_rope_oracle_against_transformers_and_properties():
    """oracle qkv_rope (solution/attention.py:28-82) against float64 torch running transformers'
    own apply_rotary_pos_emb on (base + scale * LoRA), within one fp16 ulp; v = base + LoRA
    exactly; backward is the inverse rotation; closed forms and the power-of-two scale."""
    torch = pytest.importorskip("torch")
    qwen2 = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")
    rng = np.random.default_rng(21)
    B, T, nq, nkv = 3, 37, 12, 2
    cos, sin = _qwen_cos_sin(B, T)

    def proj(h):
        return (rng.standard_normal((B, T, h * 128)) * 2).astype(np.float16)

    qa, qb, k, va, vb = proj(nq), proj(nq), proj(nkv), proj(nkv), proj(nkv)
    q, ko, v = O.qkv_rope(qa, qb, k, va, vb, cos, sin, nq, nkv, 2.0, 2.0)

    def heads(x, h):
        return torch.from_numpy(np.asarray(x, np.float64)).view(B, T, h, 128).transpose(1, 2)

    c64, s64 = torch.from_numpy(cos.astype(np.float64)), torch.from_numpy(sin.astype(np.float64))
    xq = heads(qa.astype(np.float64) + 2.0 * qb.astype(np.float64), nq)
    rq, rk = qwen2.apply_rotary_pos_emb(xq, heads(k, nkv), c64, s64)
    back = lambda t, h: t.transpose(1, 2).reshape(B, T, h * 128).numpy()  # noqa: E731
    # fp32 outputs within fp32 rounding of two products and a sum: 2^-22 (|x1 c| + |x2 s|) ...
    q32, k32o, _ = O.qkv_rope(qa, qb, k, None, None, cos, sin, nq, nkv, 2.0, 2.0,
                              out_dtype=np.float32)
    for got, ref, x, h in ((q32, back(rq, nq), qa.astype(np.float64) + 2.0 * qb, nq),
                           (k32o, back(rk, nkv), k.astype(np.float64), nkv)):
        xh = x.reshape(B, T, h, 2, 64)
        c_, s_ = cos.reshape(B, T, 1, 2, 64), sin.reshape(B, T, 1, 2, 64)
        mag = np.abs(xh) * np.abs(c_) + np.abs(xh[:, :, :, ::-1]) * np.abs(s_)
        assert np.all(np.abs(got - ref) <= 2.0 ** -22 * mag.reshape(got.shape))
    # ... and the fp16 outputs are those values rounded once (round to nearest even)
    assert np.array_equal(q, q32.astype(np.float16)) and np.array_equal(ko, k32o.astype(np.float16))
    assert np.array_equal(v, (va.astype(np.float32) + 2.0 * vb.astype(np.float32)).astype(np.float16))
    # a power-of-two scale equals adding the pre-scaled LoRA (solution/test_attention.py:226-246)
    q2, k2, v2 = O.qkv_rope(qa, (qb.astype(np.float32) * 2).astype(np.float16), k, va,
                            (vb.astype(np.float32) * 2).astype(np.float16), cos, sin, nq, nkv)
    assert np.array_equal(q2, q) and np.array_equal(k2, ko) and np.array_equal(v2, v)
    # backward rotates by the opposite angle: fp32 forward then backward restores the input
    x32 = rng.standard_normal((B, T, nq * 128)).astype(np.float32)
    k32 = rng.standard_normal((B, T, nkv * 128)).astype(np.float32)
    y, yk, _ = O.qkv_rope(x32, None, k32, None, None, cos, sin, nq, nkv, out_dtype=np.float32)
    xb, kb, _ = O.qkv_rope(y, None, yk, None, None, cos, sin, nq, nkv, backward=True,
                           out_dtype=np.float32)
    assert np.abs(xb - x32).max() < 1e-5 and np.abs(kb - k32).max() < 1e-5
    # with cos / sin rows whose halves differ (Qwen's are equal, which would hide a swapped half):
    # the forward against transformers' formula, and the backward as the forward's transpose,
    # <R x, g> = <x, R^T g>
    cr = rng.uniform(-1, 1, (B, T, 128)).astype(np.float32)
    sr = rng.uniform(-1, 1, (B, T, 128)).astype(np.float32)
    yr, _, _ = O.qkv_rope(x32, None, k32, None, None, cr, sr, nq, nkv, out_dtype=np.float32)
    ref_r, _ = qwen2.apply_rotary_pos_emb(heads(x32, nq), heads(k32, nkv),
                                          torch.from_numpy(cr.astype(np.float64)),
                                          torch.from_numpy(sr.astype(np.float64)))
    assert np.abs(yr - back(ref_r, nq)).max() < 1e-5 * np.abs(yr).max()
    g = rng.standard_normal(y.shape).astype(np.float32)
    rtg, _, _ = O.qkv_rope(g, None, k32, None, None, cr, sr, nq, nkv, backward=True,
                           out_dtype=np.float32)
    lhs = float(np.sum(yr.astype(np.float64) * g))
    rhs = float(np.sum(x32.astype(np.float64) * rtg))
    assert abs(lhs - rhs) < 1e-5 * float(np.sum(np.abs(yr.astype(np.float64) * g)))
    # pair norms preserved (Qwen's cos / sin halves are equal)
    pair = lambda t: t.reshape(B, T, nq, 2, 64)  # noqa: E731
    n_in = (pair(x32).astype(np.float64) ** 2).sum(axis=3)
    n_out = (pair(y).astype(np.float64) ** 2).sum(axis=3)
    assert np.abs(n_in - n_out).max() < 1e-4 * n_in.max()
    # closed forms: angle 0 is the identity, angle pi/2 maps (x1, x2) -> (-x2, x1)
    one, zero = np.ones((1, T, 128), np.float32), np.zeros((1, T, 128), np.float32)
    i_q, _, _ = O.qkv_rope(qa, None, k, None, None, one, zero, nq, nkv)
    assert np.array_equal(i_q.astype(np.float32), qa.astype(np.float32))
    r_q, _, _ = O.qkv_rope(qa, None, k, None, None, zero, one, nq, nkv)
    h = qa.reshape(B, T, nq, 2, 64).astype(np.float32)
    want = np.stack([-h[:, :, :, 1], h[:, :, :, 0]], axis=3).reshape(qa.shape)
    assert np.array_equal(r_q.astype(np.float32), want)
    # cos / sin shared over the batch ([1, T, 128]) equal the broadcast rows
    c1, s1 = _qwen_cos_sin(1, T, offsets=False)
    cb, sb = np.repeat(c1, B, axis=0), np.repeat(s1, B, axis=0)
    a1 = O.qkv_rope(qa, qb, k, va, vb, c1, s1, nq, nkv, 2.0, 2.0)
    a2 = O.qkv_rope(qa, qb, k, va, vb, cb, sb, nq, nkv, 2.0, 2.0)
    assert all(np.array_equal(x_, y_) for x_, y_ in zip(a1, a2))


def _finite_f16():
    v = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    return v[np.isfinite(v)]


def _single_rounding_mismatches(p):
    """Finite fp16 inputs whose exact product with fp32(1/(1-p)), rounded once to fp16 (what a
    mixed-precision FMA computes), differs from dropout_fp16's two roundings."""
    x = _finite_f16()
    s = np.float32(1.0 / (1.0 - p))
    with np.errstate(over="ignore"):
        once = (x.astype(np.float64) * np.float64(s)).astype(np.float16)  # exact in float64
    twice = O.dropout_fp16(x, np.ones(x.size, np.uint8), p)
    return int(np.sum(twice.view(np.uint16) != once.view(np.uint16)))


def test_dropout_rates_that_tell_one_rounding_from_two():
    """tests/test_dropout_bits_gpu.py pins the kernels' dropout at p = 0.05, 0.04 and 0.4: the
    workload's rate, where one rounding equals two for every input, and two rates where they
    differ for hundreds of inputs (so a kernel that rounds once fails there)."""
    assert _single_rounding_mismatches(0.05) == 0
    assert _single_rounding_mismatches(0.04) > 100
    assert _single_rounding_mismatches(0.4) > 1000
