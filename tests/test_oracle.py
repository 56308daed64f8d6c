"""Pin the CPU oracle (oracle/oracle.py) before trusting it as the parity reference.

Each check is chosen so that a plausible mistake in the oracle fails it:
  * the reference's own known-answer constructions (tests/test_cuda_ops.py:493-509,
    tests/test_quantization.py:16-24);
  * exact rational arithmetic with hand-written IEEE rounding (tests/exact.py), which
    catches a wrong rounding mode, a non-IEEE division or a reordered epilogue;
  * exhaustive sweeps over all BF16 inputs for fixed scales;
  * brute-force integer products on small shapes.
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O
from tests import exact as E


def bf16_from_f32(values):
    """BF16 bits of float32 values that are exactly representable (high half only)."""
    v = np.asarray(values, dtype=np.float32).view(np.uint32)
    assert np.all((v & 0xFFFF) == 0)
    return (v >> 16).astype(np.uint16)


def all_finite_bf16():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = O.bf16_to_f32(bits)
    return bits[np.isfinite(vals)]


# ------------------------------------------------------------------ BF16 rounding

def test_bf16_round_to_nearest_even_known_answers():
    cases = [
        (1.0, 0x3F80),
        (1.0 + 2.0**-8, 0x3F80),            # tie -> even (down)
        (1.0 + 3 * 2.0**-8, 0x3F82),        # tie -> even (up)
        (1.0 + 2.0**-8 + 2.0**-20, 0x3F81),  # above the tie
        (-2.5, 0xC020),
        (float(np.finfo(np.float32).max), 0x7F80),  # rounds up to +inf
        (0.0, 0x0000),
        (-0.0, 0x8000),
    ]
    got = O.f32_to_bf16(np.array([v for v, _ in cases], dtype=np.float32))
    assert [int(g) for g in got] == [b for _, b in cases]
    nan = O.f32_to_bf16(np.array([np.nan], dtype=np.float32))[0]
    assert np.isnan(O.bf16_to_f32(np.array([nan]))[0])


def test_bf16_rounding_matches_exact_on_random_floats():
    rng = np.random.default_rng(5)
    vals = (rng.standard_normal(3000) * np.exp2(rng.integers(-30, 30, 3000))).astype(np.float32)
    got = O.bf16_to_f32(O.f32_to_bf16(vals))
    for v, g in zip(vals, got):
        assert Fraction(float(g)) == E.bf16(Fraction(float(v)))


# ------------------------------------------------------------------ quantize_rows

@pytest.mark.parametrize("width", [4, 3072, 5120, 6144, 8704, 17408])
@pytest.mark.parametrize("rows", [2, 64])
def test_quantize_reference_construction(width, rows):
    """tests/test_cuda_ops.py:493-509: scale is exactly 1, codes are RNE(x)."""
    rng = np.random.default_rng(742)
    x = np.clip(rng.standard_normal((rows, width)).astype(np.float32) * 100, -127, 127)
    bits = O.f32_to_bf16(x)
    x = O.bf16_to_f32(bits).copy()
    x[:, 0] = -127
    x[0, :4] = [0, -127, 63.5, 127]
    x[1] = 0
    bits = bf16_from_f32(x)
    codes, scales = O.quantize_rows(bits)
    expected_scales = np.ones(rows, np.float32)
    expected_scales[1] = np.float32(1e-20)
    assert scales.dtype == np.float32
    assert np.array_equal(scales, expected_scales)
    # Python's round() is round-half-to-even on exact binary values.
    table = {v: round(float(v)) for v in np.unique(x)}
    expected = np.vectorize(table.__getitem__)(x).astype(np.int8)
    assert np.array_equal(codes, expected)
    assert codes[0, :4].tolist() == [0, -127, 64, 127]


def test_quantize_division_is_correctly_rounded():
    rng = np.random.default_rng(11)
    xs = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal(4000).astype(np.float32)))
    ss = (rng.random(4000).astype(np.float32) + np.float32(0.01)) * np.float32(0.05)
    got = (xs / ss).astype(np.float32)
    for x, s, g in zip(xs, ss, got):
        assert Fraction(float(g)) == E.f32(Fraction(float(x)) / Fraction(float(s)))


@pytest.mark.parametrize("amax", [1.0, 3.703125, 127.0, 0.0078125, 5.9e-39, 1.7e38])
def test_quantize_exhaustive_over_bf16_for_fixed_row_max(amax):
    """Every finite BF16 x with |x| <= amax, in a row whose max is amax."""
    amax_bits = bf16_from_f32(np.float32(O.bf16_to_f32(O.f32_to_bf16(np.float32(amax)))))
    amax_v = float(O.bf16_to_f32(np.array([amax_bits]))[0])
    xs_bits = all_finite_bf16()
    xs = O.bf16_to_f32(xs_bits)
    xs_bits = xs_bits[np.abs(xs) <= amax_v]
    rows = np.stack([np.full(xs_bits.shape, amax_bits, np.uint16), xs_bits], axis=1)
    codes, scales = O.quantize_rows(rows)
    scale = E.f32(Fraction(amax_v) / 127)
    scale = max(scale, Fraction(float(np.float32(1e-20))))
    assert np.all(scales == np.float32(float(scale)))
    assert np.all(np.abs(codes) <= 127)
    cache = {}
    for b, c in zip(xs_bits[::7], codes[::7, 1]):
        if b not in cache:
            x = Fraction(float(O.bf16_to_f32(np.array([b]))[0]))
            cache[b] = max(-127, min(127, E.rne_int(E.f32(x / scale))))
        assert int(c) == cache[b]
    # Dequantization error bound |x - q*s| <= s/2 (plus one FP32 rounding of x/s).
    x = O.bf16_to_f32(xs_bits).astype(np.float64)
    err = np.abs(x - codes[:, 1].astype(np.float64) * float(scale))
    assert np.all(err <= float(scale) * (0.5 + 2.0**-16) + 1e-45)


def test_quantize_zero_row_and_nan_handling():
    row = np.zeros((1, 8), np.uint16)
    codes, scales = O.quantize_rows(row)
    assert scales[0] == np.float32(1e-20) and not codes.any()
    vals = np.array([[1.0, -2.0, np.nan, 0.5]], np.float32)
    codes, scales = O.quantize_rows(O.f32_to_bf16(vals))
    assert scales[0] == np.float32(2.0) / np.float32(127.0)  # NaN ignored by the max
    assert codes[0].tolist() == [64, -127, 0, 32]


def test_grouped_row_mapping_known_answer():
    """[M,G,4096] -> [G,M,4096]: codes[g, m] come from x[m, g] (csrc/kernels.cu:46-48)."""
    m, g = 3, 2
    x = np.zeros((m, g, 4096), np.float32)
    for i in range(m):
        for j in range(g):
            x[i, j, 0] = 1 + i * g + j  # distinct row maxima
            x[i, j, 1] = 0.5
    codes, scales = O.quantize_grouped4096(O.f32_to_bf16(x))
    for i in range(m):
        for j in range(g):
            assert scales[j, i] == np.float32(1 + i * g + j) / np.float32(127)
            assert codes[j, i, 0] == 127
    empty_codes, empty_scales = O.quantize_grouped4096(np.zeros((0, 4, 4096), np.uint16))
    assert empty_codes.shape == (4, 0, 4096) and empty_scales.shape == (4, 0)


# ------------------------------------------------------------------ W8A8 GEMMs

def test_int_matmul_bruteforce_and_extremes():
    rng = np.random.default_rng(3)
    a = rng.integers(-128, 128, (5, 96)).astype(np.int8)
    w = rng.integers(-128, 128, (7, 96)).astype(np.int8)
    got = O.int_matmul(a, w)
    for i in range(5):
        for j in range(7):
            assert got[i, j] == sum(int(a[i, t]) * int(w[j, t]) for t in range(96))
    k = 65536
    ones = np.full((1, k), -128, np.int8)
    assert O.int_matmul(ones, ones)[0, 0] == 128 * 128 * k == 2**30
    assert O.int_matmul(ones, np.full((1, k), 127, np.int8))[0, 0] == -128 * 127 * k


def exact_epilogue(acc, sa, sw_bits):
    accf = E.f32(Fraction(int(acc)))
    first = E.f32(accf * Fraction(float(sa)))
    second = E.f32(first * Fraction(float(O.bf16_to_f32(np.array([sw_bits]))[0])))
    return E.bf16_bits(float(E.bf16(second)))


def test_epilogue_matches_exact_rounding():
    rng = np.random.default_rng(7)
    acc = rng.integers(-(2**28), 2**28, (40, 30)).astype(np.int32)
    acc[0, :5] = [0, 1, -1, 2**24 + 1, -(2**24) - 3]  # int->float rounding cases
    sa = (rng.random(40).astype(np.float32) / np.float32(127))
    sw = O.f32_to_bf16(rng.random(30).astype(np.float32) / np.float32(127))
    got = O.channel_epilogue(acc, sa, sw)
    for i in range(40):
        for j in range(30):
            assert int(got[i, j]) == exact_epilogue(acc[i, j], sa[i], sw[j])


def test_epilogue_applies_row_scale_first():
    """Inputs where (acc*sa)*sw and (acc*sw)*sa round to different BF16 values: the
    oracle must give the row-scale-first result, confirmed with exact arithmetic."""
    rng = np.random.default_rng(9)
    count = 1 << 22
    acc = rng.integers(1, 2**26, count).astype(np.int32)
    sa = (rng.random(count).astype(np.float32) / np.float32(127))
    swb = O.f32_to_bf16(rng.random(count).astype(np.float32) / np.float32(127))
    swf = O.bf16_to_f32(swb)
    accf = acc.astype(np.float32)
    row_first = O.f32_to_bf16((accf * sa) * swf)
    ch_first = O.f32_to_bf16((accf * swf) * sa)
    idx = np.nonzero(row_first != ch_first)[0][:20]
    assert idx.size > 0
    got = O.channel_epilogue(acc[idx][:, None], sa[idx], swb[idx])  # [i, i] pairs below
    for j, i in enumerate(idx):
        expected = exact_epilogue(acc[i], sa[i], swb[i])
        assert int(got[j, j]) == expected != int(ch_first[i])


def test_channel_mm_debias_and_cutlass_workspace():
    rng = np.random.default_rng(17)
    a = rng.integers(-127, 128, (3, 64)).astype(np.int8)
    w_u8 = rng.integers(1, 256, (5, 64)).astype(np.uint8)
    signed = (w_u8.astype(np.int16) - 128).astype(np.int8)
    assert np.array_equal(O.debias(w_u8), signed)
    sa = rng.random(3).astype(np.float32) / np.float32(127)
    sw = O.f32_to_bf16(rng.random(5).astype(np.float32) / np.float32(127))
    assert np.array_equal(O.channel_mm(a, w_u8, sa, sw), O.fused_channel_mm(a, signed, sa, sw))
    ws, out = O.cutlass_channel_mm(a, signed, sa, sw)
    assert np.array_equal(ws, a.astype(np.int64) @ signed.astype(np.int64).T)
    assert np.array_equal(out, O.fused_channel_mm(a, signed, sa, sw))


def test_grouped_summed_mm_bruteforce():
    rng = np.random.default_rng(23)
    g, m, n, k = 3, 4, 5, 32
    codes = rng.integers(-127, 128, (g, m, k)).astype(np.int8)
    w = rng.integers(-127, 128, (g, n, k)).astype(np.int8)
    sa = rng.random((g, m)).astype(np.float32) / np.float32(127)
    sw = O.f32_to_bf16(rng.random(n).astype(np.float32) / np.float32(127))
    got = O.grouped_summed_mm(codes, sa, w, sw)
    swf = O.bf16_to_f32(sw)
    for i in range(m):
        for j in range(n):
            total = None
            for gg in range(g):
                acc = sum(int(codes[gg, i, t]) * int(w[gg, j, t]) for t in range(k))
                term = E.f32(E.f32(E.f32(Fraction(acc)) * Fraction(float(sa[gg, i]))) * Fraction(float(swf[j])))
                total = term if total is None else E.f32(total + term)
            assert int(got[i, j]) == E.bf16_bits(float(E.bf16(total)))


# ------------------------------------------------------------------ W8A16 GEMV

def test_gemv_dequant_and_dot_exact_small():
    rng = np.random.default_rng(134)
    m, n, k = 2, 3, 48
    x = O.f32_to_bf16(rng.standard_normal((m, k)).astype(np.float32))
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s = O.f32_to_bf16((rng.random(n) * 0.002).astype(np.float32))
    wq = O.dequantize_bf16(w, s)
    sf = O.bf16_to_f32(s)
    for j in range(n):
        for t in range(k):
            exp = E.bf16(Fraction(int(w[j, t])) * Fraction(float(sf[j])))  # product exact in FP32
            assert Fraction(float(O.bf16_to_f32(np.array([wq[j, t]]))[0])) == exp
    out, exact_vals = O.channel_gemv(x, w, s)
    xf = O.bf16_to_f32(x)
    wqf = O.bf16_to_f32(wq)
    for i in range(m):
        for j in range(n):
            dot = sum(Fraction(float(xf[i, t])) * Fraction(float(wqf[j, t])) for t in range(k))
            assert abs(Fraction(exact_vals[i, j]) - dot) <= abs(dot) * Fraction(1, 2**50) + Fraction(1, 2**120)
            # double rounding f64 -> f32 -> bf16, as torch's .bfloat16() on a double
            assert int(out[i, j]) == E.bf16_bits(float(E.bf16(E.f32(Fraction(float(exact_vals[i, j]))))))


# ------------------------------------------------------------------ weight encoding

def test_quantize_channel_known_answer():
    """tests/test_quantization.py:16-24."""
    weight = np.array([[0.0, -127.0, 63.5, 127.0], [0.0, 0.0, 0.0, 0.0]], np.float32)
    codes, scale = O.quantize_channel(weight)
    assert codes.dtype == np.uint8
    assert codes.tolist() == [[128, 1, 192, 255], [128, 128, 128, 128]]
    assert O.bf16_to_f32(scale)[0] == 1.0
    deq = O.dequantize_channel(codes, scale)
    assert np.isfinite(deq).all()
    assert np.array_equal(deq[1], weight[1])


def test_quantize_channel_rejects_nonfinite_and_matches_exact():
    with pytest.raises(ValueError, match="non-finite"):
        O.quantize_channel(np.array([[1.0, np.inf]], np.float32))
    rng = np.random.default_rng(4)
    w = rng.standard_normal((6, 40)).astype(np.float32)
    codes, scale_bits = O.quantize_channel(w)
    for i in range(6):
        amax = max(abs(Fraction(float(v))) for v in w[i])
        s = E.f32(amax / 127)
        for t in range(40):
            q = max(-128, min(127, E.rne_int(E.f32(Fraction(float(w[i, t])) / s))))
            assert int(codes[i, t]) == q + 128
        assert int(scale_bits[i]) == E.bf16_bits(float(E.bf16(s)))


# ------------------------------------------------------------------ SwiGLU

def swiglu_bits(gate, up):
    """BF16 x [M, 2K] = [gate | up] from float values that are exact in BF16."""
    return np.concatenate([bf16_from_f32(gate), bf16_from_f32(up)], axis=-1)


def test_round_bf16_f64_matches_exact_rational_rounding():
    """Midpoints, near-midpoints, subnormals and the overflow edge against
    tests/exact.py's hand-written round-half-to-even."""
    vals = O.bf16_to_f32(all_finite_bf16()).astype(np.float64)
    vals = np.unique(np.abs(vals))
    mids = (vals[:-1] + vals[1:]) / 2
    rng = np.random.default_rng(21)
    cases = np.concatenate([mids, mids * (1 + 2.0**-40), mids * (1 - 2.0**-40),
                            rng.standard_normal(4000) * 10.0 ** rng.uniform(-40, 38, 4000)])
    cases = rng.choice(cases, 6000, replace=False)
    cases = np.concatenate([cases, -cases, [3.3961e38, 3.3963e38, 1e-45, 2.0**-134]])
    got = O.round_bf16_f64(cases)
    for v, g in zip(cases, got):
        want = E.bf16(Fraction(float(v)))
        assert float(want) == g, (v, g, want)


def test_silu_mul_known_answers():
    """Closed forms: silu(0) = 0, silu(1) = 1/(1 + 1/e), silu(g) -> g for large g, and
    the FP32 overflow of e^-g for g <= -89 (the quotient is then -0)."""
    gate = np.array([[0.0, 1.0, 100.0, -89.0, 2.0, -1.0]], np.float32)
    up = np.array([[5.0, 1.0, 1.0, 1.0, -3.0, 1.0]], np.float32)
    x = swiglu_bits(gate, up)
    exact = O.silu_mul_exact(x)
    assert exact[0, 0] == 0.0
    assert exact[0, 1] == pytest.approx(1.0 / (1.0 + np.exp(-1.0)), rel=1e-15)
    assert exact[0, 2] == 100.0
    assert exact[0, 3] == 0.0 and np.signbit(exact[0, 3])
    assert exact[0, 4] == pytest.approx(-3.0 * 2.0 / (1.0 + np.exp(-2.0)), rel=1e-15)
    bits = O.silu_mul(x)
    # 0.7310585786 / 2^-8 = 187.15 -> 187 * 2^-8 = 0.73046875 = 0x3F3B
    assert int(bits[0, 1]) == 0x3F3B
    assert int(bits[0, 2]) == E.bf16_bits(100.0)
    # -0.2689414214 (silu(-1)): 2^-9 spacing in [0.25, 0.5): 137.70 -> 138 * 2^-9
    assert O.bf16_to_f32(bits[0, 5:6])[0] == np.float32(-138 * 2.0**-9)


def test_silu_mul_matches_independent_sigmoid_and_identity():
    """silu(g) * u = g * expit(g) * u (scipy's logistic, a separate implementation), and
    silu(g) - silu(-g) = g; a swapped gate/up, a sign slip in the exponent or a missing
    factor fails one of them."""
    from scipy.special import expit

    rng = np.random.default_rng(31)
    g = O.bf16_to_f32(O.f32_to_bf16((rng.standard_normal((3, 64)) * 6).astype(np.float32)))
    u = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((3, 64)).astype(np.float32)))
    exact = O.silu_mul_exact(swiglu_bits(g, u))
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    assert np.allclose(exact, g64 * expit(g64) * u64, rtol=1e-14, atol=0)
    ones = np.ones_like(g)
    pos = O.silu_mul_exact(swiglu_bits(g, ones))
    neg = O.silu_mul_exact(swiglu_bits(-g, ones))
    assert np.allclose(pos - neg, g64, rtol=1e-13, atol=1e-13)


def test_silu_mul_bounds_contain_fp32_evaluations_and_reject_planted_mistakes():
    """The tolerance interval holds an FP32 step-by-step evaluation (correctly rounded
    exp, division and product), is a single BF16 value for almost every element, and
    excludes the outputs of plausible mistakes planted in a copy of the formula."""
    rng = np.random.default_rng(41)
    x = O.f32_to_bf16((rng.standard_normal((8, 2 * 8704)) * 3).astype(np.float32))
    lo, hi = O.silu_mul_bounds(x)
    assert np.mean(lo != hi) < 2e-3
    assert np.all(O.within_bounds(O.silu_mul(x), lo, hi))

    f = O.bf16_to_f32(x)
    g, u = f[:, :8704], f[:, 8704:]
    e = np.exp(-g.astype(np.float64)).astype(np.float32)
    d = (np.float32(1) + e).astype(np.float32)
    p = ((g / d).astype(np.float32) * u).astype(np.float32)
    assert np.all(O.within_bounds(O.f32_to_bf16(p), lo, hi))

    def fraction_outside(values):
        return np.mean(~O.within_bounds(O.f32_to_bf16(values.astype(np.float32)), lo, hi))

    assert fraction_outside(g / (1 + np.exp(g)) * u) > 0.5           # sign slip
    assert fraction_outside(u / (1 + np.exp(-u)) * g) > 0.5          # gate and up swapped
    assert fraction_outside(g / (1 + np.exp(-g))) > 0.5              # product dropped
    bf16_silu = O.bf16_to_f32(O.f32_to_bf16((g / d).astype(np.float32)))
    assert fraction_outside(bf16_silu * u) > 0.01                    # extra BF16 rounding


def test_silu_mul_quantize_is_quantize_rows_of_the_activations():
    """csrc/silu_quant.cu:32-56 quantizes the BF16-rounded values with quantize_rows'
    arithmetic; a zero row (tests/test_cuda_ops.py:884) gets scale 1e-20 and zero codes."""
    rng = np.random.default_rng(51)
    x = O.f32_to_bf16((rng.standard_normal((5, 2 * 8704)) * 3).astype(np.float32))
    x[0] = 0
    codes, scales = O.silu_mul_quantize(x)
    ref_codes, ref_scales = O.quantize_rows(O.silu_mul(x))
    assert np.array_equal(codes, ref_codes) and np.array_equal(scales, ref_scales)
    assert scales[0] == np.float32(1e-20) and not codes[0].any()
    act = O.bf16_to_f32(O.silu_mul(x)[1:]).astype(np.float64)
    amax = np.abs(act).max(axis=1)
    assert np.array_equal(scales[1:], np.maximum((amax / 127).astype(np.float32), np.float32(1e-20)))
    for r in range(1, 5):
        s = E.f32(Fraction(float(amax[r - 1])) / 127)
        for t in rng.choice(8704, 40, replace=False):
            q = E.rne_int(E.f32(Fraction(float(act[r - 1, t])) / s))
            assert int(codes[r, t]) == max(-127, min(127, q))


# ------------------------------------------------------------------ AllSpark N32K16

def reference_unpack_loops(packed, packed_scales, n, k):
    """The reference kernel's word operations (csrc/allspark_layout.cu:10-26) one vector
    at a time on little-endian uint32 words: an independent restatement of the oracle's
    vectorised index map."""
    words = packed.reshape(-1).view("<u4")
    weight = np.zeros((n, k), np.uint8)
    scales = np.zeros(n, np.uint16)
    for vector in range(n * (k // 16)):
        row, tile = divmod(vector, k // 16)
        packed_row = (row // 32) * 8 + row % 8
        offset = packed_row * k * 4 + tile * 64 + ((row % 32) // 16) * 8 + ((row % 16) // 8) * 4
        a, b, c, d = (int(words[offset // 4 + 4 * j]) for j in range(4))
        out = [((a & 0xFFFF) | (b << 16)) & 0xFFFFFFFF, ((c & 0xFFFF) | (d << 16)) & 0xFFFFFFFF,
               (a >> 16) | (b & 0xFFFF0000), (c >> 16) | (d & 0xFFFF0000)]
        piece = np.array([w ^ 0x80808080 for w in out], "<u4").view(np.uint8)
        weight[row, tile * 16:(tile + 1) * 16] = piece
        if tile == 0:
            scales[row] = packed_scales[(row // 32) * 32 + (row % 8) * 4 + (row % 32) // 8]
    return weight.view(np.int8), scales


@pytest.mark.parametrize("n,k", [(16, 16), (48, 80), (64, 32), (128, 512)])
def test_allspark_unpack_matches_the_reference_word_operations(n, k):
    rng = np.random.default_rng(319 + n + k)
    padded = O.allspark_padded_rows(n)
    packed = rng.integers(0, 256, (padded, k)).astype(np.uint8)
    packed_scales = rng.integers(0, 1 << 16, padded).astype(np.uint16)
    w, s = O.unpack_allspark(packed, packed_scales, n)
    rw, rs = reference_unpack_loops(packed, packed_scales, n, k)
    assert np.array_equal(w, rw) and np.array_equal(s, rs)


@pytest.mark.parametrize("n,k", [(16, 16), (48, 80), (128, 512), (5120, 3072)])
def test_allspark_pack_is_the_inverse_and_padding_is_never_read(n, k):
    """tests/test_cuda_ops.py:440-471's shapes: unpack(pack(codes)) == codes - 128 and the
    scales, the index map is a bijection onto the valid bytes, and the padding bytes can
    hold anything."""
    rng = np.random.default_rng(319)
    codes = rng.integers(0, 256, (n, k)).astype(np.uint8)
    scales = rng.integers(0, 1 << 16, n).astype(np.uint16)
    byte, sidx = O.allspark_unpack_index(n, k)
    assert np.unique(byte).size == n * k and np.unique(sidx).size == n
    assert byte.max() < O.allspark_padded_rows(n) * k
    for fill in (0x80, 0x00, 0xFF):
        packed, packed_scales = O.pack_allspark(codes, scales, fill=fill)
        assert packed.shape == (O.allspark_padded_rows(n), k)
        w, s = O.unpack_allspark(packed, packed_scales, n)
        assert np.array_equal(w, (codes.astype(np.int16) - 128).astype(np.int8))
        assert np.array_equal(s, scales)


def test_allspark_known_layout():
    """Hand-read N32K16 placement: packed row 0, tile 0 holds rows 0, 8, 16, 24 for
    k = 0..15; its first 16 bytes are, per row, the codes of k = 0, 1, 8, 9, and its
    second 16 bytes those of k = 2, 3, 10, 11. Packed row 1 holds rows 1, 9, 17, 25;
    scales of rows 0, 8, 16, 24, 1 sit at packed positions 0, 1, 2, 3, 4."""
    n, k = 32, 32
    codes = np.zeros((n, k), np.uint8)
    for r in range(n):
        for c in range(k):
            codes[r, c] = (r * 5 + c * 3) % 256
    scales = np.arange(100, 100 + n, dtype=np.uint16)
    packed, packed_scales = O.pack_allspark(codes, scales)
    flat = packed.reshape(-1)
    expect0 = [codes[r, c] for r in (0, 8, 16, 24) for c in (0, 1, 8, 9)]
    expect1 = [codes[r, c] for r in (0, 8, 16, 24) for c in (2, 3, 10, 11)]
    assert flat[:16].tolist() == expect0
    assert flat[16:32].tolist() == expect1
    # tile 1 of packed row 0 (k = 16..31) follows at byte 64; packed row 1 at 4k = 128
    assert flat[64:68].tolist() == [codes[0, c] for c in (16, 17, 24, 25)]
    assert flat[128:132].tolist() == [codes[1, c] for c in (0, 1, 8, 9)]
    assert packed_scales[:5].tolist() == [100, 108, 116, 124, 101]


# ------------------------------------------------------------------ block-32 Q8_0

def test_fma_f32_matches_exact_single_rounding():
    """Random operands and constructed halfway cases (a*b + c exactly between two
    float32 values, then nudged by a tiny c) against exact rationals."""
    rng = np.random.default_rng(61)
    a = (rng.standard_normal(3000) * 10.0 ** rng.integers(-8, 8, 3000)).astype(np.float32)
    b = (rng.standard_normal(3000) * 10.0 ** rng.integers(-8, 8, 3000)).astype(np.float32)
    c = (rng.standard_normal(3000) * 10.0 ** rng.integers(-12, 12, 3000)).astype(np.float32)
    # halfway constructions: (1 + i 2^-12)(1 + j 2^-12) with i, j odd has 25 significant
    # bits, so it lies exactly halfway between two float32 values; c = 0 ties to even,
    # c = +/- 2^-60 decides the side.
    i = rng.integers(0, 512, 300) * 2 + 1
    j = rng.integers(0, 512, 300) * 2 + 1
    ha = (1 + i * 2.0**-12).astype(np.float32)
    hb = (1 + j * 2.0**-12).astype(np.float32)
    assert all(E.f32(Fraction(float(p)) * Fraction(float(q))) != Fraction(float(p)) * Fraction(float(q))
               for p, q in zip(ha[:20], hb[:20]))
    tiny = np.float32(2.0**-60)
    a = np.concatenate([a, ha, ha, ha]).astype(np.float32)
    b = np.concatenate([b, hb, hb, hb]).astype(np.float32)
    c = np.concatenate([c, np.zeros(300, np.float32), np.full(300, tiny), np.full(300, -tiny)])
    plain = (a.astype(np.float64) * b + c).astype(np.float32)  # double rounding
    assert np.sum(plain != O.fma_f32(a, b, c)) > 100         # the cases that matter
    got = O.fma_f32(a, b, c)
    for x, y, z, g in zip(a, b, c, got):
        exact = Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z))
        want = E.f32(exact)
        assert float(want) == float(g), (x, y, z, g, float(want))


def test_quantize_block32_is_quantize_rows_per_block():
    """benchmarks/cuda/q8_block_int8.cu:11-23: a zero block gets 1e-20, a x100 block is
    scaled on its own, and each block matches quantize_rows of those 32 values."""
    rng = np.random.default_rng(62)
    x = (rng.standard_normal((5, 96)) * 0.1).astype(np.float32)
    x[:, :32] = 0
    x[:, 32:64] *= 100
    bits = O.f32_to_bf16(x)
    codes, scales = O.quantize_block32(bits)
    assert scales.shape == (5, 3) and codes.shape == (5, 96)
    assert np.all(scales[:, 0] == np.float32(1e-20)) and not codes[:, :32].any()
    for r in range(5):
        for blk in range(3):
            c, s = O.quantize_rows(bits[r:r + 1, 32 * blk:32 * blk + 32])
            assert np.array_equal(codes[r:r + 1, 32 * blk:32 * blk + 32], c)
            assert scales[r, blk] == s[0]


def test_q8_block_mm_matches_exact_rationals_and_the_reference_tolerance():
    """The oracle's GEMM against a Fraction evaluation of the same rounding sequence on
    a tiny case, and against the reference benchmark's own checks
    (benchmarks/benchmark_q8_block_int8.py:90-121): the blockwise dot-product oracle
    within rtol 0.008 / atol 1e-5 and the dense product within 1.5% relative."""
    rng = np.random.default_rng(63)
    m, n, k = 3, 5, 96
    x = (rng.standard_normal((m, k)) * 0.1).astype(np.float32)
    x[:, 32:64] *= 100
    bits = O.f32_to_bf16(x)
    a, sa = O.quantize_block32(bits)
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    sw = (rng.standard_normal((n, k // 32)) * 0.01).astype(np.float16).view(np.uint16)
    y = O.q8_block_mm(a, sa, w, sw)
    swf = O.f16_to_f32(sw)
    for r in range(m):
        for c in range(n):
            total = Fraction(0)
            for blk in range(k // 32):
                acc = int(np.dot(a[r, 32 * blk:32 * blk + 32].astype(np.int64),
                                 w[c, 32 * blk:32 * blk + 32].astype(np.int64)))
                scale = E.f32(Fraction(float(sa[r, blk])) * Fraction(float(swf[c, blk])))
                total = E.f32(Fraction(acc) * scale + total)
            assert int(y[r, c]) == E.bf16_bits(float(E.bf16(total)))
    # the reference benchmark's checks
    blockwise = np.zeros((m, n))
    for blk in range(k // 32):
        dot = a[:, 32 * blk:32 * blk + 32].astype(np.float64) @ w[:, 32 * blk:32 * blk + 32].astype(np.float64).T
        blockwise += dot * (sa[:, blk, None] * swf[None, :, blk])
    got = O.bf16_to_f32(y).astype(np.float64)
    ref_bf16 = O.bf16_to_f32(O.f64_to_bf16(blockwise)).astype(np.float64)
    assert np.all(np.abs(got - ref_bf16) <= 1e-5 + 0.008 * np.abs(ref_bf16))
    dense = O.q8_block_dense_reference(bits, w, sw)
    assert np.linalg.norm(got - dense) / np.linalg.norm(dense) < 0.015


# ------------------------------------------------------------------ GGUF grouped Q8 W8A16

def test_dequantize_q8_0_exact_rationals():
    """bf16_rn(code * fp16 scale), per run of 32 codes: every code, FP16 normal,
    subnormal, negative and zero scales, against Fraction arithmetic with one rounding."""
    codes = np.arange(-128, 128, dtype=np.int32).astype(np.int8).reshape(2, 128)
    scales = np.array([[1.0, -0.0999, 6.1e-5, 3e-7], [0.0, 65504.0, -2.5e-3, 1 / 3]],
                      np.float16).view(np.uint16)
    wq = O.dequantize_q8_0(codes, scales)
    assert wq.shape == (2, 128) and wq.dtype == np.uint16
    sf = scales.view(np.float16).astype(np.float64)
    for r in range(2):
        for t in range(128):
            want = E.bf16(Fraction(int(codes[r, t])) * Fraction(float(sf[r, t // 32])))
            assert int(wq[r, t]) == E.bf16_bits(float(want)), (r, t)
    # grouped leading dimensions dequantize each [N, K] independently
    g3 = np.stack([codes, -codes.astype(np.int16).clip(-128, 127).astype(np.int8), codes])
    s3 = np.stack([scales, scales, scales[::-1]])
    wq3 = O.dequantize_q8_0(g3, s3)
    for g in range(3):
        assert np.array_equal(wq3[g], O.dequantize_q8_0(g3[g], s3[g]))


def test_gguf_q8_packed_mm_brute_force_per_group():
    """Exact rational dot products per (row, group, channel) on a tiny grouped case, with
    distinct groups so that a swapped row/group index or a transposed operand fails."""
    rng = np.random.default_rng(95)
    m, g, n, k = 2, 3, 4, 64
    x = O.f32_to_bf16(rng.standard_normal((m, g, k)).astype(np.float32))
    codes = rng.integers(-128, 128, (g, n, k)).astype(np.int8)
    scales = (rng.random((g, n, k // 32)) * 0.1 * np.array([1, 10, 100])[:, None, None]
              ).astype(np.float16).view(np.uint16)
    out, exact_vals = O.gguf_q8_packed_mm(x, codes, scales)
    assert out.shape == (m, g, n) and exact_vals.shape == (m, g, n)
    xf = O.bf16_to_f32(x)
    sf = scales.view(np.float16).astype(np.float64)
    for i in range(m):
        for gg in range(g):
            for j in range(n):
                dot = Fraction(0)
                for t in range(k):
                    wq = E.bf16(Fraction(int(codes[gg, j, t])) * Fraction(float(sf[gg, j, t // 32])))
                    dot += Fraction(float(xf[i, gg, t])) * wq
                assert abs(Fraction(exact_vals[i, gg, j]) - dot) <= abs(dot) * Fraction(1, 2**50) + Fraction(1, 2**120)
                assert int(out[i, gg, j]) == E.bf16_bits(float(E.bf16(E.f32(Fraction(float(exact_vals[i, gg, j]))))))
    bound = O.gguf_q8_abs_bound(x, codes, scales)
    assert bound.shape == (m, g, n) and np.all(bound > 0)


def test_gguf_q8_oracle_meets_the_reference_test():
    """tests/test_gguf_q8.py:22-59 construction: raw blocks = FP16 scale bytes then 32
    codes; pack_q8 recovers codes and scales; the oracle is within the reference's
    relative-norm 0.001 of a float32 bmm of the BF16 dense weights."""
    rng = np.random.default_rng(37)
    groups, n, k, m = 3, 37, 128, 17
    scales = (rng.random((groups, n, k // 32, 1)) * 0.1).astype(np.float16)
    codes = rng.integers(-128, 128, (groups, n, k // 32, 32)).astype(np.int8)
    raw = np.concatenate((scales.view(np.uint8), codes.view(np.uint8)), axis=-1)
    assert raw.shape == (groups, n, k // 32, 34)
    pc, ps = O.pack_q8(raw)
    assert np.array_equal(pc, codes.reshape(groups, n, k))
    assert np.array_equal(ps, scales.view(np.uint16).reshape(groups, n, k // 32))
    # little-endian FP16 scale in the first two bytes of each block
    assert ps[0, 0, 0] == int(raw[0, 0, 0, 0]) | (int(raw[0, 0, 0, 1]) << 8)
    dense = O.f32_to_bf16((scales.astype(np.float32) * codes.astype(np.float32)).reshape(groups, n, k))
    assert np.array_equal(dense, O.dequantize_q8_0(pc, ps))
    x = O.f32_to_bf16(rng.standard_normal((m, groups, k)).astype(np.float32))
    out, _ = O.gguf_q8_packed_mm(x, pc, ps)
    xf = O.bf16_to_f32(x)
    ref = np.stack([xf[:, g] @ O.bf16_to_f32(dense[g]).T for g in range(groups)], axis=1)
    ref = O.bf16_to_f32(O.f32_to_bf16(ref.astype(np.float32))).astype(np.float64)
    got = O.bf16_to_f32(out).astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 0.001
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 0
