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
