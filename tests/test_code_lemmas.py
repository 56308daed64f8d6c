"""CPU checks of two arithmetic shortcuts of the kernels, in numpy float32 (IEEE
round-to-nearest-even, the rounding of v_mul_f32 and of the IEEE division).

1. Codes from the row reciprocal (codes8 in csrc/ci8_device.h, used by quantize_rows,
   quantize_grouped4096, silu_mul_quantize and quantize_block32): with
   inv = fl(1/scale), q0 = fl(v * inv) rounds to the same integer as fl(v / scale)
   whenever q0 is more than 2^-15 from every half-integer; the kernels divide for the
   other values.
2. Reach of the SwiGLU fast path (csrc/silu.hip): for |g| < 87, 1 + e^-g stays below
   2^126, so its reciprocal is a normal number.
"""

import numpy as np

from oracle import oracle as O

BAND = np.float32(2.0**-15)


def finite_bf16_values():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = O.bf16_to_f32(bits)
    return vals[np.isfinite(vals)]


def rne(q):
    return np.rint(q.astype(np.float64))


def test_row_reciprocal_codes_equal_ieee_division_outside_the_band():
    vals = finite_bf16_values()
    positive = np.unique(np.abs(vals[vals != 0]))
    rng = np.random.default_rng(5)
    amaxes = np.concatenate([rng.choice(positive, 400, replace=False),
                             positive[:8], positive[-8:],
                             O.bf16_to_f32(O.f32_to_bf16(np.float32([127.0, 1.0, 3.0, 1e-18, 7e-19])))])
    checked = near_total = 0
    for amax in amaxes.astype(np.float32):
        scale = np.maximum(np.float32(amax / np.float32(127)), np.float32(1e-20))
        inv = np.float32(np.float32(1) / scale)
        v = vals[np.abs(vals) <= amax]
        q0 = (v * inv).astype(np.float32)
        ieee = (v / scale).astype(np.float32)
        assert np.all(np.abs(ieee) < 128)
        frac = (q0 - np.floor(q0)).astype(np.float32)
        near = np.abs((frac - np.float32(0.5)).astype(np.float32)) <= BAND
        assert np.array_equal(rne(q0)[~near], rne(ieee)[~near]), amax
        checked += v.size
        near_total += int(near.sum())
    assert checked > 10_000_000
    assert near_total / checked < 1e-3


def test_fast_path_reciprocal_stays_normal():
    """|g| < 87 for every BF16 gate the fast path takes: 1 + e^87 < 2^126."""
    vals = finite_bf16_values().astype(np.float64)
    fast = vals[np.abs(vals) < 87]
    assert np.max(-fast) < 87
    assert 1 + np.exp(87.0) < 2.0**126
    assert 1 / (1 + np.exp(87.0)) > np.finfo(np.float32).tiny
