"""Writes the golden fixtures in this directory. Run from the repository root:

    python tests/golden/make_golden.py

known_answers.json holds the known-answer vectors of the reference's own tests as data
(inputs and the expected outputs those tests assert), with their source lines:
  * quantize_channel: tests/test_quantization.py:16-24 of the reference;
  * quantize_rows: the construction of tests/test_cuda_ops.py:493-509 (BF16 values of
    x*100 clamped to [-127, 127], column 0 set to -127 so every scale is exactly 1, row 1
    zero so its scale is 1e-20, row 0 starting [0, -127, 63.5, 127]); the expected codes
    are round-half-to-even of x, which is what that test asserts (x.float().round()).
The construction's random values come from numpy here (the reference draws them from
torch's generator); the asserted property is the same for any values.

vectors.npz holds small seeded inputs for every op with the oracle's outputs, so GPU
runs compare against committed data and any change to the oracle shows up as a diff.
"""

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import oracle as O  # noqa: E402


def bf16_exact(values):
    """BF16 bits of float32 values that BF16 represents exactly."""
    v = np.asarray(values, dtype=np.float32).view(np.uint32)
    assert np.all((v & 0xFFFF) == 0), "value not exactly representable in BF16"
    return (v >> 16).astype(np.uint16)


def quantize_rows_construction(rows, width, seed):
    rng = np.random.default_rng(seed)
    x = np.clip(O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((rows, width)).astype(np.float32)))
                * np.float32(100), -127, 127).astype(np.float32)
    x = O.bf16_to_f32(O.f32_to_bf16(x))  # the multiply and clamp happen in BF16 there
    x[:, 0] = -127
    x[0, :4] = [0, -127, 63.5, 127]
    x[1] = 0
    bits = bf16_exact(x)
    expected_codes = np.rint(O.bf16_to_f32(bits)).astype(np.int8)  # torch.round: half to even
    expected_scales = np.ones(rows, np.float32)
    expected_scales[1] = np.float32(1e-20)
    return bits, expected_codes, expected_scales


def known_answers():
    cases = {
        "quantize_channel": {
            "source": "tests/test_quantization.py:16-24",
            "weight": [[0.0, -127.0, 63.5, 127.0], [0.0, 0.0, 0.0, 0.0]],
            "codes": [[128, 1, 192, 255], [128, 128, 128, 128]],
            "scale0": 1.0,
        },
        "quantize_rows": [],
    }
    for width in (4, 3072, 5120):
        bits, codes, scales = quantize_rows_construction(3, width, seed=742 + width)
        cases["quantize_rows"].append({
            "source": "tests/test_cuda_ops.py:493-509",
            "x_bf16_bits": bits.tolist(),
            "codes": codes.tolist(),
            "scales_f32_bits": scales.view(np.uint32).tolist(),
        })
    return cases


def vectors():
    rng = np.random.default_rng(2026)
    out = {}
    x = O.f32_to_bf16(rng.standard_normal((8, 4096)).astype(np.float32))
    x[3, :] = 0
    out["q_x"] = x
    out["q_codes"], out["q_scales"] = O.quantize_rows(x)
    xg = O.f32_to_bf16(rng.standard_normal((5, 2, 4096)).astype(np.float32))
    out["qg_x"] = xg
    out["qg_codes"], out["qg_scales"] = O.quantize_grouped4096(xg)
    m, n, k = 16, 68, 256
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    sa = (rng.random(m).astype(np.float32) / np.float32(127)).astype(np.float32)
    sw = O.f32_to_bf16((rng.random(n).astype(np.float32) - np.float32(0.5)) / np.float32(64))
    out.update(mm_a=a, mm_w=w, mm_sa=sa, mm_sw=sw)
    out["mm_acc"], out["mm_out"] = O.cutlass_channel_mm(a, w, sa, sw)
    w_u8 = rng.integers(0, 256, (n, k)).astype(np.uint8)
    out["cm_w"] = w_u8
    out["cm_out"] = O.channel_mm(a, w_u8, sa, sw)
    gx = O.f32_to_bf16(rng.standard_normal((4, 512)).astype(np.float32))
    gw = rng.integers(-127, 128, (64, 512)).astype(np.int8)
    gs = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, 64).astype(np.float32))
    out.update(gv_x=gx, gv_w=gw, gv_s=gs)
    out["gv_ref"], out["gv_exact"] = O.channel_gemv(gx, gw, gs)
    g, gm, gn, gk = 3, 8, 12, 64
    ga = rng.integers(-127, 128, (g, gm, gk)).astype(np.int8)
    gww = rng.integers(-127, 128, (g, gn, gk)).astype(np.int8)
    gsa = (rng.random((g, gm)).astype(np.float32) / np.float32(127)).astype(np.float32)
    gsw = O.f32_to_bf16((rng.random(gn).astype(np.float32) - np.float32(0.5)) / np.float32(64))
    out.update(gs_a=ga, gs_w=gww, gs_sa=gsa, gs_sw=gsw)
    out["gs_out"] = O.grouped_summed_mm(ga, gsa, gww, gsw)
    return out


def main():
    (HERE / "known_answers.json").write_text(json.dumps(known_answers()) + "\n")
    np.savez_compressed(HERE / "vectors.npz", **vectors())


if __name__ == "__main__":
    main()
