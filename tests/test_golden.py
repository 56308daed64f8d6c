"""Committed golden fixtures (tests/golden/): the reference tests' known answers and
small seeded vectors for every op.

CPU: the oracle reproduces the known answers of the reference's own tests and the
committed vectors. GPU: the HIP ops reproduce the same fixtures (bit-exact, the GEMV
within its tolerance).
"""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def known_answers():
    return json.loads((GOLDEN / "known_answers.json").read_text())


def vectors():
    with np.load(GOLDEN / "vectors.npz") as data:
        return {name: data[name] for name in data.files}


def test_oracle_quantize_channel_known_answer():
    case = known_answers()["quantize_channel"]
    codes, scale_bits = O.quantize_channel(np.asarray(case["weight"], np.float32))
    assert codes.tolist() == case["codes"]
    assert O.bf16_to_f32(scale_bits)[0] == np.float32(case["scale0"])


def test_oracle_quantize_rows_known_answers():
    for case in known_answers()["quantize_rows"]:
        x = np.asarray(case["x_bf16_bits"], np.uint16)
        codes, scales = O.quantize_rows(x)
        assert np.array_equal(codes, np.asarray(case["codes"], np.int8))
        assert np.array_equal(scales.view(np.uint32), np.asarray(case["scales_f32_bits"], np.uint32))


def test_oracle_reproduces_committed_vectors():
    v = vectors()
    codes, scales = O.quantize_rows(v["q_x"])
    assert np.array_equal(codes, v["q_codes"]) and np.array_equal(scales, v["q_scales"])
    codes, scales = O.quantize_grouped4096(v["qg_x"])
    assert np.array_equal(codes, v["qg_codes"]) and np.array_equal(scales, v["qg_scales"])
    acc, out = O.cutlass_channel_mm(v["mm_a"], v["mm_w"], v["mm_sa"], v["mm_sw"])
    assert np.array_equal(acc, v["mm_acc"]) and np.array_equal(out, v["mm_out"])
    assert np.array_equal(O.channel_mm(v["mm_a"], v["cm_w"], v["mm_sa"], v["mm_sw"]), v["cm_out"])
    ref, exact = O.channel_gemv(v["gv_x"], v["gv_w"], v["gv_s"])
    assert np.array_equal(ref, v["gv_ref"]) and np.array_equal(exact, v["gv_exact"])
    out = O.grouped_summed_mm(v["gs_a"], v["gs_sa"], v["gs_w"], v["gs_sw"])
    assert np.array_equal(out, v["gs_out"])


@pytest.mark.gpu
def test_gpu_quantize_rows_known_answers(ops):
    import torch

    from tests.helpers import host, to_dev

    for case in known_answers()["quantize_rows"]:
        x = np.asarray(case["x_bf16_bits"], np.uint16)
        codes = torch.empty(x.shape, dtype=torch.int8, device="cuda")
        scales = torch.empty(x.shape[0], device="cuda")
        ops.quantize_rows(to_dev(x), codes, scales)
        torch.cuda.synchronize()
        assert np.array_equal(host(codes), np.asarray(case["codes"], np.int8))
        assert np.array_equal(host(scales).view(np.uint32),
                              np.asarray(case["scales_f32_bits"], np.uint32))


@pytest.mark.gpu
def test_gpu_ops_reproduce_committed_vectors(ops):
    import torch

    from tests.helpers import bf16_bits, host, to_dev

    v = vectors()
    dev = "cuda"
    codes = torch.empty(v["q_x"].shape, dtype=torch.int8, device=dev)
    scales = torch.empty(v["q_x"].shape[0], device=dev)
    ops.quantize_rows(to_dev(v["q_x"]), codes, scales)
    m, g, k = v["qg_x"].shape
    gcodes = torch.empty(g, m, k, dtype=torch.int8, device=dev)
    gscales = torch.empty(g, m, device=dev)
    ops.quantize_grouped4096(to_dev(v["qg_x"]), gcodes, gscales)
    a, w, sa, sw = to_dev(v["mm_a"]), to_dev(v["mm_w"]), to_dev(v["mm_sa"]), to_dev(v["mm_sw"])
    mm, mn = v["mm_out"].shape
    fused = torch.empty(mm, mn, dtype=torch.bfloat16, device=dev)
    ops.fused_channel_mm(a, w, sa, sw, fused, 0)
    ws = torch.empty(mm, mn, dtype=torch.int32, device=dev)
    cut = torch.empty(mm, mn, dtype=torch.bfloat16, device=dev)
    ops.cutlass_channel_mm(a, w, sa, sw, ws, cut)
    cm = torch.empty(mm, mn, dtype=torch.bfloat16, device=dev)
    ops.channel_mm(a, to_dev(v["cm_w"]), sa, sw, cm)
    gm_, gk = v["gv_x"].shape
    gv = torch.empty(gm_, v["gv_w"].shape[0], dtype=torch.bfloat16, device=dev)
    ops.channel_gemv(to_dev(v["gv_x"]), to_dev(v["gv_w"]), to_dev(v["gv_s"]), gv)
    gs = torch.empty(v["gs_out"].shape, dtype=torch.bfloat16, device=dev)
    ops.grouped_summed_mm(to_dev(v["gs_a"]), to_dev(v["gs_w"]), to_dev(v["gs_sa"]),
                          to_dev(v["gs_sw"]), gs)
    torch.cuda.synchronize()
    assert np.array_equal(host(codes), v["q_codes"]) and np.array_equal(host(scales), v["q_scales"])
    assert np.array_equal(host(gcodes), v["qg_codes"]) and np.array_equal(host(gscales), v["qg_scales"])
    assert np.array_equal(bf16_bits(fused), v["mm_out"])
    assert np.array_equal(host(ws), v["mm_acc"]) and np.array_equal(bf16_bits(cut), v["mm_out"])
    assert np.array_equal(bf16_bits(cm), v["cm_out"])
    got = O.bf16_to_f32(bf16_bits(gv)).astype(np.float64)
    bound = O.bf16_ulp(v["gv_exact"]) + O.gemv_abs_bound(v["gv_x"], v["gv_w"], v["gv_s"])
    assert np.all(np.abs(got - v["gv_exact"]) <= bound)
    assert np.array_equal(bf16_bits(gs), v["gs_out"])
