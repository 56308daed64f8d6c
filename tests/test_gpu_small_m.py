"""GPU parity of the small-M GEMM path (M <= 256 under schedule 0), bit-exact.

configs[0] of the benchmark: quantize_rows on BF16 [128, 4096] N(0,1),
then fused_channel_mm against signed INT8 weights [4096, 4096] U[-127,127] with BF16
channel scales U[1e-3, 1e-2]. The reference runs this shape through its small-M tile
(csrc/fused_mm.cu:89-91) and checks it against the integer product plus the FP32
epilogue (tests/test_cuda_ops.py:596-599); here the whole output is compared with the
oracle bit for bit, inside guard sentinels and under graph replay.

The other cases reach every tile shape the small-M kernel picks (16..64 rows by 16..64
columns), K tails (K % 128 in {32, 64, 96}), K shorter than the four-way K split, and
the workspace and biased-UINT8 variants.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, guard_intact, host, to_dev, with_guard

pytestmark = pytest.mark.gpu


def config0_inputs(seed, m=128, k=4096, n=4096):
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16(rng.standard_normal((m, k)).astype(np.float32))
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sw = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    return x, w, sw


def test_config0_quantize_then_fused_exact_with_guards_and_graph(ops):
    m, k, n = 128, 4096, 4096
    x_np, w_np, sw_np = config0_inputs(128)
    x, w, sw = to_dev(x_np), to_dev(w_np), to_dev(sw_np)
    codes = torch.empty(m, k, device="cuda", dtype=torch.int8)
    scales = torch.empty(m, device="cuda", dtype=torch.float32)
    out, buf = with_guard((m, n), torch.bfloat16, float("nan"))

    def step():
        ops.quantize_rows(x, codes, scales)
        ops.fused_channel_mm(codes, w, scales, sw, out, 0)

    step()
    torch.cuda.synchronize()
    want_codes, want_scales = O.quantize_rows(x_np)
    assert np.array_equal(host(codes), want_codes)
    assert np.array_equal(host(scales).view(np.uint32), want_scales.view(np.uint32))
    want = O.fused_channel_mm(want_codes, w_np, want_scales, sw_np)
    assert np.array_equal(bf16_bits(out), want)
    assert guard_intact(buf, float("nan"))

    # Captured once, replayed on new activations written in place.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for seed in (1, 2):
        x2_np, _, _ = config0_inputs(1000 + seed)
        x.copy_(to_dev(x2_np))
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        c2, s2 = O.quantize_rows(x2_np)
        assert np.array_equal(host(codes), c2)
        assert np.array_equal(bf16_bits(out), O.fused_channel_mm(c2, w_np, s2, sw_np))
        assert guard_intact(buf, float("nan"))


SHAPES = [
    (128, 4096, 4096),   # configs[0]: 64 x 32 tiles
    (17, 17408, 5120),   # 32 x 64
    (33, 5120, 544),     # 16 x 64, K % 128 == 32
    (32, 4096, 1440),    # 32 x 32, K % 128 == 32
    (32, 2560, 96),      # 32 x 16, one K stage: three of the four waves have no K
    (4, 5120, 5120),     # 16 x 32
    (1, 4096, 4096),     # 16 x 16
    (100, 1000, 4000),   # ragged M and N tiles, K % 128 == 32
    (255, 132, 4064),    # K % 128 == 96
    (256, 4096, 576),    # largest M of the path, K % 128 == 64
]


def gemm_inputs(rng, m, n, k, biased=False):
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    w = (rng.integers(1, 256, (n, k)).astype(np.uint8) if biased
         else rng.integers(-127, 128, (n, k)).astype(np.int8))
    sa = (rng.random(m).astype(np.float32) / np.float32(127)).astype(np.float32)
    sw = O.f32_to_bf16(rng.random(n).astype(np.float32) / np.float32(127))
    return a, w, sa, sw


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_small_m_fused_and_workspace_exact(ops, m, n, k):
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k)
    a, w, sa, sw = to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np)
    acc, want = O.cutlass_channel_mm(a_np, w_np, sa_np, sw_np)
    out, buf = with_guard((m, n), torch.bfloat16, float("nan"))
    ops.fused_channel_mm(a, w, sa, sw, out, 0)
    ws = torch.full((m, n), -1, device="cuda", dtype=torch.int32)
    out2 = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.cutlass_channel_mm(a, w, sa, sw, ws, out2)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), want)
    assert guard_intact(buf, float("nan"))
    assert np.array_equal(host(ws), acc)
    assert np.array_equal(bf16_bits(out2), want)


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (17, 37, 544), (33, 5121, 544),
                                   (128, 4096, 4096), (200, 999, 1440), (256, 130, 96)])
def test_small_m_channel_mm_biased_exact(ops, m, n, k):
    rng = np.random.default_rng(m + n + k)
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k, biased=True)
    out, buf = with_guard((m, n), torch.bfloat16, float("nan"))
    ops.channel_mm(to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np), out)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), O.channel_mm(a_np, w_np, sa_np, sw_np))
    assert guard_intact(buf, float("nan"))


def test_small_m_extremes_at_max_k(ops):
    """|acc| = 2^30 at K = 65536 through the four-way K split."""
    m, n, k = 5, 12, 65536
    a_np = np.full((m, k), -128, np.int8)
    a_np[1] = 127
    a_np[2, ::2] = 127
    a_np[3, 1::3] = 0
    w_np = np.full((n, k), -128, np.int8)
    w_np[1::2] = 127
    sa_np = np.array([1.0, 0.5, 3e-3, 1e-7, 2.0], np.float32)
    sw_np = O.f32_to_bf16(np.linspace(0.001, 0.01, n).astype(np.float32))
    ws = torch.empty(m, n, device="cuda", dtype=torch.int32)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.cutlass_channel_mm(to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np), ws, out)
    torch.cuda.synchronize()
    acc, want = O.cutlass_channel_mm(a_np, w_np, sa_np, sw_np)
    assert acc[0, 0] == 2**30
    assert np.array_equal(host(ws), acc) and np.array_equal(bf16_bits(out), want)
