"""GPU parity of grouped_summed_mm, configs[4]'s grouped W8A8 with the per-group INT32
partials scaled and summed (bit-exact against the oracle's closed form).

The reference has no such op (its grouped benchmark keeps separate per-group outputs,
benchmarks/benchmark_grouped_w8a8.py:100-107), so the contract is the build's own:
out = bf16(sum over ascending g of fl(fl(float(acc_g) * sa[g, m]) * float(sw[n]))),
pinned by oracle.grouped_summed_mm's brute-force test. Inputs follow the reference's
grouped call pattern: quantize_grouped4096 codes and scales feed the GEMM directly.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, guard_intact, to_dev, with_guard

pytestmark = pytest.mark.gpu


def grouped_inputs(rng, g, m, n, k, signed_scales=False):
    a = rng.integers(-127, 128, (g, m, k)).astype(np.int8)
    w = rng.integers(-127, 128, (g, n, k)).astype(np.int8)
    sa = (rng.random((g, m)).astype(np.float32) / np.float32(127)).astype(np.float32)
    sw_f = rng.random(n).astype(np.float32) / np.float32(127)
    if signed_scales:  # mixed signs exercise cancellation and signed zeros in the sum
        sw_f *= np.where(rng.random(n) < 0.5, -1, 1).astype(np.float32)
    return a, w, sa, O.f32_to_bf16(sw_f)


@pytest.mark.parametrize("g", [1, 2, 4])
@pytest.mark.parametrize("m", [1, 17, 32, 33, 130, 300])
@pytest.mark.parametrize("n,k", [(4, 32), (132, 96), (256, 4096)])
def test_grouped_summed_matches_oracle(ops, g, m, n, k):
    rng = np.random.default_rng(g * 100003 + m * 101 + n + k)
    a_np, w_np, sa_np, sw_np = grouped_inputs(rng, g, m, n, k, signed_scales=(m % 2 == 1))
    out, buf = with_guard((m, n), torch.bfloat16, float("nan"))
    ops.grouped_summed_mm(to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np), out)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), O.grouped_summed_mm(a_np, sa_np, w_np, sw_np))
    assert guard_intact(buf, float("nan"))


def test_grouped_zero_terms_keep_the_first_terms_sign(ops):
    """A column whose every term is zero: the sum starts from the first term itself, so
    -0 from a negative channel scale survives as the oracle's does."""
    g, m, n, k = 3, 8, 8, 64
    a_np = np.zeros((g, m, k), np.int8)
    w_np = np.ones((g, n, k), np.int8)
    sa_np = np.ones((g, m), np.float32)
    sw_np = O.f32_to_bf16(np.where(np.arange(n) % 2 == 0, -1.0, 1.0).astype(np.float32))
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.grouped_summed_mm(to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np), out)
    torch.cuda.synchronize()
    expected = O.grouped_summed_mm(a_np, sa_np, w_np, sw_np)
    assert np.array_equal(bf16_bits(out), expected)
    assert expected[0, 0] == 0x8000 and expected[0, 1] == 0x0000


def test_grouped_pipeline_from_quantize_grouped4096_and_graph_replay(ops):
    """BF16 [M, G*4096] -> quantize_grouped4096 -> grouped_summed_mm, captured in a HIP
    graph and replayed with new activations."""
    m, g, n = 96, 4, 384
    rng = np.random.default_rng(137)
    x_bits = O.f32_to_bf16(rng.standard_normal((m, g, 4096)).astype(np.float32))
    w_np = rng.integers(-127, 128, (g, n, 4096)).astype(np.int8)
    sw_np = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    x = to_dev(x_bits)
    codes = torch.empty(g, m, 4096, device="cuda", dtype=torch.int8)
    scales = torch.empty(g, m, device="cuda")
    w, sw = to_dev(w_np), to_dev(sw_np)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)

    def run():
        ops.quantize_grouped4096(x, codes, scales)
        ops.grouped_summed_mm(codes, w, scales, sw, out)

    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for replay in range(3):
        x_bits = O.f32_to_bf16(rng.standard_normal((m, g, 4096)).astype(np.float32))
        x.copy_(to_dev(x_bits))
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        c_np, s_np = O.quantize_grouped4096(x_bits)
        assert np.array_equal(bf16_bits(out), O.grouped_summed_mm(c_np, s_np, w_np, sw_np)), replay


def test_grouped_config5_full_size(ops):
    """BF16 [2048, 16384] quantized per 4096-channel group, then the summed
    grouped W8A8 against INT8 weights [4][4096][4096]; the whole output is bit-exact."""
    m, g, n = 2048, 4, 4096
    rng = np.random.default_rng(5)
    x_bits = O.f32_to_bf16(rng.standard_normal((m, g * 4096)).astype(np.float32))
    w_np = rng.integers(-127, 128, (g, n, 4096)).astype(np.int8)
    sw_np = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    codes = torch.empty(g, m, 4096, device="cuda", dtype=torch.int8)
    scales = torch.empty(g, m, device="cuda")
    ops.quantize_grouped4096(to_dev(x_bits).view(m, g, 4096), codes, scales)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.grouped_summed_mm(codes, to_dev(w_np), scales, to_dev(sw_np), out)
    torch.cuda.synchronize()
    c_np, s_np = O.quantize_grouped4096(x_bits.reshape(m, g, 4096))
    assert np.array_equal(codes.cpu().numpy(), c_np) and np.array_equal(scales.cpu().numpy(), s_np)
    assert np.array_equal(bf16_bits(out), O.grouped_summed_mm(c_np, s_np, w_np, sw_np))


@pytest.mark.parametrize("g,m,n,k", [
    (3, 1100, 500, 1056),   # ragged M tile, K tail (8.25 stages of 128)
    (2, 1024, 132, 128),    # one stage per group: copies cross group boundaries at once
    (1, 1500, 260, 640),    # one group
    (5, 2048, 256, 256),    # two stages per group
    (48, 1024, 128, 96),    # the most groups whose row scales fit in LDS, K < one stage
    (49, 1024, 128, 96),    # one more: the 128 x 128 kernel
])
def test_grouped_large_m_two_waves_per_simd(ops, g, m, n, k):
    """M >= 1024 (n % 4 == 0) runs the two-waves-per-SIMD kernel over the groups' K stages
    as one stream; mixed-sign channel scales, guard sentinels and a graph replay."""
    rng = np.random.default_rng(g * 1009 + m + n + k)
    a_np, w_np, sa_np, sw_np = grouped_inputs(rng, g, m, n, k, signed_scales=True)
    a, w, sa, sw = to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np)
    out, buf = with_guard((m, n), torch.bfloat16, float("nan"))
    ops.grouped_summed_mm(a, w, sa, sw, out)
    torch.cuda.synchronize()
    want = O.grouped_summed_mm(a_np, sa_np, w_np, sw_np)
    assert np.array_equal(bf16_bits(out), want)
    assert guard_intact(buf, float("nan"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.grouped_summed_mm(a, w, sa, sw, out)
    for replay in range(2):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(out), want), replay


@pytest.mark.parametrize("g,m,n,k,sa_offset", [
    (3, 1027, 132, 256, 0),  # m % 4 != 0: groups' row scales not on 16-byte boundaries
    (2, 1024, 132, 256, 1),  # a_scale viewed 4 bytes past a 16-byte boundary
    (3, 1028, 132, 384, 0),  # m % 4 == 0 and aligned: the two-waves-per-SIMD kernel
])
def test_grouped_large_m_row_scale_alignment(ops, g, m, n, k, sa_offset):
    """The M >= 1024 kernel copies row scales four rows (16 bytes) at a time; shapes and
    a_scale views it cannot copy that way (a copy would straddle a group boundary, be
    misaligned or run past the end of a_scale) take the row-by-row kernel. Either way the
    output is the oracle's, bit for bit, including the last group's last rows."""
    rng = np.random.default_rng(g * 7919 + m + n + k + sa_offset)
    a_np, w_np, sa_np, sw_np = grouped_inputs(rng, g, m, n, k, signed_scales=True)
    sa_store = torch.full((g * m + sa_offset,), float("nan"), device="cuda")
    sa = sa_store[sa_offset:].view(g, m)
    sa.copy_(to_dev(sa_np))
    assert sa.is_contiguous() and sa.data_ptr() % 16 == 4 * sa_offset % 16
    out, buf = with_guard((m, n), torch.bfloat16, float("nan"))
    ops.grouped_summed_mm(to_dev(a_np), to_dev(w_np), sa, to_dev(sw_np), out)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), O.grouped_summed_mm(a_np, sa_np, w_np, sw_np))
    assert guard_intact(buf, float("nan"))


def test_grouped_rejections(ops):
    dev = "cuda"
    a = torch.zeros(2, 8, 64, dtype=torch.int8, device=dev)
    w = torch.zeros(2, 8, 64, dtype=torch.int8, device=dev)
    sa = torch.zeros(2, 8, device=dev)
    sw = torch.zeros(8, dtype=torch.bfloat16, device=dev)
    out = torch.empty(8, 8, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="Expected INT8 a"):
        ops.grouped_summed_mm(a, w[:1], sa, sw, out)
    with pytest.raises(RuntimeError, match="Expected INT8 a"):
        ops.grouped_summed_mm(a, w, sa, sw, out[:4])
    with pytest.raises(RuntimeError, match="Invalid grouped GEMM geometry"):
        ops.grouped_summed_mm(a[:, :, :48].contiguous(), w[:, :, :48].contiguous(), sa, sw, out)
    with pytest.raises(RuntimeError, match="Unexpected dtype"):
        ops.grouped_summed_mm(a, w.to(torch.uint8), sa, sw, out)


def test_c_abi_grouped_matches_oracle(ops, lib):
    from consumer_int8 import _abi

    rng = np.random.default_rng(77)
    g, m, n, k = 3, 200, 260, 512
    a_np, w_np, sa_np, sw_np = grouped_inputs(rng, g, m, n, k)
    a, w, sa, sw = to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    _abi.check(lib.ci8_grouped_summed_mm(a.data_ptr(), w.data_ptr(), sa.data_ptr(),
                                         sw.data_ptr(), out.data_ptr(), g, m, n, k, stream))
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), O.grouped_summed_mm(a_np, sa_np, w_np, sw_np))
