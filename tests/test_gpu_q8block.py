"""GPU parity of the block-32 Q8_0 W8A8 path (the reference's benchmark-only
benchmarks/cuda/q8_block_int8.cu, called through the C ABI as its harness calls it,
benchmarks/benchmark_q8_block_int8.py:36-80).

Bit-exact against the oracle: the block scales and codes, and the GEMM output for the
codes the kernel produced. The reference harness's own checks are kept beside it: the
quantizer error bound, the blockwise dot-product oracle within rtol 0.008 / atol 1e-5,
the dense product within 1.5% relative, and graph replay with the input negated.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, host, to_dev

pytestmark = pytest.mark.gpu


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def make_case(m, n, k, seed):
    """benchmarks/benchmark_q8_block_int8.py:62-72: x ~ N(0, 0.1^2) with a zero block and
    a x100 block, Q8_0 codes in [-128, 127], FP16 block scales ~ N(0, 0.01^2)."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * 0.1).astype(np.float32)
    x[:, :32] = 0
    if k >= 64:
        x[:, 32:64] *= 100
    x_bits = O.f32_to_bf16(x)
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    sw = (rng.standard_normal((n, k // 32)) * 0.01).astype(np.float16).view(np.uint16)
    return x_bits, w, sw


def run_fused(lib, x, w, sw, m, n, k):
    a = torch.empty(m, k, device="cuda", dtype=torch.int8)
    sa = torch.empty(m, k // 32, device="cuda", dtype=torch.float32)
    y = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    status = lib.ci8_q8_block_int8(x.data_ptr(), a.data_ptr(), sa.data_ptr(), w.data_ptr(),
                                   sw.data_ptr(), y.data_ptr(), m, n, k, stream())
    assert status == 0, status
    return a, sa, y


def check_against_oracle(x_bits, w, sw, a, sa, y):
    oa, osa = O.quantize_block32(x_bits)
    assert np.array_equal(host(sa), osa)
    assert np.array_equal(host(a), oa)
    assert np.array_equal(bf16_bits(y), O.q8_block_mm(oa, osa, w, sw))


@pytest.mark.parametrize("m,n,k", [(1, 1, 32), (17, 33, 96), (129, 65, 256), (63, 130, 160),
                                   (64, 128, 128), (200, 300, 1056), (128, 1024, 4096)])
def test_q8_block_int8_matches_oracle(lib, m, n, k):
    x_bits, w, sw = make_case(m, n, k, 137 + m + n + k)
    a, sa, y = run_fused(lib, to_dev(x_bits), to_dev(w), to_dev(sw), m, n, k)
    torch.cuda.synchronize()
    check_against_oracle(x_bits, w, sw, a, sa, y)


@pytest.mark.parametrize("m", [512, 2048])
def test_q8_block_int8_benchmark_shapes(lib, m):
    """The harness's shapes (m, 1024, 4096): bit-exact on sampled rows (the full oracle
    is a loop over 128 blocks), and the harness's tolerance checks on the whole output."""
    n, k = 1024, 4096
    torch.manual_seed(137)
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16) * 0.1
    x[:, :32] = 0
    x[:, 32:64] *= 100
    w = torch.randint(-128, 128, (n, k), device="cuda", dtype=torch.int8)
    sw = (torch.randn(n, k // 32, device="cuda") * 0.01).half()
    a, sa, y = run_fused(lib, x, w, sw, m, n, k)
    torch.cuda.synchronize()
    rows = np.array([0, 1, m // 3, m - 1])
    x_bits = bf16_bits(x)
    oa, osa = O.quantize_block32(x_bits[rows])
    assert np.array_equal(host(a)[rows], oa) and np.array_equal(host(sa)[rows], osa)
    w_np, sw_bits = host(w), sw.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(bf16_bits(y)[rows], O.q8_block_mm(oa, osa, w_np, sw_bits))
    # benchmarks/benchmark_q8_block_int8.py:94-121 on the whole output
    xb = x.float().reshape(m, k // 32, 32)
    expected_s = (xb.abs().amax(-1) / 127).clamp_min(1e-20)
    torch.testing.assert_close(sa, expected_s, rtol=1e-6, atol=0)
    assert ((a.reshape_as(xb).float() - xb / expected_s[..., None]).abs() <= 0.50002).all()
    oracle = torch.zeros(m, n, device="cuda")
    for block in range(k // 32):
        dot = a[:, 32 * block:32 * block + 32].float() @ w[:, 32 * block:32 * block + 32].float().T
        oracle += dot * (expected_s[:, block, None] * sw[None, :, block].float())
    torch.testing.assert_close(y, oracle.bfloat16(), rtol=0.008, atol=1e-5)
    dense = x.float() @ (w.float().reshape(n, k // 32, 32) * sw[..., None].float()).reshape(n, k).T
    assert ((y.float() - dense).norm() / dense.norm()).item() < 0.015


def test_q8_block_int8_graph_replay(lib):
    """benchmarks/benchmark_q8_block_int8.py:82-92: captured once, replayed with the input
    negated in place each time; every replay equals the oracle."""
    m, n, k = 96, 160, 512
    x_bits, w, sw = make_case(m, n, k, 5)
    x, dw, dsw = to_dev(x_bits), to_dev(w), to_dev(sw)
    a = torch.empty(m, k, device="cuda", dtype=torch.int8)
    sa = torch.empty(m, k // 32, device="cuda", dtype=torch.float32)
    y = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)

    def run():
        assert lib.ci8_q8_block_int8(x.data_ptr(), a.data_ptr(), sa.data_ptr(), dw.data_ptr(),
                                     dsw.data_ptr(), y.data_ptr(), m, n, k, stream()) == 0

    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for _ in range(2):
        x.neg_()
        y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        check_against_oracle(bf16_bits(x), w, sw, a, sa, y)


def test_q8_block_stages_and_unaligned_input(lib):
    """The two stages called separately give the fused result; an input view two bytes
    into its storage takes the scalar quantizer with the same codes."""
    m, n, k = 40, 72, 288
    x_bits, w, sw = make_case(m, n, k, 9)
    storage = to_dev(np.concatenate([np.zeros(1, np.uint16), x_bits.reshape(-1)]))
    x_odd = storage[1:].view(m, k)
    a = torch.empty(m, k, device="cuda", dtype=torch.int8)
    sa = torch.empty(m, k // 32, device="cuda", dtype=torch.float32)
    assert lib.ci8_quantize_block32(x_odd.data_ptr(), a.data_ptr(), sa.data_ptr(), m, k,
                                    stream()) == 0
    y = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    dw, dsw = to_dev(w), to_dev(sw)
    assert lib.ci8_q8_block_mm(a.data_ptr(), sa.data_ptr(), dw.data_ptr(), dsw.data_ptr(),
                               y.data_ptr(), m, n, k, stream()) == 0
    torch.cuda.synchronize()
    check_against_oracle(x_bits, w, sw, a, sa, y)
    a2, sa2, y2 = run_fused(lib, to_dev(x_bits), dw, dsw, m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(a, a2) and torch.equal(sa, sa2) and torch.equal(y, y2)


def test_q8_block_special_values(lib):
    """Infinite and NaN activations: a block holding inf gets scale inf, its finite
    values code 0 and inf/NaN code 0 (as the reference's float-to-int conversion);
    the GEMM then follows IEEE arithmetic like the oracle."""
    m, n, k = 8, 16, 64
    x_bits, w, sw = make_case(m, n, k, 3)
    vals = O.bf16_to_f32(x_bits).copy()
    vals[1, 40] = np.inf
    vals[2, 5] = np.nan
    vals[3, 33] = -np.inf
    x_bits = O.f32_to_bf16(vals)
    a, sa, y = run_fused(lib, to_dev(x_bits), to_dev(w), to_dev(sw), m, n, k)
    torch.cuda.synchronize()
    oa, osa = O.quantize_block32(x_bits)
    assert np.array_equal(host(sa), osa) and np.array_equal(host(a), oa)
    with np.errstate(invalid="ignore", over="ignore"):
        expected = O.q8_block_mm(oa, osa, w, sw)
    got = bf16_bits(y)
    same = (got == expected) | (np.isnan(O.bf16_to_f32(got)) & np.isnan(O.bf16_to_f32(expected)))
    assert same.all()


@pytest.mark.parametrize("m,n,k", [(100, 70, 384), (65, 129, 128), (300, 200, 1024),
                                   (2048, 4096, 256), (2000, 4100, 128)])
def test_q8_block_ring_tiles(lib, m, n, k):
    """K a multiple of 128 takes the LDS-ring kernel: 64 x 64 tiles, and 128 x 128 tiles
    once there are two per CU (the last two shapes on a 256-CU GPU, the second with
    ragged row and column tiles). Bit-exact against the oracle."""
    x_bits, w, sw = make_case(m, n, k, 71 + m + n + k)
    a, sa, y = run_fused(lib, to_dev(x_bits), to_dev(w), to_dev(sw), m, n, k)
    torch.cuda.synchronize()
    check_against_oracle(x_bits, w, sw, a, sa, y)


def test_q8_block_ring_needs_aligned_scales(lib):
    """Block scales two bytes off 4-byte alignment take the step kernel, same bits."""
    m, n, k = 70, 90, 256
    x_bits, w, sw = make_case(m, n, k, 13)
    storage = to_dev(np.concatenate([np.zeros(1, np.uint16), sw.reshape(-1)]))
    sw_odd = storage[1:].view(n, k // 32)
    a = torch.empty(m, k, device="cuda", dtype=torch.int8)
    sa = torch.empty(m, k // 32, device="cuda", dtype=torch.float32)
    y = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    dx, dw = to_dev(x_bits), to_dev(w)
    assert lib.ci8_q8_block_int8(dx.data_ptr(), a.data_ptr(), sa.data_ptr(), dw.data_ptr(),
                                 sw_odd.data_ptr(), y.data_ptr(), m, n, k, stream()) == 0
    torch.cuda.synchronize()
    check_against_oracle(x_bits, w, sw, a, sa, y)
    a2, sa2, y2 = run_fused(lib, dx, dw, to_dev(sw), m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


def test_q8_block_ring_special_values(lib):
    """Infinite and NaN activations and zero or negative-zero weight scales through the
    ring kernel (its scale products come from an MFMA outer product): the same values as
    the oracle, NaN for NaN."""
    m, n, k = 24, 40, 256
    x_bits, w, sw = make_case(m, n, k, 21)
    vals = O.bf16_to_f32(x_bits).copy()
    vals[1, 140] = np.inf
    vals[2, 5] = np.nan
    vals[3, 200] = -np.inf
    x_bits = O.f32_to_bf16(vals)
    sw = sw.copy()
    sw[0, :] = 0x0000
    sw[1, 2] = 0x8000
    sw[2, 3] = 0x0001  # the smallest FP16 subnormal
    a, sa, y = run_fused(lib, to_dev(x_bits), to_dev(w), to_dev(sw), m, n, k)
    torch.cuda.synchronize()
    oa, osa = O.quantize_block32(x_bits)
    assert np.array_equal(host(sa), osa) and np.array_equal(host(a), oa)
    with np.errstate(invalid="ignore", over="ignore"):
        expected = O.q8_block_mm(oa, osa, w, sw)
    got = bf16_bits(y)
    same = (got == expected) | (np.isnan(O.bf16_to_f32(got)) & np.isnan(O.bf16_to_f32(expected)))
    assert same.all()
