"""GPU parity of channel_gemv (W8A16) against the FP64 oracle.

Tolerance, as the reference (tests/test_gemv.py:10-33): atol 0.004, rtol 0.008 and
relative L2 < 0.003 against the FP64 dot of the BF16-dequantized weights; in addition
every output must lie within 1 BF16 ulp of the exact value plus the worst-case FP32
summation error K * 2^-24 * sum|x * wq| (the bound of an FP32-accumulated reference).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, host, randn_bf16, to_dev

pytestmark = pytest.mark.gpu


def check_gemv(out_bits, x_bits, w, s_bits):
    ref_bits, exact = O.channel_gemv(x_bits, w, s_bits)
    actual = O.bf16_to_f32(out_bits).astype(np.float64)
    reference = O.bf16_to_f32(ref_bits).astype(np.float64)
    np.testing.assert_allclose(actual, reference, atol=0.004, rtol=0.008)
    norm = np.linalg.norm(reference)
    if norm > 0:
        assert np.linalg.norm(actual - reference) / norm < 0.003
    bound = O.bf16_ulp(exact) + O.gemv_abs_bound(x_bits, w, s_bits)
    assert np.all(np.abs(actual - exact) <= bound)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 8, 16])
@pytest.mark.parametrize("n,k", [(37, 528), (512, 5120)])
def test_w8a16_small_batch_matches_bf16_dequantized_linear(ops, m, n, k):
    rng = np.random.default_rng(134)
    x_bits = randn_bf16(rng, (m, k))
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s_bits = O.f32_to_bf16((rng.random(n) * 0.002).astype(np.float32))
    x = to_dev(x_bits)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.channel_gemv(x, to_dev(w), to_dev(s_bits), out)
    graph = torch.cuda.CUDAGraph()
    wt, st = to_dev(w), to_dev(s_bits)
    with torch.cuda.graph(graph):
        ops.channel_gemv(x, wt, st, out)
    x.mul_(0.75)
    graph.replay()
    torch.cuda.synchronize()
    check_gemv(bf16_bits(out), bf16_bits(x), w, s_bits)


@pytest.mark.parametrize("m", [1, 4, 6, 8, 16])
def test_decode_shape_full_size(ops, m):
    """Config 2: K = 5120, N = 17408, scales uniform in [1e-3, 1e-2]."""
    k, n = 5120, 17408
    rng = np.random.default_rng(2 + m)
    x_bits = randn_bf16(rng, (m, k))
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s_bits = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.channel_gemv(to_dev(x_bits), to_dev(w), to_dev(s_bits), out)
    torch.cuda.synchronize()
    check_gemv(bf16_bits(out), x_bits, w, s_bits)


@pytest.mark.parametrize("m,n,k", [(12, 1000, 5104), (10, 4100, 5120), (14, 250, 5120),
                                   (9, 17, 8192), (10, 16 * 256 * 3 + 16, 5120),
                                   (7, 300, 5120), (16, 36869, 2048), (5, 2000, 4096),
                                   (2, 16 * 256 * 9 + 5, 1024), (1, 17408, 5120)])
def test_balanced_spans(ops, m, n, k):
    """K <= 8192 (m >= 2) runs one workgroup per CU over equal channel spans (N = 17408:
    68 per CU): fewer channels than CUs x 16, spans that end inside a block of 16, more
    than 8 blocks per span (two partial-sum batches), every x-register configuration (K
    ranges of 2, 4, 5 and 8 blocks of 64) and a K tail; m = 1 takes the row kernel."""
    rng = np.random.default_rng(m * 7 + n + k)
    x_bits = randn_bf16(rng, (m, k))
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    s_bits = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    ops.channel_gemv(to_dev(x_bits), to_dev(w), to_dev(s_bits), out)
    torch.cuda.synchronize()
    check_gemv(bf16_bits(out), x_bits, w, s_bits)


@pytest.mark.parametrize("m,n,k", [(2, 4096, 4096), (3, 1001, 4112), (4, 33000, 4096),
                                   (5, 20002, 6144), (7, 3001, 7168), (8, 4099, 8192),
                                   (6, 517, 8176), (2, 17408, 5120)])
def test_quad_block_kernel(ops, m, n, k):
    """2 <= m <= 4 with 4096 <= K <= 8192, and 5 <= m <= 8 with 5120 < K <= 8192, run the
    interleaved 4-channel-block kernel: every K range length (4 to 8 units of 64), one
    and two batch groups, a ragged last K range (4112, 8176), N not a multiple of 4,
    fewer blocks than CUs, and more blocks per CU than one partial-sum batch holds (N =
    33000 at one batch group, N = 20002 at two), so the waves also meet mid-way."""
    rng = np.random.default_rng(m * 11 + n + k)
    x_bits = randn_bf16(rng, (m, k))
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    s_bits = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    ops.channel_gemv(to_dev(x_bits), to_dev(w), to_dev(s_bits), out)
    torch.cuda.synchronize()
    check_gemv(bf16_bits(out), x_bits, w, s_bits)


@pytest.mark.parametrize("m,n,k", [(1, 5000, 16384), (5, 600, 12288), (8, 300, 12288),
                                   (16, 70, 9216)])
def test_long_k_kernels(ops, m, n, k):
    """K > 8192: x resident in LDS (m * K * 2 <= 64 KiB), the persistent walk over channel
    blocks (up to 144 KiB) and the LDS ring beyond."""
    rng = np.random.default_rng(m * 5 + n + k)
    x_bits = randn_bf16(rng, (m, k))
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    s_bits = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    ops.channel_gemv(to_dev(x_bits), to_dev(w), to_dev(s_bits), out)
    torch.cuda.synchronize()
    check_gemv(bf16_bits(out), x_bits, w, s_bits)


@pytest.mark.parametrize("m,n,k", [(3, 100, 16), (5, 64, 48), (16, 7, 1040), (2, 33, 65536),
                                   # m = 1 row kernel: one 16-value piece, the longest K it
                                   # takes, more rows than waves with a ragged last piece
                                   (1, 7, 16), (1, 33, 8192), (1, 20003, 1040)])
def test_gemv_tails_and_unaligned_activations(ops, m, n, k):
    rng = np.random.default_rng(m * n + k)
    x_bits = randn_bf16(rng, (m, k))
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    s_bits = O.f32_to_bf16((rng.random(n) * 0.01).astype(np.float32))
    # x starts 4 bytes past a 16-byte boundary (the reference only asks for 4).
    storage = to_dev(np.concatenate([np.zeros(2, np.uint16), x_bits.ravel()]))
    x = storage[2:].view(m, k)
    out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    ops.channel_gemv(x, to_dev(w), to_dev(s_bits), out)
    torch.cuda.synchronize()
    check_gemv(bf16_bits(out), x_bits, w, s_bits)


def test_gemv_rejects_unsupported_geometry(ops):
    x = torch.zeros(17, 64, device="cuda", dtype=torch.bfloat16)
    w = torch.zeros(8, 64, device="cuda", dtype=torch.int8)
    s = torch.ones(8, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="Unsupported W8A16 GEMV geometry"):
        ops.channel_gemv(x, w, s, torch.empty(17, 8, device="cuda", dtype=torch.bfloat16))
    x = torch.zeros(1, 40, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="geometry"):
        ops.channel_gemv(x, torch.zeros(8, 40, device="cuda", dtype=torch.int8), s,
                         torch.empty(1, 8, device="cuda", dtype=torch.bfloat16))
