"""GPU parity of gguf_q8_packed_mm (grouped W8A16 on GGUF Q8_0 codes and FP16 scales).

The reference's own test (tests/test_gguf_q8.py:20-59) is mirrored case for case: raw
[G,N,K/32,34] blocks built from FP16 scales and INT8 codes, x [M,G,K] row-major or
group-major (a transposed view, so row and group strides differ), one eager call, a
captured graph replayed three times on rescaled activations with no allocation, and a
relative-norm 0.001 check against a float32 product of the BF16 dense weights.

On top of that every output element is held to the oracle (oracle.gguf_q8_packed_mm,
a float64 product of the same BF16 weights): |out - exact| <= one BF16 ulp of the exact
value + K * 2^-24 * sum_k |x * wq| (any FP32 summation order). Further cases reach
ragged N (scalar stores), padded row strides, a single K stage, large K, M on both
sides of the 16-row switch (m <= 16 runs the balanced-span kernel of the W8A16 GEMV,
in chunks of 8192 along K beyond that while a workgroup spans at most 8 channel
blocks), the 256- and 128-row tiles of larger batches (1, 2, 3, 7 and 8 K
stages), the 64-row tile kernel that takes x beyond a 2 GiB buffer range, extreme codes
and scales, and guard sentinels around the output.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, guard_intact, to_dev, with_guard

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gguf(ops):
    from consumer_int8 import gguf as module

    return module


def check(out_bits, x_bits, codes, scale_bits, rel_norm=None):
    ref_bits, exact = O.gguf_q8_packed_mm(x_bits, codes, scale_bits)
    got = O.bf16_to_f32(out_bits).astype(np.float64)
    assert np.all(np.isfinite(got))
    bound = O.bf16_ulp(exact) + O.gguf_q8_abs_bound(x_bits, codes, scale_bits)
    bad = np.abs(got - exact) > bound
    assert not bad.any(), (np.argwhere(bad)[:5], got[bad][:5], exact[bad][:5])
    if rel_norm is not None:
        reference = O.bf16_to_f32(ref_bits).astype(np.float64)
        assert np.linalg.norm(got - reference) / np.linalg.norm(reference) < rel_norm


def raw_blocks(gen, groups, n, k):
    """tests/test_gguf_q8.py:25-28: FP16 scales (rand * 0.1) and codes in [-128, 127]."""
    scales = (torch.rand(groups, n, k // 32, 1, generator=gen) * 0.1).half()
    codes = torch.randint(-128, 128, (groups, n, k // 32, 32), dtype=torch.int8, generator=gen)
    raw = torch.cat((scales.view(torch.uint8), codes.view(torch.uint8)), dim=-1)
    return raw, codes.reshape(groups, n, k), scales.reshape(groups, n, k // 32)


@pytest.mark.parametrize("m", [1, 17, 32, 127, 128, 513])
@pytest.mark.parametrize("group_major", [False, True])
def test_reference_cases_with_graph_replay(gguf, m, group_major):
    gen = torch.Generator().manual_seed(37 + m)
    groups, n, k = 3, 37, 128
    raw, codes_cpu, scales_cpu = raw_blocks(gen, groups, n, k)
    codes, scales = gguf.pack_q8(raw.cuda())
    assert torch.equal(codes.cpu(), codes_cpu) and torch.equal(scales.cpu(), scales_cpu)
    shape = (groups, m, k) if group_major else (m, groups, k)
    x = torch.randn(shape, generator=gen).bfloat16().cuda()
    if group_major:
        x = x.transpose(0, 1)
    out = torch.empty(m, groups, n, device="cuda", dtype=torch.bfloat16)
    codes_np = codes_cpu.numpy()
    scales_np = scales_cpu.view(torch.int16).numpy().view(np.uint16)

    gguf.q8_packed_mm(x, codes, scales, out)
    torch.cuda.synchronize()
    x_np = bf16_bits(x.contiguous())
    check(bf16_bits(out), x_np, codes_np, scales_np, rel_norm=0.001)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gguf.q8_packed_mm(x, codes, scales, out)
    for _ in range(3):
        x.mul_(0.75)
        out.fill_(float("nan"))
        allocated = torch.cuda.memory_allocated()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == allocated
        check(bf16_bits(out), bf16_bits(x.contiguous()), codes_np, scales_np, rel_norm=0.001)
        assert out.float().abs().max() > 0


CASES = [
    # m, groups, n, k, row padding (elements beyond G*K per row)
    (16, 1, 4096, 4096, 0),     # largest M of the 16-row tile
    (17, 1, 1000, 5120, 0),     # smallest M past the span kernel, ragged N
    (200, 2, 130, 1536, 64),    # ragged M and N (N % 4 == 2: scalar stores), padded rows
    (64, 4, 96, 64, 8),         # one K stage
    (5, 2, 37, 16384, 0),       # long K at m <= 16: the span kernel in two K chunks
    (8, 1, 4096, 14336, 0),     # span kernel, K chunks of 128 and 96 blocks of 64
    (3, 2, 300, 9216, 64),      # span kernel, a last K chunk of one block per wave
    (2, 1, 33280, 9216, 0),     # K > 8192 with 9 channel blocks per CU: the tile kernel
    (256, 1, 512, 2048, 0),
    (7, 3, 300, 2048, 64),      # m <= 16 span kernel: groups, padded rows, ragged spans
    (16, 2, 4100, 8192, 0),     # span kernel at its longest K, more channels than CUs x 16
    (2, 5, 16, 64, 8),          # one channel block per group, one K block
    # M > 16: 128-channel tiles of 256 or 128 rows (the smaller shapes above run 128 rows)
    (2048, 1, 4096, 512, 0),    # 256-row tiles, even stage count
    (1100, 2, 4002, 192, 8),    # 256-row tiles, ragged M, N % 4 == 2, three stages
    (600, 4, 2000, 448, 24),    # 128-row tiles, ragged M and N, odd stage count
    (2048, 1, 4096, 64, 0),     # a single K stage
    (1024, 2, 4096, 128, 0),    # two K stages
]


@pytest.mark.parametrize("m,groups,n,k,pad", CASES)
def test_shapes_strides_and_guards(gguf, m, groups, n, k, pad):
    rng = np.random.default_rng(m * 31 + n + k)
    row = groups * k + pad
    x_full = O.f32_to_bf16(rng.standard_normal((m, row)).astype(np.float32))
    x_np = x_full[:, : groups * k].reshape(m, groups, k)
    codes_np = rng.integers(-128, 128, (groups, n, k)).astype(np.int8)
    scales_np = (rng.random((groups, n, k // 32)) * 0.02).astype(np.float16).view(np.uint16)
    x = to_dev(x_full)[:, : groups * k].view(m, groups, k) if pad == 0 else \
        torch.as_strided(to_dev(x_full), (m, groups, k), (row, k, 1))
    assert x.stride() == (row, k, 1)
    codes = to_dev(codes_np)
    scales = to_dev(scales_np).view(torch.float16)
    out, buf = with_guard((m, groups, n), torch.bfloat16, float("nan"))
    gguf.q8_packed_mm(x, codes, scales, out)
    torch.cuda.synchronize()
    assert guard_intact(buf, float("nan"))
    check(bf16_bits(out), x_np, codes_np, scales_np, rel_norm=0.001)


def test_extreme_codes_and_scales(gguf):
    """Codes -128 and 127 with the largest FP16 scale, subnormal scales and zero scales."""
    m, groups, n, k = 33, 2, 12, 256
    rng = np.random.default_rng(5)
    codes_np = np.where(rng.random((groups, n, k)) < 0.5, -128, 127).astype(np.int8)
    scales = np.empty((groups, n, k // 32), np.float16)
    scales[0] = 65504.0
    scales[1, :4] = 6e-8          # FP16 subnormals
    scales[1, 4:8] = 0.0
    scales[1, 8:] = -1.5
    scales_np = scales.view(np.uint16)
    x_np = O.f32_to_bf16((rng.standard_normal((m, groups, k)) * 0.01).astype(np.float32))
    out = torch.empty(m, groups, n, device="cuda", dtype=torch.bfloat16)
    gguf.q8_packed_mm(to_dev(x_np), to_dev(codes_np), to_dev(scales_np).view(torch.float16), out)
    torch.cuda.synchronize()
    got = bf16_bits(out)
    check(got, x_np, codes_np, scales_np)
    assert np.all(O.bf16_to_f32(got[:, 1, 4:8]) == 0)


def test_empty_outputs_and_rejections(gguf):
    codes = torch.zeros(2, 8, 64, device="cuda", dtype=torch.int8)
    scales = torch.zeros(2, 8, 2, device="cuda", dtype=torch.float16)
    x = torch.zeros(0, 2, 64, device="cuda", dtype=torch.bfloat16)
    gguf.q8_packed_mm(x, codes, scales, torch.empty(0, 2, 8, device="cuda", dtype=torch.bfloat16))
    x = torch.zeros(4, 2, 64, device="cuda", dtype=torch.bfloat16)
    out = torch.empty(4, 2, 8, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="BF16 input/output, INT8 codes"):
        gguf.q8_packed_mm(x, codes, scales.bfloat16(), out)
    with pytest.raises(RuntimeError, match="K must be a multiple of 64"):
        gguf.q8_packed_mm(x[:, :, :32], codes[:, :, :32], scales[:, :, :1], out)
    with pytest.raises(RuntimeError, match="K must be a multiple of 64"):
        gguf.q8_packed_mm(x, codes.transpose(0, 1).contiguous().transpose(0, 1), scales, out)
    with pytest.raises(RuntimeError, match="copy alignment"):
        wide = torch.zeros(4, 2, 68, device="cuda", dtype=torch.bfloat16)
        gguf.q8_packed_mm(wide[:, :, 4:], codes, scales, out)
    with pytest.raises(RuntimeError, match="must not alias"):
        alias = torch.zeros(4 * 2 * 64, device="cuda", dtype=torch.bfloat16)
        gguf.q8_packed_mm(alias.view(4, 2, 64), codes, scales, alias[:64].view(4, 2, 8))
    with pytest.raises(ValueError, match="K divisible by 64"):
        gguf.pack_q8(torch.zeros(1, 2, 3, 34, device="cuda", dtype=torch.uint8))
    bad = torch.zeros(1, 2, 2, 34, dtype=torch.uint8)
    bad[0, 0, 0, :2] = torch.tensor([0x00, 0x7C], dtype=torch.uint8)  # FP16 +inf
    with pytest.raises(ValueError, match="must be finite"):
        gguf.pack_q8(bad.cuda())


def test_group_major_large_tiles(gguf):
    """x as a group-major view (group stride < row stride is not required: here the
    group stride is M * K and the row stride K) on the 128-row tiles."""
    gen = torch.Generator().manual_seed(91)
    m, groups, n, k = 512, 4, 2048, 256
    raw, codes_cpu, scales_cpu = raw_blocks(gen, groups, n, k)
    codes, scales = gguf.pack_q8(raw.cuda())
    x = torch.randn(groups, m, k, generator=gen).bfloat16().cuda().transpose(0, 1)
    assert x.stride() == (k, m * k, 1)
    out = torch.empty(m, groups, n, device="cuda", dtype=torch.bfloat16)
    gguf.q8_packed_mm(x, codes, scales, out)
    torch.cuda.synchronize()
    check(bf16_bits(out), bf16_bits(x.contiguous()), codes_cpu.numpy(),
          scales_cpu.view(torch.int16).numpy().view(np.uint16), rel_norm=0.001)


def test_x_beyond_buffer_range_takes_the_tile_kernel(gguf):
    """A row stride of 2^27 elements puts x's byte range (19 rows x 256 MiB) past what a
    buffer descriptor addresses, so M = 20 runs the 64-row tile kernel."""
    m, groups, n, k, xs = 20, 1, 200, 256, 1 << 27
    rng = np.random.default_rng(5)
    x_np = O.f32_to_bf16(rng.standard_normal((m, groups, k)).astype(np.float32))
    codes_np = rng.integers(-128, 128, (groups, n, k)).astype(np.int8)
    scales_np = (rng.random((groups, n, k // 32)) * 0.02).astype(np.float16).view(np.uint16)
    big = torch.zeros((m - 1) * xs + groups * k, device="cuda", dtype=torch.bfloat16)
    x = torch.as_strided(big, (m, groups, k), (xs, k, 1))
    x.copy_(to_dev(x_np))
    out = torch.empty(m, groups, n, device="cuda", dtype=torch.bfloat16)
    gguf.q8_packed_mm(x, to_dev(codes_np), to_dev(scales_np).view(torch.float16), out)
    torch.cuda.synchronize()
    check(bf16_bits(out), x_np, codes_np, scales_np, rel_norm=0.001)
    del big
