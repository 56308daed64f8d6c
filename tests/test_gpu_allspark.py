"""GPU parity of unpack_allspark (AllSpark N32K16 -> row-major INT8 + channel scales).

Mirrors tests/test_cuda_ops.py:440-471 of the reference, with the packed input made by
the oracle's forward packer (the inverse of the reference's index map) instead of
vLLM's repacker: restored codes and scales must be exact, under graph capture and
replay with the packed data changed in place between replays.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, guard_intact, host, to_dev, with_guard

pytestmark = pytest.mark.gpu


def packed_case(n, k, seed, fill=0x80):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, (n, k)).astype(np.uint8)
    scales = O.f32_to_bf16(rng.standard_normal(n).astype(np.float32))
    packed, packed_scales = O.pack_allspark(codes, scales, fill=fill)
    return codes, scales, packed, packed_scales


def expected(codes):
    return (codes.astype(np.int16) - 128).astype(np.int8)


@pytest.mark.parametrize("n,k", [(16, 16), (48, 80), (128, 512), (5120, 3072), (5120, 17408),
                                 (17408, 5120), (16, 65536), (80, 4096)])
def test_unpack_allspark_restores_every_code_and_scale(ops, n, k):
    codes, scales, packed, packed_scales = packed_case(n, k, 319 + n + k, fill=0x11)
    weight = torch.empty(n, k, device="cuda", dtype=torch.int8)
    out_scales = torch.empty(n, device="cuda", dtype=torch.bfloat16)
    ops.unpack_allspark(to_dev(packed), to_dev(packed_scales), weight, out_scales)
    torch.cuda.synchronize()
    assert np.array_equal(host(weight), expected(codes))
    assert np.array_equal(bf16_bits(out_scales), scales)


@pytest.mark.parametrize("n,k", [(16, 16), (48, 80), (128, 512), (5120, 3072)])
def test_allspark_unpack_preserves_every_code_and_scale_in_graph(ops, n, k):
    """tests/test_cuda_ops.py:440-471: capture once, replay twice; between replays the
    codes are inverted (xor 255) and the scales negated, repacked and copied in place."""
    codes, scales, packed, packed_scales = packed_case(n, k, 319)
    d_packed, d_pscales = to_dev(packed), to_dev(packed_scales)
    restored = torch.empty(n, k, device="cuda", dtype=torch.int8)
    restored_scales = torch.empty(n, device="cuda", dtype=torch.bfloat16)
    ops.unpack_allspark(d_packed, d_pscales, restored, restored_scales)  # warm up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.unpack_allspark(d_packed, d_pscales, restored, restored_scales)
    for _ in range(2):
        restored.zero_()
        restored_scales.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(restored), expected(codes))
        assert np.array_equal(bf16_bits(restored_scales), scales)
        codes ^= 255
        scales = scales ^ np.uint16(0x8000)
        changed, changed_scales = O.pack_allspark(codes, scales)
        d_packed.copy_(to_dev(changed))
        d_pscales.copy_(to_dev(changed_scales))


def test_unpack_allspark_word_aligned_packed_view(ops):
    """The reference accepts a packed buffer aligned to 4 bytes only
    (csrc/bindings.cpp:282-283): a view 4 bytes into its storage gives the same result."""
    n, k = 48, 80
    codes, scales, packed, packed_scales = packed_case(n, k, 5)
    storage = torch.zeros(packed.size + 4, device="cuda", dtype=torch.uint8)
    storage[4:].copy_(to_dev(packed).view(-1))
    view = storage[4:].view(packed.shape)
    assert view.data_ptr() % 16 == 4
    weight = torch.empty(n, k, device="cuda", dtype=torch.int8)
    out_scales = torch.empty(n, device="cuda", dtype=torch.bfloat16)
    ops.unpack_allspark(view, to_dev(packed_scales), weight, out_scales)
    torch.cuda.synchronize()
    assert np.array_equal(host(weight), expected(codes))
    assert np.array_equal(bf16_bits(out_scales), scales)


def test_unpack_allspark_writes_only_its_outputs(ops):
    n, k = 48, 96  # n % 32 == 16: the last group's rows 48..63 are padding
    codes, scales, packed, packed_scales = packed_case(n, k, 9)
    weight, wbuf = with_guard((n, k), torch.int8, 55)
    out_scales, sbuf = with_guard((n,), torch.bfloat16, -7.0)
    ops.unpack_allspark(to_dev(packed), to_dev(packed_scales), weight, out_scales)
    torch.cuda.synchronize()
    assert guard_intact(wbuf, 55) and guard_intact(sbuf, -7.0)
    assert np.array_equal(host(weight), expected(codes))


def test_unpack_then_fused_mm_equals_channel_mm_on_the_biased_codes(ops):
    """benchmarks/microbench.py:50-53's serving pattern: restore a layer, then
    quantize_rows + fused_channel_mm; equal to channel_mm on the biased UINT8 weights."""
    n, k, m = 256, 512, 64
    codes, scales, packed, packed_scales = packed_case(n, k, 21)
    weight = torch.empty(n, k, device="cuda", dtype=torch.int8)
    w_scales = torch.empty(n, device="cuda", dtype=torch.bfloat16)
    ops.unpack_allspark(to_dev(packed), to_dev(packed_scales), weight, w_scales)
    x = torch.randn(m, k, device="cuda").to(torch.bfloat16)
    a = torch.empty(m, k, device="cuda", dtype=torch.int8)
    sa = torch.empty(m, device="cuda")
    ops.quantize_rows(x, a, sa)
    fused = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.fused_channel_mm(a, weight, sa, w_scales, fused, 0)
    biased = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.channel_mm(a, to_dev(codes), sa, to_dev(scales), biased)
    torch.cuda.synchronize()
    assert torch.equal(fused, biased)


def test_unpack_allspark_rejections(ops):
    u8 = dict(device="cuda", dtype=torch.uint8)
    bf = dict(device="cuda", dtype=torch.bfloat16)
    i8 = dict(device="cuda", dtype=torch.int8)
    with pytest.raises(RuntimeError, match="Expected AllSpark N32K16"):
        ops.unpack_allspark(torch.zeros(32, 16, **u8), torch.zeros(32, **bf),
                            torch.empty(24, 16, **i8), torch.empty(24, **bf))
    with pytest.raises(RuntimeError, match="Expected AllSpark N32K16"):
        ops.unpack_allspark(torch.zeros(16, 16, **u8), torch.zeros(16, **bf),
                            torch.empty(16, 16, **i8), torch.empty(16, **bf))
    with pytest.raises(RuntimeError, match="Wrong tensor ranks"):
        ops.unpack_allspark(torch.zeros(32, 16, **u8), torch.zeros(1, 32, **bf),
                            torch.empty(16, 16, **i8), torch.empty(16, **bf))
    with pytest.raises(RuntimeError, match="Unexpected dtype or noncontiguous tensor"):
        ops.unpack_allspark(torch.zeros(32, 16, **i8), torch.zeros(32, **bf),
                            torch.empty(16, 16, **i8), torch.empty(16, **bf))
    storage = torch.zeros(32 * 16 + 2, **u8)
    with pytest.raises(RuntimeError, match="Unaligned weights"):
        ops.unpack_allspark(storage[2:].view(32, 16), torch.zeros(32, **bf),
                            torch.empty(16, 16, **i8), torch.empty(16, **bf))


def test_unpack_allspark_through_the_c_abi(lib):
    n, k = 80, 4096
    codes, scales, packed, packed_scales = packed_case(n, k, 33)
    d_packed, d_pscales = to_dev(packed), to_dev(packed_scales)
    weight = torch.empty(n, k, device="cuda", dtype=torch.int8)
    out_scales = torch.empty(n, device="cuda", dtype=torch.bfloat16)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.ci8_unpack_allspark(d_packed.data_ptr(), d_pscales.data_ptr(), weight.data_ptr(),
                                   out_scales.data_ptr(), n, k, stream) == 0
    torch.cuda.synchronize()
    assert np.array_equal(host(weight), expected(codes))
    assert np.array_equal(bf16_bits(out_scales), scales)
