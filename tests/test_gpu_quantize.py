"""GPU parity of quantize_rows / quantize_grouped4096 against the oracle (bit-exact).

Mirrors tests/test_cuda_ops.py:10-52 and :493-509 of the reference, with inputs drawn
from a seeded CPU generator so the same bits reach the kernel and the oracle.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, guard_intact, host, randn_bf16, to_dev, with_guard

pytestmark = pytest.mark.gpu


def run_quantize(ops, x):
    codes = torch.empty(x.shape, device="cuda", dtype=torch.int8)
    scales = torch.empty(x.shape[0], device="cuda", dtype=torch.float32)
    ops.quantize_rows(x, codes, scales)
    torch.cuda.synchronize()
    return host(codes), host(scales)


@pytest.mark.parametrize("width", [4, 3072, 5120, 6144, 8704, 17408])
@pytest.mark.parametrize("rows,misaligned", [(2, False), (1024, False), (1024, True)])
def test_quantize_rows_preserves_zero_rows_and_round_to_even(ops, width, rows, misaligned):
    rng = np.random.default_rng(742)
    base = O.bf16_to_f32(randn_bf16(rng, rows * width + 1)).copy()
    x = np.clip(base * 100, -127, 127).astype(np.float32)
    x = O.bf16_to_f32(O.f32_to_bf16(x)).copy()
    view = x[int(misaligned) : rows * width + int(misaligned)].reshape(rows, width)
    view[:, 0] = -127
    view[0, :4] = [0, -127, 63.5, 127]
    view[1] = 0
    storage = to_dev(O.f32_to_bf16(x))
    xt = storage[int(misaligned) : rows * width + int(misaligned)].view(rows, width)
    codes, scales = run_quantize(ops, xt)
    expected_scale = np.ones(rows, np.float32)
    expected_scale[1] = np.float32(1e-20)
    assert np.array_equal(scales, expected_scale)
    assert np.array_equal(codes, np.rint(view).astype(np.int8))
    ocodes, oscales = O.quantize_rows(O.f32_to_bf16(view))
    assert np.array_equal(codes, ocodes) and np.array_equal(scales, oscales)


SHAPES = [(1, 1), (3, 7), (5, 100), (2, 512), (4, 4096), (17, 5120), (1024, 5120),
          (4096, 5120), (7, 17408), (9, 4100), (33, 20000), (3, 20480), (2, 65536),
          (2, 70000), (5, 129),
          # eight waves per row (at most 256 rows of 2,561..4,096 values), and either side
          (128, 4096), (256, 2568), (100, 2576), (257, 3072), (1, 2560)]


@pytest.mark.parametrize("rows,width", SHAPES)
@pytest.mark.parametrize("misaligned", [False, True])
def test_quantize_rows_matches_oracle(ops, rows, width, misaligned):
    rng = np.random.default_rng(1000 + rows * 7 + width)
    bits = randn_bf16(rng, (rows, width))
    if width >= 1000:  # 0.1% outlier channels scaled x50 (the prefill config)
        cols = rng.choice(width, max(1, width // 1000), replace=False)
        vals = O.bf16_to_f32(bits).copy()
        vals[:, cols] *= 50
        bits = O.f32_to_bf16(vals)
    if rows > 1:
        bits[rows // 2] = 0
    flat = np.zeros(rows * width + 1, np.uint16)
    flat[int(misaligned):int(misaligned) + rows * width] = bits.ravel()
    storage = to_dev(flat)
    x = storage[int(misaligned):int(misaligned) + rows * width].view(rows, width)
    codes, scales = run_quantize(ops, x)
    ocodes, oscales = O.quantize_rows(bits)
    assert np.array_equal(scales, oscales)
    assert np.array_equal(codes, ocodes)


def test_quantize_rows_non_finite_rows_match_oracle(ops):
    vals = np.array([[1.0, -2.0, np.nan, 0.5] * 128, [np.inf, 1.0, -3.0, 2.0] * 128,
                     [-np.inf, np.nan, 0.0, 1.0] * 128], np.float32)
    bits = O.f32_to_bf16(vals)
    codes, scales = run_quantize(ops, to_dev(bits))
    ocodes, oscales = O.quantize_rows(bits)
    assert np.array_equal(codes, ocodes)
    np.testing.assert_array_equal(scales, oscales)


def test_quantize_rows_graph_replay_no_allocation_and_guards(ops):
    rng = np.random.default_rng(5)
    bits = randn_bf16(rng, (1024, 5120))
    x = to_dev(bits)
    codes, cbuf = with_guard((1024, 5120), torch.int8, -100)
    scales, sbuf = with_guard((1024,), torch.float32, float("nan"))
    ops.quantize_rows(x, codes, scales)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.quantize_rows(x, codes, scales)
    x.neg_()
    codes.fill_(-128)
    scales.fill_(float("nan"))
    allocations = torch.cuda.memory_stats()["allocation.all.allocated"]
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        ocodes, oscales = O.quantize_rows(bf16_bits(x))
        assert np.array_equal(host(codes), ocodes) and np.array_equal(host(scales), oscales)
    assert torch.cuda.memory_stats()["allocation.all.allocated"] == allocations
    assert guard_intact(cbuf, -100) and guard_intact(sbuf, float("nan"))


@pytest.mark.parametrize("rows,groups", [(0, 4), (1, 1), (3, 2), (128, 4), (2048, 4)])
def test_grouped4096_preserves_native_codes_and_graph_replay(ops, rows, groups):
    rng = np.random.default_rng(137)
    bits = randn_bf16(rng, (rows, groups, 4096))
    if rows:
        bits[0] = 0
    x = to_dev(bits)
    q = torch.empty(groups, rows, 4096, device="cuda", dtype=torch.int8)
    scales = torch.empty(groups, rows, device="cuda", dtype=torch.float32)
    ops.quantize_grouped4096(x, q, scales)
    torch.cuda.synchronize()
    if not rows:
        return
    ocodes, oscales = O.quantize_grouped4096(bits)
    assert np.array_equal(host(q), ocodes) and np.array_equal(host(scales), oscales)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.quantize_grouped4096(x, q, scales)
    x.neg_()
    q.fill_(-128)
    scales.fill_(float("nan"))
    allocations = torch.cuda.memory_stats()["allocation.all.allocated"]
    graph.replay()
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats()["allocation.all.allocated"] == allocations
    for group in range(groups):
        expected_q = torch.empty_like(q[group])
        expected_s = torch.empty_like(scales[group])
        ops.quantize_rows(x[:, group].contiguous(), expected_q, expected_s)
        assert torch.equal(q[group], expected_q)
        assert torch.equal(scales[group], expected_s)
    ocodes, oscales = O.quantize_grouped4096(bf16_bits(x))
    assert np.array_equal(host(q), ocodes) and np.array_equal(host(scales), oscales)


def test_grouped4096_rejects_wrong_shape_alignment_and_aliases(ops):
    x = torch.randn(3, 4, 4096, device="cuda", dtype=torch.bfloat16)
    q = torch.empty(4, 3, 4096, device="cuda", dtype=torch.int8)
    scales = torch.empty(4, 3, device="cuda")
    with pytest.raises(RuntimeError, match="Expected BF16"):
        ops.quantize_grouped4096(x, q.transpose(0, 1).contiguous(), scales)
    storage = torch.empty(x.numel() + 1, device="cuda", dtype=x.dtype)
    with pytest.raises(RuntimeError, match="aligned"):
        ops.quantize_grouped4096(storage[1:].view_as(x), q, scales)
    aliased = x.view(torch.int8).flatten()[: q.numel()].view_as(q)
    with pytest.raises(RuntimeError, match="overlap"):
        ops.quantize_grouped4096(x, aliased, scales)


def test_quantize_rows_rejects_bad_shapes(ops):
    x = torch.zeros(4, 8, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="Wrong output shapes"):
        ops.quantize_rows(x, torch.empty(4, 7, device="cuda", dtype=torch.int8),
                          torch.empty(4, device="cuda"))
    with pytest.raises(RuntimeError, match="Unexpected dtype"):
        ops.quantize_rows(x.float(), torch.empty(4, 8, device="cuda", dtype=torch.int8),
                          torch.empty(4, device="cuda"))


def test_c_abi_quantize_rows_matches_op(ops, lib):
    """The C ABI called directly (ctypes, the FFI a non-torch caller would use)."""
    from consumer_int8 import _abi

    rng = np.random.default_rng(99)
    bits = randn_bf16(rng, (300, 5120))
    x = to_dev(bits)
    codes = torch.empty(300, 5120, device="cuda", dtype=torch.int8)
    scales = torch.empty(300, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _abi.check(lib.ci8_quantize_rows(x.data_ptr(), codes.data_ptr(), scales.data_ptr(),
                                     300, 5120, stream))
    torch.cuda.synchronize()
    ocodes, oscales = O.quantize_rows(bits)
    assert np.array_equal(host(codes), ocodes) and np.array_equal(host(scales), oscales)
