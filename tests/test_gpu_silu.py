"""GPU parity of silu_mul / silu_mul_quantize (the SwiGLU producers of configs[3]).

Mirrors tests/test_cuda_ops.py:874-921 of the reference. The reference compares with a
compiled FP32 SwiGLU bit for bit; exp and division are not correctly rounded on either
side, so here the activations are checked against the exact SwiGLU with the tolerance
of oracle.silu_mul_bounds (the BF16 rounding of a value within 2^-20 relative of the
exact one), and the quantized codes and scales bit for bit against quantize_rows
applied to the activations the kernel produced, on the GPU and in the oracle.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, guard_intact, host, to_dev, with_guard

pytestmark = pytest.mark.gpu

WIDTHS = [8704, 17408]


def swiglu_input(rows, width, seed, scale=3.0):
    rng = np.random.default_rng(seed)
    bits = O.f32_to_bf16((rng.standard_normal((rows, 2 * width)) * scale).astype(np.float32))
    if rows:
        bits[0] = 0  # the reference zeroes row 0 (tests/test_cuda_ops.py:884)
    return bits


def run_both(ops, x, width):
    rows = x.shape[0]
    act = torch.empty(rows, width, device="cuda", dtype=torch.bfloat16)
    codes = torch.empty(rows, width, device="cuda", dtype=torch.int8)
    scales = torch.empty(rows, device="cuda", dtype=torch.float32)
    ops.silu_mul(x, act)
    ops.silu_mul_quantize(x, codes, scales)
    return act, codes, scales


def gpu_quantize_rows(ops, act):
    codes = torch.empty(act.shape, device="cuda", dtype=torch.int8)
    scales = torch.empty(act.shape[0], device="cuda", dtype=torch.float32)
    ops.quantize_rows(act, codes, scales)
    return codes, scales


def assert_activations_within_bounds(got_bits, x_bits):
    lo, hi = O.silu_mul_bounds(x_bits)
    ok = O.within_bounds(got_bits, lo, hi)
    bad = np.argwhere(~ok)
    assert ok.all(), f"{len(bad)} activations outside the bound, first at {bad[:4].tolist()}"
    # Outside the narrow ambiguous bands the result is the correctly rounded value.
    off = np.mean(got_bits != O.silu_mul(x_bits))
    assert off < 1e-3, off


@pytest.mark.parametrize("width", WIDTHS)
@pytest.mark.parametrize("rows", [1, 4, 37, 256])
def test_swiglu_matches_oracle(ops, rows, width):
    x_bits = swiglu_input(rows, width, 775 + rows + width)
    act, codes, scales = run_both(ops, to_dev(x_bits), width)
    torch.cuda.synchronize()
    got = bf16_bits(act)
    assert_activations_within_bounds(got, x_bits)
    ocodes, oscales = O.silu_mul_quantize(x_bits, activations=got)
    assert np.array_equal(host(codes), ocodes)
    assert np.array_equal(host(scales), oscales)
    assert host(scales)[0] == np.float32(1e-20) and not host(codes)[0].any()


@pytest.mark.parametrize("width", WIDTHS)
@pytest.mark.parametrize("rows", [0, 1024, 3904, 4096])
def test_swiglu_quantization_equals_quantize_rows_of_silu_mul(ops, rows, width):
    """tests/test_cuda_ops.py:879-900 at the reference's sizes: the fused producer equals
    quantize_rows(silu_mul(x)) bit for bit; M = 0 is a no-op."""
    torch.manual_seed(775 + rows + width)
    x = torch.randn(rows, 2 * width, device="cuda", dtype=torch.bfloat16) * 3
    if rows:
        x[0].zero_()
    act, codes, scales = run_both(ops, x, width)
    if not rows:
        torch.cuda.synchronize()
        return
    ref_codes, ref_scales = gpu_quantize_rows(ops, act)
    torch.cuda.synchronize()
    assert torch.equal(codes, ref_codes)
    assert torch.equal(scales, ref_scales)
    # The activations against the oracle on a sample of rows.
    sample = torch.tensor([0, 1, rows // 2, rows - 1], device="cuda")
    assert_activations_within_bounds(bf16_bits(act[sample]), bf16_bits(x[sample]))


def test_swiglu_down_projection_shape(ops):
    """configs[3]'s producer: M = 16384, K = 17408 (1.1 GB of BF16 input)."""
    rows, width = 16384, 17408
    torch.manual_seed(3)
    x = torch.randn(rows, 2 * width, device="cuda", dtype=torch.bfloat16)
    act, codes, scales = run_both(ops, x, width)
    ref_codes, ref_scales = gpu_quantize_rows(ops, act)
    torch.cuda.synchronize()
    assert torch.equal(codes, ref_codes) and torch.equal(scales, ref_scales)
    sample = torch.tensor([0, 4097, 9999, rows - 1], device="cuda")
    assert_activations_within_bounds(bf16_bits(act[sample]), bf16_bits(x[sample]))


def test_swiglu_matches_torch_fp32(ops):
    """Plain PyTorch FP32 SwiGLU (the reference test's formula, eager) within the same
    bound: both are FP32 evaluations of the exact value."""
    rows, width = 64, 8704
    x_bits = swiglu_input(rows, width, 99)
    x = to_dev(x_bits)
    act, _, _ = run_both(ops, x, width)
    gate, up = x[:, :width].float(), x[:, width:].float()
    expected = (torch.nn.functional.silu(gate) * up).bfloat16()
    lo, hi = O.silu_mul_bounds(x_bits)
    assert O.within_bounds(bf16_bits(expected), lo, hi).all()
    assert O.within_bounds(bf16_bits(act), lo, hi).all()
    assert (act != expected).float().mean().item() < 1e-3


@pytest.mark.parametrize("width", WIDTHS)
def test_swiglu_special_values(ops, width):
    """Zeros, infinities, NaN, the FP32 overflow of e^-g (g <= -89), the small-quotient
    range just above it, and huge products; codes follow quantize_rows on the same
    activations (NaN -> 0, an infinite row maximum gives scale inf)."""
    rng = np.random.default_rng(7)
    gate_vals = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -89.0, -88.5, -87.5, -100.0,
                          100.0, 1e-30, -1e-30, 3e38, -3e38, 20.0, -20.0], np.float32)
    up_vals = np.array([1.0, -1.0, 0.0, np.inf, np.nan, 3e38, 1e-30, -2.0], np.float32)
    rows = 6
    gate = rng.choice(gate_vals, (rows, width)).astype(np.float32)
    up = rng.choice(up_vals, (rows, width)).astype(np.float32)
    gate[0] = rng.standard_normal(width)
    up[0] = rng.standard_normal(width)
    gate[0, :len(gate_vals)] = gate_vals          # one of each on an otherwise finite row
    up[0, :len(gate_vals)] = 1.0
    gate[1] = -88.5                               # a row of values near 1e-36
    up[1] = rng.standard_normal(width)
    x_bits = np.concatenate([O.f32_to_bf16(gate), O.f32_to_bf16(up)], axis=1)
    x = to_dev(x_bits)
    act, codes, scales = run_both(ops, x, width)
    torch.cuda.synchronize()
    got = bf16_bits(act)
    lo, hi = O.silu_mul_bounds(x_bits)
    assert O.within_bounds(got, lo, hi).all()
    ocodes, oscales = O.silu_mul_quantize(x_bits, activations=got)
    assert np.array_equal(host(codes), ocodes)
    assert np.array_equal(host(scales), oscales, equal_nan=True)
    ref_codes, ref_scales = gpu_quantize_rows(ops, act)
    assert torch.equal(codes, ref_codes)
    assert np.array_equal(host(scales), host(ref_scales), equal_nan=True)


@pytest.mark.parametrize("up", ["one", "random"])
def test_swiglu_every_bf16_gate(ops, up):
    """All 65536 BF16 gate patterns (zeros, subnormals, normals, infinities, NaNs) with
    u = 1 and with random u, through both ops and the unaligned scalar path: every
    activation within the bound, the codes equal to quantize_rows of the activations."""
    width, rows = 8704, 8  # 69632 slots hold every pattern once
    gate = np.zeros(rows * width, np.uint16)
    gate[:65536] = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    gate = gate.reshape(rows, width)
    if up == "one":
        up_bits = np.full((rows, width), 0x3F80, np.uint16)
    else:
        rng = np.random.default_rng(65536)
        up_bits = O.f32_to_bf16(rng.standard_normal((rows, width)).astype(np.float32))
    x_bits = np.concatenate([gate, up_bits], axis=1)
    x = to_dev(x_bits)
    act, codes, scales = run_both(ops, x, width)
    storage = torch.empty(rows * 2 * width + 1, device="cuda", dtype=torch.bfloat16)
    storage[1:].copy_(x.view(-1))
    scalar = torch.empty(rows, width, device="cuda", dtype=torch.bfloat16)
    ops.silu_mul(storage[1:].view(rows, 2 * width), scalar)
    torch.cuda.synchronize()
    got = bf16_bits(act)
    lo, hi = O.silu_mul_bounds(x_bits)
    ok = O.within_bounds(got, lo, hi)
    bad = np.argwhere(~ok)
    assert ok.all(), [(hex(int(gate[r, c])), hex(int(got[r, c])), lo[r, c], hi[r, c])
                      for r, c in bad[:6]]
    assert O.within_bounds(bf16_bits(scalar), lo, hi).all()
    ocodes, oscales = O.silu_mul_quantize(x_bits, activations=got)
    assert np.array_equal(host(codes), ocodes)
    assert np.array_equal(host(scales), oscales, equal_nan=True)


def test_swiglu_graph_replay(ops):
    """tests/test_cuda_ops.py:901-911: both ops captured in a graph, the input changed in
    place, several replays with eager work between them, each equal to eager calls."""
    rows, width = 512, 8704
    torch.manual_seed(5)
    x = torch.randn(rows, 2 * width, device="cuda", dtype=torch.bfloat16) * 3
    act, codes, scales = run_both(ops, x, width)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.silu_mul(x, act)
        ops.silu_mul_quantize(x, codes, scales)
    for step in range(3):
        x.mul_(0.75)
        graph.replay()
        torch.cuda.synchronize()
        ref_act, ref_codes, ref_scales = run_both(ops, x, width)
        torch.cuda.synchronize()
        assert torch.equal(act, ref_act), step
        assert torch.equal(codes, ref_codes), step
        assert torch.equal(scales, ref_scales), step


def test_swiglu_writes_only_its_outputs(ops):
    rows, width = 3, 17408
    x = to_dev(swiglu_input(rows, width, 11))
    act, act_buf = with_guard((rows, width), torch.bfloat16, float("nan"))
    codes, codes_buf = with_guard((rows, width), torch.int8, 77)
    scales, scales_buf = with_guard((rows,), torch.float32, -5.0)
    ops.silu_mul(x, act)
    ops.silu_mul_quantize(x, codes, scales)
    torch.cuda.synchronize()
    assert guard_intact(act_buf, float("nan"))
    assert guard_intact(codes_buf, 77)
    assert guard_intact(scales_buf, -5.0)
    assert not torch.isnan(act.float()).any()


def test_swiglu_silu_mul_accepts_unaligned_views(ops):
    """silu_mul has no alignment requirement (csrc/bindings.cpp:32-44): a view that
    starts one element into its storage runs the scalar path with the same results."""
    rows, width = 4, 8704
    x_bits = swiglu_input(rows, width, 13)
    storage = to_dev(np.concatenate([np.zeros(1, np.uint16), x_bits.reshape(-1)]))
    x = storage[1:].view(rows, 2 * width)
    out_storage = torch.empty(rows * width + 1, device="cuda", dtype=torch.bfloat16)
    out = out_storage[1:].view(rows, width)
    ops.silu_mul(x, out)
    aligned = torch.empty(rows, width, device="cuda", dtype=torch.bfloat16)
    ops.silu_mul(to_dev(x_bits), aligned)
    torch.cuda.synchronize()
    assert torch.equal(out, aligned)


def test_swiglu_quantization_rejects_unaligned_input_before_vector_load(ops):
    """tests/test_cuda_ops.py:914-921."""
    width = 8704
    x = torch.empty(2 * width + 1, device="cuda", dtype=torch.bfloat16)[1:]
    codes = torch.empty(1, width, device="cuda", dtype=torch.int8)
    scales = torch.empty(1, device="cuda")
    with pytest.raises(RuntimeError, match="aligned buffers"):
        ops.silu_mul_quantize(x.view(1, -1), codes, scales)


def test_swiglu_rejects_unsupported_shapes(ops):
    x = torch.zeros(2, 2 * 4096, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="Unsupported SwiGLU shape"):
        ops.silu_mul(x, torch.empty(2, 4096, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="Unsupported SwiGLU quantization shape"):
        ops.silu_mul_quantize(x, torch.empty(2, 4096, device="cuda", dtype=torch.int8),
                              torch.empty(2, device="cuda"))
    x = torch.zeros(2, 2 * 8704, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="Unsupported SwiGLU quantization shape"):
        ops.silu_mul_quantize(x, torch.empty(2, 8704, device="cuda", dtype=torch.int8),
                              torch.empty(3, device="cuda"))
    with pytest.raises(RuntimeError, match="Unexpected dtype or noncontiguous tensor"):
        ops.silu_mul(x.float(), torch.empty(2, 8704, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="Unexpected dtype or noncontiguous tensor"):
        ops.silu_mul(x, torch.empty(8704, 2, device="cuda", dtype=torch.bfloat16).t())


def test_swiglu_through_the_c_abi(lib):
    """The C entry points on raw device pointers and the current stream give the same
    bits as the torch ops."""
    from consumer_int8 import ops

    rows, width = 8, 17408
    x = to_dev(swiglu_input(rows, width, 17))
    act, codes, scales = run_both(ops, x, width)
    act2 = torch.empty_like(act)
    codes2 = torch.empty_like(codes)
    scales2 = torch.empty_like(scales)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.ci8_silu_mul(x.data_ptr(), act2.data_ptr(), rows, width, stream) == 0
    assert lib.ci8_silu_mul_quantize(x.data_ptr(), codes2.data_ptr(), scales2.data_ptr(),
                                     rows, width, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(act, act2) and torch.equal(codes, codes2) and torch.equal(scales, scales2)
