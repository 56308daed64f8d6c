"""GPU checks of ci8_cutlass_channel_mm_noalloc, through the C ABI.

The no-allocation variant runs cutlass_channel_mm's kernels with the INT32 accumulators
in the library's own device array instead of a caller workspace, so its BF16 output
must equal cutlass_channel_mm's bit for bit (and the oracle's). Consecutive calls share
the array; each case makes two calls in a row, the second on smaller inputs, and checks
both against the workspace entry point on the same inputs.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, guard_intact, to_dev, with_guard

pytestmark = pytest.mark.gpu

GUARD = 0x7F7F  # BF16 bit pattern of the sentinel around each output


def gemm_inputs(rng, m, n, k):
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sa = (rng.random(m).astype(np.float32) / np.float32(127)).astype(np.float32)
    sw = O.f32_to_bf16(rng.random(n).astype(np.float32) / np.float32(127))
    return a, w, sa, sw


def run_both(lib, rng, m, n, k, oracle_check):
    from consumer_int8 import _abi

    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k)
    a, w, sa, sw = to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np)
    stream = torch.cuda.current_stream().cuda_stream
    guard_bf16 = torch.tensor([GUARD], dtype=torch.int16).view(torch.bfloat16).item()
    out, buf = with_guard((m, n), torch.bfloat16, guard_bf16)
    print(f"noalloc m={m} n={n} k={k}", flush=True)
    _abi.check(lib.ci8_cutlass_channel_mm_noalloc(a.data_ptr(), w.data_ptr(), sa.data_ptr(),
                                                  sw.data_ptr(), out.data_ptr(), m, n, k,
                                                  stream))
    workspace = torch.empty(m, n, device="cuda", dtype=torch.int32)
    ref = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    _abi.check(lib.ci8_cutlass_channel_mm(a.data_ptr(), w.data_ptr(), sa.data_ptr(),
                                          sw.data_ptr(), workspace.data_ptr(), ref.data_ptr(),
                                          m, n, k, stream))
    torch.cuda.synchronize()
    bits = bf16_bits(out)
    assert np.array_equal(bits, bf16_bits(ref))
    assert guard_intact(buf.view(torch.int16), GUARD)
    if oracle_check:
        assert np.array_equal(bits, O.fused_channel_mm(a_np, w_np, sa_np, sw_np))
    return bits


@pytest.mark.parametrize("first,second", [
    ((128, 4096, 4096), (37, 1000, 512)),   # configs[0] (small-M kernel), then ragged
    ((1024, 4096, 1024), (300, 1028, 544)),  # large-M tiles, then medium tiles, K tail
    ((2048, 4096, 64), (1, 4, 32)),          # the scratch limit exactly, then minimal
])
def test_noalloc_matches_cutlass_on_two_calls(ops, lib, first, second):
    rng = np.random.default_rng(sum(first) + sum(second))
    run_both(lib, rng, *first, oracle_check=first[0] * first[1] * first[2] <= 1 << 31)
    run_both(lib, rng, *second, oracle_check=True)


def test_noalloc_rejects_beyond_scratch_without_launching(ops, lib):
    from consumer_int8 import _abi

    out = torch.full((4,), 1.0, device="cuda", dtype=torch.bfloat16)
    big = 1 << 20
    status = lib.ci8_cutlass_channel_mm_noalloc(big, big, big, big, out.data_ptr(), 4096,
                                                4096, 32, None)
    assert status == _abi.CI8_ERR_TOO_LARGE
    assert "scratch" in _abi.last_error()
    torch.cuda.synchronize()
    assert bool((out == 1.0).all())


def test_noalloc_graph_replays(ops, lib):
    """Captured after one eager call (which resolves the array's address on this device),
    replayed three times with eager work between the replays; every replay equals the
    workspace entry point's output."""
    from consumer_int8 import _abi

    rng = np.random.default_rng(5)
    m, n, k = 96, 2048, 1024
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k)
    a, w, sa, sw = to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ref = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    workspace = torch.empty(m, n, device="cuda", dtype=torch.int32)

    def call():
        stream = torch.cuda.current_stream().cuda_stream
        _abi.check(lib.ci8_cutlass_channel_mm_noalloc(a.data_ptr(), w.data_ptr(),
                                                      sa.data_ptr(), sw.data_ptr(),
                                                      out.data_ptr(), m, n, k, stream))

    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    stream = torch.cuda.current_stream().cuda_stream
    _abi.check(lib.ci8_cutlass_channel_mm(a.data_ptr(), w.data_ptr(), sa.data_ptr(),
                                          sw.data_ptr(), workspace.data_ptr(), ref.data_ptr(),
                                          m, n, k, stream))
    torch.cuda.synchronize()
    expected = bf16_bits(ref)
    assert np.array_equal(expected, O.fused_channel_mm(a_np, w_np, sa_np, sw_np))
    for replay in range(3):
        out.fill_(0.0)
        # Other work on the same scratch between replays: a differently shaped call.
        other = torch.empty(16, 256, device="cuda", dtype=torch.bfloat16)
        _abi.check(lib.ci8_cutlass_channel_mm_noalloc(a.data_ptr(), w.data_ptr(),
                                                      sa.data_ptr(), sw.data_ptr(),
                                                      other.data_ptr(), 16, 256, k, stream))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(out), expected), replay
