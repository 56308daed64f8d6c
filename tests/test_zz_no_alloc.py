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


FIRST_CALL_UNDER_CAPTURE = r"""
import numpy as np
import torch
from consumer_int8 import _abi

lib = _abi.load()
m, n, k = 64, 256, 128
g = torch.Generator().manual_seed(3)
a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g).cuda()
w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).cuda()
sa = (torch.rand(m, generator=g) / 127).cuda()
sw = (torch.rand(n, generator=g) / 127).to(torch.bfloat16).cuda()
out = torch.zeros(m, n, device="cuda", dtype=torch.bfloat16)
ref = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
ws = torch.empty(m, n, device="cuda", dtype=torch.int32)


def call(target):
    stream = torch.cuda.current_stream().cuda_stream
    return lib.ci8_cutlass_channel_mm_noalloc(a.data_ptr(), w.data_ptr(), sa.data_ptr(),
                                              sw.data_ptr(), target.data_ptr(), m, n, k, stream)


# The process's first call, under capture: refused before any HIP work is recorded.
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    out.zero_()
    status = call(out)
assert status == _abi.CI8_ERR_LAUNCH, status
assert "outside graph capture" in _abi.last_error(), _abi.last_error()
# An eager call sets up the device; a captured call then works and replays exactly.
_abi.check(call(out))
_abi.check(lib.ci8_cutlass_channel_mm(a.data_ptr(), w.data_ptr(), sa.data_ptr(), sw.data_ptr(),
                                      ws.data_ptr(), ref.data_ptr(), m, n, k,
                                      torch.cuda.current_stream().cuda_stream))
torch.cuda.synchronize()
assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    _abi.check(call(out))
for replay in range(2):
    out.fill_(7.0)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), replay
print("first-call-under-capture: ok", flush=True)
"""


def test_noalloc_first_call_under_capture_is_refused(ops, lib):
    """In a fresh process (a child, started after this one has initialised the GPU; no
    exec), the first call on the device is made under graph capture: it is refused with a
    clear error and records nothing; after one eager call, captured calls replay exactly.
    (Calls past the scratch limit are refused on the host; tests/test_abi.py checks that
    without a GPU.)"""
    import os
    import subprocess
    import sys

    from tests.conftest import PKG, REPO

    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(REPO), str(PKG), env.get("PYTHONPATH", "")])
    print("noalloc first call under capture (child process)", flush=True)
    result = subprocess.run([sys.executable, "-c", FIRST_CALL_UNDER_CAPTURE], cwd=str(REPO),
                            env=env, capture_output=True, text=True, timeout=240)
    assert result.returncode == 0, result.stdout[-2000:] + result.stderr[-4000:]
    assert "first-call-under-capture: ok" in result.stdout


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
