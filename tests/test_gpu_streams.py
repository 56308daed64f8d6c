"""The ops run on the current stream of the input's device, asynchronously, as the
reference's bindings do (csrc/bindings.cpp:23-27, `stream_for`: the current stream of
the tensor's device, from aoti_torch_get_current_cuda_stream).

The chain quantize_rows -> fused_channel_mm -> channel_gemv is issued on a side stream
(default priority) right after that stream produces its input behind a long kernel, and
must give the same bits as on the default stream. An op launched on any other stream
would read the input before it was written.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, host, to_dev

pytestmark = pytest.mark.gpu


def chain(ops, x, w, sw, xg):
    m, k = x.shape
    codes = torch.empty(m, k, device=x.device, dtype=torch.int8)
    sa = torch.empty(m, device=x.device)
    ops.quantize_rows(x, codes, sa)
    out = torch.empty(m, w.shape[0], device=x.device, dtype=torch.bfloat16)
    ops.fused_channel_mm(codes, w, sa, sw, out, 0)
    gv = torch.empty(xg.shape[0], w.shape[0], device=x.device, dtype=torch.bfloat16)
    ops.channel_gemv(xg, w, sw, gv)
    return codes, sa, out, gv


def test_ops_follow_the_current_stream(ops):
    rng = np.random.default_rng(77)
    m, k, n = 1024, 1024, 1152
    x_bits = O.f32_to_bf16(rng.standard_normal((m, k)).astype(np.float32))
    w_np = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sw_np = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    xg_bits = O.f32_to_bf16(rng.standard_normal((4, k)).astype(np.float32))
    x, w, sw, xg = to_dev(x_bits), to_dev(w_np), to_dev(sw_np), to_dev(xg_bits)
    expected = chain(ops, x, w, sw, xg)
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        # A long producer first, then the input copy, both on the side stream.
        big = torch.randn(4096, 4096, device="cuda")
        for _ in range(4):
            big = big @ big.T / 4096
        x2 = torch.empty_like(x)
        x2.copy_(x)
        got = chain(ops, x2, w, sw, xg)
    side.synchronize()
    for e, g in zip(expected, got):
        assert torch.equal(e, g)
    # And against the oracle for the quantizer and GEMM.
    a_np, sa_np = O.quantize_rows(x_bits)
    assert np.array_equal(host(got[0]), a_np) and np.array_equal(host(got[1]), sa_np)
    assert np.array_equal(bf16_bits(got[2]), O.fused_channel_mm(a_np, w_np, sa_np, sw_np))
