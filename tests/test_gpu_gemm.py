"""GPU parity of fused_channel_mm, cutlass_channel_mm and channel_mm (bit-exact).

Mirrors tests/test_cuda_ops.py:474-490, :563-600 of the reference (schedules, partial
tiles, graph replay, exact INT32 workspace, biased-UINT8 weights), against the oracle
on the same CPU-generated inputs. Full-size configurations are checked through exact
row/column checksums of the INT32 accumulators plus sampled rows and columns.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, guard_intact, host, to_dev, with_guard

pytestmark = pytest.mark.gpu


def gemm_inputs(rng, m, n, k, biased=False):
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    if biased:
        w = rng.integers(1, 256, (n, k)).astype(np.uint8)
    else:
        w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sa = (rng.random(m).astype(np.float32) / np.float32(127)).astype(np.float32)
    sw = O.f32_to_bf16(rng.random(n).astype(np.float32) / np.float32(127))
    return a, w, sa, sw


@pytest.mark.parametrize("m", [1, 17, 64, 256, 1024, 1041, 2048, 2057])
@pytest.mark.parametrize("fused", [None, 0, 1, 2, 3, 4, 5, 6])
@pytest.mark.parametrize("n,k", [(128, 512), (132, 544)])
def test_gemm_schedules_match_integer_products_and_capture(ops, m, fused, n, k):
    rng = np.random.default_rng(m * 1000 + n + k + (fused if fused is not None else 9))
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k)
    a, w, sa, sw = to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np)
    workspace = torch.empty(m, n, device="cuda", dtype=torch.int32)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)

    def run():
        if fused is not None:
            ops.fused_channel_mm(a, w, sa, sw, out, fused)
        else:
            ops.cutlass_channel_mm(a, w, sa, sw, workspace, out)

    run()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    out.fill_(float("nan"))
    workspace.fill_(-1)
    graph.replay()
    torch.cuda.synchronize()
    acc, expected = O.cutlass_channel_mm(a_np, w_np, sa_np, sw_np)
    if fused is None:
        assert np.array_equal(host(workspace), acc)
    assert np.array_equal(bf16_bits(out), expected)


@pytest.mark.parametrize("m,n,k", [(1, 5120, 5120), (4, 2560, 3072), (17, 37, 128),
                                   # M >= 1024: the persistent 224-wide kernel (n % 4 == 0),
                                   # which debiases W fragments in registers, or the
                                   # large-tile kernel; one stage, ragged K, partial tiles
                                   (1024, 224, 128), (1041, 232, 544), (2057, 480, 4096),
                                   (1100, 17, 96), (3000, 452, 1440), (5000, 2244, 2176)])
def test_channel_mm_matches_integer_product_with_output_tails(ops, m, n, k):
    rng = np.random.default_rng(17)
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k, biased=True)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.channel_mm(to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np), out)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), O.channel_mm(a_np, w_np, sa_np, sw_np))


@pytest.mark.parametrize("a_off,w_off", [(1, 0), (0, 4), (3, 7), (16, 8)])
@pytest.mark.parametrize("m,n,k", [(5, 70, 96), (130, 300, 544)])
def test_channel_mm_accepts_operands_at_any_offset(ops, a_off, w_off, m, n, k):
    """Operands sliced out of larger buffers at byte offsets the 16-byte copies cannot
    take (csrc/bindings.cpp:238-265 accepts any view) run the byte-load kernel, with the
    same bits as the oracle."""
    rng = np.random.default_rng(a_off * 100 + w_off + m)
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k, biased=True)
    a_buf = torch.zeros(m * k + 32, dtype=torch.int8, device="cuda")
    w_buf = torch.zeros(n * k + 32, dtype=torch.uint8, device="cuda")
    a = a_buf[a_off : a_off + m * k].view(m, k)
    w = w_buf[w_off : w_off + n * k].view(n, k)
    a.copy_(to_dev(a_np))
    w.copy_(to_dev(w_np))
    assert a.data_ptr() % 16 == a_off % 16 and w.data_ptr() % 16 == w_off % 16
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.channel_mm(a, w, to_dev(sa_np), to_dev(sw_np), out)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), O.channel_mm(a_np, w_np, sa_np, sw_np))


def test_channel_mm_rejects_unaligned_k_before_launch(ops):
    with pytest.raises(RuntimeError, match="geometry"):
        ops.channel_mm(
            torch.zeros(1, 33, dtype=torch.int8, device="cuda"),
            torch.zeros(4, 33, dtype=torch.uint8, device="cuda"),
            torch.ones(1, device="cuda"),
            torch.ones(4, dtype=torch.bfloat16, device="cuda"),
            torch.empty(1, 4, dtype=torch.bfloat16, device="cuda"),
        )


def test_fused_rejects_bad_geometry_and_schedule(ops):
    a = torch.zeros(4, 64, dtype=torch.int8, device="cuda")
    w = torch.zeros(6, 64, dtype=torch.int8, device="cuda")
    sa = torch.ones(4, device="cuda")
    sw = torch.ones(6, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(4, 6, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="geometry"):  # n % 4 != 0
        ops.fused_channel_mm(a, w, sa, sw, out, 0)
    w = torch.zeros(8, 64, dtype=torch.int8, device="cuda")
    sw = torch.ones(8, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(4, 8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="schedule"):
        ops.fused_channel_mm(a, w, sa, sw, out, 7)


@pytest.mark.parametrize("m,n,k", [(64, 256, 2048), (300, 1000, 4096), (4, 4096, 4096)])
def test_fused_output_guards_and_odd_tiles(ops, m, n, k):
    rng = np.random.default_rng(m + n + k)
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k)
    out, buf = with_guard((m, n), torch.bfloat16, float("nan"))
    ops.fused_channel_mm(to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np), out, 0)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), O.fused_channel_mm(a_np, w_np, sa_np, sw_np))
    assert guard_intact(buf, float("nan"))


def test_workspace_extremes_at_max_k(ops):
    """|acc| up to 2^30 at K = 65536: exact INT32 and the INT32 -> FP32 rounding."""
    m, n, k = 3, 8, 65536
    a_np = np.full((m, k), -128, np.int8)
    a_np[1] = 127
    a_np[2, ::2] = 127
    w_np = np.full((n, k), -128, np.int8)
    w_np[1::2] = 127
    sa_np = np.array([1.0, 0.5, 3e-3], np.float32)
    sw_np = O.f32_to_bf16(np.linspace(0.001, 0.01, n).astype(np.float32))
    ws = torch.empty(m, n, device="cuda", dtype=torch.int32)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.cutlass_channel_mm(to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np), ws, out)
    torch.cuda.synchronize()
    acc, expected = O.cutlass_channel_mm(a_np, w_np, sa_np, sw_np)
    assert acc[0, 0] == 2**30
    assert np.array_equal(host(ws), acc) and np.array_equal(bf16_bits(out), expected)


def full_size_check(a_np, w_signed, sa_np, sw_np, acc_dev, out_bits, samples=24, seed=0):
    """Exact checks that cover every accumulator at sizes the CPU cannot multiply fast.

    All sums below are integers below 2^53 in magnitude (|acc| < 2^31, at most 2^15
    terms of at most 2^34), so float64 BLAS computes them exactly.
    """
    acc = host(acc_dev)
    accf = acc.astype(np.float64)
    af = a_np.astype(np.float64)
    wf = w_signed.astype(np.float64)
    # Row and column checksums: sum_n acc[m, n] = a[m] . colsum(w), and the transpose.
    assert np.array_equal(accf.sum(axis=1), af @ wf.sum(axis=0))
    assert np.array_equal(accf.sum(axis=0), wf @ af.sum(axis=0))
    # Weighted checksums catch compensating errors that plain sums miss.
    rng = np.random.default_rng(seed)
    u = rng.integers(-3, 4, acc.shape[1]).astype(np.float64)
    v = rng.integers(-3, 4, acc.shape[0]).astype(np.float64)
    assert np.array_equal(accf @ u, af @ (wf.T @ u))
    assert np.array_equal(v @ accf, (v @ af) @ wf.T)
    del accf, af, wf
    rows = rng.choice(acc.shape[0], samples, replace=False)
    cols = rng.choice(acc.shape[1], samples, replace=False)
    assert np.array_equal(acc[rows], O.int_matmul(a_np[rows], w_signed))
    assert np.array_equal(acc[:, cols], O.int_matmul(a_np, w_signed[cols]))
    # The BF16 output is the oracle epilogue of those (now verified) accumulators.
    assert np.array_equal(out_bits, O.channel_epilogue(acc, sa_np, sw_np))


def test_prefill_projection_full_size(ops):
    """Config 3: quantize_rows on BF16 [4096, 5120] with outlier channels, then
    fused_channel_mm with N = 17408."""
    m, k, n = 4096, 5120, 17408
    rng = np.random.default_rng(20261011)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, rng.choice(k, 5, replace=False)] *= 50
    x_bits = O.f32_to_bf16(x)
    w_np = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sw_np = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    xt = to_dev(x_bits)
    codes = torch.empty(m, k, device="cuda", dtype=torch.int8)
    sa = torch.empty(m, device="cuda")
    ops.quantize_rows(xt, codes, sa)
    w = to_dev(w_np)
    sw = to_dev(sw_np)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.fused_channel_mm(codes, w, sa, sw, out, 0)
    ws = torch.empty(m, n, device="cuda", dtype=torch.int32)
    out2 = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.cutlass_channel_mm(codes, w, sa, sw, ws, out2)
    torch.cuda.synchronize()
    a_np, sa_np = O.quantize_rows(x_bits)
    assert np.array_equal(host(codes), a_np) and np.array_equal(host(sa), sa_np)
    out_bits = bf16_bits(out)
    assert np.array_equal(out_bits, bf16_bits(out2))
    full_size_check(a_np, w_np, sa_np, sw_np, ws, out_bits)


def test_down_projection_biased_weights_full_size(ops):
    """Config 4: M = 16384, K = 17408, N = 5120 with SiLU-gated activations quantized per
    row and biased UINT8 weights debiased on load (channel_mm)."""
    m, k, n = 16384, 17408, 5120
    rng = np.random.default_rng(4)
    g = rng.standard_normal((m, k), dtype=np.float32)
    u = rng.standard_normal((m, k), dtype=np.float32)
    x_bits = O.f32_to_bf16((g / (1 + np.exp(-g))) * u)
    del g, u
    w_u8 = rng.integers(1, 256, (n, k)).astype(np.uint8)
    sw_np = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    codes = torch.empty(m, k, device="cuda", dtype=torch.int8)
    sa = torch.empty(m, device="cuda")
    ops.quantize_rows(to_dev(x_bits), codes, sa)
    w = to_dev(w_u8)
    sw = to_dev(sw_np)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.channel_mm(codes, w, sa, sw, out)
    # The same product with signed weights exposes the accumulators.
    w_signed = O.debias(w_u8)
    ws = torch.empty(m, n, device="cuda", dtype=torch.int32)
    out2 = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.cutlass_channel_mm(codes, to_dev(w_signed), sa, sw, ws, out2)
    torch.cuda.synchronize()
    a_np, sa_np = O.quantize_rows(x_bits)
    assert np.array_equal(host(codes), a_np) and np.array_equal(host(sa), sa_np)
    out_bits = bf16_bits(out)
    assert np.array_equal(out_bits, bf16_bits(out2))
    full_size_check(a_np, w_signed, sa_np, sw_np, ws, out_bits, samples=8)


@pytest.mark.parametrize("biased", [False, True])
def test_wide_tiles_where_they_fill_the_rounds(ops, biased):
    """M = N = 4096: 304 tiles of 256 x 224 need 2 rounds on 256 CUs and 256 tiles of
    256 x 256 need 1, so schedule 0 (and channel_mm) runs the 256-wide kernel rather than
    the persistent 224-wide one, with a
    K that is not a whole number of 128-byte stages. It agrees bit for bit with the
    128 x 128 tiling (schedule 1) and, through the exact INT32 accumulators of the
    workspace variant, with the oracle on sampled rows and columns."""
    m, n, k = 4096, 4096, 1056
    rng = np.random.default_rng(256 + biased)
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k, biased=biased)
    w_signed = O.debias(w_np) if biased else w_np
    a, sa, sw, ws_dev = to_dev(a_np), to_dev(sa_np), to_dev(sw_np), to_dev(w_signed)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    if biased:
        ops.channel_mm(a, to_dev(w_np), sa, sw, out)
    else:
        ops.fused_channel_mm(a, ws_dev, sa, sw, out, 0)
    ref = torch.empty_like(out)
    ops.fused_channel_mm(a, ws_dev, sa, sw, ref, 1)
    acc = torch.empty(m, n, device="cuda", dtype=torch.int32)
    out2 = torch.empty_like(out)
    ops.cutlass_channel_mm(a, ws_dev, sa, sw, acc, out2)
    torch.cuda.synchronize()
    out_bits = bf16_bits(out)
    assert np.array_equal(out_bits, bf16_bits(ref))
    assert np.array_equal(out_bits, bf16_bits(out2))
    full_size_check(a_np, w_signed, sa_np, sw_np, acc, out_bits, samples=8)


@pytest.mark.parametrize("m,n,k,biased", [
    (2048, 17408, 128, False),   # one K stage: the next tile's copies go out at the switch
    (2048, 17408, 256, True),    # two stages: group 1 copies the next tile from stage 0
    (2048, 17408, 384, False),   # an odd stage count: ring slots alternate across tiles
    (3000, 9000, 1056, True),    # K tail, ragged M and N tiles
    # On 256 CUs the persistent kernel splits the columns of these: a round of 224-wide
    # tiles, then one of 160-wide tiles over the rest (tests/test_tile_plan.py checks the
    # plans), with one K stage, a K tail, a ragged last tile, rows that are not 16-byte
    # aligned (N = 18500) and ragged M.
    (1024, 23040, 128, True),
    (1024, 23040, 640, False),
    (1100, 18500, 1056, True),
])
def test_persistent_tile_switches(ops, m, n, k, biased):
    """Shapes where the persistent kernel runs two or more tiles per workgroup, so each
    workgroup's copy stream runs on from one tile's last stages into the next tile's first
    (ring slots numbered over the whole launch). The output equals the 128 x 128 tiling's
    (schedule 1) and the workspace kernel's, whose exact INT32 accumulators are checked
    against the oracle through checksums and sampled rows and columns."""
    rng = np.random.default_rng(m + n + k + biased)
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k, biased=biased)
    w_signed = O.debias(w_np) if biased else w_np
    a, sa, sw, ws_dev = to_dev(a_np), to_dev(sa_np), to_dev(sw_np), to_dev(w_signed)
    out, buf = with_guard((m, n), torch.bfloat16, float("nan"))
    print(f"persistent tile switches m={m} n={n} k={k} biased={biased}", flush=True)
    if biased:
        ops.channel_mm(a, to_dev(w_np), sa, sw, out)
    else:
        ops.fused_channel_mm(a, ws_dev, sa, sw, out, 0)
    ref = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.fused_channel_mm(a, ws_dev, sa, sw, ref, 1)
    acc = torch.empty(m, n, device="cuda", dtype=torch.int32)
    out2 = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.cutlass_channel_mm(a, ws_dev, sa, sw, acc, out2)
    torch.cuda.synchronize()
    out_bits = bf16_bits(out)
    assert guard_intact(buf, float("nan"))
    assert np.array_equal(out_bits, bf16_bits(ref))
    assert np.array_equal(out_bits, bf16_bits(out2))
    full_size_check(a_np, w_signed, sa_np, sw_np, acc, out_bits, samples=8)


@pytest.mark.parametrize("m,n,k,biased", [
    # 128 < M <= 256 on 256 CUs (tests/test_tile_plan.py checks the choices): 128 x 128
    # tiles in one round, in 1.5 rounds with a K tail, and at M = 160; 256 x 224 tiles.
    (256, 11264, 256, False),
    (256, 24576, 160, False),
    (160, 16384, 96, True),
    (200, 34816, 128, True),
    # M >= 1024 with under half the CUs' worth of persistent tiles: 128 x 128 tiles.
    (1024, 2560, 544, True),
    (1100, 2000, 256, False),
])
def test_schedule0_mid_m_and_few_tile_choices(ops, m, n, k, biased):
    """Schedule 0 where it runs the 128 x 128 or the 256 x 224 kernel in place of the
    small-M or the persistent kernel. The output equals the 256 x 32 tiling's (schedule 5)
    and that of the workspace op (which takes the same choice), whose exact INT32
    accumulators are checked against the oracle through checksums and sampled rows and
    columns."""
    rng = np.random.default_rng(m * 7 + n + k + biased)
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k, biased=biased)
    w_signed = O.debias(w_np) if biased else w_np
    a, sa, sw, ws_dev = to_dev(a_np), to_dev(sa_np), to_dev(sw_np), to_dev(w_signed)
    out, buf = with_guard((m, n), torch.bfloat16, float("nan"))
    print(f"schedule 0 choice m={m} n={n} k={k} biased={biased}", flush=True)
    if biased:
        ops.channel_mm(a, to_dev(w_np), sa, sw, out)
    else:
        ops.fused_channel_mm(a, ws_dev, sa, sw, out, 0)
    ref = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.fused_channel_mm(a, ws_dev, sa, sw, ref, 5)
    acc = torch.empty(m, n, device="cuda", dtype=torch.int32)
    out2 = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.cutlass_channel_mm(a, ws_dev, sa, sw, acc, out2)
    torch.cuda.synchronize()
    out_bits = bf16_bits(out)
    assert guard_intact(buf, float("nan"))
    assert np.array_equal(out_bits, bf16_bits(ref))
    assert np.array_equal(out_bits, bf16_bits(out2))
    full_size_check(a_np, w_signed, sa_np, sw_np, acc, out_bits, samples=8)


@pytest.mark.parametrize("biased", [False, True])
def test_column_split_in_graph_replays(ops, biased):
    """The column split (a launch of 224-wide tiles over whole rounds, then one of
    160-wide tiles; M = 1024, N = 23040 on 256 CUs: a round over 14,336 columns, then
    220 narrow tiles) captured into a HIP graph: three replays, each after eager work that
    overwrites the output, equal the eager call bit for bit, and the eager call equals the
    128 x 128 tiling (schedule 1)."""
    m, n, k = 1024, 23040, 640
    rng = np.random.default_rng(23040 + biased)
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k, biased=biased)
    w_signed = O.debias(w_np) if biased else w_np
    a, sa, sw, w, ws_dev = to_dev(a_np), to_dev(sa_np), to_dev(sw_np), to_dev(w_np), to_dev(w_signed)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    print(f"column split graph replay biased={biased}", flush=True)

    def run():
        if biased:
            ops.channel_mm(a, w, sa, sw, out)
        else:
            ops.fused_channel_mm(a, w, sa, sw, out, 0)

    run()
    ref = torch.empty_like(out)
    ops.fused_channel_mm(a, ws_dev, sa, sw, ref, 1)
    torch.cuda.synchronize()
    eager = bf16_bits(out)
    assert np.array_equal(eager, bf16_bits(ref))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for rep in range(3):
        out.fill_(float(rep) - 7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(out), eager), rep


def test_c_abi_fused_matches_oracle(ops, lib):
    from consumer_int8 import _abi

    rng = np.random.default_rng(31)
    m, n, k = 333, 1028, 1056
    a_np, w_np, sa_np, sw_np = gemm_inputs(rng, m, n, k)
    a, w, sa, sw = to_dev(a_np), to_dev(w_np), to_dev(sa_np), to_dev(sw_np)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    _abi.check(lib.ci8_fused_channel_mm(a.data_ptr(), w.data_ptr(), sa.data_ptr(),
                                        sw.data_ptr(), out.data_ptr(), m, n, k, 0, stream))
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), O.fused_channel_mm(a_np, w_np, sa_np, sw_np))
