"""Benchmark of the INT8 linear-layer hot path on one MI355X.

Metric: INT8 TOPS and % of dense INT8 MFMA peak for fused_channel_mm at
M=4096, K=5120, N=17408. One step is the prefill-projection pass of configs[2]:
quantize_rows on BF16 [4096, 5120] (N(0,1), 0.1% of channels x50) followed by
fused_channel_mm against signed INT8 weights [17408, 5120] with BF16 channel scales.
`value` is 2*M*N*K / (wall time per step), i.e. the quantizer's time is charged to the
GEMM. Inputs are resident in HBM before timing; the weights, activations and codes
rotate over enough copies that no step finds its inputs in the 256 MB Infinity Cache.

Also reported: `roofline` for the dominant kernel (the GEMM, timed per launch with HIP
events on the stream it runs on); `mfma_probe`, the INT8 MFMA rate and shader clock
under a full-chip pure-MFMA loop, with the dense INT8 peak at that measured clock
(`roofline.frac_at_measured_clock` divides by it); `hbm_probe`, what plain streams of the
GEMV's and the quantizer's bytes achieve (the HBM lines' `frac_of_stream` divides by
it); `roofline.graph_median_us`, the GEMM
timed as in the reference microbenchmark (graph replays of 10 launches, median); extra roofline lines for the quantizer, the W8A16
GEMV, the grouped summed GEMM, the biased-UINT8 down
projection with its SwiGLU activation producers (silu_mul_quantize,
silu_mul), the AllSpark weight restore (unpack_allspark), the block-32 Q8_0 W8A8 GEMM,
the GGUF Q8_0 grouped W8A16 op (gguf_q8_packed_mm) and the small quantize + GEMM pass
(configs[0]); `vendor_int_mm_cfg3`, the vendor library's INT8 GEMM (torch._int_mm, i.e.
hipBLASLt, INT32 output) on the headline shape and inputs, for reference; and
`cpu_baseline`, the reference's torch CPU math for the same step on a bounded row slice,
on this host's cores.

Inputs of the step are generated on the host from recorded seeds (`seeds`) and copied to
the device. After the timed region the run checks its own output, as the reference
microbenchmark does before reporting a time (benchmarks/microbench.py:205-214, :296-303):
the leading rows of one step are recomputed by the reference's CPU math on the same host
tensors (the cpu_baseline sample, or 64 rows without it), and the GPU's codes, row scales,
INT32 products (cutlass_channel_mm's workspace) and BF16 outputs of those rows must equal
them bit for bit; fused_channel_mm must equal cutlass_channel_mm over the whole output.
The result is the `parity` record; any mismatch makes the script exit with status 1.

Before the W warm-up steps the same step runs untimed for `--condition-seconds` (0.15 s),
because the chip ramps its clock over tens of milliseconds after idle; the count is
reported as `conditioning`. The timed region is exactly K steps. The two other
MFMA-bound extras (the grouped summed GEMM and the down projection) get 0.15 s of
untimed launches of their own before they are timed.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-extras]
                      [--copy-calibration] [--condition-seconds S]
       python bench.py --phase-profile   (the GEMM's per-phase cycle table; no bench line)
       python bench.py --linear-sweep OUT.json [--fused-only [--fused-paired]
                      [--fused-schedules S ...]] [--fused-schedule S] [--prefill-only]
                      [--linear-rows M ...] [--linear-shape N K ...]
                      (the reference microbenchmark's linear-layer table; no bench line)
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "consumer-int8-kernels_amd"))
sys.path.insert(0, str(REPO))

M, K, N = 4096, 5120, 17408
GEMM_OPS = 2 * M * N * K  # 730,144,440,320
QUANT_BYTES = 3 * M * K + 4 * M  # BF16 read + INT8 write + FP32 scales
PEAK_INT8_TOPS = 256 * 2.4e9 * 8192 / 1e12  # 5033.2: 256 CUs x 2.4 GHz x 8192 op/clk/CU
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # dense BF16 MFMA
GEMV_K, GEMV_N = 5120, 17408
# HBM-side bytes per GEMM launch at this shape, from two rocprofv3 --pmc runs of this
# script (FETCH_SIZE x 2.00 + WRITE_SIZE x 1.00; the factors make a plain 512 MiB copy
# read back its own size): 628.4 MB read + 143.5 MB written. Counters cannot be read
# from inside a timed run, so the value is carried here and re-measured whenever the
# GEMM kernel changes.
GEMM_TRAFFIC_BYTES = 771_858_240


def gemv_bytes(m: int) -> int:
    return GEMV_N * GEMV_K + 2 * GEMV_N + 2 * m * GEMV_K + 2 * m * GEMV_N


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=30)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extras", action="store_true")
    p.add_argument("--condition-seconds", type=float, default=0.15,
                   help="untimed steps run before the warm-up steps so the GPU is at its "
                        "steady clock (the first ~100 steps after idle run up to 18%% slower)")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="approximate CPU time budget of the cpu_baseline sample")
    p.add_argument("--phase-profile", action="store_true",
                   help="print the persistent GEMM's per-phase cycle table at configs[2] "
                        "(clock-stamped build of the same kernel) instead of the bench line")
    p.add_argument("--copy-calibration", action="store_true",
                   help="also run a plain 512 MiB device copy three times (a kernel of known "
                        "traffic that scales FETCH_SIZE / WRITE_SIZE counters)")
    # The reference microbenchmark's linear-layer options (benchmarks/microbench.py:56-73).
    p.add_argument("--linear-sweep", metavar="OUTPUT",
                   help="run the linear-layer sweep (linear_sweep) instead of the bench line, "
                        "writing its rows to OUTPUT as JSON")
    p.add_argument("--prefill-only", action="store_true")
    p.add_argument("--linear-rows", type=int, nargs="+")
    p.add_argument("--linear-shape", dest="linear_shapes", type=int, nargs=2, action="append")
    p.add_argument("--fused-schedule", type=int, choices=range(7), default=0)
    p.add_argument("--fused-only", action="store_true")
    p.add_argument("--fused-paired", action="store_true")
    p.add_argument("--fused-schedules", type=int, nargs="+", choices=range(7),
                   default=list(range(7)))
    return p.parse_args()


SEED_X = 20261011        # activation copy i uses SEED_X + i
SEED_W = 20261111        # weight copy i uses SEED_W + i
SEED_SW = 20261211       # channel scales


def host_activations(torch, seed):
    """configs[2]'s activations on the host: BF16 [M, K] ~ N(0,1), 0.1% of the channels x50."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=gen, dtype=torch.float32)
    cols = torch.randperm(K, generator=gen)[: max(1, K // 1000)]
    x[:, cols] *= 50
    return x.to(torch.bfloat16)


def device_activations(torch, gen):
    """configs[2]'s activation distribution drawn on the device (the extras' inputs):
    BF16 [M, K] ~ N(0,1) with 0.1% of the channels x50."""
    x = torch.randn(M, K, generator=gen, device="cuda")
    cols = torch.randperm(K, generator=gen, device="cuda")[: max(1, K // 1000)]
    x[:, cols] *= 50
    return x.to(torch.bfloat16)


def host_weights(torch, seed):
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, (N, K), generator=gen, dtype=torch.int8)


def host_channel_scales(torch, seed):
    gen = torch.Generator().manual_seed(seed)
    return (torch.rand(N, generator=gen) * 9e-3 + 1e-3).to(torch.bfloat16)


def make_inputs(torch, copies_w=3, copies_x=3):
    """The step's inputs, generated on the host from the SEED_* seeds and copied to the
    device; copy 0 of the host tensors is kept for the parity check and the CPU baseline."""
    dev = "cuda"
    host = {"x": host_activations(torch, SEED_X), "w": host_weights(torch, SEED_W),
            "sw": host_channel_scales(torch, SEED_SW)}
    xs = [host["x"].to(dev)] + [host_activations(torch, SEED_X + i).to(dev)
                                for i in range(1, copies_x)]
    ws = [host["w"].to(dev)] + [host_weights(torch, SEED_W + i).to(dev)
                                for i in range(1, copies_w)]
    sw = host["sw"].to(dev)
    codes = [torch.empty(M, K, device=dev, dtype=torch.int8) for _ in range(copies_x)]
    sa = torch.empty(M, device=dev, dtype=torch.float32)
    out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    return host, xs, ws, sw, codes, sa, out


def condition(torch, calls, seconds=0.15):
    """Untimed launches for about `seconds`, so an MFMA-bound kernel is timed at the
    clock it holds under sustained load, as the headline GEMM is (the chip runs faster
    for the first ~100 launches after lighter work)."""
    end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < end:
        calls[i % len(calls)]()
        i += 1
        if i % len(calls) == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_kernel(torch, calls, reps, batch=10, settle_s=0.05):
    """Mean and median per-launch time (us) of a rotating list of launch closures: the
    launches run untimed for `settle_s` seconds first (after the previous, different
    workload the chip's clocks take milliseconds to settle on this one; a decode or
    prefill loop runs the kernel continuously), then `reps` event pairs on the current
    stream, each around `batch` back-to-back launches (so the per-launch figure carries no
    event or launch-gap overhead of its own). Eager launches: HIP graph replays of the same
    batches measured 0.7 - 0.9 us more per launch for the 10 - 20 us kernels here."""
    condition(torch, calls, settle_s)
    events = []
    for r in range(reps):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(batch):
            calls[(r * batch + i) % len(calls)]()
        end.record()
        events.append((start, end))
    torch.cuda.synchronize()
    times = [s.elapsed_time(e) * 1e3 / batch for s, e in events]
    return statistics.mean(times), statistics.median(times)


def mfma_clock_probe(torch, cus: int, rounds: int = 4000, reps: int = 5) -> dict:
    """INT8 MFMA rate and shader clock under a full-chip pure-MFMA load (one workgroup of
    4 waves per CU, csrc/probe.hip), and the dense INT8 peak at that measured clock."""
    import ctypes

    lib = ctypes.CDLL(str(REPO / "consumer-int8-kernels_amd" / "consumer_int8" / "libci8_probe.so"))
    lib.ci8probe_mfma_loop.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.ci8probe_ops_per_mfma.restype = ctypes.c_int64
    shader_khz, wall_khz = ctypes.c_int(0), ctypes.c_int(0)
    assert lib.ci8probe_clock_rates(ctypes.byref(shader_khz), ctypes.byref(wall_khz)) == 0
    record = torch.zeros(3 * cus, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    ops = cus * 4 * rounds * lib.ci8probe_mfma_per_round() * lib.ci8probe_ops_per_mfma()
    assert lib.ci8probe_mfma_loop(rounds // 10, cus, ctypes.c_void_p(record.data_ptr()), ctypes.c_void_p(stream)) == 0
    tops, mhz = [], []
    for _ in range(reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        assert lib.ci8probe_mfma_loop(rounds, cus, ctypes.c_void_p(record.data_ptr()), ctypes.c_void_p(stream)) == 0
        end.record()
        torch.cuda.synchronize()
        tops.append(ops / (start.elapsed_time(end) * 1e-3) / 1e12)
        rec = record.view(cus, 3).cpu()
        mhz.append(statistics.median((rec[:, 0].double() / rec[:, 1].double() * wall_khz.value / 1e3).tolist()))
    clock = statistics.median(mhz)
    return {"tops": round(statistics.median(tops), 1), "clock_mhz": round(clock, 1),
            "clock_mhz_max": shader_khz.value / 1e3,
            "peak_at_clock_tops": round(cus * 8192 * clock * 1e6 / 1e12, 1)}


def hbm_stream_probe(torch, cus: int) -> dict:
    """Achievable HBM rates for the two traffic shapes of the HBM-bound kernels
    (csrc/probe.hip): a plain read of the configs[1] weight bytes (K=5120, N=17408), and a
    read of the configs[2] quantizer's BF16 input with a write of half as many bytes (its
    codes), without the quantizer's per-row dependency. Rotated buffers larger than the
    MALL; the best of three grid sizes, each timed as `time_kernel` times the ops."""
    import ctypes

    lib = ctypes.CDLL(str(REPO / "consumer-int8-kernels_amd" / "consumer_int8" / "libci8_probe.so"))
    lib.ci8probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.ci8probe_stream_read2_write1.argtypes = [ctypes.c_void_p, ctypes.c_int64,
                                                 ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    out = {}
    # Random bytes, like the weights the GEMV reads (the time depends on the data).
    read_bytes = GEMV_N * GEMV_K
    gen = torch.Generator(device="cuda").manual_seed(20261311)
    srcs = [torch.randint(0, 256, (read_bytes,), generator=gen, dtype=torch.uint8, device="cuda")
            for _ in range(4)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    best = None
    for variant in (0, 1):  # 8 plain / 16 nontemporal loads in flight per thread
        for blocks in (cus * 4, cus * 8, cus * 16):
            calls = [lambda s=s, b=blocks, v=variant: lib.ci8probe_stream_read(
                         s.data_ptr(), read_bytes, sink.data_ptr(), b, v,
                         torch.cuda.current_stream().cuda_stream) for s in srcs]
            for c in calls:
                assert c() == 0
            mean_us, _ = time_kernel(torch, calls, 8)
            if best is None or mean_us < best[0]:
                best = (mean_us, blocks, variant)
    out["read"] = {"bytes": read_bytes, "mean_us": round(best[0], 2), "blocks": best[1],
                   "variant": ["8 plain loads per thread", "16 nontemporal loads per thread"][best[2]],
                   "gbs": round(read_bytes / (best[0] * 1e-6) / 1e9, 1)}
    del srcs
    rw_read = 2 * M * K
    srcs = [torch.ones(rw_read, dtype=torch.uint8, device="cuda") for _ in range(6)]
    dsts = [torch.empty(rw_read // 2, dtype=torch.uint8, device="cuda") for _ in range(6)]
    best = None
    for blocks in (cus * 4, cus * 8, cus * 16):
        calls = [lambda s=s, d=d, b=blocks: lib.ci8probe_stream_read2_write1(
                     s.data_ptr(), rw_read, d.data_ptr(), b, torch.cuda.current_stream().cuda_stream)
                 for s, d in zip(srcs, dsts)]
        for c in calls:
            assert c() == 0
        mean_us, _ = time_kernel(torch, calls, 8)
        if best is None or mean_us < best[0]:
            best = (mean_us, blocks)
    rw_bytes = rw_read + rw_read // 2
    out["read2_write1"] = {"bytes": rw_bytes, "mean_us": round(best[0], 2), "blocks": best[1],
                           "gbs": round(rw_bytes / (best[0] * 1e-6) / 1e9, 1)}
    del srcs, dsts
    torch.cuda.synchronize()
    return out


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def reference_cpu_rows(torch, x, w, sw):
    """The reference's CPU path for rows `x` [rows, K] of the step, in torch.

    Quantizer: benchmarks/microbench_quantize.py:75-76 (FP32 row max / 127 floored at
    1e-20, then round half to even and clamp to +-127). GEMM: tests/test_cuda_ops.py:596-599
    (INT32 matmul `a.int() @ w.int().T`, then the FP32 epilogue: row scale first, channel
    scale second, rounded to BF16). Returns codes, scales, INT32 products and outputs."""
    scale = (x.float().abs().amax(-1) / 127).clamp_min(1e-20)
    codes = (x.float() / scale[:, None]).round().clamp(-127, 127).to(torch.int8)
    integer = codes.int() @ w.int().T
    out = (integer.float() * scale[:, None] * sw.float()[None, :]).to(torch.bfloat16)
    return {"codes": codes, "scale": scale, "integer": integer, "out": out}


def cpu_baseline(torch, host, budget_s: float) -> tuple[dict, dict]:
    """The reference's own CPU path for the step (reference_cpu_rows) on this host's cores,
    on the same host tensors the GPU step uses. The full 4096-row step takes minutes on a
    CPU, so a leading slice of rows is timed (sized to about `budget_s` seconds) and the rate
    is reported per op, i.e. extrapolated by 4096 / rows to the whole step. Returns the
    baseline record and the slice's results (for the parity check)."""
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    x, w, sw = host["x"], host["w"], host["sw"]

    def run(rows):
        t0 = time.perf_counter()
        ref = reference_cpu_rows(torch, x[:rows], w, sw)
        elapsed = time.perf_counter() - t0
        assert ref["out"].shape == (rows, N)
        return elapsed, ref

    rows = 32
    elapsed, _ = run(rows)
    rows = int(min(M, max(32, rows * budget_s / max(elapsed, 1e-3))))
    elapsed, ref = run(rows)
    tops = 2 * rows * N * K / elapsed / 1e12
    record = {
        "value": round(tops, 5),
        "unit": "TOPS",
        "cores": cores,
        "kind": "port",
        "path": "the reference's torch CPU math, restated here",
        "sample": f"reference torch CPU math (benchmarks/microbench_quantize.py:75-76 quantizer, "
                  f"tests/test_cuda_ops.py:596-599 INT32 matmul + FP32 epilogue) on the first "
                  f"{rows} of {M} rows (K={K}, N={N}) of the GPU step's own inputs, in "
                  f"{elapsed:.2f} s, extrapolated x{M / rows:.2f} to the full step "
                  f"({M / rows * elapsed:.1f} s)",
        "cpu_model": _cpu_model(),
        "torch": torch.__version__,
        "threads": torch.get_num_threads(),
    }
    return record, ref


def parity_record(torch, gpu: dict, ref: dict, fused_equals_cutlass: bool) -> dict:
    """Bit-for-bit comparison of the GPU's leading rows (host copies of codes, row scales,
    INT32 products and BF16 outputs) with the reference's CPU results for the same rows."""
    rows = ref["out"].shape[0]
    checks = {
        "codes": torch.equal(gpu["codes"][:rows], ref["codes"]),
        "row_scales": torch.equal(gpu["scale"][:rows].view(torch.int32),
                                  ref["scale"].view(torch.int32)),
        "int32_products": torch.equal(gpu["integer"][:rows], ref["integer"]),
        "bf16_outputs": torch.equal(gpu["out"][:rows].view(torch.int16),
                                    ref["out"].view(torch.int16)),
        "fused_equals_cutlass": bool(fused_equals_cutlass),
    }
    return {"rows_compared": rows, "of_rows": M, "input_copy": 0,
            "against": "the reference's torch CPU math on the same host tensors",
            **checks, "all_equal": all(checks.values())}


def parity_check(torch, ops, xs, ws, sw, ref) -> dict:
    """One more step on copy 0 of the inputs (untimed): its leading rows against the
    reference's CPU results for the same host tensors (`ref`), bit for bit, and
    fused_channel_mm against cutlass_channel_mm on the same codes over the whole output."""
    rows = ref["out"].shape[0]
    codes = torch.empty(M, K, device="cuda", dtype=torch.int8)
    sa = torch.empty(M, device="cuda", dtype=torch.float32)
    fused = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    cut = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    workspace = torch.empty(M, N, device="cuda", dtype=torch.int32)
    ops.quantize_rows(xs[0], codes, sa)
    ops.fused_channel_mm(codes, ws[0], sa, sw, fused, 0)
    ops.cutlass_channel_mm(codes, ws[0], sa, sw, workspace, cut)
    torch.cuda.synchronize()
    same = torch.equal(fused.view(torch.int16), cut.view(torch.int16))
    gpu = {"codes": codes[:rows].cpu(), "scale": sa[:rows].cpu(),
           "integer": workspace[:rows].cpu(), "out": fused[:rows].cpu()}
    del codes, sa, fused, cut, workspace
    return parity_record(torch, gpu, ref, same)


# The persistent GEMM's MFMA floor per K stage: each SIMD runs two waves, each issuing
# TM x TN x 2 = 4 x 7 x 2 = 56 v_mfma_i32_16x16x64_i8 per stage, and one such MFMA
# (32,768 ops) occupies a SIMD's matrix core for 16 cycles (8,192 ops/clk per CU over 4
# SIMDs): 2 x 56 x 16 = 1,792 cycles.
PP_BM, PP_BN, PP_BK = 256, 224, 128
PP_STAGE_FLOOR_CYCLES = 2 * 4 * 7 * 2 * 16
PHASES = ["memory phase (fragment reads + copies issued)", "wait for W(t+1) (group 1)",
          "barrier 1", "compute phase (56 MFMAs)", "wait for A(t+1) (group 0)", "barrier 2"]
TILE_PHASES = ["tile start (scale copies, zeroing, group 1's offset barrier)",
               "drain (the ping-pong's last phase, barriers)",
               "epilogue (scaling, BF16 packing, LDS-staged stores)",
               "tile switch (wait for the next tile's first copies and this tile's stores, barrier)"]


def phase_profile(torch, ops, xs, ws, sw, codes, sa, out, reps: int = 6) -> tuple[str, bool]:
    """Per-phase cycle table of the persistent GEMM at configs[2] (csrc/probe_pp.hip: the
    library's kernel source with clock stamps). Mode 1 stamps only each workgroup's start
    and end (shader clock and the 100 MHz wall clock); mode 2 also sums each wave's cycles
    per phase kind for wave 0 (copies A) and wave 4 (copies W). Launches rotate over the
    bench's input copies; both modes' last output must equal fused_channel_mm's bit for bit.
    Record layout (pp_gemm_kernel): wave 0's clock start, end, wall start, end; the
    `kinds` sums of wave 0, then of wave 4; wave 4's clock start and end."""
    import ctypes

    lib = ctypes.CDLL(str(REPO / "consumer-int8-kernels_amd" / "consumer_int8" / "libci8_probe.so"))
    lib.ci8probe_pp_gemm_stamped.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [
        ctypes.c_void_p, ctypes.c_void_p]
    shader_khz, wall_khz = ctypes.c_int(0), ctypes.c_int(0)
    assert lib.ci8probe_clock_rates(ctypes.byref(shader_khz), ctypes.byref(wall_khz)) == 0
    grid = lib.ci8probe_pp_grid(M, N)
    words, kinds = lib.ci8probe_pp_stamp_words(), lib.ci8probe_pp_stamp_kinds()
    assert kinds == len(PHASES) + len(TILE_PHASES) and words >= 6 + 2 * kinds
    tiles = -(-M // PP_BM) * -(-N // PP_BN)
    ns = -(-K // PP_BK)
    my_tiles = torch.tensor([(tiles - b + grid - 1) // grid for b in range(grid)], dtype=torch.float64)
    ops.quantize_rows(xs[0], codes[0], sa)
    want = torch.empty_like(out)
    ops.fused_channel_mm(codes[0], ws[0], sa, sw, want, 0)
    record = torch.zeros(reps, grid * words, dtype=torch.int64, device="cuda")

    def stamped(i, mode, rec):
        j = i % len(ws)
        assert lib.ci8probe_pp_gemm_stamped(
            codes[j % len(codes)].data_ptr(), ws[j].data_ptr(), sa.data_ptr(), sw.data_ptr(),
            out.data_ptr(), M, N, K, mode, rec.data_ptr(),
            torch.cuda.current_stream().cuda_stream) == 0

    def product(i):
        j = i % len(ws)
        ops.fused_channel_mm(codes[j % len(codes)], ws[j], sa, sw, out, 0)

    def timed(launch):
        condition(torch, [lambda i=i: launch(i, 0) for i in range(len(ws))], 0.15)
        events = []
        for r in range(reps):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            launch(r, r)
            end.record()
            events.append((start, end))
        torch.cuda.synchronize()
        return statistics.mean(s.elapsed_time(e) * 1e3 for s, e in events)

    kernel_us = {0: timed(lambda i, r: product(i))}
    recs, exact = {}, True
    for mode in (1, 2):
        kernel_us[mode] = timed(lambda i, r, mode=mode: stamped(i, mode, record[r]))
        recs[mode] = record.view(reps, grid, words).cpu().double()
        out.zero_()
        stamped(0, mode, record[0])
        torch.cuda.synchronize()
        exact = exact and torch.equal(out.view(torch.int16), want.view(torch.int16))

    r1 = recs[1]
    cycles = r1[:, :, 1] - r1[:, :, 0]
    mhz = cycles / (r1[:, :, 3] - r1[:, :, 2]) * wall_khz.value / 1e3
    clock = float(mhz.median())
    per_tile = float((cycles / my_tiles).mean())
    floor_tile = ns * PP_STAGE_FLOOR_CYCLES
    r2 = recs[2]
    loop = len(PHASES)
    per_stage = [(r2[:, :, 4 + kinds * g:4 + kinds * g + loop] / (my_tiles * ns)[:, None])
                 .mean(dim=(0, 1)) for g in (0, 1)]
    per_tile2 = [(r2[:, :, 4 + kinds * g + loop:4 + kinds * (g + 1)] / my_tiles[:, None])
                 .mean(dim=(0, 1)) for g in (0, 1)]
    lines = [
        f"configs[2] M={M} K={K} N={N}: {tiles} tiles of {PP_BM}x{PP_BN} on {grid} workgroups "
        f"({tiles / grid:.3f} rounds), {ns} K stages of {PP_BK} per tile.",
        "",
        "| launch | mean us | note |",
        "|---|---|---|",
        f"| library kernel (fused_channel_mm) | {kernel_us[0]:.1f} | no stamps |",
        f"| mode 1 (start/end stamps) | {kernel_us[1]:.1f} | same code plus 4 clock reads per workgroup |",
        f"| mode 2 (per-phase stamps) | {kernel_us[2]:.1f} | 8 clock reads per stage per wave: slower than the kernel it describes |",
        "",
        f"Mode 1: shader clock {clock:.0f} MHz (median over workgroups, cycles / wall-clock "
        f"ticks); {per_tile:,.0f} cycles per tile against the MFMA floor of "
        f"{floor_tile:,} ({ns} x {PP_STAGE_FLOOR_CYCLES}): {floor_tile / per_tile:.3f} of "
        f"the matrix cores' time at that clock.",
        "",
        "Mode 2, cycles per K stage (mean over workgroups and stages; floor "
        f"{PP_STAGE_FLOOR_CYCLES}):",
        "",
        "| phase | wave 0 (group 0, copies A) | wave 4 (group 1, copies W) |",
        "|---|---|---|",
    ]
    for i, name in enumerate(PHASES):
        lines.append(f"| {name} | {per_stage[0][i]:.0f} | {per_stage[1][i]:.0f} |")
    lines.append(f"| **K stage total** | **{per_stage[0].sum():.0f}** | **{per_stage[1].sum():.0f}** |")
    lines += ["", "Mode 2, cycles per tile outside the K loop:", "",
              "| phase | wave 0 | wave 4 |", "|---|---|---|"]
    for i, name in enumerate(TILE_PHASES):
        lines.append(f"| {name} | {per_tile2[0][i]:.0f} | {per_tile2[1][i]:.0f} |")
    total2 = [float(per_stage[g].sum() * ns + per_tile2[g].sum()) for g in (0, 1)]
    lines.append(f"| **tile total (K loop + outside)** | **{total2[0]:,.0f}** | **{total2[1]:,.0f}** |")
    lines += ["", f"Outputs of both stamped modes equal fused_channel_mm's bit for bit: {exact}."]
    return "\n".join(lines), exact


# (N, K) of the reference microbenchmark's linear layers (benchmarks/microbench.py:175-188):
# GDN QKVZ, full-attention QKV, MLP gate/up, MLP down, attention output and MTP fusion, each
# at a two-way pipeline split and a two-way tensor split.
LINEAR_SHAPES = [(16384, 5120), (8192, 5120), (14336, 5120), (7168, 5120), (34816, 5120),
                 (17408, 5120), (5120, 17408), (5120, 8704), (5120, 6144), (5120, 3072),
                 (5120, 10240), (2560, 10240)]


def graph_time_us(torch, call, repeats=7, launches=100) -> dict:
    """Per-call time of `call` as benchmarks/microbench.py:15-38 takes it: five eager calls,
    `launches` calls captured in one graph, `repeats` event-timed replays; median, min and
    max in us."""
    for _ in range(5):
        call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(launches):
            call()
    times = []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) * 1e3 / launches)
    del graph
    return {"median_us": round(statistics.median(times), 3), "min_us": round(min(times), 3),
            "max_us": round(max(times), 3)}


def linear_sweep(torch, ops, args) -> int:
    """The reference microbenchmark's linear mode (benchmarks/microbench.py:172-361) on this
    build's ops, without its vLLM lines (allspark_w8a16_gemm and allspark_repack_weight are
    vLLM's, which this build does not carry). For each (N, K) of LINEAR_SHAPES (or
    --linear-shape) and each row count M (--linear-rows; 1, 2, 4, 16, 256, 1024, or 256 and
    1024 with --prefill-only):
      * --fused-only (microbench.py:205-252): quantize_rows once, then each schedule of
        --fused-schedules, checked bit for bit against schedule 0 before it is timed (and
        here also after its graph replays), timed alone; --fused-paired adds three
        baseline / candidate / baseline triples of schedule 0 against it.
      * otherwise (:254-358): quantize + cutlass_channel_mm into the INT32 workspace and
        quantize + fused_channel_mm (--fused-schedule), checked bit-equal (:298-301) and
        timed, with quantize + channel_mm on the biased UINT8 codes (native_w8a8, not with
        --prefill-only), the AllSpark restore followed by each of the two (M >= 256) and
        channel_gemv (M <= 8).
    Weights are BF16 randn * 0.01 encoded by quantize_channel (the reference's per-channel
    encoder), activations BF16 randn, both from torch's generator seeded as microbench.py:75
    seeds it. The restore lines read random bytes of the packed shape (its packer is vLLM's)
    and write buffers of their own, so they time the same work on other weights. Every row
    is printed and the whole table rewritten to OUTPUT as it grows; a schedule whose output
    differs is recorded with `"exact": false`, not timed, and makes the exit status 1."""
    from consumer_int8.quantization import quantize_channel

    torch.manual_seed(20261011)
    results = {"gpu": torch.cuda.get_device_name(), "torch": torch.__version__,
               "device": {"cus": torch.cuda.get_device_properties(0).multi_processor_count},
               "rows": []}
    shapes = [tuple(s) for s in args.linear_shapes] if args.linear_shapes else LINEAR_SHAPES
    row_counts = args.linear_rows or ((256, 1024) if args.prefill_only else (1, 2, 4, 16, 256, 1024))
    output = Path(args.linear_sweep)
    output.parent.mkdir(parents=True, exist_ok=True)
    failed = False

    def record(row):
        results["rows"].append(row)
        output.write_text(json.dumps(results, indent=2))
        print(json.dumps(row), flush=True)

    def same_bits(x, y):
        return bool(torch.equal(x.view(torch.int16), y.view(torch.int16)))

    for n, k in shapes:
        weight = torch.randn(n, k, device="cuda", dtype=torch.bfloat16) * 0.01
        codes, scale = quantize_channel(weight)
        signed = (codes.to(torch.int16) - 128).to(torch.int8)
        del weight
        padded_n = (n + 31) // 32 * 32
        packed = torch.randint(0, 256, (padded_n, k), device="cuda", dtype=torch.uint8)
        packed_scale = (torch.rand(padded_n, device="cuda") * 1e-3).to(torch.bfloat16)
        restored = torch.empty(n, k, device="cuda", dtype=torch.int8)
        restored_scale = torch.empty(n, device="cuda", dtype=torch.bfloat16)
        for m in row_counts:
            x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
            a = torch.empty_like(x, dtype=torch.int8)
            sa = torch.empty(m, device="cuda")
            out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
            workspace = torch.empty(m, n, device="cuda", dtype=torch.int32)
            if args.fused_only:
                ops.quantize_rows(x, a, sa)
                ops.fused_channel_mm(a, signed, sa, scale, out, 0)
                expected = out.clone()
                for schedule in args.fused_schedules:
                    def call(schedule=schedule):
                        ops.fused_channel_mm(a, signed, sa, scale, out, schedule)

                    call()
                    row = {"op": "fused_channel_mm", "m": m, "n": n, "k": k, "schedule": schedule}
                    if not same_bits(out, expected):
                        failed = True
                        record({**row, "exact": False})
                        continue
                    timing = graph_time_us(torch, call, repeats=5, launches=10)
                    pairs = []
                    if args.fused_paired:
                        def baseline():
                            ops.fused_channel_mm(a, signed, sa, scale, out, 0)

                        for _ in range(3):
                            before = graph_time_us(torch, baseline, 3, 20)["median_us"]
                            candidate = graph_time_us(torch, call, 3, 20)["median_us"]
                            after = graph_time_us(torch, baseline, 3, 20)["median_us"]
                            pairs.append({"before_us": before, "candidate_us": candidate,
                                          "after_us": after,
                                          "speedup": round((before + after) / 2 / candidate, 4)})
                    exact = same_bits(out, expected)
                    failed |= not exact
                    record({**row, "exact": exact, "paired": pairs, **timing,
                            "tflops": round(2 * m * n * k / (timing["median_us"] * 1e6), 2)})
                del expected, x, a, sa, out, workspace
                continue

            def quantized(gemm, *operands):
                ops.quantize_rows(x, a, sa)
                gemm(a, *operands)

            def cutlass():
                quantized(ops.cutlass_channel_mm, signed, sa, scale, workspace, out)

            def fused():
                quantized(ops.fused_channel_mm, signed, sa, scale, out, args.fused_schedule)

            cutlass()
            expected = out.clone()
            fused()
            row = {"op": "linear", "m": m, "n": n, "k": k, "fused_schedule": args.fused_schedule}
            if not same_bits(out, expected):
                failed = True
                record({**row, "fused_matches_separate_exactly": False})
                del expected, x, a, sa, out, workspace
                continue
            if not args.prefill_only:
                row["native_w8a8"] = graph_time_us(
                    torch, lambda: quantized(ops.channel_mm, codes, sa, scale, out))
            row["cutlass_w8a8"] = graph_time_us(torch, cutlass)
            row["fused_w8a8"] = graph_time_us(torch, fused)
            row["fused_matches_separate_exactly"] = same_bits(out, expected)
            failed |= not row["fused_matches_separate_exactly"]
            if m >= 256:
                def restore():
                    ops.unpack_allspark(packed, packed_scale, restored, restored_scale)

                row["unpack_fused_w8a8"] = graph_time_us(torch, lambda: (
                    restore(), quantized(ops.fused_channel_mm, restored, sa, restored_scale,
                                         out, args.fused_schedule)))
                row["unpack_cutlass_w8a8"] = graph_time_us(torch, lambda: (
                    restore(), quantized(ops.cutlass_channel_mm, restored, sa, restored_scale,
                                         workspace, out)))
            if m <= 8:
                row["canonical_gemv_w8a16"] = graph_time_us(
                    torch, lambda: ops.channel_gemv(x, signed, scale, out))
            row["fused_tops"] = round(2 * m * n * k / (row["fused_w8a8"]["median_us"] * 1e6), 2)
            record(row)
            del expected, x, a, sa, out, workspace
        del codes, scale, signed, packed, packed_scale, restored, restored_scale
        torch.cuda.empty_cache()
    return 1 if failed else 0


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (--gpus {args.gpus} requested): this build has "
              "no multi-GPU path; see DESIGN.md for how the op would shard.", file=sys.stderr)
        return 2

    import torch

    from consumer_int8 import ops

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    props = torch.cuda.get_device_properties(0)
    cus = props.multi_processor_count
    peak_tops = PEAK_INT8_TOPS * cus / 256
    if args.linear_sweep:
        return linear_sweep(torch, ops, args)
    host, xs, ws, sw, codes, sa, out = make_inputs(torch)
    if args.phase_profile:
        table, exact = phase_profile(torch, ops, xs, ws, sw, codes, sa, out)
        print(table)
        return 0 if exact else 1
    gen = torch.Generator(device="cuda").manual_seed(20261011)  # the extras' own inputs

    def step(i):
        x, c, w = xs[i % len(xs)], codes[i % len(codes)], ws[i % len(ws)]
        ops.quantize_rows(x, c, sa)
        ops.fused_channel_mm(c, w, sa, sw, out, 0)

    # Conditioning: after idle the chip ramps its clock over tens of milliseconds of load
    # (measured: 412 us per GEMM in steps 0-9 of this loop, 350 us from step ~100 on), so
    # the same step runs untimed for `--condition-seconds` before the warm-up steps.
    conditioning = 0
    t_cond = time.perf_counter() + args.condition_seconds
    while conditioning < 10 or time.perf_counter() < t_cond:
        step(conditioning)
        conditioning += 1
        if conditioning % 10 == 0:
            torch.cuda.synchronize()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # Timed region: exactly K steps between synchronizations; GEMM launches bracketed by
    # events on the current stream (the stream the ops launch on).
    gemm_events = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        x, c, w = xs[i % len(xs)], codes[i % len(codes)], ws[i % len(ws)]
        ops.quantize_rows(x, c, sa)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        ops.fused_channel_mm(c, w, sa, sw, out, 0)
        end.record()
        gemm_events.append((start, end))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    gemm_us = [s.elapsed_time(e) * 1e3 for s, e in gemm_events]
    gemm_mean_us = statistics.mean(gemm_us)
    gemm_tops = GEMM_OPS / (gemm_mean_us * 1e-6) / 1e12
    value = GEMM_OPS / (ms_per_step * 1e-3) / 1e12

    result = {
        "metric": "INT8 TOPS + %MFMA peak, fused_channel_mm M=4096 K=5120 N=17408",
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded on the host, copied to the device): x BF16 N(0,1) with "
                "0.1% channels x50, w INT8 U[-127,127], w_scale BF16 U[1e-3,1e-2]",
        "seeds": {"x": [SEED_X + i for i in range(len(xs))],
                  "w": [SEED_W + i for i in range(len(ws))], "w_scale": SEED_SW,
                  "generator": "torch.Generator() (CPU): randn / randperm / randint / rand"},
        "config": {"workload": "configs[2] prefill projection: quantize_rows BF16[4096,5120] "
                               "+ fused_channel_mm M=4096 K=5120 N=17408",
                   "M": M, "K": K, "N": N, "schedule": 0},
        "pct_mfma_peak": round(100 * value / peak_tops, 2),
        "conditioning": {"steps": conditioning, "seconds": args.condition_seconds},
        "roofline": {
            "kernel": "fused_channel_mm",
            "bound": "mfma",
            "achieved": round(gemm_tops, 2),
            "peak": round(peak_tops, 1),
            "unit": "TFLOP/s",
            "frac": round(gemm_tops / peak_tops, 4),
            "traffic": GEMM_TRAFFIC_BYTES,
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (calibrated by a copy)",
            "mean_us": round(gemm_mean_us, 2),
            "median_us": round(statistics.median(gemm_us), 2),
            "ops_per_launch": GEMM_OPS,
        },
        "device": {"name": props.name, "cus": cus, "gcn_arch": getattr(props, "gcnArchName", "")},
    }
    # Cross-check by the reference microbenchmark's method (benchmarks/microbench.py:15-38):
    # a graph of 10 back-to-back GEMM launches, event-timed per replay, median of 9
    # replays. The weights rotate over 6 copies (5 other launches, ~550 MB, between two
    # uses of one copy), so no launch finds its weights in the 256 MB Infinity Cache.
    ws_g = ws + [torch.randint(-127, 128, (N, K), generator=gen, device="cuda", dtype=torch.int8)
                 for _ in range(6 - len(ws))]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(10):
            ops.fused_channel_mm(codes[i % len(codes)], ws_g[i % len(ws_g)], sa, sw, out, 0)
    graph.replay()
    torch.cuda.synchronize()
    replay_us = []
    for _ in range(9):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        replay_us.append(start.elapsed_time(end) * 1e3 / 10)
    result["roofline"]["graph_median_us"] = round(statistics.median(replay_us), 2)
    del graph, ws_g

    # The nominal peak above assumes 2.4 GHz. The probe measures the clock the chip holds
    # under a full-chip MFMA load and the dense INT8 peak at that clock.
    probe = mfma_clock_probe(torch, cus)
    result["mfma_probe"] = probe
    result["roofline"]["frac_at_measured_clock"] = round(gemm_tops / probe["peak_at_clock_tops"], 4)

    if not args.no_extras:
        extras = {}
        # What a pure stream of the same bytes achieves at these sizes: the practical
        # ceiling for the HBM-bound lines below (their `frac_of_stream`).
        hbm = hbm_stream_probe(torch, cus)
        result["hbm_probe"] = hbm
        # quantize_rows [4096, 5120] on configs[2]'s activations (N(0,1), 0.1% of the
        # channels x50, as in the timed step): rotate 5 (x, codes) pairs = 315 MB > MALL.
        # The kernel's time depends on the data (its bytes do not): plain N(0,1) rows, whose
        # codes fill more of [-127, 127], measured ~10% slower than these on MI355X.
        qx = [device_activations(torch, gen) for _ in range(5)]
        qc = [torch.empty(M, K, device="cuda", dtype=torch.int8) for _ in range(5)]
        calls = [lambda i=i: ops.quantize_rows(qx[i], qc[i], sa) for i in range(5)]
        for c in calls:
            c()
        mean_us, med_us = time_kernel(torch, calls, 10)
        gbs = QUANT_BYTES / (mean_us * 1e-6) / 1e9
        extras["quantize_rows"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                   "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                                   "mean_us": round(mean_us, 2), "bytes": QUANT_BYTES,
                                   "frac_of_stream": round(gbs / hbm["read2_write1"]["gbs"], 4)}
        del qx, qc
        # channel_gemv K=5120, N=17408: rotate 4 weight copies = 356 MB > MALL.
        gw = [torch.randint(-127, 128, (GEMV_N, GEMV_K), generator=gen, device="cuda",
                            dtype=torch.int8) for _ in range(4)]
        gs = (torch.rand(GEMV_N, generator=gen, device="cuda") * 9e-3 + 1e-3).to(torch.bfloat16)
        for m in (1, 4, 8, 16):
            gx = torch.randn(m, GEMV_K, generator=gen, device="cuda").to(torch.bfloat16)
            go = torch.empty(m, GEMV_N, device="cuda", dtype=torch.bfloat16)
            calls = [lambda i=i: ops.channel_gemv(gx, gw[i], gs, go) for i in range(4)]
            for c in calls:
                c()
            mean_us, med_us = time_kernel(torch, calls, 8)
            gbs = gemv_bytes(m) / (mean_us * 1e-6) / 1e9
            extras[f"channel_gemv_m{m}"] = {"bound": "hbm", "achieved": round(gbs, 1),
                                            "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                            "frac": round(gbs / PEAK_HBM_GBS, 4),
                                            "mean_us": round(mean_us, 2), "bytes": gemv_bytes(m),
                                            "frac_of_stream": round(gbs / hbm["read"]["gbs"], 4)}
        del gw, gs
        # grouped W8A8 summed over 4 groups of 4096, M=2048, N=4096 (4 weight
        # copies of 67 MB rotate, more than the MALL holds together with the codes).
        G5, M5, N5, K5 = 4, 2048, 4096, 4096
        c5 = torch.randint(-127, 128, (G5, M5, K5), generator=gen, device="cuda", dtype=torch.int8)
        s5 = torch.rand(G5, M5, generator=gen, device="cuda") / 127
        w5 = [torch.randint(-127, 128, (G5, N5, K5), generator=gen, device="cuda",
                            dtype=torch.int8) for _ in range(4)]
        sw5 = (torch.rand(N5, generator=gen, device="cuda") * 9e-3 + 1e-3).to(torch.bfloat16)
        o5 = torch.empty(M5, N5, device="cuda", dtype=torch.bfloat16)
        calls = [lambda i=i: ops.grouped_summed_mm(c5, w5[i], s5, sw5, o5) for i in range(4)]
        condition(torch, calls)
        mean_us, _ = time_kernel(torch, calls, 4)
        tops = 2 * M5 * N5 * G5 * K5 / (mean_us * 1e-6) / 1e12
        extras["grouped_summed_mm_cfg5"] = {"bound": "mfma", "achieved": round(tops, 1),
                                            "peak": round(peak_tops, 1), "unit": "TFLOP/s",
                                            "frac": round(tops / peak_tops, 4),
                                            "mean_us": round(mean_us, 2),
                                            "ops": 2 * M5 * N5 * G5 * K5}
        del c5, s5, w5, o5
        # down projection M=16384, K=17408, N=5120 with biased UINT8 weights;
        # the activations are SiLU(gate) * up of N(0,1) gate and up, quantized per row
        # (silu_mul_quantize), as configs[3] defines them. (Uniform random codes measured
        # ~2-3% slower: the MFMA-bound kernels' time, too, depends on the data.)
        M4, K4, N4 = 16384, 17408, 5120
        x_glu = torch.randn(M4, 2 * K4, generator=gen, device="cuda").to(torch.bfloat16)
        a4 = torch.empty(M4, K4, device="cuda", dtype=torch.int8)
        s4 = torch.empty(M4, device="cuda")
        ops.silu_mul_quantize(x_glu, a4, s4)
        w4 = [torch.randint(0, 256, (N4, K4), generator=gen, device="cuda", dtype=torch.uint8)
              for _ in range(2)]
        sw4 = (torch.rand(N4, generator=gen, device="cuda") * 9e-3 + 1e-3).to(torch.bfloat16)
        o4 = torch.empty(M4, N4, device="cuda", dtype=torch.bfloat16)
        calls = [lambda i=i: ops.channel_mm(a4, w4[i], s4, sw4, o4) for i in range(2)]
        condition(torch, calls)
        mean_us, _ = time_kernel(torch, calls, 2, batch=4)
        tops = 2 * M4 * N4 * K4 / (mean_us * 1e-6) / 1e12
        extras["channel_mm_cfg4"] = {"bound": "mfma", "achieved": round(tops, 1),
                                     "peak": round(peak_tops, 1), "unit": "TFLOP/s",
                                     "frac": round(tops / peak_tops, 4),
                                     "mean_us": round(mean_us, 2), "ops": 2 * M4 * N4 * K4}
        del a4, s4, w4, o4
        # configs[3]'s activation producer: SwiGLU of BF16 [16384, 2*17408] quantized per
        # row (silu_mul_quantize), and the unquantized silu_mul, both far beyond the MALL.
        cs = torch.empty(M4, K4, device="cuda", dtype=torch.int8)
        ss = torch.empty(M4, device="cuda")
        ops.silu_mul_quantize(x_glu, cs, ss)
        mean_us, _ = time_kernel(torch, [lambda: ops.silu_mul_quantize(x_glu, cs, ss)], 3, batch=4)
        bs = 4 * M4 * K4 + M4 * K4 + 4 * M4
        extras["silu_mul_quantize_cfg4"] = {"bound": "hbm", "achieved": round(bs / (mean_us * 1e-6) / 1e9, 1),
                                            "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                            "frac": round(bs / (mean_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                                            "mean_us": round(mean_us, 2), "bytes": bs}
        del cs, ss
        act = torch.empty(M4, K4, device="cuda", dtype=torch.bfloat16)
        ops.silu_mul(x_glu, act)
        mean_us, _ = time_kernel(torch, [lambda: ops.silu_mul(x_glu, act)], 3, batch=4)
        bs = 4 * M4 * K4 + 2 * M4 * K4
        extras["silu_mul_cfg4"] = {"bound": "hbm", "achieved": round(bs / (mean_us * 1e-6) / 1e9, 1),
                                   "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                   "frac": round(bs / (mean_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                                   "mean_us": round(mean_us, 2), "bytes": bs}
        del x_glu, act
        # unpack_allspark of configs[3]'s weights [5120, 17408]: 3 packed copies rotate
        # (267 MB of input plus the 89 MB output exceed the MALL).
        pk = [torch.randint(0, 256, (N4, K4), generator=gen, device="cuda", dtype=torch.uint8)
              for _ in range(3)]
        pks = torch.randn(N4, generator=gen, device="cuda").to(torch.bfloat16)
        wu = torch.empty(N4, K4, device="cuda", dtype=torch.int8)
        su = torch.empty(N4, device="cuda", dtype=torch.bfloat16)
        calls = [lambda i=i: ops.unpack_allspark(pk[i], pks, wu, su) for i in range(3)]
        for c in calls:
            c()
        mean_us, _ = time_kernel(torch, calls, 6)
        bu = 2 * N4 * K4 + 4 * N4
        extras["unpack_allspark_cfg4"] = {"bound": "hbm", "achieved": round(bu / (mean_us * 1e-6) / 1e9, 1),
                                          "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                          "frac": round(bu / (mean_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                                          "mean_us": round(mean_us, 2), "bytes": bu}
        del pk, pks, wu, su
        # Block-32 Q8_0 W8A8 at the reference harness's largest default shape
        # (benchmarks/benchmark_q8_block_int8.py:45, :253): M=2048, N=1024, K=4096,
        # through the C ABI as that harness calls it. The per-block FP32 rescale (a convert
        # and a multiply-add, 2 VALU instructions per output per block; the scale products
        # run on the MFMA pipe) bounds it, so the VALU fraction is reported beside the
        # MFMA one.
        from consumer_int8 import _abi

        lib = _abi.load()
        MQ, NQ, KQ = 2048, 1024, 4096
        xq = (torch.randn(MQ, KQ, generator=gen, device="cuda") * 0.1).to(torch.bfloat16)
        wq = torch.randint(-128, 128, (NQ, KQ), generator=gen, device="cuda", dtype=torch.int8)
        swq = (torch.randn(NQ, KQ // 32, generator=gen, device="cuda") * 0.01).half()
        aq = torch.empty(MQ, KQ, device="cuda", dtype=torch.int8)
        saq = torch.empty(MQ, KQ // 32, device="cuda")
        yq = torch.empty(MQ, NQ, device="cuda", dtype=torch.bfloat16)
        args_q = [t.data_ptr() for t in (xq, aq, saq, wq, swq, yq)]

        def q8_fused():
            assert lib.ci8_q8_block_int8(*args_q, MQ, NQ, KQ,
                                         torch.cuda.current_stream().cuda_stream) == 0

        def q8_mm():
            assert lib.ci8_q8_block_mm(aq.data_ptr(), saq.data_ptr(), wq.data_ptr(),
                                       swq.data_ptr(), yq.data_ptr(), MQ, NQ, KQ,
                                       torch.cuda.current_stream().cuda_stream) == 0

        q8_fused()
        ops_q = 2 * MQ * NQ * KQ
        valu_peak = cus * 64 * 2.4e9  # lane-instructions per second, 64 lanes/clk/CU
        for name, call in (("q8_block_int8", q8_fused), ("q8_block_mm", q8_mm)):
            mean_us, _ = time_kernel(torch, [call], 8)
            tops = ops_q / (mean_us * 1e-6) / 1e12
            rescale = 2 * MQ * NQ * (KQ // 32) / (mean_us * 1e-6)
            # `frac` is against the dense INT8 MFMA peak; the kernel is bounded by the VALU
            # rescale (2 instructions per output and block), whose share is `valu_frac`.
            extras[name] = {"bound": "valu", "achieved": round(tops, 1), "peak": round(peak_tops, 1),
                            "unit": "TOPS", "frac": round(tops / peak_tops, 4),
                            "valu_frac": round(rescale / valu_peak, 4),
                            "mean_us": round(mean_us, 2), "ops": ops_q}
        del xq, wq, swq, aq, saq, yq
        # GGUF Q8_0 grouped W8A16 (gguf_q8_packed_mm) at N = K = 4096, one group, rows as
        # in the reference harness (benchmarks/benchmark_gguf_q8.py:477): 16 weight copies
        # (285 MB) rotate so that the decode row count streams from HBM; 2048 rows are
        # bounded by the dense BF16 MFMA peak.
        from consumer_int8 import gguf

        NG, KG = 4096, 4096
        gq = [torch.randint(-128, 128, (1, NG, KG), generator=gen, device="cuda", dtype=torch.int8)
              for _ in range(16)]
        gs = (torch.rand(1, NG, KG // 32, generator=gen, device="cuda") * 0.01).half()
        for mg in (16, 2048):
            xg = torch.randn(mg, 1, KG, generator=gen, device="cuda").to(torch.bfloat16)
            og = torch.empty(mg, 1, NG, device="cuda", dtype=torch.bfloat16)
            calls = [lambda i=i: gguf.q8_packed_mm(xg, gq[i], gs, og) for i in range(16)]
            for c in calls:
                c()
            mean_us, _ = time_kernel(torch, calls, 4)
            bg = NG * KG + NG * KG // 16 + 2 * mg * KG + 2 * mg * NG
            fg = 2 * mg * NG * KG
            if mg <= 16:
                gbs = bg / (mean_us * 1e-6) / 1e9
                extras[f"gguf_q8_packed_m{mg}"] = {
                    "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4), "mean_us": round(mean_us, 2), "bytes": bg}
            else:
                tf = fg / (mean_us * 1e-6) / 1e12
                extras[f"gguf_q8_packed_m{mg}"] = {
                    "bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                    "mean_us": round(mean_us, 2), "flops": fg}
            del xg, og
        del gq, gs
        # The vendor library on the headline shape, for reference: torch._int_mm (hipBLASLt's
        # INT8 GEMM, INT32 output, no scale epilogue) on the same codes and weights.
        try:
            calls = [lambda i=i: torch._int_mm(codes[i % len(codes)], ws[i % len(ws)].t())
                     for i in range(len(ws))]
            for c in calls:
                c()
            condition(torch, calls)
            mean_us, _ = time_kernel(torch, calls, 4)
            tops = GEMM_OPS / (mean_us * 1e-6) / 1e12
            extras["vendor_int_mm_cfg3"] = {
                "bound": "mfma", "achieved": round(tops, 1), "peak": round(peak_tops, 1),
                "unit": "TOPS", "frac": round(tops / peak_tops, 4), "mean_us": round(mean_us, 2),
                "library": "torch._int_mm (hipBLASLt), INT32 output"}
        except RuntimeError as error:  # an INT8 GEMM the installed torch does not offer
            extras["vendor_int_mm_cfg3"] = {"error": str(error)[:200]}
        torch.cuda.synchronize()
        # quantize_rows + fused_channel_mm at M=128, K=4096, N=4096; AI 234
        # op/B is below the ridge, so this small case is bounded by HBM (bytes below).
        M1, K1, N1 = 128, 4096, 4096
        x1 = torch.randn(M1, K1, generator=gen, device="cuda").to(torch.bfloat16)
        c1 = torch.empty(M1, K1, device="cuda", dtype=torch.int8)
        s1 = torch.empty(M1, device="cuda")
        w1 = [torch.randint(-127, 128, (N1, K1), generator=gen, device="cuda", dtype=torch.int8)
              for _ in range(16)]
        sw1 = (torch.rand(N1, generator=gen, device="cuda") * 9e-3 + 1e-3).to(torch.bfloat16)
        o1 = torch.empty(M1, N1, device="cuda", dtype=torch.bfloat16)

        def cfg1(i):
            ops.quantize_rows(x1, c1, s1)
            ops.fused_channel_mm(c1, w1[i], s1, sw1, o1, 0)

        calls = [lambda i=i: cfg1(i) for i in range(16)]
        for c in calls:
            c()
        mean_us, _ = time_kernel(torch, calls, 8)
        b1 = 3 * M1 * K1 + 4 * M1 + N1 * K1 + 2 * N1 + 2 * M1 * N1 + M1 * K1 + 4 * M1
        extras["quantize_fused_cfg1"] = {"bound": "hbm", "achieved": round(b1 / (mean_us * 1e-6) / 1e9, 1),
                                         "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                         "frac": round(b1 / (mean_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                                         "mean_us": round(mean_us, 2), "bytes": b1,
                                         "tops": round(2 * M1 * N1 * K1 / (mean_us * 1e-6) / 1e12, 1)}
        del x1, c1, s1, w1, o1
        result["extras"] = extras

    if args.copy_calibration:
        src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["copy_calibration_bytes"] = src.numel()
        del src, dst

    if not args.no_cpu_baseline:
        result["cpu_baseline"], ref = cpu_baseline(torch, host, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
        ref = reference_cpu_rows(torch, host["x"][:64], host["w"], host["sw"])
    result["parity"] = parity_check(torch, ops, xs, ws, sw, ref)

    print(json.dumps(result), flush=True)
    if not result["parity"]["all_equal"]:
        print("bench.py: the GPU output differs from the reference's CPU results "
              f"({result['parity']})", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
