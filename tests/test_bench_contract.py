"""bench.py's command-line contract on the CPU: more than one GPU is refused with a
message and exit status 2 before anything touches a GPU or imports torch."""

import subprocess
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120, cwd=REPO)
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr
    assert proc.stdout == ""


def _bench():
    sys.path.insert(0, str(REPO))
    import bench

    return bench


def test_bench_cpu_reference_is_the_oracle():
    """The CPU math bench.py compares the GPU step with (the reference's torch expressions)
    gives the oracle's codes, scales, INT32 products and BF16 outputs on a small seeded
    case with an outlier column, a zero row and a tie."""
    import numpy as np
    import torch

    from oracle import oracle as O

    bench = _bench()
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((9, 96)) * 2).astype(np.float32)
    x[:, 5] *= 50
    x[3] = 0
    x[4, :2] = [127.0, 0.5]  # scale exactly 1: code of 0.5 is a tie (rounds to 0)
    x[4, 2:] = 0
    x_bits = O.f32_to_bf16(x)
    w = rng.integers(-127, 128, (40, 96)).astype(np.int8)
    sw_bits = O.f32_to_bf16(rng.uniform(1e-3, 1e-2, 40).astype(np.float32))
    as_bf16 = lambda bits: torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    ref = bench.reference_cpu_rows(torch, as_bf16(x_bits), torch.from_numpy(w), as_bf16(sw_bits))
    codes, scales = O.quantize_rows(x_bits)
    assert np.array_equal(ref["codes"].numpy(), codes)
    assert np.array_equal(ref["scale"].numpy().view(np.uint32), scales.view(np.uint32))
    assert np.array_equal(ref["integer"].numpy(), O.int_matmul(codes, w))
    assert np.array_equal(ref["out"].view(torch.int16).numpy().view(np.uint16),
                          O.fused_channel_mm(codes, w, scales, sw_bits))


def test_bench_parity_record_flags_a_planted_difference():
    """parity_record reports every check equal for identical rows, and flags a single
    flipped output bit, a changed code, a changed INT32 product and a fused/cutlass
    disagreement (the mistakes are planted in copies of the reference rows, on the CPU)."""
    import torch

    bench = _bench()
    gen = torch.Generator().manual_seed(1)
    rows = {"codes": torch.randint(-127, 128, (4, 64), generator=gen, dtype=torch.int8),
            "scale": torch.rand(4, generator=gen),
            "integer": torch.randint(-1000, 1000, (4, 8), generator=gen, dtype=torch.int32),
            "out": torch.randn(4, 8, generator=gen).to(torch.bfloat16)}
    gpu = {key: torch.cat([value, value[:1]]) for key, value in rows.items()}  # extra row
    assert bench.parity_record(torch, gpu, rows, True)["all_equal"]
    for key, field in (("out", "bf16_outputs"), ("codes", "codes"),
                       ("integer", "int32_products"), ("scale", "row_scales")):
        bad = {k: v.clone() for k, v in gpu.items()}
        flat = bad[key].view(torch.int16 if key == "out" else bad[key].dtype).view(-1)
        if key == "scale":
            bad[key] = torch.nextafter(bad[key], torch.tensor(2.0))
        else:
            flat[5] ^= 1
        record = bench.parity_record(torch, bad, rows, True)
        assert not record[field] and not record["all_equal"], key
    record = bench.parity_record(torch, gpu, rows, False)
    assert not record["fused_equals_cutlass"] and not record["all_equal"]
