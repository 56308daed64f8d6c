"""The checkpoint encoder on the MI355X and the encoded layer through the INT8 ops.

`encode(..., device="cuda")` must write the same shard bytes as the host encoder, and a
channel-UINT8 layer loaded back (debiased for fused_channel_mm, biased for channel_mm)
must give the oracle's bits through silu_mul_quantize -> GEMM, the configs[3] flow.
"""

import hashlib

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_bits, host
from tests.test_checkpoint import LAYOUT, make_snapshot

pytestmark = pytest.mark.gpu


def test_encode_on_gpu_writes_the_host_bytes(ops, tmp_path):
    from consumer_int8.checkpoint import encode

    src = tmp_path / "src"
    make_snapshot(src, seed=3)
    cpu = encode(src, tmp_path / "cpu", source_revision="r", device="cpu")
    gpu = encode(src, tmp_path / "gpu", source_revision="r", device="cuda")
    for shard in LAYOUT:
        a = hashlib.sha256((tmp_path / "cpu" / shard).read_bytes()).hexdigest()
        b = hashlib.sha256((tmp_path / "gpu" / shard).read_bytes()).hexdigest()
        assert a == b == cpu["shards"][shard]["sha256"] == gpu["shards"][shard]["sha256"]
    for name, rec in cpu["tensors"].items():
        if "rmse" in rec:
            assert gpu["tensors"][name]["rmse"] == pytest.approx(rec["rmse"], rel=1e-5)
            assert gpu["tensors"][name]["max_abs_error"] == rec["max_abs_error"]


def test_down_projection_from_an_encoded_checkpoint(ops, tmp_path):
    """configs[3] shapes: a [5120, 17408] down projection encoded on the GPU, loaded
    back, and applied to SwiGLU activations quantized by silu_mul_quantize."""
    from consumer_int8.checkpoint import encode, load_channel_linear

    n, k, m = 5120, 17408, 48
    module = "model.language_model.layers.0.mlp.down_proj"
    layout = {s: dict(e) for s, e in LAYOUT.items()}
    layout["model-00001-of-00002.safetensors"][module + ".weight"] = (n, k)
    src = tmp_path / "src"
    tensors = make_snapshot(src, layout=layout, seed=11)
    encode(src, tmp_path / "dst", source_revision="r", device="cuda")
    w_signed, scale = load_channel_linear(tmp_path / "dst", module, device="cuda")
    w_biased, _ = load_channel_linear(tmp_path / "dst", module, device="cuda", signed=False)

    codes_u8, scale_bits = O.quantize_channel(tensors[module + ".weight"].float().numpy())
    assert np.array_equal(host(w_biased), codes_u8)
    assert np.array_equal(bf16_bits(scale), scale_bits)

    torch.manual_seed(0)
    x = torch.randn(m, 2 * k, device="cuda").to(torch.bfloat16)
    a = torch.empty(m, k, device="cuda", dtype=torch.int8)
    sa = torch.empty(m, device="cuda")
    ops.silu_mul_quantize(x, a, sa)
    fused = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    biased = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.fused_channel_mm(a, w_signed, sa, scale, fused, 0)
    ops.channel_mm(a, w_biased, sa, scale, biased)
    torch.cuda.synchronize()
    assert torch.equal(fused, biased)
    expected = O.channel_mm(host(a), codes_u8, host(sa), scale_bits)
    assert np.array_equal(bf16_bits(fused), expected)
