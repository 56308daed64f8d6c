"""consumer_int8.quantization (channel UINT8 weight encoding) against the oracle and the
reference's known answer (tests/test_quantization.py:16-24 of the reference)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O


def check_known_answer(device):
    from consumer_int8.quantization import dequantize_channel, quantize_channel

    weight = torch.tensor([[0.0, -127.0, 63.5, 127.0], [0.0, 0.0, 0.0, 0.0]], device=device)
    codes, scale = quantize_channel(weight)
    assert codes.dtype == torch.uint8 and scale.dtype == torch.bfloat16
    assert codes.tolist() == [[128, 1, 192, 255], [128, 128, 128, 128]]
    assert scale[0] == 1
    assert torch.isfinite(dequantize_channel(codes, scale)).all()
    assert torch.equal(dequantize_channel(codes, scale)[1], weight[1])


def check_matches_oracle(device):
    from consumer_int8.quantization import quantize_channel

    rng = np.random.default_rng(22)
    w = rng.standard_normal((64, 300)).astype(np.float32) * np.float32(0.02)
    w[3] = 0
    w[5, :] = np.float32(1e-30)  # tiny rows: scale hits the FP32 tiny floor
    codes, scale = quantize_channel(torch.from_numpy(w).to(device))
    o_codes, o_scale = O.quantize_channel(w)
    assert np.array_equal(codes.cpu().numpy(), o_codes)
    assert np.array_equal(scale.view(torch.int16).cpu().numpy().view(np.uint16), o_scale)


def test_quantize_channel_known_answer_cpu():
    check_known_answer("cpu")


def test_quantize_channel_matches_oracle_cpu():
    check_matches_oracle("cpu")


def test_quantize_channel_rejections():
    from consumer_int8.quantization import quantize_channel

    with pytest.raises(ValueError, match="nonempty floating-point"):
        quantize_channel(torch.zeros(4, dtype=torch.float32))
    with pytest.raises(ValueError, match="nonempty floating-point"):
        quantize_channel(torch.zeros(2, 3, dtype=torch.int32))
    with pytest.raises(ValueError, match="non-finite"):
        quantize_channel(torch.tensor([[1.0, float("inf")]]))


def scale_sensitive_weights():
    """Rows whose maximum A gives fl(A / 127) != fl(A * fl(1 / 127)), filled with values
    midway between (c + 0.5) times either scale: they round to different codes under the
    two scales, so only the correctly rounded scale reproduces the oracle's codes.
    Returns (weights, codes under the reciprocal scale)."""
    rng = np.random.default_rng(5)
    amax = (rng.random(20000) * 10 + 0.1).astype(np.float32)
    ieee = (amax / np.float32(127)).astype(np.float32)
    recip = (amax * (np.float32(1) / np.float32(127))).astype(np.float32)
    pick = np.flatnonzero(ieee != recip)[:512]
    assert pick.size == 512
    c = np.arange(1, 126, dtype=np.float64) + 0.5
    mid = (ieee[pick, None].astype(np.float64) + recip[pick, None]) / 2 * c[None, :]
    w = np.concatenate([amax[pick, None], mid.astype(np.float32)], axis=1)
    wrong = np.clip(np.rint((w / recip[pick, None]).astype(np.float32)), -128, 127) + 128
    return w, wrong.astype(np.uint8)


def test_scale_sensitive_weights_separate_the_two_scales():
    w, wrong = scale_sensitive_weights()
    o_codes, _ = O.quantize_channel(w)
    assert (wrong != o_codes).sum() > 1000


@pytest.mark.gpu
def test_quantize_channel_on_gpu(ops):
    """Includes rows where a scale quotient off by one ULP changes the codes: torch's GPU
    division by a host scalar is a reciprocal multiplication, off in about 5% of rows."""
    from consumer_int8.quantization import quantize_channel

    check_known_answer("cuda")
    check_matches_oracle("cuda")
    w, _ = scale_sensitive_weights()
    codes, scale = quantize_channel(torch.from_numpy(w).to("cuda"))
    o_codes, o_scale = O.quantize_channel(w)
    assert np.array_equal(codes.cpu().numpy(), o_codes)
    assert np.array_equal(scale.view(torch.int16).cpu().numpy().view(np.uint16), o_scale)
