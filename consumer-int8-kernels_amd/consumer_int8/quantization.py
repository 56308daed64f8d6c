"""Checkpoint weight encodings (offline checkpoint preparation).

Same functions, arguments, results and errors as src/consumer_int8/quantization.py of
the reference:
  * channel UINT8 (:22-32, :46-47): biased UINT8 codes (signed code + 128) with one BF16
    scale per output channel, the format channel_mm (and configs[3]'s weights) consume;
  * group32 INT8 (:35-47, :50-51): signed codes with one FP32 scale per 32 input
    channels, the encoding of the vision tower's linear layers.
This is offline weight preparation, not a hot-path op: it runs as torch arithmetic on
whatever device the weights are on, with the same IEEE FP32 operations as the reference
(division and round-half-to-even are correctly rounded on CPU and GPU alike), so an
encoding made on the MI355X is bit-identical to one made on the host.
"""

import torch


def _matrix(weight: torch.Tensor) -> torch.Tensor:
    # src/consumer_int8/quantization.py:13-19
    if weight.ndim != 2 or not weight.is_floating_point() or not weight.numel():
        raise ValueError("Expected a nonempty floating-point weight matrix")
    value = weight.float()
    if not torch.isfinite(value).all():
        raise ValueError("Weight contains non-finite values")
    return value


def _div127(value: torch.Tensor) -> torch.Tensor:
    """value / 127 with IEEE division on every device. The divisor is a 0-dim tensor on
    value's device, not a Python number: torch's GPU kernels turn division by a host
    scalar into a multiplication by its reciprocal, which is not the correctly rounded
    quotient (about 4.6% of quotients differ on the MI355X)."""
    return value / torch.full((), 127.0, dtype=value.dtype, device=value.device)


def quantize_channel(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Encode [N, K] as biased UINT8 codes [N, K] and BF16 scales [N].

    scale = max(amax_row, FP32 tiny) / 127 in FP32; codes = clamp(rne(w / scale), -128,
    127) + 128; the stored scale is the BF16 rounding of the FP32 scale, taken after the
    codes (src/consumer_int8/quantization.py:22-32).
    """
    value = _matrix(weight)
    scale = _div127(value.abs().amax(dim=1).clamp_min(torch.finfo(torch.float32).tiny))
    codes = torch.round(value / scale[:, None]).clamp(-128, 127)
    stored_scale = scale.to(torch.bfloat16)
    if not torch.isfinite(stored_scale).all() or (stored_scale == 0).any():
        raise ValueError("Channel scales are not representable as nonzero BF16")
    return (codes.to(torch.int16) + 128).to(torch.uint8), stored_scale


def quantize_group32(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Encode [N, K] as signed INT8 codes [N, K] and FP32 scales [N, ceil(K / 32)].

    Per block of 32 input channels (the last one zero-padded): scale = amax / 127 in
    FP32, or 1 for an all-zero block; codes = clamp(rne(w / scale), -127, 127)
    (src/consumer_int8/quantization.py:35-47).
    """
    value = _matrix(weight)
    n, k = value.shape
    blocks = -(-k // 32)
    padded = value.new_zeros(n, blocks * 32)
    padded[:, :k] = value
    padded = padded.view(n, blocks, 32)
    scale = _div127(padded.abs().amax(dim=2))
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    codes = torch.round(padded / scale[:, :, None]).clamp(-127, 127).to(torch.int8)
    return codes.view(n, blocks * 32)[:, :k].contiguous(), scale


def dequantize_channel(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """FP32 [N, K] = (codes - 128) * scale[:, None] (src/consumer_int8/quantization.py:46-47)."""
    return (codes.float() - 128) * scale.float()[:, None]


def dequantize_group32(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """FP32 [N, K] = codes * scale of each one's 32-channel block
    (src/consumer_int8/quantization.py:50-51)."""
    k = codes.shape[1]
    return codes.float() * scale.repeat_interleave(32, dim=1)[:, :k]
