"""Channel UINT8 weight encoding (offline checkpoint preparation).

Same functions, arguments, results and errors as src/consumer_int8/quantization.py:22-32
and :46-47 of the reference: biased UINT8 codes (signed code + 128) with one BF16 scale
per output channel, the format channel_mm (and configs[3]'s weights) consume. This is
offline weight preparation, not a hot-path op: it runs as torch arithmetic on whatever
device the weights are on, with the same IEEE FP32 operations as the reference (division
and round-half-to-even are correctly rounded on CPU and GPU alike).
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


def quantize_channel(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Encode [N, K] as biased UINT8 codes [N, K] and BF16 scales [N].

    scale = max(amax_row, FP32 tiny) / 127 in FP32; codes = clamp(rne(w / scale), -128,
    127) + 128; the stored scale is the BF16 rounding of the FP32 scale, taken after the
    codes (src/consumer_int8/quantization.py:22-32).
    """
    value = _matrix(weight)
    scale = value.abs().amax(dim=1).clamp_min(torch.finfo(torch.float32).tiny) / 127.0
    codes = torch.round(value / scale[:, None]).clamp(-128, 127)
    stored_scale = scale.to(torch.bfloat16)
    if not torch.isfinite(stored_scale).all() or (stored_scale == 0).any():
        raise ValueError("Channel scales are not representable as nonzero BF16")
    return (codes.to(torch.int16) + 128).to(torch.uint8), stored_scale


def dequantize_channel(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """FP32 [N, K] = (codes - 128) * scale[:, None] (src/consumer_int8/quantization.py:46-47)."""
    return (codes.float() - 128) * scale.float()[:, None]
