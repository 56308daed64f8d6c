"""Ahead-of-time operators. Buffers belong to the caller; importing never compiles code.

Same handles and schemas as the reference's operator surface
(src/consumer_int8/ops.py:18-32; schemas csrc/bindings.cpp:594-610), implemented by
hand-written gfx950 kernels in libci8_amd.so and registered for the CUDA dispatch key
(the key PyTorch-ROCm uses for HIP tensors) by the _C module.

quantize_rows(input, codes, scales)
    BF16 [M,K] -> INT8 codes [M,K] and FP32 scales [M]; scale = max(amax/127, 1e-20),
    code = clamp(round_half_even(x/scale), -127, 127).
quantize_grouped4096(input, codes, scales)
    Contiguous BF16 [M,G,4096] -> INT8 [G,M,4096] and FP32 [G,M], each (row, group)
    quantized exactly as quantize_rows. Outputs must not overlap the input or each
    other; M = 0 is supported.
fused_channel_mm(a, w, a_scale, w_scale, out, schedule=0)
    out = bf16((float(a @ w.T) * a_scale[:, None]) * w_scale[None, :]) with exact INT32
    accumulation and no workspace. schedule (0..6) only selects a tiling.
cutlass_channel_mm(a, w, a_scale, w_scale, workspace, out)
    As fused_channel_mm, and stores the INT32 accumulators in workspace.
channel_mm(a, w, a_scale, w_scale, out)
    As fused_channel_mm with biased UINT8 weights (signed code + 128).
channel_gemv(x, w, scale, out)
    W8A16 for 1 <= M <= 16: out = bf16(x @ bf16(w * scale[:, None]).T), FP32 accumulation.
grouped_summed_mm(a, w, a_scale, w_scale, out)
    Grouped W8A8 (no reference op; the summed variant of configs[4]): a INT8 [G,M,K]
    (quantize_grouped4096's codes), w INT8 [G,N,K], a_scale FP32 [G,M], w_scale BF16 [N];
    out = bf16(sum over ascending g of (float(a[g] @ w[g].T) * a_scale[g, :, None])
    * w_scale[None, :]), each term rounded to FP32 and summed in FP32.
silu_mul(input, out)
    SwiGLU: input BF16 [M,2K] = [gate | up], K in {8704, 17408}; out BF16 [M,K] =
    bf16(silu(gate) * up) computed in FP32 (silu(g) = g / (1 + exp(-g))).
silu_mul_quantize(input, codes, scales)
    The silu_mul activations quantized per row exactly as quantize_rows, without
    writing them out: codes INT8 [M,K], scales FP32 [M].
unpack_allspark(packed, packed_scales, weight, scales)
    AllSpark N32K16 UINT8 [ceil(N/32)*32, K] weights and permuted BF16 scales ->
    row-major signed INT8 [N, K] (code = byte - 128) and BF16 [N], losslessly; N % 16 == 0.
"""

import torch

from . import _C  # noqa: F401  (registers torch.ops.consumer_int8.*; fails loudly if unbuilt)

quantize_rows = torch.ops.consumer_int8.quantize_rows
quantize_grouped4096 = torch.ops.consumer_int8.quantize_grouped4096
channel_mm = torch.ops.consumer_int8.channel_mm
channel_gemv = torch.ops.consumer_int8.channel_gemv
cutlass_channel_mm = torch.ops.consumer_int8.cutlass_channel_mm
fused_channel_mm = torch.ops.consumer_int8.fused_channel_mm
grouped_summed_mm = torch.ops.consumer_int8.grouped_summed_mm
silu_mul = torch.ops.consumer_int8.silu_mul
silu_mul_quantize = torch.ops.consumer_int8.silu_mul_quantize
unpack_allspark = torch.ops.consumer_int8.unpack_allspark


@torch.library.register_fake("consumer_int8::fused_channel_mm")
def _fused_channel_mm_fake(a, w, a_scale, w_scale, out, schedule=0):
    return None


@torch.library.register_fake("consumer_int8::quantize_rows")
def _quantize_rows_fake(input, codes, scales):
    return None


@torch.library.register_fake("consumer_int8::quantize_grouped4096")
def _quantize_grouped4096_fake(input, codes, scales):
    return None


@torch.library.register_fake("consumer_int8::channel_mm")
def _channel_mm_fake(a, w, a_scale, w_scale, out):
    return None


@torch.library.register_fake("consumer_int8::channel_gemv")
def _channel_gemv_fake(x, w, scale, out):
    return None


@torch.library.register_fake("consumer_int8::cutlass_channel_mm")
def _cutlass_channel_mm_fake(a, w, a_scale, w_scale, workspace, out):
    return None


@torch.library.register_fake("consumer_int8::grouped_summed_mm")
def _grouped_summed_mm_fake(a, w, a_scale, w_scale, out):
    return None


@torch.library.register_fake("consumer_int8::silu_mul")
def _silu_mul_fake(input, out):
    return None


@torch.library.register_fake("consumer_int8::silu_mul_quantize")
def _silu_mul_quantize_fake(input, codes, scales):
    return None


@torch.library.register_fake("consumer_int8::unpack_allspark")
def _unpack_allspark_fake(packed, packed_scales, weight, scales):
    return None
