"""CPU oracle for the INT8 linear-layer hot path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the arithmetic of AppMana/consumer-int8-kernels for
quantize_rows, quantize_grouped4096, fused/cutlass_channel_mm, channel_mm, channel_gemv,
the channel weight encoding, the SwiGLU producers silu_mul / silu_mul_quantize, the
AllSpark N32K16 weight layout (unpack_allspark, with its inverse packer), the
block-32 Q8_0 W8A8 path (quantize_block32, q8_block_mm) and the grouped GGUF Q8_0
W8A16 product (gguf_q8_packed_mm, with pack_q8). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and only as the checker (or the timed CPU baseline);
the product path never calls it and has no CPU fallback.

Every function cites the reference file:line it follows. How each one is pinned
(known-answer tests, closed forms, exhaustive and brute-force checks) is in
tests/test_oracle.py; the grouped-and-summed W8A8 closed form (grouped_summed_mm) has
no reference op and is pinned only by its own definition and brute force.

Conventions: BF16 tensors are carried as uint16 bit patterns, so no library rounding
is involved anywhere; FP32 arithmetic is numpy float32 (IEEE-754, round to nearest
even, correctly rounded division).
"""

from __future__ import annotations

import numpy as np

F32_TINY = np.float32(np.finfo(np.float32).tiny)
SCALE_FLOOR = np.float32(1e-20)  # csrc/kernels.cu:27 and :70 (fmaxf(amax / 127.f, 1e-20f))


# ---------------------------------------------------------------- BF16 <-> FP32

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of BF16 bit patterns (uint16) to float32."""
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    """float32 -> BF16 bits with IEEE round-to-nearest-even; NaN stays NaN (quieted).

    This is __float2bfloat16 / cutlass round_to_nearest as used at csrc/gemv.cu:25,
    csrc/kernels.cu:120 and csrc/fused_mm.cu:33-37.
    """
    values = np.asarray(values, dtype=np.float32)
    bits = values.view(np.uint32).astype(np.uint64)
    rounded = (bits + np.uint64(0x7FFF) + ((bits >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    nan = np.isnan(values)
    quiet = ((bits >> np.uint64(16)) | np.uint64(0x0040))
    return np.where(nan, quiet, rounded).astype(np.uint16)


def f64_to_bf16(values: np.ndarray) -> np.ndarray:
    """float64 -> BF16 bits by way of float32 (both steps round to nearest even).

    Mirrors the reference test oracle, which rounds an FP64 result with .bfloat16()
    after it is cast (tests/test_gemv.py:27-29 via torch's double->bfloat16 path).
    """
    return f32_to_bf16(np.asarray(values, dtype=np.float64).astype(np.float32))


# ---------------------------------------------------------------- quantizers

def quantize_rows(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """BF16 [M, K] bits -> (INT8 codes [M, K], FP32 scales [M]).

    csrc/kernels.cu:13-35 (scalar) and :41-86 (vector), which agree:
      amax  = fmaxf-reduction of |x| starting at 0 (NaN ignored)        :16-26, :56-69
      scale = fmaxf(amax / 127.f, 1e-20f)                                :27, :70
      code  = clamp(__float2int_rn(x / scale), -127, 127)               :33, :81-82
    __float2int_rn maps NaN to 0; fl(x/scale) never exceeds 127.0000077 for finite x.
    """
    x = bf16_to_f32(x_bits)
    amax = np.fmax.reduce(np.abs(x), axis=-1, initial=np.float32(0)).astype(np.float32)
    scale = np.fmax(amax / np.float32(127.0), SCALE_FLOOR).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        q = (x / scale[..., None]).astype(np.float32)
    q = np.rint(q)
    q = np.where(np.isnan(q), np.float32(0), q)
    q = np.clip(q, -127, 127).astype(np.int8)
    return q, scale


def quantize_grouped4096(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """BF16 [M, G, 4096] -> (codes [G, M, 4096], scales [G, M]).

    csrc/kernels.cu:46-48 (output row b reads input row (b % M)*G + b / M) and
    :293-298 (M = 0 is a no-op); equal to quantize_rows on x[:, g]
    (tests/test_cuda_ops.py:31-38).
    """
    m, g, k = x_bits.shape
    assert k == 4096
    codes, scales = quantize_rows(np.ascontiguousarray(x_bits.transpose(1, 0, 2)).reshape(g * m, k))
    return codes.reshape(g, m, k), scales.reshape(g, m)


# ---------------------------------------------------------------- SwiGLU

# ln(FLT_MAX): e^x overflows FP32 above this (e^-g for gate g <= -89 in BF16).
EXP_F32_OVERFLOW = float(np.log(np.float64(np.finfo(np.float32).max)))
# Relative error budget of an FP32 evaluation of silu(g) * u before its BF16 rounding:
# exp and reciprocal (or division) each within 2 ULP plus three correctly rounded FP32
# operations stay below 2^-20 (one ULP is at most 2^-23 relative).
SILU_REL = 2.0**-20


def round_bf16_f64(values: np.ndarray) -> np.ndarray:
    """float64 -> nearest BF16 value (ties to even) as float64, in one rounding.

    BF16 has 8 significand bits, exponents down to 2^-126 (subnormal spacing 2^-133)
    and overflows to infinity at (2 - 2^-8) * 2^127. NaN and infinities pass through.
    """
    v = np.asarray(values, dtype=np.float64)
    finite = np.isfinite(v)
    safe = np.where(finite, v, 0.0)
    _, e = np.frexp(safe)
    e = np.maximum(e, -125)
    r = np.ldexp(np.rint(np.ldexp(safe, 8 - e)), e - 8)
    r = np.where(np.abs(r) >= 2.0**128, np.copysign(np.inf, r), r)
    return np.where(finite, r, v)


def silu_mul_exact(x_bits: np.ndarray) -> np.ndarray:
    """SwiGLU of BF16 x [M, 2K] = [gate | up] as float64 values [M, K].

    csrc/silu_quant.cu:27-31 and :69-71: gate = x[:, :K], up = x[:, K:], silu(g) =
    g / (1 + e^-g) and value = silu(g) * up, in FP32, then rounded to BF16. Here the
    value is computed in float64 (exact up to float64 rounding), keeping the one FP32
    effect that moves a result by more than SILU_REL: e^-g overflows FP32 for
    -g > ln(FLT_MAX), and the FP32 quotient g / inf is then -0.
    """
    with np.errstate(over="ignore", invalid="ignore"):
        x = bf16_to_f32(x_bits).astype(np.float64)  # signalling NaNs raise "invalid"
        k = x.shape[-1] // 2
        g, u = x[..., :k], x[..., k:]
        e = np.where(-g > EXP_F32_OVERFLOW, np.inf, np.exp(-g))
        return g / (1.0 + e) * u


def silu_mul(x_bits: np.ndarray) -> np.ndarray:
    """silu_mul (csrc/silu_quant.cu:63-72, :83-88): BF16 bits [M, K], the BF16 value
    nearest the exact SwiGLU."""
    return f32_to_bf16(round_bf16_f64(silu_mul_exact(x_bits)).astype(np.float32))


def silu_mul_bounds(x_bits: np.ndarray, rel: float = SILU_REL) -> tuple[np.ndarray, np.ndarray]:
    """Interval [lo, hi] (float64, per element) holding the BF16 output of any FP32
    evaluation whose pre-rounding value p satisfies |p - v| <= rel*|v| + 2^-126 for the
    exact value v. BF16 rounding is monotonic, so bf16(v - d) <= bf16(p) <= bf16(v + d)
    with d = rel*|v| + 2^-126 (the absolute term admits FP32 subnormal flushing). Where
    v is infinite or NaN the interval is [v, v]. lo == hi except where v lies within d
    of a BF16 rounding midpoint.
    """
    v = silu_mul_exact(x_bits)
    with np.errstate(invalid="ignore"):
        d = rel * np.abs(v) + 2.0**-126
        lo = round_bf16_f64(v - d)
        hi = round_bf16_f64(v + d)
    special = ~np.isfinite(v)
    return np.where(special, v, lo), np.where(special, v, hi)


def within_bounds(got_bits: np.ndarray, lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    """Elementwise: BF16 `got_bits` lies in [lo, hi]; NaN matches NaN."""
    got = bf16_to_f32(got_bits).astype(np.float64)
    both_nan = np.isnan(got) & np.isnan(lo)
    with np.errstate(invalid="ignore"):
        return both_nan | ((got >= lo) & (got <= hi))


def silu_mul_quantize(x_bits: np.ndarray, activations: np.ndarray | None = None):
    """silu_mul_quantize (csrc/silu_quant.cu:10-60): (codes [M, K], scales [M]).

    The BF16 activations are quantized per row with quantize_rows' arithmetic
    (:32-43 max of |value| from 0, :44 scale = max(amax/127, 1e-20), :55-56 code =
    clamp(rne(value/scale), -127, 127)). `activations` (BF16 bits) replaces the
    nearest-BF16 SwiGLU, for checking a producer whose values differ from it only
    within silu_mul_bounds.
    """
    if activations is None:
        activations = silu_mul(x_bits)
    return quantize_rows(activations)


# ---------------------------------------------------------------- W8A8 GEMMs

def int_matmul(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact INT32 accumulators acc[m, n] = sum_k a[m, k] * w[n, k].

    The reference oracle is the CPU integer product a.int() @ w.int().T
    (tests/test_cuda_ops.py:596, :488). Here the same integers are summed in float64
    through BLAS: every product is at most 128*128 = 2^14 in magnitude and every
    partial sum at most K * 2^14 <= 2^30 < 2^53, so each float64 operation is exact
    whatever the summation order, and the result is the exact integer.
    """
    a = np.asarray(a)
    w = np.asarray(w)
    assert a.shape[1] == w.shape[1] and a.shape[1] <= 65536
    acc = a.astype(np.float64) @ w.astype(np.float64).T
    return acc.astype(np.int64).astype(np.int32)


def channel_epilogue(acc: np.ndarray, sa: np.ndarray, sw_bits: np.ndarray) -> np.ndarray:
    """bf16_rn( fl( fl(float_rn(acc) * sa[m]) * float(sw[n]) ) ).

    csrc/fused_mm.cu:24-38 (EVT: accumulator x row scale in FP32, then x channel scale,
    then BF16 round to nearest), csrc/cutlass_mm.cu:35 and csrc/kernels.cu:120 (same
    left-to-right order); the row scale is applied first (README.md:111-113; the
    opposite order is a known mismatch, benchmarks/consumer_arch.py:124-129).
    """
    accf = np.asarray(acc, dtype=np.int32).astype(np.float32)  # int32 -> float32, RNE
    sa = np.asarray(sa, dtype=np.float32)
    swf = bf16_to_f32(sw_bits)
    with np.errstate(over="ignore", invalid="ignore"):
        first = (accf * sa[:, None]).astype(np.float32)
        second = (first * swf[None, :]).astype(np.float32)
    return f32_to_bf16(second)


def fused_channel_mm(a, w, sa, sw_bits) -> np.ndarray:
    """fused_channel_mm (csrc/fused_mm.cu:17-93): BF16 bits [M, N]."""
    return channel_epilogue(int_matmul(a, w), sa, sw_bits)


def cutlass_channel_mm(a, w, sa, sw_bits) -> tuple[np.ndarray, np.ndarray]:
    """cutlass_channel_mm (csrc/cutlass_mm.cu:10-50): (INT32 workspace, BF16 bits)."""
    acc = int_matmul(a, w)
    return acc, channel_epilogue(acc, sa, sw_bits)


def debias(w_u8: np.ndarray) -> np.ndarray:
    """Biased UINT8 -> signed code: u ^ 0x80 == u - 128 (csrc/kernels.cu:107)."""
    return (np.asarray(w_u8, dtype=np.uint8) ^ np.uint8(0x80)).view(np.int8)


def channel_mm(a, w_u8, sa, sw_bits) -> np.ndarray:
    """channel_mm (csrc/kernels.cu:88-122): biased UINT8 weights, same epilogue."""
    return channel_epilogue(int_matmul(a, debias(w_u8)), sa, sw_bits)


def grouped_summed_mm(codes, scales, w, sw_bits) -> np.ndarray:
    """Grouped W8A8 with the per-group partials scaled and summed (no reference op).

    codes INT8 [G, M, Kg], scales FP32 [G, M], w INT8 [G, N, Kg], sw BF16 [N]:
      out[m, n] = bf16_rn( sum_g fl( fl(float_rn(acc_g[m, n]) * sa[g, m]) * float(sw[n]) ) )
    summed over ascending g with FP32 additions. Per-group terms follow the
    fused_channel_mm epilogue; the FP32 sum of scaled INT32 partials follows
    benchmarks/cuda/q8_block_int8.cu:54-55. Parity of this closed form is unpinned by
    the reference (it has no such op).
    """
    g_count = codes.shape[0]
    swf = bf16_to_f32(sw_bits)
    total = None
    for g in range(g_count):
        acc = int_matmul(codes[g], w[g]).astype(np.float32)
        with np.errstate(over="ignore", invalid="ignore"):
            term = ((acc * np.asarray(scales[g], np.float32)[:, None]).astype(np.float32)
                    * swf[None, :]).astype(np.float32)
        total = term if total is None else (total + term).astype(np.float32)
    return f32_to_bf16(total)


# ---------------------------------------------------------------- W8A16 GEMV

def dequantize_bf16(w: np.ndarray, scale_bits: np.ndarray) -> np.ndarray:
    """wq[n, k] = bf16_rn(float(code) * float(scale[n])) as bits (csrc/gemv.cu:25)."""
    prod = (np.asarray(w, dtype=np.int8).astype(np.float32)
            * bf16_to_f32(scale_bits)[:, None]).astype(np.float32)
    return f32_to_bf16(prod)


def channel_gemv(x_bits, w, scale_bits) -> tuple[np.ndarray, np.ndarray]:
    """channel_gemv reference: (BF16 bits [M, N], exact-ish float64 values [M, N]).

    FP64 dot product of the BF16 activations with the BF16-dequantized weights,
    rounded to BF16 -- the reference test oracle (tests/test_gemv.py:26-29) for the
    kernel at csrc/gemv.cu:8-59.
    """
    xf = bf16_to_f32(x_bits).astype(np.float64)
    wq = bf16_to_f32(dequantize_bf16(w, scale_bits)).astype(np.float64)
    exact = xf @ wq.T
    return f64_to_bf16(exact), exact


def gemv_abs_bound(x_bits, w, scale_bits) -> np.ndarray:
    """Worst-case FP32 summation error bound K * 2^-24 * sum_k |x * wq| per output."""
    xf = np.abs(bf16_to_f32(x_bits).astype(np.float64))
    wq = np.abs(bf16_to_f32(dequantize_bf16(w, scale_bits)).astype(np.float64))
    k = xf.shape[1]
    return k * 2.0**-24 * (xf @ wq.T)


def bf16_ulp(values: np.ndarray) -> np.ndarray:
    """Spacing of BF16 numbers at |values| (8 significand bits)."""
    v = np.abs(np.asarray(values, dtype=np.float64))
    exp = np.floor(np.log2(np.where(v > 0, v, 2.0**-126)))
    exp = np.maximum(exp, -126)
    return 2.0 ** (exp - 7)


# ---------------------------------------------------------------- block-32 Q8_0 W8A8

def fma_f32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """fl32(a * b + c) with a single rounding, for float32 inputs (finite results).

    a * b is exact in float64 (48 significant bits); the float64 sum s = fl64(p + c)
    and its exact error e (Knuth's TwoSum) carry a + b*c exactly. Rounding s to float32
    is the correct result unless s is exactly halfway between two float32 values, in
    which case e (if nonzero) decides the side.
    """
    p = np.asarray(a, np.float64) * np.asarray(b, np.float64)
    c = np.asarray(c, np.float64)
    s = p + c
    bp = s - p
    e = (p - (s - bp)) + (c - bp)
    r = s.astype(np.float32)
    up = np.nextafter(r, np.float32(np.inf))
    down = np.nextafter(r, np.float32(-np.inf))
    mid_up = (r.astype(np.float64) + up) / 2
    mid_down = (r.astype(np.float64) + down) / 2
    r = np.where((s == mid_up) & (e > 0), up, r)
    r = np.where((s == mid_down) & (e < 0), down, r)
    return r.astype(np.float32)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    """IEEE binary16 bit patterns (uint16) -> float32, exactly."""
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def quantize_block32(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """BF16 [M, K] -> (INT8 codes [M, K], FP32 scales [M, K/32]).

    benchmarks/cuda/q8_block_int8.cu:11-23: per run of 32 consecutive values, amax by
    fmaxf from |v| (:16-18), s = fmaxf(amax / 127, 1e-20) (:19), code =
    __float2int_rn(v / s) (:20) -- quantize_rows' arithmetic on rows of 32.
    """
    m, k = x_bits.shape
    codes, scales = quantize_rows(np.ascontiguousarray(x_bits).reshape(m * k // 32, 32))
    return codes.reshape(m, k), scales.reshape(m, k // 32)


def q8_block_mm(a: np.ndarray, sa: np.ndarray, w: np.ndarray, sw_bits: np.ndarray) -> np.ndarray:
    """Block-32 W8A8 GEMM: BF16 bits [M, N].

    benchmarks/cuda/q8_block_int8.cu:25-63: for each block b of 32 K values in ascending
    order, acc_b = exact INT32 dot product (:43-46), then
    sum = fma(float(acc_b), fl(sa[m, b] * float(sw[n, b])), sum) (:52-53, the product
    and add contracted as the CUDA compiler does), sum from 0; out = bf16_rn(sum) (:61).
    sw holds FP16 bit patterns.
    """
    m, k = a.shape
    n = w.shape[0]
    total = np.zeros((m, n), np.float32)
    sw = f16_to_f32(sw_bits)
    for b in range(k // 32):
        cols = slice(32 * b, 32 * b + 32)
        acc = (a[:, cols].astype(np.float64) @ w[:, cols].astype(np.float64).T).astype(np.float32)
        scale = (sa[:, b, None].astype(np.float32) * sw[None, :, b]).astype(np.float32)
        total = fma_f32(acc, scale, total)
    return f32_to_bf16(total)


def q8_block_dense_reference(x_bits: np.ndarray, w: np.ndarray, sw_bits: np.ndarray) -> np.ndarray:
    """float64 x @ (w * sw)^T, the unquantized product the reference benchmark compares
    against (benchmarks/benchmark_q8_block_int8.py:112-115)."""
    n, k = w.shape
    dense = w.astype(np.float64).reshape(n, k // 32, 32) * f16_to_f32(sw_bits)[..., None]
    return bf16_to_f32(x_bits).astype(np.float64) @ dense.reshape(n, k).T


# ---------------------------------------------------------------- GGUF grouped Q8 W8A16

def dequantize_q8_0(codes: np.ndarray, scale_bits: np.ndarray) -> np.ndarray:
    """GGUF Q8_0 weights [..., K] as BF16 bits: bf16_rn(float(code) * float(scale)).

    csrc/gguf_q8_packed.cu:208-210: the FP16 scale of each run of 32 codes widened to
    FP32, multiplied by the signed code (exact in FP32: 8 x 11 significant bits) and
    rounded once to BF16 (__floats2bfloat162_rn). scale_bits holds FP16 bit patterns
    [..., K / 32].
    """
    codes = np.asarray(codes, dtype=np.int8)
    *lead, k = codes.shape
    blocks = codes.astype(np.float32).reshape(*lead, k // 32, 32)
    prod = (blocks * f16_to_f32(scale_bits)[..., None]).astype(np.float32)
    return f32_to_bf16(prod.reshape(*lead, k))


def gguf_q8_packed_mm(x_bits, codes, scale_bits) -> tuple[np.ndarray, np.ndarray]:
    """gguf_q8_packed_mm reference: (BF16 bits [M, G, N], float64 values [M, G, N]).

    x [M, G, K] BF16 bits, codes [G, N, K] INT8, scale_bits [G, N, K / 32] FP16 bits.
    out[m, g, :] = x[m, g, :] @ wq[g]^T with wq = dequantize_q8_0(codes, scales): the
    product of csrc/gguf_q8_packed.cu:161-273 (BF16 tensor-core products with FP32
    accumulation, :243, rounded to BF16 at :270), evaluated here in float64 and rounded
    to BF16 -- the reference test's oracle (tests/test_gguf_q8.py:28-59, a float32 bmm of
    the BF16 dense weights). The kernel's FP32 summation order is its own, so parity is
    by tolerance: gguf_q8_abs_bound.
    """
    xf = bf16_to_f32(x_bits).astype(np.float64)
    wq = bf16_to_f32(dequantize_q8_0(codes, scale_bits)).astype(np.float64)
    exact = np.stack([xf[:, g, :] @ wq[g].T for g in range(wq.shape[0])], axis=1)
    return f64_to_bf16(exact), exact


def gguf_q8_abs_bound(x_bits, codes, scale_bits) -> np.ndarray:
    """Worst-case FP32 summation error K * 2^-24 * sum_k |x * wq| per output [M, G, N]."""
    xf = np.abs(bf16_to_f32(x_bits).astype(np.float64))
    wq = np.abs(bf16_to_f32(dequantize_q8_0(codes, scale_bits)).astype(np.float64))
    k = xf.shape[2]
    return k * 2.0**-24 * np.stack([xf[:, g, :] @ wq[g].T for g in range(wq.shape[0])], axis=1)


def pack_q8(raw: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Raw GGUF Q8_0 blocks [G, N, K/32, 34] (2-byte little-endian FP16 scale, then 32
    INT8 codes) -> (codes INT8 [G, N, K], scales FP16 bits [G, N, K/32]), losslessly
    (src/consumer_int8/gguf.py:79-96)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    g, n, blocks, width = raw.shape
    assert width == 34
    scales = raw[..., :2].copy().view("<u2").reshape(g, n, blocks)
    codes = raw[..., 2:].copy().view(np.int8).reshape(g, n, blocks * 32)
    return codes, scales.astype(np.uint16)


# ---------------------------------------------------------------- AllSpark N32K16

def allspark_padded_rows(n: int) -> int:
    """Packed rows of an N32K16 weight: n rounded up to 32 (csrc/bindings.cpp:276)."""
    return (n + 31) // 32 * 32


def allspark_unpack_index(n: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """(byte_index [n, k], scale_index [n]): where weight[row, col] and scale[row] are
    read from the flat packed buffers, restated from csrc/allspark_layout.cu:10-26:

      packed_row = (row / 32) * 8 + row % 8                                   :14
      word       = packed_row * 4k + tile * 64 + ((row % 32) / 16) * 8
                   + ((row % 16) / 8) * 4,  tile = col / 16                   :15-16
      words a, b, c, d at word + 0, 16, 32, 48 bytes                          :17-18
      restored bytes of the tile: a0 a1 b0 b1 c0 c1 d0 d1 a2 a3 b2 b3 c2 c3 d2 d3  :20-23
      scale      = packed_scales[(row / 32) * 32 + (row % 8) * 4 + (row % 32) / 8]   :26
    """
    row = np.arange(n, dtype=np.int64)[:, None]
    col = np.arange(k, dtype=np.int64)[None, :]
    packed_row = (row // 32) * 8 + row % 8
    word = packed_row * 4 * k + (col // 16) * 64 + ((row % 32) // 16) * 8 + ((row % 16) // 8) * 4
    c = col % 16
    # position c of the restored 16 bytes: word (c % 8) // 2 of a, b, c, d; byte half c // 8
    byte = word + ((c % 8) // 2) * 16 + (c // 8) * 2 + c % 2
    r = np.arange(n, dtype=np.int64)
    scale = (r // 32) * 32 + (r % 8) * 4 + (r % 32) // 8
    return byte, scale


def unpack_allspark(packed: np.ndarray, packed_scales: np.ndarray, n: int):
    """unpack_allspark (csrc/allspark_layout.cu:8-35): (INT8 weight [n, k], BF16 scale
    bits [n]) from packed UINT8 [padded_n, k] and BF16 bits [padded_n]; code = byte ^ 0x80
    (:20-23)."""
    k = packed.shape[1]
    byte, scale = allspark_unpack_index(n, k)
    weight = (packed.reshape(-1)[byte] ^ np.uint8(0x80)).view(np.int8)
    return weight, np.asarray(packed_scales)[scale]


def pack_allspark(codes_u8: np.ndarray, scale_bits: np.ndarray, fill: int = 0x80):
    """Forward N32K16 packer: the inverse of unpack_allspark's index map. Biased UINT8
    codes [n, k] and BF16 scale bits [n] -> (packed [padded_n, k], packed scales
    [padded_n]); bytes and scales of padding rows are `fill` and 0 (never read)."""
    n, k = codes_u8.shape
    padded = allspark_padded_rows(n)
    packed = np.full(padded * k, fill, dtype=np.uint8)
    packed_scales = np.zeros(padded, dtype=np.uint16)
    byte, scale = allspark_unpack_index(n, k)
    packed[byte] = codes_u8
    packed_scales[scale] = scale_bits
    return packed.reshape(padded, k), packed_scales


# ---------------------------------------------------------------- weight encoding

def quantize_channel(weight: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[N, K] float -> (biased UINT8 codes [N, K], BF16 scale bits [N]).

    src/consumer_int8/quantization.py:22-32: scale = max(amax_row, FP32 tiny) / 127 in
    FP32; codes = clamp(rne(w / scale), -128, 127) + 128; the stored scale is the BF16
    rounding of the FP32 scale, taken after the codes. Rejects non-finite weights and
    scales that round to zero or infinity in BF16 (:16-17, :30-31).
    """
    value = np.asarray(weight, dtype=np.float32)
    if value.ndim != 2 or value.size == 0:
        raise ValueError("Expected a nonempty floating-point weight matrix")
    if not np.isfinite(value).all():
        raise ValueError("Weight contains non-finite values")
    scale = np.maximum(np.abs(value).max(axis=1), F32_TINY).astype(np.float32)
    scale = (scale / np.float32(127.0)).astype(np.float32)
    codes = np.clip(np.rint((value / scale[:, None]).astype(np.float32)), -128, 127)
    stored = f32_to_bf16(scale)
    stored_f = bf16_to_f32(stored)
    if not np.isfinite(stored_f).all() or (stored_f == 0).any():
        raise ValueError("Channel scales are not representable as nonzero BF16")
    return (codes.astype(np.int16) + 128).astype(np.uint8), stored


def quantize_group32(weight: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[N, K] float -> (INT8 codes [N, K], FP32 scales [N, ceil(K/32)]).

    src/consumer_int8/quantization.py:35-47: blocks of 32 input channels, the last one
    zero-padded (:38); scale = amax_block / 127 in FP32, 1 where that is 0 (:39-40);
    codes = clamp(rne(w / scale), -127, 127) (:41). Rejects non-finite weights (:17-18).
    """
    value = np.asarray(weight, dtype=np.float32)
    if value.ndim != 2 or value.size == 0:
        raise ValueError("Expected a nonempty floating-point weight matrix")
    if not np.isfinite(value).all():
        raise ValueError("Weight contains non-finite values")
    n, k = value.shape
    blocks = -(-k // 32)
    padded = np.zeros((n, blocks * 32), np.float32)
    padded[:, :k] = value
    padded = padded.reshape(n, blocks, 32)
    scale = (np.abs(padded).max(axis=2) / np.float32(127.0)).astype(np.float32)
    scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    codes = np.clip(np.rint((padded / scale[:, :, None]).astype(np.float32)), -127, 127)
    return codes.astype(np.int8).reshape(n, blocks * 32)[:, :k].copy(), scale


def dequantize_group32(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """codes * scale of each 32-channel block in FP32 (src/consumer_int8/quantization.py:50-51)."""
    k = codes.shape[1]
    return (codes.astype(np.float32) * np.repeat(scale, 32, axis=1)[:, :k]).astype(np.float32)


def dequantize_channel(codes_u8: np.ndarray, scale_bits: np.ndarray) -> np.ndarray:
    """(codes - 128) * scale in FP32 (src/consumer_int8/quantization.py:46-47)."""
    return ((np.asarray(codes_u8).astype(np.float32) - np.float32(128))
            * bf16_to_f32(scale_bits)[:, None]).astype(np.float32)
