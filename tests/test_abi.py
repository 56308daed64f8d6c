"""CPU checks of the drop-in boundary: the C ABI library and the torch op surface.

No kernel is launched here. Every rejection is exercised through the C ABI with fake
(never dereferenced) pointers, because validation runs before any HIP call.
"""

import ctypes
import re

import pytest

from tests.conftest import HEADER_PATH, LIB_PATH


def declared_functions():
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(ci8_\w+)\s*\(", text, re.M)))


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == sorted([
        "ci8_last_error", "ci8_version", "ci8_quantize_rows", "ci8_quantize_grouped4096",
        "ci8_fused_channel_mm", "ci8_cutlass_channel_mm", "ci8_cutlass_channel_mm_noalloc",
        "ci8_channel_mm",
        "ci8_channel_gemv", "ci8_grouped_summed_mm", "ci8_silu_mul", "ci8_silu_mul_quantize",
        "ci8_unpack_allspark", "ci8_quantize_block32", "ci8_q8_block_mm", "ci8_q8_block_int8",
        "ci8_gguf_q8_packed_mm",
    ])


def test_library_loads_and_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIB_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_ctypes_binding_covers_header(lib):
    from consumer_int8 import _abi

    assert sorted(_abi.SIGNATURES) == declared_functions()
    assert lib.ci8_version().decode().count(".") == 2


FAKE = 0x10000  # 64 KiB-aligned fake device address, never dereferenced


def expect(lib, status, code, text):
    from consumer_int8 import _abi

    assert status == code, (status, _abi.last_error())
    assert text in _abi.last_error()


def test_quantize_rows_rejections(lib):
    from consumer_int8 import _abi as A

    expect(lib, lib.ci8_quantize_rows(FAKE, FAKE, FAKE, 0, 8, None), A.CI8_ERR_GEOMETRY,
           "Expected a nonempty BF16 matrix")
    expect(lib, lib.ci8_quantize_rows(FAKE, FAKE, FAKE, 4, 0, None), A.CI8_ERR_GEOMETRY,
           "nonempty")
    expect(lib, lib.ci8_quantize_rows(FAKE, FAKE, FAKE, 1 << 16, 1 << 16, None),
           A.CI8_ERR_TOO_LARGE, "Matrix too large")
    expect(lib, lib.ci8_quantize_rows(FAKE + 1, FAKE, FAKE, 4, 8, None), A.CI8_ERR_ALIGNMENT,
           "aligned")


def test_grouped_rejections(lib):
    from consumer_int8 import _abi as A

    msg = "Expected BF16 input[M,G,4096], INT8 codes[G,M,4096], FP32 scales[G,M]"
    expect(lib, lib.ci8_quantize_grouped4096(FAKE, FAKE, FAKE, 3, 0, None), A.CI8_ERR_GEOMETRY, msg)
    expect(lib, lib.ci8_quantize_grouped4096(FAKE, FAKE, FAKE, -1, 4, None), A.CI8_ERR_GEOMETRY, msg)
    expect(lib, lib.ci8_quantize_grouped4096(FAKE + 2, 1 << 30, 1 << 31, 3, 4, None),
           A.CI8_ERR_ALIGNMENT, "Grouped quantization requires aligned buffers")
    # codes start inside x (3*4*4096*2 bytes long)
    expect(lib, lib.ci8_quantize_grouped4096(FAKE, FAKE + 4096, 1 << 31, 3, 4, None),
           A.CI8_ERR_OVERLAP, "must not overlap")
    expect(lib, lib.ci8_quantize_grouped4096(1 << 20, 1 << 24, (1 << 24) + 8, 3, 4, None),
           A.CI8_ERR_OVERLAP, "must not overlap")


@pytest.mark.parametrize("m,n,k", [(0, 4, 32), (4, 0, 32), (4, 4, 0), (4, 4, 33), (4, 6, 32),
                                   (4, 4, 65568)])
def test_fused_and_cutlass_geometry_rejections(lib, m, n, k):
    from consumer_int8 import _abi as A

    expect(lib, lib.ci8_fused_channel_mm(FAKE, FAKE, FAKE, FAKE, FAKE, m, n, k, 0, None),
           A.CI8_ERR_GEOMETRY, "Invalid CUTLASS geometry")
    expect(lib, lib.ci8_cutlass_channel_mm(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, m, n, k, None),
           A.CI8_ERR_GEOMETRY, "Invalid CUTLASS geometry")
    expect(lib, lib.ci8_cutlass_channel_mm_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, m, n, k, None),
           A.CI8_ERR_GEOMETRY, "Invalid CUTLASS geometry")


def test_noalloc_scratch_limit_and_alignment(lib):
    """The no-allocation variant refuses m * n beyond its 8,388,608-entry scratch (the
    limit itself is accepted up to the alignment check) and checks alignment like
    cutlass_channel_mm."""
    from consumer_int8 import _abi as A

    f = lib.ci8_cutlass_channel_mm_noalloc
    expect(lib, f(FAKE, FAKE, FAKE, FAKE, FAKE, 2048, 4100, 32, None), A.CI8_ERR_TOO_LARGE,
           "exceeds the library's scratch of 8388608 INT32 accumulators")
    expect(lib, f(FAKE, FAKE, FAKE, FAKE, FAKE, 8192, 1028, 32, None), A.CI8_ERR_TOO_LARGE,
           "exceeds the library's scratch")
    expect(lib, f(FAKE + 8, FAKE, FAKE, FAKE, FAKE, 2048, 4096, 32, None), A.CI8_ERR_ALIGNMENT,
           "cutlass_channel_mm requires aligned buffers")
    expect(lib, f(FAKE, FAKE, FAKE, FAKE, FAKE + 1, 4, 4, 32, None), A.CI8_ERR_ALIGNMENT,
           "aligned")


def test_fused_schedule_alignment_and_size_rejections(lib):
    from consumer_int8 import _abi as A

    for schedule in (-1, 7):
        expect(lib, lib.ci8_fused_channel_mm(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 4, 32, schedule,
                                             None), A.CI8_ERR_SCHEDULE,
               "Invalid fused GEMM schedule")
    expect(lib, lib.ci8_fused_channel_mm(FAKE + 8, FAKE, FAKE, FAKE, FAKE, 4, 4, 32, 0, None),
           A.CI8_ERR_ALIGNMENT, "aligned")
    expect(lib, lib.ci8_fused_channel_mm(FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 16, 4, 1 << 16, 0,
                                         None), A.CI8_ERR_TOO_LARGE, "Matrix too large")


def test_channel_mm_and_gemv_rejections(lib):
    from consumer_int8 import _abi as A

    expect(lib, lib.ci8_channel_mm(FAKE, FAKE, FAKE, FAKE, FAKE, 1, 4, 33, None),
           A.CI8_ERR_GEOMETRY, "Invalid matrix geometry")
    for m, n, k in [(0, 8, 64), (17, 8, 64), (1, 0, 64), (1, 8, 40), (1, 8, 65552)]:
        expect(lib, lib.ci8_channel_gemv(FAKE, FAKE, FAKE, FAKE, m, n, k, None),
               A.CI8_ERR_GEOMETRY, "Unsupported W8A16 GEMV geometry")
    expect(lib, lib.ci8_channel_gemv(FAKE, FAKE + 4, FAKE, FAKE, 1, 8, 64, None),
           A.CI8_ERR_ALIGNMENT, "Unaligned vector inputs")
    expect(lib, lib.ci8_channel_gemv(FAKE + 2, FAKE, FAKE, FAKE, 1, 8, 64, None),
           A.CI8_ERR_ALIGNMENT, "Unaligned vector inputs")


def test_grouped_summed_rejections(lib):
    from consumer_int8 import _abi as A

    msg = "Invalid grouped GEMM geometry"
    for g, m, n, k in [(0, 4, 4, 32), (2, 0, 4, 32), (2, 4, 6, 32), (2, 4, 4, 48),
                       (2, 4, 4, 65568)]:
        expect(lib, lib.ci8_grouped_summed_mm(FAKE, FAKE, FAKE, FAKE, FAKE, g, m, n, k, None),
               A.CI8_ERR_GEOMETRY, msg)
    expect(lib, lib.ci8_grouped_summed_mm(FAKE + 8, FAKE, FAKE, FAKE, FAKE, 2, 4, 4, 32, None),
           A.CI8_ERR_ALIGNMENT, "grouped_summed_mm requires aligned buffers")
    expect(lib, lib.ci8_grouped_summed_mm(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 1 << 16, 4, 1 << 16,
                                          None), A.CI8_ERR_TOO_LARGE, "Matrix too large")


def test_swiglu_rejections(lib):
    """csrc/bindings.cpp:36-40 and :51-59: the two widths, the INT_MAX bound, and the
    quantizing op's 16-byte input and 8-byte code alignment."""
    from consumer_int8 import _abi as A

    for m, k in [(-1, 8704), (4, 4096), (4, 8703), (4, 17409), (1 << 17, 17408)]:
        expect(lib, lib.ci8_silu_mul(FAKE, FAKE, m, k, None), A.CI8_ERR_GEOMETRY,
               "Unsupported SwiGLU shape")
        expect(lib, lib.ci8_silu_mul_quantize(FAKE, FAKE, FAKE, m, k, None),
               A.CI8_ERR_GEOMETRY, "Unsupported SwiGLU quantization shape")
    expect(lib, lib.ci8_silu_mul(FAKE + 1, FAKE, 4, 8704, None), A.CI8_ERR_ALIGNMENT,
           "aligned buffers")
    for x, codes in [(FAKE + 2, FAKE), (FAKE + 8, FAKE), (FAKE, FAKE + 4)]:
        expect(lib, lib.ci8_silu_mul_quantize(x, codes, FAKE, 4, 8704, None),
               A.CI8_ERR_ALIGNMENT, "SwiGLU quantization requires aligned buffers")
    expect(lib, lib.ci8_silu_mul(FAKE, FAKE + 4 * 8704, 4, 8704, None), A.CI8_ERR_OVERLAP,
           "must not overlap")
    expect(lib, lib.ci8_silu_mul_quantize(FAKE, FAKE + (1 << 20), FAKE + 64, 4, 8704, None),
           A.CI8_ERR_OVERLAP, "must not overlap")


def test_unpack_allspark_rejections_cpu(lib):
    """csrc/bindings.cpp:276-284: N % 16, K % 16, K <= 65536, the INT_MAX bound on the
    padded buffer, 4-byte packed and 16-byte weight alignment."""
    from consumer_int8 import _abi as A

    for n, k in [(0, 16), (24, 16), (16, 0), (16, 24), (16, 65552), (1 << 16, 1 << 16)]:
        status = lib.ci8_unpack_allspark(FAKE, FAKE, FAKE, FAKE, n, k, None)
        assert status in (A.CI8_ERR_GEOMETRY, A.CI8_ERR_TOO_LARGE)
    expect(lib, lib.ci8_unpack_allspark(FAKE, FAKE, FAKE, FAKE, 1 << 16, 1 << 16, None),
           A.CI8_ERR_TOO_LARGE, "Weight too large")
    expect(lib, lib.ci8_unpack_allspark(FAKE, FAKE, FAKE, FAKE, 24, 16, None),
           A.CI8_ERR_GEOMETRY, "Expected AllSpark N32K16 weights and channel scales")
    expect(lib, lib.ci8_unpack_allspark(FAKE + 2, FAKE, FAKE << 4, FAKE << 5, 16, 16, None),
           A.CI8_ERR_ALIGNMENT, "Unaligned weights")
    expect(lib, lib.ci8_unpack_allspark(FAKE, FAKE << 6, (FAKE << 4) + 8, FAKE << 5, 16, 16, None),
           A.CI8_ERR_ALIGNMENT, "Unaligned weights")
    expect(lib, lib.ci8_unpack_allspark(FAKE, FAKE << 6, FAKE + 256, FAKE << 5, 16, 16, None),
           A.CI8_ERR_OVERLAP, "must not overlap")


def test_q8_block_rejections(lib):
    """benchmarks/cuda/q8_block_int8.cu:145-146: m, n, k > 0 and k % 32 == 0; plus the
    INT_MAX bound, alignment and overlap."""
    from consumer_int8 import _abi as A

    for m, n, k in [(0, 4, 32), (4, 0, 32), (4, 4, 0), (4, 4, 48), (-1, 4, 32)]:
        expect(lib, lib.ci8_q8_block_int8(FAKE, FAKE << 1, FAKE << 2, FAKE << 3, FAKE << 4,
                                          FAKE << 5, m, n, k, None),
               A.CI8_ERR_GEOMETRY, "Invalid block-32 geometry")
        expect(lib, lib.ci8_q8_block_mm(FAKE, FAKE << 1, FAKE << 2, FAKE << 3, FAKE << 4,
                                        m, n, k, None),
               A.CI8_ERR_GEOMETRY, "Invalid block-32 geometry")
    expect(lib, lib.ci8_quantize_block32(FAKE, FAKE << 1, FAKE << 2, 4, 48, None),
           A.CI8_ERR_GEOMETRY, "Invalid block-32 geometry")
    expect(lib, lib.ci8_q8_block_mm(FAKE, FAKE << 1, FAKE << 2, FAKE << 3, FAKE << 4,
                                    1 << 16, 4, 1 << 16, None),
           A.CI8_ERR_TOO_LARGE, "Matrix too large")
    expect(lib, lib.ci8_q8_block_mm(FAKE + 8, FAKE << 1, FAKE << 2, FAKE << 3, FAKE << 4,
                                    4, 4, 32, None),
           A.CI8_ERR_ALIGNMENT, "aligned buffers")
    expect(lib, lib.ci8_q8_block_mm(FAKE, FAKE << 1, FAKE << 2, FAKE << 3, FAKE + 64,
                                    4, 4, 32, None),
           A.CI8_ERR_OVERLAP, "must not overlap")
    expect(lib, lib.ci8_quantize_block32(FAKE, FAKE + 64, FAKE << 2, 4, 32, None),
           A.CI8_ERR_OVERLAP, "must not overlap")


def test_gguf_q8_packed_rejections(lib):
    """csrc/gguf_bindings.cpp:148-161 in order: shape/strides (K % 64, positive strides),
    grid limits, copy alignment; then an empty output returns without a launch, and an
    output overlapping an input is refused."""
    from consumer_int8 import _abi as A

    def call(x=FAKE, q=FAKE << 1, s=FAKE << 2, out=FAKE << 3, m=4, n=8, k=64, g=2,
             xs=128, xg=64):
        return lib.ci8_gguf_q8_packed_mm(x, q, s, out, m, n, k, g, xs, xg, None)

    shape = "Invalid packed Q8 shape/strides; K must be a multiple of 64"
    for bad in [dict(k=32), dict(k=96), dict(k=0), dict(m=-1), dict(n=-1), dict(g=-1),
                dict(xs=0), dict(xg=-64)]:
        expect(lib, call(**bad), A.CI8_ERR_GEOMETRY, shape)
    for bad in [dict(m=65535 * 32 + 1), dict(g=65536), dict(n=2147483584 + 1)]:
        expect(lib, call(**bad), A.CI8_ERR_TOO_LARGE, "Packed Q8 grid too large")
    for bad in [dict(xs=132), dict(xg=68), dict(x=FAKE + 8), dict(q=(FAKE << 1) + 8),
                dict(s=(FAKE << 2) + 2)]:
        expect(lib, call(**bad), A.CI8_ERR_ALIGNMENT, "Packed Q8 copy alignment violation")
    # checks precede the empty-output return, as in the reference
    expect(lib, call(m=0, k=32), A.CI8_ERR_GEOMETRY, shape)
    for empty in [dict(m=0), dict(n=0), dict(g=0)]:
        assert call(**empty) == A.CI8_OK, A.last_error()
    # extents that would overflow 64-bit offsets
    expect(lib, call(m=65535 * 32, n=2147483584, g=65535), A.CI8_ERR_TOO_LARGE, "too large")
    expect(lib, call(xs=1 << 60, m=64), A.CI8_ERR_TOO_LARGE, "too large")
    for alias in [dict(out=FAKE), dict(out=FAKE << 1), dict(out=FAKE << 2),
                  dict(out=FAKE + 200)]:
        expect(lib, call(**alias), A.CI8_ERR_OVERLAP, "Packed Q8 output must not alias inputs")


def test_torch_surface_matches_reference_schemas():
    import torch

    from consumer_int8 import ops

    expected = {
        "fused_channel_mm": "(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor(a!) out, int schedule=0) -> ()",
        "quantize_rows": "(Tensor input, Tensor(a!) codes, Tensor(b!) scales) -> ()",
        "quantize_grouped4096": "(Tensor input, Tensor(a!) codes, Tensor(b!) scales) -> ()",
        "channel_mm": "(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor(a!) out) -> ()",
        "channel_gemv": "(Tensor x, Tensor w, Tensor scale, Tensor(a!) out) -> ()",
        "cutlass_channel_mm": "(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor(a!) workspace, Tensor(b!) out) -> ()",
        # no reference counterpart (configs[4]'s summed grouped W8A8)
        "grouped_summed_mm": "(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor(a!) out) -> ()",
        "silu_mul": "(Tensor input, Tensor(a!) out) -> ()",
        "silu_mul_quantize": "(Tensor input, Tensor(a!) codes, Tensor(b!) scales) -> ()",
        "unpack_allspark": "(Tensor packed, Tensor packed_scales, Tensor(a!) weight, Tensor(b!) scales) -> ()",
        # csrc/gguf_bindings.cpp:496
        "gguf_q8_packed_mm": "(Tensor x, Tensor codes, Tensor scales, Tensor(a!) out) -> ()",
    }
    from consumer_int8 import gguf

    assert gguf.q8_packed_mm is torch.ops.consumer_int8.gguf_q8_packed_mm
    for name, schema in expected.items():
        handle = getattr(torch.ops.consumer_int8, name)
        if hasattr(ops, name):
            assert getattr(ops, name) is handle
        assert str(handle.default._schema) == f"consumer_int8::{name}{schema}"


def test_no_cpu_fallback():
    """The product path has no CPU implementation: CPU tensors are refused."""
    import torch

    from consumer_int8 import ops

    x = torch.zeros(2, 8, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        ops.quantize_rows(x, torch.empty(2, 8, dtype=torch.int8), torch.empty(2))


def test_fake_tensor_registration():
    """register_fake impls exist (torch.compile / meta tracing of the in-place ops)."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode

    from consumer_int8 import ops

    with FakeTensorMode():
        a = torch.empty(4, 64, dtype=torch.int8)
        w = torch.empty(8, 64, dtype=torch.int8)
        sa = torch.empty(4)
        sw = torch.empty(8, dtype=torch.bfloat16)
        out = torch.empty(4, 8, dtype=torch.bfloat16)
        assert ops.fused_channel_mm(a, w, sa, sw, out, 0) is None
        x = torch.empty(2, 2 * 8704, dtype=torch.bfloat16)
        act = torch.empty(2, 8704, dtype=torch.bfloat16)
        codes = torch.empty(2, 8704, dtype=torch.int8)
        assert ops.silu_mul(x, act) is None
        assert ops.silu_mul_quantize(x, codes, torch.empty(2)) is None
        packed = torch.empty(32, 16, dtype=torch.uint8)
        assert ops.unpack_allspark(packed, torch.empty(32, dtype=torch.bfloat16),
                                   torch.empty(16, 16, dtype=torch.int8),
                                   torch.empty(16, dtype=torch.bfloat16)) is None
        from consumer_int8 import gguf

        assert gguf.q8_packed_mm(torch.empty(3, 2, 64, dtype=torch.bfloat16),
                                 torch.empty(2, 5, 64, dtype=torch.int8),
                                 torch.empty(2, 5, 2, dtype=torch.float16),
                                 torch.empty(3, 2, 5, dtype=torch.bfloat16)) is None
