"""The bench-only MFMA clock probe library: built, loadable, exporting its entry points.

No kernel is launched here (that needs a GPU); bench.py runs it on the MI355X.
"""

import ctypes

from tests.conftest import PKG

PROBE_PATH = PKG / "consumer_int8" / "libci8_probe.so"


def test_probe_library_exports():
    lib = ctypes.CDLL(str(PROBE_PATH))
    for name in ("ci8probe_mfma_loop", "ci8probe_clock_rates", "ci8probe_mfma_per_round",
                 "ci8probe_ops_per_mfma", "ci8probe_pp_gemm_stamped", "ci8probe_pp_grid",
                 "ci8probe_pp_stamp_words", "ci8probe_pp_stamp_kinds"):
        assert hasattr(lib, name), name
    lib.ci8probe_ops_per_mfma.restype = ctypes.c_int64
    assert lib.ci8probe_mfma_per_round() == 32
    assert lib.ci8probe_ops_per_mfma() == 16 * 16 * 64 * 2
    # The stamp record holds wave 0's four times, two waves' phase sums and wave 4's two.
    assert lib.ci8probe_pp_stamp_words() >= 6 + 2 * lib.ci8probe_pp_stamp_kinds()


def test_probe_rejects_bad_launches_before_any_hip_call():
    lib = ctypes.CDLL(str(PROBE_PATH))
    lib.ci8probe_mfma_loop.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    assert lib.ci8probe_mfma_loop(0, 256, ctypes.c_void_p(0x10000), None) != 0
    assert lib.ci8probe_mfma_loop(10, 256, None, None) != 0


def test_stream_probes_export_and_reject_bad_arguments():
    """The HBM stream probes bench.py times (plain read; read 2 / write 1) validate their
    arguments before any HIP call."""
    lib = ctypes.CDLL(str(PROBE_PATH))
    read = lib.ci8probe_stream_read
    read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                     ctypes.c_void_p]
    rw = lib.ci8probe_stream_read2_write1
    rw.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    buf = ctypes.c_void_p(0x10000)
    for fn in (lambda *a: read(*a[:4], 0, a[4]), lambda *a: read(*a[:4], 1, a[4]), rw):
        assert fn(None, 1024, buf, 256, None) != 0          # no source
        assert fn(buf, 1024, None, 256, None) != 0          # no sink / destination
        assert fn(buf, 1000, buf, 256, None) != 0           # not a multiple of 16 bytes
        assert fn(buf, 0, buf, 256, None) != 0              # empty
        assert fn(buf, 1024, buf, 0, None) != 0             # no workgroups
    assert read(buf, 1024, buf, 256, 2, None) != 0          # no such variant
    assert read(buf, 1024, buf, 256, -1, None) != 0


def test_stamped_gemm_rejects_bad_arguments_before_any_hip_call():
    """The clock-stamped persistent GEMM (bench.py --phase-profile) validates pointers,
    alignment, shape and mode before it queries the device."""
    lib = ctypes.CDLL(str(PROBE_PATH))
    fn = lib.ci8probe_pp_gemm_stamped
    fn.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [ctypes.c_void_p] * 2
    p = ctypes.c_void_p(0x10000)
    ok = dict(a=p, w=p, sa=p, sw=p, out=p, m=256, n=224, k=128, mode=1, stamps=p)

    def call(**change):
        args = {**ok, **change}
        return fn(args["a"], args["w"], args["sa"], args["sw"], args["out"], args["m"],
                  args["n"], args["k"], args["mode"], args["stamps"], None)

    assert call(a=None) != 0 and call(stamps=None) != 0
    assert call(mode=0) != 0 and call(mode=3) != 0
    assert call(n=226) != 0 and call(k=100) != 0 and call(m=0) != 0
    assert call(a=ctypes.c_void_p(0x10008)) != 0      # A not 16-byte aligned
    assert call(sw=ctypes.c_void_p(0x10004)) != 0     # channel scales not 8-byte aligned
