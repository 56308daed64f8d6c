"""The bench-only MFMA clock probe library: built, loadable, exporting its entry points.

No kernel is launched here (that needs a GPU); bench.py runs it on the MI355X.
"""

import ctypes

from tests.conftest import PKG

PROBE_PATH = PKG / "consumer_int8" / "libci8_probe.so"


def test_probe_library_exports():
    lib = ctypes.CDLL(str(PROBE_PATH))
    for name in ("ci8probe_mfma_loop", "ci8probe_clock_rates", "ci8probe_mfma_per_round",
                 "ci8probe_ops_per_mfma"):
        assert hasattr(lib, name), name
    lib.ci8probe_ops_per_mfma.restype = ctypes.c_int64
    assert lib.ci8probe_mfma_per_round() == 32
    assert lib.ci8probe_ops_per_mfma() == 16 * 16 * 64 * 2


def test_probe_rejects_bad_launches_before_any_hip_call():
    lib = ctypes.CDLL(str(PROBE_PATH))
    lib.ci8probe_mfma_loop.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    assert lib.ci8probe_mfma_loop(0, 256, ctypes.c_void_p(0x10000), None) != 0
    assert lib.ci8probe_mfma_loop(10, 256, None, None) != 0
