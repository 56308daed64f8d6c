"""The clock-stamped build of the persistent GEMM (bench.py --phase-profile) computes the
library kernel's outputs bit for bit, and its stamps are self-consistent.

The stamps are taken on the same code path the library runs (gemm_pp_kernel.h compiled
with stamps), so the per-phase table describes that kernel only if the stamped build
still produces the same outputs; this test checks that, at shapes with a ragged M tile, a
ragged N tile and a K tail, and for both stamp modes.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.conftest import PKG
from tests.helpers import bf16_bits, to_dev

pytestmark = pytest.mark.gpu



def probe():
    lib = ctypes.CDLL(str(PKG / "consumer_int8" / "libci8_probe.so"))
    lib.ci8probe_pp_gemm_stamped.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [
        ctypes.c_void_p] * 2
    return lib


@pytest.mark.parametrize("m,n,k", [(1024, 896, 640), (1100, 900, 608), (2048, 4096, 1024),
                                   (2048, 4096, 128), (1300, 3000, 256)])
@pytest.mark.parametrize("mode", [1, 2])
def test_stamped_kernel_matches_fused_channel_mm(ops, m, n, k, mode):
    rng = np.random.default_rng(m + n + k + mode)
    a = to_dev(rng.integers(-127, 128, (m, k)).astype(np.int8))
    w = to_dev(rng.integers(-127, 128, (n, k)).astype(np.int8))
    sa = to_dev((rng.random(m).astype(np.float32) / np.float32(127)).astype(np.float32))
    sw = to_dev(O.f32_to_bf16(rng.uniform(-1e-2, 1e-2, n).astype(np.float32)))
    want = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ops.fused_channel_mm(a, w, sa, sw, want, 0)
    lib = probe()
    grid = lib.ci8probe_pp_grid(m, n)
    words, kinds = lib.ci8probe_pp_stamp_words(), lib.ci8probe_pp_stamp_kinds()
    assert words >= 6 + 2 * kinds
    tiles = -(-m // 256) * -(-n // 224)
    assert 0 < grid <= tiles
    stamps = torch.zeros(grid * words, dtype=torch.int64, device="cuda")
    out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.ci8probe_pp_gemm_stamped(a.data_ptr(), w.data_ptr(), sa.data_ptr(), sw.data_ptr(),
                                        out.data_ptr(), m, n, k, mode, stamps.data_ptr(),
                                        stream) == 0
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), bf16_bits(want))
    rec = stamps.view(grid, words).cpu()
    start4, end4 = 4 + 2 * kinds, 5 + 2 * kinds
    assert bool((rec[:, 1] > rec[:, 0]).all()) and bool((rec[:, 3] > rec[:, 2]).all())
    assert bool((rec[:, end4] > rec[:, start4]).all()) and bool((rec[:, 6 + 2 * kinds:] == 0).all())
    phases = rec[:, 4:4 + 2 * kinds]
    if mode == 1:
        assert bool((phases == 0).all())
    else:
        # Every phase sum is non-negative, the compute phase of both waves is nonzero, and
        # a wave's sums add up to its own start-to-end time less the cycles between its
        # last stamp and its end-time read: two s_memtime round trips, whose return can
        # queue behind other scalar requests (measured 112-632 cycles per workgroup).
        assert bool((phases >= 0).all())
        assert bool((rec[:, 4 + 3] > 0).all()) and bool((rec[:, 4 + kinds + 3] > 0).all())
        for first, start, end in ((4, 0, 1), (4 + kinds, start4, end4)):
            total = rec[:, first:first + kinds].sum(dim=1)
            span = rec[:, end] - rec[:, start]
            assert bool((total <= span).all() and (total >= span - 1000).all()), (first, total, span)
