"""The compositing kernels' G = 2^x (vs_compositing_exp2, the hardware's exp2
instruction) against numpy's float64 exp2 at every f32 input from -0 down to
-128: the table the oracle composites with in the GPU parity tests.  Within
1 ulp wherever the result is a normal float ([-126, 0]); below that, under
2^-126, so opacity x G is under every cutoff and both sides reject the pair.
"""
import numpy as np
import pytest
import torch

import vauss_amd as va
from tests._util import EXP2_COUNT, EXP2_FIRST, device_comp_exp2_table

pytestmark = pytest.mark.gpu


def _bits_to_f32(lo: int, hi: int, step: int = 1) -> np.ndarray:
    return np.arange(lo, hi, step, dtype=np.uint64).astype(np.uint32).view(np.float32)


def test_compositing_exp2_within_one_ulp_everywhere():
    tab = device_comp_exp2_table()
    assert tab.shape == (EXP2_COUNT,) and tab.dtype == np.float32
    chunk = 1 << 26
    worst = 0.0
    for i0 in range(0, EXP2_COUNT, chunk):
        i1 = min(EXP2_COUNT, i0 + chunk)
        x = _bits_to_f32(EXP2_FIRST + i0, EXP2_FIRST + i1)
        got = tab[i0:i1]
        normal = x >= np.float32(-126.0)
        ref = np.exp2(x[normal].astype(np.float64))
        spacing = np.spacing(ref.astype(np.float32)).astype(np.float64)
        err = np.abs(got[normal].astype(np.float64) - ref) / spacing
        worst = max(worst, float(err.max(initial=0.0)))
        low = got[~normal]
        assert ((low >= 0.0) & (low < np.float32(2.0 ** -126))).all()
    print(f"max error {worst:.3f} ulp on [-126, 0]", flush=True)
    assert worst <= 1.0, worst


def test_compositing_exp2_special_values_and_range():
    specials = {0x00000000: 1.0, 0x80000000: 1.0, 0xBF800000: 0.5, 0xC1200000: 2.0 ** -10, 0xFF800000: 0.0}
    for b, want in specials.items():
        got = float(va.compositing_exp2(b, 1).cpu()[0])
        assert got == want, (hex(b), got, want)
    for b in (0x7FC00000, 0xFFC00000):
        assert np.isnan(float(va.compositing_exp2(b, 1).cpu()[0]))
    # beyond the table (x < -128): below 2^-126, as the oracle's exp2n there
    far = va.compositing_exp2(0xC3000001, 0xFF800000 - 0xC3000001).cpu().numpy()
    assert ((far >= 0.0) & (far < np.float32(2.0 ** -126))).all()
    with pytest.raises(va.VsError):
        va.compositing_exp2(0xFFFFFFF0, 32)
    torch.cuda.synchronize()
