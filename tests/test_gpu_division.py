"""The raster kernels' refined quotient a / b (vs_raster_division): the
hardware reciprocal refined by a Newton step and a remainder correction for
2^-100 <= |b| <= 2^100, the division elsewhere.  The surfel backward replays
the forward's ray-plane sample with it (1 / q.z) while the forward and the
oracle divide, so the replay's agreement with the forward rests on these
being the IEEE quotients (a = 1; a = 0.2 is checked as well):

* on the device, at every one of the 2^32 divisor bit patterns, against the
  kernels' own division (vs_raster_division_mismatches);
* against numpy's float32 division (IEEE, round to nearest even) on a random
  sample of bit patterns, every power of two, the range ends and their
  neighbours, zeros, subnormals, infinities and NaNs.
"""
import numpy as np
import pytest
import torch

import vauss_amd as va

pytestmark = pytest.mark.gpu

NUMERATORS = (1.0, 0.2)


@pytest.mark.parametrize("a", NUMERATORS)
def test_quotient_matches_the_division_at_every_divisor(a):
    print(f"[case] raster division, all 2^32 divisors, a={a}", flush=True)
    assert va.raster_division_mismatches(a) == 0


def _sample_bits(seed: int = 11) -> np.ndarray:
    rng = np.random.default_rng(seed)
    rand = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    pow2 = np.arange(0, 255, dtype=np.uint32) << np.uint32(23)               # +2^e, and +0 at e = 0
    ends = np.array([0x0D800000, 0x71800000], dtype=np.uint32)               # 2^-100, 2^100
    near = (ends[:, None].astype(np.int64) + np.arange(-3, 4)[None, :]).ravel().astype(np.uint32)
    special = np.array([0x00000000, 0x00000001, 0x007FFFFF, 0x00800000, 0x7F7FFFFF, 0x7F800000, 0x7FC00000,
                        0x7F800001, 0x3F800000, 0x3F800001, 0x3F7FFFFF, 0x3E4CCCCD], dtype=np.uint32)
    pos = np.concatenate([rand, pow2, near, special])
    return np.concatenate([pos, pos | np.uint32(0x80000000)])


@pytest.mark.parametrize("a", NUMERATORS)
def test_quotient_matches_numpy_division_on_a_sample(a):
    bits = _sample_bits()
    print(f"[case] raster division sample n={bits.size} a={a}", flush=True)
    got = va.raster_division(a, torch.from_numpy(bits.view(np.int32)).cuda()).cpu().numpy()
    with np.errstate(all="ignore"):
        want = np.float32(a) / bits.view(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    bad = np.nonzero(~same)[0]
    assert bad.size == 0, (f"{bad.size} quotients differ, first at b bits {bits[bad[0]]:#010x}: "
                           f"{got[bad[0]]!r} vs {want[bad[0]]!r}")
