"""Pins the oracle's stochastic-rounding hash (the packed Adam moments,
crates/splat-train-render/src/bwd/kernels/geo_moments.rs:54-99, and the SH
step's f16 writes, crates/splat-train/src/quant_kernels.rs:866-894) against
the published function it is, restated here from its definition rather than
from the oracle:

* the seed mix index ^ (step * G) with G = floor(2^32 / phi), the golden-ratio
  word (computed here from phi);
* Chris Wellons' "lowbias32" integer hash (hash-prospector, 2018): x ^= x >> 16;
  x *= 0x7feb352d; x ^= x >> 15; x *= 0x846ca68b; x ^= x >> 16;
* the packed moments take (h >> 16) / 65536 as the log-scale code's offset and
  (h & 0xffff) / 65536 as the magnitude code's; the f16 writes take the top 24
  bits, (h >> 8) / 2^24, as the uniform that picks the upper neighbour when it
  is below (|v| - lo) / (hi - lo).

The GPU kernels are held to the oracle bit for bit, so these fix the kernels'
constants too.
"""
import math

import numpy as np

from oracle import pyoracle as po

M32 = 0xFFFFFFFF


def _golden_word() -> int:
    phi = (1 + math.sqrt(5)) / 2
    return int(math.floor(2 ** 32 / phi))


def _lowbias32(x: int) -> int:
    x &= M32
    x ^= x >> 16
    x = (x * 0x7FEB352D) & M32
    x ^= x >> 15
    x = (x * 0x846CA68B) & M32
    x ^= x >> 16
    return x


def _mix(index: int, step: int) -> int:
    return _lowbias32((index ^ ((step * _golden_word()) & M32)) & M32)


def test_step_multiplier_is_the_golden_ratio_word():
    assert _golden_word() == 0x9E3779B9


def test_mix_hash_is_lowbias32_of_the_golden_ratio_mix():
    rng = np.random.default_rng(3)
    pairs = [(0, 0), (1, 0), (0, 1), (M32, M32), (12345, 678)]
    pairs += [(int(a), int(b)) for a, b in rng.integers(0, 2 ** 32, (2000, 2), dtype=np.uint64)]
    for i, s in pairs:
        assert po.mix_hash(i, s) == _mix(i, s), (i, s)
    # lowbias32 is a bijection: distinct inputs, distinct outputs
    xs = rng.integers(0, 2 ** 32, 4096, dtype=np.uint64)
    assert len({po.mix_hash(int(x), 0) for x in xs}) == len(set(int(x) for x in xs))


def test_packed_moment_offsets_come_from_the_hash_halves():
    """One packed Adam step with beta1 = beta2 = 1/2 (exact in f32) re-encodes
    m1 = m/2 + g/2, v1 = v/2 + g^2/2 with the hash's high half as the
    log-scale offset and its low half as the magnitude offset."""
    rng = np.random.default_rng(4)
    eps = np.float32(1e-8)
    adam = po.OrAdam(0.5, 0.5, 1.0, 1.0, float(eps), 0.0, 0.0, 0)
    moved = 0
    for k in range(3000):
        m0 = np.float32(rng.normal() * 10 ** rng.uniform(-9, -5))
        v0 = np.float32(10 ** rng.uniform(-18, -10))
        word = po.geo_encode(float(m0), float(v0), float(eps))
        g = np.float32(rng.normal() * 10 ** rng.uniform(-9, -5))
        index, seed = int(rng.integers(0, 2 ** 32)), int(rng.integers(0, 2 ** 32))
        _, got = po.adam_packed(0.0, word, index, float(g), 0.0, adam, seed)
        md, vd = (np.float32(x) for x in po.geo_decode(word, float(eps)))
        half = np.float32(0.5)
        m1 = md * half + g * half
        v1 = vd * half + (g * g) * half
        h = _mix(index, seed)
        want = po.geo_pack(float(m1), float(v1), float(eps), (h >> 16) / 65536.0, (h & 0xFFFF) / 65536.0)
        assert got == want, (k, hex(got), hex(want))
        # the offsets matter: rounding both codes down gives another word for most draws
        moved += po.geo_pack(float(m1), float(v1), float(eps), 0.0, 0.0) != want
    assert moved > 1000


def test_f16_writes_round_up_when_the_hash_uniform_is_below_the_fraction():
    rng = np.random.default_rng(5)
    ups = 0
    for k in range(4000):
        v = float(np.float32(rng.uniform(-8.0, 8.0)))
        index, step = int(rng.integers(0, 2 ** 32)), int(rng.integers(0, 2 ** 32))
        got = po.stochastic_half(v, index, step)
        lo = float(np.float16(abs(v)))
        if lo > abs(v):
            lo = float(np.nextafter(np.float16(lo), np.float16(0)))
        hi = float(np.nextafter(np.float16(lo), np.float16(np.inf)))
        if lo == abs(v):
            assert got == v
            continue
        p = np.float32((np.float32(abs(v)) - np.float32(lo)) / (np.float32(hi) - np.float32(lo)))
        u = np.float32(_mix(index, step) >> 8) / np.float32(16777216.0)
        want = hi if u < p else lo
        assert abs(got) == want and (got < 0) == (v < 0), (k, v, got, want)
        ups += want == hi
    assert 1000 < ups < 3000
