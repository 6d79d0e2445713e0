"""Pins the oracle's packed Adam moments and fused update (CPU only).

The reference's geometry/opacity moments (crates/splat-train-render/src/bwd/
kernels/geo_moments.rs) have no golden vectors in the reference's tests, so
the restatement is pinned by what the codec's definition fixes:
  * word 0 decodes to exactly m = v = 0;
  * round-to-nearest decode-then-encode is the identity on words;
  * decode(encode(m, v)) lands within half a code step of (m, v), with the
    step sizes the codec's ranges give (u over [0, 8] in 32767 codes, l over
    [0, 64] in 65535 codes);
  * the stochastic offsets are unbiased: averaging floor(x + k/K) over a
    uniform grid of offsets recovers x;
  * one packed Adam step moves the parameter by the float64 textbook Adam
    step on the decoded moments;
  * the fused update equals the projection VJP followed by per-element Adam
    steps (indices, seeds, per-column learning rates, opacity regulariser).
The integer hash's constants follow the reference source
(geo_moments.rs:58-66); only the GPU-vs-oracle bit parity checks them.
"""
import math

import numpy as np
import pytest

from oracle import pyoracle as po
from vauss_amd import scenes

EPS = 1e-15
U_STEP = 8.0 / 32767.0
L_STEP = 64.0 / 65535.0


def test_zero_word_is_reset_moment():
    assert po.geo_decode(0, EPS) == (0.0, 0.0)
    assert po.geo_encode(0.0, 0.0, EPS) == 0


def test_decode_encode_is_identity_on_words():
    rng = np.random.default_rng(1)
    l_codes = rng.integers(0, 65536, 2000)
    u_codes = rng.integers(0, 32768, 2000)
    signs = rng.integers(0, 2, 2000)
    for lc, uc, sg in zip(l_codes, u_codes, signs):
        w = (int(lc) << 16) | (0x8000 if (sg and uc) else 0) | int(uc)
        m, v = po.geo_decode(w, EPS)
        # growth = e^(l step) is rounded once, so a code may land one step
        # below; round-to-nearest must still give back the word for all but
        # a sliver of codes whose decoded value sits on a rounding boundary.
        assert po.geo_encode(m, v, EPS) == w or abs(po.geo_encode(m, v, EPS) - w) <= 1, hex(w)
    same = sum(po.geo_encode(*po.geo_decode(w, EPS), EPS) == w for w in
               [(int(a) << 16) | int(b) for a, b in zip(l_codes[:500], u_codes[:500])])
    assert same >= 495


@pytest.mark.parametrize("scale", [1e-12, 1e-8, 1e-4, 1.0, 1e3])
def test_round_trip_within_half_a_code(scale):
    rng = np.random.default_rng(2)
    for _ in range(300):
        root = float(scale * rng.uniform(0.01, 10.0))
        v = root * root
        u = float(rng.uniform(-7.5, 7.5))
        m = u * (root + EPS)
        m2, v2 = po.geo_decode(po.geo_encode(m, v, EPS), EPS)
        # l = ln(1 + sqrt(v)/e) is kept to half a step: sqrt(v) + e to a
        # relative e^(step/2) - 1, plus f32 rounding of the decode
        r, r2 = math.sqrt(v) + EPS, math.sqrt(v2) + EPS
        assert abs(r2 / r - 1.0) <= math.expm1(L_STEP / 2) + 1e-6
        # u to half a u step, measured on the stored scale
        assert abs(m2 - m) <= (U_STEP / 2) * r2 * 1.001 + 1e-6 * abs(m)
        assert (m2 < 0) == (m < 0) or m2 == 0.0


def test_codes_clamp_at_their_ranges():
    w = po.geo_encode(1e30, 0.0, EPS)            # |u| far past 8
    assert w & 0x7FFF == 0x7FFF
    w = po.geo_encode(0.0, 1e300 if False else 3.0e38, EPS)   # l past 64
    assert w >> 16 == 0xFFFF
    assert po.geo_encode(-1e-9, 1e-18, EPS) & 0x8000
    assert not po.geo_encode(-0.0, 1e-18, EPS) & 0x8000


def test_stochastic_rounding_is_unbiased():
    # E[floor(x + U)] = x for U uniform on [0, 1): averaging over a uniform
    # grid of K offsets recovers x to 1/K, in both codes.
    K = 256
    root = 3.7e-7
    m = 1.9 * (root + EPS)
    l_exact = math.log1p(root / EPS) * (65535.0 / 64.0)
    lc = [po.geo_pack(m, root * root, EPS, k / K, 0.5) >> 16 for k in range(K)]
    assert abs(np.mean(lc) - l_exact) <= 1.0 / K + 1e-3
    w0 = po.geo_pack(m, root * root, EPS, 0.5, 0.5)
    scale = EPS * math.exp((w0 >> 16) * L_STEP)
    u_exact = m / scale * (32767.0 / 8.0)
    uc = [po.geo_pack(m, root * root, EPS, 0.5, k / K) & 0x7FFF for k in range(K)]
    assert abs(np.mean(uc) - u_exact) <= 1.0 / K + 1e-2


def test_mix_hash_spreads_offsets_uniformly():
    h = np.array([po.mix_hash(i, 7) for i in range(1 << 14)], np.uint64)
    hi = (h >> np.uint64(16)).astype(np.float64) / 65536.0
    lo = (h & np.uint64(0xFFFF)).astype(np.float64) / 65536.0
    for x in (hi, lo):
        counts, _ = np.histogram(x, bins=16, range=(0, 1))
        assert counts.min() > 0.8 * len(x) / 16 and counts.max() < 1.2 * len(x) / 16
    assert len(np.unique(h)) == len(h)
    assert po.mix_hash(0, 0) == 0


def _adam(step=3, lr_opac=0.05, opac_reg=0.0):
    b1, b2 = 0.9, 0.999
    return po.OrAdam(b1, b2, 1.0 / (1.0 - b1 ** step), 1.0 / (1.0 - b2 ** step), EPS, lr_opac, opac_reg, step)


def test_packed_step_matches_float64_adam():
    rng = np.random.default_rng(3)
    a = _adam()
    for _ in range(500):
        root = float(10 ** rng.uniform(-9, -2))
        w = po.geo_encode(float(rng.uniform(-3, 3)) * root, root * root, EPS)
        g = float(rng.normal() * 10 ** rng.uniform(-9, -2))
        lr = float(10 ** rng.uniform(-5, -1))
        p0 = float(np.float32(rng.normal()))
        p1, w1 = po.adam_packed(p0, w, int(rng.integers(0, 1 << 30)), g, lr, a, 3)
        m0, v0 = po.geo_decode(w, EPS)
        m1 = a.beta1 * m0 + (1 - a.beta1) * g
        v1 = a.beta2 * v0 + (1 - a.beta2) * g * g
        step = (m1 * a.inv1) / (math.sqrt(v1 * a.inv2) + EPS) * lr
        assert abs((p0 - p1) - step) <= 2e-5 * abs(step) + 4 * np.spacing(np.float32(abs(p0) + abs(step)))
        # the new word holds (m1, v1) to within one code of each half
        m2, v2 = po.geo_decode(w1, EPS)
        r1, r2 = math.sqrt(v1) + EPS, math.sqrt(v2) + EPS
        assert abs(r2 / r1 - 1.0) <= math.expm1(L_STEP) + 1e-6
        assert abs(m2 - m1) <= U_STEP * r2 * 1.001 + 1e-6 * abs(m1)


def test_fused_update_equals_vjp_then_adam():
    w = scenes.workload("c1", 600)
    cam = w.cameras[0].uniforms(w.img_size)
    sc = w.scene
    f = po.render_forward(cam, w.img_size, sc.transforms, sc.sh_coeffs, sc.raw_opacities, flags=po.FLAG_BWD_INFO)
    img = f.get(po.F_OUT_IMG)
    rng = np.random.default_rng(4)
    v_out = (rng.standard_normal(img.shape) / img[..., 0].size).astype(np.float32)
    vc = f.backward(v_out)["v_combined"]
    n = sc.num_splats
    w_t = rng.integers(0, 1 << 32, (n, 10), dtype=np.uint64).astype(np.uint32) & np.uint32(0x3FFF7FFF)
    w_o = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32) & np.uint32(0x3FFF7FFF)
    lr_scale = np.linspace(1e-4, 1e-2, 10).astype(np.float32)
    a = _adam(step=5, opac_reg=3e-3)
    up = f.project_update(vc, sc.transforms, sc.raw_opacities, w_t, lr_scale, w_o, a)
    pg = f.project_backward(vc)
    gfc = set(f.get(po.F_GLOBAL_FROM_COMPACT).tolist())
    seed_t, seed_o = 5 ^ (10 << 24), 5 ^ (1 << 24)
    for g in rng.choice(n, 80, replace=False):
        for k in range(10):
            p1, w1 = po.adam_packed(float(sc.transforms[g, k]), int(w_t[g, k]), g * 10 + k, float(pg["v_transforms"][g, k]),
                                    float(lr_scale[k]), a, seed_t)
            assert np.float32(p1) == up["transforms"][g, k] and w1 == up["w_t"][g, k]
        sig = 1.0 / (1.0 + math.exp(-float(sc.raw_opacities[g])))
        g_op = float(pg["v_raw_opac"][g]) + 3e-3 * sig * (1 - sig)
        p1, w1 = po.adam_packed(float(sc.raw_opacities[g]), int(w_o[g]), g, g_op, a.lr_opac, a, seed_o)
        assert abs(np.float32(p1) - up["raw_opac"][g]) <= 2 * np.spacing(np.float32(abs(p1)))
        assert w1 == up["w_o"][g]
        row = up["color_dir"][g + 1]
        if g in gfc and vc[g].any():
            np.testing.assert_array_equal(row[:3], vc[g, 5:8])
            assert abs(np.linalg.norm(row[3:]) - 1.0) < 1e-6
            c = 0.2820948 * vc[g, 5:8].astype(np.float64)
            assert abs(up["grad_sq"][g] - (c * c).sum() / 3) <= 1e-6 * (c * c).sum() + 1e-30
            assert up["v_refine"][g] == np.clip(vc[g, 9], 0, 1e32)
        else:
            assert not row.any() and up["grad_sq"][g] == 0 and up["v_refine"][g] == 0
    assert not up["color_dir"][0].any()
