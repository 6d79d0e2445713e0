"""Pins the oracle's scalar math against what mathematics fixes, independently of
the oracle's own formulas:

* exp / exp2n / log / atan2 against numpy's float64 functions (error in f32
  ulps) and the C99 special values;
* the real spherical-harmonic basis (kernels/sh.rs:8-140, Sloan's
  convention) against scipy's complex spherical harmonics, and its
  orthonormality over the sphere by Gauss-Legendre quadrature;
* the L1 cotangent's closed form against central differences of the loss.
"""
import numpy as np
import pytest
import scipy.special as sp

from oracle import pyoracle as po
from tests._util import l1_cotangent_np


def _ulp_err(got, ref64):
    ref32 = ref64.astype(np.float32)
    spacing = np.spacing(np.abs(ref32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - ref64) / spacing


def test_expf_within_one_ulp():
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.uniform(-87.3, 88.7, 1_000_000), rng.uniform(-1, 1, 200_000),
                        rng.uniform(-1e-3, 1e-3, 50_000)]).astype(np.float32)
    err = _ulp_err(po.expf(x), np.exp(x.astype(np.float64)))
    assert err.max() <= 1.0, err.max()


def test_expf_special_values():
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -87.33655, -100.0, 88.8, 1.0], np.float32)
    y = po.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == np.inf and y[3] == 0.0 and np.isnan(y[4])
    assert y[5] == 0.0 and y[6] == 0.0          # flushed below -87.33654: results are never subnormal
    assert y[7] == np.inf
    assert abs(float(y[8]) - np.e) <= np.spacing(np.float32(np.e))


def test_exp2n_within_2_1_ulp():
    """The compositing exp (2^x of -sigma in base-2 units) against numpy's
    float64 exp2: <= 2.1 ulp on [-126, 0] (the contributing pairs' sigma lies in
    [0, 8]), every grid point of 2^-12 on [-12, 0] included."""
    rng = np.random.default_rng(21)
    x = np.concatenate([rng.uniform(-126.0, 0.0, 1_000_000), rng.uniform(-12.0, 0.0, 1_000_000),
                        -np.arange(0.0, 12.0, 2.0 ** -12), rng.uniform(-1e-3, 0.0, 50_000)]).astype(np.float32)
    err = _ulp_err(po.exp2n(x), np.exp2(x.astype(np.float64)))
    assert err.max() <= 2.1, err.max()
    # e^-sigma through the base-2 conic: exp2n(-sigma log2 e) within 1e-6 relative of
    # float64 e^-sigma on the live range (the conic's own rounding adds an ulp of sigma)
    sig = rng.uniform(0.0, 6.0, 200_000).astype(np.float32)
    g = po.exp2n(-(sig * np.float32(1.44269502)))
    np.testing.assert_allclose(g, np.exp(-sig.astype(np.float64)), rtol=1e-6, atol=0)


def test_exp2n_special_values():
    x = np.array([0.0, -0.0, -1.0, -10.0, -np.inf, np.nan, -1e30, -127.0, -200.0, 1.0, 5.0, 1e30, np.inf],
                 np.float32)
    y = po.exp2n(x)
    assert y[0] == 1.0 and y[1] == 1.0 and y[2] == 0.5 and y[3] == np.float32(2.0 ** -10)
    # arguments below -127 (and NaN) clamp to -127: 2^-127, a subnormal, never above the cutoffs
    assert (y[4:9] == np.float32(2.0 ** -127)).all()
    assert y[9] == 2.0 and y[10] == 32.0 and y[11] == np.inf and y[12] == np.inf


def test_logf_within_two_ulp():
    rng = np.random.default_rng(12)
    bits = rng.integers(1, 0x7F800000, 1_000_000, dtype=np.uint32)   # every positive finite binade, subnormals too
    x = np.concatenate([bits.view(np.float32), rng.uniform(0.5, 2.0, 300_000).astype(np.float32)])
    err = _ulp_err(po.logf(x), np.log(x.astype(np.float64)))
    assert err.max() <= 2.0, err.max()


def test_logf_special_values():
    y = po.logf(np.array([1.0, 0.0, -0.0, -1.0, np.inf, np.nan, 2.0], np.float32))
    assert y[0] == 0.0
    assert y[1] == -np.inf and y[2] == -np.inf
    assert np.isnan(y[3]) and np.isnan(y[5])
    assert y[4] == np.inf
    assert abs(float(y[6]) - np.log(2.0)) <= np.spacing(np.float32(np.log(2.0)))


def test_atan2f_within_three_ulp():
    rng = np.random.default_rng(13)
    n = 1_000_000
    a = (rng.standard_normal(n) * np.exp(rng.uniform(-10, 10, n))).astype(np.float32)
    b = (rng.standard_normal(n) * np.exp(rng.uniform(-10, 10, n))).astype(np.float32)
    got = po.atan2f(a, b)
    ref = np.arctan2(a.astype(np.float64), b.astype(np.float64))
    assert _ulp_err(got, ref).max() <= 3.0
    assert np.abs(got - ref).max() <= 4e-7


def test_atan2f_special_values():
    inf = np.inf
    ys = np.array([0.0, -0.0, 0.0, -0.0, 1.0, -1.0, inf, inf, -inf, 1.0, 1.0, 0.0, 3.0], np.float32)
    xs = np.array([0.0, 0.0, -0.0, -0.0, 0.0, 0.0, inf, -inf, 1.0, inf, -inf, 1.0, np.nan], np.float32)
    got = po.atan2f(ys, xs)
    ref = np.arctan2(ys.astype(np.float64), xs.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(np.signbit(got[:12]), np.signbit(ref[:12]))   # signed zeros and pi
    np.testing.assert_allclose(got[:12], ref[:12], rtol=0, atol=3e-7)
    assert np.isnan(got[12])


def _real_sh(l, m, v):
    """Real orthonormal SH with the Condon-Shortley phase, from scipy's complex ones."""
    x, y, z = v
    theta = np.arccos(np.clip(z, -1, 1))
    phi = np.arctan2(y, x)
    if m == 0:
        return sp.sph_harm_y(l, 0, theta, phi).real
    c = sp.sph_harm_y(l, abs(m), theta, phi)
    return np.sqrt(2.0) * (-1.0) ** m * (c.imag if m < 0 else c.real)


@pytest.mark.parametrize("degree", [0, 1, 2, 3, 4])
def test_sh_basis_matches_closed_form(degree):
    """kernels/sh.rs evaluates Sloan's real SH basis, which is the standard one
    times (-1)^m (the sign convention 3DGS training uses)."""
    rng = np.random.default_rng(20 + degree)
    for _ in range(50):
        v = rng.standard_normal(3)
        v = v / np.linalg.norm(v)
        got = po.sh_basis(degree, v.astype(np.float32))
        k = 0
        for l in range(degree + 1):
            for m in range(-l, l + 1):
                ref = (-1.0) ** m * _real_sh(l, m, v)
                assert abs(got[k] - ref) <= 2e-6 * max(1.0, abs(ref)), (l, m, got[k], ref)
                k += 1


def test_sh_basis_orthonormal():
    """Gram matrix of the degree-4 basis over the sphere by Gauss-Legendre x uniform azimuth."""
    deg = 4
    nt, nphi = 24, 48
    ct, wt = np.polynomial.legendre.leggauss(nt)
    phis = np.arange(nphi) * (2 * np.pi / nphi)
    gram = np.zeros(((deg + 1) ** 2,) * 2)
    for c, w in zip(ct, wt):
        s = np.sqrt(1 - c * c)
        for ph in phis:
            b = po.sh_basis(deg, np.array([s * np.cos(ph), s * np.sin(ph), c], np.float32)).astype(np.float64)
            gram += w * (2 * np.pi / nphi) * np.outer(b, b)
    np.testing.assert_allclose(gram, np.eye(gram.shape[0]), atol=2e-5)


def test_l1_cotangent_is_the_gradient_of_the_mean_abs_error():
    """crates/splat-train-loss/src/lib.rs:786-811: d/dpred mean|pred - gt| over rgb."""
    rng = np.random.default_rng(5)
    h, w = 6, 7
    pred = rng.uniform(0, 1, (h, w, 4)).astype(np.float32)
    gt = (np.round(rng.uniform(0, 1, (h, w, 3)) * 255) / 255).astype(np.float32)
    pred[0, 0, :3] = gt[0, 0]                       # sign(0) = 0
    v = l1_cotangent_np(pred, gt)

    def loss(p):
        return np.abs(p[..., :3].astype(np.float64) - gt).mean()

    eps = 1e-6
    for idx in [(0, 1, 0), (3, 4, 2), (5, 6, 1), (2, 2, 0)]:
        pp = pred.astype(np.float64).copy(); pp[idx] += eps
        pm = pred.astype(np.float64).copy(); pm[idx] -= eps
        fd = (loss(pp) - loss(pm)) / (2 * eps)
        assert abs(fd - v[idx]) <= 1e-6 * abs(v[idx]) + 1e-9
    assert np.all(v[0, 0, :3] == 0.0) and np.all(v[..., 3] == 0.0)
    np.testing.assert_allclose(np.abs(v[..., :3]).max(), 1.0 / (3 * h * w), rtol=1e-6)
