"""Pins the oracle's compact neural appearance (kernels/neural.rs,
bwd/kernels/neural_backwards.rs) and the transcendentals it adds.

* sin, cos and tanh against numpy's float64 functions (error in f32 ulps of
  the result, or of 1 for sin/cos near their zeros, where an argument
  reduction's absolute error is what any f32 implementation leaves) and
  their special values.
* The decoder colour of rendered splats against a float64 decoder built from
  numpy's sin / cos / tanh, matrix products of the packed [816] weights and
  the real SH basis from scipy (Condon-Shortley phase times (-1)^m, the
  convention of the colour SH), for every direction band 0..3.
* The backward against central differences of that float64 decoder: each
  row's gradient (base in DC units, latents), the view-direction term of the
  mean gradient, and the decoder gradient summed over the splats.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.test_oracle_math import _real_sh, _ulp_err
from vauss_amd import camera as vcam

IMG = (64, 48)
C0 = 0.2820948
POSITION = (0.9, -0.5, -3.2)


def test_sincos_accuracy():
    rng = np.random.default_rng(31)
    x = np.concatenate([rng.uniform(-np.pi / 4, np.pi / 4, 300_000), rng.uniform(-100, 100, 700_000),
                        rng.uniform(-1e4, 1e4, 100_000), np.arange(-64, 65) * (np.pi / 2)]).astype(np.float32)
    s, c = po.sincosf(x)
    x64 = x.astype(np.float64)
    for got, ref in ((s, np.sin(x64)), (c, np.cos(x64))):
        ulps = _ulp_err(got, ref)
        near_zero = np.abs(ref) < 2 ** -6
        assert ulps[~near_zero].max() <= 2.0, ulps[~near_zero].max()
        # near a zero the result is the reduced argument: its absolute error counts
        assert np.abs(got[near_zero] - ref[near_zero]).max() <= 2 ** -24 * np.maximum(1.0, np.abs(x64[near_zero]) / 64).max()


def test_sincos_special_values():
    s, c = po.sincosf(np.array([0.0, -0.0, np.inf, -np.inf, np.nan], np.float32))
    assert s[0] == 0.0 and c[0] == 1.0 and c[1] == 1.0
    assert np.all(np.isnan(s[2:])) and np.all(np.isnan(c[2:]))
    # sin^2 + cos^2 = 1 within rounding
    x = np.random.default_rng(3).uniform(-50, 50, 100_000).astype(np.float32)
    s, c = po.sincosf(x)
    assert np.abs(s.astype(np.float64) ** 2 + c.astype(np.float64) ** 2 - 1).max() < 5e-7


def test_tanh_accuracy_and_special_values():
    rng = np.random.default_rng(32)
    x = np.concatenate([rng.uniform(-0.6, 0.6, 400_000), rng.uniform(-12, 12, 600_000),
                        rng.uniform(-1e-4, 1e-4, 50_000), [0.5625, -0.5625, np.nextafter(np.float32(0.5625), 0)]])
    x = x.astype(np.float32)
    got = po.tanhf(x)
    assert _ulp_err(got, np.tanh(x.astype(np.float64))).max() <= 2.0
    y = po.tanhf(np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 60.0, -60.0], np.float32))
    assert y[0] == 0.0 and not np.signbit(y[0]) and y[1] == 0.0 and np.signbit(y[1])
    assert y[2] == 1.0 and y[3] == -1.0 and np.isnan(y[4]) and y[5] == 1.0 and y[6] == -1.0


def _basis64(dirs, deg):
    out = np.zeros((len(dirs), 16))
    k = 0
    for l in range(4):
        for m in range(-l, l + 1):
            if l <= deg:
                out[:, k] = [(-1.0) ** m * _real_sh(l, m, d) for d in dirs]
            k += 1
    return out


def _decode64(rows, W, dirs, deg, basis=None):
    """Colour [n,3] of the float64 decoder."""
    rows = np.asarray(rows, np.float64)
    lat = rows[:, 3:11]
    x = np.empty((len(rows), 32))
    x[:, 0:16:2] = np.sin(lat)
    x[:, 1:16:2] = np.cos(lat)
    x[:, 16:] = _basis64(dirs, deg) if basis is None else basis
    W = np.asarray(W, np.float64)
    h1 = np.maximum(x @ W[:512].reshape(16, 32).T, 0)
    h2 = np.maximum(h1 @ W[512:768].reshape(16, 16).T, 0)
    o = h2 @ W[768:].reshape(3, 16).T
    return np.maximum(C0 * rows[:, :3] + np.tanh(o) + 0.5, 0)


def _scene(n, seed):
    rng = np.random.default_rng(seed)
    t = np.concatenate([rng.uniform(-0.4, 0.4, (n, 3)), rng.standard_normal((n, 4)),
                        rng.uniform(-3.0, -2.0, (n, 3))], 1).astype(np.float32)
    rows = np.zeros((n, 4, 3), np.float32)
    flat = rows.reshape(n, 12)
    flat[:, :3] = rng.uniform(-1, 1, (n, 3))
    flat[:, 3:11] = rng.uniform(-3, 3, (n, 8))
    op = rng.uniform(0, 2, n).astype(np.float32)
    W = (rng.standard_normal(816) * 0.35).astype(np.float32)
    return t, rows, op, W


def _cam():
    rot = vcam.look_at_rotation(POSITION, (0.0, 0.0, 0.0))
    return vcam.Camera(0.9, 0.9, (0.5, 0.5), POSITION, rot).uniforms(IMG)


def _dirs(cam, means):
    d = means.astype(np.float64) - np.array(cam.cam_pos[:], np.float64)
    return d / np.linalg.norm(d, axis=1, keepdims=True)


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_colour_matches_float64_decoder(deg):
    cam = _cam()
    t, rows, op, W = _scene(60, 40 + deg)
    f = po.render_forward(cam, IMG, t, rows, op, decoder=W, neural_degree=deg)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    assert len(gfc) > 40
    got = f.get(po.F_PROJECTED)[:, 6:9].astype(np.float64)
    want = _decode64(rows.reshape(-1, 12)[gfc], W, _dirs(cam, t[gfc, :3]), deg)
    assert np.abs(got - want).max() < 2e-5, np.abs(got - want).max()
    assert (want > 0).mean() > 0.5 and want.std() > 0.05          # the decoder is not saturated or dead
    # the single-row hook agrees with the render
    u = t[gfc[0], :3] - np.array(cam.cam_pos[:], np.float32)            # the f32 normalize of the projection
    inv = np.float32(1.0) / np.sqrt((u[0] * u[0] + u[1] * u[1]) + u[2] * u[2])
    one = po.neural_color(rows.reshape(-1, 12)[gfc[0]], W, (u * inv).astype(np.float32), deg)
    np.testing.assert_array_equal(one, f.get(po.F_PROJECTED)[0, 6:9])


@pytest.mark.parametrize("deg", [1, 3])
def test_backward_matches_central_differences(deg):
    cam = _cam()
    t, rows, op, W = _scene(24, 7 + deg)
    f = po.render_forward(cam, IMG, t, rows, op, decoder=W, neural_degree=deg)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    n = len(t)
    rng = np.random.default_rng(70 + deg)
    vc = np.zeros((n, 10), np.float32)
    vc[gfc, 5:8] = rng.standard_normal((len(gfc), 3)).astype(np.float32)
    g = f.project_backward(vc)
    flat = rows.reshape(n, 12).astype(np.float64)
    wts = vc[gfc, 5:8].astype(np.float64)
    dirs0 = _dirs(cam, t[gfc, :3])

    def loss(r=None, w=None, means=None):
        r = flat[gfc] if r is None else r
        w = W if w is None else w
        d = dirs0 if means is None else _dirs(cam, means)
        return float(np.sum(wts * _decode64(r, w, d, deg)))

    eps = 1e-6
    # row gradients: base (DC units) and latents
    v_rows = g["v_sh"].reshape(n, 12)[gfc].astype(np.float64)
    num = np.zeros((len(gfc), 11))
    for i in range(11):
        for s in (1, -1):
            r = flat[gfc].copy()
            r[np.arange(len(gfc)), i] += s * eps      # each row only moves its own splat's colour
            num[:, i] += s * _per_splat(wts, _decode64(r, W, dirs0, deg)) / (2 * eps)
    assert np.abs(v_rows[:, :11] - num).max() <= 1e-4 * np.abs(num).max() + 1e-9, np.abs(v_rows[:, :11] - num).max()
    assert np.all(g["v_sh"].reshape(n, 12)[:, 11] == 0)
    np.testing.assert_allclose(g["v_coeffs_sq"][gfc], (g["v_sh"].reshape(n, 12)[gfc].astype(np.float64) ** 2).mean(1),
                               rtol=1e-5)
    # view-direction term of the mean gradient (no other raster gradient here)
    v_mean = g["v_transforms"][gfc, 0:3].astype(np.float64)
    numm = np.zeros((len(gfc), 3))
    for i in range(3):
        for s in (1, -1):
            m = t[gfc, :3].astype(np.float64).copy()
            m[:, i] += s * eps
            numm[:, i] += s * _per_splat(wts, _decode64(flat[gfc], W, _dirs(cam, m), deg)) / (2 * eps)
    assert np.abs(v_mean - numm).max() <= 1e-4 * np.abs(numm).max() + 1e-9, np.abs(v_mean - numm).max()
    assert np.abs(numm).max() > 1e-3
    # decoder gradient
    numw = np.zeros(816)
    for i in range(816):
        wp, wm = W.astype(np.float64).copy(), W.astype(np.float64).copy()
        wp[i] += eps
        wm[i] -= eps
        numw[i] = (loss(w=wp) - loss(w=wm)) / (2 * eps)
    got = g["v_decoder"].astype(np.float64)
    assert np.abs(got - numw).max() <= 1e-4 * np.abs(numw).max() + 1e-9, np.abs(got - numw).max()
    assert np.count_nonzero(numw) > 400


def _per_splat(wts, col):
    return np.sum(wts * col, axis=1)


def test_neural_rows_without_colour_gradient_are_zero():
    cam = _cam()
    t, rows, op, W = _scene(20, 5)
    f = po.render_forward(cam, IMG, t, rows, op, decoder=W, neural_degree=2)
    vc = np.zeros((20, 10), np.float32)
    vc[:, 8] = 1.0
    g = f.project_backward(vc)
    assert np.all(g["v_sh"] == 0) and np.all(g["v_decoder"] == 0) and np.all(g["v_coeffs_sq"] == 0)
