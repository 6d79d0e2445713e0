"""Camera known-answer tests of the reference (crates/splat-train-render/src/camera.rs:385-595
and src/tests/mod.rs:807-885), run against both the oracle's f64 camera math and
the library's host camera functions (vs_fov_to_focal, vs_focal_to_fov,
vs_max_render_theta), which need no GPU."""
import math

import numpy as np
import pytest

from oracle import pyoracle as po
from vauss_amd import camera as vcam

# camera.rs:385-392: a near-rectilinear phone ultrawide fit that peaks at 65 deg.
ULTRAWIDE = (0.278781, 0.464781, -0.148871, -0.150010)
ULTRAWIDE_IMG = (4032, 3024)
ULTRAWIDE_FOCAL = 1606.3915
ULTRAWIDE_FOV_X = 103.5
KB4 = 1


class _Oracle:
    name = "oracle"

    @staticmethod
    def focal_to_fov(f, px, k=None):
        return po.focal_to_fov(f, px, 0 if k is None else KB4, k or (0, 0, 0, 0))

    @staticmethod
    def fov_to_focal(fov, px, k=None):
        return po.fov_to_focal(fov, px, 0 if k is None else KB4, k or (0, 0, 0, 0))

    @staticmethod
    def max_render_theta(k=None):
        return po.max_render_theta(0 if k is None else KB4, k or (0, 0, 0, 0))


class _Library:
    name = "library"

    @staticmethod
    def _model(k):
        return None if k is None else vcam.KannalaBrandt4(*k)

    @classmethod
    def focal_to_fov(cls, f, px, k=None):
        return vcam.focal_to_fov(f, px, cls._model(k))

    @classmethod
    def fov_to_focal(cls, fov, px, k=None):
        return vcam.fov_to_focal(fov, px, cls._model(k))

    @classmethod
    def max_render_theta(cls, k=None):
        return vcam.max_render_theta(cls._model(k))


IMPLS = [_Oracle, _Library]


def deg(r):
    return math.degrees(r)


def test_ultrawide_polynomial_folds_inside_hemisphere():
    fold = po.max_render_theta(KB4, ULTRAWIDE)
    assert abs(deg(fold) - 65.0) < 0.1
    assert abs(po.kb4_dd_dtheta(fold, ULTRAWIDE)) < 1e-6
    prev = 0.0
    for i in range(1, 1001):
        d = po.kb4_d(fold * i / 1000.0, ULTRAWIDE)
        assert d > prev
        prev = d
    assert po.kb4_d(math.radians(70.0), ULTRAWIDE) < po.kb4_d(fold, ULTRAWIDE)
    assert po.kb4_d(math.radians(85.0), ULTRAWIDE) < 0.0


@pytest.mark.parametrize("impl", IMPLS, ids=lambda c: c.name)
def test_ultrawide_fov_from_focal_stays_on_rising_branch(impl):
    fov_x = deg(impl.focal_to_fov(ULTRAWIDE_FOCAL, ULTRAWIDE_IMG[0], ULTRAWIDE))
    assert abs(fov_x - ULTRAWIDE_FOV_X) < 0.01, fov_x
    fov_y = deg(impl.focal_to_fov(ULTRAWIDE_FOCAL, ULTRAWIDE_IMG[1], ULTRAWIDE))
    assert abs(fov_y - 85.6) < 0.1, fov_y


@pytest.mark.parametrize("impl", IMPLS, ids=lambda c: c.name)
def test_ultrawide_focal_round_trips(impl):
    for pixels, focal in [(ULTRAWIDE_IMG[0], ULTRAWIDE_FOCAL), (ULTRAWIDE_IMG[1], ULTRAWIDE_FOCAL), (1920, 900.0),
                          (640, 260.0)]:
        fov = impl.focal_to_fov(focal, pixels, ULTRAWIDE)
        back = impl.fov_to_focal(fov, pixels, ULTRAWIDE)
        assert abs(back - focal) < 1e-6 * focal
    for fov_deg in [10.0, 60.0, 103.5, 125.0]:
        fov = math.radians(fov_deg)
        focal = impl.fov_to_focal(fov, ULTRAWIDE_IMG[0], ULTRAWIDE)
        back = impl.focal_to_fov(focal, ULTRAWIDE_IMG[0], ULTRAWIDE)
        assert abs(back - fov) < 1e-9
    # image edge past the polynomial's peak: the fov saturates at the fold
    fold = po.max_render_theta(KB4, ULTRAWIDE)
    assert impl.focal_to_fov(200.0, 640, ULTRAWIDE) == 2.0 * fold


def test_targets_past_the_fold_clamp_to_it():
    fold = po.max_render_theta(KB4, ULTRAWIDE)
    d_max = po.kb4_d(fold, ULTRAWIDE)
    assert po.kb4_invert_d(d_max, ULTRAWIDE) == fold
    assert po.kb4_invert_d(d_max * 10.0, ULTRAWIDE) == fold
    assert po.kb4_invert_d(0.0, ULTRAWIDE) == 0.0
    assert po.kb4_invert_d(-1.0, ULTRAWIDE) == 0.0


@pytest.mark.parametrize("impl", IMPLS, ids=lambda c: c.name)
def test_render_theta_is_capped_at_the_fold(impl):
    fov_x = impl.focal_to_fov(ULTRAWIDE_FOCAL, ULTRAWIDE_IMG[0], ULTRAWIDE)
    fov_y = impl.focal_to_fov(ULTRAWIDE_FOCAL, ULTRAWIDE_IMG[1], ULTRAWIDE)
    uncapped = math.hypot(fov_x, fov_y) * 1.05 * 0.5
    cap = impl.max_render_theta(ULTRAWIDE)
    assert cap < uncapped
    assert abs(deg(cap) - 65.0) < 0.1
    assert impl.max_render_theta(None) == math.pi


@pytest.mark.parametrize("impl", IMPLS, ids=lambda c: c.name)
def test_equidistant_lens_has_no_fold(impl):
    ident = (0.0, 0.0, 0.0, 0.0)
    assert impl.max_render_theta(ident) == math.pi
    for theta in [0.1, 1.0, 2.0, 3.0]:
        assert abs(po.kb4_invert_d(theta, ident) - theta) < 1e-12


@pytest.mark.parametrize("impl", IMPLS, ids=lambda c: c.name)
def test_pinhole_focal_to_fov_and_back(impl):
    fov = impl.focal_to_fov(800.0, 1920)
    assert abs(fov - 2.0 * math.atan(1920 / (2 * 800.0))) < 1e-12
    assert abs(impl.fov_to_focal(fov, 1920) - 800.0) < 1e-9


@pytest.mark.parametrize("impl", IMPLS, ids=lambda c: c.name)
def test_kb4_focal_to_fov_and_back(impl):
    # zero distortion: r_pix = f theta, so the full fov is pixels / f
    fov = impl.focal_to_fov(300.0, 1024, (0.0, 0.0, 0.0, 0.0))
    assert abs(fov - 1024 / 300.0) < 1e-9
    assert abs(impl.fov_to_focal(fov, 1024, (0.0, 0.0, 0.0, 0.0)) - 300.0) < 1e-9
    k = (-0.01, 0.003, -0.0005, 0.00002)
    fov = impl.focal_to_fov(280.0, 1024, k)
    assert abs(impl.fov_to_focal(fov, 1024, k) - 280.0) < 1e-6


def test_kb4_derivative_matches_central_differences():
    rng = np.random.default_rng(3)
    for _ in range(20):
        k = tuple(float(np.float32(v)) for v in rng.uniform(-0.05, 0.05, 4))
        th = float(rng.uniform(0.05, 1.5))
        h = 1e-6
        fd = (po.kb4_d(th + h, k) - po.kb4_d(th - h, k)) / (2 * h)
        assert abs(fd - po.kb4_dd_dtheta(th, k)) < 1e-7
        # d(theta) = theta (1 + k1 t^2 + k2 t^4 + k3 t^6 + k4 t^8), kannala_brandt_4.rs
        t2 = th * th
        closed = th * (1 + k[0] * t2 + k[1] * t2 ** 2 + k[2] * t2 ** 3 + k[3] * t2 ** 4)
        assert abs(po.kb4_d(th, k) - closed) < 1e-12


@pytest.mark.parametrize("model", [None, (0.03, -0.02, 0.01, -0.005)])
def test_camera_uniforms_agree_between_oracle_and_library(model):
    """vs_camera_uniforms (render.rs:478-503) against the closed forms it restates."""
    from vauss_amd import scenes
    img = (640, 480)
    m = None if model is None else vcam.KannalaBrandt4(*model)
    cam = vcam.Camera(0.9, 0.7, (0.45, 0.55), (0.3, -0.2, -4.0), (0.0, 0.0, 0.0, 1.0), m)
    u = cam.uniforms(img)
    fx = vcam.fov_to_focal(0.9, img[0], m)
    fy = vcam.fov_to_focal(0.7, img[1], m)
    assert u.fx == np.float32(fx) and u.fy == np.float32(fy)
    assert u.cx == np.float32(np.float32(0.45) * np.float32(640)) and u.cy == np.float32(np.float32(0.55) * np.float32(480))
    # identity rotation: world-to-camera is a pure translation by -position
    np.testing.assert_array_equal(np.array(u.viewmat[:9], np.float32), np.eye(3, dtype=np.float32).T.ravel())
    np.testing.assert_allclose(np.array(u.viewmat[9:]), [-0.3, 0.2, 4.0], rtol=0, atol=1e-7)
    np.testing.assert_allclose(np.array(u.cam_pos), [0.3, -0.2, -4.0], rtol=0, atol=1e-7)
    half = min(min(math.hypot(0.9, 0.7) * 1.05, 2 * math.pi - 1e-6) / 2, vcam.max_render_theta(m))
    assert abs(u.half_max_render_fov - half) < 1e-6
    if model is None:   # camera.rs:327-332
        assert abs(u.lim_pos_x - (1.15 * 640 - u.cx) / u.fx) < 1e-6
        assert abs(u.lim_neg_y - (-0.15 * 480 - u.cy) / u.fy) < 1e-6


# ---- RT8 and thin-prism fisheye (camera.rs:425-431, 494-575; tests/mod.rs:844-883) ----

RT8_PINCUSHION = (0.15, 0.08, 0.02, 0.03, 0.0, 0.0, 0.001, -0.002)   # k1..k6, p1, p2
KB4_MILD = (-0.01, 0.003, -0.0005, 0.00002)


def _library_limits(model, img, f, c):
    """Clamp limits from vs_camera_uniforms for a camera of focal f (both axes)."""
    cam = vcam.Camera.from_focal(f, f, img, center=c, model=model)
    u = cam.uniforms(img)
    return (u.lim_pos_x, u.lim_pos_y, u.lim_neg_x, u.lim_neg_y, u.lim_r), u


def test_rt8_radial_cap_matches_image_corner():
    img = (1920, 1080)
    corner_d = math.hypot((1.15 * 1920.0 - 960.0) / 800.0, (1.15 * 1080.0 - 540.0) / 800.0)
    lims = [po.clamp_limits(po.MODEL_RT8, img, 800.0, 800.0, 960.0, 540.0, RT8_PINCUSHION)]
    lib_lims, u = _library_limits(vcam.RadialTangential8(*RT8_PINCUSHION), img, 800.0, (960.0, 540.0))
    assert abs(u.fx - 800.0) < 1e-3
    lims.append(lib_lims)
    for (lim_pos_x, lim_pos_y, _, _, lim_r), tol in zip(lims, (1e-5, 1e-4)):   # the library's fx is f32 of a round trip
        assert abs(lim_r * po.rt8_radial(lim_r, RT8_PINCUSHION) - corner_d) < tol
        assert lim_r < math.hypot(lim_pos_x, lim_pos_y)
        assert lim_pos_x < lim_r and lim_pos_y < lim_r
    np.testing.assert_allclose(lims[0], lims[1], rtol=1e-5)


def test_rt8_radial_cap_is_unbounded_when_the_polynomial_folds():
    img = (1920, 1080)
    barrel = (-0.5, 0, 0, 0, 0, 0, 0, 0)
    assert po.clamp_limits(po.MODEL_RT8, img, 500.0, 500.0, 960.0, 540.0, barrel)[4] == np.float32(3.40282347e38)
    lib_lims, _ = _library_limits(vcam.RadialTangential8(*barrel), img, 500.0, (960.0, 540.0))
    assert lib_lims[4] == np.float32(3.40282347e38)
    assert po.rt8_undistort_corner_radius(10.0, barrel) is None
    for model, m in ((po.MODEL_PINHOLE, None), (po.MODEL_KB4, vcam.KannalaBrandt4(*ULTRAWIDE))):
        assert po.clamp_limits(model, img, 500.0, 500.0, 960.0, 540.0)[4] == np.float32(3.40282347e38)
        assert _library_limits(m, img, 500.0, (960.0, 540.0))[0][4] == np.float32(3.40282347e38)
    # the fisheye models leave the per-axis limits at zero
    assert _library_limits(vcam.KannalaBrandt4(*ULTRAWIDE), img, 500.0, (960.0, 540.0))[0][:4] == (0.0,) * 4


def test_rt8_focal_to_fov_and_back():
    rt8 = (-0.2, 0.05, -0.001, 0.0, 0.0, 0.0, 0.0, 0.0)
    fov = po.focal_to_fov(900.0, 1920, po.MODEL_RT8, dist=rt8)
    assert abs(po.fov_to_focal(fov, 1920, po.MODEL_RT8, dist=rt8) - 900.0) < 1e-6
    m = vcam.RadialTangential8(*rt8)
    fov_l = vcam.focal_to_fov(900.0, 1920, m)
    assert abs(vcam.fov_to_focal(fov_l, 1920, m) - 900.0) < 1e-6
    assert abs(fov - fov_l) < 1e-12
    # a radial factor below 1 (barrel) widens the fov past the pinhole's
    assert fov > po.focal_to_fov(900.0, 1920)


def test_tpf_focal_to_fov_and_back_follows_kb4():
    tp = (1e-3, -2e-3, 5e-4, -5e-4)
    for impl_fov, impl_focal, impl_theta in (
            (lambda f, px: po.focal_to_fov(f, px, po.MODEL_TPF, KB4_MILD, tp),
             lambda v, px: po.fov_to_focal(v, px, po.MODEL_TPF, KB4_MILD, tp),
             lambda k: po.max_render_theta(po.MODEL_TPF, k, tp)),
            (lambda f, px: vcam.focal_to_fov(f, px, vcam.ThinPrismFisheye(vcam.KannalaBrandt4(*KB4_MILD), *tp)),
             lambda v, px: vcam.fov_to_focal(v, px, vcam.ThinPrismFisheye(vcam.KannalaBrandt4(*KB4_MILD), *tp)),
             lambda k: vcam.max_render_theta(vcam.ThinPrismFisheye(vcam.KannalaBrandt4(*k), *tp)))):
        fov = impl_fov(280.0, 1024)
        assert abs(impl_focal(fov, 1024) - 280.0) < 1e-6
        assert abs(fov - po.focal_to_fov(280.0, 1024, po.MODEL_KB4, KB4_MILD)) < 1e-12
        # camera.rs:505-514: the thin-prism model folds where its KB4 part does
        assert impl_theta(ULTRAWIDE) == po.max_render_theta(po.MODEL_KB4, ULTRAWIDE)


def test_rt8_and_tpf_uniforms():
    img = (640, 480)
    rt8 = vcam.RadialTangential8(-0.05, 0.01, 0.0, 0.0, 0.0, 0.0, 1e-3, -1e-3)
    u = vcam.Camera(0.9, 0.7, (0.5, 0.5), (0.0, 0.0, -4.0), (0.0, 0.0, 0.0, 1.0), rt8).uniforms(img)
    assert u.model == 2 and tuple(u.dist) == tuple(np.float32(v) for v in (-0.05, 0.01, 0, 0, 0, 0, 1e-3, -1e-3))
    assert tuple(u.kb4) == (0.0,) * 4 and abs(u.half_max_render_fov - math.hypot(0.9, 0.7) * 1.05 / 2) < 1e-6
    want = po.clamp_limits(po.MODEL_RT8, img, u.fx, u.fy, u.cx, u.cy, list(u.dist))
    np.testing.assert_array_equal(np.array([u.lim_pos_x, u.lim_pos_y, u.lim_neg_x, u.lim_neg_y, u.lim_r], np.float32),
                                  np.array(want, np.float32))
    tpf = vcam.ThinPrismFisheye(vcam.KannalaBrandt4(*ULTRAWIDE), 1e-3, -2e-3, 5e-4, -5e-4)
    u = vcam.Camera(1.2, 1.0, (0.5, 0.5), (0.0, 0.0, -4.0), (0.0, 0.0, 0.0, 1.0), tpf).uniforms(img)
    assert u.model == 3 and tuple(u.kb4) == tuple(np.float32(v) for v in ULTRAWIDE)
    assert tuple(u.dist)[:4] == tuple(np.float32(v) for v in (1e-3, -2e-3, 5e-4, -5e-4))
    assert abs(u.half_max_render_fov - min(math.hypot(1.2, 1.0) * 1.05 / 2,
                                           po.max_render_theta(po.MODEL_KB4, ULTRAWIDE))) < 1e-6
