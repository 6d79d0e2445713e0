"""Pins the oracle's Mip render mode and scale floor (kernels/helpers.rs:
195-245, 497-553; bwd/kernels/project_backwards.rs:132-274) on the CPU.

* The reference's own known-answer test of the floor
  (gaussian_splats.rs:727-764, min_scale_fold_is_stable_for_tiny_scales):
  log-scale -20 floored at e^-20 gives opacity 0.5 * 0.5^1.5 and
  d logit(opacity) / d log-scale = 0.5 / (1 - opacity).
* Projected rows against float64 closed forms: Mip adds 0.1 to the 2-D
  covariance and multiplies the opacity by sqrt(det / det_blurred); the floor
  replaces each scale by sqrt(s^2 + f^2) and the opacity by
  clamp(sigmoid(raw) prod(s / s'), 1e-6, 1 - 1e-6).
* The projection VJP against central differences of a float64 projection of
  one splat.  The reference differentiates the opacity of Mip mode with the
  compensation factor held fixed (project_backwards.rs:218-220), so the
  float64 function holds it at its value at the expansion point; the floor's
  opacity factor is differentiated.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from vauss_amd import scenes

IMG = (96, 80)


def _quat_to_mat(q):
    w, x, y, z = q / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def _project64(t, raw, floor, mip, cam, fc_fixed=None):
    """Float64 projected row (x, y, c00, c01, c11, opacity) of one splat seen
    by the pinhole test camera (identity rotation, centre z = -4), plus the
    Mip factor and the floored opacity."""
    fx, fy, cx, cy = (float(v) for v in (cam.fx, cam.fy, cam.cx, cam.cy))
    pc = t[:3] + np.array([0.0, 0.0, 4.0])
    x, y, z = pc
    J = np.array([[fx / z, 0.0, -fx * x / (z * z)], [0.0, fy / z, -fy * y / (z * z)]])
    s = np.exp(t[7:10])
    o = _sig(raw)
    if floor is not None:
        sf = np.sqrt(s * s + floor * floor)
        o = np.clip(o * np.prod(s / sf), 1e-6, 1 - 1e-6)
        s = sf
    R = _quat_to_mat(t[3:7])
    M = R @ np.diag(s)
    raw_cov = J @ M @ M.T @ J.T
    blur = 0.1 if mip else 0.3
    cov = raw_cov + blur * np.eye(2)
    fc = np.sqrt(max(np.linalg.det(raw_cov), 0.0) / np.linalg.det(cov)) if mip else 1.0
    if fc_fixed is not None:
        fc = fc_fixed
    conic = np.linalg.inv(cov)
    row = np.array([fx * x / z + cx, fy * y / z + cy, conic[0, 0], conic[0, 1], conic[1, 1], o * fc])
    return row, fc, o


def _scene(n, seed):
    rng = np.random.default_rng(seed)
    means = np.stack([rng.uniform(-0.6, 0.6, n), rng.uniform(-0.5, 0.5, n), rng.uniform(-0.5, 0.5, n)], 1)
    quats = rng.standard_normal((n, 4))
    log_s = rng.uniform(-4.0, -2.0, (n, 3))
    t = np.concatenate([means, quats, log_s], 1).astype(np.float32)
    sh = (rng.standard_normal((n, 1, 3)) * 0.2).astype(np.float32)
    op = rng.uniform(-1, 2, n).astype(np.float32)
    floor = rng.uniform(0.0, 0.06, n).astype(np.float32)
    return t, sh, op, floor


def test_floor_known_answer():
    """gaussian_splats.rs:727-764 on one splat in front of the camera."""
    cam = scenes.test_camera(IMG, fov=0.9, position=(0.0, 0.0, -4.0)).uniforms(IMG)
    t = np.array([[0, 0, 0, 1, 0, 0, 0, -20, -20, -20]], np.float32)
    f = po.render_forward(cam, IMG, t, np.zeros((1, 1, 3), np.float32), np.zeros(1, np.float32),
                          min_scale=np.array([np.exp(np.float32(-20))], np.float32))
    expected = 0.5 * np.sqrt(0.5) ** 3
    opac = float(f.get(po.F_OPACITIES)[0])
    assert abs(opac - expected) < 1e-6
    vc = np.zeros((1, 10), np.float32)
    vc[0, 8] = 1.0                                  # d loss / d opacity = 1
    g = f.project_backward(vc)
    d_logit = g["v_transforms"][0, 7:10] / (opac * (1 - opac))
    assert np.all(np.abs(d_logit - 0.5 / (1 - expected)) < 2e-4), d_logit


@pytest.mark.parametrize("mip,use_floor", [(True, False), (False, True), (True, True)])
def test_projection_closed_form(mip, use_floor):
    cam_obj = scenes.test_camera(IMG, fov=0.9, position=(0.0, 0.0, -4.0))
    cam = cam_obj.uniforms(IMG)
    t, sh, op, floor = _scene(40, 3)
    flags = po.FLAG_BWD_INFO | (po.FLAG_MIP if mip else 0)
    f = po.render_forward(cam, IMG, t, sh, op, flags=flags, min_scale=floor if use_floor else None)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    rows = f.get(po.F_PROJECTED).astype(np.float64)
    opacities = f.get(po.F_OPACITIES)
    assert len(gfc) > 30
    for row, g in zip(rows, gfc):
        want, fc, o = _project64(t[g].astype(np.float64), float(op[g]), float(floor[g]) if use_floor else None, mip,
                                 cam)
        np.testing.assert_allclose(row[:2], want[:2], rtol=0, atol=2e-3)
        np.testing.assert_allclose(row[2:5], want[2:5], rtol=0, atol=3e-4 * np.abs(want[2:5]).max())
        assert abs(row[5] - want[5]) <= 2e-5 * max(1.0, want[5]), (row[5], want[5])
        assert abs(opacities[g] - o) <= 2e-6                # the aux opacity is the floored one, before Mip
        if mip:
            assert fc < 1.0


@pytest.mark.parametrize("mip,use_floor", [(False, False), (True, False), (False, True), (True, True)])
def test_vjp_matches_central_differences(mip, use_floor):
    cam = scenes.test_camera(IMG, fov=0.9, position=(0.0, 0.0, -4.0)).uniforms(IMG)
    t, sh, op, floor = _scene(12, 5)
    flags = po.FLAG_BWD_INFO | (po.FLAG_MIP if mip else 0)
    f = po.render_forward(cam, IMG, t, sh, op, flags=flags, min_scale=floor if use_floor else None)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    rng = np.random.default_rng(8)
    vc = np.zeros((len(t), 10), np.float32)
    vc[:, [0, 1, 2, 3, 4, 8]] = rng.standard_normal((len(t), 6)).astype(np.float32)
    vc[:, 2:5] *= 1e-2                               # conic entries are ~1e2 larger than positions
    g = f.project_backward(vc)
    checked = 0
    for gi in gfc:
        p0 = np.concatenate([t[gi].astype(np.float64), [float(op[gi])]])
        fl = float(floor[gi]) if use_floor else None
        _, fc0, _ = _project64(p0[:10], p0[10], fl, mip, cam)
        w = vc[gi, [0, 1, 2, 3, 4, 8]].astype(np.float64)

        def loss(p):
            return float(w @ _project64(p[:10], p[10], fl, mip, cam, fc_fixed=fc0)[0])
        num = np.zeros(11)
        for i in range(11):
            e = 1e-5 * max(1.0, abs(p0[i]))
            dp = np.zeros(11)
            dp[i] = e
            num[i] = (loss(p0 + dp) - loss(p0 - dp)) / (2 * e)
        got = np.concatenate([g["v_transforms"][gi], [g["v_raw_opac"][gi]]]).astype(np.float64)
        for grp in (slice(0, 3), slice(3, 7), slice(7, 10), slice(10, 11)):     # mean, quat, log-scale, opacity
            tol = 2e-3 * np.abs(num[grp]) + 2e-3 * np.abs(num[grp]).max() + 1e-9
            assert np.all(np.abs(got[grp] - num[grp]) <= tol), (gi, grp, got[grp], num[grp])
        checked += 1
    assert checked >= 10


@pytest.mark.parametrize("mip,use_floor", [(False, False), (False, True), (True, False), (True, True)])
def test_log_scale_offset_matches_materialized(mip, use_floor):
    """tests/mod.rs:287-382 (viewer_scale_matches_materialized_transforms) on
    the oracle: an offset of ln(s) renders exactly like log-scales shifted by
    ln(s) in f32 beforehand (counts, lists, aux, image, every dense gradient),
    and ln(2) visibly changes the render."""
    cam = scenes.test_camera(IMG, fov=0.9, position=(0.0, 0.0, -4.0)).uniforms(IMG)
    t, sh, op, floor = _scene(300, 11)
    flags = po.FLAG_BWD_INFO | (po.FLAG_MIP if mip else 0)
    fl = floor if use_floor else None
    base = po.render_forward(cam, IMG, t, sh, op, flags=flags, min_scale=fl)
    for scale in (0.5, 2.0):
        lso = np.float32(np.log(scale))
        tm = t.copy()
        tm[:, 7:10] = tm[:, 7:10] + lso
        a = po.render_forward(cam, IMG, t, sh, op, flags=flags, min_scale=fl, log_scale_offset=float(lso))
        b = po.render_forward(cam, IMG, tm, sh, op, flags=flags, min_scale=fl)
        assert a.info.num_visible == b.info.num_visible and a.info.num_intersections == b.info.num_intersections
        for field in (po.F_INTERSECT_COUNTS, po.F_ISECT_GID, po.F_TILE_OFFSETS_SHRUNK, po.F_MAX_RADIUS,
                      po.F_OPACITIES, po.F_PROJECTED, po.F_OUT_IMG):
            np.testing.assert_array_equal(a.get(field).view(np.uint32), b.get(field).view(np.uint32))
        assert not np.array_equal(a.get(po.F_OUT_IMG), base.get(po.F_OUT_IMG))
        v_out = (np.random.default_rng(4).standard_normal(a.get(po.F_OUT_IMG).shape) * 1e-3).astype(np.float32)
        ga, gb = a.backward(v_out), b.backward(v_out)
        for key in ("v_combined", "v_transforms", "v_sh", "v_raw_opac", "v_refine"):
            np.testing.assert_array_equal(ga[key].view(np.uint32), gb[key].view(np.uint32))
        assert np.abs(ga["v_transforms"][:, 7:10]).max() > 0
