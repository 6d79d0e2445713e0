"""Pins the oracle's camera gradient (bwd/kernels/pose_backwards.rs,
bwd/render_bwd.rs:224-288) on the CPU.

The gradient is d loss / d [A, b] of a camera-space perturbation
x_c' = (I + A) x_c + b applied after the world-to-camera transform, with A
pivoting on the camera centre, which b moves to c - M^-1 (I + A)^-1 b.

* Per-splat rows against central differences of a float64 pinhole projection
  of one splat (position, conic and SH degree-1 colour) under that
  perturbation, for a rotated camera (so M^-T and M^-1 differ), with the
  Default and Mip blurs and the scale floor.
* For every camera model, without restating the gradient:
  - the translation block equals M times the splat's dense mean gradient
    (a translation b moves every camera-space point by b and the camera
    centre by -M^-1 b);
  - the trace of the A block vanishes: every model projects x_c and x_c s
    alike (the 2-D covariance J S J^T is unchanged when x_c and S scale by s
    and s^2), and A = eps I pivots on the centre, so no direction moves.
* Rows whose position, conic and colour gradients are zero (only opacity or
  refine) are zero, as the reference's any_grad test skips them.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from vauss_amd import camera as vcam
from vauss_amd import scenes

IMG = (96, 80)
C0, C1 = 0.2820948, 0.4886025
POSITION = (1.2, -0.7, -3.6)


def _cam(model=None, img=IMG, fov=0.9):
    rot = vcam.look_at_rotation(POSITION, (0.05, -0.02, 0.1))
    kw = {} if model is None else {"model": model}
    return vcam.Camera(fov, fov, (0.5, 0.5), POSITION, rot, **kw).uniforms(img)


def _view(cam):
    vm = np.array(cam.viewmat[:], np.float64)
    return vm[:9].reshape(3, 3).T, vm[9:12], np.array(cam.cam_pos[:], np.float64)


def _quat_to_mat(q):
    w, x, y, z = q / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _project64(p, t, sh, floor, mip, cam):
    """[x, y, c00, c01, c11, r, g, b] of one splat under the perturbation p = [A (3x3 row-major), b]."""
    R, tr, c = _view(cam)
    A = p[:9].reshape(3, 3)
    b = p[9:12]
    IA = np.eye(3) + A
    mc = IA @ (R @ t[:3] + tr) + b
    s = np.exp(t[7:10])
    if floor is not None:
        s = np.sqrt(s * s + floor * floor)
    M = _quat_to_mat(t[3:7]) @ np.diag(s)
    S = IA @ R @ M @ M.T @ R.T @ IA.T
    fx, fy, cx, cy = (float(v) for v in (cam.fx, cam.fy, cam.cx, cam.cy))
    x, y, z = mc
    J = np.array([[fx / z, 0.0, -fx * x / (z * z)], [0.0, fy / z, -fy * y / (z * z)]])
    cov = J @ S @ J.T + (0.1 if mip else 0.3) * np.eye(2)
    conic = np.linalg.inv(cov)
    centre = c - np.linalg.solve(R, np.linalg.solve(IA, b))
    d = t[:3] - centre
    d /= np.linalg.norm(d)
    basis = np.array([C0, -C1 * d[1], C1 * d[2], -C1 * d[0]])
    rgb = basis @ sh + 0.5
    return np.array([fx * x / z + cx, fy * y / z + cy, conic[0, 0], conic[0, 1], conic[1, 1], *rgb])


def _scene(n, seed):
    rng = np.random.default_rng(seed)
    means = rng.uniform(-0.35, 0.35, (n, 3))
    quats = rng.standard_normal((n, 4))
    log_s = rng.uniform(-3.5, -2.0, (n, 3))
    t = np.concatenate([means, quats, log_s], 1).astype(np.float32)
    sh = (rng.standard_normal((n, 4, 3)) * 0.3).astype(np.float32)
    op = rng.uniform(-1, 2, n).astype(np.float32)
    floor = rng.uniform(0.0, 0.05, n).astype(np.float32)
    return t, sh, op, floor


@pytest.mark.parametrize("mip,use_floor", [(False, False), (True, False), (False, True)])
def test_rows_match_central_differences(mip, use_floor):
    cam = _cam()
    t, sh, op, floor = _scene(14, 21)
    flags = po.FLAG_BWD_INFO | (po.FLAG_MIP if mip else 0)
    f = po.render_forward(cam, IMG, t, sh, op, flags=flags, min_scale=floor if use_floor else None)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    assert len(gfc) >= 12
    rng = np.random.default_rng(9)
    vc = np.zeros((len(t), 10), np.float32)
    vc[:, :8] = rng.standard_normal((len(t), 8)).astype(np.float32)
    vc[:, 2:5] *= 1e-2                               # conic entries are ~1e2 larger than positions
    vc[:, 8:10] = rng.standard_normal((len(t), 2)).astype(np.float32)   # opacity, refine: no pose path
    total, rows = f.pose_backward(vc)
    np.testing.assert_allclose(total, rows[gfc].astype(np.float64).sum(0), rtol=1e-12, atol=1e-12)
    for g in gfc:
        fl = float(floor[g]) if use_floor else None
        tg = t[g].astype(np.float64)
        shg = sh[g].astype(np.float64)
        w = vc[g, :8].astype(np.float64)

        def loss(p):
            return float(w @ _project64(p, tg, shg, fl, mip, cam))
        num = np.zeros(12)
        for i in range(12):
            dp = np.zeros(12)
            dp[i] = 1e-6
            num[i] = (loss(dp) - loss(-dp)) / 2e-6
        got = rows[g].astype(np.float64)
        for grp in (slice(0, 9), slice(9, 12)):
            # the float64 differences agree with the float32 rows to ~1e-7 of the group's largest entry
            tol = 1e-4 * np.abs(num[grp]) + 1e-5 * np.abs(num[grp]).max() + 1e-12
            assert np.all(np.abs(got[grp] - num[grp]) <= tol), (g, grp, got[grp], num[grp])


MODELS = [None, vcam.KannalaBrandt4(0.03, -0.02, 0.01, -0.005),
          vcam.RadialTangential8(-0.15, 0.06, -0.01, 0.05, 0.02, -0.005, 0.03, -0.02),
          vcam.ThinPrismFisheye(vcam.KannalaBrandt4(0.03, -0.02, 0.01, -0.005), 0.02, -0.015, 0.01, -0.01)]


@pytest.mark.parametrize("model", MODELS, ids=["pinhole", "kb4", "rt8", "tpf"])
def test_translation_block_and_trace(model):
    img = (128, 96)
    cam = _cam(model, img, fov=1.1)
    sc = scenes.rng_scene(1500, 1.2, (-0.5, 0.5), (-2.0, -0.5), 0x9051)
    f = po.render_forward(cam, img, sc.transforms, sc.sh_coeffs, sc.raw_opacities)
    target = np.full((img[1], img[0], 3), 0.25, np.float32)
    img_out = f.get(po.F_OUT_IMG)
    v_out = np.zeros_like(img_out)
    v_out[..., :3] = np.sign(img_out[..., :3] - target) / (3.0 * img[0] * img[1])
    g = f.backward(v_out)
    vc = g["v_combined"]
    total, rows = f.pose_backward(vc)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    live = gfc[np.any(vc[gfc, :8] != 0, axis=1)]
    assert len(live) > 100
    R, _, _ = _view(cam)
    # translation block = M v_mean
    want_b = (R @ g["v_transforms"][live, 0:3].astype(np.float64).T).T
    got_b = rows[live, 9:12].astype(np.float64)
    scale_b = np.abs(want_b).max(1, keepdims=True) + 1e-30
    assert np.all(np.abs(got_b - want_b) <= 1e-4 * scale_b + 1e-12), np.abs(got_b - want_b).max()
    # trace of the A block vanishes per splat, against the size of its terms
    A = rows[live, :9].astype(np.float64).reshape(-1, 3, 3)
    tr = np.trace(A, axis1=1, axis2=2)
    size = np.abs(A).max((1, 2))
    assert np.all(np.abs(tr) <= 2e-4 * size + 1e-12), (np.abs(tr) / size).max()
    # the off-diagonal blocks do not vanish (the check above is not vacuous)
    assert np.median(np.abs(A[:, 0, 1]) / size) > 1e-3
    # rows without position, conic or colour gradients are zero
    dead = np.setdiff1d(np.arange(sc.num_splats), live)
    assert np.all(rows[dead] == 0)
    np.testing.assert_allclose(total, rows[live].astype(np.float64).sum(0), rtol=1e-12, atol=1e-15)


def test_opacity_only_rows_are_zero():
    cam = _cam()
    t, sh, op, _ = _scene(10, 3)
    f = po.render_forward(cam, IMG, t, sh, op)
    vc = np.zeros((len(t), 10), np.float32)
    vc[:, 8] = 1.0
    vc[:, 9] = 0.5
    total, rows = f.pose_backward(vc)
    assert np.all(rows == 0) and np.all(total == 0)
