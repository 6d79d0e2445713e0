"""Pins of hot-path details of the oracle that its other tests leave open:
constants of the culling (Appendix-A values of the reference), the colour
clamp, the covariance clamp, the backward's alpha-saturation gate, the
max_radius axes, the refine weight's normalisation and the depth key order of
splats behind a fisheye's camera plane.  Each check comes from the reference's
constants and from mathematics the oracle does not share (float64 closed
forms, exact equalities), so a mistake common to the oracle and the kernels
fails here:

* opacity cull (kernels/project_forward.rs:157): splats at opacity
  (1/255)(1 +- 1e-3) and (1 +- 1e-2) are kept exactly when above;
* pinhole near plane (project_forward.rs:78-83): z = 0.01 and 0.01(1 + 1e-3)
  kept, the f32 below 0.01 and 0.01(1 - 1e-3) culled; a fisheye keeps z = 0.005
  on its axis (its cull is angular);
* every pixel whose float64 alpha (from a float64 projection of every input
  splat, culls included) reaches the cutoff lies in a tile the splat was
  emitted to, in a scene with splats just above the opacity cutoff and just
  beyond the near plane;
* covariance clamp (kernels/helpers.rs:217-224): the conic of a splat with
  log-scales ~25 is the float64 inverse of the 2-D covariance rescaled to a
  largest entry of 1e18, plus the 0.3 blur; one at ~16.5 is not rescaled;
* colour clamp (kernels/project_visible.rs:52-60): SH DC terms driving the
  colour past +-100 give exactly +-100, ones just inside are kept, non-finite
  colours become 0;
* saturation gate (bwd/kernels/rasterize_backwards_planes.rs:579-593): where
  opacity * G > 0.999 the capped alpha (0.999) is flat, so a cotangent on that
  pixel alone gives position, shape, opacity and refine gradients of exactly
  0 (central differences of the forward agree), and a non-saturated copy of
  the splat gets the central-difference opacity gradient;
* max_radius (project_forward.rs:191): max(ex / W, ey / H) with
  ex = sqrt(2 ln(255 o) Sigma00), ey = sqrt(2 ln(255 o) Sigma11) in float64,
  for elongated splats in a 4:1 image;
* refine weight (rasterize_backwards_planes.rs:209, 588-592): with a
  cotangent on one pixel p it is the equality
  |(v_x W, v_y H)| / max(a_p, 1e-5), a_p the pixel's final alpha;
* depth order (render.rs:689-694): in a wide Kannala-Brandt camera with
  splats behind its camera plane, each tile's list is the stable order of the
  raw f32 bits of the float64 view z (negative z after every positive one).
"""
import math

import numpy as np
import pytest

from oracle import pyoracle as po
from vauss_amd import camera as vcam
from vauss_amd import scenes

SH_C0 = 0.28209479177387814


def _ident_cam(img, fov=0.8, model=None):
    """A camera at the origin looking down +z: view space equals world space."""
    return vcam.Camera(fov, fov, (0.5, 0.5), (0.0, 0.0, 0.0), (0.0, 0.0, 0.0, 1.0), model).uniforms(img)


def _logit(p):
    p = np.asarray(p, np.float64)
    return np.log(p / (1.0 - p)).astype(np.float32)


def _quat_to_mat(q):
    w, x, y, z = q / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _pinhole_cov64(cam, t):
    """float64 (mean2d, raw 2-D covariance) of one splat under the identity
    pinhole camera, with the Jacobian's frustum clamp
    (kernels/camera_model/pinhole.rs: tx = z clamp(x/z, lim_neg, lim_pos))."""
    fx, fy, cx, cy = (float(v) for v in (cam.fx, cam.fy, cam.cx, cam.cy))
    x, y, z = (float(v) for v in t[:3])
    tx = z * min(max(x / z, float(cam.lim_neg_x)), float(cam.lim_pos_x))
    ty = z * min(max(y / z, float(cam.lim_neg_y)), float(cam.lim_pos_y))
    J = np.array([[fx / z, 0.0, -fx * tx / (z * z)], [0.0, fy / z, -fy * ty / (z * z)]])
    M = _quat_to_mat(t[3:7].astype(np.float64)) @ np.diag(np.exp(t[7:10].astype(np.float64)))
    return np.array([fx * x / z + cx, fy * y / z + cy]), J @ M @ M.T @ J.T


def _splats_at(cam, uv, z, log_scale, raw, dc=(0.5, 0.5, 0.5)):
    """Splats whose means project (in float64) to pixel positions uv at depth z."""
    n = len(uv)
    fx, fy, cx, cy = (float(v) for v in (cam.fx, cam.fy, cam.cx, cam.cy))
    z = np.broadcast_to(np.asarray(z, np.float64), (n,))
    t = np.zeros((n, 10), np.float32)
    t[:, 0] = (np.array([p[0] for p in uv]) - cx) * z / fx
    t[:, 1] = (np.array([p[1] for p in uv]) - cy) * z / fy
    t[:, 2] = z
    t[:, 3] = 1.0
    t[:, 7:10] = np.broadcast_to(np.asarray(log_scale, np.float32), (n, 3))
    sh = np.tile(np.asarray(dc, np.float32), (n, 1)).reshape(n, 1, 3)
    return scenes.Scene(t, sh, np.broadcast_to(np.asarray(raw, np.float32), (n,)).copy())


def _render(scene, cam, img, flags=po.FLAG_BWD_INFO):
    return po.render_forward(cam, img, scene.transforms, scene.sh_coeffs, scene.raw_opacities, flags=flags)


# ---- culling constants ------------------------------------------------------------


def test_opacity_cull_threshold():
    img = (64, 64)
    cam = _ident_cam(img)
    rel = np.array([1 + 1e-3, 1 - 1e-3, 1 + 1e-2, 1 - 1e-2])
    uv = [(8.5, 8.5), (24.5, 8.5), (40.5, 8.5), (56.5, 8.5)]
    sc = _splats_at(cam, uv, 3.0, -3.0, _logit(rel / 255.0))
    f = _render(sc, cam, img)
    opac = 1.0 / (1.0 + np.exp(-sc.raw_opacities.astype(np.float64)))
    keep = opac >= 1.0 / 255.0
    np.testing.assert_array_equal(keep, rel > 1)
    counts = f.get(po.F_INTERSECT_COUNTS)
    assert (counts[keep] >= 1).all() and (counts[~keep] == 0).all(), counts
    assert f.info.num_visible == int(keep.sum())


def test_pinhole_near_plane():
    img = (64, 64)
    cam = _ident_cam(img)
    z01 = np.float32(0.01)
    zs = np.array([z01, np.nextafter(z01, np.float32(0)), 0.01 * (1 + 1e-3), 0.01 * (1 - 1e-3), 0.5], np.float32)
    sc = _splats_at(cam, [(32.0, 32.0)] * len(zs), zs.astype(np.float64), -12.0, 2.0)
    sc.transforms[:, 2] = zs                       # exactly these f32 depths
    f = _render(sc, cam, img)
    counts = f.get(po.F_INTERSECT_COUNTS)
    keep = zs >= z01
    np.testing.assert_array_equal(keep, [True, False, True, False, True])
    assert (counts[keep] >= 1).all() and (counts[~keep] == 0).all(), counts
    # a fisheye culls by angle only: a splat on its axis at z = 0.005 is kept
    kb = _ident_cam(img, fov=1.2, model=vcam.KannalaBrandt4(0.01, 0.0, 0.0, 0.0))
    near = _splats_at(cam, [(32.0, 32.0)], 0.005, -12.0, 2.0)
    fk = _render(near, kb, img)
    assert fk.info.num_visible == 1 and fk.get(po.F_INTERSECT_COUNTS)[0] >= 1


def _pinhole_footprint_scene(seed=0xF00F):
    """Regular splats, splats just above the opacity cutoff with wide
    footprints, and small splats just beyond the near plane."""
    rng = np.random.default_rng(seed)
    base = scenes.rng_scene(240, 1.2, (-2.8, -1.5), (-1.0, 3.0), 0xA5A5)
    t0 = base.transforms.copy()
    t0[:, 2] += 4.0
    n1 = 80
    z1 = rng.uniform(2.0, 5.0, n1)
    t1 = np.concatenate([np.stack([rng.uniform(-0.4, 0.4, n1) * z1, rng.uniform(-0.4, 0.4, n1) * z1, z1], 1),
                         rng.standard_normal((n1, 4)), rng.uniform(-2.6, -1.8, (n1, 3))], 1).astype(np.float32)
    o1 = _logit(rng.uniform(1.02, 2.5, n1) / 255.0)
    n2 = 60
    z2 = rng.uniform(0.0105, 0.3, n2)
    t2 = np.concatenate([np.stack([rng.uniform(-0.35, 0.35, n2) * z2, rng.uniform(-0.35, 0.35, n2) * z2, z2], 1),
                         rng.standard_normal((n2, 4)), np.log(z2)[:, None] + rng.uniform(-5.5, -4.0, (n2, 3))],
                        1).astype(np.float32)
    o2 = rng.uniform(-1.0, 2.0, n2).astype(np.float32)
    t = np.concatenate([t0, t1, t2])
    sh = rng.uniform(0.0, 1.0, (len(t), 1, 3)).astype(np.float32)
    return scenes.Scene(t, sh, np.concatenate([base.raw_opacities, o1, o2]).astype(np.float32))


def test_tile_hits_cover_float64_footprints():
    """Conservativeness from a float64 projection of every input splat (not
    from the oracle's own visible rows): a splat the oracle culls or bins
    short shows up as a pixel whose float64 alpha reaches the cutoff outside
    the splat's emitted tiles."""
    img = (96, 80)
    cam = _ident_cam(img, fov=0.9)
    sc = _pinhole_footprint_scene()
    f = _render(sc, cam, img)
    hit = set(zip(f.get(po.F_ISECT_TILE).tolist(), f.get(po.F_ISECT_GID).tolist()))
    w, h = img
    tbw = (w + 15) // 16
    yy, xx = np.mgrid[0:h, 0:w]
    px, py = xx.ravel() + 0.5, yy.ravel() + 0.5
    tiles = (yy.ravel() // 16) * tbw + xx.ravel() // 16
    checked = {"low_opacity": 0, "near": 0}
    for g in range(sc.num_splats):
        t = sc.transforms[g].astype(np.float64)
        op = 1.0 / (1.0 + math.exp(-float(sc.raw_opacities[g])))
        z = t[2]
        if z < 0.01 * (1 + 1e-6) or op < (1.0 / 255.0) * (1 + 1e-6):
            continue                                  # culled by the reference's definition (or on the edge)
        m2, raw = _pinhole_cov64(cam, sc.transforms[g])
        scale = min(1.0, 1e18 / np.abs(raw).max())
        conic = np.linalg.inv(raw * scale + 0.3 * np.eye(2))
        dx, dy = px - m2[0], py - m2[1]
        sig = 0.5 * (conic[0, 0] * dx * dx + conic[1, 1] * dy * dy) + conic[0, 1] * dx * dy
        alpha = np.minimum(0.999, op * np.exp(-sig))
        need = np.nonzero((sig >= 0) & (alpha >= (1.0 / 255.0) * (1 + 1e-4)))[0]
        missing = [int(tiles[p]) for p in need if (int(tiles[p]), g) not in hit]
        assert not missing, (g, z, op, missing[:5])
        if len(need):
            if op < 2.5 / 255.0:
                checked["low_opacity"] += 1
            if z < 0.3:
                checked["near"] += 1
    assert checked["low_opacity"] >= 20 and checked["near"] >= 20, checked


# ---- clamps -------------------------------------------------------------------------


def test_covariance_clamp():
    img = (64, 64)
    cam = _ident_cam(img)
    rng = np.random.default_rng(21)
    t = np.zeros((3, 10), np.float32)
    t[:, 0:3] = [[0.3, -0.2, 5.0], [-0.25, 0.1, 4.0], [0.1, 0.2, 6.0]]
    t[:, 3:7] = rng.standard_normal((3, 4)).astype(np.float32)
    t[:, 7:10] = [[25.0, 24.6, 24.2], [25.3, 25.0, 24.1], [16.5, 16.2, 16.0]]
    sc = scenes.Scene(t, np.full((3, 1, 3), 0.5, np.float32), np.full(3, 1.0, np.float32))
    f = _render(sc, cam, img)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    np.testing.assert_array_equal(gfc, [0, 1, 2])
    rows = f.get(po.F_PROJECTED).astype(np.float64)
    for g in range(3):
        _, raw = _pinhole_cov64(cam, t[g])
        big = np.abs(raw).max()
        assert (big > 1e20) if g < 2 else (1e15 < big < 1e18), big
        want = np.linalg.inv(raw * min(1.0, 1e18 / big) + 0.3 * np.eye(2))
        got = np.array([[rows[g, 2], rows[g, 3]], [rows[g, 3], rows[g, 4]]])
        np.testing.assert_allclose(got, want, rtol=0, atol=2e-3 * np.abs(want).max())


def test_colour_clamp():
    img = (64, 64)
    cam = _ident_cam(img)
    c0 = np.float64(SH_C0)
    # DC terms giving colours 300 (clamped), -300 (clamped), 100.6 (clamped),
    # 99.2 (kept), -99.2 (kept), +inf and nan (0)
    targets = [300.0, -300.0, 100.6, 99.2, -99.2]
    dc = [(v - 0.5) / c0 for v in targets] + [np.inf, np.nan]
    n = len(dc)
    sc = _splats_at(cam, [(8.5 + 7 * i, 32.5) for i in range(n)], 3.0, -3.0, 1.0)
    sh = np.zeros((n, 1, 3), np.float32)
    sh[:, 0, 0] = np.array(dc, np.float64).astype(np.float32)
    sh[:, 0, 1] = 0.5                              # colour 0.5 + 0.5 C0
    sh[:, 0, 2] = -sh[:, 0, 0]
    sc = scenes.Scene(sc.transforms, sh, sc.raw_opacities)
    f = _render(sc, cam, img)
    np.testing.assert_array_equal(f.get(po.F_GLOBAL_FROM_COMPACT), np.arange(n))
    col = f.get(po.F_PROJECTED)[:, 6:9]
    expect_r = [100.0, -100.0, 100.0, 99.2, -99.2, 0.0, 0.0]
    expect_b = [-100.0, 100.0, -99.6, None, None, 0.0, 0.0]
    for i in range(n):
        if abs(expect_r[i]) == 100.0 or expect_r[i] == 0.0:
            assert col[i, 0] == np.float32(expect_r[i]), (i, col[i])
        else:
            assert abs(col[i, 0] - expect_r[i]) < 1e-4, (i, col[i])
        if expect_b[i] is not None and (abs(expect_b[i]) == 100.0 or expect_b[i] == 0.0):
            assert col[i, 2] == np.float32(expect_b[i]), (i, col[i])
        assert abs(col[i, 1] - (0.5 + 0.5 * SH_C0)) < 1e-6
    # -(100.6 - 0.5) + 0.5 = -99.6 is inside the clamp
    assert abs(col[2, 2] - (-99.6)) < 1e-4


# ---- backward -----------------------------------------------------------------------


def _gate_scene(cam, raw):
    """One splat of 2-D std ~10 px whose mean sits 0.2, 0.1 px off the centre
    of pixel (24, 20)."""
    fx = float(cam.fx)
    z = 3.0
    ls = math.log(10.0 * z / fx)
    return _splats_at(cam, [(24.5 + 0.2, 20.5 + 0.1)], z, ls, raw, dc=(0.4, 0.6, 0.2))


def test_saturated_pixels_give_no_geometry_gradient():
    img = (48, 40)
    cam = _ident_cam(img)
    v_out = np.zeros((img[1], img[0], 4), np.float32)
    v_out[20, 24] = [0.3, -0.2, 0.5, 0.7]
    for raw, saturated in ((8.0, True), (5.0, False)):
        sc = _gate_scene(cam, raw)
        f = _render(sc, cam, img)
        row = f.get(po.F_PROJECTED)[0].astype(np.float64)
        dx, dy = 24.5 - row[0], 20.5 - row[1]
        G = math.exp(-(0.5 * (row[2] * dx * dx + row[4] * dy * dy) + row[3] * dx * dy))
        assert (row[5] * G > 0.999 + 1e-4) if saturated else (row[5] * G < 0.999 - 1e-3), row[5] * G
        g = f.backward(v_out)
        vc = g["v_combined"][0]
        assert np.abs(vc[5:8]).max() > 1e-3                    # colour gradients flow either way

        def loss(t, o):
            img_ = po.render_forward(cam, img, t, sc.sh_coeffs, o, flags=po.FLAG_BWD_INFO).get(po.F_OUT_IMG)
            return float((img_.astype(np.float64) * v_out).sum())
        eps = 1e-3
        num_o = (loss(sc.transforms, sc.raw_opacities + eps) - loss(sc.transforms, sc.raw_opacities - eps)) / (2 * eps)
        d = np.zeros_like(sc.transforms)
        d[0, 0] = 1e-3
        num_x = (loss(sc.transforms + d, sc.raw_opacities) - loss(sc.transforms - d, sc.raw_opacities)) / 2e-3
        if saturated:
            assert num_o == 0.0 and abs(num_x) < 1e-7, (num_o, num_x)
            assert not vc[0:5].any() and vc[8] == 0 and vc[9] == 0, vc
            assert not g["v_transforms"].any() and g["v_raw_opac"][0] == 0 and g["v_refine"][0] == 0
        else:
            assert abs(g["v_raw_opac"][0] - num_o) <= 1e-3 * abs(num_o) + 1e-6, (g["v_raw_opac"][0], num_o)
            assert abs(num_o) > 1e-4 and vc[9] > 0


def test_refine_weight_with_a_one_pixel_cotangent():
    img = (64, 48)
    cam = scenes.test_camera(img, fov=0.6, position=(0.0, 0.0, -3.0)).uniforms(img)
    scene = scenes.rng_scene(150, 1.0, (-2.5, -1.0), (-3.0, 0.0), 0x7E57)
    f = _render(scene, cam, img)
    out = f.get(po.F_OUT_IMG)
    rng = np.random.default_rng(6)
    alphas = out[..., 3]
    cand = np.argwhere((alphas > 0.15) & (alphas < 0.85))
    assert len(cand) > 50
    checked = 0
    for py, px in cand[rng.choice(len(cand), 6, replace=False)]:
        v = np.zeros_like(out)
        v[py, px] = rng.standard_normal(4).astype(np.float32) * 1e-2
        vc = f.backward(v)["v_combined"].astype(np.float64)
        on = np.hypot(vc[:, 0], vc[:, 1]) > 0
        assert on.sum() >= 1
        a = max(float(alphas[py, px]), 1e-5)
        want = np.hypot(vc[on, 0] * img[0], vc[on, 1] * img[1]) / a
        np.testing.assert_allclose(vc[on, 9], want, rtol=2e-6, atol=0)
        assert not vc[~on, 9].any()
        checked += int(on.sum())
    assert checked >= 10


def test_max_radius_axes():
    img = (192, 48)
    cam = vcam.Camera(1.2, 0.35, (0.5, 0.5), (0.0, 0.0, 0.0), (0.0, 0.0, 0.0, 1.0)).uniforms(img)
    rng = np.random.default_rng(31)
    n = 40
    z = rng.uniform(3.0, 6.0, n)
    t = np.concatenate([np.stack([rng.uniform(-0.4, 0.4, n) * z, rng.uniform(-0.1, 0.1, n) * z, z], 1),
                        rng.standard_normal((n, 4)),
                        np.stack([rng.uniform(-1.5, -0.8, n), rng.uniform(-4.5, -3.5, n), rng.uniform(-4.5, -3.5, n)], 1)],
                       1).astype(np.float32)
    op = rng.uniform(0.0, 3.0, n).astype(np.float32)
    sc = scenes.Scene(t, np.full((n, 1, 3), 0.5, np.float32), op)
    f = _render(sc, cam, img)
    got = f.get(po.F_MAX_RADIUS).astype(np.float64)
    counts = f.get(po.F_INTERSECT_COUNTS)
    ratio_seen = []
    for g in range(n):
        if counts[g] == 0:
            continue
        _, raw = _pinhole_cov64(cam, t[g])
        cov = raw + 0.3 * np.eye(2)
        p = math.log(255.0 / (1.0 + math.exp(-float(op[g]))))
        ex, ey = math.sqrt(2 * p * cov[0, 0]), math.sqrt(2 * p * cov[1, 1])
        want = max(ex / img[0], ey / img[1])
        assert abs(got[g] - want) <= 1e-4 * want, (g, got[g], want, ex / img[1], ey / img[0])
        ratio_seen.append(max(ex / img[1], ey / img[0]) / want)
    assert len(ratio_seen) >= 30 and max(ratio_seen) > 1.5     # the swapped axes would differ


# ---- depth order behind a fisheye's camera plane ----------------------------------


def test_depth_order_with_splats_behind_the_camera_plane():
    img = (96, 96)
    model = vcam.KannalaBrandt4(0.01, -0.004, 0.001, -0.0002)
    cam_obj = vcam.Camera.from_focal(14.0, 14.0, img, model=model)
    cam = cam_obj.uniforms(img)
    assert float(cam.half_max_render_fov) > 2.0
    rng = np.random.default_rng(77)
    n = 1500
    d = rng.standard_normal((n, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    r = rng.uniform(2.0, 4.0, n)
    t = np.concatenate([d * r[:, None], rng.standard_normal((n, 4)), rng.uniform(-2.6, -1.8, (n, 3))],
                       1).astype(np.float32)
    sc = scenes.Scene(t, rng.uniform(0, 1, (n, 1, 3)).astype(np.float32), rng.uniform(0.0, 3.0, n).astype(np.float32))
    f = _render(sc, cam, img)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT).astype(np.int64)
    z64 = t[:, 2].astype(np.float64)                  # view space is world space for this camera
    zf = z64.astype(np.float32)
    assert (zf[gfc] < 0).sum() >= 20 and (zf[gfc] > 0).sum() >= 100
    # keys are view z (sign included) within 2 ulp
    key = f.get(po.F_DEPTHS).astype(np.float64)
    np.testing.assert_array_less(np.abs(key - zf[gfc]), 2.0 * np.spacing(np.abs(zf[gfc])).astype(np.float64) + 1e-30)
    # within every tile: the stable order of the raw bits of f32(z64)
    tile = f.get(po.F_ISECT_TILE).astype(np.int64)
    gid = f.get(po.F_ISECT_GID).astype(np.int64)
    bits = zf.view(np.uint32).astype(np.int64)
    want = np.lexsort((gid, bits[gid], tile))
    # the seed leaves no two splats of a tile within 8 ulp of each other, so f32(z64) and the key order agree
    same = tile[want][1:] == tile[want][:-1]
    gap = np.abs(np.diff(zf[gid[want]].astype(np.float64)))[same]
    assert (gap > 8 * np.spacing(np.abs(zf[gid[want]][1:]))[same]).all()
    np.testing.assert_array_equal(want, np.arange(len(tile)))
    neg_after_pos = 0
    for tt in np.unique(tile):
        zs = zf[gid[tile == tt]]
        if (zs < 0).any() and (zs > 0).any():
            assert (np.nonzero(zs < 0)[0].min() > np.nonzero(zs > 0)[0].max())
            neg_after_pos += 1
    assert neg_after_pos >= 5
