"""Pins the oracle's render path (projection, binning, compositing, VJP) with
checks that do not restate its formulas:

* tiled compositing equals a brute-force composite of every pixel over the
  whole depth-sorted visible list, bit for bit (binning drops nothing);
* the tile-hit test is conservative: every pixel centre that reaches the
  alpha cutoff lies in a tile its splat was emitted to;
* compositing matches a float64 textbook front-to-back "over" with the
  reference's skip/stop rules (kernels/rasterize.rs:309-396);
* the reference's invariance tests (src/tests/mod.rs: hidden splats 411,
  culled prefix 456, zero quaternions 772, mega stress 496);
* gradients agree with central differences of the forward along random
  directions (crates/splat-brush/src/fixture.rs:319-374 protocol, smooth
  cutoff), for a pinhole and a Kannala-Brandt-4 camera;
* the refine weight dominates the 2-D mean gradient it sums the norms of.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from vauss_amd import camera as vcam
from vauss_amd import scenes

KB4_MODEL = vcam.KannalaBrandt4(0.02, -0.01, 0.005, -0.001)


def _render(scene, cam, img, flags=po.FLAG_BWD_INFO, background=(0.0, 0.0, 0.0)):
    return po.render_forward(cam, img, scene.transforms, scene.sh_coeffs, scene.raw_opacities, flags=flags,
                             background=background)


def _cases():
    return [
        ("pinhole", scenes.rng_scene(3000, 1.5, (-2.5, 0.0), (-1.0, 3.0), 0xA11CE), (128, 96), None),
        ("kb4", scenes.rng_scene(2000, 1.5, (-2.5, -0.5), (-1.0, 3.0), 0xB0B), (96, 96), KB4_MODEL),
        ("large", scenes.rng_scene(400, 0.8, (-0.5, 1.0), (-2.0, 0.0), 0xC0DE), (80, 64), None),
    ]


@pytest.mark.parametrize("name,scene,img,model", _cases(), ids=[c[0] for c in _cases()])
def test_tiled_composite_equals_brute_force(name, scene, img, model):
    cam = scenes.test_camera(img, fov=0.5, model=model).uniforms(img)
    tiled = _render(scene, cam, img).get(po.F_OUT_IMG)
    brute = _render(scene, cam, img, po.FLAG_BWD_INFO | po.FLAG_BRUTE_FORCE).get(po.F_OUT_IMG)
    assert tiled.max() > 0.05
    np.testing.assert_array_equal(tiled.view(np.uint32), brute.view(np.uint32))


def _pixel_sigma_alpha(proj, img):
    """float64 sigma and alpha of every (visible splat, pixel centre) pair."""
    w, h = img
    yy, xx = np.mgrid[0:h, 0:w]
    px = xx.ravel() + 0.5
    py = yy.ravel() + 0.5
    x, y, c00, c01, c11, op = (proj[:, i:i + 1].astype(np.float64) for i in range(6))
    dx = px[None] - x
    dy = py[None] - y
    sig = 0.5 * (c00 * dx * dx + c11 * dy * dy) + c01 * dx * dy
    return sig, np.minimum(0.999, op * np.exp(-sig))


@pytest.mark.parametrize("name,scene,img,model", _cases(), ids=[c[0] for c in _cases()])
def test_tile_hit_test_is_conservative(name, scene, img, model):
    cam = scenes.test_camera(img, fov=0.5, model=model).uniforms(img)
    f = _render(scene, cam, img)
    proj = f.get(po.F_PROJECTED)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    tile_bw = (img[0] + 15) // 16
    hit = set(zip(f.get(po.F_ISECT_TILE).tolist(), f.get(po.F_ISECT_GID).tolist()))
    sig, alpha = _pixel_sigma_alpha(proj, img)
    w = img[0]
    need = (sig >= 0) & (alpha >= (1.0 / 255.0) * (1 + 1e-4))
    ci, pi = np.nonzero(need)
    tiles = (pi // w // 16) * tile_bw + (pi % w) // 16
    missing = [(int(t), int(gfc[c])) for c, t in zip(ci, tiles) if (int(t), int(gfc[c])) not in hit]
    assert not missing, missing[:10]
    # and the per-splat counts are the number of emitted tiles
    counts = f.get(po.F_INTERSECT_COUNTS)
    np.testing.assert_array_equal(np.bincount(f.get(po.F_ISECT_GID), minlength=scene.num_splats), counts)


def _rect_min_sigma(mx, my, a, b, c, x0, y0, x1, y1):
    """float64 minimum of sigma = (a dx^2 + c dy^2)/2 + b dx dy (d = p - mean) over
    the rectangle [x0, x1] x [y0, y1], for positive-definite conics: 0 when the
    mean lies inside, otherwise the least of the four edges' minima (sigma is
    convex along each edge, so each edge minimum is its clamped stationary
    point).  All arguments broadcast."""
    def edge(u, lo, hi, p, q, r):
        # sigma(u, t) = p u^2 / 2 + q u t + r t^2 / 2 on t in [lo, hi]
        t = np.clip(-q * u / r, lo, hi)
        return 0.5 * p * u * u + q * u * t + 0.5 * r * t * t
    ux0, ux1, uy0, uy1 = x0 - mx, x1 - mx, y0 - my, y1 - my
    m = np.minimum.reduce([edge(ux0, uy0, uy1, a, b, c), edge(ux1, uy0, uy1, a, b, c),
                           edge(uy0, ux0, ux1, c, b, a), edge(uy1, ux0, ux1, c, b, a)])
    inside = (ux0 <= 0) & (ux1 >= 0) & (uy0 <= 0) & (uy1 >= 0)
    return np.where(inside, 0.0, m)


def _view_z64(cam, transforms):
    """float64 view-space z of every splat mean: row 2 of the 3x4 world-to-camera
    matrix (column-major in vs_camera.viewmat) applied to (x, y, z, 1)."""
    vm = np.array(cam.viewmat, np.float64).reshape(4, 3).T
    means = transforms[:, 0:3].astype(np.float64)
    return means @ vm[2, :3] + vm[2, 3]


def _pin_cases():
    return _cases() + [("c1", scenes.scene_c1(), (256, 256), None)]


@pytest.mark.parametrize("name,scene,img,model", _pin_cases(), ids=[c[0] for c in _pin_cases()])
def test_tile_hits_equal_exact_rectangle_test(name, scene, img, model):
    """Each (tile, splat) pair the oracle emits, and each it does not, against a
    float64 exact ellipse-rectangle test: the minimum of sigma over the tile's
    pixel rectangle [16 tx, 16 tx + 16] x [16 ty, 16 ty + 16] against
    ln(255 opacity) (kernels/helpers.rs:254-314 decide the same set).  Pairs whose
    minimum lies within 1e-4 (relative) of the threshold may go either way."""
    if name == "c1":
        cam = scenes.workload("c1").cameras[0].uniforms(img)
    else:
        cam = scenes.test_camera(img, fov=0.5, model=model).uniforms(img)
    f = _render(scene, cam, img)
    proj = f.get(po.F_PROJECTED).astype(np.float64)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT).astype(np.int64)
    tbw, tbh = (img[0] + 15) // 16, (img[1] + 15) // 16
    tx, ty = np.meshgrid(np.arange(tbw), np.arange(tbh))
    tx, ty = tx.ravel().astype(np.float64), ty.ravel().astype(np.float64)
    x, y, c00, c01, c11, op = (proj[:, i:i + 1] for i in range(6))
    power = np.log(255.0 * op)
    smin = _rect_min_sigma(x, y, c00, c01, c11, 16 * tx[None], 16 * ty[None], 16 * tx[None] + 16, 16 * ty[None] + 16)
    exact = smin <= power                                           # [V, T]
    emitted = np.zeros_like(exact)
    comp_of = np.full(scene.num_splats, -1, np.int64)
    comp_of[gfc] = np.arange(len(gfc))
    emitted[comp_of[f.get(po.F_ISECT_GID).astype(np.int64)], f.get(po.F_ISECT_TILE).astype(np.int64)] = True
    boundary = np.abs(smin - power) <= 1e-4 * np.maximum(np.abs(power), 1.0)
    wrong = (exact != emitted) & ~boundary
    assert emitted.sum() > 1000 and (exact & ~emitted).sum() + (emitted & ~exact).sum() <= boundary.sum()
    assert not wrong.any(), [(int(gfc[c]), int(t), bool(emitted[c, t])) for c, t in zip(*np.nonzero(wrong))][:10]
    # and every splat's count is its number of emitted tiles
    counts = f.get(po.F_INTERSECT_COUNTS)
    np.testing.assert_array_equal(counts[gfc], emitted.sum(axis=1))


@pytest.mark.parametrize("name,scene,img,model", _pin_cases(), ids=[c[0] for c in _pin_cases()])
def test_depth_keys_are_view_z(name, scene, img, model):
    """The depth key (render.rs:689-694) is view-space z: each visible splat's
    key is within 2 ulp of the f32 rounding of the float64 (W x + t).z, and the
    sorted list is ordered by it within every tile."""
    if name == "c1":
        cam = scenes.workload("c1").cameras[0].uniforms(img)
    else:
        cam = scenes.test_camera(img, fov=0.5, model=model).uniforms(img)
    f = _render(scene, cam, img)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT).astype(np.int64)
    z64 = _view_z64(cam, scene.transforms)
    key = f.get(po.F_DEPTHS)
    ref = z64[gfc].astype(np.float32)
    ulp = np.spacing(np.abs(ref))
    assert (ref > 0).all()
    np.testing.assert_array_less(np.abs(key.astype(np.float64) - ref.astype(np.float64)), 2.0 * ulp + 1e-30)
    tile = f.get(po.F_ISECT_TILE).astype(np.int64)
    zs = z64[f.get(po.F_ISECT_GID).astype(np.int64)]
    same = tile[1:] == tile[:-1]
    dz = zs[1:] - zs[:-1]
    tol = 4.0 * np.spacing(np.abs(zs[1:]).astype(np.float32)).astype(np.float64)
    assert (dz[same] >= -tol[same]).all()


def test_composite_matches_float64_over():
    img = (40, 32)
    scene = scenes.rng_scene(60, 0.9, (-2.3, -1.0), (-1.0, 2.0), 0x5151)
    # DC terms in [-3, 1]: some colours come out negative and must be clamped at 0
    sh = (scene.sh_coeffs * np.float32(4.0) - np.float32(3.0)).astype(np.float32)
    scene = scenes.Scene(scene.transforms, sh, scene.raw_opacities)
    cam = scenes.test_camera(img, fov=0.6, position=(0.0, 0.0, -3.0)).uniforms(img)
    bg = (0.2, 0.4, 0.6)
    f = _render(scene, cam, img, background=bg)
    out = f.get(po.F_OUT_IMG).reshape(-1, 4).astype(np.float64)
    proj = f.get(po.F_PROJECTED).astype(np.float64)
    # front to back by float64 view z (not the oracle's own keys), ties by id
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    z64 = _view_z64(cam, scene.transforms)[gfc.astype(np.int64)]
    assert len(np.unique(z64)) == len(z64)
    order = np.lexsort((gfc, z64))
    sig, alpha = _pixel_sigma_alpha(proj[order], img)
    assert (proj[:, 6:9] < 0).any()
    rgb = np.maximum(proj[order][:, 6:9], 0.0)
    npix = img[0] * img[1]
    ref = np.zeros((npix, 4))
    for p in range(npix):
        T, C = 1.0, np.zeros(3)
        for j in range(len(order)):
            a = alpha[j, p]
            if sig[j, p] < 0 or a < 1.0 / 255.0:
                continue
            nt = T * (1 - a)
            if nt <= 1e-4:
                break
            C += rgb[j] * a * T
            T = nt
        ref[p, :3] = C + T * np.array(bg)
        ref[p, 3] = 1 - T
    assert out[:, 3].max() > 0.5
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-5)


def test_hidden_splats_do_not_perturb_render():
    img = (128, 128)
    cam = scenes.test_camera(img).uniforms(img)
    visible = scenes.rng_scene(3000, 1.5, (-2.5, 0.0), (0.0, 3.0), 0xBEEF)
    hidden = scenes.rng_scene(6000, 1.0, (-1.0, 1.0), (-20.0, -20.0), 0xDEAD)
    t = hidden.transforms.copy()
    t[1::3, 0:3] = (0.0, 0.0, -1000.0)       # behind the camera
    t[2::3, 0:3] = (1e6, 1e6, 10.0)          # far off-screen
    hidden = scenes.Scene(t, hidden.sh_coeffs, hidden.raw_opacities)
    a = _render(visible, cam, img)
    b = _render(visible.concat(hidden), cam, img)
    assert b.info.num_visible == a.info.num_visible
    np.testing.assert_array_equal(a.get(po.F_OUT_IMG), b.get(po.F_OUT_IMG))


def test_culled_prefix_does_not_perturb_render():
    img = (128, 128)
    cam = scenes.test_camera(img).uniforms(img)
    visible = scenes.rng_scene(2000, 1.5, (-2.5, 0.0), (0.0, 3.0), 0xC0FFEE)
    prefix = scenes.rng_scene(20_000, 1.0, (-1.0, 1.0), (-20.0, -20.0), 0xF00D)
    a = _render(visible, cam, img)
    b = _render(prefix.concat(visible), cam, img)
    np.testing.assert_array_equal(a.get(po.F_OUT_IMG), b.get(po.F_OUT_IMG))
    # the visible splats keep their tile lists, shifted by the prefix length
    np.testing.assert_array_equal(a.get(po.F_ISECT_GID) + 20_000, b.get(po.F_ISECT_GID))


def test_zero_quaternion_splats_are_culled():
    img = (64, 64)
    cam = scenes.test_camera(img, position=(0.0, 0.0, -3.0)).uniforms(img)
    valid = scenes.rng_scene(500, 1.0, (-1.0, 1.0), (0.0, 2.0), 0xDEAD)
    t = valid.transforms.copy()
    t[:, 3:7] = 0.0
    with_zeros = valid.concat(scenes.Scene(t, valid.sh_coeffs, valid.raw_opacities))
    a = _render(valid, cam, img)
    b = _render(with_zeros, cam, img)
    assert b.info.num_visible == a.info.num_visible
    np.testing.assert_array_equal(a.get(po.F_OUT_IMG), b.get(po.F_OUT_IMG))


def test_non_finite_parameters_are_culled():
    """kernels/project_forward.rs:74-109: a NaN/Inf mean, scale or opacity culls the splat."""
    img = (64, 64)
    cam = scenes.test_camera(img, position=(0.0, 0.0, -3.0)).uniforms(img)
    valid = scenes.rng_scene(300, 1.0, (-1.5, 0.0), (0.0, 2.0), 0xF1F1)
    bad = scenes.rng_scene(4, 1.0, (-1.5, 0.0), (0.0, 2.0), 0xF2F2)
    t = bad.transforms.copy()
    o = bad.raw_opacities.copy()
    t[0, 0] = np.nan
    t[1, 8] = np.inf
    o[2] = np.nan
    t[3, 2] = np.inf
    a = _render(valid, cam, img)
    b = _render(valid.concat(scenes.Scene(t, bad.sh_coeffs, o)), cam, img)
    assert b.info.num_visible == a.info.num_visible
    np.testing.assert_array_equal(a.get(po.F_OUT_IMG), b.get(po.F_OUT_IMG))


def test_fullscreen_splats_drop_no_tile():
    """Scaled-down mega stress (src/tests/mod.rs:496-546): every tile receives alpha."""
    img = (128, 128)
    cam = scenes.test_camera(img).uniforms(img)
    scene = scenes.rng_scene(3000, 0.1, (3.5, 4.0), (-3.0, -1.5), 0x5EED)
    f = _render(scene, cam, img)
    alpha = f.get(po.F_OUT_IMG)[..., 3]
    tile_sums = alpha.reshape(8, 16, 8, 16).sum(axis=(1, 3))
    assert (tile_sums > 1e-3).all()
    # every visible splat covers every tile
    assert f.info.num_intersections == f.info.num_visible * 64


def test_sorted_order_is_tile_then_depth_then_id():
    img = (96, 80)
    scene = scenes.rng_scene(2500, 1.5, (-2.5, 0.0), (-1.0, 3.0), 0x0DE7)
    cam = scenes.test_camera(img).uniforms(img)
    f = _render(scene, cam, img)
    tile = f.get(po.F_ISECT_TILE).astype(np.int64)
    gid = f.get(po.F_ISECT_GID).astype(np.int64)
    depth_of = np.zeros(scene.num_splats, np.uint32)
    depth_of[f.get(po.F_GLOBAL_FROM_COMPACT)] = f.get(po.F_DEPTHS).view(np.uint32)
    keys = np.stack([tile, depth_of[gid].astype(np.int64), gid], axis=1)
    order = np.lexsort((keys[:, 2], keys[:, 1], keys[:, 0]))
    np.testing.assert_array_equal(order, np.arange(len(order)))
    ranges = f.get(po.F_TILE_OFFSETS).reshape(-1, 2)
    for t in range(ranges.shape[0]):
        lo, hi = ranges[t]
        assert (tile[lo:hi] == t).all()


def _fd_check(model, seed):
    img = (48, 40)
    wide = model is not None           # a strongly distorted wide lens exercises the KB4 terms
    scene = scenes.rng_scene(40, 2.0 if wide else 0.7, (-2.0 if wide else -2.3, -1.3 if wide else -1.6),
                             (-1.5, 0.5), seed)
    cam = scenes.test_camera(img, fov=1.8 if wide else 0.6, position=(0.0, 0.0, -3.0), model=model).uniforms(img)
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((img[1], img[0], 4)) / (img[0] * img[1])).astype(np.float32)
    flags = po.FLAG_BWD_INFO | po.FLAG_SMOOTH_CUTOFF

    def render(t, s, o):
        f = po.render_forward(cam, img, t, s, o, flags=flags)
        return float((f.get(po.F_OUT_IMG).astype(np.float64) * w).sum()), f

    _, base = render(scene.transforms, scene.sh_coeffs, scene.raw_opacities)
    g = base.backward(w)
    base_lists = [base.get(k) for k in (po.F_ISECT_TILE, po.F_ISECT_GID)]
    groups = [("means", 0, 3), ("quats", 3, 7), ("log_scales", 7, 10), ("sh", None, None), ("opacity", None, None)]
    checked = 0
    for _ in range(6):
        support = rng.choice(scene.num_splats, 3, replace=False)
        for name, a, b in groups:
            arrs = {"means": scene.transforms, "quats": scene.transforms, "log_scales": scene.transforms,
                    "sh": scene.sh_coeffs, "opacity": scene.raw_opacities}
            grads = {"means": g["v_transforms"], "quats": g["v_transforms"], "log_scales": g["v_transforms"],
                     "sh": g["v_sh"], "opacity": g["v_raw_opac"]}
            base_arr, grad = arrs[name], grads[name]
            d = np.zeros(base_arr.shape)
            if a is None:
                d[support] = rng.standard_normal(d[support].shape)
            else:
                d[support, a:b] = rng.standard_normal((3, b - a))
            d /= np.linalg.norm(d)
            analytic = float((grad.astype(np.float64) * d).sum())
            errors = []
            for eps in (3e-3, 1e-3):
                vals = []
                for sgn in (1.0, -1.0):
                    p = (base_arr.astype(np.float64) + sgn * eps * d).astype(np.float32)
                    t = p if name in ("means", "quats", "log_scales") else scene.transforms
                    s = p if name == "sh" else scene.sh_coeffs
                    o = p if name == "opacity" else scene.raw_opacities
                    val, f = render(t, s, o)
                    # a change of binning or depth order is a step, not a slope: not comparable
                    if any(not np.array_equal(f.get(k), ref) for k, ref in
                           zip((po.F_ISECT_TILE, po.F_ISECT_GID), base_lists)):
                        vals = None
                        break
                    vals.append(val)
                if vals is None:
                    break
                numerical = (vals[0] - vals[1]) / (2 * eps)
                errors.append(abs(analytic - numerical) - 0.02 * max(abs(analytic), abs(numerical)))
            if len(errors) < 2:
                continue
            checked += 1
            # f32 renders: the central difference carries ~5e-7 of rounding noise
            assert min(errors) <= 1.5e-6, (name, support, analytic, errors)
    assert checked >= 20


@pytest.mark.parametrize("model", [None, vcam.KannalaBrandt4(0.08, -0.05, 0.03, -0.02),
                                   vcam.RadialTangential8(-0.15, 0.06, -0.01, 0.05, 0.02, -0.005, 0.03, -0.02),
                                   vcam.ThinPrismFisheye(vcam.KannalaBrandt4(0.08, -0.05, 0.03, -0.02),
                                                         0.03, -0.02, 0.015, -0.015)],
                         ids=["pinhole", "kb4", "rt8", "tpf"])
@pytest.mark.parametrize("seed", [0x1234, 2])
def test_gradients_match_central_differences(model, seed):
    _fd_check(model, seed)


def test_refine_weight_dominates_the_mean_gradient():
    """v_refine = sum over pixels of |(g_x W, g_y H)| / max(a_final, 1e-5) with
    a_final <= 1, so by the triangle inequality it is at least the norm of the
    summed 2-D mean gradient scaled the same way (bwd/kernels/rasterize_backwards_planes.rs:579-593)."""
    img = (64, 48)
    scene = scenes.rng_scene(300, 1.0, (-2.5, -1.0), (-1.0, 2.0), 0x7E57)
    cam = scenes.test_camera(img, fov=0.6, position=(0.0, 0.0, -3.0)).uniforms(img)
    f = _render(scene, cam, img)
    rng = np.random.default_rng(1)
    g = f.backward((rng.standard_normal((img[1], img[0], 4)) / 1000).astype(np.float32))
    vc = g["v_combined"].astype(np.float64)
    lower = np.hypot(vc[:, 0] * img[0], vc[:, 1] * img[1])
    assert (vc[:, 9] >= lower * (1 - 1e-5) - 1e-12).all()
    assert (vc[:, 9] >= 0).all() and vc[:, 9].max() > 0
    np.testing.assert_allclose(g["v_refine"], vc[:, 9].astype(np.float32), rtol=1e-6)
    # culled splats get no gradient
    culled = f.get(po.F_INTERSECT_COUNTS) == 0
    assert np.all(g["v_transforms"][culled] == 0) and np.all(g["v_raw_opac"][culled] == 0)


def _quat_to_mat(q):
    w, x, y, z = q / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _project_closed_form(p, model, fx, fy, cx, cy):
    """Pixel position of a camera-space point: pinhole; Kannala-Brandt-4
    d(theta) = theta (1 + k1 theta^2 + k2 theta^4 + k3 theta^6 + k4 theta^8);
    OpenCV's rational radial + tangential model on (x/z, y/z); COLMAP's thin
    prism fisheye = KB4 + (2 p1 uv + p2 (r^2 + 2u^2) + sx1 r^2, ...) on (u, v) =
    (x/z, y/z)."""
    x, y, z = p
    if model is None:
        return np.array([fx * x / z + cx, fy * y / z + cy])
    if isinstance(model, vcam.RadialTangential8):
        m = model
        u, v = x / z, y / z
        r2 = u * u + v * v
        rad = (1 + m.k1 * r2 + m.k2 * r2 ** 2 + m.k3 * r2 ** 3) / (1 + m.k4 * r2 + m.k5 * r2 ** 2 + m.k6 * r2 ** 3)
        ud = u * rad + 2 * m.p1 * u * v + m.p2 * (r2 + 2 * u * u)
        vd = v * rad + 2 * m.p2 * u * v + m.p1 * (r2 + 2 * v * v)
        return np.array([fx * ud + cx, fy * vd + cy])
    kb = model.kb4 if isinstance(model, vcam.ThinPrismFisheye) else model
    r = np.hypot(x, y)
    th = np.arctan2(r, z)
    k = (kb.k1, kb.k2, kb.k3, kb.k4)
    t2 = th * th
    d = th * (1 + k[0] * t2 + k[1] * t2 ** 2 + k[2] * t2 ** 3 + k[3] * t2 ** 4)
    out = np.array([fx * d * x / r + cx, fy * d * y / r + cy])
    if isinstance(model, vcam.ThinPrismFisheye):
        m = model
        u, v = x / z, y / z
        r2 = u * u + v * v
        out += np.array([fx * (2 * m.p1 * u * v + m.p2 * (r2 + 2 * u * u) + m.sx1 * r2),
                         fy * (2 * m.p2 * u * v + m.p1 * (r2 + 2 * v * v) + m.sy1 * r2)])
    return out


RT8_MODEL = vcam.RadialTangential8(-0.15, 0.06, -0.01, 0.05, 0.02, -0.005, 0.03, -0.02)
TPF_MODEL = vcam.ThinPrismFisheye(vcam.KannalaBrandt4(0.02, -0.01, 0.005, -0.001), 0.03, -0.02, 0.015, -0.015)


@pytest.mark.parametrize("model", [None, KB4_MODEL, RT8_MODEL, TPF_MODEL], ids=["pinhole", "kb4", "rt8", "tpf"])
def test_projection_matches_closed_form(model):
    """Mean, conic, opacity and colour of each projected row against float64
    closed forms: mean = proj(W x + t); Sigma2D = J R S^2 R^T J^T + 0.3 I with J
    the projection's Jacobian (central differences); conic = Sigma2D^-1;
    opacity = sigmoid(logit); colour = sum_k Y_k(dir) c_k + 0.5."""
    img = (96, 80)
    cam_obj = scenes.test_camera(img, fov=0.9, position=(0.0, 0.0, -4.0), model=model)
    cam = cam_obj.uniforms(img)
    rng = np.random.default_rng(4)
    n = 40
    means = np.stack([rng.uniform(-0.8, 0.8, n), rng.uniform(-0.6, 0.6, n), rng.uniform(-0.5, 0.5, n)], 1)
    quats = rng.standard_normal((n, 4))
    log_s = rng.uniform(-3.5, -2.0, (n, 3))
    t = np.concatenate([means, quats, log_s], 1).astype(np.float32)
    sh = (rng.standard_normal((n, 16, 3)) * 0.2).astype(np.float32)
    op = rng.uniform(-1, 2, n).astype(np.float32)
    f = po.render_forward(cam, img, t, sh, op, flags=po.FLAG_BWD_INFO)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    rows = f.get(po.F_PROJECTED).astype(np.float64)
    assert len(gfc) == n
    fx, fy, cx, cy = (float(v) for v in (cam.fx, cam.fy, cam.cx, cam.cy))
    for row, g in zip(rows, gfc):
        pc = t[g, :3].astype(np.float64) + np.array([0.0, 0.0, 4.0])      # identity rotation, camera at z=-4
        mean2d = _project_closed_form(pc, model, fx, fy, cx, cy)
        np.testing.assert_allclose(row[:2], mean2d, rtol=0, atol=2e-3)
        J = np.zeros((2, 3))
        for i in range(3):
            h = np.zeros(3)
            h[i] = 1e-6
            J[:, i] = (_project_closed_form(pc + h, model, fx, fy, cx, cy) -
                       _project_closed_form(pc - h, model, fx, fy, cx, cy)) / 2e-6
        R = _quat_to_mat(t[g, 3:7].astype(np.float64))
        M = R @ np.diag(np.exp(t[g, 7:10].astype(np.float64)))
        cov = J @ M @ M.T @ J.T + 0.3 * np.eye(2)
        conic = np.linalg.inv(cov)
        got = np.array([[row[2], row[3]], [row[3], row[4]]])
        np.testing.assert_allclose(got, conic, rtol=0, atol=2e-4 * np.abs(conic).max())
        assert abs(row[5] - 1 / (1 + np.exp(-float(op[g])))) < 1e-6
        v = t[g, :3].astype(np.float64) - np.array([0.0, 0.0, -4.0])
        basis = po.sh_basis(3, (v / np.linalg.norm(v)).astype(np.float32)).astype(np.float64)
        color = basis @ sh[g].astype(np.float64) + 0.5
        np.testing.assert_allclose(row[6:9], color, rtol=0, atol=2e-5)


@pytest.mark.parametrize("model", [None, KB4_MODEL, vcam.RadialTangential8(-0.1, 0.15, -0.02, 0.05, 0.1, -0.01, 0.03, -0.02),
                                   TPF_MODEL], ids=["pinhole", "kb4", "rt8", "tpf"])
def test_covariance_path_of_the_mean_gradient(model):
    """The mean gradient carried by the conic alone (v_xy = 0): the derivative
    of the projection Jacobian in the EWA covariance, which each camera model's
    VJP writes out by hand (second derivatives of the distortion).  Checked
    against central differences of a float64 conic whose Jacobian is itself a
    central difference of the closed-form projection."""
    img = (96, 80)
    cam_obj = scenes.test_camera(img, fov=1.5, position=(0.0, 0.0, -4.0), model=model)
    cam = cam_obj.uniforms(img)
    fx, fy, cx, cy = (float(v) for v in (cam.fx, cam.fy, cam.cx, cam.cy))
    rng = np.random.default_rng(12)
    n = 24
    means = np.stack([rng.uniform(-2.0, 2.0, n), rng.uniform(-1.6, 1.6, n), rng.uniform(-0.5, 0.5, n)], 1)
    t = np.concatenate([means, rng.standard_normal((n, 4)), rng.uniform(-2.5, -1.5, (n, 3))], 1).astype(np.float32)
    f = po.render_forward(cam, img, t, np.zeros((n, 1, 3), np.float32), np.full(n, 2.0, np.float32))
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    vc = np.zeros((n, 10), np.float32)
    vc[:, 2:5] = rng.standard_normal((n, 3)).astype(np.float32)
    g = f.project_backward(vc)["v_transforms"][:, 0:3].astype(np.float64)

    def conic(g_, mean):
        pc = mean + np.array([0.0, 0.0, 4.0])
        J = np.zeros((2, 3))
        for i in range(3):
            h = np.zeros(3)
            h[i] = 1e-6
            J[:, i] = (_project_closed_form(pc + h, model, fx, fy, cx, cy) -
                       _project_closed_form(pc - h, model, fx, fy, cx, cy)) / 2e-6
        M = _quat_to_mat(t[g_, 3:7].astype(np.float64)) @ np.diag(np.exp(t[g_, 7:10].astype(np.float64)))
        c = np.linalg.inv(J @ M @ M.T @ J.T + 0.3 * np.eye(2))
        return np.array([c[0, 0], c[0, 1], c[1, 1]])

    assert len(gfc) >= 16
    for gi in gfc:
        m0 = t[gi, :3].astype(np.float64)
        num = np.zeros(3)
        for i in range(3):
            e = np.zeros(3)
            e[i] = 1e-4
            num[i] = vc[gi, 2:5].astype(np.float64) @ (conic(gi, m0 + e) - conic(gi, m0 - e)) / 2e-4
        assert np.all(np.abs(g[gi] - num) <= 3e-4 * np.abs(num).max() + 1e-6), (gi, g[gi], num)
