"""Pins the oracle's surfel (2DGS) render mode (kernels/helpers.rs:316-423,
kernels/rasterize.rs:181-364, bwd/kernels/rasterize_backwards_planes.rs:
266-480, bwd/kernels/project_backwards.rs:426-570) on the CPU.

* One surfel against a float64 ray-plane intersection built from the
  camera and the surfel's frame alone: each pixel ray meets the plane
  p + u s_u t_u + v s_v t_v at (u, v, z) (a 3x3 linear solve), the
  low-pass disk sits at the projected centre, sigma = min(u^2 + v^2,
  2 |pixel - centre|^2) / 2; the image's alpha, colour and all geometry
  channels (depth sum, median depth and its intersection index, normal sum,
  distortion moments) follow, within 1e-5.
* The binning ellipse is conservative: every pixel a surfel reaches (float64
  alpha >= 1/255) lies in a tile it was emitted to.
* Gradients of every parameter against central differences of full renders
  with the smooth cutoff, through colour, alpha and every geometry channel,
  rejecting directions that change the binning or a pixel's median
  contributor (the median depth is piecewise constant in that choice).
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from vauss_amd import camera as vcam
from vauss_amd import scenes

IMG = (64, 48)
C0 = 0.2820948


def _quat_to_mat(q):
    w, x, y, z = q / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _cam(img=IMG, fov=0.9, position=(0.4, -0.3, -3.0)):
    rot = vcam.look_at_rotation(position, (0.0, 0.0, 0.0))
    return vcam.Camera(fov, fov, (0.5, 0.5), position, rot).uniforms(img)


def _surfel64(cam, t, img):
    """Per pixel (alpha-free) sigma, z and validity of one surfel, float64."""
    vm = np.array(cam.viewmat[:], np.float64)
    R, tr = vm[:9].reshape(3, 3).T, vm[9:12]
    fx, fy, cx, cy = (float(v) for v in (cam.fx, cam.fy, cam.cx, cam.cy))
    pc = R @ t[:3] + tr
    Rq = R @ _quat_to_mat(t[3:7])
    s = np.exp(t[7:10])
    a, b = Rq[:, 0] * s[0], Rq[:, 1] * s[1]
    n = Rq[:, 2] * (-1.0 if Rq[:, 2] @ pc > 0 else 1.0)
    w, h = img
    ys, xs = np.mgrid[0:h, 0:w]
    px, py = xs + 0.5, ys + 0.5
    d = np.stack([(px - cx) / fx, (py - cy) / fy, np.ones_like(px)], -1)
    A = np.zeros(d.shape[:2] + (3, 3))
    A[..., :, 0] = a
    A[..., :, 1] = b
    A[..., :, 2] = -d
    sol = np.linalg.solve(A, np.broadcast_to(-pc, d.shape)[..., None])[..., 0]
    u, v, z = sol[..., 0], sol[..., 1], sol[..., 2]
    centre = np.array([fx * pc[0] / pc[2] + cx, fy * pc[1] / pc[2] + cy])
    s2d = 2 * ((px - centre[0]) ** 2 + (py - centre[1]) ** 2)
    sigma = 0.5 * np.minimum(u * u + v * v, s2d)
    return sigma, z, z >= 0.01, n


@pytest.mark.parametrize("surface", [False, True])
def test_single_surfel_matches_float64(surface):
    cam = _cam()
    t = np.array([[0.1, -0.05, 0.2, 0.8, 0.3, -0.4, 0.2, np.log(0.35), np.log(0.2), np.log(0.05)]], np.float32)
    sh = np.array([[[0.6, -0.2, 0.3]]], np.float32)
    op = np.array([1.2], np.float32)
    flags = po.FLAG_BWD_INFO | po.FLAG_SURFEL | (po.FLAG_SURFACE if surface else 0)
    f = po.render_forward(cam, IMG, t, sh, op, flags=flags)
    out = f.get(po.F_OUT_IMG).astype(np.float64)
    assert out.shape == IMG[::-1] + (12,)
    sigma, z, valid, n = _surfel64(cam, t[0].astype(np.float64), IMG)
    opac = 1.0 / (1.0 + np.exp(-1.2))
    alpha = np.minimum(0.999, opac * np.exp(-sigma))
    live = valid & (alpha >= 1.0 / 255.0)
    sure = np.abs(alpha - 1.0 / 255.0) > 1e-4          # away from the cutoff's f32 boundary
    assert live.sum() > 200 and (~live).sum() > 200
    a = np.where(live, alpha, 0.0)
    np.testing.assert_allclose(out[..., 3][sure], a[sure], atol=1e-5)
    col = C0 * sh[0, 0].astype(np.float64) + 0.5
    for c in range(3):
        np.testing.assert_allclose(out[..., c][sure], (col[c] * a)[sure], atol=1e-5)
    m = lambda zz: 100.0 / (100.0 - 0.2) * (1.0 - 0.2 / np.maximum(zz, 0.2))
    sl = sure & live
    np.testing.assert_allclose(out[..., 4][sl], (z * a)[sl], rtol=2e-5, atol=1e-5)
    np.testing.assert_allclose(out[..., 5][sl], z[sl], rtol=2e-5)
    for k in range(3):
        np.testing.assert_allclose(out[..., 6 + k][sl], (n[k] * a)[sl], atol=1e-5)
    np.testing.assert_allclose(out[..., 9][sl], (m(z) * a)[sl], atol=1e-5)
    np.testing.assert_allclose(out[..., 10][sl], (m(z) ** 2 * a)[sl], atol=1e-5)
    # the median's intersection index is the splat's slot in its tile's list
    ranges = f.get(po.F_TILE_OFFSETS).reshape(-1, 2)
    tbw = (IMG[0] + 15) // 16
    ys, xs = np.nonzero(sl)
    tiles = (ys // 16) * tbw + xs // 16
    np.testing.assert_array_equal(out[ys, xs, 11].astype(np.float32).view(np.uint32), ranges[tiles, 0])
    dead = sure & ~live
    assert np.all(out[..., 3][dead] == 0.0) and np.all(out[..., 11][dead].astype(np.float32).view(np.uint32) == 0xFFFFFFFF)


def test_binning_is_conservative():
    cam = _cam(img=(96, 80), fov=1.0)
    sc = scenes.rng_scene(60, 0.8, (-2.5, -1.2), (-1.0, 2.0), 0x5EF)
    f = po.render_forward(cam, (96, 80), sc.transforms, sc.sh_coeffs, sc.raw_opacities,
                          flags=po.FLAG_BWD_INFO | po.FLAG_SURFEL)
    gfc = f.get(po.F_GLOBAL_FROM_COMPACT)
    hit = set(zip(f.get(po.F_ISECT_TILE).tolist(), f.get(po.F_ISECT_GID).tolist()))
    tbw = (96 + 15) // 16
    checked = 0
    for g in range(sc.num_splats):
        sigma, z, valid, _ = _surfel64(cam, sc.transforms[g].astype(np.float64), (96, 80))
        opac = 1.0 / (1.0 + np.exp(-float(sc.raw_opacities[g])))
        alpha = np.minimum(0.999, opac * np.exp(-sigma))
        need = valid & (alpha >= (1.0 / 255.0) * (1 + 1e-4))
        if not need.any():
            continue
        assert g in set(gfc.tolist()), g
        ys, xs = np.nonzero(need)
        for tile in set(((ys // 16) * tbw + xs // 16).tolist()):
            assert (tile, g) in hit, (g, tile)
        checked += 1
    assert checked > 30


@pytest.mark.parametrize("surface", [False, True])
def test_median_criteria_on_a_stack(surface):
    """Three surfels facing the camera at increasing depths: the median depth
    is the last contributor reached with transmittance above 1/2 (training), or
    the first one where sum(alpha + 0.1 G) exceeds 0.6 (the surface criterion,
    until then the transmittance rule), per pixel in float64."""
    cam = _cam(position=(0.0, 0.0, -3.0))
    vm = np.array(cam.viewmat[:], np.float64)
    R = vm[:9].reshape(3, 3).T
    # a quaternion whose rotation equals the camera's: the surfel plane faces the camera
    q = vcam.quat_from_matrix(R.T)                     # (x, y, z, w)
    qw = np.array([q[3], q[0], q[1], q[2]])
    depths = [-0.3, 0.0, 0.3]
    t = np.array([[0.02 * i, -0.01 * i, d, *qw, np.log(0.3), np.log(0.25), np.log(0.1)] for i, d in enumerate(depths)],
                 np.float32)
    sh = np.zeros((3, 1, 3), np.float32)
    op = np.array([-0.3, 0.4, 1.5], np.float32)
    flags = po.FLAG_BWD_INFO | po.FLAG_SURFEL | (po.FLAG_SURFACE if surface else 0)
    f = po.render_forward(cam, IMG, t, sh, op, flags=flags)
    out = f.get(po.F_OUT_IMG).astype(np.float64)
    per = [_surfel64(cam, t[i].astype(np.float64), IMG) for i in range(3)]
    T = np.ones(IMG[::-1])
    so = np.zeros(IMG[::-1])
    found = np.zeros(IMG[::-1], bool)
    median = np.zeros(IMG[::-1])
    border = np.zeros(IMG[::-1], bool)
    for i in range(3):                                   # already in depth order
        sigma, z, valid, _ = per[i]
        opac = 1.0 / (1.0 + np.exp(-float(op[i])))
        G = np.exp(-sigma)
        alpha = np.minimum(0.999, opac * G)
        live = valid & (alpha >= 1.0 / 255.0)
        border |= np.abs(alpha - 1.0 / 255.0) < 1e-4
        if surface:
            so = np.where(live, so + alpha + 0.1 * G, so)
            border |= live & (np.abs(so - 0.6) < 1e-4)
            take = live & ~found & ((so > 0.6) | (T > 0.5))
            median = np.where(take, z, median)
            found |= take & (so > 0.6)
        else:
            take = live & (T > 0.5)
            median = np.where(take, z, median)
        border |= live & (np.abs(T - 0.5) < 1e-4)
        T = np.where(live, T * (1 - alpha), T)
    ok = ~border
    assert ok.mean() > 0.95
    np.testing.assert_allclose(out[..., 5][ok], median[ok], rtol=2e-5, atol=1e-6)
    # the two rules disagree on a good share of the covered pixels
    assert len(np.unique(np.round(median[ok & (median > 0)], 3))) >= 2


def test_low_pass_dominated_gradients():
    """Surfels far below a pixel: the low-pass disk around the projected
    centre carries the coverage, so the gradient flows through (M02, M12) / M22."""
    # the scales barely matter here; the means carry the centre's gradient
    checked = _fd_surfel(21, log_scale=(-7.0, -6.0), steps=(3e-4, 1e-4), skip=("log_scales",), by_group=True)
    assert sum(checked.values()) >= 10 and checked["means"] >= 3, checked


def _fd_surfel(seed, log_scale=(-2.2, -1.4), steps=(1e-3, 3e-4), skip=(), by_group=False):
    img = (48, 40)
    cam = _cam(img=img, fov=0.8, position=(0.3, -0.2, -2.6))
    sc = scenes.rng_scene(30, 0.6, log_scale, (-1.5, 0.5), seed)
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((img[1], img[0], 12)) / (img[0] * img[1])).astype(np.float32)
    w[..., 4:6] *= 0.3                 # depths are ~3x larger than the other channels
    w[..., 11] = 0.0                   # the median's id is an index, not a value
    flags = po.FLAG_BWD_INFO | po.FLAG_SMOOTH_CUTOFF | po.FLAG_SURFEL

    def render(t, s, o):
        f = po.render_forward(cam, img, t, s, o, flags=flags)
        out = f.get(po.F_OUT_IMG)
        # channel 11 holds an index's bits (NaN patterns): it takes no part in the loss
        return float((out[..., :11].astype(np.float64) * w[..., :11]).sum()), f, out[..., 11].view(np.uint32).copy()

    _, base, base_med = render(sc.transforms, sc.sh_coeffs, sc.raw_opacities)
    g = base.backward(w)
    assert g["v_combined"].shape == (sc.num_splats, 17)
    base_lists = [base.get(k) for k in (po.F_ISECT_TILE, po.F_ISECT_GID)]
    groups = [("means", 0, 3), ("quats", 3, 7), ("log_scales", 7, 10), ("sh", None, None), ("opacity", None, None)]
    checked = 0
    per_group = {name: 0 for name, _, _ in groups}
    for _ in range(10):
        support = rng.choice(sc.num_splats, 3, replace=False)
        for name, a, b in groups:
            if name in skip:
                continue
            arrs = {"means": sc.transforms, "quats": sc.transforms, "log_scales": sc.transforms,
                    "sh": sc.sh_coeffs, "opacity": sc.raw_opacities}
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
            # sigma = min(s3d, s2d) / 2 has a kink where the low-pass takes over:
            # the central difference converges only at small steps
            for eps in steps:
                vals = []
                for sgn in (1.0, -1.0):
                    p = (base_arr.astype(np.float64) + sgn * eps * d).astype(np.float32)
                    t = p if name in ("means", "quats", "log_scales") else sc.transforms
                    s = p if name == "sh" else sc.sh_coeffs
                    o = p if name == "opacity" else sc.raw_opacities
                    val, f, med = render(t, s, o)
                    # a change of binning, depth order or median contributor is a step, not a slope
                    if not np.array_equal(med, base_med) or any(
                            not np.array_equal(f.get(k), ref) for k, ref in
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
            per_group[name] += 1
            assert min(errors) <= 3e-6, (name, support, analytic, errors)
    return per_group if by_group else checked


@pytest.mark.parametrize("seed", [11, 12])
def test_surfel_gradients_match_central_differences(seed):
    assert _fd_surfel(seed) >= 15
