"""GPU parity of the render path against the CPU oracle on identical seeded inputs.

Bars (the contract of this build):
  * tile-intersection counts, the sorted (tile, depth, splat) order, tile
    ranges, projected rows and aux outputs: bit for bit;
  * forward RGBA (and geometry channels): within 1e-4 absolute (expected
    bit-exact: the kernels follow the oracle's arithmetic contract);
  * per-splat gradients: within 1e-3 relative / 1e-5 absolute, and within
    1e-3 of the largest gradient of the same parameter group (f32 atomics
    reorder the per-splat sums).
"""
import numpy as np
import pytest
import torch

import vauss_amd as va
from vauss_amd import scenes
from oracle import pyoracle as po
from tests._util import circle_mask, gpu_state_arrays, l1_cotangent_np, to_gpu

pytestmark = pytest.mark.gpu

CASES = [("c1", None, 0), ("c2", 20_000, 0), ("c3", 20_000, 3), ("c4", 20_000, 0), ("c5", 20_000, 0)]


def _render_both(cfg, n, view, pass_=va.RasterPass.BACKWARD, background=(0.0, 0.0, 0.0)):
    w = scenes.workload(cfg, n)
    cam = w.cameras[view].uniforms(w.img_size)
    t, s, o = to_gpu(w.scene)
    print(f"[case] {cfg} n={w.scene.num_splats} view={view} pass={pass_.name}", flush=True)
    out = va.render(cam, w.img_size, t, s, o, background=background, pass_=pass_)
    flags = po.FLAG_BWD_INFO if pass_.bwd_info() else 0
    if pass_.geometry():
        flags |= po.FLAG_GEOMETRY
    if pass_ == va.RasterPass.BACKWARD_SMOOTH_CUTOFF:
        flags |= po.FLAG_SMOOTH_CUTOFF
    ref = po.render_forward(cam, w.img_size, w.scene.transforms, w.scene.sh_coeffs, w.scene.raw_opacities,
                            background=background, flags=flags)
    return w, (t, s, o), out, ref


def _check_forward(out, ref, gpu):
    info = ref.info
    assert out.aux.num_visible == info.num_visible
    assert out.aux.num_intersections == info.num_intersections
    # per-splat tile counts, bit for bit
    np.testing.assert_array_equal(gpu["counts"], ref.get(po.F_INTERSECT_COUNTS))
    # sorted intersection order: tile, then raw depth bits, then splat id
    np.testing.assert_array_equal(gpu["tile"], ref.get(po.F_ISECT_TILE))
    np.testing.assert_array_equal(gpu["gid"], ref.get(po.F_ISECT_GID))
    np.testing.assert_array_equal(gpu["ranges"], ref.get(po.F_TILE_OFFSETS))
    # projected rows of the visible splats
    gfc = ref.get(po.F_GLOBAL_FROM_COMPACT)
    proj = ref.get(po.F_PROJECTED)
    got = np.concatenate([gpu["proj_a"][gfc], gpu["proj_b"][gfc], gpu["proj_c"][gfc, None]], axis=1)
    got = got[:, [0, 1, 2, 3, 4, 5, 6, 7, 8]]
    np.testing.assert_array_equal(got.view(np.uint32), proj.view(np.uint32))
    # the row's footprint exponent, logf(255 opacity), which emission reads back
    np.testing.assert_array_equal(gpu["proj_power"][gfc].view(np.uint32),
                                  po.logf(proj[:, 5] * np.float32(255.0)).view(np.uint32))
    # the depth key of every visible splat is its raw view-z bits
    np.testing.assert_array_equal(gpu["depth_bits"][gfc], ref.get(po.F_DEPTHS).view(np.uint32))
    # aux outputs
    np.testing.assert_array_equal(out.aux.opacities.cpu().numpy().view(np.uint32), ref.get(po.F_OPACITIES).view(np.uint32))
    np.testing.assert_array_equal(out.aux.max_radius.cpu().numpy().view(np.uint32), ref.get(po.F_MAX_RADIUS).view(np.uint32))


@pytest.mark.parametrize("cfg,n,view", CASES)
def test_forward_parity(cfg, n, view):
    w, _, out, ref = _render_both(cfg, n, view)
    gpu = gpu_state_arrays(out)
    _check_forward(out, ref, gpu)
    img = out.out_img.cpu().numpy()
    rimg = ref.get(po.F_OUT_IMG)
    diff = np.abs(img - rimg)
    assert diff.max() <= 1e-4, f"max |rgba diff| {diff.max()}"
    assert np.array_equal(img.view(np.uint32), rimg.view(np.uint32)), f"{(diff > 0).sum()} channels differ in the last bits"
    np.testing.assert_array_equal(out.aux.visible.cpu().numpy(), ref.get(po.F_VISIBLE))
    np.testing.assert_array_equal(out.aux.tile_offsets.cpu().numpy().view(np.uint32), ref.get(po.F_TILE_OFFSETS_SHRUNK))


def _check_grads(got, want, name, rtol=1e-3, atol=1e-5, group_rtol=1e-3):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    if bad.any():
        flat = np.argsort(-(err / (atol + rtol * np.abs(want))).ravel())[:4]
        worst = [(np.unravel_index(i, err.shape), float(got.ravel()[i]), float(want.ravel()[i])) for i in flat]
        raise AssertionError(f"{name}: {bad.sum()} entries exceed {rtol:g} rel / {atol:g} abs (max err {err.max():.3e}); "
                             f"worst (index, gpu, oracle): {worst}")
    if group_rtol is None:
        return
    scale = np.abs(want).max(axis=0, keepdims=True) if want.ndim > 1 else np.abs(want).max()
    tight = err > rtol * np.abs(want) + group_rtol * scale
    assert not tight.any(), f"{name}: {tight.sum()} entries exceed {group_rtol:g} of the group maximum (max err {err.max():.3e})"


def _check_param_grads(g, rg, ref, vc, exclude=None):
    """Dense parameter gradients, end to end and per stage.

    End to end (GPU raster + projection VJPs vs the oracle's) at the contract
    bar, 1e-3 relative / 1e-5 absolute.  The projection VJP can amplify the
    ~1e-6 relative atomic-order differences of v_combined by orders of
    magnitude where its terms cancel (a splat with |v_conic| ~ 1 and
    |v_quat| ~ 1e-6), so the projection stage is also checked on its own: the
    oracle's projection VJP applied to the GPU's own v_combined must agree to
    1e-5 relative / 1e-3 of the group maximum.  `exclude` (a boolean row mask)
    drops rows from the end-to-end check only: rows whose gradients the
    oracle itself moves past the bar under 1e-6 relative noise in v_combined
    (see ill_conditioned_rows)."""
    vt = g.v_transforms.cpu().numpy()
    vs = g.v_coeffs.cpu().numpy().reshape(len(vt), -1)
    vo = g.v_raw_opac.cpu().numpy()
    vr = g.v_refine_weight.cpu().numpy()
    assert np.isfinite(vt).all() and np.isfinite(vs).all()
    keep = slice(None) if exclude is None else ~exclude
    for got, want, name in ((vt[:, 0:3], rg["v_transforms"][:, 0:3], "v_means"),
                            (vt[:, 3:7], rg["v_transforms"][:, 3:7], "v_quats"),
                            (vt[:, 7:10], rg["v_transforms"][:, 7:10], "v_log_scales"),
                            (vo, rg["v_raw_opac"], "v_raw_opacity"),
                            (vs, rg["v_sh"].reshape(len(vt), -1), "v_sh"),
                            (vr, rg["v_refine"], "v_refine_weight")):
        _check_grads(got[keep], want[keep], name, group_rtol=None)
    pg = ref.project_backward(vc)
    for got, want, name in ((vt[:, 0:3], pg["v_transforms"][:, 0:3], "v_means (projection stage)"),
                            (vt[:, 3:7], pg["v_transforms"][:, 3:7], "v_quats (projection stage)"),
                            (vt[:, 7:10], pg["v_transforms"][:, 7:10], "v_log_scales (projection stage)"),
                            (vo, pg["v_raw_opac"], "v_raw_opacity (projection stage)"),
                            (vs, pg["v_sh"].reshape(len(vt), -1), "v_sh (projection stage)"),
                            (vr, pg["v_refine"], "v_refine_weight (projection stage)")):
        _check_grads(got, want, name, rtol=1e-5, atol=0.0, group_rtol=1e-3)


@pytest.mark.parametrize("cfg,n,view", [("c1", None, 0), ("c2", 20_000, 0), ("c3", 20_000, 5), ("c5", 20_000, 0)])
def test_backward_parity(cfg, n, view):
    w, (t, s, o), out, ref = _render_both(cfg, n, view)
    img = out.out_img.cpu().numpy()
    mask = circle_mask(w.img_size, w.mask_center, w.mask_radius) if w.mask_radius > 0 else None
    v_out = l1_cotangent_np(img, scenes.loss_target(w.img_size), mask)
    g = va.render_backward(out, t, s, o, torch.from_numpy(v_out).cuda())
    rg = ref.backward(v_out)
    vc = g.v_combined.cpu().numpy()
    _check_grads(vc[:, 0:2], rg["v_combined"][:, 0:2], "v_xy")
    _check_grads(vc[:, 2:5], rg["v_combined"][:, 2:5], "v_conic")
    _check_grads(vc[:, 5:8], rg["v_combined"][:, 5:8], "v_rgb")
    _check_grads(vc[:, 8], rg["v_combined"][:, 8], "v_opacity")
    _check_grads(vc[:, 9], rg["v_combined"][:, 9], "v_refine")
    _check_param_grads(g, rg, ref, vc)


@pytest.mark.parametrize("pass_", [va.RasterPass.GEOMETRY, va.RasterPass.GEOMETRY_TRAIN_DEPTH],
                         ids=["geometry", "geometry_train_depth"])
def test_geometry_pass_parity(pass_):
    """Both geometry passes; for gaussians they agree (the surface criterion is surfels' only)."""
    w, _, out, ref = _render_both("c1", None, 0, pass_=pass_)
    gpu = gpu_state_arrays(out)
    _check_forward(out, ref, gpu)
    gfc = ref.get(po.F_GLOBAL_FROM_COMPACT)
    np.testing.assert_array_equal(gpu["proj_aux"][gfc].view(np.uint32), ref.get(po.F_AUX).view(np.uint32))
    img = out.out_img.cpu().numpy()
    rimg = ref.get(po.F_OUT_IMG)
    assert img.shape == rimg.shape == (256, 256, 12)
    assert np.abs(img[..., :11] - rimg[..., :11]).max() <= 1e-4
    np.testing.assert_array_equal(img.view(np.uint32), rimg.view(np.uint32))


def test_packed_forward_pass_parity():
    w, _, out, ref = _render_both("c1", None, 0, pass_=va.RasterPass.FORWARD)
    got = out.out_img.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, ref.get(po.F_OUT_IMG))
    assert out.state is None


def test_smooth_cutoff_pass_parity():
    w, (t, s, o), out, ref = _render_both("c1", None, 0, pass_=va.RasterPass.BACKWARD_SMOOTH_CUTOFF)
    img = out.out_img.cpu().numpy()
    np.testing.assert_array_equal(img.view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))
    v_out = l1_cotangent_np(img, scenes.loss_target(w.img_size))
    g = va.render_backward(out, t, s, o, torch.from_numpy(v_out).cuda())
    rg = ref.backward(v_out)
    _check_grads(g.v_transforms.cpu().numpy(), rg["v_transforms"], "v_transforms")


def test_background_parity():
    _, _, out, ref = _render_both("c1", 2000, 0, background=(0.7, 0.3, 0.1))
    np.testing.assert_array_equal(out.out_img.cpu().numpy().view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))


def _culling_stress_scene(n=1200, seed=0x0C0A):
    """Splats centred on quadrant and tile boundaries, thin and rotated, some
    barely above the alpha cutoff: the cases where the kernels' per-quadrant
    skip test is tightest."""
    rng = np.random.default_rng(seed)
    w, h, f = 128, 96, 100.0
    z = rng.uniform(2.0, 6.0, n)
    u = 8.0 * rng.integers(0, w // 8 + 1, n) + rng.choice([-0.5, 0.0, 0.5, 0.25], n)
    v = 8.0 * rng.integers(0, h // 8 + 1, n) + rng.choice([-0.5, 0.0, 0.5, 0.25], n)
    means = np.stack([(u - w / 2) * z / f, (v - h / 2) * z / f, z], 1)
    quats = rng.standard_normal((n, 4))
    kind = rng.integers(0, 3, n)
    ls = np.where(kind[:, None] == 0, np.stack([rng.uniform(-2.0, -1.0, n), rng.uniform(-7, -5, n),
                                                rng.uniform(-7, -5, n)], 1),           # needles
                  np.where(kind[:, None] == 1, rng.uniform(-3.5, -2.0, (n, 3)),          # blobs
                           np.stack([rng.uniform(-2.5, -1.5, n), rng.uniform(-4.0, -3.0, n),
                                     rng.uniform(-4.0, -3.0, n)], 1)))                  # ellipses
    near_cut = rng.random(n) < 0.4
    p = np.where(near_cut, (1.0 / 255.0) * (1.0 + rng.uniform(0.0, 0.05, n)), rng.uniform(0.05, 0.9, n))
    logit = np.log(p / (1 - p))
    t = np.concatenate([means, quats, ls], 1).astype(np.float32)
    sh = rng.uniform(-0.5, 1.5, (n, 1, 3)).astype(np.float32)
    return scenes.Scene(t, sh, logit.astype(np.float32)), (w, h), f


@pytest.mark.parametrize("pass_", [va.RasterPass.BACKWARD, va.RasterPass.BACKWARD_SMOOTH_CUTOFF])
def test_quadrant_culling_stress(pass_):
    scene, img, f = _culling_stress_scene()
    cam = va.Camera.from_focal(f, f, img).uniforms(img)
    t, s, o = to_gpu(scene)
    print(f"[case] culling stress pass={pass_.name}", flush=True)
    out = va.render(cam, img, t, s, o, pass_=pass_)
    flags = po.FLAG_BWD_INFO | (po.FLAG_SMOOTH_CUTOFF if pass_ == va.RasterPass.BACKWARD_SMOOTH_CUTOFF else 0)
    ref = po.render_forward(cam, img, scene.transforms, scene.sh_coeffs, scene.raw_opacities, flags=flags)
    _check_forward(out, ref, gpu_state_arrays(out))
    gimg = out.out_img.cpu().numpy()
    np.testing.assert_array_equal(gimg.view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))
    np.testing.assert_array_equal(out.aux.tile_offsets.cpu().numpy().view(np.uint32), ref.get(po.F_TILE_OFFSETS_SHRUNK))
    rng = np.random.default_rng(3)
    v_out = (rng.standard_normal(gimg.shape) / gimg[..., 0].size).astype(np.float32)
    g = va.render_backward(out, t, s, o, torch.from_numpy(v_out).cuda())
    rg = ref.backward(v_out)
    vc = g.v_combined.cpu().numpy()
    _check_grads(vc[:, 0:5], rg["v_combined"][:, 0:5], "v_xy_conic")
    _check_grads(vc[:, 5:9], rg["v_combined"][:, 5:9], "v_rgb_opacity")
    _check_grads(vc[:, 9], rg["v_combined"][:, 9], "v_refine")


def row_sensitivity(ref, vc, vc_ref=None, seed=1):
    """Per row, the largest change of the oracle's projection-VJP output per
    unit of relative noise in that row of v_combined, measured with 1e-6
    relative noise (the size of the f32 atomic-order differences between two
    correct raster backwards), and the rows where that noise alone already
    moves an output past the end-to-end bar (1e-3 relative / 1e-5 absolute).
    The measurement starts from the GPU's v_combined and, given `vc_ref`,
    from the oracle's too, and keeps the larger response: in the rows it is
    for (raster gradients of 1e9..1e12 that the VJP cancels down to O(100),
    splats beside and behind a wide fisheye's camera plane) the response from
    one starting point is itself rounding noise."""
    sens = np.zeros(vc.shape[0])
    bad = np.zeros(vc.shape[0], bool)
    for base in (vc, vc_ref):
        if base is None:
            continue
        rng = np.random.default_rng(seed)
        noisy = (base.astype(np.float64) * (1 + 1e-6 * rng.standard_normal(base.shape))).astype(np.float32)
        a, b = ref.project_backward(base), ref.project_backward(noisy)
        for key in ("v_transforms", "v_sh", "v_raw_opac"):
            x = a[key].reshape(base.shape[0], -1).astype(np.float64)
            y = b[key].reshape(base.shape[0], -1).astype(np.float64)
            d = np.abs(x - y)
            sens = np.maximum(sens, d.max(axis=1) / 1e-6)
            bad |= (d > 1e-5 + 1e-3 * np.abs(x)).any(axis=1)
    return bad, sens


def ill_conditioned_rows(ref, vc, vc_ref=None, seed=1):
    """Rows whose projection-VJP output the oracle itself moves past the
    end-to-end bar under 1e-6 relative noise in v_combined (row_sensitivity)."""
    return row_sensitivity(ref, vc, vc_ref, seed)[0]


def check_ill_conditioned_rows(got, want, vc, vc_ref, bad, sens, name, safety=10.0):
    """The end-to-end gradients of the rows the contract bar cannot hold, at
    a bar scaled to each row's condition: the contract bar plus `safety`
    times the row's sensitivity (output change per unit relative noise in
    v_combined, row_sensitivity) times that row's observed relative
    difference between the GPU's and the oracle's raster gradients (at least
    1e-6).  A wrong projection VJP on such a row still fails: the bar only
    admits what the row's own raster-stage difference explains."""
    if not bad.any():
        return
    g = np.asarray(got, np.float64).reshape(len(bad), -1)[bad]
    w = np.asarray(want, np.float64).reshape(len(bad), -1)[bad]
    d_rows = np.abs(vc[bad].astype(np.float64) - vc_ref[bad].astype(np.float64)).max(axis=1)
    rel = np.maximum(d_rows / np.maximum(np.abs(vc_ref[bad].astype(np.float64)).max(axis=1), 1e-30), 1e-6)
    bar = 1e-5 + 1e-3 * np.abs(w) + safety * (sens[bad] * rel)[:, None]
    err = np.abs(g - w)
    assert (err <= bar).all(), (f"{name}: {int((err > bar).any(axis=1).sum())} of {int(bad.sum())} ill-conditioned "
                                f"rows exceed their condition-scaled bar (max err / bar {float((err / bar).max()):.3g})")
