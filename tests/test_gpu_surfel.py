"""GPU parity of the surfel (2DGS) render mode (kernels/helpers.rs:316-423,
kernels/rasterize.rs:267-301, bwd/kernels/rasterize_backwards_planes.rs:266-480,
bwd/kernels/project_backwards.rs:426-570) against the CPU oracle: counts, key
order, projected rows and the surfel rows (M, low-pass centre, normal) bit for
bit; the 12-channel image (colour, alpha, depth, normal and the median channels
under the training rule or the surface criterion) bit for bit in every float
pass and the packed pass; the 17 raster gradient components and the parameter
gradients at the contract bar (1e-3 relative / 1e-5 absolute), the projection
stage on its own against the oracle's VJP of the GPU's raster gradients; and
the entry points that reject surfels."""
import numpy as np
import pytest
import torch

import vauss_amd as va
from oracle import pyoracle as po
from tests._util import circle_mask, gpu_state_arrays, l1_cotangent_np, to_gpu
from tests.test_gpu_parity import _check_forward, _check_grads, check_ill_conditioned_rows, row_sensitivity
from vauss_amd import scenes

pytestmark = pytest.mark.gpu

SURFEL = va.SplatRenderMode.SURFEL


def _flags(pass_):
    f = po.FLAG_SURFEL
    if pass_.bwd_info():
        f |= po.FLAG_BWD_INFO
    if pass_.geometry():
        f |= po.FLAG_GEOMETRY
    if pass_ == va.RasterPass.BACKWARD_SMOOTH_CUTOFF:
        f |= po.FLAG_SMOOTH_CUTOFF
    if pass_.surface_criterion():                # inference passes but GEOMETRY_TRAIN_DEPTH (gaussian_splats.rs:100-106)
        f |= po.FLAG_SURFACE
    return f


def _surfel_both(cfg, n, view, pass_=va.RasterPass.BACKWARD):
    w = scenes.workload(cfg, n)
    cam = w.cameras[view].uniforms(w.img_size)
    t, s, o = to_gpu(w.scene)
    print(f"[case] surfel {cfg} n={w.scene.num_splats} view={view} pass={pass_.name}", flush=True)
    out = va.render(cam, w.img_size, t, s, o, pass_=pass_, render_mode=SURFEL)
    ref = po.render_forward(cam, w.img_size, w.scene.transforms, w.scene.sh_coeffs, w.scene.raw_opacities,
                            flags=_flags(pass_))
    return w, (t, s, o), out, ref


def _check_surfel_rows(out, ref):
    gpu = gpu_state_arrays(out)
    _check_forward(out, ref, gpu)
    gfc = ref.get(po.F_GLOBAL_FROM_COMPACT)
    rows = gpu["proj_surf"][gfc, :14]
    np.testing.assert_array_equal(rows.view(np.uint32), ref.get(po.F_SURFEL_AUX).view(np.uint32))


PASSES = [va.RasterPass.BACKWARD, va.RasterPass.FLOAT, va.RasterPass.GEOMETRY, va.RasterPass.BACKWARD_SMOOTH_CUTOFF,
          va.RasterPass.GEOMETRY_TRAIN_DEPTH, va.RasterPass.EXPOSURE, va.RasterPass.BACKWARD_DENSE,
          va.RasterPass.BACKWARD_FUSED_UPDATE]


@pytest.mark.parametrize("pass_", PASSES, ids=[p.name for p in PASSES])
def test_surfel_forward_passes(pass_):
    w, _, out, ref = _surfel_both("c1", None, 0, pass_)
    _check_surfel_rows(out, ref)
    img = out.out_img.cpu().numpy()
    rimg = ref.get(po.F_OUT_IMG)
    assert img.shape == rimg.shape == (256, 256, 12)
    assert np.abs(img[..., :11] - rimg[..., :11]).max() <= 1e-4
    np.testing.assert_array_equal(img.view(np.uint32), rimg.view(np.uint32))
    assert img[..., 3].max() > 0.5 and np.count_nonzero(img[..., 4]) > 1000
    out.state.free()


def test_surfel_train_depth_rule_differs_from_the_surface_criterion():
    """GEOMETRY_TRAIN_DEPTH keeps the training median where GEOMETRY takes the
    surface criterion: the median channels differ, colour and alpha do not."""
    _, _, a, _ = _surfel_both("c1", None, 0, va.RasterPass.GEOMETRY)
    _, _, b, _ = _surfel_both("c1", None, 0, va.RasterPass.GEOMETRY_TRAIN_DEPTH)
    ia, ib = a.out_img.cpu().numpy(), b.out_img.cpu().numpy()
    np.testing.assert_array_equal(ia[..., :5].view(np.uint32), ib[..., :5].view(np.uint32))
    assert (ia[..., 5] != ib[..., 5]).mean() > 0.01
    a.state.free()
    b.state.free()


def test_surfel_packed_forward():
    w, _, out, ref = _surfel_both("c1", None, 0, va.RasterPass.FORWARD)
    np.testing.assert_array_equal(out.out_img.cpu().numpy().view(np.uint32), ref.get(po.F_OUT_IMG))
    assert out.state is None


@pytest.mark.parametrize("cfg,n,view", [("c1", None, 0), ("c2", 20_000, 0), ("c3", 20_000, 2)])
def test_surfel_forward_bit_exact(cfg, n, view):
    w, _, out, ref = _surfel_both(cfg, n, view)
    _check_surfel_rows(out, ref)
    np.testing.assert_array_equal(out.out_img.cpu().numpy().view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))
    out.state.free()


def _check_surfel_grads(g, rg, ref, vc):
    for sl, name in ((slice(0, 9), "v_M"), (slice(9, 12), "v_normal"), (slice(12, 15), "v_rgb"),
                     (15, "v_alpha"), (16, "v_refine")):
        _check_grads(vc[:, sl], rg["v_combined"][:, sl], name)
    vt = g.v_transforms.cpu().numpy()
    vs = g.v_coeffs.cpu().numpy().reshape(len(vt), -1)
    vo = g.v_raw_opac.cpu().numpy()
    vr = g.v_refine_weight.cpu().numpy()
    assert np.isfinite(vt).all() and np.isfinite(vs).all()
    bad, sens = row_sensitivity(ref, vc, rg["v_combined"])
    visible = int((ref.get(po.F_INTERSECT_COUNTS) > 0).sum())
    print(f"[ill-conditioned] surfels: {int(bad.sum())} of {visible} visible rows", flush=True)
    assert bad.sum() <= 0.0005 * visible + 3, (int(bad.sum()), visible)
    keep = ~bad
    for got, want, name in ((vt, rg["v_transforms"], "v_transforms"), (vo, rg["v_raw_opac"], "v_raw_opacity"),
                            (vs, rg["v_sh"].reshape(len(vt), -1), "v_sh"), (vr, rg["v_refine"], "v_refine_weight")):
        _check_grads(got[keep], want[keep], name, group_rtol=None)
        check_ill_conditioned_rows(got, want, vc, rg["v_combined"], bad, sens, name)
    pg = ref.project_backward(vc)
    for got, want, name in ((vt, pg["v_transforms"], "v_transforms (projection stage)"),
                            (vo, pg["v_raw_opac"], "v_raw_opacity (projection stage)"),
                            (vs, pg["v_sh"].reshape(len(vt), -1), "v_sh (projection stage)"),
                            (vr, pg["v_refine"], "v_refine_weight (projection stage)")):
        _check_grads(got, want, name, rtol=1e-5, atol=0.0, group_rtol=1e-3)


@pytest.mark.parametrize("cfg,n,view,pass_", [("c1", None, 0, va.RasterPass.BACKWARD),
                                              ("c2", 20_000, 0, va.RasterPass.BACKWARD),
                                              ("c3", 20_000, 2, va.RasterPass.BACKWARD),
                                              ("c1", None, 0, va.RasterPass.BACKWARD_SMOOTH_CUTOFF)],
                         ids=["c1", "c2", "c3", "c1-smooth"])
def test_surfel_backward_parity(cfg, n, view, pass_):
    w, (t, s, o), out, ref = _surfel_both(cfg, n, view, pass_)
    img = out.out_img.cpu().numpy()
    mask = circle_mask(w.img_size, w.mask_center, w.mask_radius) if w.mask_radius > 0 else None
    v_rgb = l1_cotangent_np(img[..., :4], scenes.loss_target(w.img_size), mask)
    rng = np.random.default_rng(7)
    v_out = np.zeros_like(img)
    v_out[..., :4] = v_rgb
    # depth and normal channels carry a small loss too; the median channels are not differentiable
    v_out[..., 4:8] = (rng.standard_normal(img[..., 4:8].shape) * 0.1 / img[..., 0].size).astype(np.float32)
    g = va.render_backward(out, t, s, o, torch.from_numpy(v_out).cuda())
    rg = ref.backward(v_out)
    vc = g.v_combined.cpu().numpy()
    assert vc.shape == (w.scene.num_splats, 17)
    assert np.count_nonzero(np.any(vc != 0, axis=1)) > 100
    _check_surfel_grads(g, rg, ref, vc)
    out.state.free()


def test_surfel_rejections():
    w = scenes.workload("c1", 500)
    cam = w.cameras[0].uniforms(w.img_size)
    t, s, o = to_gpu(w.scene)
    out = va.render(cam, w.img_size, t, s, o, render_mode=SURFEL)
    with pytest.raises(va.VsError):                 # the camera gradient is built for gaussians
        va.pose_backward(out, t, s, o, torch.zeros((500, 10), device="cuda"))
    adam = va.FusedAdam.at_step(1, lr_opac=0.05)
    with pytest.raises(va.VsError):                 # surfels train unfused
        va.project_update(out, t.clone(), s, o.clone(), torch.zeros((500, 10), device="cuda"),
                          torch.zeros((500, 10), dtype=torch.int32, device="cuda"),
                          torch.full((10,), 1e-3, device="cuda"), torch.zeros(500, dtype=torch.int32, device="cuda"),
                          adam)
    out.state.free()
    rows = torch.zeros((500, 4, 3), device="cuda")
    with pytest.raises(va.VsError):                 # surfels take SH colour
        va.render(cam, w.img_size, t, rows, o, render_mode=SURFEL, decoder=torch.zeros(816, device="cuda"))


def test_surfel_floor_background_f16():
    """Surfels under the scale floor, a background (colour composites over it,
    the geometry channels do not) and f16 SH rows."""
    w = scenes.workload("c2", 20_000)
    sc = w.scene
    cam = w.cameras[0].uniforms(w.img_size)
    t, _, o = to_gpu(sc)
    sh16 = sc.sh_coeffs.astype(np.float16)
    s = torch.from_numpy(sh16).cuda()
    floor = np.random.default_rng(23).uniform(0.0, 0.02, sc.num_splats).astype(np.float32)
    floor_gpu = torch.from_numpy(floor).cuda()
    bg = (0.7, 0.3, 0.1)
    print("[case] surfel c2 floor + background + f16", flush=True)
    out = va.render(cam, w.img_size, t, s, o, background=bg, render_mode=SURFEL, min_scale=floor_gpu)
    ref = po.render_forward(cam, w.img_size, sc.transforms, sh16.astype(np.float32), sc.raw_opacities,
                            background=bg, flags=_flags(va.RasterPass.BACKWARD), min_scale=floor)
    _check_surfel_rows(out, ref)
    img = out.out_img.cpu().numpy()
    np.testing.assert_array_equal(img.view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))
    v_out = l1_cotangent_np(img, scenes.loss_target(w.img_size))
    g = va.render_backward(out, t, s, o, torch.from_numpy(v_out).cuda(), min_scale=floor_gpu)
    rg = ref.backward(v_out)
    _check_surfel_grads(g, rg, ref, g.v_combined.cpu().numpy())
    out.state.free()


def _grazing_scene(n, rng):
    """Surfels whose normal lies within 10 degrees of perpendicular to the ray from
    the camera at (0, 0, -5): the disk is seen almost edge-on."""
    mean = rng.uniform([-1.2, -0.9, -1.5], [1.2, 0.9, 2.0], (n, 3))
    view = mean - np.array([0.0, 0.0, -5.0])
    view /= np.linalg.norm(view, axis=1, keepdims=True)
    w = rng.standard_normal((n, 3))
    w -= (w * view).sum(1, keepdims=True) * view
    w /= np.linalg.norm(w, axis=1, keepdims=True)
    tilt = np.radians(rng.uniform(-10.0, 10.0, (n, 1)))
    nrm = np.cos(tilt) * w + np.sin(tilt) * view
    a = np.cross(nrm, rng.standard_normal((n, 3)))
    a /= np.linalg.norm(a, axis=1, keepdims=True)
    b = np.cross(nrm, a)
    rot = np.stack([a, b, nrm], axis=2)                       # columns: disk axes, normal
    # rotation matrix -> quaternion (w, x, y, z), the largest-component branch per row
    q = np.zeros((n, 4))
    for i in range(n):
        m = rot[i]
        tr = np.trace(m)
        if tr > 0:
            s = np.sqrt(tr + 1.0) * 2
            q[i] = [0.25 * s, (m[2, 1] - m[1, 2]) / s, (m[0, 2] - m[2, 0]) / s, (m[1, 0] - m[0, 1]) / s]
        else:
            k = int(np.argmax(np.diag(m)))
            j, l = (k + 1) % 3, (k + 2) % 3
            s = np.sqrt(1.0 + m[k, k] - m[j, j] - m[l, l]) * 2
            v = np.zeros(3)
            v[k] = 0.25 * s
            v[j] = (m[j, k] + m[k, j]) / s
            v[l] = (m[l, k] + m[k, l]) / s
            q[i] = [(m[l, j] - m[j, l]) / s, *v]
    t = np.zeros((n, 10), np.float32)
    t[:, 0:3] = mean
    t[:, 3:7] = q
    t[:, 7:9] = rng.uniform(-3.0, 0.0, (n, 2))
    t[:, 9] = -6.0
    sh = rng.uniform(0.0, 1.0, (n, 1, 3)).astype(np.float32)
    o = rng.uniform(-1.0, 4.0, n).astype(np.float32)
    return t, sh, o


@pytest.mark.parametrize("pass_", [va.RasterPass.BACKWARD, va.RasterPass.BACKWARD_SMOOTH_CUTOFF],
                         ids=["hard", "smooth"])
def test_surfel_grazing_bit_exact(pass_):
    """Nearly edge-on surfels, where the ray-plane footprint is ill-conditioned
    and the raster's quadrant culling (surfel_quadrant_live) rests on its
    rounding bound: the image stays bit-exact and the raster gradients at the
    contract bar."""
    rng = np.random.default_rng(11)
    t, sh, o = _grazing_scene(3000, rng)
    img = (256, 192)
    cam = scenes.test_camera(img, fov=0.6).uniforms(img)
    print(f"[case] surfel grazing pass={pass_.name}", flush=True)
    args = [torch.from_numpy(x).cuda() for x in (t, sh, o)]
    out = va.render(cam, img, *args, pass_=pass_, render_mode=SURFEL)
    ref = po.render_forward(cam, img, t, sh, o, flags=_flags(pass_))
    assert ref.info.num_visible > 1000
    _check_surfel_rows(out, ref)
    got = out.out_img.cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))
    v_out = np.zeros_like(got)
    v_out[..., :4] = l1_cotangent_np(got[..., :4], np.full(got.shape[:2] + (3,), 0.5, np.float32))
    g = va.render_backward(out, *args, torch.from_numpy(v_out).cuda())
    rg = ref.backward(v_out)
    vc = g.v_combined.cpu().numpy()
    assert np.count_nonzero(np.any(vc != 0, axis=1)) > 100
    for sl, name in ((slice(0, 9), "v_M"), (slice(9, 12), "v_normal"), (slice(12, 15), "v_rgb"), (15, "v_alpha")):
        _check_grads(vc[:, sl], rg["v_combined"][:, sl], name)
    out.state.free()
