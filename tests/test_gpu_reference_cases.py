"""The reference's own hot-path render tests, run through the C ABI.

* viewer_scale_matches_materialized_transforms
  (crates/splat-train-render/src/tests/mod.rs:287-382): a render with
  log_scale_offset = ln(s) must equal, bit for bit, the render of transforms
  whose log-scales were shifted by ln(s) beforehand: image (float and packed),
  num_visible, num_intersections, max_radius, opacities and tile offsets, with
  Mip on and off and the scale floor on and off.  The reference's three-splat
  scene is run as written; a 20k-splat cut of the 1080p workload extends it to
  every stage of the backward (gradients at the contract bar, the camera
  gradient too), and the oracle's render with the offset is compared bit for
  bit as well.
* renders_many_splats (tests/mod.rs:73-120): 30M splats in front of a 64x64
  pinhole camera must leave some splat visible and a finite, non-empty image.
  Beyond the reference's assertions: the binned list's oracle-free
  invariants, and per-splat tile counts, depth keys, projected rows and the
  projection VJP of a 100k-splat sample against the oracle (each of these
  depends on its own splat only, so the oracle need not render all 30M).
"""
import math

import numpy as np
import pytest
import torch

import vauss_amd as va
from oracle import pyoracle as po
from tests._util import gpu_state_arrays, l1_cotangent_np, to_gpu
from tests.test_gpu_fullsize import _check_list_properties
from tests.test_gpu_parity import _check_grads
from vauss_amd import scenes

pytestmark = pytest.mark.gpu


def _reference_scale_scene():
    """tests/mod.rs:300-306: one splat behind the camera, two in front at
    distinct depths; identity quaternions, log-scales (-3, -2.5, -2), DC
    (0.5, 0.2, 0.1), opacity logit 2."""
    means = np.array([[0.0, 0.0, -1.0], [-0.1, 0.0, 3.0], [0.1, 0.0, 4.0]], np.float32)
    t = np.zeros((3, 10), np.float32)
    t[:, 0:3] = means
    t[:, 3] = 1.0                                    # quaternion w, x, y, z = identity
    t[:, 7:10] = np.array([-3.0, -2.5, -2.0], np.float32)
    sh = np.tile(np.array([0.5, 0.2, 0.1], np.float32), (3, 1)).reshape(3, 1, 3)
    return scenes.Scene(t, sh, np.full(3, 2.0, np.float32))


def _materialize(scene, log_offset):
    t = scene.transforms.copy()
    t[:, 7:10] = t[:, 7:10] + np.float32(log_offset)   # the f32 sum the kernels form
    return scenes.Scene(t, scene.sh_coeffs, scene.raw_opacities)


def _aux_arrays(out):
    a = out.aux
    return (a.num_visible, a.num_intersections, a.max_radius.cpu().numpy().view(np.uint32),
            a.opacities.cpu().numpy().view(np.uint32), a.tile_offsets.cpu().numpy())


@pytest.mark.parametrize("mip,floor", [(False, False), (False, True), (True, False), (True, True)])
def test_viewer_scale_matches_materialized_transforms(mip, floor):
    cam = va.Camera(0.5, 0.5, (0.5, 0.5), (0.0, 0.0, 0.0), (0.0, 0.0, 0.0, 1.0)).uniforms((32, 32))
    scene = _reference_scale_scene()
    mode = va.SplatRenderMode.MIP if mip else va.SplatRenderMode.DEFAULT
    floor_np = np.full(3, 0.1, np.float32) if floor else None
    floor_gpu = torch.from_numpy(floor_np).cuda() if floor else None
    t, s, o = to_gpu(scene)
    for scale in (None, 1.0, 0.5, 2.0):
        lso = np.float32(0.0 if scale is None else math.log(scale))
        tm, sm, om = to_gpu(_materialize(scene, lso))
        for pass_ in (va.RasterPass.FLOAT, va.RasterPass.FORWARD):
            print(f"[case] viewer scale mip={mip} floor={floor} scale={scale} pass={pass_.name}", flush=True)
            got = va.render(cam, (32, 32), t, s, o, pass_=pass_, render_mode=mode, min_scale=floor_gpu,
                            log_scale_offset=float(lso))
            want = va.render(cam, (32, 32), tm, sm, om, pass_=pass_, render_mode=mode, min_scale=floor_gpu)
            np.testing.assert_array_equal(got.out_img.cpu().numpy().view(np.uint32),
                                          want.out_img.cpu().numpy().view(np.uint32))
            ga, wa = _aux_arrays(got), _aux_arrays(want)
            assert ga[0] == 2 and ga[0] == wa[0]
            assert ga[1] == wa[1]
            for x, y in zip(ga[2:], wa[2:]):
                np.testing.assert_array_equal(x, y)
            # the oracle with the same offset agrees bit for bit
            flags = (po.FLAG_BWD_INFO if pass_ == va.RasterPass.FLOAT else 0) | (po.FLAG_MIP if mip else 0)
            ref = po.render_forward(cam, (32, 32), scene.transforms, scene.sh_coeffs, scene.raw_opacities,
                                    flags=flags, log_scale_offset=float(lso), min_scale=floor_np)
            np.testing.assert_array_equal(got.out_img.cpu().numpy().view(np.uint32),
                                          ref.get(po.F_OUT_IMG).view(np.uint32))
            for st in (got.state, want.state):
                if st is not None:
                    st.free()


@pytest.mark.parametrize("mip,floor", [(False, False), (True, True)])
@pytest.mark.parametrize("scale", [0.5, 2.0])
def test_viewer_scale_backward_matches_materialized(mip, floor, scale):
    """The same invariance on a 20k-splat cut of the 1080p workload, through
    the backward: the offset render's dense gradients equal the materialised
    render's (d/d log-scale is the same function of the same scale), and the
    camera gradient too; the forward's binning and image are bit-equal."""
    w = scenes.workload("c2", 20_000)
    cam = w.cameras[0].uniforms(w.img_size)
    sc = w.scene
    lso = np.float32(math.log(scale))
    mode = va.SplatRenderMode.MIP if mip else va.SplatRenderMode.DEFAULT
    floor_np = np.random.default_rng(9).uniform(0.0, 0.02, sc.num_splats).astype(np.float32) if floor else None
    floor_gpu = torch.from_numpy(floor_np).cuda() if floor else None
    t, s, o = to_gpu(sc)
    tm, sm, om = to_gpu(_materialize(sc, lso))
    print(f"[case] c2 20k viewer scale {scale} mip={mip} floor={floor}", flush=True)
    got = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD, render_mode=mode, min_scale=floor_gpu,
                    log_scale_offset=float(lso))
    want = va.render(cam, w.img_size, tm, sm, om, pass_=va.RasterPass.BACKWARD, render_mode=mode, min_scale=floor_gpu)
    img = got.out_img.cpu().numpy()
    np.testing.assert_array_equal(img.view(np.uint32), want.out_img.cpu().numpy().view(np.uint32))
    ga, wa = _aux_arrays(got), _aux_arrays(want)
    assert ga[:2] == wa[:2] and ga[0] > 1000
    for x, y in zip(ga[2:], wa[2:]):
        np.testing.assert_array_equal(x, y)
    gs, ws = gpu_state_arrays(got), gpu_state_arrays(want)
    for key in ("tile", "gid", "counts"):
        np.testing.assert_array_equal(gs[key], ws[key])
    listed = gs["counts"] > 0            # rows and keys are written for splats with tiles only
    for key in ("depth_bits", "proj_a", "proj_b", "proj_c"):
        np.testing.assert_array_equal(gs[key][listed].view(np.uint32), ws[key][listed].view(np.uint32))
    del gs, ws
    v_out = torch.from_numpy(l1_cotangent_np(img, scenes.loss_target(w.img_size))).cuda()
    gg = va.render_backward(got, t, s, o, v_out, min_scale=floor_gpu)
    gw = va.render_backward(want, tm, sm, om, v_out, min_scale=floor_gpu)
    vc = gg.v_combined.cpu().numpy()
    _check_grads(vc, gw.v_combined.cpu().numpy(), "v_combined")
    # the projection stage on the same raster gradients is a pure function of
    # the same scales: check it at 1e-5 through the oracle, offset vs none
    flags = po.FLAG_BWD_INFO | (po.FLAG_MIP if mip else 0)
    ref = po.render_forward(cam, w.img_size, sc.transforms, sc.sh_coeffs, sc.raw_opacities, flags=flags,
                            log_scale_offset=float(lso), min_scale=floor_np)
    refm = po.render_forward(cam, w.img_size, _materialize(sc, lso).transforms, sc.sh_coeffs, sc.raw_opacities,
                             flags=flags, min_scale=floor_np)
    pg, pm = ref.project_backward(vc), refm.project_backward(vc)
    for key in ("v_transforms", "v_sh", "v_raw_opac", "v_refine"):
        np.testing.assert_array_equal(pg[key].view(np.uint32), pm[key].view(np.uint32))
    vt = gg.v_transforms.cpu().numpy()
    _check_grads(vt, pg["v_transforms"], "v_transforms (projection stage, offset)", rtol=1e-5, atol=0.0)
    _check_grads(gg.v_raw_opac.cpu().numpy(), pg["v_raw_opac"], "v_raw_opacity (projection stage, offset)",
                 rtol=1e-5, atol=0.0)
    # the camera gradient of the offset render equals the materialised one's
    # on the same raster gradients
    vc_dev = gg.v_combined
    pose_g = va.pose_backward(got, t, s, o, vc_dev, min_scale=floor_gpu).cpu().numpy()
    pose_w = va.pose_backward(want, tm, sm, om, vc_dev, min_scale=floor_gpu).cpu().numpy()
    np.testing.assert_array_equal(pose_g.view(np.uint32), pose_w.view(np.uint32))
    got.state.free()
    want.state.free()


def _many_splats(n, seed):
    """tests/mod.rs:77-106: means U(-2,2)^3 in front of a camera at z=-5,
    log-scales U(-4,-2), quaternions U(-1,1)^4, DC colours U(0,1), opacity
    logits U(-2,2)."""
    rng = np.random.default_rng(seed)
    t = np.empty((n, 10), np.float32)
    t[:, 0:3] = rng.uniform(-2.0, 2.0, (n, 3)).astype(np.float32)
    t[:, 3:7] = rng.uniform(-1.0, 1.0, (n, 4)).astype(np.float32)
    t[:, 7:10] = rng.uniform(-4.0, -2.0, (n, 3)).astype(np.float32)
    sh = rng.uniform(0.0, 1.0, (n, 1, 3)).astype(np.float32)
    op = rng.uniform(-2.0, 2.0, n).astype(np.float32)
    return scenes.Scene(t, sh, op)


def test_renders_many_splats():
    n = 30_000_000
    img = (64, 64)
    sc = _many_splats(n, 0x3000)
    cam = va.Camera(0.5, 0.5, (0.5, 0.5), (0.0, 0.0, -5.0), (0.0, 0.0, 0.0, 1.0)).uniforms(img)
    t, s, o = to_gpu(sc)
    print(f"[case] {n} splats at {img}", flush=True)
    out = va.render(cam, img, t, s, o, pass_=va.RasterPass.BACKWARD)
    px = out.out_img.cpu().numpy()
    assert out.aux.num_visible > 0, "30M splats in front of the camera, none survived projection"
    assert np.isfinite(px).all()
    assert (px[..., 3] > 1e-3).any(), "30M splats rendered to an entirely empty image"
    gpu = gpu_state_arrays(out)
    print(f"[case] {out.aux.num_visible} visible, {out.aux.num_intersections} intersections", flush=True)
    assert out.aux.num_intersections == int(gpu["counts"].sum(dtype=np.uint64))
    _check_list_properties(gpu, n)
    # per-splat outputs of a sample against the oracle (each depends on its own splat only)
    rng = np.random.default_rng(5)
    pick = np.sort(rng.choice(n, 100_000, replace=False))
    sub = scenes.Scene(sc.transforms[pick], sc.sh_coeffs[pick], sc.raw_opacities[pick])
    ref = po.render_forward(cam, img, sub.transforms, sub.sh_coeffs, sub.raw_opacities, flags=po.FLAG_BWD_INFO)
    np.testing.assert_array_equal(gpu["counts"][pick], ref.get(po.F_INTERSECT_COUNTS))
    gfc = pick[ref.get(po.F_GLOBAL_FROM_COMPACT)]
    np.testing.assert_array_equal(gpu["depth_bits"][gfc], ref.get(po.F_DEPTHS).view(np.uint32))
    rows = np.concatenate([gpu["proj_a"][gfc], gpu["proj_b"][gfc], gpu["proj_c"][gfc, None]], axis=1)
    np.testing.assert_array_equal(rows.view(np.uint32), ref.get(po.F_PROJECTED).view(np.uint32))
    np.testing.assert_array_equal(out.aux.max_radius.cpu().numpy()[pick].view(np.uint32),
                                  ref.get(po.F_MAX_RADIUS).view(np.uint32))
    counts = gpu["counts"]
    del gpu, rows
    # the backward at 30M: raster gradients are finite and vanish exactly on
    # splats without tiles; the projection VJP of the sample's rows matches
    v_out = l1_cotangent_np(px, np.full((img[1], img[0], 3), 0.5, np.float32))
    g = va.render_backward(out, t, s, o, torch.from_numpy(v_out).cuda())
    vc = g.v_combined.cpu().numpy()
    assert np.isfinite(vc).all()
    assert not vc[counts == 0].any()
    pg = ref.project_backward(vc[pick])
    vt = g.v_transforms.cpu().numpy()[pick]
    _check_grads(vt, pg["v_transforms"], "v_transforms (projection stage, 30M sample)", rtol=1e-5, atol=0.0)
    _check_grads(g.v_raw_opac.cpu().numpy()[pick], pg["v_raw_opac"], "v_raw_opacity (30M sample)",
                 rtol=1e-5, atol=0.0)
    out.state.free()
