"""GPU camera gradient (bwd/kernels/pose_backwards.rs, bwd/render_bwd.rs:
224-288) against the CPU oracle, fed the GPU's own raster gradient rows so
the check isolates the pose stage: every camera model, both render modes, the
scale floor, f16 coefficients.  The per-splat rows follow the same f32
operations, so the sums differ only by summation order: the bar is 1e-5 of
the sum of the rows' magnitudes per component.  At full size (1M splats) the
translation block must equal M times the summed dense mean gradient."""
import dataclasses

import numpy as np
import pytest
import torch

import vauss_amd as va
from oracle import pyoracle as po
from tests._util import circle_mask, l1_cotangent_np, to_gpu
from vauss_amd import scenes

pytestmark = pytest.mark.gpu

RT8 = va.RadialTangential8(-0.15, 0.06, -0.01, 0.05, 0.02, -0.005, 0.03, -0.02)
TPF = va.ThinPrismFisheye(va.KannalaBrandt4(0.03, -0.02, 0.01, -0.005), 0.02, -0.015, 0.01, -0.01)

CASES = [("c2", 0, None, False, False, False), ("c3", 2, RT8, True, False, False), ("c5", 0, None, False, True, False),
         ("c3", 5, TPF, False, True, True), ("c1", 0, None, True, True, True)]


@pytest.mark.parametrize("cfg,view,model,mip,use_floor,half", CASES,
                         ids=["c2", "c3-rt8-mip", "c5-kb4-floor", "c3-tpf-floor-f16", "c1-mip-floor-f16"])
def test_pose_gradient_parity(cfg, view, model, mip, use_floor, half):
    w = scenes.workload(cfg, 20_000)
    sc = w.scene
    cam_obj = w.cameras[view] if model is None else dataclasses.replace(w.cameras[view], model=model)
    cam = cam_obj.uniforms(w.img_size)
    t, s, o = to_gpu(sc)
    sh_ref = sc.sh_coeffs
    if half:
        sh16 = sc.sh_coeffs.astype(np.float16)
        s = torch.from_numpy(sh16).cuda()
        sh_ref = sh16.astype(np.float32)
    floor = np.random.default_rng(17).uniform(0.0, 0.02, sc.num_splats).astype(np.float32) if use_floor else None
    floor_gpu = torch.from_numpy(floor).cuda() if use_floor else None
    mode = va.SplatRenderMode.MIP if mip else va.SplatRenderMode.DEFAULT
    print(f"[case] {cfg} view={view} model={type(model).__name__} mip={mip} floor={use_floor} f16={half}", flush=True)
    out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD, render_mode=mode, min_scale=floor_gpu)
    img = out.out_img.cpu().numpy()
    mask = circle_mask(w.img_size, w.mask_center, w.mask_radius) if w.mask_radius > 0 else None
    v_out = l1_cotangent_np(img, scenes.loss_target(w.img_size), mask)
    g = va.render_backward(out, t, s, o, torch.from_numpy(v_out).cuda(), fused=True, min_scale=floor_gpu)
    v_pose = va.pose_backward(out, t, s, o, g.v_combined, min_scale=floor_gpu).cpu().numpy().astype(np.float64)

    flags = po.FLAG_BWD_INFO | (po.FLAG_MIP if mip else 0)
    ref = po.render_forward(cam, w.img_size, sc.transforms, sh_ref, sc.raw_opacities, flags=flags, min_scale=floor)
    np.testing.assert_array_equal(img.view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))
    total, rows = ref.pose_backward(g.v_combined.cpu().numpy())
    mag = np.abs(rows.astype(np.float64)).sum(0)
    assert np.count_nonzero(rows.any(1)) > 500
    assert np.all(np.abs(v_pose - total) <= 1e-5 * mag + 1e-12), (v_pose, total, mag)
    # a deterministic sum: the same call again gives the same bits
    again = va.pose_backward(out, t, s, o, g.v_combined, min_scale=floor_gpu).cpu().numpy()
    np.testing.assert_array_equal(again.view(np.uint32), v_pose.astype(np.float32).view(np.uint32))
    out.state.free()


def test_pose_translation_block_full_size():
    w = scenes.workload("c3")
    sc = w.scene
    cam = w.cameras[1].uniforms(w.img_size)
    t, s, o = to_gpu(sc)
    print(f"[case] c3 full n={sc.num_splats} view=1", flush=True)
    out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
    v_out = torch.from_numpy(l1_cotangent_np(out.out_img.cpu().numpy(), scenes.loss_target(w.img_size))).cuda()
    g = va.render_backward(out, t, s, o, v_out)
    v_pose = va.pose_backward(out, t, s, o, g.v_combined).cpu().numpy().astype(np.float64)
    vm = np.array(cam.viewmat[:], np.float64)
    R = vm[:9].reshape(3, 3).T
    v_mean = g.v_transforms[:, 0:3].double().cpu().numpy()
    per_splat = v_mean @ R.T
    want = per_splat.sum(0)
    assert np.all(np.abs(v_pose[9:12] - want) <= 1e-4 * np.abs(per_splat).sum(0) + 1e-12), (v_pose[9:12], want)
    assert np.abs(want).max() > 0
    out.state.free()


def test_pose_errors():
    w = scenes.workload("c1", 500)
    cam = w.cameras[0].uniforms(w.img_size)
    t, s, o = to_gpu(w.scene)
    out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD,
                    min_scale=torch.full((500,), 0.01, device="cuda"))
    vc = torch.zeros((500, 10), device="cuda")
    with pytest.raises(va.VsError):                 # the pose stage must see the forward's floor
        va.pose_backward(out, t, s, o, vc)
    out.state.free()
    fwd = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.FORWARD)
    with pytest.raises(ValueError):
        va.pose_backward(fwd, t, s, o, vc)
