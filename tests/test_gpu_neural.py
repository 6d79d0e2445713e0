"""GPU parity of the compact neural appearance (kernels/neural.rs,
bwd/kernels/neural_backwards.rs) against the CPU oracle: the forward bit for
bit (image, projected rows), the backward fed the GPU's own raster gradients
(rows and mean gradients bit for bit, the decoder gradient within 1e-5 of the
summed magnitudes of its products, since its sums run in another order), in
f32 and f16 rows, every direction band; and the entry points that reject it
(fused update, camera gradient)."""
import numpy as np
import pytest
import torch

import vauss_amd as va
from oracle import pyoracle as po
from tests._util import circle_mask, gpu_state_arrays, l1_cotangent_np, to_gpu
from tests.test_gpu_parity import _check_forward, _check_grads
from vauss_amd import scenes

pytestmark = pytest.mark.gpu


def _neural_inputs(n, seed):
    rng = np.random.default_rng(seed)
    rows = np.zeros((n, 4, 3), np.float32)
    flat = rows.reshape(n, 12)
    flat[:, :3] = rng.uniform(-1.5, 1.5, (n, 3))
    flat[:, 3:11] = rng.uniform(-3, 3, (n, 8))
    W = (rng.standard_normal(816) * 0.35).astype(np.float32)
    return rows, W


CASES = [("c2", 0, 3, False), ("c3", 4, 1, False), ("c5", 0, 2, True), ("c1", 0, 0, False)]


@pytest.mark.parametrize("cfg,view,deg,half", CASES, ids=["c2-b3", "c3-b1", "c5-b2-f16", "c1-b0"])
def test_neural_parity(cfg, view, deg, half):
    w = scenes.workload(cfg, 20_000)
    sc = w.scene
    cam = w.cameras[view].uniforms(w.img_size)
    t, _, o = to_gpu(sc)
    rows, W = _neural_inputs(sc.num_splats, 5 + deg)
    rows_ref = rows
    if half:
        rows16 = rows.astype(np.float16)
        s = torch.from_numpy(rows16).cuda()
        rows_ref = rows16.astype(np.float32)
    else:
        s = torch.from_numpy(rows).cuda()
    dec = torch.from_numpy(W).cuda()
    print(f"[case] {cfg} view={view} band={deg} f16={half}", flush=True)
    out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD, decoder=dec, neural_degree=deg)
    ref = po.render_forward(cam, w.img_size, sc.transforms, rows_ref, sc.raw_opacities, decoder=W, neural_degree=deg)
    _check_forward(out, ref, gpu_state_arrays(out))
    img = out.out_img.cpu().numpy()
    np.testing.assert_array_equal(img.view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))
    assert img[..., :3].std() > 0.02

    mask = circle_mask(w.img_size, w.mask_center, w.mask_radius) if w.mask_radius > 0 else None
    v_out = l1_cotangent_np(img, scenes.loss_target(w.img_size), mask)
    g = va.render_backward(out, t, s, o, torch.from_numpy(v_out).cuda(), decoder=dec)
    vc = g.v_combined.cpu().numpy()
    pg = ref.project_backward(vc)
    gfc = ref.get(po.F_GLOBAL_FROM_COMPACT)
    live = gfc[np.any(vc[gfc, 5:8] != 0, axis=1)]
    assert len(live) > 200
    np.testing.assert_array_equal(g.v_coeffs.cpu().numpy().view(np.uint32), pg["v_sh"].view(np.uint32))
    np.testing.assert_array_equal(g.v_coeffs_sq.cpu().numpy().view(np.uint32), pg["v_coeffs_sq"].view(np.uint32))
    _check_grads(g.v_transforms.cpu().numpy(), pg["v_transforms"], "v_transforms (projection + neural stage)")
    got = g.v_decoder.cpu().numpy().astype(np.float64)
    want = pg["v_decoder"].astype(np.float64)
    bound = 1e-5 * ref.decoder_abs + 1e-12
    assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) / bound)
    assert np.count_nonzero(want) > 400
    out.state.free()


def test_neural_rejections():
    w = scenes.workload("c1", 500)
    sc = w.scene
    cam = w.cameras[0].uniforms(w.img_size)
    t, s_sh, o = to_gpu(sc)
    rows, W = _neural_inputs(500, 1)
    s = torch.from_numpy(rows).cuda()
    dec = torch.from_numpy(W).cuda()
    out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD, decoder=dec, neural_degree=1)
    vc = torch.zeros((500, 10), device="cuda")
    with pytest.raises(va.VsError):                     # the camera gradient follows SH colour only
        va.pose_backward(out, t, s, o, vc)
    with pytest.raises(va.VsError):                     # the backward must be given the forward's decoder
        va.render_backward(out, t, s, o, torch.zeros_like(out.out_img))
    adam = va.FusedAdam.at_step(1, lr_opac=0.05)
    with pytest.raises(va.VsError):                     # the fused update takes SH colour
        va.project_update(out, t.clone(), s, o.clone(), vc, torch.zeros((500, 10), dtype=torch.int32, device="cuda"),
                          torch.full((10,), 1e-3, device="cuda"), torch.zeros(500, dtype=torch.int32, device="cuda"),
                          adam)
    with pytest.raises(ValueError):
        va.render(cam, w.img_size, t, s_sh, o, decoder=dec, neural_degree=1)     # SH3 rows are not neural rows
    with pytest.raises(ValueError):
        va.render(cam, w.img_size, t, s, o, decoder=dec, neural_degree=4)
    out.state.free()
