"""GPU parity of the fused projection update (projection VJP + packed-moment
Adam, bwd/kernels/project_update.rs) and of the moment codec
(bwd/kernels/geo_moments.rs) against the CPU oracle.

Bars: the codec bit for bit; the fused update, fed the same raster gradients,
parameters and moments as the oracle, bit for bit in every output: color_dir,
refine weights, SH second moments, the stepped parameters and the packed
moment words (stochastic rounding included).
"""
import numpy as np
import pytest
import torch

import vauss_amd as va
from oracle import pyoracle as po
from tests._util import circle_mask, l1_cotangent_np, to_gpu
from vauss_amd import scenes

pytestmark = pytest.mark.gpu

EPS = 1e-15


def _words(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int32).copy()).cuda()


def test_codec_matches_oracle_bit_for_bit():
    rng = np.random.default_rng(11)
    n = 20000
    root = (10.0 ** rng.uniform(-16, 6, n)).astype(np.float32)
    u = rng.uniform(-9, 9, n).astype(np.float32)
    m = (u * (root + np.float32(EPS))).astype(np.float32)
    v = (root * root).astype(np.float32)
    m[:8] = [0.0, -0.0, 1e30, -1e30, 0.0, 1e-20, -1e-20, 3.0]
    v[:8] = [0.0, 0.0, 0.0, 1.0, 3.0e38, 0.0, 1e-40, 1e-30]
    words = va.geo_encode(torch.from_numpy(m).cuda(), torch.from_numpy(v).cuda(), EPS).cpu().numpy().view(np.uint32)
    want = np.array([po.geo_encode(float(a), float(b), EPS) for a, b in zip(m, v)], np.uint32)
    np.testing.assert_array_equal(words, want)
    w = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    w[:3] = [0, 0x8000, 0xFFFFFFFF]
    gm, gv = va.geo_decode(_words(w), EPS)
    ref = np.array([po.geo_decode(int(x), EPS) for x in w], np.float32)
    np.testing.assert_array_equal(gm.cpu().numpy().view(np.uint32), ref[:, 0].view(np.uint32))
    np.testing.assert_array_equal(gv.cpu().numpy().view(np.uint32), ref[:, 1].view(np.uint32))


def test_zero_rows():
    w = torch.full((50, 10), 0x12345678, dtype=torch.int32, device="cuda")
    rows = torch.tensor([3, 17, 49, 1000], dtype=torch.int32, device="cuda")   # 1000 is past the end: ignored
    va.geo_zero_rows(w, rows)
    out = w.cpu().numpy()
    assert (out[[3, 17, 49]] == 0).all()
    keep = np.setdiff1d(np.arange(50), [3, 17, 49])
    assert (out[keep] == 0x12345678).all()


def _update_case(cfg, n, view, step, opac_reg):
    w = scenes.workload(cfg, n)
    cam = w.cameras[view].uniforms(w.img_size)
    sc = w.scene
    n = sc.num_splats
    t, s, o = to_gpu(sc)
    print(f"[case] {cfg} n={n} view={view} step={step}", flush=True)
    out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
    img = out.out_img.cpu().numpy()
    mask = circle_mask(w.img_size, w.mask_center, w.mask_radius) if w.mask_radius > 0 else None
    v_out = torch.from_numpy(l1_cotangent_np(img, scenes.loss_target(w.img_size), mask)).cuda()
    full = va.render_backward(out, t, s, o, v_out)
    fused = va.render_backward(out, t, s, o, v_out, fused=True)
    assert fused.v_transforms is None
    vc = fused.v_combined.cpu().numpy()
    # the fused pass stops at the same raster gradients (up to atomic order)
    np.testing.assert_allclose(vc, full.v_combined.cpu().numpy(), rtol=1e-4, atol=1e-9)

    rng = np.random.default_rng(step)
    w_t = rng.integers(0, 1 << 32, (n, 10), dtype=np.uint64).astype(np.uint32) & np.uint32(0x4FFF7FFF)
    w_o = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32) & np.uint32(0x4FFF7FFF)
    w_t[: n // 10] = 0                       # reset moments
    lr_scale = np.array([1.6e-4, 1.6e-4, 1.6e-4, 1e-3, 1e-3, 1e-3, 1e-3, 5e-3, 5e-3, 5e-3], np.float32)
    adam = va.FusedAdam.at_step(step, lr_opac=0.05, epsilon=EPS, opac_reg=opac_reg)
    tg, og = t.clone(), o.clone()
    wtg, wog = _words(w_t), _words(w_o)
    res = va.project_update(out, tg, s, og, fused.v_combined, wtg, torch.from_numpy(lr_scale).cuda(), wog, adam)

    ref = po.render_forward(cam, w.img_size, sc.transforms, sc.sh_coeffs, sc.raw_opacities, flags=po.FLAG_BWD_INFO)
    oa = po.OrAdam(adam.beta1, adam.beta2, adam.inv1, adam.inv2, adam.epsilon, adam.lr_opac, adam.opac_reg,
                   adam.round_seed)
    want = ref.project_update(vc, sc.transforms, sc.raw_opacities, w_t, lr_scale, w_o, oa)

    cfg_rows = res.compact_from_global.cpu().numpy()
    vis = np.zeros(n, bool)
    vis[ref.get(po.F_GLOBAL_FROM_COMPACT)] = True
    np.testing.assert_array_equal(cfg_rows, np.where(vis, np.arange(n) + 1, 0))
    np.testing.assert_array_equal(res.color_dir.cpu().numpy(), want["color_dir"])
    np.testing.assert_array_equal(res.v_refine_weight.cpu().numpy(), want["v_refine"])
    np.testing.assert_array_equal(res.coeffs_grad_sq.cpu().numpy().reshape(-1), want["grad_sq"])

    got_t, got_o = tg.cpu().numpy(), og.cpu().numpy()
    got_wt, got_wo = wtg.cpu().numpy().view(np.uint32), wog.cpu().numpy().view(np.uint32)
    # Same inputs, same operation sequence: stepped parameters and moment
    # words agree bit for bit.
    np.testing.assert_array_equal(got_t.view(np.uint32), want["transforms"].view(np.uint32))
    np.testing.assert_array_equal(got_o.view(np.uint32), want["raw_opac"].view(np.uint32))
    np.testing.assert_array_equal(got_wt, want["w_t"])
    np.testing.assert_array_equal(got_wo, want["w_o"])
    assert (got_t != sc.transforms).any() and (got_wt != w_t).any()     # the step did move them
    out.state.free()


@pytest.mark.parametrize("cfg,n,view,step,opac_reg", [("c1", None, 0, 1, 0.0), ("c2", 20_000, 0, 7, 2e-7),
                                                      ("c5", 20_000, 0, 40, 0.0), ("c3", None, 2, 3, 1e-6)])
def test_project_update_parity(cfg, n, view, step, opac_reg):
    _update_case(cfg, n, view, step, opac_reg)


def test_fused_training_reduces_loss():
    """Twenty fused steps (render, L1 cotangent, fused backward, project_update)
    fit a perturbed copy of a scene towards the original's image."""
    w = scenes.workload("c1", 3000)
    cam = w.cameras[0].uniforms(w.img_size)
    t0, s, o0 = to_gpu(w.scene)
    gt = va.render(cam, w.img_size, t0, s, o0, pass_=va.RasterPass.FLOAT).out_img[..., :3].contiguous()
    g = torch.Generator(device="cpu").manual_seed(5)
    t = t0.clone()
    t[:, 0:3] += (torch.randn((t.shape[0], 3), generator=g) * 0.01).cuda()
    o = o0.clone()
    n = t.shape[0]
    w_t = torch.zeros((n, 10), dtype=torch.int32, device="cuda")
    w_o = torch.zeros(n, dtype=torch.int32, device="cuda")
    lr_scale = torch.tensor([2e-3] * 3 + [0.0] * 7, dtype=torch.float32, device="cuda")
    losses = []
    for step in range(1, 21):
        out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
        losses.append(float((out.out_img[..., :3] - gt).abs().mean()))
        v = va.l1_cotangent(out.out_img, gt, (0.0, 0.0), 0.0)
        gr = va.render_backward(out, t, s, o, v, fused=True)
        va.project_update(out, t, s, o, gr.v_combined, w_t, lr_scale, w_o,
                          va.FusedAdam.at_step(step, lr_opac=0.0, epsilon=EPS))
        out.state.free()
    assert np.isfinite(losses).all()
    assert losses[-1] < 0.7 * losses[0], losses
