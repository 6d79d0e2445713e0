"""GPU parity of the SH step (crates/splat-train/src/optim.rs:391-498,
quant.rs, quant_kernels.rs) and of f16 SH coefficients in the render path
(render.rs:683-687, bwd/render_bwd.rs:275,384, bwd/project_update.rs:210)
against the CPU oracle on identical inputs.

Bars: the Block8 codec and the SH step bit for bit (coefficient bits,
variance, codes, scales; stochastic rounding included).  f16 rendering: the
oracle renders the same coefficients widened to f32 (exact), so the forward is
bit for bit, the fused update bit for bit, and the dense gradients meet the
backward contract (1e-3 relative / 1e-5 absolute).
"""
import numpy as np
import pytest
import torch

import vauss_amd as va
from oracle import pyoracle as po
from tests._util import circle_mask, gpu_state_arrays, l1_cotangent_np, to_gpu
from vauss_amd import scenes

pytestmark = pytest.mark.gpu


def _i32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32).copy()).cuda()


def test_block8_codec_bit_for_bit():
    rng = np.random.default_rng(21)
    n = 128 * 300 + 77
    v = (rng.standard_normal(n) * 10.0 ** rng.uniform(-9, 3, n)).astype(np.float32)
    v[:128] = 0.0                                   # an all-zero block
    v[200] = 1e30
    m = va.Block8Moment.encode(torch.from_numpy(v).cuda())
    rc, rs = po.block8_encode(v)
    np.testing.assert_array_equal(m.codes.cpu().numpy().view(np.uint32), rc)
    np.testing.assert_array_equal(m.scales.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    codes = rng.integers(0, 1 << 32, rc.size, dtype=np.uint64).astype(np.uint32)
    scales = (10.0 ** rng.uniform(-8, 2, rs.size)).astype(np.float32)
    mm = va.Block8Moment(_i32(codes), torch.from_numpy(scales).cuda(), n)
    np.testing.assert_array_equal(mm.decode().cpu().numpy().view(np.uint32),
                                  po.block8_decode(codes, scales, n).view(np.uint32))
    rows = np.array([0, 5, 17, 300, 10 ** 6], np.uint32)    # the last row is past the end: ignored
    mm.zero_rows(torch.from_numpy(rows.view(np.int32)).cuda(), 27)
    np.testing.assert_array_equal(mm.codes.cpu().numpy().view(np.uint32), po.block8_zero_rows(codes, n, rows, 27))


def _synthetic(degree, n, seed, first):
    rng = np.random.default_rng(seed)
    k = (degree + 1) ** 2
    sh = rng.uniform(-2, 2, (n, k, 3)).astype(np.float16)
    vis = rng.uniform(size=n) < 0.5
    vis[n // 3: n // 3 + 200] = False                       # whole blocks without a visible splat
    rows = np.where(vis, np.arange(n) + 1, 0).astype(np.uint32)
    cd = np.zeros((n + 1, 6), np.float32)
    cd[1:, :3] = rng.standard_normal((n, 3)) * 1e-3
    d = rng.standard_normal((n, 3))
    cd[1:, 3:] = d / np.linalg.norm(d, axis=1, keepdims=True)
    gsq = np.where(vis, rng.uniform(1e-9, 1e-6, n), 0.0).astype(np.float32)
    nv = n * k * 3
    blocks = (nv + 127) // 128
    if first:
        codes, scales, var = np.zeros(blocks * 32, np.uint32), np.zeros(blocks, np.float32), np.zeros(n, np.float32)
    else:
        codes, scales = po.block8_encode((rng.standard_normal(nv) * 1e-4).astype(np.float32))
        var = rng.uniform(0, 1e-6, n).astype(np.float32)
    lr_scale = np.where(np.arange(k * 3) < 3, 1.0, 0.05).astype(np.float32)
    return sh, cd, rows, gsq, var, codes, scales, lr_scale


def _run_both(sh, cd, rows, gsq, var, codes, scales, lr_scale, time, lr=2.5e-3):
    n = sh.shape[0]
    inv1, inv2 = va.adam_bias_corrections(time + 1, 0.9, 0.999)
    want = po.sh_step(sh, cd, rows, gsq, var, codes, scales, lr_scale, beta1=0.9, beta2=0.999, inv1=inv1,
                      inv2=inv2, epsilon=1e-15, lr=lr, round_seed=time + 1, first=time == 0)
    st = va.ShStepState(va.Block8Moment(_i32(codes), torch.from_numpy(scales.copy()).cuda(), sh.size),
                        torch.from_numpy(var.copy()).cuda(), time)
    got = va.sh_step(torch.from_numpy(sh.copy()).cuda(), torch.from_numpy(cd).cuda(),
                     torch.from_numpy(rows.view(np.int32)).cuda(), torch.from_numpy(gsq).cuda(), st, lr,
                     torch.from_numpy(lr_scale).cuda())
    assert st.time == time + 1 and got.shape == sh.shape and n > 0
    return want, (got.cpu().numpy(), st.variance.cpu().numpy(), st.moment.codes.cpu().numpy().view(np.uint32),
                  st.moment.scales.cpu().numpy())


def _assert_same(want, got):
    np.testing.assert_array_equal(got[0].view(np.uint16), want[0].view(np.uint16))
    np.testing.assert_array_equal(got[1].view(np.uint32), want[1].view(np.uint32))
    np.testing.assert_array_equal(got[2], want[2])
    np.testing.assert_array_equal(got[3].view(np.uint32), want[3].view(np.uint32))


@pytest.mark.parametrize("degree", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("first", [True, False])
def test_sh_step_synthetic(degree, first):
    n = 1531                                                 # rows end mid-block and mid-word
    print(f"[case] degree={degree} first={first} n={n}", flush=True)
    case = _synthetic(degree, n, 100 + degree, first)
    want, got = _run_both(*case, time=0 if first else 6)
    _assert_same(want, got)
    vis = case[2] != 0
    assert (got[0][vis].view(np.uint16) != case[0][vis].view(np.uint16)).any()
    np.testing.assert_array_equal(got[0][~vis].view(np.uint16), case[0][~vis].view(np.uint16))


@pytest.mark.parametrize("cfg,n,view", [("c2", 20_000, 0), ("c5", 20_000, 0)])
def test_f16_render_parity(cfg, n, view):
    """Forward bit for bit, dense gradients at the contract bar, fused update
    bit for bit, all with f16 coefficients."""
    w = scenes.workload(cfg, n)
    sc = w.scene
    cam = w.cameras[view].uniforms(w.img_size)
    sh16 = sc.sh_coeffs.astype(np.float16)
    t, _, o = to_gpu(sc)
    s = torch.from_numpy(sh16).cuda()
    print(f"[case] {cfg} n={sc.num_splats} view={view} f16 SH", flush=True)
    out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
    ref = po.render_forward(cam, w.img_size, sc.transforms, sh16.astype(np.float32), sc.raw_opacities,
                            flags=po.FLAG_BWD_INFO)
    img = out.out_img.cpu().numpy()
    np.testing.assert_array_equal(img.view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))
    gpu = gpu_state_arrays(out)
    np.testing.assert_array_equal(gpu["gid"], ref.get(po.F_ISECT_GID))
    gfc = ref.get(po.F_GLOBAL_FROM_COMPACT)
    proj = ref.get(po.F_PROJECTED)
    np.testing.assert_array_equal(gpu["proj_b"][gfc][:, 2:4].view(np.uint32), proj[:, 6:8].view(np.uint32))
    mask = circle_mask(w.img_size, w.mask_center, w.mask_radius) if w.mask_radius > 0 else None
    v_out = l1_cotangent_np(img, scenes.loss_target(w.img_size), mask)
    g = va.render_backward(out, t, s, o, torch.from_numpy(v_out).cuda())
    vc = g.v_combined.cpu().numpy()
    pg = ref.project_backward(vc)
    np.testing.assert_allclose(g.v_coeffs.cpu().numpy(), pg["v_sh"], rtol=1e-5, atol=1e-12)
    err = np.abs(g.v_transforms.cpu().numpy() - pg["v_transforms"])
    assert (err <= 1e-5 * np.abs(pg["v_transforms"]) + 1e-3 * np.abs(pg["v_transforms"]).max(axis=0)).all()
    # fused update on f16 coefficients, fed the GPU's raster gradients
    nn = sc.num_splats
    rng = np.random.default_rng(3)
    w_t = rng.integers(0, 1 << 32, (nn, 10), dtype=np.uint64).astype(np.uint32) & np.uint32(0x4FFF7FFF)
    w_o = rng.integers(0, 1 << 32, nn, dtype=np.uint64).astype(np.uint32) & np.uint32(0x4FFF7FFF)
    lr_scale = np.full(10, 1e-3, np.float32)
    adam = va.FusedAdam.at_step(4, lr_opac=0.05)
    tg, og, wtg, wog = t.clone(), o.clone(), _i32(w_t), _i32(w_o)
    res = va.project_update(out, tg, s, og, g.v_combined, wtg, torch.from_numpy(lr_scale).cuda(), wog, adam)
    oa = po.OrAdam(adam.beta1, adam.beta2, adam.inv1, adam.inv2, adam.epsilon, adam.lr_opac, adam.opac_reg,
                   adam.round_seed)
    want = ref.project_update(vc, sc.transforms, sc.raw_opacities, w_t, lr_scale, w_o, oa)
    np.testing.assert_array_equal(res.color_dir.cpu().numpy(), want["color_dir"])
    np.testing.assert_array_equal(tg.cpu().numpy().view(np.uint32), want["transforms"].view(np.uint32))
    np.testing.assert_array_equal(wtg.cpu().numpy().view(np.uint32), want["w_t"])
    out.state.free()


def test_fused_step_with_sh_step_parity():
    """The trainer's fused pass end to end on the GPU (render, fused backward,
    project_update, SH step); the SH step's outputs match the oracle's fed the
    GPU's color_dir and grad_sq, over two consecutive steps."""
    w = scenes.workload("c2", 20_000)
    sc = w.scene
    cam = w.cameras[0].uniforms(w.img_size)
    t, s32, o = to_gpu(sc)
    s = s32.half()
    n, k = sc.sh_coeffs.shape[:2]
    st = va.ShStepState.fresh(n, 3, "cuda")
    w_t = torch.zeros((n, 10), dtype=torch.int32, device="cuda")
    w_o = torch.zeros(n, dtype=torch.int32, device="cuda")
    lr_t = torch.full((10,), 1e-4, device="cuda")
    lr_sh = torch.from_numpy(np.where(np.arange(k * 3) < 3, 1.0, 0.05).astype(np.float32)).cuda()
    gt = torch.from_numpy(scenes.loss_target(w.img_size)).cuda()
    for step in (1, 2):
        print(f"[case] fused step {step}", flush=True)
        out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
        v = va.l1_cotangent(out.out_img, gt, (0.0, 0.0), 0.0)
        gr = va.render_backward(out, t, s, o, v, fused=True)
        res = va.project_update(out, t, s, o, gr.v_combined, w_t, lr_t, w_o, va.FusedAdam.at_step(step, lr_opac=0.05))
        before = (s.cpu().numpy(), st.variance.cpu().numpy(), st.moment.codes.cpu().numpy().view(np.uint32),
                  st.moment.scales.cpu().numpy())
        cd, rows = res.color_dir.cpu().numpy(), res.compact_from_global.cpu().numpy().view(np.uint32)
        gsq = res.coeffs_grad_sq.cpu().numpy().reshape(-1)
        time = st.time
        s = va.sh_step(s, res.color_dir, res.compact_from_global, res.coeffs_grad_sq, st, 2.5e-3, lr_sh)
        inv1, inv2 = va.adam_bias_corrections(time + 1, 0.9, 0.999)
        want = po.sh_step(before[0], cd, rows, gsq, before[1], before[2], before[3], lr_sh.cpu().numpy(), beta1=0.9,
                          beta2=0.999, inv1=inv1, inv2=inv2, epsilon=1e-15, lr=2.5e-3, round_seed=time + 1,
                          first=time == 0)
        got = (s.cpu().numpy(), st.variance.cpu().numpy(), st.moment.codes.cpu().numpy().view(np.uint32),
               st.moment.scales.cpu().numpy())
        _assert_same(want, got)
        assert (got[0].view(np.uint16) != before[0].view(np.uint16)).any()
        out.state.free()


def test_sh_learning_reduces_colour_error():
    """Forty fused steps with the SH step fit the colours of a scene whose DC
    coefficients were perturbed (geometry learning rate 0)."""
    w = scenes.workload("c1", 3000)
    cam = w.cameras[0].uniforms(w.img_size)
    t, s0, o = to_gpu(w.scene)
    gt = va.render(cam, w.img_size, t, s0, o, pass_=va.RasterPass.FLOAT).out_img[..., :3].contiguous()
    g = torch.Generator(device="cpu").manual_seed(9)
    s = (s0 + (torch.randn(s0.shape, generator=g) * 0.2).cuda()).half()
    n = t.shape[0]
    st = va.ShStepState.fresh(n, 0, "cuda")
    w_t = torch.zeros((n, 10), dtype=torch.int32, device="cuda")
    w_o = torch.zeros(n, dtype=torch.int32, device="cuda")
    zero_lr = torch.zeros(10, device="cuda")
    losses = []
    for step in range(1, 41):
        out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
        losses.append(float((out.out_img[..., :3] - gt).abs().mean()))
        v = va.l1_cotangent(out.out_img, gt, (0.0, 0.0), 0.0)
        gr = va.render_backward(out, t, s, o, v, fused=True)
        res = va.project_update(out, t, s, o, gr.v_combined, w_t, zero_lr, w_o,
                                va.FusedAdam.at_step(step, lr_opac=0.0))
        s = va.sh_step(s, res.color_dir, res.compact_from_global, res.coeffs_grad_sq, st, 5e-3)
        out.state.free()
    assert np.isfinite(losses).all()
    assert losses[-1] < 0.5 * losses[0], losses
