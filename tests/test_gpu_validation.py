"""Validation readbacks and poisoned allocations at the C ABI.

* With validation on (validation.rs:1-140), a render whose parameters hold a
  NaN or Inf fails with VS_ERR_NONFINITE naming the tensor and its first bad
  element, as the reference's render panics on NaN positions
  (src/tests/mod.rs:684); values outside the reference's ranges are logged;
  a backward whose gradients come out non-finite fails the same way.
  Without validation the same render culls the splat and succeeds.
* A context that fills every library allocation with -12345.0 before use
  (crates/splat-train-cube/src/host.rs:23-36) renders, bins, differentiates
  and runs the fused update exactly as a fresh context does: no kernel reads a
  slot it did not write.
"""
import numpy as np
import pytest
import torch

import vauss_amd as va
from tests._util import gpu_state_arrays, l1_cotangent_np, to_gpu
from tests.test_gpu_parity import _check_grads
from vauss_amd import scenes

pytestmark = pytest.mark.gpu
_KEEP = []


@pytest.fixture
def own_ctx():
    """A context of its own (validation and poison stay local to the test)."""
    idx = torch.cuda.current_device()
    old = va.Context._cache.get(idx)
    ctx = va.Context(idx)
    _KEEP.append(ctx)
    va.Context._cache[idx] = ctx
    try:
        yield ctx
    finally:
        ctx.set_validation(False)
        ctx.set_poison(False)
        if old is None:
            va.Context._cache.pop(idx, None)
        else:
            va.Context._cache[idx] = old


def _small_scene(n=16):
    """The reference's NaN test scene: n splats at the origin, unit quaternions, small scales."""
    t = np.zeros((n, 10), np.float32)
    t[:, 3] = 1.0
    t[:, 7:10] = -2.0
    sh = np.full((n, 1, 3), 0.5, np.float32)
    o = np.zeros(n, np.float32)
    return t, sh, o


def _cam():
    return scenes.test_camera((32, 32), position=(0.0, 0.0, -3.0))


def test_validation_rejects_nan_positions(own_ctx):
    t, sh, o = _small_scene()
    t[1, 0] = np.nan                                   # means[3] of the reference's [16, 3] means
    args = [torch.from_numpy(x).cuda() for x in (t, sh, o)]
    print("[case] validation: NaN mean", flush=True)
    out = va.render(_cam(), (32, 32), *args)           # no validation: the splat is culled
    assert out.aux.num_visible == 15
    out.state.free()
    with pytest.raises(va.VsError, match=r"VS_ERR_NONFINITE.*'means' has 1 NaN \(first @ element 10\)"):
        va.render(_cam(), (32, 32), *args, validate=True)
    assert not own_ctx.validation


@pytest.mark.parametrize("half", [False, True], ids=["sh_f32", "sh_f16"])
def test_validation_names_each_tensor(own_ctx, half):
    t, sh, o = _small_scene()
    sh[4, 0, 2] = np.inf
    o[7] = np.nan
    o[9] = -np.inf
    s = torch.from_numpy(sh).cuda()
    if half:
        s = s.half()
    own_ctx.set_validation(True)
    print(f"[case] validation: Inf SH (half={half}), NaN/Inf opacity", flush=True)
    with pytest.raises(va.VsError) as e:
        va.render(_cam(), (32, 32), torch.from_numpy(t).cuda(), s, torch.from_numpy(o).cuda())
    msg = str(e.value)
    assert e.value.status == va._lib.VS_ERR_NONFINITE
    assert "'sh_coeffs' has 0 NaN (first @ element -1), 1 Inf (first @ element 14)" in msg
    assert "'raw_opacity' has 1 NaN (first @ element 7), 1 Inf (first @ element 9)" in msg
    assert "'means'" not in msg


def test_validation_logs_ranges(own_ctx, capfd):
    t, sh, o = _small_scene()
    t[2, 8] = 12.0                                     # log-scale above 10
    sh[3, 0, 0] = -6.0                                 # SH below -5
    o[5] = 25.0                                        # raw opacity above 20
    own_ctx.set_validation(True)
    print("[case] validation: ranges", flush=True)
    out = va.render(_cam(), (32, 32), *[torch.from_numpy(x).cuda() for x in (t, sh, o)])
    err = capfd.readouterr().err
    assert "tensor 'log_scales': 1 values > 10 of 48" in err
    assert "tensor 'sh_coeffs': 1 values < -5 of 48" in err
    assert "tensor 'raw_opacity': 1 values > 20 of 16" in err
    out.state.free()


def test_validation_of_gradients(own_ctx):
    w = scenes.workload("c1")
    t, s, o = to_gpu(w.scene)
    cam = w.cameras[0].uniforms(w.img_size)
    print("[case] validation: c1 backward with a NaN cotangent pixel", flush=True)
    out = va.render(cam, w.img_size, t, s, o)
    v = l1_cotangent_np(out.out_img.cpu().numpy(), scenes.loss_target(w.img_size))
    own_ctx.set_validation(True)
    g = va.render_backward(out, t, s, o, torch.from_numpy(v).cuda())    # finite: passes
    assert torch.isfinite(g.v_transforms).all()
    v[128, 128, 0] = np.nan
    with pytest.raises(va.VsError, match="gradient_transforms"):
        va.render_backward(out, t, s, o, torch.from_numpy(v).cuda())
    out.state.free()


@pytest.mark.parametrize("lagged", [False, True], ids=["exact", "lagged"])
def test_poisoned_allocations_change_nothing(own_ctx, lagged):
    w = scenes.workload("c2", 20_000)
    t, s, o = to_gpu(w.scene)
    cams = [c.uniforms(w.img_size) for c in w.cameras[:1]] * 2
    print(f"[case] poison: c2 n=20000 lagged={lagged}", flush=True)

    def run(poison):
        own_ctx.set_poison(poison)
        own_ctx.set_lagged_counts(lagged)
        try:
            outs = [va.render(c, w.img_size, t, s, o) for c in cams]   # the second is lagged when enabled
            out = outs[-1]
            v = l1_cotangent_np(out.out_img.cpu().numpy(), scenes.loss_target(w.img_size))
            g = va.render_backward(out, t, s, o, torch.from_numpy(v).cuda())
            fused = va.render_backward(out, t, s, o, torch.from_numpy(v).cuda(), fused=True)
            keys = torch.from_numpy(np.arange(100_000, dtype=np.uint32)[::-1].copy().view(np.int32)).cuda()
            sk, sv = va.radix_argsort(keys, keys.clone(), 32)
            res = (out.out_img.cpu().numpy(), gpu_state_arrays(out), g, fused.v_combined.cpu().numpy(),
                   sk.cpu().numpy(), sv.cpu().numpy(), out.aux.visible.cpu().numpy())
            for x in outs:
                x.state.free()
            return res
        finally:
            own_ctx.set_lagged_counts(False)
            own_ctx.set_poison(False)

    a = run(False)
    b = run(True)
    np.testing.assert_array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
    sa, sb = a[1], b[1]
    np.testing.assert_array_equal(sa["ranges"], sb["ranges"])
    np.testing.assert_array_equal(sa["counts"], sb["counts"])
    used = int(sa["ranges"].reshape(-1, 2)[:, 1].max())      # the list's valid part (a lagged arena is larger)
    assert used > 10_000
    for k in ("tile", "gid"):
        np.testing.assert_array_equal(sa[k][:used], sb[k][:used], err_msg=k)
    hits = sa["counts"] > 0                                 # rows the projection wrote for binned splats
    for k in ("proj_a", "proj_b", "proj_c"):
        np.testing.assert_array_equal(sa[k][hits].view(np.uint32), sb[k][hits].view(np.uint32), err_msg=k)
    np.testing.assert_array_equal(a[6], b[6])
    _check_grads(b[2].v_combined.cpu().numpy(), a[2].v_combined.cpu().numpy(), "v_combined")
    _check_grads(b[2].v_transforms.cpu().numpy(), a[2].v_transforms.cpu().numpy(), "v_transforms")
    _check_grads(b[3], a[3], "v_combined (fused)")
    np.testing.assert_array_equal(a[4], b[4])
    np.testing.assert_array_equal(a[5], b[5])
