"""Lagged counts of training renders (crates/splat-train-render/src/render.rs:
38-304, 741-768, 887-915) on the GPU.

* Without an overflow a lagged render (capacity hint, every stage after the
  projection on device counts, no wait) is bit-identical to the exact render
  of the same view: image, visibility, tile ranges and the sorted
  intersection list; its gradients meet the contract bar against the exact
  render's; its reported counts are the previous lagged render's.
* On an overflow the list keeps exactly the intersections whose depth-ordered
  slot lies below the capacity (the farthest splats' tiles are dropped): the
  exact list filtered to the splats that kept all their tiles, in the same
  order, plus at most one partly kept splat; tiles that lost nothing render
  bit-identically; the overflow is counted and logged, and the grown hint
  makes the next lagged render exact again.
Each test runs on a context of its own so capacity hints of other tests do
not leak in.
"""
import numpy as np
import pytest
import torch

import vauss_amd as va
from tests._util import gpu_state_arrays, l1_cotangent_np, to_gpu
from tests.test_gpu_parity import _check_grads
from vauss_amd import scenes

pytestmark = pytest.mark.gpu

TILE = 16
_KEEP = []          # contexts stay alive: forward states hold them


@pytest.fixture
def lagged_ctx():
    idx = torch.cuda.current_device()
    old = va.Context._cache.get(idx)
    ctx = va.Context(idx)
    _KEEP.append(ctx)
    va.Context._cache[idx] = ctx
    ctx.set_lagged_counts(True)
    try:
        yield ctx
    finally:
        ctx.set_lagged_counts(False)
        if old is None:
            va.Context._cache.pop(idx, None)
        else:
            va.Context._cache[idx] = old


def _list(out):
    """(tile ids, ids, ranges) of the sorted intersection list, valid part only."""
    a = gpu_state_arrays(out)
    ranges = a["ranges"].reshape(-1, 2)
    n = int(ranges[:, 1].max()) if ranges.size else 0
    return a["tile"][:n], a["gid"][:n], ranges, a


def _render(ctx, cam, size, t, s, o, pass_=va.RasterPass.BACKWARD, lagged=True):
    ctx.set_lagged_counts(lagged)
    try:
        return va.render(cam, size, t, s, o, pass_=pass_)
    finally:
        ctx.set_lagged_counts(True)


def test_lagged_render_matches_exact(lagged_ctx):
    w = scenes.workload("c3", 20_000)
    sc = w.scene
    t, s, o = to_gpu(sc)
    cams = [c.uniforms(w.img_size) for c in w.cameras[:3]]
    print("[case] c3 n=20000 views 0..2, lagged", flush=True)
    r0 = _render(lagged_ctx, cams[0], w.img_size, t, s, o)          # first at this size: exact, seeds the hint
    e0 = _render(lagged_ctx, cams[0], w.img_size, t, s, o, lagged=False)
    assert (r0.aux.num_visible, r0.aux.num_intersections) == (e0.aux.num_visible, e0.aux.num_intersections)
    assert r0.state.view().num_intersections == e0.aux.num_intersections

    r1 = _render(lagged_ctx, cams[1], w.img_size, t, s, o)          # lagged: counts not known yet
    e1 = _render(lagged_ctx, cams[1], w.img_size, t, s, o, lagged=False)
    assert (r1.aux.num_visible, r1.aux.num_intersections) == (0, 0)
    v1 = r1.state.view()
    assert v1.num_intersections >= e1.aux.num_intersections > 10_000      # capacity, not the count
    np.testing.assert_array_equal(r1.out_img.cpu().numpy().view(np.uint32), e1.out_img.cpu().numpy().view(np.uint32))
    np.testing.assert_array_equal(r1.aux.visible.cpu().numpy(), e1.aux.visible.cpu().numpy())
    lt, lg, lr, la = _list(r1)
    et, eg, er, ea = _list(e1)
    assert len(et) == e1.aux.num_intersections
    np.testing.assert_array_equal(lr, er)
    np.testing.assert_array_equal(lt, et)
    np.testing.assert_array_equal(lg, eg)
    np.testing.assert_array_equal(la["counts"], ea["counts"])
    np.testing.assert_array_equal(la["proj_a"].view(np.uint32), ea["proj_a"].view(np.uint32))

    v_out = torch.from_numpy(l1_cotangent_np(e1.out_img.cpu().numpy(), scenes.loss_target(w.img_size))).cuda()
    gl = va.render_backward(r1, t, s, o, v_out)
    ge = va.render_backward(e1, t, s, o, v_out)
    lc, ec = gl.v_combined.cpu().numpy(), ge.v_combined.cpu().numpy()
    _check_grads(lc[:, 0:5], ec[:, 0:5], "v_xy_conic")
    _check_grads(lc[:, 5:9], ec[:, 5:9], "v_rgb_opacity")
    _check_grads(gl.v_transforms.cpu().numpy(), ge.v_transforms.cpu().numpy(), "v_transforms")

    # Forward-only passes stay exact with lagged counts on.
    f1 = _render(lagged_ctx, cams[1], w.img_size, t, s, o, pass_=va.RasterPass.FLOAT)
    assert f1.aux.num_intersections == e1.aux.num_intersections

    r2 = _render(lagged_ctx, cams[2], w.img_size, t, s, o)          # reports r1's counts
    assert (r2.aux.num_visible, r2.aux.num_intersections) == (e1.aux.num_visible, e1.aux.num_intersections)
    assert lagged_ctx.settle_lagged_counts() == (2, 0)
    for x in (r0, e0, r1, e1, f1, r2):
        if x.state is not None:
            x.state.free()


def test_overflow_clamps_farthest_and_grows(lagged_ctx, capfd):
    w = scenes.workload("c2", 20_000)
    sc = w.scene
    small = sc.transforms.copy()
    small[:, 7:10] -= 1.0                                          # e^-1 scales: far fewer intersections
    cam = w.cameras[0].uniforms(w.img_size)
    t, s, o = to_gpu(sc)
    ts = torch.from_numpy(small).cuda()
    print("[case] c2 n=20000 view 0, small-scale seed then full scale, lagged", flush=True)
    r_small = _render(lagged_ctx, cam, w.img_size, ts, s, o)       # exact: hint = 1.5x its count
    seed = r_small.aux.num_intersections
    r = _render(lagged_ctx, cam, w.img_size, t, s, o)              # lagged at that hint: overflows
    cap = r.state.view().num_intersections
    e = _render(lagged_ctx, cam, w.img_size, t, s, o, lagged=False)
    need = e.aux.num_intersections
    assert cap == seed + (seed + 1) // 2 and cap < need, (seed, cap, need)

    lt, lg, lr, la = _list(r)
    et, eg, er, ea = _list(e)
    assert len(lt) == cap                                          # filled to the capacity
    counts = ea["counts"].astype(np.int64)
    np.testing.assert_array_equal(la["counts"], ea["counts"])
    # Slots in depth order: emitters sorted by (depth key, id), exclusive prefix of their counts.
    emit = np.nonzero(counts > 0)[0]
    order = emit[np.lexsort((emit, ea["depth_bits"][emit]))]
    base = np.zeros(len(counts), np.int64)
    base[order] = np.concatenate([[0], np.cumsum(counts[order])[:-1]])
    kept = np.clip(cap - base, 0, counts)
    full = (kept == counts) & (counts > 0)
    partial = (kept > 0) & (kept < counts)
    assert partial.sum() <= 1 and kept.sum() == cap
    assert np.all(kept[lg] > 0)                                    # nothing of a dropped splat
    lf, ef = full[lg], full[eg]
    np.testing.assert_array_equal(lt[lf], et[ef])                  # whole splats: same pairs, same order
    np.testing.assert_array_equal(lg[lf], eg[ef])
    assert int((~lf).sum()) == int(kept[partial].sum())
    # Tiles that lost nothing render bit for bit as in the exact render.
    ll = (lr[:, 1] - lr[:, 0]).astype(np.int64)
    el = (er[:, 1] - er[:, 0]).astype(np.int64)
    same = (ll == el).reshape(la["ranges"].shape[:2])
    assert 0 < same.mean() < 1
    pix = np.repeat(np.repeat(same, TILE, 0), TILE, 1)[:w.img_size[1], :w.img_size[0]]
    li = r.out_img.cpu().numpy().view(np.uint32)
    ei = e.out_img.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(li[pix], ei[pix])
    assert np.isfinite(r.out_img.cpu().numpy()).all()

    assert lagged_ctx.settle_lagged_counts() == (1, 1)
    err = capfd.readouterr().err
    assert "intersection capacity overflow" in err and f"required={need}" in err

    r2 = _render(lagged_ctx, cam, w.img_size, t, s, o)             # the grown hint covers it
    assert r2.state.view().num_intersections == need + (need + 1) // 2
    assert (r2.aux.num_visible, r2.aux.num_intersections) == (0, 0)   # the settle above took r's counts
    t2, g2, rr2, _ = _list(r2)
    np.testing.assert_array_equal(rr2, er)
    np.testing.assert_array_equal(g2, eg)
    np.testing.assert_array_equal(r2.out_img.cpu().numpy().view(np.uint32), ei)
    r3 = _render(lagged_ctx, cam, w.img_size, t, s, o)             # reports r2's (unclamped) counts
    assert (r3.aux.num_visible, r3.aux.num_intersections) == (e.aux.num_visible, need)
    assert lagged_ctx.settle_lagged_counts() == (3, 1)
    assert "lagged render counts: 1 overflows / 3 renders" in capfd.readouterr().err
    for x in (r_small, r, e, r2, r3):
        x.state.free()


def test_lagged_surfel_render_matches_exact(lagged_ctx):
    """Surfel training renders on lagged counts: the same list, 12-channel
    image and raster gradients as an exact render of the view."""
    w = scenes.workload("c3", 20_000)
    t, s, o = to_gpu(w.scene)
    cams = [c.uniforms(w.img_size) for c in w.cameras[:2]]
    print("[case] c3 n=20000 views 0..1, surfel, lagged", flush=True)
    mode = va.SplatRenderMode.SURFEL

    def render(cam, lagged):
        lagged_ctx.set_lagged_counts(lagged)
        try:
            return va.render(cam, w.img_size, t, s, o, render_mode=mode)
        finally:
            lagged_ctx.set_lagged_counts(True)
    r0 = render(cams[0], True)                     # seeds the hint at this size
    r1 = render(cams[1], True)
    e1 = render(cams[1], False)
    assert (r1.aux.num_visible, r1.aux.num_intersections) == (0, 0)
    np.testing.assert_array_equal(r1.out_img.cpu().numpy().view(np.uint32), e1.out_img.cpu().numpy().view(np.uint32))
    lt, lg, lr, _ = _list(r1)
    et, eg, er, _ = _list(e1)
    np.testing.assert_array_equal(lr, er)
    np.testing.assert_array_equal(lg, eg)
    v_out = torch.from_numpy(l1_cotangent_np(e1.out_img.cpu().numpy(), scenes.loss_target(w.img_size))).cuda()
    gl = va.render_backward(r1, t, s, o, v_out)
    ge = va.render_backward(e1, t, s, o, v_out)
    _check_grads(gl.v_combined.cpu().numpy(), ge.v_combined.cpu().numpy(), "v_combined (surfel)")
    _check_grads(gl.v_transforms.cpu().numpy(), ge.v_transforms.cpu().numpy(), "v_transforms (surfel)")
    assert lagged_ctx.settle_lagged_counts()[1] == 0
    for x in (r0, r1, e1):
        x.state.free()


def test_count_slots_keep_renders_apart(lagged_ctx):
    """Two training renders per step at one size in different count slots
    (RasterPass::BackwardDense { slot }, Exposure { slot }; render.rs:741-747):
    each slot keeps its own capacity hint and pending counts.  Slot 1 renders
    a small-scale cloud, slot 2 the full one: slot 2's lagged render fits its
    own hint (a single shared hint from slot 1 would overflow it), every lagged
    render is bit-identical to the exact render, and each reports its own
    slot's previous counts."""
    w = scenes.workload("c2", 20_000)
    sc = w.scene
    small = sc.transforms.copy()
    small[:, 7:10] -= 1.0
    cam = w.cameras[0].uniforms(w.img_size)
    t, s, o = to_gpu(sc)
    ts = torch.from_numpy(small).cuda()
    dense, expo = va.RasterPass.BACKWARD_DENSE, va.RasterPass.EXPOSURE
    print("[case] c2 n=20000 view 0, slots 1 (small scales) and 2 (full), lagged", flush=True)

    def render(x, pass_, slot, lagged=True):
        lagged_ctx.set_lagged_counts(lagged)
        try:
            return va.render(cam, w.img_size, x, s, o, pass_=pass_, count_slot=slot)
        finally:
            lagged_ctx.set_lagged_counts(True)

    a0 = render(ts, dense, 1)                      # exact: seeds slot 1 with the small count
    b0 = render(t, expo, 2)                        # exact: seeds slot 2 with the full count
    ea = render(ts, va.RasterPass.BACKWARD, 0, lagged=False)
    eb = render(t, va.RasterPass.BACKWARD, 0, lagged=False)
    assert ea.aux.num_intersections * 2 < eb.aux.num_intersections
    a1 = render(ts, dense, 1)
    b1 = render(t, expo, 2)
    assert (a1.aux.num_visible, a1.aux.num_intersections) == (0, 0)
    assert (b1.aux.num_visible, b1.aux.num_intersections) == (0, 0)
    cap_a, cap_b = a1.state.view().num_intersections, b1.state.view().num_intersections
    assert ea.aux.num_intersections <= cap_a < eb.aux.num_intersections <= cap_b, (cap_a, cap_b)
    for lag, ex in ((a1, ea), (b1, eb)):
        np.testing.assert_array_equal(lag.out_img.cpu().numpy().view(np.uint32), ex.out_img.cpu().numpy().view(np.uint32))
        lt, lg, lr, _ = _list(lag)
        et, eg, er, _ = _list(ex)
        np.testing.assert_array_equal(lr, er)
        np.testing.assert_array_equal(lg, eg)
    a2 = render(ts, dense, 1)                      # reports a1's counts
    b2 = render(t, expo, 2)                        # reports b1's counts
    assert (a2.aux.num_visible, a2.aux.num_intersections) == (ea.aux.num_visible, ea.aux.num_intersections)
    assert (b2.aux.num_visible, b2.aux.num_intersections) == (eb.aux.num_visible, eb.aux.num_intersections)
    assert lagged_ctx.settle_lagged_counts() == (4, 0)
    # the fused-update pass is a training pass of slot 0 whose backward stops at the raster gradients
    f = render(t, va.RasterPass.BACKWARD_FUSED_UPDATE, 0)
    v_out = torch.from_numpy(l1_cotangent_np(eb.out_img.cpu().numpy(), scenes.loss_target(w.img_size))).cuda()
    g = va.render_backward(f, t, s, o, v_out)
    assert g.v_transforms is None and g.v_combined is not None
    for x in (a0, b0, ea, eb, a1, b1, a2, b2, f):
        x.state.free()


def test_lagged_depth_sort_over_the_full_key_width(lagged_ctx):
    """A wide Kannala-Brandt camera with splats on both sides of its camera
    plane: the visible depth bits span more than 27 bits (negative z sorts
    after every positive one by raw bits, render.rs:689-694), so the depth
    sort's fourth 9-bit pass ranks instead of copying, in the lagged render
    (32-bit keys) and the exact one (bitlen of the span).  Both lists, images
    and gradients agree bit for bit / at the contract bar, and each tile's list
    is the stable order of (raw depth bits, id) of its splats."""
    from vauss_amd import camera as vcam
    img = (256, 256)
    model = vcam.KannalaBrandt4(0.01, -0.004, 0.001, -0.0002)
    cam = vcam.Camera.from_focal(40.0, 40.0, img, model=model).uniforms(img)
    rng = np.random.default_rng(78)
    n = 30_000
    d = rng.standard_normal((n, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    r = rng.uniform(2.0, 4.0, n)
    tr = np.concatenate([d * r[:, None], rng.standard_normal((n, 4)), rng.uniform(-3.2, -2.4, (n, 3))],
                        1).astype(np.float32)
    sc = scenes.Scene(tr, rng.uniform(0, 1, (n, 1, 3)).astype(np.float32), rng.uniform(0.0, 3.0, n).astype(np.float32))
    t, s, o = to_gpu(sc)
    print(f"[case] kb4 wide n={n} {img}, both sides of the camera plane, lagged", flush=True)
    r0 = _render(lagged_ctx, cam, img, t, s, o)          # seeds the hint
    r1 = _render(lagged_ctx, cam, img, t, s, o)          # lagged
    e1 = _render(lagged_ctx, cam, img, t, s, o, lagged=False)
    lt, lg, lr, la = _list(r1)
    et, eg, er, ea = _list(e1)
    db = ea["depth_bits"]
    vis = ea["counts"] > 0
    assert vis.sum() >= 4096                             # the one-sweep schedule, where 9-bit digits apply
    span = int(db[vis].max()) - int(db[vis].min())
    assert span.bit_length() > 27 and (db[vis] >= 0x80000000).sum() >= 100
    np.testing.assert_array_equal(lr, er)
    np.testing.assert_array_equal(lt, et)
    np.testing.assert_array_equal(lg, eg)
    np.testing.assert_array_equal(r1.out_img.cpu().numpy().view(np.uint32), e1.out_img.cpu().numpy().view(np.uint32))
    # each tile's entries in (raw depth bits, id) order
    key = (et.astype(np.uint64) << np.uint64(52)) | (db[eg].astype(np.uint64) << np.uint64(20)) | eg.astype(np.uint64)
    assert eg.max() < (1 << 20) and et.max() < (1 << 11)
    assert (key[1:] > key[:-1]).all()
    v_out = torch.from_numpy(l1_cotangent_np(e1.out_img.cpu().numpy(), np.full(img[::-1] + (3,), 0.5, np.float32))).cuda()
    gl = va.render_backward(r1, t, s, o, v_out)
    ge = va.render_backward(e1, t, s, o, v_out)
    _check_grads(gl.v_transforms.cpu().numpy(), ge.v_transforms.cpu().numpy(), "v_transforms")
    for x in (r0, r1, e1):
        x.state.free()
