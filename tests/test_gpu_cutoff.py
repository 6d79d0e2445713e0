"""GPU depth cutoff of the tile lists (vs_ctx_set_depth_cutoff).

The cutoff stops each tile's list at the depth bin by which a lower bound on
the opacity that splats lay over the whole tile has brought every pixel of it
below the stopping transmittance, so the raster never reaches what it drops.
Checked against the oracle's full lists on the same seeded inputs:
  * every tile's list is the front of the oracle's list for that tile and
    holds at least the pairs the tile's pixels consume (the oracle's shrunk
    range); each splat's listed pairs match its listed count;
  * per-splat tile counts and num_intersections still count every pair;
  * the image (and geometry channels), visibility and consumed ranges bit for
    bit, and per-splat gradients at the parity bar (1e-3 relative / 1e-5
    absolute);
and without the oracle: on the heavy-tailed workload the lists shrink to a
small part while images, consumed ranges and gradients equal the full
lists', also for lagged renders and the packed FORWARD pass.
"""
import numpy as np
import pytest
import torch

import vauss_amd as va
from oracle import pyoracle as po
from tests._util import circle_mask, gpu_state_arrays, l1_cotangent_np, to_gpu
from tests.test_gpu_parity import _check_grads
from vauss_amd import scenes

pytestmark = pytest.mark.gpu


@pytest.fixture
def ctx():
    c = va.Context.get(torch.device("cuda", 0))
    yield c
    c.set_depth_cutoff(c.CUTOFF_OFF)
    c.set_lagged_counts(False)


def _consumed(tile_offsets):
    """Pairs each tile's pixels consumed (the shrunk ranges' lengths; their
    offsets index a list whose length depends on the cutoff)."""
    r = np.asarray(tile_offsets).reshape(-1, 2).view(np.uint32).astype(np.int64)
    return np.maximum(r[:, 1] - r[:, 0], 0)


def _check_cut_lists(gpu, ref, t_count):
    """Every tile's list is the front of the oracle's full list for the tile
    and covers what the tile's pixels consume."""
    assert gpu["view"].depth_cutoff == 1
    r = gpu["ranges"].reshape(t_count, 2).astype(np.int64)
    o = ref.get(po.F_TILE_OFFSETS).reshape(t_count, 2).astype(np.int64)
    sh = ref.get(po.F_TILE_OFFSETS_SHRUNK).reshape(t_count, 2).astype(np.int64)
    glen = np.maximum(r[:, 1] - r[:, 0], 0)
    olen = np.maximum(o[:, 1] - o[:, 0], 0)
    used = np.maximum(sh[:, 1] - sh[:, 0], 0)
    assert (glen <= olen).all(), "a tile lists more than its full list"
    assert (glen >= used).all(), "a tile's list stops before what its pixels consume"
    assert gpu["view"].listed_intersections == glen.sum()
    pos = np.arange(glen.sum()) - np.repeat(np.cumsum(glen) - glen, glen)
    gi = np.repeat(r[:, 0], glen) + pos
    oi = np.repeat(o[:, 0], glen) + pos
    np.testing.assert_array_equal(gpu["gid"][gi], ref.get(po.F_ISECT_GID)[oi])
    np.testing.assert_array_equal(gpu["tile"][gi], np.repeat(np.arange(t_count), glen))
    np.testing.assert_array_equal(np.bincount(gpu["gid"][gi], minlength=gpu["listed_counts"].shape[0]),
                                  gpu["listed_counts"])
    return int(glen.sum()), int(olen.sum())


def _check_cut_offsets(tile_offsets, gpu_ranges, ref):
    """The aux tile offsets of a cut render, bit for bit: each tile's shrunk
    range of the full list (the oracle's RenderAux.tile_offsets) moved to the
    tile's start in the shortened list; tiles with an empty full list keep the
    full list's entry."""
    got = np.asarray(tile_offsets).reshape(-1, 2).view(np.uint32).astype(np.int64)
    r = np.asarray(gpu_ranges).reshape(-1, 2).astype(np.int64)
    o = ref.get(po.F_TILE_OFFSETS).reshape(-1, 2).astype(np.int64)
    sh = ref.get(po.F_TILE_OFFSETS_SHRUNK).reshape(-1, 2).astype(np.int64)
    nonempty = (o[:, 1] - o[:, 0]) > 0
    want = np.where(nonempty[:, None], sh - o[:, :1] + r[:, :1], sh)
    np.testing.assert_array_equal(got, want)


def _check_median_ids(got, want, ranges, ref_ranges):
    """Median ids (list indices, 0xFFFFFFFF for none) at the same position within each pixel's tile list."""
    h, w = got.shape
    bw = ranges.shape[1]
    tile = (np.arange(h)[:, None] // 16) * bw + (np.arange(w)[None, :] // 16)
    gstart = ranges.reshape(-1, 2)[tile, 0].astype(np.int64)
    ostart = np.asarray(ref_ranges).reshape(-1, 2)[tile, 0].astype(np.int64)
    none = want == 0xFFFFFFFF
    np.testing.assert_array_equal(got[none], want[none])
    np.testing.assert_array_equal(got[~none].astype(np.int64) - gstart[~none], want[~none].astype(np.int64) - ostart[~none])


CASES = [("c2", 20_000, 0, "BACKWARD", "DEFAULT"), ("c3", 20_000, 3, "BACKWARD", "DEFAULT"),
         ("c4", 60_000, 0, "BACKWARD", "DEFAULT"), ("c5", 20_000, 0, "BACKWARD", "DEFAULT"),
         ("c3", 20_000, 1, "BACKWARD_SMOOTH_CUTOFF", "DEFAULT"), ("c4", 60_000, 0, "GEOMETRY", "DEFAULT"),
         ("c4", 60_000, 0, "BACKWARD", "MIP")]


@pytest.mark.parametrize("cfg,n,view,pass_name,mode_name", CASES)
def test_cutoff_lists_are_fronts_of_the_full_lists(ctx, cfg, n, view, pass_name, mode_name):
    ctx.set_depth_cutoff(ctx.CUTOFF_ON)
    pass_ = va.RasterPass[pass_name]
    mode = va.SplatRenderMode[mode_name]
    w = scenes.workload(cfg, n)
    cam = w.cameras[view].uniforms(w.img_size)
    t, s, o = to_gpu(w.scene)
    print(f"[case] cutoff {cfg} n={n} view={view} pass={pass_name} mode={mode_name}", flush=True)
    out = va.render(cam, w.img_size, t, s, o, pass_=pass_, render_mode=mode)
    torch.cuda.synchronize()
    gpu = gpu_state_arrays(out)
    flags = po.FLAG_BWD_INFO
    if pass_.geometry():
        flags |= po.FLAG_GEOMETRY
    if pass_ == va.RasterPass.BACKWARD_SMOOTH_CUTOFF:
        flags |= po.FLAG_SMOOTH_CUTOFF
    if mode == va.SplatRenderMode.MIP:
        flags |= po.FLAG_MIP
    ref = po.render_forward(cam, w.img_size, w.scene.transforms, w.scene.sh_coeffs, w.scene.raw_opacities, flags=flags)
    assert out.aux.num_intersections == ref.info.num_intersections
    np.testing.assert_array_equal(gpu["counts"], ref.get(po.F_INTERSECT_COUNTS))
    t_count = gpu["ranges"].shape[0] * gpu["ranges"].shape[1]
    listed, full = _check_cut_lists(gpu, ref, t_count)
    print(f"[cutoff] {cfg}: {listed} of {full} pairs listed", flush=True)
    img = out.out_img.cpu().numpy()
    rimg = ref.get(po.F_OUT_IMG)
    if img.shape[-1] == 12:
        # the median id indexes the listed pairs: its position within the tile's list is the full list's
        _check_median_ids(img[..., 11].view(np.uint32), rimg[..., 11].view(np.uint32), gpu["ranges"],
                          ref.get(po.F_TILE_OFFSETS))
        img_cmp, rimg_cmp = img[..., :11], rimg[..., :11]
    else:
        img_cmp, rimg_cmp = img, rimg
    assert np.array_equal(img_cmp.view(np.uint32), rimg_cmp.view(np.uint32)), f"{(img_cmp != rimg_cmp).sum()} channels differ"
    np.testing.assert_array_equal(out.aux.visible.cpu().numpy(), ref.get(po.F_VISIBLE))
    np.testing.assert_array_equal(_consumed(out.aux.tile_offsets.cpu().numpy()), _consumed(ref.get(po.F_TILE_OFFSETS_SHRUNK)))
    _check_cut_offsets(out.aux.tile_offsets.cpu().numpy(), gpu["ranges"], ref)
    del gpu
    if pass_.geometry():
        out.state.free()
        return
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
    out.state.free()


def _render_pair(ctx, w, cam, t, s, o, pass_, lagged=False):
    """The same render with the cutoff off, then on (twice when lagged, so the
    second render runs on the first's capacity hint)."""
    res = []
    for mode in (ctx.CUTOFF_OFF, ctx.CUTOFF_ON):
        ctx.set_depth_cutoff(mode)
        ctx.set_lagged_counts(lagged and mode == ctx.CUTOFF_ON)
        reps = 2 if lagged and mode == ctx.CUTOFF_ON else 1
        for k in range(reps):
            out = va.render(cam, w.img_size, t, s, o, pass_=pass_)
            torch.cuda.synchronize()
            if k + 1 < reps:
                out.state.free()
        res.append(out)
    ctx.set_lagged_counts(False)
    ctx.settle_lagged_counts()
    return res


@pytest.mark.parametrize("lagged", [False, True])
def test_cutoff_shrinks_heavy_tailed_lists(ctx, lagged):
    w = scenes.workload("c4", 400_000)
    cam = w.cameras[0].uniforms(w.img_size)
    t, s, o = to_gpu(w.scene)
    print(f"[case] cutoff c4 n=400000 lagged={lagged}", flush=True)
    full, cut = _render_pair(ctx, w, cam, t, s, o, va.RasterPass.BACKWARD, lagged)
    vf, vcut = full.state.view(), cut.state.view()
    assert vf.depth_cutoff == 0 and vcut.depth_cutoff == 1
    print(f"[cutoff] listed {vcut.listed_intersections} of {vf.listed_intersections}", flush=True)
    assert vcut.listed_intersections < 0.2 * vf.listed_intersections
    assert np.array_equal(full.out_img.cpu().numpy().view(np.uint32), cut.out_img.cpu().numpy().view(np.uint32))
    np.testing.assert_array_equal(_consumed(full.aux.tile_offsets.cpu().numpy()), _consumed(cut.aux.tile_offsets.cpu().numpy()))
    np.testing.assert_array_equal(full.aux.visible.cpu().numpy(), cut.aux.visible.cpu().numpy())
    v_out = torch.from_numpy(l1_cotangent_np(full.out_img.cpu().numpy(), scenes.loss_target(w.img_size))).cuda()
    gf = va.render_backward(full, t, s, o, v_out)
    gc = va.render_backward(cut, t, s, o, v_out)
    _check_grads(gc.v_combined.cpu().numpy(), gf.v_combined.cpu().numpy(), "v_combined (cutoff vs full)")
    full.state.free()
    cut.state.free()


def test_cutoff_forward_pass_packs_the_same_image(ctx):
    w = scenes.workload("c4", 400_000)
    cam = w.cameras[0].uniforms(w.img_size)
    t, s, o = to_gpu(w.scene)
    print("[case] cutoff c4 n=400000 FORWARD", flush=True)
    res = []
    for mode in (ctx.CUTOFF_OFF, ctx.CUTOFF_ON):
        ctx.set_depth_cutoff(mode)
        res.append(va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.FORWARD).out_img.cpu().numpy())
    np.testing.assert_array_equal(res[0], res[1])


def test_cutoff_auto_turns_on_for_long_lists(ctx):
    """AUTO lists every pair of a short-list render and cuts a render with
    thousands of pairs per tile."""
    ctx.set_depth_cutoff(ctx.CUTOFF_AUTO)
    for cfg, n, want in (("c3", 100_000, 0), ("c4", 3_000_000, 1)):
        w = scenes.workload(cfg, n)
        cam = w.cameras[0].uniforms(w.img_size)
        t, s, o = to_gpu(w.scene)
        print(f"[case] cutoff auto {cfg} n={n}", flush=True)
        out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
        v = out.state.view()
        assert v.depth_cutoff == want, (cfg, v.num_intersections)
        if not want:
            assert v.listed_intersections == v.num_intersections
        out.state.free()
        del t, s, o
