"""GPU parity at the workloads' full sizes against the CPU oracle.

Each case renders one view of a benchmark workload at its full size (200k,
1M, 2M and 3M splats) on the GPU and in the oracle on the same seeded
inputs, then checks:
  * per-splat tile counts, the sorted (tile, depth, splat) order, tile ranges,
    projected rows and aux outputs bit for bit, and the RGBA image bit for bit
    (bar: 1e-4 absolute);
  * per-splat gradients within 1e-3 relative / 1e-5 absolute (f32 atomics
    reorder the per-splat sums), and the projection backward on its own
    against the oracle's projection VJP of the same raster gradients;
  * properties that hold at any size without the oracle: every splat's
    intersections appear exactly `count` times, tile ranges partition the
    sorted list, the list is ordered by (tile, depth bits, splat id), and the
    backward is linear in the image cotangent.
The 3M-splat heavy-tailed case has 3.6e8 intersections; the oracle's render
of it takes ~20 s on the host's cores.  These checks run on the full lists
(the depth cutoff is off by default); the same view is then rendered with the
depth cutoff opted in and checked against the same oracle render: every
tile's list is the front of the full one and covers what the tile consumes,
the image, consumed ranges and gradients are unchanged, and the aux tile
offsets are the full list's shrunk ranges moved to each tile's start in the
shortened list.
"""
import time

import numpy as np
import pytest
import torch

import vauss_amd as va
from oracle import pyoracle as po
from tests._util import circle_mask, gpu_state_arrays, l1_cotangent_np, to_gpu
from tests.test_gpu_cutoff import _check_cut_lists, _check_cut_offsets, _consumed
from tests.test_gpu_parity import _check_forward, _check_grads, _check_param_grads
from vauss_amd import scenes

pytestmark = pytest.mark.gpu


def _log(msg):
    print(f"[fullsize] {time.strftime('%H:%M:%S')} {msg}", flush=True)


def _check_list_properties(gpu, n):
    """Oracle-independent invariants of the binned, sorted intersection list."""
    tile, gid, counts, ranges = gpu["tile"], gpu["gid"], gpu["counts"], gpu["ranges"]
    t_count = ranges.shape[0] * ranges.shape[1]
    # every splat's slots appear exactly `count` times (no slot lost or duplicated)
    np.testing.assert_array_equal(np.bincount(gid, minlength=n), counts)
    # sorted by tile, and inside a tile by (depth bits, splat id)
    assert (np.diff(tile.astype(np.int64)) >= 0).all()
    same = tile[1:] == tile[:-1]
    d = gpu["depth_bits"][gid].astype(np.int64)
    key = d * n + gid            # (depth bits, id) as one exact int64 key
    assert (np.diff(key)[same] > 0).all()
    # ranges partition the non-sentinel prefix of the list
    flat = ranges.reshape(t_count, 2).astype(np.int64)
    real = tile < t_count
    lens = np.maximum(flat[:, 1] - flat[:, 0], 0)
    assert lens.sum() == real.sum()
    np.testing.assert_array_equal(lens, np.bincount(tile[real], minlength=t_count))


@pytest.mark.parametrize("cfg,view", [("c2", 0), ("c3", 6), ("c5", 0), ("c4", 0)])
def test_full_size_parity(cfg, view):
    _log(f"case {cfg} view {view}: generating the workload")
    w = scenes.workload(cfg)
    n = w.scene.num_splats
    cam = w.cameras[view].uniforms(w.img_size)
    t, s, o = to_gpu(w.scene)
    _log(f"{cfg}: GPU render of {n} splats at {w.img_size}")
    ctx = va.Context.get(torch.device("cuda", 0))
    ctx.set_depth_cutoff(ctx.CUTOFF_OFF)
    try:
        out = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
        torch.cuda.synchronize()
    finally:
        ctx.set_depth_cutoff(ctx.CUTOFF_OFF)
    gpu = gpu_state_arrays(out)
    _log(f"{cfg}: {out.aux.num_visible} visible, {out.aux.num_intersections} intersections; oracle forward")
    ref = po.render_forward(cam, w.img_size, w.scene.transforms, w.scene.sh_coeffs, w.scene.raw_opacities,
                            flags=po.FLAG_BWD_INFO)
    _log(f"{cfg}: comparing the forward")
    _check_list_properties(gpu, n)
    _check_forward(out, ref, gpu)
    img = out.out_img.cpu().numpy()
    rimg = ref.get(po.F_OUT_IMG)
    diff = np.abs(img - rimg)
    assert diff.max() <= 1e-4, f"max |rgba diff| {diff.max()}"
    assert np.array_equal(img.view(np.uint32), rimg.view(np.uint32)), f"{(diff > 0).sum()} channels differ in the last bits"
    np.testing.assert_array_equal(out.aux.visible.cpu().numpy(), ref.get(po.F_VISIBLE))
    np.testing.assert_array_equal(out.aux.tile_offsets.cpu().numpy().view(np.uint32), ref.get(po.F_TILE_OFFSETS_SHRUNK))
    del gpu

    mask = circle_mask(w.img_size, w.mask_center, w.mask_radius) if w.mask_radius > 0 else None
    v_out = l1_cotangent_np(img, scenes.loss_target(w.img_size), mask)
    v_dev = torch.from_numpy(v_out).cuda()
    _log(f"{cfg}: backward (GPU, then oracle)")
    g = va.render_backward(out, t, s, o, v_dev)
    g2 = va.render_backward(out, t, s, o, v_dev * 2.0)
    rg = ref.backward(v_out)
    vc = g.v_combined.cpu().numpy()
    _check_grads(vc[:, 0:2], rg["v_combined"][:, 0:2], "v_xy")
    _check_grads(vc[:, 2:5], rg["v_combined"][:, 2:5], "v_conic")
    _check_grads(vc[:, 5:8], rg["v_combined"][:, 5:8], "v_rgb")
    _check_grads(vc[:, 8], rg["v_combined"][:, 8], "v_opacity")
    _check_grads(vc[:, 9], rg["v_combined"][:, 9], "v_refine")
    _check_param_grads(g, rg, ref, vc)
    # linearity in the cotangent: doubling it doubles every raster gradient
    # (exact per term; only the atomic summation order may differ)
    _check_grads(g2.v_combined.cpu().numpy(), 2.0 * vc, "v_combined under a doubled cotangent")
    out.state.free()

    _log(f"{cfg}: depth cutoff on")
    ctx.set_depth_cutoff(ctx.CUTOFF_ON)
    try:
        cut = va.render(cam, w.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
        torch.cuda.synchronize()
    finally:
        ctx.set_depth_cutoff(ctx.CUTOFF_OFF)
    gc = gpu_state_arrays(cut)
    t_count = gc["ranges"].shape[0] * gc["ranges"].shape[1]
    listed, full = _check_cut_lists(gc, ref, t_count)
    _log(f"{cfg}: {listed} of {full} pairs listed under the cutoff")
    assert np.array_equal(cut.out_img.cpu().numpy().view(np.uint32), rimg.view(np.uint32))
    np.testing.assert_array_equal(_consumed(cut.aux.tile_offsets.cpu().numpy()), _consumed(ref.get(po.F_TILE_OFFSETS_SHRUNK)))
    # with the cutoff opted in, the aux offsets index the shortened list: the
    # full list's shrunk ranges moved to each tile's start in it
    _check_cut_offsets(cut.aux.tile_offsets.cpu().numpy(), gc["ranges"], ref)
    del gc
    gcut = va.render_backward(cut, t, s, o, v_dev)
    _check_grads(gcut.v_combined.cpu().numpy(), vc, "v_combined (cutoff vs full lists)")
    cut.state.free()
    _log(f"{cfg}: done")
