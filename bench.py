"""Benchmark: fwd+bwd rasterization ms per view on one MI355X.

Workload (default): 1,000,000 SH-degree-3 Gaussians at 1920x1080 (fx=fy=1600,
16x16 tiles) seen from 8 seeded poses on a radius-6 orbit; one step = one
view's full training render: forward (projection, tile binning, sort,
compositing, with the L1 loss cotangent written by the compositing pass),
raster backward and projection backward to dense parameter gradients.
Inputs are resident in HBM before timing.

Prints one JSON line (contract: metric/value/unit/.../roofline/cpu_baseline).

    python bench.py [--gpus 1] [--steps 40] [--warmup 8] [--workload c3] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E
FP32_VALU_PEAK_TFLOPS = 157.3    # MI355X vector fp32 (packed) peak
VALU_ISSUE_PEAK_G = 256 * 4 * 2.4 / 4   # G wave64 VALU instructions/s without packed fp32 (614.4)
SIMD_CYCLES_G = 256 * 4 * 2.4           # G SIMD cycles/s across the chip
# Cycles per wave64 instruction by counter class, relative to FP32 add at 4,
# as a one-off per-class issue probe measured them on gfx950: FP32 add/mul/fma 4,
# int32 2, conversions 4, transcendentals 8.  The remainder (moves 2;
# max/min, compares, selects 4) is bracketed by its two rates.
VALU_CLASS_CYCLES = {"SQ_INSTS_VALU_ADD_F32": 4, "SQ_INSTS_VALU_MUL_F32": 4, "SQ_INSTS_VALU_FMA_F32": 4,
                     "SQ_INSTS_VALU_TRANS_F32": 8, "SQ_INSTS_VALU_INT32": 2, "SQ_INSTS_VALU_CVT": 4,
                     "SQ_INSTS_VALU_INT64": 4}

METRIC = "fwd+bwd raster ms/view, 1M Gaussians SH3 1080p; achieved HBM GB/s vs peak"
EVENT_EVERY = 4      # timed steps per dispatch-time sample of the dominant kernel

WORKLOAD_DESC = {
    "c1": "10k Gaussians SH0, 256x256, fx=fy=256",
    "c2": "200k Gaussians SH3, 1920x1080, fx=fy=1600",
    "c3": "1M Gaussians SH3, 1920x1080, fx=fy=1600, 8 orbit views (radius 6)",
    "c4": "3M Gaussians SH3 heavy-tailed scales, 2560x1440, fx=fy=2000",
    "c5": "2M Gaussians SH3, KB4 fisheye f=600, 1920x1920, mask r=940",
}


def algorithmic_bytes(stage: str, n: int, v: int, i: int, t: int, p: int, k: int, used: int | None = None,
                      graded: int | None = None) -> int:
    """Compulsory HBM bytes of one launch (4-byte words).  The raster kernels
    are charged for the intersections they consume, the shrunk tile ranges
    (`used`: every pair past a tile's last blended one is never needed), not
    for the whole list; the projection backward reads parameters and SH rows
    only of the splats with a nonzero raster-gradient row (`graded`; the
    others get zero rows, bwd/kernels/project_backwards.rs:311-382)."""
    u = i if used is None else used
    c = v if graded is None else graded
    if stage == "raster_bwd_ms":      # ranges, ids + 36 B rows per used intersection, RGBA + cotangent, 40 B/visible grads
        return 8 * t + 40 * u + 32 * p + 40 * v
    if stage == "raster_fwd_ms":      # ranges in/out, ids + rows, RGBA out, visible marks
        return 16 * t + 40 * u + 16 * p + 4 * n
    if stage == "project_ms":         # 44 B params for all, SH for visible, 16 B out + 36 B row per visible
        return 44 * n + 16 * n + v * (12 * k + 36)
    if stage == "project_bwd_ms":     # 40 B raster grads, params + SH of graded rows, dense grads out
        return 40 * n + c * (44 + 12 * k) + n * (48 + 12 * k)
    if stage == "sort_ms":            # one read + one write of the 8 B (key, id) pairs: depth sort + tile sort
        return 16 * v + 16 * i
    if stage == "emit_ms":            # compaction (8N in, 8V out), slot scan (12V), emission (4N + 36V in, 8I out)
        return 12 * n + 56 * v + 8 * i
    return 0


def measure_next_rows(va, wl, cam, t, s, o, gt, dev, reps: int = 10) -> dict:
    """Kernel times (HIP events on the library's stream, outside the timed
    region) of the rows after the render: the L1 + SSIM loss (training
    forward with SSIM coefficients, and its backward) on the view's image, and
    the fused projection backward + packed-moment Adam on its raster
    gradients.  Algorithmic bytes: loss forward 20 B/px in + 36 B/px of
    coefficients out; backward 56 B/px in + 16 B/px out; update per splat
    40 + 4 + 4 + 40 + 40 + 4 B in and 40 + 4 + 40 + 4 + 24 + 8 B out, plus the
    192 B SH row of each splat with gradients; the camera gradient as noted
    where it is timed."""
    import torch

    def timed(fn):
        fn()
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        return sorted(ts)[len(ts) // 2]

    out = va.render(cam, wl.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
    h, w = out.out_img.shape[:2]
    gt_rgba = torch.cat([gt, torch.ones((h, w, 1), device=dev)], dim=-1)
    gtp = va.pack_rgba8(gt_rgba.cpu()).to(dev)
    cfg = va.ImageLossConfig.l1_dssim(0.2)
    box = {}

    def fwd():
        box["p"], box["c"], box["t"] = va.image_loss_forward_train(out.out_img, gtp, cfg)
    f_ms = timed(fwd)
    one = torch.ones(1, device=dev)
    b_ms = timed(lambda: va.image_loss_backward(out.out_img, gtp, one, cfg, box["c"]))
    px = h * w
    v = va.l1_cotangent(out.out_img, gt, (0.0, 0.0), 0.0)
    g = va.render_backward(out, t, s, o, v, fused=True)
    n = t.shape[0]
    tw, ow = t.clone(), o.clone()
    w_t = torch.zeros((n, 10), dtype=torch.int32, device=dev)
    w_o = torch.zeros(n, dtype=torch.int32, device=dev)
    lr = torch.full((10,), 1e-4, device=dev)
    adam = va.FusedAdam.at_step(1, lr_opac=0.05)
    res = va.project_update(out, tw, s, ow, g.v_combined, w_t, lr, w_o, adam)
    u_ms = timed(lambda: va.project_update(out, tw, s, ow, g.v_combined, w_t, lr, w_o, adam))
    with_grad = int((g.v_combined.abs().sum(dim=1) > 0).sum().item())
    u_bytes = n * (132 + 120) + with_grad * 192
    # camera gradient: 32 B of raster gradients per splat, the 44 B parameters
    # and the SH row of each splat with position, conic or colour gradients
    p_ms = timed(lambda: va.pose_backward(out, t, s, o, g.v_combined))
    pose_rows = int((g.v_combined[:, :8].abs().sum(dim=1) > 0).sum().item())
    p_bytes = 32 * n + pose_rows * (44 + 12 * s.shape[1])
    # SH step on f16 coefficients: every block holding a value of a splat with
    # a gradient row reads and writes 128 x (2 B coefficient + 1 B code) and
    # its scale; per splat 4 B row + 4 B grad_sq + 4 + 4 B variance, per
    # visible splat its 24 B colour row.
    sh16 = s.half()
    k3 = sh16.shape[1] * 3
    st = va.ShStepState.fresh(n, wl.scene.sh_degree, dev)
    rows = res.compact_from_global
    sh_ms = timed(lambda: va.sh_step(sh16, res.color_dir, rows, res.coeffs_grad_sq, st, 1e-3))
    vis_vals = (rows != 0).repeat_interleave(k3)
    pad = (-vis_vals.numel()) % 128
    touched = int(torch.nn.functional.pad(vis_vals, (0, pad)).view(-1, 128).any(dim=1).sum().item())
    nvis = int((rows != 0).sum().item())
    sh_bytes = touched * (128 * 6 + 8) + n * 16 + nvis * 24
    out.state.free()
    # neural appearance (render_neural): the same view with random [N,4,3]
    # rows and an [816] decoder at direction band 3; one training view
    # (render, L1 cotangent, dense backward incl. the decoder gradient), with
    # the projection and projection + neural backward stages from HIP events.
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    nrows = torch.rand((n, 4, 3), generator=gen, device=dev) * 3.0 - 1.5
    dec = torch.randn(816, generator=gen, device=dev) * 0.35

    def neural_step():
        o2 = va.render(cam, wl.img_size, t, nrows, o, pass_=va.RasterPass.BACKWARD, decoder=dec, neural_degree=3,
                       l1_target=gtp)
        va.render_backward(o2, t, nrows, o, o2.v_l1, decoder=dec)
        o2.state.free()
    n_ms = timed(neural_step)
    ctx = va.Context.get(dev)
    ctx.enable_timing(True, stages=["project", "project_bwd"])
    ctx.stage_times()
    for _ in range(reps):
        neural_step()
    st_ms = ctx.stage_times()
    ctx.enable_timing(False)

    # surfels (SplatRenderMode::Surfel): the same view and splats as 2DGS
    # disks, 12-channel training render, L1 cotangent on the colour, the
    # 17-component raster backward and the surfel projection VJP.
    def surfel_step():
        o3 = va.render(cam, wl.img_size, t, s, o, pass_=va.RasterPass.BACKWARD, render_mode=va.SplatRenderMode.SURFEL)
        v3 = va.l1_cotangent(o3.out_img, gt, (0.0, 0.0), 0.0)
        va.render_backward(o3, t, s, o, v3)
        o3.state.free()
    sf_ms = timed(surfel_step)
    ctx.enable_timing(True, stages=["raster_fwd", "raster_bwd", "project_bwd"])
    ctx.stage_times()
    for _ in range(reps):
        surfel_step()
    sf_st = ctx.stage_times()
    ctx.enable_timing(False)
    return {"neural_appearance": {"view_ms": round(n_ms, 4), "band": 3,
                                  "project_ms": round(st_ms["project_ms"] / reps, 4),
                                  "project_bwd_with_neural_ms": round(st_ms["project_bwd_ms"] / reps, 4)},
            "surfel": {"view_ms": round(sf_ms, 4), "channels": 12,
                       "raster_fwd_ms": round(sf_st["raster_fwd_ms"] / reps, 4),
                       "raster_bwd_ms": round(sf_st["raster_bwd_ms"] / reps, 4),
                       "project_bwd_ms": round(sf_st["project_bwd_ms"] / reps, 4)},
            "image_loss_l1_ssim": {"img": [w, h], "fwd_ms": round(f_ms, 4), "bwd_ms": round(b_ms, 4),
                                   "fwd_alg_GBs": round(56 * px / (f_ms * 1e-3) / 1e9, 1),
                                   "bwd_alg_GBs": round(72 * px / (b_ms * 1e-3) / 1e9, 1)},
            "project_update": {"ms": round(u_ms, 4), "splats": n, "with_gradient": with_grad,
                               "alg_GBs": round(u_bytes / (u_ms * 1e-3) / 1e9, 1)},
            "sh_step": {"ms": round(sh_ms, 4), "blocks_stepped": touched, "coeff_dtype": "f16",
                        "alg_GBs": round(sh_bytes / (sh_ms * 1e-3) / 1e9, 1)},
            "pose_backward": {"ms": round(p_ms, 4), "rows": pose_rows,
                              "alg_GBs": round(p_bytes / (p_ms * 1e-3) / 1e9, 1)}}


def list_length_histogram(ranges) -> dict:
    """Per-tile list lengths from tile ranges [.., 2] (before the forward
    shrinks their ends) as a power-of-two histogram."""
    import numpy as np
    import torch
    r = ranges.to(torch.int64).reshape(-1, 2)
    lens = (r[:, 1] - r[:, 0]).clamp_min(0).cpu().numpy()
    top = max(int(lens.max()), 1)
    edges = [0, 1] + [1 << e for e in range(1, 32) if (1 << (e - 1)) <= top]
    counts, _ = np.histogram(lens, bins=edges + [edges[-1] * 2])
    return {"tiles": int(lens.size), "mean": round(float(lens.mean()), 1), "max": int(lens.max()),
            "p50": int(np.percentile(lens, 50)), "p99": int(np.percentile(lens, 99)),
            "hist_lower_edges": edges, "hist_counts": [int(c) for c in counts]}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="c3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-next-rows", action="store_true",
                    help="skip the timings of the rows after the render (loss, update, SH step, pose, neural, surfel)")
    ap.add_argument("--depth-cutoff", choices=("off", "on", "auto"), default="off",
                    help="depth cutoff of the tile lists (vs_ctx_set_depth_cutoff; off, as the reference lists "
                         "every pair, unless opted in)")
    ap.add_argument("--exact-counts", action="store_true",
                    help="time training renders that wait for their own counts (the default times lagged counts, "
                         "as the reference's training renders run)")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB (counter calibration for HBM traffic)")
    ap.add_argument("--summarize-stats", metavar="CSV", help="summarise a rocprofv3 kernel_stats.csv as markdown")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --pmc output directories (one counter group each) as markdown")
    ap.add_argument("--summary-out", metavar="MD", help="where --summarize-* writes its markdown")
    ap.add_argument("--traffic-out", metavar="JSON", help="where --summarize-pmc writes calibrated HBM bytes per kernel")
    ap.add_argument("--command", default="", help="the profiling command, recorded in the summary")
    args = ap.parse_args()
    if args.summarize_stats or args.summarize_pmc:
        return summarize(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the rasterizer runs one view per process on one device "
              f"(--gpus {args.gpus} is not supported in this build)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import vauss_amd as va
    from vauss_amd import scenes

    dev = torch.device("cuda:0")
    wl = scenes.workload(args.workload)
    print(f"[bench] workload {args.workload}: {WORKLOAD_DESC[args.workload]}", file=sys.stderr, flush=True)
    sc = wl.scene
    t = torch.from_numpy(sc.transforms).to(dev)
    s = torch.from_numpy(sc.sh_coeffs).to(dev)
    o = torch.from_numpy(sc.raw_opacities).to(dev)
    cams = [c.uniforms(wl.img_size) for c in wl.cameras]
    gt = torch.from_numpy(scenes.loss_target(wl.img_size)).to(dev)
    # the training target as the reference's loss reads it: u32 RGBA8 per pixel
    gt_packed = va.pack_rgba8(torch.cat([gt, torch.ones_like(gt[..., :1])], dim=-1).cpu()).to(dev)
    mc, mr = wl.mask_center, wl.mask_radius
    n = sc.num_splats
    k = (sc.sh_degree + 1) ** 2
    w, h = wl.img_size
    T = ((w + 15) // 16) * ((h + 15) // 16)
    P = w * h

    tile_lists = None

    def step(view: int, list_histogram: bool = False, used: bool = False):
        nonlocal tile_lists
        # the L1 cotangent is written by the raster pass with the image
        out = va.render(cams[view], wl.img_size, t, s, o, pass_=va.RasterPass.BACKWARD, l1_target=gt_packed,
                        l1_mask_center=mc, l1_mask_radius=mr)
        g = va.render_backward(out, t, s, o, out.v_l1)
        aux = (out.aux.num_visible, out.aux.num_intersections)
        if used:      # intersections the raster kernels consume: the shrunk tile ranges
            r = out.aux.tile_offsets.reshape(-1, 2).to(torch.int64) & 0xFFFFFFFF
            aux = aux + (int((r[:, 1] - r[:, 0]).clamp(min=0).sum().item()),
                         int((g.v_combined != 0).any(dim=1).sum().item()))
        if list_histogram:
            tile_lists = list_length_histogram(out.state.tile_ranges(dev))
        out.state.free()
        return g, aux

    ctx = va.Context.get(dev)
    ctx.set_depth_cutoff({"off": ctx.CUTOFF_OFF, "on": ctx.CUTOFF_ON, "auto": ctx.CUTOFF_AUTO}[args.depth_cutoff])
    lagged = not args.exact_counts
    ctx.set_lagged_counts(lagged)
    for i in range(args.warmup):
        step(i % len(cams))
    torch.cuda.synchronize()

    # Stage breakdown: one pass over the views with every stage bracketed by
    # HIP events (each bracket adds a few microseconds of stream time, so this
    # pass is not the timed one), on exact counts so each view's counts are its
    # own.  It runs once before the timed region (to pick the dominant stage)
    # and once after it, when clocks and caches are at their steady state as
    # in the timed steps: the second pass gives the per-launch times.
    nb = len(cams)

    def stage_pass(first: bool):
        ctx.set_lagged_counts(False)
        ctx.enable_timing(True)
        ctx.stage_times()                # drop anything recorded before
        counts = []
        for i in range(nb):
            _, aux = step(i % len(cams), list_histogram=first and i == 0, used=True)
            counts.append(aux)
        stages = ctx.stage_times()
        ctx.enable_timing(False)
        return counts, {name: ms / nb for name, ms in stages.items()}

    counts, per_launch = stage_pass(True)
    dom = max(("raster_bwd_ms", "raster_fwd_ms", "project_ms", "project_bwd_ms", "sort_ms"), key=lambda x: per_launch[x])

    # Timed region: K steps; only the dominant kernel's stage is bracketed by
    # events (its live launch time is the roofline's denominator).  With
    # lagged counts a render that overflowed its capacity would drop work, so
    # the overflow count is read before and after and must not move.
    def timed_steps(lagged_counts: bool):
        ctx.set_lagged_counts(lagged_counts)
        for i in range(len(cams)):          # settle the hints on this mode
            step(i % len(cams))
        before = ctx.settle_lagged_counts()[1]
        ctx.stage_times()                  # drop anything recorded before
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        timed = 0
        for i in range(args.steps):
            # the dominant kernel's launch is bracketed by HIP events on every
            # EVENT_EVERY-th step: each event pair holds the stream a few
            # microseconds, which would otherwise add to every step
            on = i % EVENT_EVERY == 0
            ctx.enable_timing(on, stages=[dom.replace("_ms", "")])
            timed += on
            step(i % len(cams))
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        launch_ms = ctx.stage_times()[dom] / max(timed, 1)
        ctx.enable_timing(False)
        overflows = ctx.settle_lagged_counts()[1] - before
        ctx.set_lagged_counts(False)
        if overflows:
            raise SystemExit(f"bench: {overflows} lagged renders overflowed their capacity in the timed region")
        return (t1 - t0) * 1000.0 / args.steps, launch_ms

    ms_per_step, dom_ms = timed_steps(lagged)
    other_ms = timed_steps(not lagged)[0]
    counts, per_launch = stage_pass(False)
    print(f"[bench] {args.steps} steps, {ms_per_step:.3f} ms/view ({'lagged' if lagged else 'exact'} counts; "
          f"{other_ms:.3f} with {'exact' if lagged else 'lagged'} counts)", file=sys.stderr, flush=True)

    V = float(np.mean([c[0] for c in counts]))
    I = float(np.mean([c[1] for c in counts]))
    U = float(np.mean([c[2] for c in counts]))      # intersections inside the shrunk ranges
    Cg = float(np.mean([c[3] for c in counts]))     # splats with a nonzero raster-gradient row
    kernels = {}
    for name, ms in per_launch.items():
        b = algorithmic_bytes(name, n, int(V), int(I), T, P, k, int(U), int(Cg))
        kernels[name.replace("_ms", "")] = {"ms": round(ms, 4),
                                             "alg_GBs": round(b / (ms * 1e-3) / 1e9, 1) if ms > 0 and b else None}
    # The roofline's denominator is the dominant kernel's dispatch time: the
    # stage pass brackets its dispatch alone with events (the raster backward
    # is launched with its own start and stop events), which agrees with
    # rocprofv3's per-dispatch average for the kernel.  The same kernel's
    # events inside the back-to-back timed region also carry dispatch-queue
    # time and are reported beside it.
    dom_bytes = algorithmic_bytes(dom, n, int(V), int(I), T, P, k, int(U), int(Cg))
    disp_ms = per_launch[dom]
    achieved = dom_bytes / (disp_ms * 1e-3) / 1e9
    traffic, traffic_note = measured_traffic(args.workload, dom.replace("_ms", ""))
    valu, valu_classes = measured_valu_insts(args.workload, dom.replace("_ms", "")) or (None, None)
    roofline = {"bound": "hbm", "kernel": dom.replace("_ms", ""), "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": traffic, "traffic_source": traffic_note, "alg_bytes_per_launch": dom_bytes,
                "intersections_used": round(U), "ms_per_launch": round(disp_ms, 4),
                "ms_per_launch_timed_region": round(dom_ms, 4)}
    # The raster kernels are bound by VALU instruction issue, not HBM: their
    # wave instructions per launch (counter summary) over the dispatch time,
    # against MI355X's FP32 issue rate (256 CUs x 4 SIMDs x 2.4 GHz / 4
    # cycles per wave64 instruction).  Integer, move and conversion
    # instructions issue in 2 cycles, so "frac" is not a bound by itself:
    # "utilization" weighs the counter classes by their measured cycles
    # (the unclassified remainder between 2 and 4) against the SIMD cycles.
    if valu:
        rate = valu / (disp_ms * 1e-3) / 1e9
        roofline["valu_issue"] = {"achieved": round(rate, 1), "peak": VALU_ISSUE_PEAK_G, "unit": "G wave-instr/s",
                                  "frac": round(rate / VALU_ISSUE_PEAK_G, 4), "insts_per_launch": int(valu),
                                  "utilization": issue_utilization(valu, valu_classes, disp_ms),
                                  "source": traffic_note}
    # forward and backward of one view from the stage pass's events
    fwd_ms = sum(per_launch[x] for x in ("project_ms", "emit_ms", "sort_ms", "ranges_ms", "raster_fwd_ms"))
    bwd_ms = per_launch["raster_bwd_ms"] + per_launch["project_bwd_ms"]

    if args.copy_calib:
        # kernels of known traffic for the memory counters: a device copy, and
        # the library's streaming read and write kernels (16- and 4-byte words)
        nbytes = args.copy_calib * (1 << 20)
        src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        for mode in (0, 1, 2, 3):
            for _ in range(3):
                va._lib.check(ctx.lib.vs_stream_probe(ctx.handle, dst.data_ptr(), nbytes, mode))
        torch.cuda.synchronize()
        print(f"[bench] counter calibration: {args.copy_calib} MiB per copy (read + write), streaming read and write "
              f"(16- and 4-byte words)", file=sys.stderr, flush=True)

    next_rows = None if args.no_next_rows else measure_next_rows(va, wl, cams[0], t, s, o, gt, dev)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(wl, cams)

    line = {
        "metric": METRIC,
        "value": round(ms_per_step, 4),
        "unit": "ms/view",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64 cloud, random-init parameters)",
        "config": {"workload": f"{args.workload}: {WORKLOAD_DESC[args.workload]}", "num_splats": n,
                   "sh_degree": sc.sh_degree, "img": [w, h], "tile": 16, "views": len(cams),
                   "mean_visible": round(V), "mean_intersections": round(I), "mean_graded_rows": round(Cg),
                   "counts": "lagged" if lagged else "exact", "depth_cutoff": args.depth_cutoff},
        ("ms_per_view_exact_counts" if lagged else "ms_per_view_lagged_counts"): round(other_ms, 4),
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "gaussians_per_s": round(n / (ms_per_step * 1e-3)),
        "stage_ms": {k2: v2["ms"] for k2, v2 in kernels.items()},
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "tile_lists": tile_lists,
        "next_rows": next_rows,
    }
    print(json.dumps(line))
    return 0


PROFILES = os.path.join(ROOT, "profiles")
def _kernel_sources():
    from vauss_amd.build import HEADERS, SOURCES
    return [os.path.join(ROOT, "vauss_amd", "csrc", f) for f in SOURCES + HEADERS if not f.endswith(".cpp")]


KERNEL_SOURCES = _kernel_sources()

# rocprofv3 kernel names -> bench stage names
STAGE_OF_KERNEL = [("raster_bwd_kernel", "raster_bwd"), ("raster_fwd_kernel", "raster_fwd"),
                   ("project_bwd_kernel", "project_bwd"), ("project_kernel", "project"), ("emit_kernel", "emit"),
                   ("finalize_counts", "project"), ("compact_kernel", "emit"), ("scan_", "emit"), ("sort_", "sort"),
                   ("tile_ranges", "ranges"),
                   ("l1_cotangent", "loss"), ("loss_", "image_loss"), ("project_update", "project_update"),
                   ("sh_step", "sh_step"), ("sh_variance", "sh_step"), ("b8_", "sh_step"),
                   ("pose_", "pose_backward"), ("neural_", "neural"),
                   ("fill", "fill"), ("copyBuffer", "copy"), ("stream_", "calib"), ("elementwise", "torch")]


def stage_of_kernel(k: str) -> str:
    """The bench stage of a (short) kernel name; the surfel and neural render
    modes' kernels (bench rows of their own) are kept apart from the gaussian
    SH stages they share names with."""
    if k.startswith("raster_bwd_surfel") or (k.startswith("raster_fwd_kernel") and k.endswith(", true>")):
        return "surfel"
    if k.startswith(("project_kernel<-1", "project_bwd_kernel<-1")):
        return "surfel"
    if k.startswith(("project_kernel<3, 16", "project_bwd_kernel<3, 16")):
        return "neural"
    return next((st for pat, st in STAGE_OF_KERNEL if pat in k), k)


# what the markdown summary lists (the traffic file keeps every kernel)
SUMMARY_COUNTERS = ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_VALU_TRANS_F32",
                    "SQ_LDS_BANK_CONFLICT", "SQ_THREAD_CYCLES_VALU", "SQ_ACTIVE_INST_VALU", "TCC_ATOMIC_sum",
                    "TCC_EA0_ATOMIC_sum", "TCC_HIT_sum", "TCC_MISS_sum", "FETCH_SIZE", "WRITE_SIZE",
                    "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_sum",
                    "TCC_EA0_RDREQ_DRAM_sum", "TCC_EA0_WRREQ_DRAM_sum",
                    "SQ_INSTS_VALU_ADD_F32", "SQ_INSTS_VALU_MUL_F32", "SQ_INSTS_VALU_FMA_F32", "SQ_INSTS_VALU_INT32",
                    "SQ_INSTS_VALU_CVT", "SQ_INSTS_VALU_INT64")
SUMMARY_KERNELS = ("raster_", "project_", "emit", "sort_", "loss_", "sh_step", "pose_", "neural_", "copyBuffer",
                   "stream_")


def source_digest() -> str:
    import hashlib
    h = hashlib.sha256()
    for f in KERNEL_SOURCES:
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary,
    when it was measured on the kernel sources in this tree."""
    path = os.path.join(PROFILES, f"hbm_traffic_{workload}.json")
    if not os.path.exists(path):
        return None, "no counter summary for this workload"
    with open(path) as fh:
        data = json.load(fh)
    if data.get("source_digest") != source_digest():
        return None, f"{os.path.relpath(path, ROOT)} was measured on other kernel sources"
    k = data["kernels"].get(kernel)
    if not k:
        return None, f"{kernel} missing from {os.path.relpath(path, ROOT)}"
    return int(k["fetch_bytes"] + k["write_bytes"]), os.path.relpath(path, ROOT)


def measured_valu_insts(workload: str, kernel: str):
    """Wave-level VALU instructions per launch of `kernel` (SQ_INSTS_VALU)
    from the committed counter summary, when measured on these sources."""
    path = os.path.join(PROFILES, f"hbm_traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        data = json.load(fh)
    if data.get("source_digest") != source_digest():
        return None
    k = data["kernels"].get(kernel, {})
    return k.get("valu_insts"), k.get("valu_classes")


def issue_utilization(insts: float, classes: dict, ms: float):
    """Fraction of the SIMDs' cycles the kernel's VALU instructions occupy,
    [low, high] with the unclassified remainder at 2 and 4 cycles."""
    if not classes or not insts:
        return None
    known = sum(classes.get(c, 0.0) * cyc for c, cyc in VALU_CLASS_CYCLES.items())
    rest = max(0.0, insts - sum(classes.get(c, 0.0) for c in VALU_CLASS_CYCLES))
    avail = SIMD_CYCLES_G * 1e9 * ms * 1e-3
    return [round((known + 2 * rest) / avail, 3), round((known + 4 * rest) / avail, 3)]


def _short_kernel(name: str) -> str:
    base = name.split("(")[0].replace("void ", "")
    return base.replace("vs::", "")


def summarize(args) -> int:
    import csv
    lines = []
    if args.summarize_stats:
        with open(args.summarize_stats) as fh:
            rows = list(csv.DictReader(fh))
        lines += ["| kernel | calls | avg us | min us | max us | % of GPU time |", "|---|---|---|---|---|---|"]
        for r in rows:
            lines.append(f"| `{_short_kernel(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                         f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.2f} |")
    traffic = None
    if args.summarize_pmc:
        per = {}          # kernel -> counter -> {dispatch: value}
        durs = {}         # kernel -> {dispatch: ns}
        for d in args.summarize_pmc:
            for f in os.listdir(d):
                if not f.endswith("counter_collection.csv"):
                    continue
                with open(os.path.join(d, f)) as fh:
                    for r in csv.DictReader(fh):
                        k = _short_kernel(r["Kernel_Name"])
                        # rows of one dispatch (one per counter instance) add up; the same
                        # counter collected in two runs averages over both
                        key = (d, r["Dispatch_Id"], r["Grid_Size"])
                        per.setdefault(k, {}).setdefault(r["Counter_Name"], {}).setdefault(key, 0.0)
                        per[k][r["Counter_Name"]][key] += float(r["Counter_Value"])
                        durs.setdefault(k, {})[key] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        dur = {k: sum(v.values()) / len(v) for k, v in durs.items()}

        def mean_of(cs, c):
            v = cs.get(c)
            return sum(v.values()) / len(v) if v else None

        def read_bytes(cs):
            """L2->memory read bytes per dispatch from the request-size counters
            (32, 64 and 128-byte requests), or None when a pass is missing."""
            r32, r64, r128 = (mean_of(cs, f"TCC_EA0_RDREQ_{w}B_sum") for w in (32, 64, 128))
            if r32 is None or r64 is None or r128 is None:
                return None
            return 32.0 * r32 + 64.0 * r64 + 128.0 * r128

        def write_bytes(cs):
            """Write bytes per dispatch: WRITE_SIZE, whose expression counts the
            32- and 64-byte write requests (atomics travel as 32-byte ones)."""
            w = mean_of(cs, "WRITE_SIZE")
            return None if w is None else w * 1024.0

        # Calibration: kernels whose traffic is known exactly (each byte of an
        # N-byte buffer read and/or written once).
        calib = args.copy_calib * (1 << 20) if args.copy_calib else 0
        known = {"__amd_rocclr_copyBuffer": ("device copy", calib, calib),
                 "stream_read_kernel<16>": ("streaming read, 16-byte words", calib, 0),
                 "stream_read_kernel<4>": ("streaming read, 4-byte words", calib, 0),
                 "stream_write_kernel<16>": ("streaming write, 16-byte words", 0, calib),
                 "stream_write_kernel<4>": ("streaming write, 4-byte words", 0, calib)}
        cal = {}
        if calib:
            lines += ["", f"Calibration ({args.copy_calib} MiB buffers): counter bytes per dispatch / known bytes", "",
                      "| kernel | known read | known write | requests read / known | FETCH_SIZE / known | "
                      "WRITE_SIZE / known |", "|---|---|---|---|---|---|"]
            for k, (desc, kr, kw) in known.items():
                cs = per.get(k)
                if not cs:
                    continue
                if k == "__amd_rocclr_copyBuffer":      # the largest of the run's copies is the calibration copy
                    cs = {c: {0: max(v.values())} for c, v in cs.items()}
                rb, wb = read_bytes(cs), write_bytes(cs)
                fs = mean_of(cs, "FETCH_SIZE")
                cal[k] = {"read": rb / kr if (rb is not None and kr) else None,
                          "fetch_size": fs * 1024.0 / kr if (fs is not None and kr) else None,
                          "write": wb / kw if (wb is not None and kw) else None}
                fmt = lambda x: "-" if x is None else f"{x:.3f}"
                lines.append(f"| `{k}` ({desc}) | {kr >> 20} MiB | {kw >> 20} MiB | {fmt(cal[k]['read'])} | "
                             f"{fmt(cal[k]['fetch_size'])} | {fmt(cal[k]['write'])} |")
        # Reads: the request-size counters, exact where the streaming reads
        # show it (ratio 1); FETCH_SIZE's expression, which counts a 128-byte
        # request as 64 bytes, is kept only as a fallback scaled by the copy.
        copy = per.get("__amd_rocclr_copyBuffer", {})
        f_scale = None
        if calib and mean_of(copy, "FETCH_SIZE"):
            f_scale = calib / (max(copy["FETCH_SIZE"].values()) * 1024.0)
        lines += ["", "| kernel | dispatches | counter | mean per dispatch | derived |", "|---|---|---|---|---|"]
        traffic = {"source_digest": source_digest(), "calibration_mib": args.copy_calib, "calibration": cal,
                   "read_method": "32 RDREQ_32B + 64 RDREQ_64B + 128 RDREQ_128B",
                   "write_method": "WRITE_SIZE (32- and 64-byte write requests)",
                   "fetch_size_scale": f_scale, "kernels": {}}
        def per_run(v):        # dispatches of one run (the same counter may come from two runs)
            runs = {key[0] for key in v}
            return max(sum(1 for key in v if key[0] == r) for r in runs) if v else 0
        # per render: the forward stages' kernels (sort passes, histograms,
        # compaction, scan ...) add up over the gaussian training renders of
        # the run (launches of the bwd-info gaussian raster forward); the two
        # backward kernels are taken per launch (some of the run's backwards
        # stop at the raster gradients)
        nrender = max([1] + [max(per_run(c) for c in v.values()) for k, v in per.items()
                             if k.startswith("raster_fwd_kernel<true, false, false, false>")])
        for k, cs in sorted(per.items()):
            n = max(per_run(v) for v in cs.values())
            mean = {c: sum(v.values()) / len(v) for c, v in cs.items()}
            dur_ns = dur.get(k)
            rb, wb = read_bytes(cs), write_bytes(cs)
            if rb is None and f_scale and "FETCH_SIZE" in mean:
                rb = mean["FETCH_SIZE"] * 1024.0 * f_scale
            for c in sorted(mean):
                if c not in SUMMARY_COUNTERS or not any(x in k for x in SUMMARY_KERNELS):
                    continue
                derived = ""
                if c == "SQ_INSTS_VALU" and dur_ns:
                    derived = f"{mean[c] / dur_ns:.0f} G wave-instr/s over {dur_ns / 1e3:.1f} us"
                elif c == "TCC_EA0_RDREQ_128B_sum" and rb is not None:
                    derived = f"{rb / 1e6:.1f} MB read (32/64/128-byte requests)"
                elif c == "WRITE_SIZE" and wb is not None:
                    derived = f"{wb / 1e6:.1f} MB written"
                lines.append(f"| `{k}` | {n} | {c} | {mean[c]:.5g} | {derived} |")
            if rb is not None and wb is not None:
                stage = stage_of_kernel(k)
                if stage in ("copy", "torch", "fill", "calib"):
                    continue
                e = traffic["kernels"].setdefault(stage, {"fetch_bytes": 0.0, "write_bytes": 0.0, "valu_insts": 0.0,
                                                          "valu_classes": {}, "kernels": []})
                # per render: a kernel launched several times a render (sort passes) adds up
                reps = 1.0 if stage in ("raster_bwd", "project_bwd") else n / nrender
                e["fetch_bytes"] += rb * reps
                e["write_bytes"] += wb * reps
                e["valu_insts"] += mean.get("SQ_INSTS_VALU", 0.0) * reps
                for c in VALU_CLASS_CYCLES:
                    if c in mean:
                        e["valu_classes"][c] = e["valu_classes"].get(c, 0.0) + mean[c] * reps
                e["kernels"].append(k)
    text = "\n".join(lines) + "\n"
    if args.command:
        text = f"Command:\n\n```\n{args.command}\n```\n\n" + text
    if args.summary_out:
        with open(args.summary_out, "w") as fh:
            fh.write(text)
    else:
        print(text)
    if traffic is not None and args.traffic_out:
        with open(args.traffic_out, "w") as fh:
            json.dump(traffic, fh, indent=1)
    return 0


def cpu_baseline(wl, cams, min_seconds: float = 10.0):
    """The oracle (CPU restatement of the reference path) on all host threads:
    full training renders (forward + L1 cotangent + backward) of consecutive
    views until at least `min_seconds` of CPU work or every view is done."""
    import numpy as np
    from oracle import pyoracle as po
    from vauss_amd import scenes
    sc = wl.scene
    threads = po.max_threads()
    gt = scenes.loss_target(wl.img_size)
    fwd_ms, bwd_ms = [], []
    t_start = time.perf_counter()
    for cam in cams:
        t0 = time.perf_counter()
        f = po.render_forward(cam, wl.img_size, sc.transforms, sc.sh_coeffs, sc.raw_opacities, flags=po.FLAG_BWD_INFO,
                              threads=threads)
        img = f.get(po.F_OUT_IMG)
        v = np.zeros_like(img)
        hh, ww = img.shape[:2]
        v[..., :3] = np.sign(img[..., :3] - gt) / np.float32(3 * hh * ww)
        t1 = time.perf_counter()
        f.backward(v, threads=threads)
        t2 = time.perf_counter()
        fwd_ms.append(1000 * (t1 - t0))
        bwd_ms.append(1000 * (t2 - t1))
        if t2 - t_start >= min_seconds:
            break
    k = len(fwd_ms)
    ms = (sum(fwd_ms) + sum(bwd_ms)) / k
    return {"value": round(ms, 1), "unit": "ms/view", "cores": threads, "kind": "port",
            "sample": f"{k} full view(s) of {wl.name} (views 0..{k - 1}), mean fwd {sum(fwd_ms) / k:.0f} ms + "
                      f"bwd {sum(bwd_ms) / k:.0f} ms per view, OpenMP over {threads} threads, "
                      f"{(time.perf_counter() - t_start):.1f} s in total"}


if __name__ == "__main__":
    sys.exit(main())
