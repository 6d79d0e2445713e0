"""Benchmark: fwd+bwd rasterization ms per view on one MI355X.

Workload (default): 1,000,000 SH-degree-3 Gaussians at 1920x1080 (fx=fy=1600,
16x16 tiles) seen from 8 seeded poses on a radius-6 orbit; one step = one
view's full training render: forward (projection, tile binning, sort,
compositing), L1 loss cotangent, raster backward and projection backward to
dense parameter gradients.  Inputs are resident in HBM before timing.

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

METRIC = "fwd+bwd raster ms/view, 1M Gaussians SH3 1080p; achieved HBM GB/s vs peak"

WORKLOAD_DESC = {
    "c1": "10k Gaussians SH0, 256x256, fx=fy=256",
    "c2": "200k Gaussians SH3, 1920x1080, fx=fy=1600",
    "c3": "1M Gaussians SH3, 1920x1080, fx=fy=1600, 8 orbit views (radius 6)",
    "c4": "3M Gaussians SH3 heavy-tailed scales, 2560x1440, fx=fy=2000",
    "c5": "2M Gaussians SH3, KB4 fisheye f=600, 1920x1920, mask r=940",
}


def algorithmic_bytes(stage: str, n: int, v: int, i: int, t: int, p: int, k: int) -> int:
    """Compulsory HBM bytes of one launch (4-byte words)."""
    if stage == "raster_bwd_ms":      # ranges, ids + 36 B rows per intersection, RGBA + cotangent, 40 B/visible grads
        return 8 * t + 40 * i + 32 * p + 40 * v
    if stage == "raster_fwd_ms":      # ranges in/out, ids + rows, RGBA out, visible marks
        return 16 * t + 40 * i + 16 * p + 4 * n
    if stage == "project_ms":         # 44 B params for all, SH for visible, 16 B out + 36 B row per visible
        return 44 * n + 16 * n + v * (12 * k + 36)
    if stage == "project_bwd_ms":     # 40 B raster grads, params + SH for visible, dense grads out
        return 40 * n + v * (44 + 12 * k) + n * (48 + 12 * k)
    if stage == "sort_ms":            # one read + one write of the 12 B (key, id) pairs
        return 24 * i
    if stage == "emit_ms":
        return 4 * n + 40 * v + 12 * i
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="c3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB (counter calibration for HBM traffic)")
    args = ap.parse_args()
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
    mc, mr = wl.mask_center, wl.mask_radius
    n = sc.num_splats
    k = (sc.sh_degree + 1) ** 2
    w, h = wl.img_size
    T = ((w + 15) // 16) * ((h + 15) // 16)
    P = w * h

    def step(view: int):
        out = va.render(cams[view], wl.img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
        v = va.l1_cotangent(out.out_img, gt, mc, mr)
        g = va.render_backward(out, t, s, o, v)
        aux = (out.aux.num_visible, out.aux.num_intersections)
        out.state.free()
        return g, aux

    for i in range(args.warmup):
        step(i % len(cams))
    torch.cuda.synchronize()

    ctx = va.Context.get(dev)
    ctx.enable_timing(True)
    ctx.stage_times()                # drop anything recorded before the timed region
    counts = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        _, aux = step(i % len(cams))
        counts.append(aux)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    stages = ctx.stage_times()
    ctx.enable_timing(False)
    ms_per_step = (t1 - t0) * 1000.0 / args.steps
    print(f"[bench] {args.steps} steps, {ms_per_step:.3f} ms/view", file=sys.stderr, flush=True)

    V = float(np.mean([c[0] for c in counts]))
    I = float(np.mean([c[1] for c in counts]))
    per_launch = {name: ms / args.steps for name, ms in stages.items()}
    kernels = {}
    for name, ms in per_launch.items():
        b = algorithmic_bytes(name, n, int(V), int(I), T, P, k)
        kernels[name.replace("_ms", "")] = {"ms": round(ms, 4),
                                             "alg_GBs": round(b / (ms * 1e-3) / 1e9, 1) if ms > 0 and b else None}
    dom = max(("raster_bwd_ms", "raster_fwd_ms", "project_ms", "project_bwd_ms", "sort_ms"), key=lambda x: per_launch[x])
    dom_bytes = algorithmic_bytes(dom, n, int(V), int(I), T, P, k)
    dom_ms = per_launch[dom]
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "kernel": dom.replace("_ms", ""), "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": None, "alg_bytes_per_launch": dom_bytes, "ms_per_launch": round(dom_ms, 4)}

    if args.copy_calib:
        src = torch.empty(args.copy_calib * (1 << 20) // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] copy calibration: {args.copy_calib} MiB read + {args.copy_calib} MiB written per copy",
              file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(wl, cams[0])

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
                   "mean_visible": round(V), "mean_intersections": round(I)},
        "gaussians_per_s": round(n / (ms_per_step * 1e-3)),
        "stage_ms": {k2: v2["ms"] for k2, v2 in kernels.items()},
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


def cpu_baseline(wl, cam):
    """The oracle (CPU restatement of the reference path) on one view, all host threads."""
    import numpy as np
    from oracle import pyoracle as po
    from vauss_amd import scenes
    sc = wl.scene
    threads = po.max_threads()
    t0 = time.perf_counter()
    f = po.render_forward(cam, wl.img_size, sc.transforms, sc.sh_coeffs, sc.raw_opacities, flags=po.FLAG_BWD_INFO,
                          threads=threads)
    img = f.get(po.F_OUT_IMG)
    v = np.zeros_like(img)
    hh, ww = img.shape[:2]
    v[..., :3] = np.sign(img[..., :3] - scenes.loss_target(wl.img_size)) / np.float32(3 * hh * ww)
    t1 = time.perf_counter()
    f.backward(v, threads=threads)
    t2 = time.perf_counter()
    ms = (t2 - t0) * 1000.0
    return {"value": round(ms, 1), "unit": "ms/view", "cores": threads, "kind": "port",
            "sample": f"one full view (view 0) of {wl.name}: fwd {1000 * (t1 - t0):.0f} ms + bwd {1000 * (t2 - t1):.0f} ms, "
                      f"OpenMP over {threads} threads",
            "evaluations": int(f.info.num_evaluations)}


if __name__ == "__main__":
    sys.exit(main())
