"""Writes the golden render fixtures under tests/golden/ from the oracle.

    python tests/golden/make_golden.py

Each fixture is an .npz of one small render: the inputs (splat parameters,
the raw vs_camera struct, image size, background, the loss cotangent) and the
oracle's outputs (per-splat tile counts, the sorted intersection list, tile
ranges, RGBA, visibility and the dense gradients).  The reference ships no
numeric render vectors, so these pin the oracle against regressions and give
the GPU tests fixed expectations that need no oracle at run time.
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import pyoracle as po  # noqa: E402
from vauss_amd import camera as vcam  # noqa: E402
from vauss_amd import scenes  # noqa: E402


def cases():
    """(name, scene, img, camera, background, flags)."""
    c1 = scenes.scene_c1(400)
    yield ("c1_sh0_pinhole", c1, (64, 64), vcam.Camera.from_focal(64.0, 64.0, (64, 64)), (0.0, 0.0, 0.0),
           po.FLAG_BWD_INFO)
    rng = np.random.default_rng(0x601D)
    base = scenes.rng_scene(400, 1.2, (-2.6, -1.2), (-1.0, 2.5), 0x601D)
    sh = np.concatenate([base.sh_coeffs, (rng.standard_normal((400, 15, 3)) * 0.15).astype(np.float32)], axis=1)
    sh3 = scenes.Scene(base.transforms, sh, base.raw_opacities)
    yield ("sh3_pinhole_bg", sh3, (64, 48), scenes.test_camera((64, 48), fov=0.6, position=(0.0, 0.0, -3.0)),
           (0.25, 0.5, 0.75), po.FLAG_BWD_INFO)
    kb4 = vcam.KannalaBrandt4(0.05, -0.03, 0.01, -0.005)
    yield ("sh3_kb4_wide", sh3, (64, 64), scenes.test_camera((64, 64), fov=1.7, position=(0.0, 0.0, -2.5), model=kb4),
           (0.0, 0.0, 0.0), po.FLAG_BWD_INFO)
    yield ("sh3_pinhole_smooth", sh3, (64, 48), scenes.test_camera((64, 48), fov=0.6, position=(0.0, 0.0, -3.0)),
           (0.0, 0.0, 0.0), po.FLAG_BWD_INFO | po.FLAG_SMOOTH_CUTOFF)


def make(name, scene, img, camera, background, flags):
    cam = camera.uniforms(img)
    f = po.render_forward(cam, img, scene.transforms, scene.sh_coeffs, scene.raw_opacities, background=background,
                          flags=flags)
    out = f.get(po.F_OUT_IMG)
    rng = np.random.default_rng(7)
    v_out = (rng.standard_normal(out.shape) / (img[0] * img[1])).astype(np.float32)
    g = f.backward(v_out)
    np.savez_compressed(
        os.path.join(HERE, name + ".npz"),
        transforms=scene.transforms, sh_coeffs=scene.sh_coeffs, raw_opacities=scene.raw_opacities,
        camera=np.frombuffer(bytes(cam), dtype=np.uint8), img_size=np.array(img, np.uint32),
        background=np.array(background, np.float32), flags=np.array(flags, np.uint32), v_out=v_out,
        intersect_counts=f.get(po.F_INTERSECT_COUNTS), isect_tile=f.get(po.F_ISECT_TILE),
        isect_gid=f.get(po.F_ISECT_GID), tile_offsets=f.get(po.F_TILE_OFFSETS), out_img=out,
        visible=f.get(po.F_VISIBLE), num_visible=np.array(f.info.num_visible, np.uint32),
        v_combined=g["v_combined"], v_transforms=g["v_transforms"], v_sh=g["v_sh"], v_raw_opac=g["v_raw_opac"],
        v_refine=g["v_refine"])
    print(f"{name}: {f.info.num_visible} visible, {f.info.num_intersections} intersections")


if __name__ == "__main__":
    for c in cases():
        make(*c)
