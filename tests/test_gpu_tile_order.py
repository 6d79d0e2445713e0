"""Order of the tile lists against the oracle, bit for bit, where ties and
long lists make it delicate:

* a stack of splats over the image centre whose four central tiles each list
  12,000 splats (far past any in-LDS sort), at three exact depths, so most
  pairs tie on depth and the splat id breaks the tie (render.rs:689-694 sorts
  64-bit (tile, depth bits) keys stably over the emission order);
* a spread of the same kind with short lists and ties.
"""
import numpy as np
import pytest

import vauss_amd as va
from oracle import pyoracle as po
from tests._util import gpu_state_arrays, to_gpu
from vauss_amd import scenes
from vauss_amd.camera import Camera

pytestmark = pytest.mark.gpu


def _tie_scene(n: int, half_width: float, seed: int) -> scenes.Scene:
    rng = np.random.default_rng(seed)
    means = np.stack([rng.uniform(-half_width, half_width, n), rng.uniform(-half_width, half_width, n),
                      rng.choice(np.array([3.0, 3.5, 4.0]), n)], axis=1)
    log_scales = rng.normal(-2.6, 0.2, (n, 3))
    q = rng.normal(size=(n, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    sh = rng.uniform(0.0, 1.0, (n, 1, 3)).astype(np.float32)
    raw = rng.normal(-2.0, 0.5, n)
    return scenes.Scene(scenes._pack(means.astype(np.float32), q.astype(np.float32), log_scales.astype(np.float32)),
                        sh, raw.astype(np.float32))


def _check(scene, img_size, focal):
    cam = Camera.from_focal(focal, focal, img_size).uniforms(img_size)
    t, s, o = to_gpu(scene)
    print(f"[case] tie scene n={scene.num_splats} img={img_size}", flush=True)
    out = va.render(cam, img_size, t, s, o, pass_=va.RasterPass.BACKWARD)
    ref = po.render_forward(cam, img_size, scene.transforms, scene.sh_coeffs, scene.raw_opacities, flags=po.FLAG_BWD_INFO)
    gpu = gpu_state_arrays(out)
    assert out.aux.num_intersections == ref.info.num_intersections
    np.testing.assert_array_equal(gpu["tile"], ref.get(po.F_ISECT_TILE))
    np.testing.assert_array_equal(gpu["gid"], ref.get(po.F_ISECT_GID))
    np.testing.assert_array_equal(gpu["ranges"], ref.get(po.F_TILE_OFFSETS))
    img = out.out_img.cpu().numpy()
    assert np.array_equal(img.view(np.uint32), ref.get(po.F_OUT_IMG).view(np.uint32))
    np.testing.assert_array_equal(out.aux.tile_offsets.cpu().numpy().view(np.uint32), ref.get(po.F_TILE_OFFSETS_SHRUNK))
    return ref.get(po.F_TILE_OFFSETS).reshape(-1, 2)


def test_long_tile_lists_with_depth_ties():
    ranges = _check(_tie_scene(12_000, 0.02, 7), (256, 256), 256.0)
    longest = int((ranges[:, 1] - ranges[:, 0]).max())
    assert longest >= 12_000, longest


def test_short_tile_lists_with_depth_ties():
    ranges = _check(_tie_scene(6_000, 1.0, 11), (256, 256), 256.0)
    longest = int((ranges[:, 1] - ranges[:, 0]).max())
    assert 1 < longest <= 1024, longest
