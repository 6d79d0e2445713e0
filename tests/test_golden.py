"""Golden render fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

The CPU tests check that the oracle still reproduces every fixture bit for
bit; the GPU tests check the HIP path against the fixtures with the parity
bars: integer outputs bit for bit, RGBA within 1e-4 absolute (the fixtures
composite with the oracle's exp2n, the kernels with the GPU's exp2
instruction, both within 2.1 ulp of 2^x) and bit for bit against the oracle
re-run with the GPU's exp2 values, gradients within 1e-3 relative / 1e-5
absolute of each entry, or 1e-3 of the group's largest gradient."""
import ctypes as C
import glob
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(glob.glob(os.path.join(HERE, "*.npz")))
IDS = [os.path.basename(f)[:-4] for f in FIXTURES]


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _camera_bytes(fx):
    """The fixture's vs_camera bytes.  Fixtures written before the struct grew
    its distortion block (dist[8], appended) hold the first 120 bytes; the
    block is zero for their pinhole and KB4 cameras."""
    from vauss_amd import _lib
    raw = fx["camera"].tobytes()
    full = C.sizeof(_lib.VsCamera)
    assert len(raw) in (120, full)
    return raw + bytes(full - len(raw))


def _camera(fx):
    from vauss_amd import _lib
    return _lib.VsCamera.from_buffer_copy(_camera_bytes(fx))


def test_fixtures_present():
    assert len(FIXTURES) >= 4


@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_oracle_reproduces_fixture(path):
    from oracle import pyoracle as po
    fx = _load(path)
    cam = po.OrCamera.from_buffer_copy(_camera_bytes(fx))
    img = tuple(int(v) for v in fx["img_size"])
    f = po.render_forward(cam, img, fx["transforms"], fx["sh_coeffs"], fx["raw_opacities"],
                          background=tuple(fx["background"]), flags=int(fx["flags"]))
    for key, field in [("intersect_counts", po.F_INTERSECT_COUNTS), ("isect_tile", po.F_ISECT_TILE),
                       ("isect_gid", po.F_ISECT_GID), ("tile_offsets", po.F_TILE_OFFSETS),
                       ("visible", po.F_VISIBLE)]:
        np.testing.assert_array_equal(f.get(field), fx[key], err_msg=key)
    np.testing.assert_array_equal(f.get(po.F_OUT_IMG).view(np.uint32), fx["out_img"].view(np.uint32))
    g = f.backward(fx["v_out"])
    for key, name in [("v_combined", "v_combined"), ("v_transforms", "v_transforms"), ("v_sh", "v_sh"),
                      ("v_raw_opac", "v_raw_opac"), ("v_refine", "v_refine")]:
        np.testing.assert_array_equal(g[name].view(np.uint32), fx[key].view(np.uint32), err_msg=key)


def _check(got, want, name, rtol=1e-3, atol=1e-5):
    """The gradient bar: every entry within 1e-3 relative or 1e-5 absolute."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), f"{name}: {bad.sum()} entries exceed {rtol:g} rel / {atol:g} abs (max err {err.max():.3e})"


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_gpu_matches_fixture(path):
    import torch
    import vauss_amd as va
    from tests._util import gpu_state_arrays
    fx = _load(path)
    img = tuple(int(v) for v in fx["img_size"])
    print(f"[case] golden {os.path.basename(path)} img={img} n={len(fx['transforms'])}", flush=True)
    smooth = bool(int(fx["flags"]) & 4)
    pass_ = va.RasterPass.BACKWARD_SMOOTH_CUTOFF if smooth else va.RasterPass.BACKWARD
    t = torch.from_numpy(fx["transforms"]).cuda()
    s = torch.from_numpy(fx["sh_coeffs"]).cuda()
    o = torch.from_numpy(fx["raw_opacities"]).cuda()
    out = va.render(_camera(fx), img, t, s, o, background=tuple(float(v) for v in fx["background"]), pass_=pass_)
    gpu = gpu_state_arrays(out)
    np.testing.assert_array_equal(gpu["counts"], fx["intersect_counts"])
    np.testing.assert_array_equal(gpu["tile"], fx["isect_tile"])
    np.testing.assert_array_equal(gpu["gid"], fx["isect_gid"])
    np.testing.assert_array_equal(gpu["ranges"], fx["tile_offsets"])
    got_img = out.out_img.cpu().numpy()
    assert float(np.abs(got_img - fx["out_img"]).max()) <= 1e-4
    from oracle import pyoracle as po
    f = po.render_forward(po.OrCamera.from_buffer_copy(_camera_bytes(fx)), img, fx["transforms"], fx["sh_coeffs"],
                          fx["raw_opacities"], background=tuple(fx["background"]), flags=int(fx["flags"]))
    np.testing.assert_array_equal(got_img.view(np.uint32), f.get(po.F_OUT_IMG).view(np.uint32))
    np.testing.assert_array_equal(out.aux.visible.cpu().numpy(), fx["visible"])
    g = va.render_backward(out, t, s, o, torch.from_numpy(fx["v_out"]).cuda())
    vc = g.v_combined.cpu().numpy()
    for name, sl in [("v_xy", slice(0, 2)), ("v_conic", slice(2, 5)), ("v_rgb", slice(5, 8)),
                     ("v_opacity", slice(8, 9)), ("v_refine", slice(9, 10))]:
        _check(vc[:, sl], fx["v_combined"][:, sl], name)
    vt = g.v_transforms.cpu().numpy()
    for name, sl in [("v_means", slice(0, 3)), ("v_quats", slice(3, 7)), ("v_log_scales", slice(7, 10))]:
        _check(vt[:, sl], fx["v_transforms"][:, sl], name)
    _check(g.v_coeffs.cpu().numpy().reshape(len(vt), -1), fx["v_sh"].reshape(len(vt), -1), "v_sh")
    _check(g.v_raw_opac.cpu().numpy(), fx["v_raw_opac"], "v_raw_opacity")
    _check(g.v_refine_weight.cpu().numpy(), fx["v_refine"], "v_refine_weight")
