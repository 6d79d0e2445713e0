"""Shared helpers for the tests: device readback and scene upload."""
from __future__ import annotations

import ctypes as C

import numpy as np

from vauss_amd._lib import PROJ_ROW_FLOATS

_HIP = None


def _hip():
    global _HIP
    if _HIP is None:
        import torch  # noqa: F401  (the HIP runtime torch loaded)
        _HIP = C.CDLL("libamdhip64.so.7")
        _HIP.hipMemcpy.restype = C.c_int
        _HIP.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    return _HIP


def dev_to_numpy(ptr, shape, dtype) -> np.ndarray:
    """Copy `shape` elements of `dtype` from a device pointer the library owns."""
    import torch
    torch.cuda.synchronize()
    out = np.empty(shape, dtype)
    if out.size:
        rc = _hip().hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), out.nbytes, 2)
        assert rc == 0, f"hipMemcpy failed ({rc})"
    return out


# The compositing kernels' G = 2^x is the GPU's exp2 instruction; the oracle
# composites with its values for every f32 x from -0 (bit pattern 0x80000000)
# down to -128 (0xC3000000).
EXP2_FIRST = 0x80000000
EXP2_COUNT = 0xC3000000 - 0x80000000 + 1
_EXP2_TABLE = None


def device_comp_exp2_table() -> np.ndarray:
    """The device's compositing 2^x over EXP2_FIRST .. + EXP2_COUNT (4.5 GB, built once)."""
    global _EXP2_TABLE
    if _EXP2_TABLE is None:
        import torch
        import vauss_amd as va
        print(f"[case] compositing exp2 table, {EXP2_COUNT} inputs", flush=True)
        d = va.compositing_exp2(EXP2_FIRST, EXP2_COUNT)
        _EXP2_TABLE = d.cpu().numpy()
        del d
        torch.cuda.empty_cache()
    return _EXP2_TABLE


def use_device_comp_exp2() -> None:
    """Makes the oracle composite with the device's 2^x (a no-op once installed)."""
    from oracle import pyoracle as po
    tab = device_comp_exp2_table()
    if po._COMP_EXP2 is not tab:
        po.set_comp_exp2_table(tab, EXP2_FIRST)


def use_default_comp_exp2() -> None:
    """Restores the oracle's own exp2n (CPU tests and golden vectors)."""
    import sys
    po = sys.modules.get("oracle.pyoracle")
    if po is not None and po._COMP_EXP2 is not None:
        po.set_comp_exp2_table(None)


def to_gpu(scene):
    import torch
    return (torch.from_numpy(scene.transforms).cuda(), torch.from_numpy(scene.sh_coeffs).cuda(),
            torch.from_numpy(scene.raw_opacities).cuda())


def l1_cotangent_np(img: np.ndarray, gt: np.ndarray, mask=None) -> np.ndarray:
    """sign(pred - gt) / (3 * count) on rgb, 0 on the other channels (closed form)."""
    v = np.zeros_like(img, dtype=np.float32)
    h, w = img.shape[:2]
    count = h * w if mask is None else int(mask.sum())
    d = img[..., :3] - gt
    s = np.sign(d).astype(np.float32) * np.float32(1.0 / (3.0 * count))
    if mask is not None:
        s = np.where(mask[..., None] > 0, s, np.float32(0.0))     # masked pixels are +0
    v[..., :3] = s
    return v


def circle_mask(img_size, center, radius) -> np.ndarray:
    w, h = img_size
    yy, xx = np.mgrid[0:h, 0:w]
    dx = xx.astype(np.float32) + np.float32(0.5) - np.float32(center[0])
    dy = yy.astype(np.float32) + np.float32(0.5) - np.float32(center[1])
    return (dx * dx + dy * dy <= np.float32(radius) * np.float32(radius)).astype(np.float32)


def gpu_state_arrays(out):
    """Intermediate buffers of a GPU forward as numpy arrays keyed like the oracle's."""
    v = out.state.view()
    n, i = v.num_splats, v.listed_intersections
    rows = dev_to_numpy(v.proj_xy_conic, (n, PROJ_ROW_FLOATS), np.float32)
    return {
        "view": v,
        "tile": dev_to_numpy(v.isect_tiles, (i,), np.uint32),
        "depth_bits": dev_to_numpy(v.depth_bits, (n,), np.uint32),
        "gid": dev_to_numpy(v.isect_gids, (i,), np.uint32),
        "counts": dev_to_numpy(v.intersect_counts, (n,), np.uint32),
        "listed_counts": dev_to_numpy(v.listed_counts, (n,), np.uint32),
        # the projected rows are 16 floats apart; the three views start inside row 0
        "proj_a": rows[:, 0:4].copy(),
        "proj_b": rows[:, 4:8].copy(),
        "proj_c": rows[:, 8].copy(),
        "proj_power": rows[:, 9].copy(),
        "proj_aux": dev_to_numpy(v.proj_aux, (n, 4), np.float32) if v.proj_aux else None,
        "ranges": dev_to_numpy(v.tile_ranges, (v.tile_bh, v.tile_bw, 2), np.uint32),
        "proj_surf": dev_to_numpy(v.proj_surf, (n, 16), np.float32) if v.proj_surf else None,
    }
