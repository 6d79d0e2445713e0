"""ctypes binding of include/vsplat.h.

The library is the product path; there is no fallback.  `load()` raises if
libvsplat.so is missing.  torch must be imported before the library is
loaded so both share torch's HIP runtime (same soname).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime torch was built with first)

LIB_PATH = Path(__file__).resolve().parent / "libvsplat.so"

VS_OK, VS_ERR_INVALID, VS_ERR_HIP, VS_ERR_OOM, VS_ERR_UNSUPPORTED, VS_ERR_CAPACITY, VS_ERR_NONFINITE = range(7)
VS_SH_F32, VS_SH_F16 = 0, 1
STATUS_NAMES = ["VS_OK", "VS_ERR_INVALID", "VS_ERR_HIP", "VS_ERR_OOM", "VS_ERR_UNSUPPORTED",
                "VS_ERR_CAPACITY", "VS_ERR_NONFINITE"]

CAMERA_PINHOLE, CAMERA_KB4, CAMERA_RT8, CAMERA_TPF = 0, 1, 2, 3
(PASS_FORWARD, PASS_BACKWARD, PASS_FLOAT, PASS_BACKWARD_SMOOTH_CUTOFF, PASS_GEOMETRY, PASS_BACKWARD_DENSE,
 PASS_EXPOSURE, PASS_BACKWARD_FUSED_UPDATE, PASS_GEOMETRY_TRAIN_DEPTH) = range(9)


def pass_with_slot(pass_: int, slot: int) -> int:
    """VS_PASS_SLOT: the count slot in bits 8..15 of a vs_pass value."""
    return int(pass_) | ((int(slot) & 0xFF) << 8)
MODE_DEFAULT, MODE_MIP, MODE_SURFEL = range(3)
# stage bits of vs_ctx_enable_timing, in vs_stage_times field order
TIME_STAGES = ("project", "emit", "sort", "ranges", "raster_fwd", "raster_bwd", "project_bwd", "other")
TIME_ALL = (1 << len(TIME_STAGES)) - 1
PROJ_ROW_FLOATS = 16   # VS_PROJ_ROW_FLOATS: stride of the state view's projected rows


class VsCamera(C.Structure):
    _fields_ = [("model", C.c_int32), ("fx", C.c_float), ("fy", C.c_float), ("cx", C.c_float), ("cy", C.c_float),
                ("kb4", C.c_float * 4), ("viewmat", C.c_float * 12), ("cam_pos", C.c_float * 3),
                ("half_max_render_fov", C.c_float), ("lim_pos_x", C.c_float), ("lim_pos_y", C.c_float),
                ("lim_neg_x", C.c_float), ("lim_neg_y", C.c_float), ("lim_r", C.c_float), ("dist", C.c_float * 8)]


class VsPose(C.Structure):
    _fields_ = [("fov_x", C.c_double), ("fov_y", C.c_double), ("center_uv", C.c_float * 2),
                ("position", C.c_float * 3), ("rotation", C.c_float * 4), ("model", C.c_int32), ("kb4", C.c_float * 4),
                ("dist", C.c_float * 8)]


class VsSplats(C.Structure):
    _fields_ = [("transforms", C.c_void_p), ("sh_coeffs", C.c_void_p), ("raw_opacities", C.c_void_p),
                ("num_splats", C.c_uint32), ("sh_degree", C.c_uint32), ("log_scale_offset", C.c_float),
                ("sh_dtype", C.c_uint32), ("min_scale", C.c_void_p), ("decoder", C.c_void_p)]


class VsShStepParams(C.Structure):
    _fields_ = [("beta1", C.c_float), ("beta2", C.c_float), ("inv1", C.c_float), ("inv2", C.c_float),
                ("epsilon", C.c_float), ("lr", C.c_float), ("round_seed", C.c_uint32), ("first", C.c_uint32)]


class VsFwdOut(C.Structure):
    _fields_ = [("out_img", C.c_void_p), ("visible", C.c_void_p), ("max_radius", C.c_void_p),
                ("opacities", C.c_void_p), ("tile_offsets", C.c_void_p),
                ("num_visible", C.c_uint32), ("num_intersections", C.c_uint32)]


class VsGrads(C.Structure):
    _fields_ = [("v_transforms", C.c_void_p), ("v_sh_coeffs", C.c_void_p), ("v_raw_opacities", C.c_void_p),
                ("v_refine_weight", C.c_void_p), ("v_combined", C.c_void_p), ("v_decoder", C.c_void_p),
                ("v_coeffs_sq", C.c_void_p)]


class VsStageTimes(C.Structure):
    _fields_ = [(n, C.c_float) for n in ("project_ms", "emit_ms", "sort_ms", "ranges_ms", "raster_fwd_ms",
                                         "raster_bwd_ms", "project_bwd_ms", "other_ms")]


class VsStateView(C.Structure):
    _fields_ = [("num_splats", C.c_uint32), ("num_visible", C.c_uint32), ("num_intersections", C.c_uint32),
                ("num_tiles", C.c_uint32), ("tile_bw", C.c_uint32), ("tile_bh", C.c_uint32),
                ("isect_tiles", C.c_void_p), ("isect_gids", C.c_void_p), ("intersect_counts", C.c_void_p),
                ("depth_bits", C.c_void_p), ("compact_from_global", C.c_void_p),
                ("proj_xy_conic", C.c_void_p), ("proj_c11_opac_rg", C.c_void_p), ("proj_b", C.c_void_p),
                ("proj_aux", C.c_void_p), ("tile_ranges", C.c_void_p), ("proj_surf", C.c_void_p),
                ("listed_intersections", C.c_uint32), ("depth_cutoff", C.c_uint32), ("listed_counts", C.c_void_p)]


class VsLossCfg(C.Structure):
    _fields_ = [("l1_weight", C.c_float), ("ssim_weight", C.c_float), ("alpha_weight", C.c_float),
                ("composite", C.c_int32), ("bg", C.c_float * 3), ("mask", C.c_int32)]


class VsAdamStep(C.Structure):
    _fields_ = [("beta1", C.c_float), ("beta2", C.c_float), ("inv1", C.c_float), ("inv2", C.c_float),
                ("epsilon", C.c_float), ("lr_opac", C.c_float), ("opac_reg", C.c_float), ("round_seed", C.c_uint32)]


class VsUpdateOut(C.Structure):
    _fields_ = [("color_dir", C.c_void_p), ("v_refine_weight", C.c_void_p), ("coeffs_grad_sq", C.c_void_p)]


# name -> (restype, argtypes); the list is the ABI surface the tests check.
SIGNATURES = {
    "vs_ctx_create": (C.c_int, [C.c_int, C.c_void_p, C.POINTER(C.c_void_p)]),
    "vs_ctx_destroy": (None, [C.c_void_p]),
    "vs_ctx_set_stream": (C.c_int, [C.c_void_p, C.c_void_p]),
    "vs_last_error": (C.c_char_p, []),
    "vs_version": (C.c_char_p, []),
    "vs_ctx_set_sort_spin_limit": (C.c_int, [C.c_void_p, C.c_uint32]),
    "vs_ctx_set_validation": (C.c_int, [C.c_void_p, C.c_int]),
    "vs_ctx_set_depth_cutoff": (C.c_int, [C.c_void_p, C.c_int]),
    "vs_ctx_set_poison": (C.c_int, [C.c_void_p, C.c_int]),
    "vs_ctx_enable_timing": (C.c_int, [C.c_void_p, C.c_uint32]),
    "vs_ctx_stage_times": (C.c_int, [C.c_void_p, C.POINTER(VsStageTimes)]),
    "vs_ctx_set_lagged_counts": (C.c_int, [C.c_void_p, C.c_int]),
    "vs_ctx_settle_lagged_counts": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "vs_fov_to_focal": (C.c_double, [C.c_double, C.c_uint32, C.c_int32, C.POINTER(C.c_float)]),
    "vs_focal_to_fov": (C.c_double, [C.c_double, C.c_uint32, C.c_int32, C.POINTER(C.c_float)]),
    "vs_max_render_theta": (C.c_double, [C.c_int32, C.POINTER(C.c_float)]),
    "vs_camera_uniforms": (C.c_int, [C.POINTER(VsPose), C.c_uint32, C.c_uint32, C.POINTER(VsCamera)]),
    "vs_render_forward": (C.c_int, [C.c_void_p, C.POINTER(VsCamera), C.POINTER(VsSplats), C.c_uint32, C.c_uint32,
                                    C.POINTER(C.c_float), C.c_int, C.c_int, C.POINTER(VsFwdOut),
                                    C.POINTER(C.c_void_p)]),
    "vs_render_backward": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(VsSplats), C.c_void_p, C.c_void_p,
                                     C.POINTER(VsGrads)]),
    "vs_fwd_state_free": (None, [C.c_void_p]),
    "vs_fwd_state_view": (C.c_int, [C.c_void_p, C.POINTER(VsStateView)]),
    "vs_pose_backward": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(VsSplats), C.c_void_p, C.c_void_p]),
    "vs_project_update": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(VsAdamStep),
                                    C.POINTER(VsUpdateOut)]),
    "vs_geo_encode": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_float, C.c_void_p]),
    "vs_geo_decode": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_float, C.c_void_p, C.c_void_p]),
    "vs_geo_zero_rows": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint32, C.c_uint32]),
    "vs_block8_encode": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p]),
    "vs_block8_decode": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p]),
    "vs_block8_zero_rows": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32]),
    "vs_sh_step": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                             C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(VsShStepParams)]),
    "vs_radix_argsort_u32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32,
                                       C.c_uint32, C.c_void_p, C.c_void_p]),
    "vs_radix_argsort_u32_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p,
                                               C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]),
    "vs_radix_argsort_u64": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p,
                                       C.c_void_p]),
    "vs_prefix_sum_u32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]),
    "vs_stream_probe": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_int32]),
    "vs_compositing_exp2": (C.c_int, [C.c_void_p, C.c_uint32, C.c_uint64, C.c_void_p]),
    "vs_raster_division": (C.c_int, [C.c_void_p, C.c_float, C.c_void_p, C.c_uint64, C.c_void_p]),
    "vs_raster_division_mismatches": (C.c_int, [C.c_void_p, C.c_float, C.c_void_p]),
    "vs_render_forward_l1": (C.c_int, [C.c_void_p, C.POINTER(VsCamera), C.POINTER(VsSplats), C.c_uint32, C.c_uint32,
                                       C.POINTER(C.c_float), C.c_int, C.c_int, C.c_void_p, C.c_float, C.c_float,
                                       C.c_float, C.c_void_p, C.POINTER(VsFwdOut), C.POINTER(C.c_void_p)]),
    "vs_scan_in_place_u32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32]),
    "vs_image_loss_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32,
                                        C.POINTER(VsLossCfg), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "vs_image_loss_backward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32,
                                         C.POINTER(VsLossCfg), C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p]),
    "vs_l1_cotangent": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32,
                                  C.c_float, C.c_float, C.c_float, C.c_void_p]),
    "vs_l1_cotangent_packed": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32,
                                         C.c_float, C.c_float, C.c_float, C.c_void_p]),
}

_LIB = None


class VsError(RuntimeError):
    """A vs_status other than VS_OK, with the library's message."""

    def __init__(self, status: int, message: str):
        name = STATUS_NAMES[status] if 0 <= status < len(STATUS_NAMES) else str(status)
        super().__init__(f"{name}: {message}")
        self.status = status


def load() -> C.CDLL:
    """Load libvsplat.so (built by vauss_amd.build); raise if it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built; run `python -m vauss_amd.build` "
                          "(the renderer has no CPU or eager fallback)")
    lib = C.CDLL(os.fspath(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(status: int) -> None:
    if status != VS_OK:
        raise VsError(status, load().vs_last_error().decode(errors="replace"))
