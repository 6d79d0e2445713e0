"""vauss_amd -- an MI355X (gfx950) Gaussian-splat rasterizer behind the
splat-train-render / splat-train-sort call surface of voyager-so/vauss.

The compute path is libvsplat.so (hand-written HIP kernels + C ABI,
include/vsplat.h); this package is its host-side mirror.  Importing it
loads torch first so the library shares torch's HIP runtime.
"""
from ._lib import VsError, load  # noqa: F401
from .loss import (  # noqa: F401
    ImageLossConfig, image_loss, image_loss_backward, image_loss_eval, image_loss_forward_train,
    image_loss_partials, pack_rgba8,
)
from .camera import (  # noqa: F401
    PINHOLE, Camera, KannalaBrandt4, RadialTangential8, ThinPrismFisheye, fov_to_focal, focal_to_fov, max_render_theta,
)
from .render import (  # noqa: F401
    Block8Moment, Context, ForwardState, FusedAdam, ProjectUpdateResult, RasterPass, RenderAux, RenderOutput,
    ShStepState, SplatGrads, SplatRenderMode, adam_bias_corrections, compositing_exp2, geo_decode, geo_encode, geo_zero_rows,
    l1_cotangent, pose_backward, prefix_sum, project_update, radix_argsort, radix_argsort_skip_low_with_count, radix_argsort_u64,
    radix_argsort_with_count, raster_division, raster_division_mismatches, render, render_backward, scan_in_place,
    sh_degree_from_coeffs, sh_step, unpack_rgba8,
)

__all__ = [
    "ImageLossConfig", "image_loss", "image_loss_backward", "image_loss_eval", "image_loss_forward_train",
    "image_loss_partials", "pack_rgba8",
    "Camera", "KannalaBrandt4", "RadialTangential8", "ThinPrismFisheye", "PINHOLE", "fov_to_focal", "focal_to_fov", "max_render_theta",
    "Block8Moment", "ShStepState", "adam_bias_corrections", "sh_step",
    "Context", "ForwardState", "FusedAdam", "ProjectUpdateResult", "RasterPass", "RenderAux", "RenderOutput",
    "SplatGrads", "SplatRenderMode", "VsError", "compositing_exp2", "geo_decode", "geo_encode", "geo_zero_rows", "l1_cotangent", "load",
    "pose_backward", "prefix_sum", "project_update", "radix_argsort", "radix_argsort_skip_low_with_count",
    "radix_argsort_u64", "radix_argsort_with_count", "raster_division", "raster_division_mismatches", "render", "render_backward", "scan_in_place",
    "sh_degree_from_coeffs", "unpack_rgba8",
]
