"""Host-side mirror of the reference's render / sort / scan call surface.

The functions keep the reference's names, argument meaning and error
behaviour and drive the gfx950 kernels through the C ABI (include/vsplat.h):

  render              SplatOps::render               crates/splat-train-render/src/lib.rs:53-90
  render_backward     SplatBwdOps::rasterize_bwd +   bwd/burn_glue.rs:70-111
                      project_bwd (dense gradients)
  radix_argsort*      crates/splat-train-sort/src/lib.rs:15-189
  prefix_sum          crates/splat-train-scan/src/lib.rs:24-83
  scan_in_place       crates/splat-train-scan/src/lib.rs:85-96

Tensors are torch tensors on a ROCm device; torch provides device memory and
streams only.  u32 data travels in int32 tensors (same bits), u64 keys in
int64 tensors.
"""
from __future__ import annotations

import ctypes as C
import enum
import math
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from .camera import Camera


class RasterPass(enum.IntEnum):
    """RasterPass (gaussian_splats.rs:32-107).  BACKWARD_DENSE and EXPOSURE
    take the reference's `slot` as render()'s `count_slot`."""
    FORWARD = _lib.PASS_FORWARD
    BACKWARD = _lib.PASS_BACKWARD
    FLOAT = _lib.PASS_FLOAT
    BACKWARD_SMOOTH_CUTOFF = _lib.PASS_BACKWARD_SMOOTH_CUTOFF
    GEOMETRY = _lib.PASS_GEOMETRY
    BACKWARD_DENSE = _lib.PASS_BACKWARD_DENSE
    EXPOSURE = _lib.PASS_EXPOSURE
    BACKWARD_FUSED_UPDATE = _lib.PASS_BACKWARD_FUSED_UPDATE
    GEOMETRY_TRAIN_DEPTH = _lib.PASS_GEOMETRY_TRAIN_DEPTH

    def bwd_info(self) -> bool:
        return self is not RasterPass.FORWARD

    def training(self) -> bool:
        """Training renders, which use lagged counts when the context enables them."""
        return self in (RasterPass.BACKWARD, RasterPass.BACKWARD_DENSE, RasterPass.EXPOSURE,
                        RasterPass.BACKWARD_FUSED_UPDATE)

    def has_slot(self) -> bool:
        return self in (RasterPass.BACKWARD_DENSE, RasterPass.EXPOSURE)

    def geometry(self) -> bool:
        return self in (RasterPass.GEOMETRY, RasterPass.GEOMETRY_TRAIN_DEPTH)

    def surface_criterion(self) -> bool:
        """Surfel depth by the unbiased surface criterion rather than the training median."""
        return not self.training() and self is not RasterPass.GEOMETRY_TRAIN_DEPTH

    def out_channels(self, surfel: bool = False) -> int:
        """Image channels: 12 for the geometry passes and every surfel pass with
        backward state (render.rs:471-473), 4 for other float passes, 1 packed."""
        if self.geometry() or (surfel and self.bwd_info()):
            return 12
        return 4 if self.bwd_info() else 1


class SplatRenderMode(enum.IntEnum):
    """SplatRenderMode (gaussian_splats.rs:19-26): DEFAULT, MIP, and SURFEL (2DGS, pinhole-only,
    SH colour; v_combined rows of 17 in the backward)."""
    DEFAULT = _lib.MODE_DEFAULT
    MIP = _lib.MODE_MIP
    SURFEL = _lib.MODE_SURFEL


def sh_degree_from_coeffs(n: int) -> int:
    """crates/splat-train-render/src/sh.rs:10-19."""
    table = {1: 0, 4: 1, 9: 2, 16: 3, 25: 4}
    if n not in table:
        raise ValueError(f"Unsupported SH coefficient count {n}: expected 1, 4, 9, 16 or 25")
    return table[n]


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


class Context:
    """One vs_ctx per (device, stream); work goes on torch's current stream."""

    _cache: dict = {}

    def __init__(self, device: int):
        self.lib = _lib.load()
        h = C.c_void_p()
        _lib.check(self.lib.vs_ctx_create(device, None, C.byref(h)))
        self.handle = h
        self.device = device
        self.validation = False

    @classmethod
    def get(cls, device: torch.device) -> "Context":
        idx = device.index if device.index is not None else torch.cuda.current_device()
        ctx = cls._cache.get(idx)
        if ctx is None:
            ctx = cls._cache[idx] = Context(idx)
        stream = torch.cuda.current_stream(idx).cuda_stream
        _lib.check(ctx.lib.vs_ctx_set_stream(ctx.handle, C.c_void_p(stream)))
        return ctx

    def enable_timing(self, on: bool = True, stages: Optional[Sequence[str]] = None) -> None:
        """Bracket the named stages (all when `stages` is None) with HIP events."""
        mask = 0
        if on:
            names = _lib.TIME_STAGES if stages is None else stages
            for name in names:
                mask |= 1 << _lib.TIME_STAGES.index(name)
        _lib.check(self.lib.vs_ctx_enable_timing(self.handle, mask))

    def stage_times(self) -> dict:
        t = _lib.VsStageTimes()
        _lib.check(self.lib.vs_ctx_stage_times(self.handle, C.byref(t)))
        return {name: getattr(t, name) for name, _ in _lib.VsStageTimes._fields_}

    def set_validation(self, on: bool = True) -> None:
        """Validation readbacks (validation.rs): renders scan their inputs and
        backwards their gradients; NaN / Inf raise VsError(VS_ERR_NONFINITE)."""
        _lib.check(self.lib.vs_ctx_set_validation(self.handle, 1 if on else 0))
        self.validation = bool(on)

    CUTOFF_AUTO, CUTOFF_OFF, CUTOFF_ON = 0, 1, 2

    def set_depth_cutoff(self, mode: int) -> None:
        """Depth cutoff of the tile lists (vs_ctx_set_depth_cutoff): CUTOFF_OFF
        (the default: every pair listed, as the reference does), CUTOFF_ON
        (every gaussian render) or CUTOFF_AUTO (renders listing at least 2048
        pairs per tile).  Images, visibility, consumed tile ranges and
        gradients are the full list's either way; with the cutoff applied
        the aux tile_offsets index the shortened list (same range lengths,
        other starts)."""
        _lib.check(self.lib.vs_ctx_set_depth_cutoff(self.handle, int(mode)))

    def set_poison(self, on: bool = True) -> None:
        """Fill every library allocation with -12345.0 before first use (a debug aid)."""
        _lib.check(self.lib.vs_ctx_set_poison(self.handle, 1 if on else 0))

    def set_sort_spin_limit(self, polls: Optional[int] = None) -> None:
        """Polls of an unpublished predecessor before a one-sweep radix pass
        gives up (None: the default).  A pass that gives up makes the call that
        ran it fail with VS_ERR_HIP."""
        _lib.check(self.lib.vs_ctx_set_sort_spin_limit(self.handle, 0xFFFFFFFF if polls is None else int(polls)))

    def set_lagged_counts(self, on: bool = True) -> None:
        """Training renders (RasterPass.training()) at an already-seen image size
        and count slot run on a capacity hint and device counts without waiting
        for the GPU; their aux counts are the previous such render's at that
        (size, slot) (render.rs:741-768)."""
        _lib.check(self.lib.vs_ctx_set_lagged_counts(self.handle, 1 if on else 0))

    def settle_lagged_counts(self) -> tuple:
        """(lagged renders settled, of which overflowed their capacity)."""
        r, o = C.c_uint64(), C.c_uint64()
        _lib.check(self.lib.vs_ctx_settle_lagged_counts(self.handle, C.byref(r), C.byref(o)))
        return int(r.value), int(o.value)


@dataclass
class RenderAux:
    """RenderAux, render_aux.rs:74-100."""
    num_visible: int
    num_intersections: int
    visible: Optional[torch.Tensor]
    max_radius: torch.Tensor
    opacities: torch.Tensor
    tile_offsets: torch.Tensor
    img_size: tuple


class ForwardState:
    """Owner of the library's backward state (vs_fwd_state)."""

    def __init__(self, handle: C.c_void_p, ctx: Context, pass_: RasterPass, num_splats: int, sh_degree: int):
        self.handle = handle
        self.ctx = ctx
        self.pass_ = pass_
        self.num_splats = num_splats
        self.sh_degree = sh_degree
        self.keep = None                # tensors the library state borrows (the scale floor)

    def view(self) -> _lib.VsStateView:
        v = _lib.VsStateView()
        _lib.check(self.ctx.lib.vs_fwd_state_view(self.handle, C.byref(v)))
        return v

    def compact_from_global(self, device: torch.device) -> torch.Tensor:
        """A copy of compact_from_global [N]: g + 1 for splats past every cull, 0 if culled."""
        v = self.view()

        class _Dev:
            __cuda_array_interface__ = {"shape": (v.num_splats,), "typestr": "<i4",
                                        "data": (v.compact_from_global, False), "version": 2, "strides": None}
        with torch.cuda.device(device):
            return torch.as_tensor(_Dev(), device=device).clone()

    def tile_ranges(self, device: torch.device) -> torch.Tensor:
        """A copy of the tile ranges before the forward shrank their ends, [ty, tx, 2] (u32 bits in int32)."""
        v = self.view()

        class _Dev:   # a borrowed device array, copied at once
            __cuda_array_interface__ = {"shape": (v.tile_bh, v.tile_bw, 2), "typestr": "<i4",
                                        "data": (v.tile_ranges, False), "version": 2, "strides": None}
        with torch.cuda.device(device):
            return torch.as_tensor(_Dev(), device=device).clone()

    def free(self) -> None:
        if self.handle:
            self.ctx.lib.vs_fwd_state_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class RenderOutput:
    """RenderOutput, render_aux.rs:17-42 (state is opaque here)."""
    out_img: torch.Tensor
    aux: RenderAux
    state: Optional[ForwardState]
    camera_uniforms: _lib.VsCamera
    background: tuple
    v_l1: Optional[torch.Tensor] = None     # the L1 cotangent written with the image (render's l1_target)


@dataclass
class SplatGrads:
    """SplatGrads (bwd/burn_glue.rs:28-35), dense per global splat."""
    v_transforms: torch.Tensor
    v_coeffs: torch.Tensor
    v_raw_opac: torch.Tensor
    v_refine_weight: torch.Tensor
    v_combined: torch.Tensor
    v_decoder: Optional[torch.Tensor] = None     # neural appearance: [816]
    v_coeffs_sq: Optional[torch.Tensor] = None   # neural appearance: [N] mean square of each row gradient


NEURAL_DECODER_LEN = 816     # kernels/neural.rs:42-49: W1 16x32, W2 16x16, W3 3x16


def _check_decoder(decoder: Optional[torch.Tensor], neural_degree: int) -> Optional[torch.Tensor]:
    if decoder is None:
        return None
    if decoder.dtype != torch.float32 or decoder.numel() != NEURAL_DECODER_LEN or not decoder.is_cuda:
        raise ValueError("decoder must be a float32 GPU tensor of 816 weights")
    if not 0 <= int(neural_degree) <= 3:
        raise ValueError("neural_degree (the decoder's direction band) must be 0..3")
    return decoder.contiguous()


def _check_splats(transforms, sh_coeffs, raw_opacities, neural_degree: Optional[int] = None):
    if transforms.dim() != 2 or transforms.shape[1] != 10:
        raise ValueError(f"transforms must be [N, 10], got {tuple(transforms.shape)}")
    n = transforms.shape[0]
    if sh_coeffs.dim() != 3 or sh_coeffs.shape[0] != n or sh_coeffs.shape[2] != 3:
        raise ValueError(f"sh_coeffs must be [N, C, 3], got {tuple(sh_coeffs.shape)}")
    if raw_opacities.dim() != 1 or raw_opacities.shape[0] != n:
        raise ValueError(f"raw_opacities must be [N], got {tuple(raw_opacities.shape)}")
    for name, t in (("transforms", transforms), ("raw_opacities", raw_opacities)):
        if t.dtype != torch.float32:
            raise TypeError(f"{name} must be float32, got {t.dtype}")
    # render.rs:683-687: SH coefficients in f32 or f16.
    if sh_coeffs.dtype not in (torch.float32, torch.float16):
        raise TypeError(f"SH coefficients must use f16 or f32, got {sh_coeffs.dtype}")
    for name, t in (("transforms", transforms), ("sh_coeffs", sh_coeffs), ("raw_opacities", raw_opacities)):
        if not t.is_cuda:
            raise ValueError(f"{name} must live on the GPU")
    if neural_degree is not None:
        # neural appearance rows: base (3), latent (8), pad as 4 coefficients (kernels/neural.rs:37-40)
        if sh_coeffs.shape[1] != 4:
            raise ValueError("neural appearance rows must be [N, 4, 3]")
        return n, int(neural_degree)
    return n, sh_degree_from_coeffs(sh_coeffs.shape[1])


def _min_scale(min_scale: Optional[torch.Tensor], n: int) -> Optional[torch.Tensor]:
    if min_scale is None:
        return None
    if min_scale.dtype != torch.float32 or min_scale.numel() != n or not min_scale.is_cuda:
        raise ValueError("min_scale must be a float32 [N] GPU tensor")
    return min_scale.contiguous().reshape(n)


def _splats_struct(transforms, sh_coeffs, raw_opacities, degree, log_scale_offset, min_scale=None,
                   decoder=None) -> _lib.VsSplats:
    s = _lib.VsSplats()
    s.transforms = _ptr(transforms)
    s.sh_coeffs = _ptr(sh_coeffs)
    s.raw_opacities = _ptr(raw_opacities)
    s.num_splats = transforms.shape[0]
    s.sh_degree = degree
    s.log_scale_offset = float(log_scale_offset)
    s.sh_dtype = _lib.VS_SH_F16 if sh_coeffs.dtype == torch.float16 else _lib.VS_SH_F32
    s.min_scale = _ptr(min_scale)
    s.decoder = _ptr(decoder)
    return s


def render(camera, img_size: Sequence[int], transforms: torch.Tensor, sh_coeffs: torch.Tensor,
           raw_opacities: torch.Tensor, background=(0.0, 0.0, 0.0), pass_: RasterPass = RasterPass.BACKWARD,
           render_mode: SplatRenderMode = SplatRenderMode.DEFAULT, log_scale_offset: float = 0.0,
           validate: bool = False, min_scale: Optional[torch.Tensor] = None,
           decoder: Optional[torch.Tensor] = None, neural_degree: int = 0, count_slot: int = 0,
           l1_target: Optional[torch.Tensor] = None, l1_mask_center=(0.0, 0.0),
           l1_mask_radius: float = 0.0) -> RenderOutput:
    """SplatOps::render (SplatOps::render_neural with `decoder`).  `camera` is
    a Camera or ready-made vs_camera uniforms.  `render_mode` DEFAULT or MIP;
    `min_scale` [N] is the scale floor (render's min_scale with
    has_min_scale), None for none.  With `decoder` [816] the colour comes from
    the compact neural appearance: `sh_coeffs` holds [N,4,3] rows (base,
    latent, pad) and `neural_degree` (0..3) is its direction band.

    `count_slot` (0..255) is the slot of a BACKWARD_DENSE or EXPOSURE pass
    (RasterPass::BackwardDense { slot }): its lagged counts stay apart from
    the step's other renders at the same size.

    `l1_target` ([H,W] int32 packed RGBA8) makes the raster pass also write
    the L1 term's cotangent of its image (vs_render_forward_l1, the values of
    l1_cotangent with that target and circle mask) into `v_l1`: a float RGBA
    pass, not surfels.

    Returns the image ([H,W,C] f32, or [H,W] int32-packed RGBA8 for
    FORWARD), the aux outputs and, for every pass but FORWARD, the state the
    backward needs."""
    w, h = int(img_size[0]), int(img_size[1])
    if w <= 0 or h <= 0:
        raise ValueError("Can't render images with 0 size.")
    pass_ = RasterPass(pass_)
    if count_slot and not pass_.has_slot():
        raise ValueError("only BACKWARD_DENSE and EXPOSURE passes take a count slot")
    if not 0 <= int(count_slot) <= 255:
        raise ValueError("count_slot must be 0..255")
    transforms = transforms.contiguous()
    sh_coeffs = sh_coeffs.contiguous()
    raw_opacities = raw_opacities.contiguous()
    decoder = _check_decoder(decoder, neural_degree)
    n, degree = _check_splats(transforms, sh_coeffs, raw_opacities, None if decoder is None else neural_degree)
    dev = transforms.device
    ctx = Context.get(dev)
    cam = camera.uniforms((w, h)) if isinstance(camera, Camera) else camera
    tbw, tbh = (w + 15) // 16, (h + 15) // 16
    ch = pass_.out_channels(SplatRenderMode(render_mode) is SplatRenderMode.SURFEL)
    if ch == 1:
        out_img = torch.empty((h, w), dtype=torch.int32, device=dev)
    else:
        out_img = torch.empty((h, w, ch), dtype=torch.float32, device=dev)
    visible = torch.empty(n, dtype=torch.float32, device=dev) if pass_.bwd_info() else None
    max_radius = torch.empty(n, dtype=torch.float32, device=dev)
    opacities = torch.empty(n, dtype=torch.float32, device=dev)
    tile_offsets = torch.empty((tbh, tbw, 2), dtype=torch.int32, device=dev)
    out = _lib.VsFwdOut()
    out.out_img = _ptr(out_img)
    out.visible = _ptr(visible)
    out.max_radius = _ptr(max_radius)
    out.opacities = _ptr(opacities)
    out.tile_offsets = _ptr(tile_offsets)
    min_scale = _min_scale(min_scale, n)
    splats = _splats_struct(transforms, sh_coeffs, raw_opacities, degree, log_scale_offset, min_scale, decoder)
    bg = (C.c_float * 3)(*[float(v) for v in background])
    st = C.c_void_p()
    was_validating = ctx.validation
    if validate and not was_validating:
        ctx.set_validation(True)
    v_l1 = None
    if l1_target is not None:
        if ch != 4 or SplatRenderMode(render_mode) is SplatRenderMode.SURFEL:
            raise ValueError("the fused L1 cotangent takes a float RGBA pass (no geometry channels, no surfels)")
        l1_target = l1_target.contiguous()
        if l1_target.dtype != torch.int32 or tuple(l1_target.shape) != (h, w):
            raise ValueError(f"l1_target must be int32 [{h}, {w}] packed RGBA8, got {l1_target.dtype} "
                             f"{tuple(l1_target.shape)}")
        v_l1 = torch.empty((h, w, 4), dtype=torch.float32, device=dev)
    try:
        if v_l1 is None:
            _lib.check(ctx.lib.vs_render_forward(ctx.handle, C.byref(cam), C.byref(splats), w, h, bg,
                                                 _lib.pass_with_slot(pass_, count_slot), int(render_mode),
                                                 C.byref(out), C.byref(st)))
        else:
            _lib.check(ctx.lib.vs_render_forward_l1(ctx.handle, C.byref(cam), C.byref(splats), w, h, bg,
                                                    _lib.pass_with_slot(pass_, count_slot), int(render_mode),
                                                    _ptr(l1_target), float(l1_mask_center[0]),
                                                    float(l1_mask_center[1]), float(l1_mask_radius), _ptr(v_l1),
                                                    C.byref(out), C.byref(st)))
    finally:
        if validate and not was_validating:
            ctx.set_validation(False)
    aux = RenderAux(out.num_visible, out.num_intersections, visible, max_radius, opacities, tile_offsets, (w, h))
    state = ForwardState(st, ctx, pass_, n, degree) if st.value else None
    if state is not None:
        state.keep = min_scale          # the state borrows the floor for project_update
        state.surfel = SplatRenderMode(render_mode) is SplatRenderMode.SURFEL
    return RenderOutput(out_img, aux, state, cam, tuple(float(v) for v in background), v_l1)


def render_backward(output: RenderOutput, transforms: torch.Tensor, sh_coeffs: torch.Tensor,
                    raw_opacities: torch.Tensor, v_output: torch.Tensor,
                    fused: bool = False, min_scale: Optional[torch.Tensor] = None,
                    decoder: Optional[torch.Tensor] = None) -> SplatGrads:
    """rasterize_bwd followed by project_bwd (project_bwd_neural with
    `decoder`, the forward's), returning dense gradients.  The log-scale
    offset is the forward's (the reference's ProjectUniforms carry it from the
    forward to project_bwd).

    With `fused` the backward stops at the raster gradients (the
    BackwardFusedUpdate pass): only `v_combined` is filled, for
    project_update; the other fields are None.  In neural mode `v_coeffs`
    holds the [N,4,3] row gradients, and `v_decoder` [816] and `v_coeffs_sq`
    [N] are filled."""
    if output.state is None or output.state.handle is None:
        raise ValueError("the forward pass kept no backward state (use a bwd-info pass)")
    # a BACKWARD_FUSED_UPDATE render's backward always stops at the raster gradients
    fused = fused or output.state.pass_ is RasterPass.BACKWARD_FUSED_UPDATE
    transforms = transforms.contiguous()
    sh_coeffs = sh_coeffs.contiguous()
    raw_opacities = raw_opacities.contiguous()
    decoder = _check_decoder(decoder, output.state.sh_degree if decoder is not None else 0)
    n, degree = _check_splats(transforms, sh_coeffs, raw_opacities,
                              None if decoder is None else output.state.sh_degree)
    v_output = v_output.contiguous()
    if v_output.shape != output.out_img.shape or v_output.dtype != torch.float32:
        raise ValueError(f"v_output must be float32 {tuple(output.out_img.shape)}, got {tuple(v_output.shape)}")
    dev = transforms.device
    ctx = output.state.ctx
    Context.get(dev)
    k = 4 if decoder is not None else (degree + 1) ** 2
    n_grads = 17 if getattr(output.state, "surfel", False) else 10     # surfel rows: M, normal, rgb, alpha, refine
    if fused:
        g = SplatGrads(None, None, None, None, torch.empty((n, n_grads), dtype=torch.float32, device=dev))
    else:
        g = SplatGrads(torch.empty((n, 10), dtype=torch.float32, device=dev),
                       torch.empty((n, k, 3), dtype=torch.float32, device=dev),
                       torch.empty(n, dtype=torch.float32, device=dev),
                       torch.empty(n, dtype=torch.float32, device=dev),
                       torch.empty((n, n_grads), dtype=torch.float32, device=dev))
        if decoder is not None:
            g.v_decoder = torch.empty(NEURAL_DECODER_LEN, dtype=torch.float32, device=dev)
            g.v_coeffs_sq = torch.empty(n, dtype=torch.float32, device=dev)
    grads = _lib.VsGrads()
    grads.v_transforms = _ptr(g.v_transforms)
    grads.v_sh_coeffs = _ptr(g.v_coeffs)
    grads.v_raw_opacities = _ptr(g.v_raw_opac)
    grads.v_refine_weight = _ptr(g.v_refine_weight)
    grads.v_combined = _ptr(g.v_combined)
    grads.v_decoder = _ptr(g.v_decoder)
    grads.v_coeffs_sq = _ptr(g.v_coeffs_sq)
    splats = _splats_struct(transforms, sh_coeffs, raw_opacities, degree, 0.0, _min_scale(min_scale, n), decoder)
    _lib.check(ctx.lib.vs_render_backward(ctx.handle, output.state.handle, C.byref(splats), _ptr(output.out_img),
                                          _ptr(v_output), C.byref(grads)))
    return g


def pose_backward(output: RenderOutput, transforms: torch.Tensor, sh_coeffs: torch.Tensor,
                  raw_opacities: torch.Tensor, v_combined: torch.Tensor,
                  min_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """pose_bwd (bwd/render_bwd.rs:224-288): the camera gradient [12] =
    d loss / d [A (row-major 3x3), b] of x_c' = (I + A) x_c + b, from the raster
    gradient rows `v_combined` [N,10] of render_backward on `output`."""
    if output.state is None or output.state.handle is None:
        raise ValueError("the forward pass kept no backward state (use a bwd-info pass)")
    transforms = transforms.contiguous()
    sh_coeffs = sh_coeffs.contiguous()
    raw_opacities = raw_opacities.contiguous()
    n, degree = _check_splats(transforms, sh_coeffs, raw_opacities)
    v_combined = v_combined.contiguous()
    if tuple(v_combined.shape) != (n, 10) or v_combined.dtype != torch.float32:
        raise ValueError("v_combined must be float32 [N, 10]")
    dev = transforms.device
    ctx = output.state.ctx
    Context.get(dev)
    v_pose = torch.empty(12, dtype=torch.float32, device=dev)
    splats = _splats_struct(transforms, sh_coeffs, raw_opacities, degree, 0.0, _min_scale(min_scale, n))
    _lib.check(ctx.lib.vs_pose_backward(ctx.handle, output.state.handle, C.byref(splats), _ptr(v_combined),
                                        _ptr(v_pose)))
    return v_pose


def _powi_f32(a: float, b: int) -> np.float32:
    """f32 a^b by binary exponentiation (Rust's f32::powi, lowered to
    compiler-rt's __powisf2)."""
    x, r, recip, b = np.float32(a), np.float32(1.0), b < 0, abs(b)
    while True:
        if b & 1:
            r = np.float32(r * x)
        b >>= 1
        if b == 0:
            break
        x = np.float32(x * x)
    return np.float32(1.0) / r if recip else r


def adam_bias_corrections(step: int, beta1: float, beta2: float):
    """AdamScaled::coefficients (crates/splat-train/src/optim.rs:269-277), in
    f32: (1 / (1 - beta1^t), 1 / (1 - beta2^t))."""
    one = np.float32(1.0)
    return (float(one / (one - _powi_f32(beta1, step))), float(one / (one - _powi_f32(beta2, step))))


@dataclass
class FusedAdam:
    """FusedAdam, bwd/project_update.rs:232-250."""
    beta1: float
    beta2: float
    inv1: float
    inv2: float
    epsilon: float
    lr_opac: float
    opac_reg: float = 0.0
    round_seed: int = 0

    @classmethod
    def at_step(cls, step: int, lr_opac: float, beta1: float = 0.9, beta2: float = 0.999, epsilon: float = 1e-15,
                opac_reg: float = 0.0) -> "FusedAdam":
        """Bias corrections of Adam step `step` (1-based); the step count seeds the rounding."""
        inv1, inv2 = adam_bias_corrections(step, beta1, beta2)
        return cls(beta1, beta2, inv1, inv2, epsilon, lr_opac, opac_reg, step)


@dataclass
class ProjectUpdateResult:
    """ProjectUpdateResult minus the tensors stepped in place (bwd/project_update.rs:252-262)."""
    color_dir: torch.Tensor        # [N+1, 6]
    v_refine_weight: torch.Tensor  # [N]
    coeffs_grad_sq: torch.Tensor   # [N, 1, 1]
    compact_from_global: torch.Tensor  # [N] rows of color_dir (g + 1), 0 for culled splats


def project_update(output: RenderOutput, transforms: torch.Tensor, sh_coeffs: torch.Tensor,
                   raw_opacities: torch.Tensor, v_combined: torch.Tensor, w_t: torch.Tensor, lr_scale: torch.Tensor,
                   w_o: torch.Tensor, adam: FusedAdam) -> ProjectUpdateResult:
    """project_update (bwd/project_update.rs:264-322): projection VJP + one
    Adam step; `transforms`, `raw_opacities`, `w_t` and `w_o` are updated in
    place.  `w_t` [N,10] and `w_o` [N] hold packed moments (int32 tensors)."""
    if output.state is None or output.state.handle is None:
        raise ValueError("the forward pass kept no backward state (use a bwd-info pass)")
    n, degree = _check_splats(transforms, sh_coeffs, raw_opacities)
    for name, t in (("transforms", transforms), ("raw_opacities", raw_opacities), ("w_t", w_t), ("w_o", w_o),
                    ("v_combined", v_combined), ("lr_scale", lr_scale)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous (it is read or updated in place)")
    _u32(w_t, "w_t")
    _u32(w_o, "w_o")
    if tuple(w_t.shape) != (n, 10) or tuple(w_o.shape) != (n,):
        raise ValueError("packed moments must be [N, 10] and [N]")
    if tuple(v_combined.shape) != (n, 10) or lr_scale.numel() != 10 or lr_scale.dtype != torch.float32:
        raise ValueError("v_combined must be [N, 10] and lr_scale [10] float32")
    sh_coeffs = sh_coeffs.contiguous()
    dev = transforms.device
    ctx = output.state.ctx
    Context.get(dev)
    res = ProjectUpdateResult(torch.empty((n + 1, 6), dtype=torch.float32, device=dev),
                              torch.empty(n, dtype=torch.float32, device=dev),
                              torch.empty((n, 1, 1), dtype=torch.float32, device=dev),
                              output.state.compact_from_global(dev))
    a = _lib.VsAdamStep(adam.beta1, adam.beta2, adam.inv1, adam.inv2, adam.epsilon, adam.lr_opac, adam.opac_reg,
                        adam.round_seed & 0xFFFFFFFF)
    out = _lib.VsUpdateOut(_ptr(res.color_dir), _ptr(res.v_refine_weight), _ptr(res.coeffs_grad_sq))
    _lib.check(ctx.lib.vs_project_update(ctx.handle, output.state.handle, _ptr(transforms), _ptr(sh_coeffs),
                                         _ptr(raw_opacities), _ptr(v_combined), _ptr(w_t), _ptr(lr_scale),
                                         _ptr(w_o), C.byref(a), C.byref(out)))
    return res


def geo_encode(m: torch.Tensor, v: torch.Tensor, epsilon: float) -> torch.Tensor:
    """encode_geo (bwd/geo_moments.rs:33-39): f32 (m, v) -> packed words, rounding to nearest."""
    m = m.contiguous().float()
    v = v.contiguous().float()
    if m.shape != v.shape:
        raise ValueError("m and v must have the same shape")
    words = torch.empty(m.shape, dtype=torch.int32, device=m.device)
    ctx = Context.get(m.device)
    _lib.check(ctx.lib.vs_geo_encode(ctx.handle, _ptr(m), _ptr(v), m.numel(), float(epsilon), _ptr(words)))
    return words


def geo_decode(words: torch.Tensor, epsilon: float):
    """decode_geo (bwd/geo_moments.rs:41-48): packed words -> f32 (m, v)."""
    words = _u32(words.contiguous(), "words")
    m = torch.empty(words.shape, dtype=torch.float32, device=words.device)
    v = torch.empty_like(m)
    ctx = Context.get(words.device)
    _lib.check(ctx.lib.vs_geo_decode(ctx.handle, _ptr(words), words.numel(), float(epsilon), _ptr(m), _ptr(v)))
    return m, v


def geo_zero_rows(words: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """zero_geo_rows (bwd/geo_moments.rs:50-58): reset the moments of `rows` in place."""
    _u32(words, "words")
    rows = _u32(rows.contiguous(), "rows")
    width = words.shape[1] if words.dim() > 1 else 1
    ctx = Context.get(words.device)
    _lib.check(ctx.lib.vs_geo_zero_rows(ctx.handle, _ptr(words), words.numel(), _ptr(rows), rows.numel(), width))
    return words


def _u32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"{name} must hold u32 data (int32/uint32 tensor), got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"Please ensure {name} is contiguous")
    return t


def radix_argsort_skip_low_with_count(input_keys: torch.Tensor, input_values: torch.Tensor, skip_bits: int,
                                      sorting_bits: int, num_keys: Optional[torch.Tensor]):
    """Stable sort of (key, value) by key bits skip..skip+8*ceil(bits/8) of the
    active prefix whose length is num_keys[0] (on the GPU)."""
    _u32(input_keys, "input keys")
    _u32(input_values, "input values")
    if input_keys.shape[0] != input_values.shape[0]:
        raise ValueError("Input keys and values must have the same number of elements")
    if skip_bits + sorting_bits > 32:
        raise ValueError("Can only sort up to 32 bits")
    n = input_keys.shape[0]
    if n == 0 or sorting_bits == 0:
        return input_keys, input_values
    ctx = Context.get(input_keys.device)
    out_k = torch.empty_like(input_keys)
    out_v = torch.empty_like(input_values)
    if num_keys is not None:
        _u32(num_keys, "num_keys")
        # entries past the active prefix keep their input values
        out_k.copy_(input_keys)
        out_v.copy_(input_values)
    _lib.check(ctx.lib.vs_radix_argsort_u32(ctx.handle, _ptr(input_keys), _ptr(input_values), n, _ptr(num_keys),
                                            skip_bits, sorting_bits, _ptr(out_k), _ptr(out_v)))
    return out_k, out_v


def radix_argsort_with_count(input_keys, input_values, sorting_bits, num_keys):
    """crates/splat-train-sort/src/lib.rs:28-35."""
    return radix_argsort_skip_low_with_count(input_keys, input_values, 0, sorting_bits, num_keys)


def radix_argsort(input_keys, input_values, sorting_bits):
    """crates/splat-train-sort/src/lib.rs:15-24."""
    return radix_argsort_skip_low_with_count(input_keys, input_values, 0, sorting_bits, None)


def radix_argsort_u64(keys: torch.Tensor, values: torch.Tensor, sorting_bits: int):
    """Stable sort of packed 64-bit keys (int64 tensor) by bits [0, sorting_bits)."""
    if keys.dtype not in (torch.int64, torch.uint64) or not keys.is_contiguous():
        raise TypeError("keys must be a contiguous int64/uint64 tensor")
    _u32(values, "values")
    n = keys.shape[0]
    ctx = Context.get(keys.device)
    out_k = torch.empty_like(keys)
    out_v = torch.empty_like(values)
    if n:
        _lib.check(ctx.lib.vs_radix_argsort_u64(ctx.handle, _ptr(keys), _ptr(values), n, sorting_bits,
                                                _ptr(out_k), _ptr(out_v)))
    return out_k, out_v


def prefix_sum(x: torch.Tensor) -> torch.Tensor:
    """Inclusive prefix sum of a contiguous 1-D u32 tensor."""
    _u32(x, "input")
    if x.shape[0] == 0:
        return x
    ctx = Context.get(x.device)
    out = torch.empty_like(x)
    _lib.check(ctx.lib.vs_prefix_sum_u32(ctx.handle, _ptr(x), _ptr(out), x.shape[0]))
    return out


def scan_in_place(x: torch.Tensor) -> None:
    """Inclusive prefix sum in place (one workgroup; meant for short arrays)."""
    _u32(x, "values")
    if x.shape[0] == 0:
        return
    ctx = Context.get(x.device)
    _lib.check(ctx.lib.vs_scan_in_place_u32(ctx.handle, _ptr(x), x.shape[0]))


def compositing_exp2(first_bits: int, count: int, device=None) -> torch.Tensor:
    """The compositing kernels' 2^x for the f32 inputs whose bit patterns are
    first_bits .. first_bits + count - 1, as a float32 tensor on the device
    (vs_compositing_exp2)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    out = torch.empty(int(count), dtype=torch.float32, device=dev)
    ctx = Context.get(dev)
    _lib.check(ctx.lib.vs_compositing_exp2(ctx.handle, int(first_bits), int(count), _ptr(out) if count else None))
    return out


def raster_division(a: float, bits: torch.Tensor) -> torch.Tensor:
    """The raster kernels' quotient a / b for the f32 divisors whose bit
    patterns `bits` holds (a uint32 or int32 device tensor), as a float32
    tensor (vs_raster_division)."""
    b = bits.contiguous()
    if b.dtype not in (torch.int32, torch.uint32) or not b.is_cuda:
        raise ValueError("bits must be a 32-bit integer device tensor")
    out = torch.empty(b.shape, dtype=torch.float32, device=b.device)
    ctx = Context.get(b.device)
    _lib.check(ctx.lib.vs_raster_division(ctx.handle, float(a), _ptr(b) if b.numel() else None, b.numel(),
                                          _ptr(out) if b.numel() else None))
    return out


def raster_division_mismatches(a: float, device=None) -> int:
    """How many of the 2^32 f32 divisors b give a raster-kernel quotient a / b
    that differs from the IEEE division (vs_raster_division_mismatches)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    count = torch.zeros(1, dtype=torch.int64, device=dev)
    ctx = Context.get(dev)
    _lib.check(ctx.lib.vs_raster_division_mismatches(ctx.handle, float(a), _ptr(count)))
    return int(count.item())


def l1_cotangent(pred: torch.Tensor, gt: torch.Tensor, mask_center=(0.0, 0.0), mask_radius: float = 0.0) -> torch.Tensor:
    """d(mean L1 over rgb)/d pred for an [H,W,C] prediction and an [H,W,3]
    float32 target, or an [H,W] int32 packed RGBA8 target (the reference's
    u8 ground truth, unpacked as byte x (1/255))."""
    pred = pred.contiguous()
    gt = gt.contiguous()
    h, w, c = pred.shape
    ctx = Context.get(pred.device)
    v = torch.empty_like(pred)
    if gt.dtype == torch.int32:
        if tuple(gt.shape) != (h, w):
            raise ValueError(f"a packed target must be int32 [{h}, {w}], got {tuple(gt.shape)}")
        fn = ctx.lib.vs_l1_cotangent_packed
    else:
        if gt.dtype != torch.float32 or tuple(gt.shape) != (h, w, 3):
            raise ValueError(f"a float target must be float32 [{h}, {w}, 3], got {gt.dtype} {tuple(gt.shape)}")
        fn = ctx.lib.vs_l1_cotangent
    _lib.check(fn(ctx.handle, _ptr(pred), c, _ptr(gt), w, h, float(mask_center[0]), float(mask_center[1]),
                  float(mask_radius), _ptr(v)))
    return v


def unpack_rgba8(packed: torch.Tensor) -> torch.Tensor:
    """[H,W] packed RGBA8 (FORWARD pass) -> [H,W,4] uint8."""
    p = packed.to(torch.int64) & 0xFFFFFFFF
    return torch.stack([(p >> s) & 0xFF for s in (0, 8, 16, 24)], dim=-1).to(torch.uint8)


# ---- the trainer's SH step: f16 coefficients, block-scaled 8-bit first moment ------

BLOCK8_VALUES = 128


@dataclass
class Block8Moment:
    """BlockMoment (crates/splat-train/src/quant.rs:30-160): `codes` [blocks*32]
    int32 words of four biased 8-bit codes, `scales` [blocks] f32, for `n`
    values in blocks of 128."""
    codes: torch.Tensor
    scales: torch.Tensor
    n: int

    @classmethod
    def zeros(cls, n: int, device) -> "Block8Moment":
        if n <= 0:
            raise ValueError("cannot quantize an empty moment")
        blocks = (n + BLOCK8_VALUES - 1) // BLOCK8_VALUES
        return cls(torch.zeros(blocks * 32, dtype=torch.int32, device=device),
                   torch.zeros(blocks, dtype=torch.float32, device=device), n)

    @classmethod
    def encode(cls, values: torch.Tensor) -> "Block8Moment":
        v = values.contiguous().float().reshape(-1)
        if v.numel() == 0:
            raise ValueError("cannot quantize an empty moment")
        m = cls.zeros(v.numel(), v.device)
        ctx = Context.get(v.device)
        _lib.check(ctx.lib.vs_block8_encode(ctx.handle, _ptr(v), v.numel(), _ptr(m.codes), _ptr(m.scales)))
        return m

    def decode(self) -> torch.Tensor:
        out = torch.empty(self.n, dtype=torch.float32, device=self.codes.device)
        ctx = Context.get(self.codes.device)
        _lib.check(ctx.lib.vs_block8_decode(ctx.handle, _ptr(self.codes), _ptr(self.scales), self.n, _ptr(out)))
        return out

    def zero_rows(self, rows: torch.Tensor, row_width: int) -> "Block8Moment":
        """reset_rows' zeroing (quant.rs:93-111): the listed rows' moments become 0, in place."""
        rows = _u32(rows.contiguous(), "rows")
        ctx = Context.get(self.codes.device)
        _lib.check(ctx.lib.vs_block8_zero_rows(ctx.handle, _ptr(self.codes), self.n, _ptr(rows), rows.numel(),
                                               int(row_width)))
        return self


@dataclass
class ShStepState:
    """The SH coefficients' optimizer state (MomentumState with split moments,
    optim.rs:413-498): the Block8 first moment, the per-splat f32 variance and
    the step count t (0 before the first step)."""
    moment: Block8Moment
    variance: torch.Tensor
    time: int = 0

    @classmethod
    def fresh(cls, num_splats: int, sh_degree: int, device) -> "ShStepState":
        k = (sh_degree + 1) ** 2
        return cls(Block8Moment.zeros(num_splats * k * 3, device),
                   torch.zeros(num_splats, dtype=torch.float32, device=device), 0)


def sh_step(sh_coeffs: torch.Tensor, color_dir: torch.Tensor, compact_from_global: torch.Tensor,
            grad_sq: torch.Tensor, state: ShStepState, lr: float, lr_scale: Optional[torch.Tensor] = None,
            beta1: float = 0.9, beta2: float = 0.999, epsilon: float = 1e-15) -> torch.Tensor:
    """AdamScaled::step_sh_color (optim.rs:391-498): one lazy Adam step of the
    SH coefficients from project_update's `color_dir` and `coeffs_grad_sq`.
    `sh_coeffs` [N,K,3] is f16 (stepped in place; an f32 tensor is first cast
    to f16, as the reference's canonical half storage, and the f16 tensor is
    returned).  `state` advances one step."""
    if sh_coeffs.dim() != 3 or sh_coeffs.shape[2] != 3:
        raise ValueError(f"sh_coeffs must be [N, C, 3], got {tuple(sh_coeffs.shape)}")
    n, k = sh_coeffs.shape[0], sh_coeffs.shape[1]
    degree = sh_degree_from_coeffs(k)
    if sh_coeffs.dtype == torch.float32:
        sh_coeffs = sh_coeffs.half()
    elif sh_coeffs.dtype != torch.float16:
        raise TypeError(f"SH coefficients must use f16 or f32, got {sh_coeffs.dtype}")
    if not sh_coeffs.is_contiguous():
        raise ValueError("sh_coeffs must be contiguous (it is stepped in place)")
    dev = sh_coeffs.device
    if color_dir.dim() != 2 or color_dir.shape[1] != 6 or color_dir.dtype != torch.float32:
        raise ValueError("color_dir must be [rows, 6] float32")
    rows = _u32(compact_from_global.contiguous(), "compact_from_global")
    gsq = grad_sq.contiguous().float().reshape(-1)
    if rows.numel() != n or gsq.numel() != n:
        raise ValueError("compact_from_global and grad_sq must have one entry per splat")
    if state.moment.n != n * k * 3 or state.variance.numel() != n:
        raise ValueError("optimizer state does not match the coefficients")
    if lr_scale is None:
        lr_scale = torch.ones(k * 3, dtype=torch.float32, device=dev)
    lr_scale = lr_scale.contiguous().float().reshape(-1)
    if lr_scale.numel() != k * 3:
        raise ValueError("lr_scale must hold one factor per coefficient value [K*3]")
    t = state.time + 1
    inv1, inv2 = adam_bias_corrections(t, beta1, beta2)
    p = _lib.VsShStepParams(beta1, beta2, inv1, inv2, epsilon, lr, t & 0xFFFFFFFF, 1 if state.time == 0 else 0)
    ctx = Context.get(dev)
    _lib.check(ctx.lib.vs_sh_step(ctx.handle, _ptr(sh_coeffs), n, degree, _ptr(color_dir.contiguous()), _ptr(rows),
                                  _ptr(gsq), _ptr(state.variance), _ptr(state.moment.codes),
                                  _ptr(state.moment.scales), _ptr(lr_scale), C.byref(p)))
    state.time = t
    return sh_coeffs
