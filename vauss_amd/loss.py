"""Host-side mirror of the reference's image loss (crates/splat-train-loss):
L1 + SSIM over an [H,W,C] f32 prediction and RGBA8-packed ground truth.

  image_loss                LossOps::image_loss_total   lib.rs:1906-1913
  image_loss_partials       image_loss_partials          lib.rs:1919-1930
  image_loss_eval           image_loss_eval              lib.rs:2102-2118
  image_loss_forward_train  LossOps::image_loss_forward_train (partials + SSIM coefficients)
  image_loss_backward       LossOps::image_loss_backward(_coeffs)

Ground truth is a [H,W] int32 tensor whose bits pack r, g, b, a bytes from the
low byte up, as the reference keeps it on the GPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib
from .render import Context, _ptr


@dataclass
class ImageLossConfig:
    """ImageLossConfig, lib.rs:1227-1260.  `ssim_weight` multiplies SSIM itself."""
    l1_weight: float
    ssim_weight: float
    composite_bg: Optional[Tuple[float, float, float]] = None
    mask: bool = False
    alpha_weight: float = 0.0

    @classmethod
    def l1_dssim(cls, ssim_weight: float) -> "ImageLossConfig":
        """(1 - w) L1 - w SSIM: 3DGS's (1 - w) L1 + w (1 - SSIM) less a constant."""
        return cls(1.0 - ssim_weight, -ssim_weight)

    def struct(self) -> _lib.VsLossCfg:
        bg = self.composite_bg if self.composite_bg is not None else (0.0, 0.0, 0.0)
        return _lib.VsLossCfg(self.l1_weight, self.ssim_weight, self.alpha_weight,
                              1 if self.composite_bg is not None else 0, (C.c_float * 3)(*bg), 1 if self.mask else 0)

    def planes(self, channels: int) -> int:
        return 4 if (self.alpha_weight > 0 and channels == 4) else 3


def loss_tiles(h: int, w: int) -> int:
    return ((w + 15) // 16) * ((h + 15) // 16)


def pack_rgba8(img: torch.Tensor) -> torch.Tensor:
    """[H,W,4] values in [0, 1] (or uint8) -> [H,W] int32 packed RGBA8."""
    if img.dtype != torch.uint8:
        img = (img.clamp(0, 1) * 255.0).round().to(torch.uint8)
    b = img.to(torch.int64)
    packed = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16) | (b[..., 3] << 24)
    return packed.to(torch.uint32).view(torch.int32) if hasattr(torch, "uint32") else \
        torch.where(packed >= 2 ** 31, packed - 2 ** 32, packed).to(torch.int32)


def _check(pred: torch.Tensor, gt_packed: torch.Tensor):
    if pred.dim() != 3 or pred.shape[2] not in (3, 4) or pred.dtype != torch.float32:
        raise ValueError(f"image loss expects [H, W, 3|4] float32 pred, got {tuple(pred.shape)} {pred.dtype}")
    if tuple(gt_packed.shape) != tuple(pred.shape[:2]) or gt_packed.dtype not in (torch.int32, torch.uint32):
        raise ValueError("gt_packed must be an [H, W] int32 tensor matching pred")
    return pred.contiguous(), gt_packed.contiguous()


def _forward(pred, gt_packed, cfg: ImageLossConfig, partials=True, coeffs=False, loss_map=False, total=False):
    pred, gt_packed = _check(pred, gt_packed)
    h, w, cn = pred.shape
    dev = pred.device
    p = torch.empty((cfg.planes(cn), loss_tiles(h, w)), dtype=torch.float32, device=dev) if partials else None
    co = torch.empty((3, 3, h, w), dtype=torch.float32, device=dev) if coeffs else None
    lm = torch.zeros((h, w, cn), dtype=torch.float32, device=dev) if loss_map else None
    tot = torch.empty(1, dtype=torch.float32, device=dev) if total else None
    ctx = Context.get(dev)
    s = cfg.struct()
    _lib.check(ctx.lib.vs_image_loss_forward(ctx.handle, _ptr(pred), cn, _ptr(gt_packed), w, h, C.byref(s), _ptr(p),
                                             _ptr(co), _ptr(lm), _ptr(tot)))
    return p, co, lm, tot


def image_loss(pred: torch.Tensor, gt_packed: torch.Tensor, cfg: ImageLossConfig) -> torch.Tensor:
    """The loss total [1]: the sum of the weighted tile partials."""
    return _forward(pred, gt_packed, cfg, total=True)[3]


def image_loss_partials(pred: torch.Tensor, gt_packed: torch.Tensor, cfg: ImageLossConfig) -> torch.Tensor:
    """Weighted per-16x16-tile sums [planes, tiles] (rows r, g, b[, alpha])."""
    return _forward(pred, gt_packed, cfg)[0]


def image_loss_eval(pred: torch.Tensor, gt_packed: torch.Tensor, cfg: ImageLossConfig) -> torch.Tensor:
    """Forward-only per-pixel loss map [H,W,C] (alpha holds the alpha term when matching, else 0)."""
    return _forward(pred, gt_packed, cfg, partials=False, loss_map=True)[2]


def image_loss_forward_train(pred: torch.Tensor, gt_packed: torch.Tensor, cfg: ImageLossConfig):
    """(partials [planes, tiles], SSIM coefficients [3,3,H,W], total [1])."""
    p, co, _, tot = _forward(pred, gt_packed, cfg, coeffs=True, total=True)
    return p, co, tot


def image_loss_backward(pred: torch.Tensor, gt_packed: torch.Tensor, dl_dpartials: torch.Tensor,
                        cfg: ImageLossConfig, coeffs: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dL/dpred [H,W,C] from the gradient of the total ([1]) or of each partial
    ([planes, tiles]); without `coeffs` the SSIM coefficients are recomputed."""
    pred, gt_packed = _check(pred, gt_packed)
    h, w, cn = pred.shape
    dl = dl_dpartials.contiguous().float()
    if dl.numel() not in (1, cfg.planes(cn) * loss_tiles(h, w)):
        raise ValueError("dl_dpartials must be [1] or [planes, tiles]")
    out = torch.empty_like(pred)
    ctx = Context.get(pred.device)
    s = cfg.struct()
    _lib.check(ctx.lib.vs_image_loss_backward(ctx.handle, _ptr(pred), cn, _ptr(gt_packed), w, h, C.byref(s), _ptr(dl),
                                              dl.numel(), _ptr(coeffs.contiguous() if coeffs is not None else None),
                                              _ptr(out)))
    return out
