"""Host camera, mirroring crates/splat-train-render/src/camera.rs:11-97.

A `Camera` holds a pose and field of view; `uniforms(img_size)` produces the
device projection uniforms through the library's `vs_camera_uniforms`, which
restates render.rs:478-503.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from . import _lib


@dataclass(frozen=True)
class KannalaBrandt4:
    """KannalaBrandt4Params (kernels/camera_model/kannala_brandt_4.rs:8-16)."""
    k1: float = 0.0
    k2: float = 0.0
    k3: float = 0.0
    k4: float = 0.0

    def as_array(self):
        return (C.c_float * 4)(self.k1, self.k2, self.k3, self.k4)


@dataclass(frozen=True)
class RadialTangential8:
    """RadialTangential8Params (kernels/camera_model/radial_tangential_8.rs:9-21):
    OpenCV's rational radial (k1..k6) plus tangential (p1, p2) model."""
    k1: float = 0.0
    k2: float = 0.0
    k3: float = 0.0
    k4: float = 0.0
    k5: float = 0.0
    k6: float = 0.0
    p1: float = 0.0
    p2: float = 0.0


@dataclass(frozen=True)
class ThinPrismFisheye:
    """ThinPrismFisheyeParams (kernels/camera_model/thin_prism_fisheye.rs:21-29):
    KB4 radial plus tangential (p1, p2) plus thin-prism (sx1, sy1)."""
    kb4: KannalaBrandt4 = KannalaBrandt4()
    p1: float = 0.0
    p2: float = 0.0
    sx1: float = 0.0
    sy1: float = 0.0


PINHOLE = None   # CameraModel::Pinhole


def _model_args(model):
    """(vs_camera_model, kb4[4], dist[8])."""
    zero4, zero8 = [0.0] * 4, [0.0] * 8
    if model is None:
        return _lib.CAMERA_PINHOLE, zero4, zero8
    if isinstance(model, KannalaBrandt4):
        return _lib.CAMERA_KB4, [model.k1, model.k2, model.k3, model.k4], zero8
    if isinstance(model, RadialTangential8):
        return _lib.CAMERA_RT8, zero4, [model.k1, model.k2, model.k3, model.k4, model.k5, model.k6, model.p1, model.p2]
    if isinstance(model, ThinPrismFisheye):
        k = model.kb4
        return _lib.CAMERA_TPF, [k.k1, k.k2, k.k3, k.k4], [model.p1, model.p2, model.sx1, model.sy1, 0.0, 0.0, 0.0, 0.0]
    raise ValueError(f"unsupported camera model {model!r}")


def _params(model):
    m, k, d = _model_args(model)
    return m, (C.c_float * 12)(*(k + d))


def fov_to_focal(fov: float, pixels: int, model=PINHOLE) -> float:
    """camera.rs:99-116."""
    m, k = _params(model)
    return _lib.load().vs_fov_to_focal(float(fov), int(pixels), m, k)


def focal_to_fov(focal: float, pixels: int, model=PINHOLE) -> float:
    """camera.rs:118-134."""
    m, k = _params(model)
    return _lib.load().vs_focal_to_fov(float(focal), int(pixels), m, k)


def max_render_theta(model=PINHOLE) -> float:
    """camera.rs:166-172."""
    m, k = _params(model)
    return _lib.load().vs_max_render_theta(m, k)


@dataclass
class Camera:
    """Camera of camera.rs:11-23 (without the exposure sub-pose affine).

    rotation is the camera-to-world quaternion in (x, y, z, w) order (glam);
    camera axes follow OpenCV (+x right, +y down, +z forward)."""
    fov_x: float
    fov_y: float
    center_uv: Sequence[float] = (0.5, 0.5)
    position: Sequence[float] = (0.0, 0.0, 0.0)
    rotation: Sequence[float] = (0.0, 0.0, 0.0, 1.0)
    model: object = field(default=PINHOLE)

    @classmethod
    def from_focal(cls, fx: float, fy: float, img_size, center=None, position=(0.0, 0.0, 0.0),
                   rotation=(0.0, 0.0, 0.0, 1.0), model=PINHOLE) -> "Camera":
        w, h = int(img_size[0]), int(img_size[1])
        cuv = (0.5, 0.5) if center is None else (center[0] / w, center[1] / h)
        return cls(focal_to_fov(fx, w, model), focal_to_fov(fy, h, model), cuv, tuple(position), tuple(rotation), model)

    def pose(self) -> _lib.VsPose:
        m, k, d = _model_args(self.model)
        p = _lib.VsPose()
        p.fov_x, p.fov_y = float(self.fov_x), float(self.fov_y)
        p.center_uv[:] = [float(v) for v in self.center_uv]
        p.position[:] = [float(v) for v in self.position]
        p.rotation[:] = [float(v) for v in self.rotation]
        p.model = m
        p.kb4[:] = list(k)
        p.dist[:] = list(d)
        return p

    def uniforms(self, img_size) -> _lib.VsCamera:
        out = _lib.VsCamera()
        pose = self.pose()
        _lib.check(_lib.load().vs_camera_uniforms(C.byref(pose), int(img_size[0]), int(img_size[1]), C.byref(out)))
        return out


def look_at_rotation(position, target=(0.0, 0.0, 0.0), down=(0.0, 1.0, 0.0)):
    """Camera-to-world quaternion (x, y, z, w) of an OpenCV camera at `position`
    looking at `target` with image +y along the world `down` direction."""
    p = np.asarray(position, np.float64)
    f = np.asarray(target, np.float64) - p
    f /= np.linalg.norm(f)
    x = np.cross(np.asarray(down, np.float64), f)
    x /= np.linalg.norm(x)
    y = np.cross(f, x)
    R = np.stack([x, y, f], axis=1)
    return quat_from_matrix(R)


def quat_from_matrix(R) -> tuple:
    """Rotation matrix -> unit quaternion (x, y, z, w) (Shepperd's method)."""
    R = np.asarray(R, np.float64)
    t = np.trace(R)
    if t > 0:
        s = math.sqrt(t + 1.0) * 2.0
        w, x, y, z = 0.25 * s, (R[2, 1] - R[1, 2]) / s, (R[0, 2] - R[2, 0]) / s, (R[1, 0] - R[0, 1]) / s
    elif R[0, 0] > R[1, 1] and R[0, 0] > R[2, 2]:
        s = math.sqrt(1.0 + R[0, 0] - R[1, 1] - R[2, 2]) * 2.0
        w, x, y, z = (R[2, 1] - R[1, 2]) / s, 0.25 * s, (R[0, 1] + R[1, 0]) / s, (R[0, 2] + R[2, 0]) / s
    elif R[1, 1] > R[2, 2]:
        s = math.sqrt(1.0 + R[1, 1] - R[0, 0] - R[2, 2]) * 2.0
        w, x, y, z = (R[0, 2] - R[2, 0]) / s, (R[0, 1] + R[1, 0]) / s, 0.25 * s, (R[1, 2] + R[2, 1]) / s
    else:
        s = math.sqrt(1.0 + R[2, 2] - R[0, 0] - R[1, 1]) * 2.0
        w, x, y, z = (R[1, 0] - R[0, 1]) / s, (R[0, 2] + R[2, 0]) / s, (R[1, 2] + R[2, 1]) / s, 0.25 * s
    q = np.array([x, y, z, w])
    q /= np.linalg.norm(q)
    return tuple(float(v) for v in q)
