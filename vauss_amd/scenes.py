"""Seeded synthetic splat clouds and cameras for the five benchmark workloads.

Uniforms come from SplitMix64 (as crates/splat-train-render/src/tests/mod.rs:
168-186 generates its test scenes), normals from Box-Muller.  SH DC
coefficients are stored directly as U(0,1) values, the convention of the
reference's test scenes (tests/mod.rs:212,259-270); higher bands ~N(0, 0.05).

Workloads (W x H, 16x16 tiles):
  c1  10k splats, SH0, 256x256, fx=fy=256, identity pose
  c2  200k splats, SH3, 1920x1080, fx=fy=1600, identity pose
  c3  1M splats, SH3, 1920x1080, fx=fy=1600, 8 poses on a radius-6 orbit around the origin
  c4  3M splats, SH3, heavy-tailed scales, 2560x1440, fx=fy=2000
  c5  2M splats, SH3, KB4 fisheye f=600 1920x1920, circular mask r=940
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .camera import Camera, KannalaBrandt4, PINHOLE, focal_to_fov, look_at_rotation

MASK64 = (1 << 64) - 1
GOLDEN = np.uint64(0x9E3779B97F4A7C15)
SEED_BASE = 0xB5EED000


class SplitMix64:
    """Vectorised SplitMix64 (the generator of tests/mod.rs:168-186)."""

    def __init__(self, seed: int):
        self.state = np.uint64(seed & MASK64)

    def next_u64(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            k = np.arange(1, n + 1, dtype=np.uint64)
            z = self.state + k * GOLDEN
            self.state = self.state + np.uint64(n) * GOLDEN
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            z = z ^ (z >> np.uint64(31))
        return z

    def unit(self, n: int) -> np.ndarray:
        """(z as f64 / u64::MAX as f64) as f32, tests/mod.rs:180."""
        return (self.next_u64(n).astype(np.float64) / float(MASK64)).astype(np.float32)

    def uniform(self, n: int, lo: float, hi: float) -> np.ndarray:
        lo32, hi32 = np.float32(lo), np.float32(hi)
        return (lo32 + self.unit(n) * (hi32 - lo32)).astype(np.float32)

    def normal(self, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        m = (n + 1) // 2
        # u1 in (0, 1] from the top 53 bits, so log(u1) is always finite
        u1 = ((self.next_u64(m) >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
        u2 = self.unit(m).astype(np.float64)
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
        return (mean + std * z).astype(np.float32)


@dataclass
class Scene:
    transforms: np.ndarray      # [N,10] mean, quat (w,x,y,z), log-scale
    sh_coeffs: np.ndarray       # [N,K,3]
    raw_opacities: np.ndarray   # [N]

    @property
    def num_splats(self) -> int:
        return self.transforms.shape[0]

    @property
    def sh_degree(self) -> int:
        return int(round(math.sqrt(self.sh_coeffs.shape[1]))) - 1

    def concat(self, other: "Scene") -> "Scene":
        return Scene(np.concatenate([self.transforms, other.transforms]),
                     np.concatenate([self.sh_coeffs, other.sh_coeffs]),
                     np.concatenate([self.raw_opacities, other.raw_opacities]))


@dataclass
class Workload:
    name: str
    scene: Scene
    cameras: list
    img_size: tuple
    mask_radius: float = 0.0
    mask_center: tuple = (0.0, 0.0)
    extra: dict = field(default_factory=dict)


def _random_quats(rng: SplitMix64, n: int) -> np.ndarray:
    q = rng.normal(4 * n).reshape(n, 4).astype(np.float64)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    return q.astype(np.float32)


def _sh(rng: SplitMix64, n: int, degree: int) -> np.ndarray:
    k = (degree + 1) ** 2
    sh = np.empty((n, k, 3), np.float32)
    sh[:, 0, :] = rng.unit(3 * n).reshape(n, 3)
    if k > 1:
        sh[:, 1:, :] = rng.normal(3 * n * (k - 1), 0.0, 0.05).reshape(n, k - 1, 3)
    return sh


def _pack(means, quats, log_scales) -> np.ndarray:
    return np.ascontiguousarray(np.concatenate([means, quats, log_scales], axis=1).astype(np.float32))


def scene_c1(n: int = 10_000, seed: int = SEED_BASE + 1) -> Scene:
    rng = SplitMix64(seed)
    means = np.stack([rng.uniform(n, -1, 1), rng.uniform(n, -1, 1), rng.uniform(n, 2, 6)], axis=1)
    log_scales = rng.normal(3 * n, -4.0, 0.5).reshape(n, 3)
    quats = _random_quats(rng, n)
    raw = rng.normal(n, 0.0, 1.0)
    sh = _sh(rng, n, 0)
    return Scene(_pack(means, quats, log_scales), sh, raw)


def _scene_sh3(rng, n, mean_std, z_shift, z_lo, z_hi, ls_mean, ls_std, op_mean, op_std) -> Scene:
    means = rng.normal(3 * n, 0.0, mean_std).reshape(n, 3)
    if z_shift is not None:
        means[:, 2] = np.clip(means[:, 2] + np.float32(z_shift), z_lo, z_hi)
    log_scales = rng.normal(3 * n, ls_mean, ls_std).reshape(n, 3)
    quats = _random_quats(rng, n)
    raw = rng.normal(n, op_mean, op_std)
    sh = _sh(rng, n, 3)
    return Scene(_pack(means, quats, log_scales), sh, raw)


def scene_c2(n: int = 200_000, seed: int = SEED_BASE + 2) -> Scene:
    return _scene_sh3(SplitMix64(seed), n, 2.0, 7.5, 3.0, 12.0, -4.5, 0.7, 0.0, 1.5)


def scene_c3(n: int = 1_000_000, seed: int = SEED_BASE + 3) -> Scene:
    # Same distributions as c2, centred on the origin the orbit cameras look at.
    return _scene_sh3(SplitMix64(seed), n, 2.0, None, 0, 0, -4.5, 0.7, 0.0, 1.5)


def scene_c4(n: int = 3_000_000, seed: int = SEED_BASE + 4) -> Scene:
    return _scene_sh3(SplitMix64(seed), n, 1.5, 6.0, 2.0, 10.0, -3.0, 1.0, 1.0, 1.0)


def scene_c5(n: int = 2_000_000, seed: int = SEED_BASE + 5) -> Scene:
    rng = SplitMix64(seed)
    d = rng.normal(3 * n).reshape(n, 3).astype(np.float64)
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    r = rng.uniform(n, 3.0, 8.0).astype(np.float64)
    means = (d * r[:, None]).astype(np.float32)
    log_scales = rng.normal(3 * n, -4.5, 0.7).reshape(n, 3)
    quats = _random_quats(rng, n)
    raw = rng.normal(n, 0.0, 1.5)
    sh = _sh(rng, n, 3)
    return Scene(_pack(means, quats, log_scales), sh, raw)


def orbit_cameras(count: int = 8, radius: float = 6.0, seed: int = SEED_BASE + 30, fx: float = 1600.0,
                  img_size=(1920, 1080)) -> list:
    """`count` OpenCV pinhole cameras on a radius-`radius` orbit looking at the
    origin: azimuth 2 pi k / count + U(-0.2, 0.2), elevation U(-15, 15) deg."""
    rng = SplitMix64(seed)
    jit = rng.uniform(count, -0.2, 0.2).astype(np.float64)
    elev = np.deg2rad(rng.uniform(count, -15.0, 15.0).astype(np.float64))
    cams = []
    for k in range(count):
        az = 2 * math.pi * k / count + jit[k]
        pos = radius * np.array([math.cos(elev[k]) * math.sin(az), -math.sin(elev[k]), -math.cos(elev[k]) * math.cos(az)])
        rot = look_at_rotation(pos)
        cams.append(Camera.from_focal(fx, fx, img_size, position=tuple(float(v) for v in pos), rotation=rot))
    return cams


def workload(name: str, n: int | None = None) -> Workload:
    """The named benchmark workload; `n` shrinks the cloud for parity tests."""
    if name == "c1":
        sz = (256, 256)
        return Workload("c1", scene_c1(n or 10_000), [Camera.from_focal(256.0, 256.0, sz)], sz)
    if name == "c2":
        sz = (1920, 1080)
        return Workload("c2", scene_c2(n or 200_000), [Camera.from_focal(1600.0, 1600.0, sz)], sz)
    if name == "c3":
        sz = (1920, 1080)
        return Workload("c3", scene_c3(n or 1_000_000), orbit_cameras(8, 6.0, fx=1600.0, img_size=sz), sz)
    if name == "c4":
        sz = (2560, 1440)
        return Workload("c4", scene_c4(n or 3_000_000), [Camera.from_focal(2000.0, 2000.0, sz)], sz)
    if name == "c5":
        sz = (1920, 1920)
        rng = SplitMix64(SEED_BASE + 50)
        k = rng.uniform(4, -0.05, 0.05)
        model = KannalaBrandt4(float(k[0]), float(k[1]), float(k[2]), float(k[3]))
        cam = Camera.from_focal(600.0, 600.0, sz, model=model)
        return Workload("c5", scene_c5(n or 2_000_000), [cam], sz, mask_radius=940.0, mask_center=(960.0, 960.0))
    raise KeyError(name)


def loss_target(img_size, seed: int = SEED_BASE + 99) -> np.ndarray:
    """Seeded U[0,1] target [H,W,3], quantised to k/255 like the reference's u8 ground truth."""
    w, h = img_size
    u = SplitMix64(seed).unit(w * h * 3).reshape(h, w, 3)
    return (np.round(u * 255.0) / 255.0).astype(np.float32)


def rng_scene(num_splats: int, mean_range: float, log_scale_range, opacity_range, seed: int) -> Scene:
    """The reference's deterministic test scene generator, tests/mod.rs:168-222:
    per splat 3 means, 4 (unnormalised) quaternion, 3 log-scales, 3 DC and one
    opacity draw, in that order."""
    rng = SplitMix64(seed)
    u = rng.unit(14 * num_splats).reshape(num_splats, 14)

    def uni(col, lo, hi):
        lo32, hi32 = np.float32(lo), np.float32(hi)
        return (lo32 + u[:, col] * (hi32 - lo32)).astype(np.float32)

    means = np.stack([uni(i, -mean_range, mean_range) for i in range(3)], axis=1)
    quats = np.stack([uni(3 + i, -1.0, 1.0) for i in range(4)], axis=1)
    ls = np.stack([uni(7 + i, log_scale_range[0], log_scale_range[1]) for i in range(3)], axis=1)
    dc = np.stack([uni(10 + i, 0.0, 1.0) for i in range(3)], axis=1)
    op = uni(13, opacity_range[0], opacity_range[1])
    return Scene(_pack(means, quats, ls), dc.reshape(num_splats, 1, 3).astype(np.float32), op)


def test_camera(img_size, fov: float = 0.5, position=(0.0, 0.0, -5.0), model=PINHOLE) -> Camera:
    """Camera::new(position, IDENTITY, fov, fov, (0.5, 0.5), model) as the reference's tests build it."""
    return Camera(fov, fov, (0.5, 0.5), tuple(position), (0.0, 0.0, 0.0, 1.0), model)
