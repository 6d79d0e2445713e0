"""ctypes wrapper of oracle/liboracle.so.

TEST INFRASTRUCTURE ONLY: a CPU restatement of the reference render path used
as the parity checker by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  The product (vauss_amd) never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
# ORACLE_LIB points the tests at another build of the oracle (a deliberately
# mutated copy, to check that the tests catch the mistake).
LIB_PATH = Path(os.environ.get("ORACLE_LIB", HERE / "liboracle.so"))

FLAG_BWD_INFO, FLAG_GEOMETRY, FLAG_SMOOTH_CUTOFF, FLAG_BRUTE_FORCE, FLAG_MIP = 1, 2, 4, 8, 16
FLAG_SURFEL, FLAG_SURFACE = 32, 64
(F_INTERSECT_COUNTS, F_MAX_RADIUS, F_OPACITIES, F_GLOBAL_FROM_COMPACT, F_DEPTHS, F_PROJECTED, F_AUX, F_ISECT_TILE,
 F_ISECT_GID, F_TILE_OFFSETS, F_TILE_OFFSETS_SHRUNK, F_VISIBLE, F_OUT_IMG, F_SURFEL_AUX) = range(14)
SURFEL_GRADS = 17


class OrCamera(C.Structure):
    """Same layout as vs_camera (include/vsplat.h)."""
    _fields_ = [("model", C.c_int32), ("fx", C.c_float), ("fy", C.c_float), ("cx", C.c_float), ("cy", C.c_float),
                ("kb4", C.c_float * 4), ("viewmat", C.c_float * 12), ("cam_pos", C.c_float * 3),
                ("half_max_render_fov", C.c_float), ("lim_pos_x", C.c_float), ("lim_pos_y", C.c_float),
                ("lim_neg_x", C.c_float), ("lim_neg_y", C.c_float), ("lim_r", C.c_float), ("dist", C.c_float * 8)]


class OrAdam(C.Structure):
    """Same layout as vs_adam_step (include/vsplat.h)."""
    _fields_ = [("beta1", C.c_float), ("beta2", C.c_float), ("inv1", C.c_float), ("inv2", C.c_float),
                ("epsilon", C.c_float), ("lr_opac", C.c_float), ("opac_reg", C.c_float), ("round_seed", C.c_uint32)]


class OrLossCfg(C.Structure):
    """Same layout as vs_loss_cfg (include/vsplat.h)."""
    _fields_ = [("l1_weight", C.c_float), ("ssim_weight", C.c_float), ("alpha_weight", C.c_float),
                ("composite", C.c_int32), ("bg", C.c_float * 3), ("mask", C.c_int32)]


def loss_cfg(l1_weight=0.8, ssim_weight=-0.2, alpha_weight=0.0, composite_bg=None, mask=False) -> OrLossCfg:
    bg = composite_bg if composite_bg is not None else (0.0, 0.0, 0.0)
    return OrLossCfg(l1_weight, ssim_weight, alpha_weight, 1 if composite_bg is not None else 0,
                     (C.c_float * 3)(*bg), 1 if mask else 0)


class OrFwdInfo(C.Structure):
    _fields_ = [("num_splats", C.c_uint32), ("num_visible", C.c_uint32), ("num_intersections", C.c_uint32),
                ("num_tiles", C.c_uint32), ("tile_bw", C.c_uint32), ("tile_bh", C.c_uint32),
                ("img_w", C.c_uint32), ("img_h", C.c_uint32), ("out_channels", C.c_uint32),
                ("num_evaluations", C.c_uint64)]


_LIB = None
_F = C.POINTER(C.c_float)
_U = C.POINTER(C.c_uint32)


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def load() -> C.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        build()
    lib = C.CDLL(os.fspath(LIB_PATH))
    lib.or_render_forward.restype = C.c_int
    lib.or_render_forward.argtypes = [C.POINTER(OrCamera), C.c_uint32, C.c_uint32, _F, _F, C.c_uint32, _F, C.c_uint32,
                                      C.c_float, _F, _F, _F, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
    lib.or_fwd_get_info.argtypes = [C.c_void_p, C.POINTER(OrFwdInfo)]
    lib.or_fwd_get.restype = C.c_int
    lib.or_fwd_get.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
    lib.or_fwd_free.argtypes = [C.c_void_p]
    lib.or_render_backward.restype = C.c_int
    lib.or_render_backward.argtypes = [C.c_void_p, _F, C.c_int, _F, _F, _F, _F, _F]
    lib.or_project_backward.restype = C.c_int
    lib.or_project_backward.argtypes = [C.c_void_p, _F, C.c_int, _F, _F, _F, _F]
    lib.or_neural_backward.restype = C.c_int
    lib.or_neural_backward.argtypes = [C.c_void_p, _F, C.c_int, _F, _F, _F, _F, C.POINTER(C.c_double)]
    lib.or_sincosf_n.argtypes = [_F, _F, _F, C.c_uint64]
    lib.or_tanhf_n.argtypes = [_F, _F, C.c_uint64]
    lib.or_neural_color.argtypes = [_F, _F, _F, C.c_uint32, _F]
    lib.or_pose_backward.restype = C.c_int
    lib.or_pose_backward.argtypes = [C.c_void_p, _F, C.c_int, C.POINTER(C.c_double), _F]
    lib.or_project_update.restype = C.c_int
    lib.or_project_update.argtypes = [C.c_void_p, _F, _F, _F, _U, _F, _U, C.POINTER(OrAdam), _F, _F, _F, C.c_int]
    lib.or_image_loss_forward.restype = C.c_int
    lib.or_image_loss_forward.argtypes = [_F, C.c_uint32, _U, C.c_uint32, C.c_uint32, C.POINTER(OrLossCfg), _F, _F, _F]
    lib.or_image_loss_backward.restype = C.c_int
    lib.or_image_loss_backward.argtypes = [_F, C.c_uint32, _U, C.c_uint32, C.c_uint32, C.POINTER(OrLossCfg), _F,
                                           C.c_int, _F, _F]
    lib.or_geo_encode.restype = C.c_uint32
    lib.or_geo_encode.argtypes = [C.c_float, C.c_float, C.c_float]
    lib.or_geo_decode.argtypes = [C.c_uint32, C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_float)]
    lib.or_geo_pack.restype = C.c_uint32
    lib.or_geo_pack.argtypes = [C.c_float, C.c_float, C.c_float, C.c_float, C.c_float]
    lib.or_mix_hash.restype = C.c_uint32
    lib.or_mix_hash.argtypes = [C.c_uint32, C.c_uint32]
    lib.or_adam_packed.argtypes = [C.POINTER(C.c_float), C.POINTER(C.c_uint32), C.c_uint32, C.c_float, C.c_float,
                                   C.POINTER(OrAdam), C.c_uint32]
    lib.or_f32_to_f16.restype = C.c_uint16
    lib.or_f32_to_f16.argtypes = [C.c_float]
    lib.or_f16_to_f32.restype = C.c_float
    lib.or_f16_to_f32.argtypes = [C.c_uint16]
    lib.or_stochastic_half.restype = C.c_float
    lib.or_stochastic_half.argtypes = [C.c_float, C.c_uint32, C.c_uint32]
    lib.or_block8_encode.argtypes = [_F, C.c_uint64, _U, _F]
    lib.or_block8_decode.argtypes = [_U, _F, C.c_uint64, _F]
    lib.or_block8_zero_rows.argtypes = [_U, C.c_uint64, _U, C.c_uint32, C.c_uint32]
    lib.or_sh_step.restype = C.c_int
    lib.or_sh_step.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, _F, _U, _F, _F, _U, _F, _F, C.c_float, C.c_float,
                               C.c_float, C.c_float, C.c_float, C.c_float, C.c_uint32, C.c_int]
    lib.or_radix_argsort_u32.argtypes = [_U, _U, C.c_uint32, C.c_uint32, C.c_uint32, _U, _U]
    lib.or_prefix_sum_u32.argtypes = [_U, _U, C.c_uint32]
    for name in ("or_expf", "or_logf"):
        getattr(lib, name).restype = C.c_float
        getattr(lib, name).argtypes = [C.c_float]
    lib.or_atan2f.restype = C.c_float
    lib.or_atan2f.argtypes = [C.c_float, C.c_float]
    lib.or_expf_n.argtypes = [_F, _F, C.c_uint64]
    lib.or_exp2n_n.argtypes = [_F, _F, C.c_uint64]
    lib.or_set_comp_exp2_table.argtypes = [C.c_void_p, C.c_uint32, C.c_uint64]
    lib.or_logf_n.argtypes = [_F, _F, C.c_uint64]
    lib.or_atan2f_n.argtypes = [_F, _F, _F, C.c_uint64]
    lib.or_sh_basis.argtypes = [C.c_uint32, _F, _F]
    kb = C.POINTER(C.c_float)
    for name in ("or_rt8_radial", "or_rt8_undistort_radius", "or_rt8_undistort_corner_radius"):
        getattr(lib, name).restype = C.c_double
        getattr(lib, name).argtypes = [C.c_double, kb]
    lib.or_clamp_limits.argtypes = [C.c_int, C.c_uint32, C.c_uint32, C.c_float, C.c_float, C.c_float, C.c_float, kb, kb]
    for name, args in (("or_fov_to_focal", [C.c_double, C.c_uint32, C.c_int, kb]),
                       ("or_focal_to_fov", [C.c_double, C.c_uint32, C.c_int, kb]),
                       ("or_max_render_theta", [C.c_int, kb]), ("or_kb4_d", [C.c_double, kb]),
                       ("or_kb4_dd_dtheta", [C.c_double, kb]), ("or_kb4_invert_d", [C.c_double, kb])):
        getattr(lib, name).restype = C.c_double
        getattr(lib, name).argtypes = args
    lib.or_max_threads.restype = C.c_int
    _LIB = lib
    return lib


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _up(a: np.ndarray):
    return a.ctypes.data_as(_U)


def camera_struct(cam) -> OrCamera:
    """Copy a vs_camera (or anything with the same fields) into an OrCamera."""
    out = OrCamera()
    C.memmove(C.byref(out), C.byref(cam), C.sizeof(OrCamera))
    return out


@dataclass
class OracleForward:
    handle: C.c_void_p
    info: OrFwdInfo
    num_splats: int
    sh_degree: int
    flags: int
    neural: bool = False

    @property
    def coeffs_per_row(self) -> int:
        return 4 if self.neural else (self.sh_degree + 1) ** 2

    def _neural(self, vc, vt, vs, threads):
        """Neural rows into vs [N,4,3], the view-direction term into vt; (v_decoder, v_coeffs_sq).
        The decoder gradient's sums of |products| land in self.decoder_abs [816]."""
        sq = np.zeros(self.num_splats, np.float32)
        dec = np.zeros(816, np.float32)
        dabs = np.zeros(816, np.float64)
        rc = load().or_neural_backward(self.handle, _fp(vc), threads, _fp(vt), _fp(vs), _fp(sq), _fp(dec),
                                       dabs.ctypes.data_as(C.POINTER(C.c_double)))
        if rc != 0:
            raise RuntimeError(f"oracle neural backward failed ({rc})")
        self.decoder_abs = dabs
        return dec, sq

    def get(self, field: int) -> np.ndarray:
        inf = self.info
        n, v, i, t = inf.num_splats, inf.num_visible, inf.num_intersections, inf.num_tiles
        shapes = {F_INTERSECT_COUNTS: ((n,), np.uint32), F_MAX_RADIUS: ((n,), np.float32),
                  F_OPACITIES: ((n,), np.float32), F_GLOBAL_FROM_COMPACT: ((v,), np.uint32),
                  F_DEPTHS: ((v,), np.float32), F_PROJECTED: ((v, 9), np.float32), F_AUX: ((v, 4), np.float32),
                  F_ISECT_TILE: ((i,), np.uint32), F_ISECT_GID: ((i,), np.uint32),
                  F_TILE_OFFSETS: ((inf.tile_bh, inf.tile_bw, 2), np.uint32),
                  F_TILE_OFFSETS_SHRUNK: ((inf.tile_bh, inf.tile_bw, 2), np.uint32),
                  F_VISIBLE: ((n,), np.float32), F_SURFEL_AUX: ((v, 14), np.float32)}
        if field == F_OUT_IMG:
            if self.flags & FLAG_BWD_INFO:
                shape, dt = (inf.img_h, inf.img_w, inf.out_channels), np.float32
            else:
                shape, dt = (inf.img_h, inf.img_w), np.uint32
        else:
            shape, dt = shapes[field]
        if field == F_AUX and (not (self.flags & FLAG_GEOMETRY) or self.flags & FLAG_SURFEL):
            return np.zeros((0, 4), np.float32)
        if field == F_SURFEL_AUX and not (self.flags & FLAG_SURFEL):
            return np.zeros((0, 14), np.float32)
        out = np.empty(shape, dt)
        if out.size:
            rc = load().or_fwd_get(self.handle, field, out.ctypes.data_as(C.c_void_p))
            assert rc == 0
        return out

    def backward(self, v_out: np.ndarray, threads: int = 0):
        n = self.num_splats
        k = self.coeffs_per_row
        v_out = np.ascontiguousarray(v_out, np.float32)
        vc = np.zeros((n, SURFEL_GRADS if self.flags & FLAG_SURFEL else 10), np.float32)
        vt = np.zeros((n, 10), np.float32)
        vs = np.zeros((n, k, 3), np.float32)
        vo = np.zeros(n, np.float32)
        vr = np.zeros(n, np.float32)
        rc = load().or_render_backward(self.handle, _fp(v_out), threads, _fp(vc), _fp(vt), _fp(vs), _fp(vo), _fp(vr))
        if rc != 0:
            raise RuntimeError(f"oracle backward failed ({rc})")
        out = {"v_combined": vc, "v_transforms": vt, "v_sh": vs, "v_raw_opac": vo, "v_refine": vr}
        if self.neural:
            out["v_decoder"], out["v_coeffs_sq"] = self._neural(vc, vt, vs, threads)
        return out

    def project_update(self, v_combined, transforms, raw_opac, w_t, lr_scale, w_o, adam: "OrAdam", threads: int = 0):
        """project_update on copies of the host arrays; returns the stepped
        parameters and moments plus color_dir [N+1,6], v_refine, grad_sq."""
        n = self.num_splats
        vc = np.ascontiguousarray(v_combined, np.float32)
        t = np.array(transforms, np.float32, copy=True)
        o = np.array(raw_opac, np.float32, copy=True)
        wt = np.array(w_t, np.uint32, copy=True)
        wo = np.array(w_o, np.uint32, copy=True)
        lr = np.ascontiguousarray(lr_scale, np.float32)
        cd = np.zeros((n + 1, 6), np.float32)
        vr = np.zeros(n, np.float32)
        gs = np.zeros(n, np.float32)
        rc = load().or_project_update(self.handle, _fp(vc), _fp(t), _fp(o), _up(wt), _fp(lr), _up(wo), C.byref(adam),
                                      _fp(cd), _fp(vr), _fp(gs), threads)
        if rc != 0:
            raise RuntimeError(f"oracle project_update failed ({rc})")
        return {"transforms": t, "raw_opac": o, "w_t": wt, "w_o": wo, "color_dir": cd, "v_refine": vr, "grad_sq": gs}

    def project_backward(self, v_combined: np.ndarray, threads: int = 0):
        """The projection VJP alone (and the neural backward in neural mode),
        applied to the given v_combined [N,10]."""
        n = self.num_splats
        k = self.coeffs_per_row
        vc = np.ascontiguousarray(v_combined, np.float32)
        assert vc.shape == (n, SURFEL_GRADS if self.flags & FLAG_SURFEL else 10)
        vt = np.zeros((n, 10), np.float32)
        vs = np.zeros((n, k, 3), np.float32)
        vo = np.zeros(n, np.float32)
        vr = np.zeros(n, np.float32)
        rc = load().or_project_backward(self.handle, _fp(vc), threads, _fp(vt), _fp(vs), _fp(vo), _fp(vr))
        if rc != 0:
            raise RuntimeError(f"oracle projection backward failed ({rc})")
        out = {"v_transforms": vt, "v_sh": vs, "v_raw_opac": vo, "v_refine": vr}
        if self.neural:
            out["v_decoder"], out["v_coeffs_sq"] = self._neural(vc, vt, vs, threads)
        return out

    def pose_backward(self, v_combined: np.ndarray, threads: int = 0):
        """The camera gradient [dA (row-major 3x3), db] (f64 sum) and the per-splat rows [N,12]."""
        n = self.num_splats
        vc = np.ascontiguousarray(v_combined, np.float32)
        assert vc.shape == (n, 10)
        total = (C.c_double * 12)()
        rows = np.zeros((n, 12), np.float32)
        rc = load().or_pose_backward(self.handle, _fp(vc), threads, total, _fp(rows))
        if rc != 0:
            raise RuntimeError(f"oracle pose backward failed ({rc})")
        return np.array(total[:], np.float64), rows

    def __del__(self):
        try:
            if self.handle:
                load().or_fwd_free(self.handle)
                self.handle = None
        except Exception:
            pass


def render_forward(cam, img_size, transforms, sh_coeffs, raw_opacities, background=(0, 0, 0), flags=FLAG_BWD_INFO,
                   threads: int = 0, log_scale_offset: float = 0.0, min_scale=None, decoder=None,
                   neural_degree: int = 0) -> OracleForward:
    """`flags` may add FLAG_MIP (SplatRenderMode::Mip); `min_scale` [N] is the scale floor (None: none).
    With `decoder` [816] the colour is the neural appearance's: `sh_coeffs` holds [N,4,3] rows
    (base, latents, pad) and `neural_degree` (0..3) is the decoder's direction band."""
    lib = load()
    t = np.ascontiguousarray(transforms, np.float32)
    s = np.ascontiguousarray(sh_coeffs, np.float32)
    o = np.ascontiguousarray(raw_opacities, np.float32)
    n = t.shape[0]
    degree = int(round(np.sqrt(s.shape[1]))) - 1
    dec = None
    if decoder is not None:
        dec = np.ascontiguousarray(decoder, np.float32)
        if dec.shape != (816,) or s.shape[1:] != (4, 3):
            raise ValueError("neural mode takes a [816] decoder and [N,4,3] rows")
        degree = int(neural_degree)
    bg = np.asarray(background, np.float32)
    c = camera_struct(cam)
    h = C.c_void_p()
    ms = None if min_scale is None else np.ascontiguousarray(min_scale, np.float32)
    if ms is not None and ms.shape != (n,):
        raise ValueError("min_scale must hold one floor per splat")
    rc = lib.or_render_forward(C.byref(c), int(img_size[0]), int(img_size[1]), _fp(t), _fp(s), degree, _fp(o), n,
                               float(log_scale_offset), None if ms is None else _fp(ms),
                               None if dec is None else _fp(dec), _fp(bg), flags, threads, C.byref(h))
    if rc != 0:
        raise RuntimeError(f"oracle forward failed ({rc})")
    info = OrFwdInfo()
    lib.or_fwd_get_info(h, C.byref(info))
    return OracleForward(h, info, n, degree, flags, dec is not None)


def radix_argsort_u32(keys, vals, skip_bits, sorting_bits):
    k = np.ascontiguousarray(keys, np.uint32)
    v = np.ascontiguousarray(vals, np.uint32)
    ok, ov = np.empty_like(k), np.empty_like(v)
    if k.size:
        load().or_radix_argsort_u32(_up(k), _up(v), k.size, skip_bits, sorting_bits, _up(ok), _up(ov))
    return ok, ov


def prefix_sum_u32(x):
    a = np.ascontiguousarray(x, np.uint32)
    out = np.empty_like(a)
    if a.size:
        load().or_prefix_sum_u32(_up(a), _up(out), a.size)
    return out


def expf(x):
    a = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    load().or_expf_n(_fp(a), _fp(out), a.size)
    return out


_COMP_EXP2 = None   # the installed table; the library holds its pointer


def set_comp_exp2_table(tab, first_bits: int = 0x80000000):
    """Makes the compositing loops take G = 2^x from `tab` (float32, tab[i] for
    the f32 x whose bit pattern is first_bits + i) wherever it covers x, as the
    GPU kernels' exp2 instruction gives it; None restores exp2n everywhere."""
    global _COMP_EXP2
    lib = load()
    if tab is None:
        lib.or_set_comp_exp2_table(None, 0, 0)
        _COMP_EXP2 = None
        return
    a = np.ascontiguousarray(tab, np.float32)
    lib.or_set_comp_exp2_table(C.c_void_p(a.ctypes.data), int(first_bits), int(a.size))
    _COMP_EXP2 = a


def exp2n(x):
    """The compositing loops' default 2^x (or_math.h exp2n_c)."""
    a = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    load().or_exp2n_n(_fp(a), _fp(out), a.size)
    return out


def logf(x):
    a = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    load().or_logf_n(_fp(a), _fp(out), a.size)
    return out


def atan2f(y, x):
    a = np.ascontiguousarray(y, np.float32)
    b = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    load().or_atan2f_n(_fp(a), _fp(b), _fp(out), a.size)
    return out


def sincosf(x):
    a = np.ascontiguousarray(x, np.float32)
    s, c = np.empty_like(a), np.empty_like(a)
    load().or_sincosf_n(_fp(a), _fp(s), _fp(c), a.size)
    return s, c


def tanhf(x):
    a = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    load().or_tanhf_n(_fp(a), _fp(out), a.size)
    return out


def neural_color(row, decoder, direction, degree: int) -> np.ndarray:
    r = np.ascontiguousarray(row, np.float32)
    d = np.ascontiguousarray(decoder, np.float32)
    v = np.ascontiguousarray(direction, np.float32)
    out = np.zeros(3, np.float32)
    load().or_neural_color(_fp(r), _fp(d), _fp(v), degree, _fp(out))
    return out


def sh_basis(degree: int, v) -> np.ndarray:
    vv = np.ascontiguousarray(v, np.float32)
    out = np.zeros((degree + 1) ** 2, np.float32)
    load().or_sh_basis(degree, _fp(vv), _fp(out))
    return out


def kb4_array(k):
    return (C.c_float * 4)(*[float(v) for v in k])


MODEL_PINHOLE, MODEL_KB4, MODEL_RT8, MODEL_TPF = 0, 1, 2, 3


def _params12(k, dist):
    return (C.c_float * 12)(*([float(v) for v in k] + [float(v) for v in dist] + [0.0] * (8 - len(dist))))


def fov_to_focal(fov, pixels, model=0, k=(0, 0, 0, 0), dist=()):
    """`k`: KB4 k1..k4 (KB4, thin-prism); `dist`: RT8 k1..k6, p1, p2 or thin-prism p1, p2, sx1, sy1."""
    return load().or_fov_to_focal(fov, pixels, model, _params12(k, dist))


def focal_to_fov(focal, pixels, model=0, k=(0, 0, 0, 0), dist=()):
    return load().or_focal_to_fov(focal, pixels, model, _params12(k, dist))


def max_render_theta(model=0, k=(0, 0, 0, 0), dist=()):
    return load().or_max_render_theta(model, _params12(k, dist))


def rt8_radial(r, dist):
    return load().or_rt8_radial(r, (C.c_float * 8)(*dist))


def rt8_undistort_corner_radius(r_d, dist):
    """None when r radial(r) never reaches r_d below r = 16."""
    v = load().or_rt8_undistort_corner_radius(r_d, (C.c_float * 8)(*dist))
    return None if v < 0 else v


def clamp_limits(model, img, fx, fy, cx, cy, dist=(0,) * 8):
    """(lim_pos_x, lim_pos_y, lim_neg_x, lim_neg_y, lim_r)."""
    out = (C.c_float * 5)()
    load().or_clamp_limits(model, img[0], img[1], fx, fy, cx, cy, (C.c_float * 8)(*dist), out)
    return tuple(out)


def kb4_d(theta, k):
    return load().or_kb4_d(theta, kb4_array(k))


def kb4_dd_dtheta(theta, k):
    return load().or_kb4_dd_dtheta(theta, kb4_array(k))


def kb4_invert_d(target, k):
    return load().or_kb4_invert_d(target, kb4_array(k))


def max_threads() -> int:
    return load().or_max_threads()


def geo_encode(m: float, v: float, epsilon: float) -> int:
    return int(load().or_geo_encode(m, v, epsilon))


def geo_pack(m: float, v: float, epsilon: float, round_l: float, round_u: float) -> int:
    return int(load().or_geo_pack(m, v, epsilon, round_l, round_u))


def geo_decode(word: int, epsilon: float):
    m, v = C.c_float(), C.c_float()
    load().or_geo_decode(word & 0xFFFFFFFF, epsilon, C.byref(m), C.byref(v))
    return m.value, v.value


def mix_hash(index: int, step: int) -> int:
    return int(load().or_mix_hash(index & 0xFFFFFFFF, step & 0xFFFFFFFF))


def adam_packed(param: float, word: int, index: int, g: float, lr: float, adam: OrAdam, seed: int):
    p, w = C.c_float(param), C.c_uint32(word & 0xFFFFFFFF)
    load().or_adam_packed(C.byref(p), C.byref(w), index & 0xFFFFFFFF, g, lr, C.byref(adam), seed & 0xFFFFFFFF)
    return p.value, w.value


def image_loss_forward(pred: np.ndarray, gt_packed: np.ndarray, cfg: OrLossCfg):
    """(partials [planes, tiles], coeffs [3,3,H,W], loss_map [H,W,C])."""
    pred = np.ascontiguousarray(pred, np.float32)
    gt = np.ascontiguousarray(gt_packed, np.uint32)
    h, w, cn = pred.shape
    tiles = ((w + 15) // 16) * ((h + 15) // 16)
    planes = 4 if (cfg.alpha_weight > 0 and cn == 4) else 3
    partials = np.zeros((planes, tiles), np.float32)
    coeffs = np.zeros((3, 3, h, w), np.float32)
    lmap = np.zeros((h, w, cn), np.float32)
    rc = load().or_image_loss_forward(_fp(pred), cn, _up(gt), w, h, C.byref(cfg), _fp(partials), _fp(coeffs), _fp(lmap))
    if rc != 0:
        raise RuntimeError(f"oracle image loss failed ({rc})")
    return partials, coeffs, lmap


def image_loss_backward(pred: np.ndarray, gt_packed: np.ndarray, cfg: OrLossCfg, dl_dpartials: np.ndarray,
                        coeffs: np.ndarray) -> np.ndarray:
    pred = np.ascontiguousarray(pred, np.float32)
    gt = np.ascontiguousarray(gt_packed, np.uint32)
    dl = np.ascontiguousarray(dl_dpartials, np.float32)
    co = np.ascontiguousarray(coeffs, np.float32)
    h, w, cn = pred.shape
    out = np.zeros_like(pred)
    rc = load().or_image_loss_backward(_fp(pred), cn, _up(gt), w, h, C.byref(cfg), _fp(dl), 1 if dl.size == 1 else 0,
                                       _fp(co), _fp(out))
    if rc != 0:
        raise RuntimeError(f"oracle image loss backward failed ({rc})")
    return out


def f32_to_f16_bits(x: float) -> int:
    return int(load().or_f32_to_f16(x))


def f16_bits_to_f32(h: int) -> float:
    return float(load().or_f16_to_f32(h & 0xFFFF))


def stochastic_half(value: float, index: int, step: int) -> float:
    return float(load().or_stochastic_half(value, index & 0xFFFFFFFF, step & 0xFFFFFFFF))


def block8_encode(values: np.ndarray):
    """(codes [ceil(n/128)*32] u32, scales [ceil(n/128)] f32)."""
    v = np.ascontiguousarray(values, np.float32).reshape(-1)
    blocks = (v.size + 127) // 128
    codes = np.zeros(blocks * 32, np.uint32)
    scales = np.zeros(blocks, np.float32)
    load().or_block8_encode(_fp(v), v.size, _up(codes), _fp(scales))
    return codes, scales


def block8_decode(codes: np.ndarray, scales: np.ndarray, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    load().or_block8_decode(_up(np.ascontiguousarray(codes, np.uint32)), _fp(np.ascontiguousarray(scales, np.float32)),
                            n, _fp(out))
    return out


def block8_zero_rows(codes: np.ndarray, n: int, rows: np.ndarray, row_width: int) -> np.ndarray:
    out = np.ascontiguousarray(codes, np.uint32).copy()
    r = np.ascontiguousarray(rows, np.uint32)
    load().or_block8_zero_rows(_up(out), n, _up(r), r.size, row_width)
    return out


def sh_step(sh_half: np.ndarray, color_dir: np.ndarray, grad_rows: np.ndarray, grad_sq: np.ndarray,
            variance: np.ndarray, codes: np.ndarray, scales: np.ndarray, lr_scale: np.ndarray, *, beta1: float,
            beta2: float, inv1: float, inv2: float, epsilon: float, lr: float, round_seed: int, first: bool):
    """One SH step on copies: returns (sh [N,K,3] f16, variance, codes, scales)."""
    sh = np.ascontiguousarray(sh_half, np.float16).copy()
    n, k = sh.shape[0], sh.shape[1]
    degree = int(round(k ** 0.5)) - 1
    var = np.ascontiguousarray(variance, np.float32).copy()
    co = np.ascontiguousarray(codes, np.uint32).copy()
    sc = np.ascontiguousarray(scales, np.float32).copy()
    cd = np.ascontiguousarray(color_dir, np.float32)
    gr = np.ascontiguousarray(grad_rows, np.uint32)
    gs = np.ascontiguousarray(grad_sq, np.float32)
    ls = np.ascontiguousarray(lr_scale, np.float32)
    rc = load().or_sh_step(sh.ctypes.data_as(C.c_void_p), n, degree, _fp(cd), _up(gr), _fp(gs), _fp(var), _up(co),
                           _fp(sc), _fp(ls), beta1, beta2, inv1, inv2, epsilon, lr, round_seed & 0xFFFFFFFF,
                           1 if first else 0)
    if rc != 0:
        raise RuntimeError(f"oracle SH step failed ({rc})")
    return sh, var, co, sc
