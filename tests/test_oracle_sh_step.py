"""Pins the oracle's SH step (crates/splat-train/src/optim.rs:391-498,
quant.rs, quant_kernels.rs) on the CPU: its f16 conversions against numpy's
IEEE binary16, the stochastic f16 rounding against its defining properties,
the block-scaled 8-bit codec against the reference's own round-trip test
(quant.rs:213-249), and the step itself against a float64 restatement built
from the projection VJP's dense SH gradient (a different code path from the
step's Y_k(dir) colour rebuild).
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests._util import circle_mask, l1_cotangent_np
from vauss_amd import scenes


def test_f16_conversions_match_numpy():
    lib = po.load()
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 1 << 32, 200_000, dtype=np.uint64).astype(np.uint32)
    # bias towards the f16 range, its subnormals and the rounding ties
    near = (rng.integers(0x33000000, 0x47800000, 200_000, dtype=np.uint64).astype(np.uint32))
    ties = (near & np.uint32(0xFFFFE000)) | np.uint32(0x1000)
    edge = np.array([0, 0x80000000, 0x477FE000, 0x477FEFFF, 0x477FF000, 0x477FF001, 0x38800000, 0x387FFFFF,
                     0x33800000, 0x33000000, 0x33000001, 0x7F800000, 0xFF800000], np.uint32)
    x = np.concatenate([bits, near, ties, edge]).view(np.float32)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([lib.or_f32_to_f16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, want)
    allh = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    back = np.array([lib.or_f16_to_f32(int(h)) for h in allh], np.float32)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(back[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.isnan(back[np.isnan(ref)]).all()


def _neighbours(v: float):
    """The two f16 values adjacent to |v| (equal when |v| is one)."""
    a = abs(np.float32(v))
    h = np.float16(a)
    if np.float32(h) == a:
        return float(h), float(h)
    lo = h if np.float32(h) < a else np.nextafter(h, np.float16(0))
    hi = np.nextafter(lo, np.float16(np.inf))
    return float(lo), float(hi)


def test_stochastic_half_picks_an_adjacent_f16():
    rng = np.random.default_rng(2)
    vals = np.concatenate([rng.uniform(-3, 3, 3000), rng.uniform(-1e-5, 1e-5, 1000), 10.0 ** rng.uniform(-8, 4.8, 1000),
                           [0.0, -0.0, 65504.0, -65504.0, 1.0, 2.0 ** -24, 3 * 2.0 ** -24]]).astype(np.float32)
    for i, v in enumerate(vals):
        r = po.stochastic_half(float(v), i * 7919, 13)
        lo, hi = _neighbours(float(v))
        assert abs(r) in (lo, hi), (v, r, lo, hi)
        assert r == 0.0 or np.sign(r) == np.sign(v)
        assert float(np.float16(r)) == r                      # representable
    # values beyond the f16 range pass through
    assert po.stochastic_half(70000.0, 1, 1) == 70000.0
    assert np.isnan(po.stochastic_half(float("nan"), 1, 1))


@pytest.mark.parametrize("v", [0.1, -0.3337, 1.0001, 3.7e-6, 1234.567])
def test_stochastic_half_is_unbiased(v):
    """Over many indices the rounding picks the upper neighbour with
    probability (|v| - lo) / (hi - lo), so the mean is v."""
    lo, hi = _neighbours(v)
    p = (abs(np.float32(v)) - lo) / (hi - lo)
    n = 20000
    ups = sum(abs(po.stochastic_half(v, i, 5)) == hi for i in range(n))
    sigma = np.sqrt(n * p * (1 - p)) + 1
    assert abs(ups - n * p) <= 5 * sigma, (ups, n * p)


def test_block8_round_trip_like_the_reference():
    """quant.rs:213-249: three blocks + 7 values; an outlier block does not
    disturb its neighbours, zeros decode to exactly zero."""
    values = np.zeros(3 * 128 + 7, np.float32)
    values[:128] = (np.arange(128, dtype=np.float32) - 64.0) * 1e-7
    values[128] = 100.0
    values[129] = -100.0
    values[-1] = 0.5
    codes, scales = po.block8_encode(values)
    assert codes.size == 4 * 32 and scales.size == 4
    dec = po.block8_decode(codes, scales, values.size)
    for b in range(0, values.size, 128):
        exp = values[b:b + 128]
        mx = np.abs(exp).max()
        got = dec[b:b + 128]
        assert np.isfinite(got).all()
        assert (np.abs(exp - got) <= mx / 254.0 + mx * 1e-6).all()
        assert (got[exp == 0.0] == 0.0).all()


def test_block8_codes_scale_and_idempotence():
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(1000) * 10.0 ** rng.uniform(-6, 2, 1000)).astype(np.float32)
    codes, scales = po.block8_encode(v)
    for b in range(scales.size):
        blk = np.concatenate([v[b * 128:(b + 1) * 128], np.zeros(max(0, (b + 1) * 128 - v.size), np.float32)])
        assert scales[b] == np.float32(np.abs(blk).max()) / np.float32(127.0)
        c = (codes[b * 32:(b + 1) * 32, None] >> (8 * np.arange(4, dtype=np.uint32))) & 255
        assert c.min() >= 1 and c.max() <= 255                 # clamp to +-127 around the bias
        assert 1 in c or 255 in c                              # the absmax value takes the end code
    # decode then encode gives back the same codes
    c2, s2 = po.block8_encode(po.block8_decode(codes, scales, v.size))
    np.testing.assert_array_equal(c2, codes)
    np.testing.assert_allclose(s2, scales, rtol=2e-7)


def test_block8_zero_rows():
    rng = np.random.default_rng(4)
    v = rng.uniform(-1, 1, 27 * 40).astype(np.float32)         # SH2 rows of 27 values share words
    codes, scales = po.block8_encode(v)
    rows = np.array([0, 3, 39], np.uint32)
    z = po.block8_zero_rows(codes, v.size, rows, 27)
    dec0, dec1 = po.block8_decode(codes, scales, v.size), po.block8_decode(z, scales, v.size)
    mask = np.zeros(v.size, bool)
    for r in rows:
        mask[r * 27:(r + 1) * 27] = True
    assert (dec1[mask] == 0.0).all()
    np.testing.assert_array_equal(dec1[~mask], dec0[~mask])


def _pipeline(cfg, n, cull_run=None):
    """A rendered view's SH-step inputs, all from the oracle: color_dir and
    grad_sq from project_update, dense v_sh from project_backward."""
    w = scenes.workload(cfg, n)
    sc = w.scene
    sc.transforms = sc.transforms.copy()
    sc.transforms[::5, 2] = -3.0                     # every fifth splat behind the camera: culled
    if cull_run is not None:
        sc.transforms[cull_run, 2] = -3.0            # a run long enough to cover whole moment blocks
    cam = w.cameras[0].uniforms(w.img_size)
    fwd = po.render_forward(cam, w.img_size, sc.transforms, sc.sh_coeffs, sc.raw_opacities, flags=po.FLAG_BWD_INFO)
    img = fwd.get(po.F_OUT_IMG)
    mask = circle_mask(w.img_size, w.mask_center, w.mask_radius) if w.mask_radius > 0 else None
    v_out = l1_cotangent_np(img, scenes.loss_target(w.img_size), mask)
    vc = fwd.backward(v_out)["v_combined"]
    adam = po.OrAdam(0.9, 0.999, 10.0, 1000.0, 1e-15, 0.05, 0.0, 1)
    nn = sc.num_splats
    upd = fwd.project_update(vc, sc.transforms, sc.raw_opacities, np.zeros((nn, 10), np.uint32),
                             np.full(10, 1e-4, np.float32), np.zeros(nn, np.uint32), adam)
    dense = fwd.project_backward(vc)
    rows = np.zeros(nn, np.uint32)
    vis = fwd.get(po.F_GLOBAL_FROM_COMPACT)
    rows[vis] = vis + 1
    return sc, upd, dense, rows


@pytest.mark.parametrize("cfg,n", [("c1", 3000), ("c2", 4000)])
def test_step_matches_float64_restatement(cfg, n):
    """First step on f16 coefficients: the moments decode to (1 - beta1) times
    the dense SH gradient of the projection VJP (within the block's 8-bit step),
    each stepped coefficient is an f16 neighbour of the float64 update, and
    culled splats keep coefficients and moments."""
    sc, upd, dense, rows = _pipeline(cfg, n)
    n, k = sc.sh_coeffs.shape[:2]
    sh = sc.sh_coeffs.astype(np.float16)
    codes = np.zeros(((n * k * 3 + 127) // 128) * 32, np.uint32)
    scales = np.zeros(codes.size // 32, np.float32)
    var0 = np.zeros(n, np.float32)
    # the step's f32 constants, read back as float64
    beta1, beta2 = float(np.float32(0.9)), float(np.float32(0.999))
    eps, lr, t = 1e-15, float(np.float32(2.5e-3)), 1
    inv1, inv2 = float(np.float32(1.0 / (1 - beta1))), float(np.float32(1.0 / (1 - beta2)))
    lr_scale = np.where(np.arange(k * 3) < 3, 1.0, 1.0 / 20.0).astype(np.float32)
    gsq = upd["grad_sq"].reshape(-1)
    out, var, co, scs = po.sh_step(sh, upd["color_dir"], rows, gsq, var0, codes, scales, lr_scale, beta1=beta1,
                                   beta2=beta2, inv1=inv1, inv2=inv2, epsilon=eps, lr=lr,
                                   round_seed=t, first=True)
    np.testing.assert_allclose(var, gsq.astype(np.float64) * (1 - beta2), rtol=1e-6, atol=0)
    g64 = dense["v_sh"].reshape(n, k * 3).astype(np.float64)
    m64 = (1 - beta1) * g64
    mdec = po.block8_decode(co, scs, n * k * 3).reshape(n, k * 3)
    flat_m = m64.reshape(-1)
    for b in range(scs.size):
        sl = slice(b * 128, min((b + 1) * 128, flat_m.size))
        tol = np.abs(flat_m[sl]).max() / 254.0 * 1.0001 + 1e-30
        assert np.all(np.abs(mdec.reshape(-1)[sl] - flat_m[sl]) <= tol), b
    vis = rows != 0
    assert vis.sum() > 100 and (~vis).sum() > 100
    step64 = m64 * inv1 / (np.sqrt(var.astype(np.float64) * inv2)[:, None] + eps) * (lr_scale[None, :] * lr)
    want = sh.reshape(n, k * 3).astype(np.float64) - step64
    got = out.reshape(n, k * 3).astype(np.float64)
    spacing = np.abs(np.spacing(np.abs(want).astype(np.float16)).astype(np.float64))
    err = np.abs(got - want)
    assert np.all(err[vis] <= spacing[vis] * 1.01 + 1e-7 * np.abs(want[vis]) + 2 ** -24)
    np.testing.assert_array_equal(out[~vis].view(np.uint16), sh[~vis].view(np.uint16))
    # the colour rebuild and the dense gradient agree for every visible value
    assert np.abs(step64[vis]).max() > 0


def test_lazy_rule_and_untouched_blocks():
    """Second step: splats without a gradient row keep variance; blocks that
    hold no value of such a splat keep codes and scale bit for bit."""
    sc, upd, _, rows = _pipeline("c1", 2000, cull_run=slice(200, 400))
    n, k = sc.sh_coeffs.shape[:2]
    rng = np.random.default_rng(6)
    sh = sc.sh_coeffs.astype(np.float16)
    vals = rng.standard_normal(n * k * 3).astype(np.float32) * 1e-3
    codes, scales = po.block8_encode(vals)
    var = rng.uniform(0, 1e-4, n).astype(np.float32)
    kw = dict(beta1=0.9, beta2=0.999, inv1=5.26, inv2=500.0, epsilon=1e-15, lr=1e-3, round_seed=2, first=False)
    out, v2, c2, s2 = po.sh_step(sh, upd["color_dir"], rows, upd["grad_sq"].reshape(-1), var, codes, scales,
                                 np.ones(k * 3, np.float32), **kw)
    vis = rows != 0
    np.testing.assert_array_equal(v2[~vis], var[~vis])
    np.testing.assert_array_equal(out[~vis].view(np.uint16), sh[~vis].view(np.uint16))
    assert (out[vis].view(np.uint16) != sh[vis].view(np.uint16)).any()
    b2 = float(np.float32(0.999))
    want_v = var.astype(np.float64) * b2 + upd["grad_sq"].reshape(-1).astype(np.float64) * (1 - b2)
    np.testing.assert_allclose(v2[vis], want_v[vis], rtol=1e-6)
    per_value = np.repeat(vis, k * 3)
    nb = scales.size
    blk_any = np.zeros(nb, bool)
    for b in range(nb):
        blk_any[b] = per_value[b * 128:(b + 1) * 128].any()
    assert (~blk_any).sum() > 0 and blk_any.sum() > 0
    for b in np.nonzero(~blk_any)[0]:
        np.testing.assert_array_equal(c2[b * 32:(b + 1) * 32], codes[b * 32:(b + 1) * 32])
        assert s2[b] == scales[b]
    # the same inputs and seed give the same bits; another seed rounds differently
    again = po.sh_step(sh, upd["color_dir"], rows, upd["grad_sq"].reshape(-1), var, codes, scales,
                       np.ones(k * 3, np.float32), **kw)
    np.testing.assert_array_equal(again[0].view(np.uint16), out.view(np.uint16))
    kw["round_seed"] = 3
    other = po.sh_step(sh, upd["color_dir"], rows, upd["grad_sq"].reshape(-1), var, codes, scales,
                       np.ones(k * 3, np.float32), **kw)
    assert (other[0].view(np.uint16) != out.view(np.uint16)).any()


@pytest.mark.parametrize("degree", [0, 2, 4])
def test_rows_that_share_words(degree):
    """Degrees whose rows are not a multiple of 4 values: every stepped value
    follows its own splat's row (float64 check of the moment)."""
    rng = np.random.default_rng(degree)
    n, k = 37, (degree + 1) ** 2
    sh = rng.uniform(-1, 1, (n, k, 3)).astype(np.float16)
    rows = np.where(rng.uniform(size=n) < 0.6, np.arange(n) + 1, 0).astype(np.uint32)
    cd = np.zeros((n + 1, 6), np.float32)
    cd[1:, :3] = rng.uniform(-1, 1, (n, 3))
    d = rng.standard_normal((n, 3))
    cd[1:, 3:] = d / np.linalg.norm(d, axis=1, keepdims=True)
    gsq = rng.uniform(1e-6, 1e-4, n).astype(np.float32)
    codes = np.zeros((((n * k * 3) + 127) // 128) * 32, np.uint32)
    scales = np.zeros(codes.size // 32, np.float32)
    _, var, co, scs = po.sh_step(sh, cd, rows, gsq, np.zeros(n, np.float32), codes, scales, np.ones(k * 3, np.float32),
                                 beta1=0.9, beta2=0.999, inv1=10.0, inv2=1000.0, epsilon=1e-15, lr=1e-3, round_seed=1,
                                 first=True)
    mdec = po.block8_decode(co, scs, n * k * 3).reshape(n, k, 3)
    for g in range(n):
        y = po.sh_basis(degree, cd[g + 1, 3:]).astype(np.float64)
        want = (1 - float(np.float32(0.9))) * y[:, None] * cd[g + 1, None, :3] if rows[g] else None
        if want is None:
            continue
        b0 = (g * k * 3) // 128
        blk_max = np.abs(po.block8_decode(co, scs, n * k * 3)).reshape(-1)[b0 * 128:(b0 + 2) * 128].max()
        assert np.all(np.abs(mdec[g] - want) <= blk_max / 254.0 * 1.0001 + 1e-12), g
