"""Pins the oracle's L1 + SSIM image loss (crates/splat-train-loss/src/lib.rs)
against an independent float64 implementation (CPU only).

The float64 side builds the same quantities from their definitions with
scipy's separable correlation (zero padding) and the normalised
exp(-x^2 / 4.5) window: SSIM with C1 = 0.01^2, C2 = 0.03^2 and the
[-1, 1] clamp, the loss l1_w |p - g| + ssim_w SSIM (times gt.a when masking,
ground truth composited over a background when asked, u8 ground truth
decoded as byte / 255), per-16x16-tile sums weighted by 1 / (3 H W), and the
alpha-match term.  The backward is checked against central differences of
that float64 loss, and the stored SSIM coefficients against the partial
derivatives of the SSIM formula, also by differences.
"""
import numpy as np
import pytest
from scipy.ndimage import correlate1d

from oracle import pyoracle as po

SIGMA = 1.5


def window64():
    x = np.arange(11) - 5.0
    w = np.exp(-x * x / (2 * SIGMA * SIGMA))
    return w / w.sum()


def blur64(img):
    w = window64()
    return correlate1d(correlate1d(img, w, axis=1, mode="constant", cval=0.0), w, axis=0, mode="constant", cval=0.0)


def ssim64(p, g):
    c1, c2 = 0.01 ** 2, 0.03 ** 2
    mu1, mu2 = blur64(p), blur64(g)
    s1 = np.maximum(0.0, blur64(p * p) - mu1 * mu1)
    s2 = np.maximum(0.0, blur64(g * g) - mu2 * mu2)
    s12 = blur64(p * g) - mu1 * mu2
    raw = (2 * mu1 * mu2 + c1) * (2 * s12 + c2) / ((mu1 * mu1 + mu2 * mu2 + c1) * (s1 + s2 + c2))
    return np.clip(raw, -1.0, 1.0)


def decode_gt(gt_packed):
    b = np.stack([(gt_packed >> (8 * k)) & 0xFF for k in range(4)], axis=-1).astype(np.float64)
    return b / 255.0


def loss64(pred, gt_packed, l1_w, ssim_w, alpha_w=0.0, bg=None, mask=False):
    """The loss total in float64 (sum of every weighted tile partial)."""
    pred = pred.astype(np.float64)
    h, w, cn = pred.shape
    g = decode_gt(gt_packed)
    ga = g[..., 3]
    total = 0.0
    for c in range(3):
        ge = g[..., c] + (1.0 - ga) * bg[c] if bg is not None else g[..., c]
        lv = l1_w * np.abs(pred[..., c] - ge) + ssim_w * ssim64(pred[..., c], ge)
        if mask:
            lv = lv * ga
        total += lv.sum() / (3.0 * h * w)
    if alpha_w > 0 and cn == 4:
        v = np.abs(pred[..., 3] - ga)
        if mask:
            v = v * ga
        total += alpha_w * v.sum() / (h * w)
    return total


def make_case(h=37, w=53, cn=4, seed=0):
    rng = np.random.default_rng(seed)
    gt = rng.integers(0, 1 << 32, (h, w), dtype=np.uint64).astype(np.uint32)
    # a smooth prediction near the target plus texture, so SSIM is informative
    g = decode_gt(gt)
    pred = (0.7 * g[..., :cn] + 0.3 * rng.uniform(0, 1, (h, w, cn))).astype(np.float32)
    return pred, gt


def test_window_matches_float64():
    """The kernels' f32 taps (hex literals in oracle/vs_oracle.cpp and
    vauss_amd/csrc/k_loss.hip) are gauss_taps() (lib.rs:48-62) in f32:
    exp(-x^2 / 4.5) rounded to f32, divided by their f32 sum; that is within
    4 ulp of the float64 normalised window."""
    taps = ["0x1.0d957p-10", "0x1.f1fe04p-8", "0x1.26eb18p-5", "0x1.bff1p-4", "0x1.b43c4p-3", "0x1.106562p-2"]
    w32 = np.array([float.fromhex(t) for t in taps + taps[-2::-1]])
    w64 = window64()
    assert np.all(np.abs(w32 - w64) <= 4 * np.spacing(w64.astype(np.float32)))
    raw = [np.float32(np.exp(np.float64(np.float32(-(i - 5.0) ** 2) / np.float32(4.5)))) for i in range(11)]
    total = np.float32(0.0)
    for r in raw:
        total = np.float32(total + r)
    np.testing.assert_array_equal(w32.astype(np.float32), np.array([np.float32(r / total) for r in raw]))


@pytest.mark.parametrize("opts", [dict(), dict(bg=(0.2, 0.5, 0.9)), dict(mask=True), dict(alpha_w=0.3),
                                  dict(bg=(1.0, 0.0, 0.3), mask=True, alpha_w=0.1)])
def test_forward_matches_float64(opts):
    pred, gt = make_case(seed=1)
    l1_w, ssim_w = 0.8, -0.2
    cfg = po.loss_cfg(l1_w, ssim_w, opts.get("alpha_w", 0.0), opts.get("bg"), opts.get("mask", False))
    partials, _, lmap = po.image_loss_forward(pred, gt, cfg)
    want = loss64(pred, gt, l1_w, ssim_w, opts.get("alpha_w", 0.0), opts.get("bg"), opts.get("mask", False))
    assert abs(float(partials.astype(np.float64).sum()) - want) <= 2e-6 * abs(want) + 1e-7
    # the per-pixel map, channel by channel
    g = decode_gt(gt)
    ga = g[..., 3]
    bg = opts.get("bg")
    for c in range(3):
        ge = g[..., c] + (1.0 - ga) * bg[c] if bg is not None else g[..., c]
        lv = l1_w * np.abs(pred[..., c] - ge) + ssim_w * ssim64(pred[..., c].astype(np.float64), ge)
        if opts.get("mask"):
            lv = lv * ga
        np.testing.assert_allclose(lmap[..., c], lv, rtol=0, atol=2e-5)
    # tile partials: 16x16 sums of the map, weighted
    h, w = gt.shape
    tx = (w + 15) // 16
    for t in (0, 4, partials.shape[1] - 1):
        y0, x0 = (t // tx) * 16, (t % tx) * 16
        s = lmap[y0:y0 + 16, x0:x0 + 16, 1].astype(np.float64).sum() / (3.0 * h * w)
        assert abs(partials[1, t] - s) <= 1e-6 * abs(s) + 1e-9


def test_anticorrelated_images_give_negative_ssim():
    """pred = 1 - gt: SSIM is negative wherever the window has texture, and
    the map follows the float64 SSIM with its [-1, 1] clamp."""
    _, gt = make_case(seed=7, cn=3)
    g = decode_gt(gt)[..., :3]
    pred = (1.0 - g).astype(np.float32)
    cfg = po.loss_cfg(0.0, 1.0)
    _, _, lmap = po.image_loss_forward(pred, gt, cfg)
    for c in range(3):
        want = ssim64(pred[..., c].astype(np.float64), g[..., c])
        np.testing.assert_allclose(lmap[..., c], want, rtol=0, atol=2e-5)
    assert (lmap < -0.5).mean() > 0.5


def test_ssim_of_identical_images_is_one():
    pred, gt = make_case(seed=2, cn=3)
    exact = (decode_gt(gt)[..., :3]).astype(np.float32)
    cfg = po.loss_cfg(0.0, 1.0)
    _, _, lmap = po.image_loss_forward(exact, gt, cfg)
    assert np.all(np.abs(lmap - 1.0) <= 2e-6)


def test_coefficients_are_ssim_partials():
    """dmu1, dsigma1, dsigma12 are the partials of the SSIM formula w.r.t. the
    blurred moments mu1 = <x>, <x^2> and <xy> (sigma1^2 = <x^2> - mu1^2,
    sigma12 = <xy> - mu1 mu2), which is what the backward's
    blur(dmu1) + 2 p blur(dsigma1) + g blur(dsigma12) needs."""
    pred, gt = make_case(seed=3, cn=3)
    cfg = po.loss_cfg(0.0, 1.0)
    _, coeffs, _ = po.image_loss_forward(pred, gt, cfg)
    g = decode_gt(gt)[..., 0]
    p = pred[..., 0].astype(np.float64)
    mu1, mu2 = blur64(p), blur64(g)
    s1 = blur64(p * p) - mu1 * mu1
    s2 = blur64(g * g) - mu2 * mu2
    s12 = blur64(p * g) - mu1 * mu2
    c1, c2 = 0.01 ** 2, 0.03 ** 2

    ex2, exy = s1 + mu1 * mu1, s12 + mu1 * mu2

    def f(m1, x2, xy):
        v1, v12 = x2 - m1 * m1, xy - m1 * mu2
        return (2 * m1 * mu2 + c1) * (2 * v12 + c2) / ((m1 * m1 + mu2 * mu2 + c1) * (v1 + s2 + c2))
    e = 1e-6
    d_mu = (f(mu1 + e, ex2, exy) - f(mu1 - e, ex2, exy)) / (2 * e)
    d_v1 = (f(mu1, ex2 + e, exy) - f(mu1, ex2 - e, exy)) / (2 * e)
    d_v12 = (f(mu1, ex2, exy + e) - f(mu1, ex2, exy - e)) / (2 * e)
    for got, want in ((coeffs[0, 0], d_mu), (coeffs[0, 1], d_v1), (coeffs[0, 2], d_v12)):
        np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-3 * np.abs(want).max())


@pytest.mark.parametrize("opts", [dict(), dict(bg=(0.3, 0.6, 0.1), mask=True, alpha_w=0.25)])
def test_backward_matches_finite_differences(opts):
    pred, gt = make_case(h=24, w=29, seed=4)
    l1_w, ssim_w = 0.8, -0.2
    args = (l1_w, ssim_w, opts.get("alpha_w", 0.0), opts.get("bg"), opts.get("mask", False))
    cfg = po.loss_cfg(*args)
    _, coeffs, _ = po.image_loss_forward(pred, gt, cfg)
    grad = po.image_loss_backward(pred, gt, cfg, np.ones(1, np.float32), coeffs)
    g = decode_gt(gt)
    bgv = opts.get("bg")
    rng = np.random.default_rng(5)
    h, w, cn = pred.shape
    checked = 0
    for _ in range(400):
        y, x, c = int(rng.integers(h)), int(rng.integers(w)), int(rng.integers(cn))
        ge = g[y, x, c] if c == 3 else (g[y, x, c] + (1 - g[y, x, 3]) * bgv[c] if bgv is not None else g[y, x, c])
        if abs(float(pred[y, x, c]) - ge) < 2e-3:       # stay off the L1 kink
            continue
        e = 1e-4
        pp = pred.astype(np.float64)
        pp[y, x, c] += e
        up = loss64(pp, gt, *args)
        pp[y, x, c] -= 2 * e
        dn = loss64(pp, gt, *args)
        fd = (up - dn) / (2 * e)
        assert abs(grad[y, x, c] - fd) <= 2e-3 * abs(fd) + 2e-8, (y, x, c, grad[y, x, c], fd)
        checked += 1
    assert checked > 200
    # per-tile cotangents: a one-hot dl/dpartials gives the tile's own gradient
    planes = 4 if args[2] > 0 else 3
    tiles = ((w + 15) // 16) * ((h + 15) // 16)
    dl = np.zeros((planes, tiles), np.float32)
    dl[1, 0] = 1.0
    gt_one = po.image_loss_backward(pred, gt, cfg, dl, coeffs)
    assert np.abs(gt_one[20:, 20:, 1]).max() == 0.0 or np.abs(gt_one[..., 1]).max() > 0
    assert np.abs(gt_one[..., 0]).max() == 0.0          # other channels untouched
