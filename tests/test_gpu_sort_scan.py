"""GPU radix sort and prefix sums against the reference's known-answer tests
(crates/splat-train-sort/src/lib.rs:219-404, crates/splat-train-scan/src/lib.rs:
120-254) and numpy's stable sort / cumsum."""
import numpy as np
import pytest
import torch

import vauss_amd as va
from vauss_amd.scenes import SplitMix64

pytestmark = pytest.mark.gpu


def _sort(keys, vals, bits, skip=0, num=None):
    k = torch.from_numpy(np.asarray(keys, np.uint32).view(np.int32)).cuda()
    v = torch.from_numpy(np.asarray(vals, np.uint32).view(np.int32)).cuda()
    n = None if num is None else torch.tensor([num], dtype=torch.int32, device="cuda")
    ok, ov = va.radix_argsort_skip_low_with_count(k, v, skip, bits, n)
    return ok.cpu().numpy().view(np.uint32), ov.cpu().numpy().view(np.uint32)


def _expected(keys, vals, bits, skip=0):
    keys = np.asarray(keys, np.uint64)
    width = 8 * ((bits + 7) // 8)
    field = (keys >> np.uint64(skip)) & np.uint64((1 << width) - 1)
    idx = np.argsort(field, kind="stable")
    return np.asarray(keys, np.uint32)[idx], np.asarray(vals, np.uint32)[idx]


def test_sort_crafted_keys():
    # lib.rs:219-265: 128 crafted key sets, values 2k+5
    for i in range(128):
        keys = np.array([5 + i * 4, i, 6, 123, 74657, 123, 999, 2 ** 24 + 123, 6, 7, 8, 0, i * 2, 16 + i, 128 * i],
                        np.uint32)
        vals = keys * 2 + 5
        gk, gv = _sort(keys, vals, 32)
        ek, ev = _expected(keys, vals, 32)
        np.testing.assert_array_equal(gk, ek)
        np.testing.assert_array_equal(gv, ev)


def test_sort_gaussian_like_keys():
    # lib.rs:267-304: runs of tile-like keys
    rng = np.random.default_rng(7)
    keys = []
    for i in range(10000):
        start = rng.integers(i, i + 150)
        end = rng.integers(start, start + 250)
        js = np.arange(start, end)
        keys.extend(js[rng.random(js.size) < 0.5].tolist())
    keys = np.asarray(keys, np.uint32)
    vals = keys * 2 + 5
    gk, gv = _sort(keys, vals, 32)
    ek, ev = _expected(keys, vals, 32)
    np.testing.assert_array_equal(gk, ek)
    np.testing.assert_array_equal(gv, ev)


@pytest.mark.parametrize("n,bits,skip", [(1, 32, 0), (2047, 13, 0), (2048, 14, 0), (2049, 9, 0), (100_003, 32, 0),
                                         (1_000_000, 20, 4), (3_000_000, 32, 0), (65_537, 10, 22)])
def test_sort_random(n, bits, skip):
    rng = np.random.default_rng(n + bits)
    keys = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    vals = np.arange(n, dtype=np.uint32)
    gk, gv = _sort(keys, vals, bits, skip)
    ek, ev = _expected(keys, vals, bits, skip)
    np.testing.assert_array_equal(gk, ek)
    np.testing.assert_array_equal(gv, ev)


def test_sort_with_device_count():
    rng = np.random.default_rng(3)
    keys = rng.integers(0, 1 << 16, 50_000, dtype=np.uint64).astype(np.uint32)
    vals = np.arange(keys.size, dtype=np.uint32)
    gk, gv = _sort(keys, vals, 16, num=31_337)
    ek, ev = _expected(keys[:31_337], vals[:31_337], 16)
    np.testing.assert_array_equal(gk[:31_337], ek)
    np.testing.assert_array_equal(gv[:31_337], ev)
    np.testing.assert_array_equal(gk[31_337:], keys[31_337:])   # the inactive tail is untouched


def test_sorting_large():
    """lib.rs:308-356: 30M keys drawn from [0, 1M), values 0..n-1, all 32 bits:
    sorted, and every value points at an input with its key (checked in full
    against numpy's stable argsort, not only at the reference's sample)."""
    n = 30_000_000
    rng = np.random.default_rng(0x30)
    keys = rng.integers(0, 1_000_000, n, dtype=np.uint32)
    vals = np.arange(n, dtype=np.uint32)
    print(f"[case] sort n={n} keys < 1e6", flush=True)
    gk, gv = _sort(keys, vals, 32)
    assert (np.diff(gk.astype(np.int64)) >= 0).all()
    for idx in (0, 1000, 10_000, 100_000, 1_000_000, 10_000_000, 19_999_999):
        assert keys[gv[idx]] == gk[idx]
    idx = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(gk, keys[idx])
    np.testing.assert_array_equal(gv, idx.astype(np.uint32))


def test_sorting_above_scan_block_size():
    """lib.rs:358-403: a random permutation of 0..70M (the reference shuffles
    with SplitMix64 Fisher-Yates; any uniform permutation serves, so numpy
    draws it): sorted keys are 0..n-1 and each value is its key's position."""
    n = 70_000_000
    keys = np.random.default_rng(0xD15EA5E).permutation(n).astype(np.uint32)
    vals = np.arange(n, dtype=np.uint32)
    print(f"[case] sort permutation n={n}", flush=True)
    gk, gv = _sort(keys, vals, 32)
    np.testing.assert_array_equal(gk, np.arange(n, dtype=np.uint32))
    expected = np.empty(n, np.uint32)
    expected[keys] = vals
    np.testing.assert_array_equal(gv, expected)


@pytest.mark.parametrize("n,bits", [(5000, 46), (300_000, 40), (1_500_000, 64)])
def test_sort_u64(n, bits):
    rng = np.random.default_rng(bits)
    keys = rng.integers(0, 2 ** 64, n, dtype=np.uint64, endpoint=False) & np.uint64((1 << bits) - 1)
    keys[:n // 3] = keys[n // 3: 2 * (n // 3)]   # many exact ties to exercise stability
    vals = np.arange(n, dtype=np.uint32)
    ok, ov = va.radix_argsort_u64(torch.from_numpy(keys.view(np.int64)).cuda(),
                                  torch.from_numpy(vals.view(np.int32)).cuda(), bits)
    idx = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(ok.cpu().numpy().view(np.uint64), keys[idx])
    np.testing.assert_array_equal(ov.cpu().numpy().view(np.uint32), vals[idx])


@pytest.mark.parametrize("n", [1, 4, 255, 256, 257, 1023, 1024, 1025, 2048, 2049, 4096, 4097, 1024 * 1024,
                               1024 * 1024 + 1, 5 * (512 * 16 + 123)])
def test_prefix_sum(n):
    data = (np.arange(n) % 13).astype(np.uint32)
    if n == 5 * (512 * 16 + 123):   # scan lib.rs:173-198 pattern
        data = np.tile(np.array([2, 0, 32, 512, 30965], np.uint32), n // 5)
        data[0::5] = (2 + np.arange(n // 5)).astype(np.uint32)
    got = va.prefix_sum(torch.from_numpy(data.view(np.int32)).cuda()).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, np.cumsum(data, dtype=np.uint64).astype(np.uint32))


def test_prefix_sum_tiny_and_large():
    got = va.prefix_sum(torch.tensor([1, 1, 1, 1], dtype=torch.int32, device="cuda")).cpu().tolist()
    assert got == [1, 2, 3, 4]
    n = 30_000_000
    data = (np.arange(n) % 100).astype(np.uint32)
    got = va.prefix_sum(torch.from_numpy(data.view(np.int32)).cuda()).cpu().numpy().view(np.uint32)
    for idx in (0, 1000, 10_000, 100_000, 1_000_000, 10_000_000, 19_999_999, n - 1):
        assert int(got[idx]) == int(data[:idx + 1].sum(dtype=np.uint64))


def test_scan_in_place():
    data = (np.arange(5000) % 7 + 90).astype(np.uint32)
    t = torch.from_numpy(data.view(np.int32)).cuda()
    va.scan_in_place(t)
    np.testing.assert_array_equal(t.cpu().numpy().view(np.uint32), np.cumsum(data).astype(np.uint32))


def test_empty_inputs():
    e = torch.empty(0, dtype=torch.int32, device="cuda")
    assert va.prefix_sum(e).numel() == 0
    k, v = va.radix_argsort(e, e, 32)
    assert k.numel() == 0 and v.numel() == 0


def test_lookback_give_up_is_reported_by_the_call():
    """A one-sweep pass whose look-back gives up (forced from the host with a
    poll limit of 0: every wait ends at its first unpublished predecessor, and
    every kernel exits) makes the sort call fail; the flag is cleared, so the
    next sort with the default limit is correct."""
    ctx = va.Context.get(torch.device("cuda"))
    rng = SplitMix64(0x5717)
    keys = rng.next_u64(30_000_000).astype(np.uint32)
    vals = np.arange(keys.size, dtype=np.uint32)
    print(f"[case] sort give-up n={keys.size} spin_limit=0", flush=True)
    ctx.set_sort_spin_limit(0)
    try:
        with pytest.raises(va.VsError, match="gave up"):
            _sort(keys, vals, 32)
    finally:
        ctx.set_sort_spin_limit(None)
    gk, gv = _sort(keys[:2_000_000], vals[:2_000_000], 32)
    ek, ev = _expected(keys[:2_000_000], vals[:2_000_000], 32)
    np.testing.assert_array_equal(gk, ek)
    np.testing.assert_array_equal(gv, ev)


def test_exact_render_reports_a_sort_give_up():
    """An exact render whose depth or tile sort gave up fails in the same call."""
    from vauss_amd import scenes
    wl = scenes.workload("c2")
    sc = wl.scene
    t = torch.from_numpy(sc.transforms).cuda()
    s = torch.from_numpy(sc.sh_coeffs).cuda()
    o = torch.from_numpy(sc.raw_opacities).cuda()
    ctx = va.Context.get(t.device)
    print("[case] c2 exact render with spin_limit=0", flush=True)
    ctx.set_sort_spin_limit(0)
    try:
        with pytest.raises(va.VsError, match="gave up"):
            va.render(wl.cameras[0], wl.img_size, t, s, o, pass_=va.RasterPass.FLOAT)
    finally:
        ctx.set_sort_spin_limit(None)
    out = va.render(wl.cameras[0], wl.img_size, t, s, o, pass_=va.RasterPass.FLOAT)
    assert out.aux.num_intersections > 500_000
