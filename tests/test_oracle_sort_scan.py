"""The oracle's stable LSD radix argsort and inclusive scan against the
reference's own known-answer tests (crates/splat-train-sort/src/lib.rs:219-404,
crates/splat-train-scan/src/lib.rs:120-254) and a stable std sort / serial sum."""
import numpy as np
import pytest

from oracle import pyoracle as po
from vauss_amd.scenes import SplitMix64


def _stable(keys, vals, skip=0, bits=32):
    field = (keys.astype(np.uint64) >> np.uint64(skip)) & np.uint64((1 << (8 * ((bits + 7) // 8))) - 1)
    order = np.argsort(field, kind="stable")
    return keys[order], vals[order]


def test_sort_crafted_keys():
    for i in range(128):
        keys = np.array([5 + i * 4, i, 6, 123, 74657, 123, 999, 2 ** 24 + 123, 6, 7, 8, 0, i * 2, 16 + i, 128 * i],
                        np.uint32)
        vals = keys * np.uint32(2) + np.uint32(5)
        k, v = po.radix_argsort_u32(keys, vals, 0, 32)
        rk, rv = _stable(keys, vals)
        np.testing.assert_array_equal(k, rk)
        np.testing.assert_array_equal(v, rv)


def test_sort_gaussian_like_keys():
    rng = np.random.default_rng(0)
    keys = []
    for i in range(10_000):
        start = int(rng.integers(i, i + 150))
        end = int(rng.integers(start, start + 250))
        run = np.arange(start, end)
        keys.append(run[rng.random(run.size) < 0.5])
    keys = np.concatenate(keys).astype(np.uint32)
    vals = keys * np.uint32(2) + np.uint32(5)
    k, v = po.radix_argsort_u32(keys, vals, 0, 32)
    rk, rv = _stable(keys, vals)
    np.testing.assert_array_equal(k, rk)
    np.testing.assert_array_equal(v, rv)


def test_sort_is_stable_and_honours_skip_and_bit_count():
    rng = np.random.default_rng(1)
    keys = rng.integers(0, 2 ** 32, 50_000, dtype=np.uint64).astype(np.uint32)
    vals = np.arange(keys.size, dtype=np.uint32)
    for skip, bits in [(0, 13), (8, 8), (16, 9), (4, 32)]:
        k, v = po.radix_argsort_u32(keys, vals, skip, bits)
        rk, rv = _stable(keys, vals, skip, bits)
        np.testing.assert_array_equal(v, rv)
        np.testing.assert_array_equal(k, rk)


def test_sort_permutation_with_splitmix_shuffle():
    """A shuffled permutation sorts back to the identity (the reference's
    above-block-size regression test, at a size the CPU handles quickly)."""
    n = 300_000
    keys = np.arange(n, dtype=np.uint32)
    rng = SplitMix64(0xD15EA5E)
    z = rng.next_u64(n - 1)
    for idx, i in enumerate(range(n - 1, 0, -1)):
        j = int(z[idx] % np.uint64(i + 1))
        keys[i], keys[j] = keys[j], keys[i]
    vals = np.arange(n, dtype=np.uint32)
    expected = np.empty(n, np.uint32)
    expected[keys] = vals
    k, v = po.radix_argsort_u32(keys, vals, 0, 32)
    np.testing.assert_array_equal(k, np.arange(n, dtype=np.uint32))
    np.testing.assert_array_equal(v, expected)


@pytest.mark.parametrize("n", [0, 1, 4, 255, 256, 257, 1023, 1024, 1025, 2048, 2049, 1024 * 1024, 1024 * 1024 + 1])
def test_prefix_sum_matches_serial_sum(n):
    data = (np.arange(n) % 13).astype(np.uint32)
    got = po.prefix_sum_u32(data)
    np.testing.assert_array_equal(got, np.cumsum(data, dtype=np.uint64).astype(np.uint32))


def test_prefix_sum_known_answers():
    np.testing.assert_array_equal(po.prefix_sum_u32(np.ones(4, np.uint32)), [1, 2, 3, 4])
    data = np.array([[2 + i, 0, 32, 512, 30965] for i in range(512 * 16 + 123)], np.uint32).ravel()
    np.testing.assert_array_equal(po.prefix_sum_u32(data), np.cumsum(data, dtype=np.uint64).astype(np.uint32))
