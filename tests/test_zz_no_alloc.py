"""The allocation-free sort entry point, through the C ABI.

vs_radix_argsort_u32_noalloc sorts in a per-GPU static scratch array instead
of allocating; its output must equal vs_radix_argsort_u32's bit for bit.
Calls in a row share the array (a later, smaller one must not see an earlier
one's leftovers): 3M and 50k keys (one-sweep schedule, from 4096 keys), then
3000 keys (the three-kernel schedule below 4096), with and without a device
count, and a zero-bit sort (a plain copy).  Two contexts on two streams
sorting back to back without a host wait must not share the array at the
same time.  Sizes past the array's maximum are refused before any GPU work."""
import ctypes as C

import numpy as np
import pytest
import torch

import vauss_amd as va
from vauss_amd import _lib
from vauss_amd.scenes import SplitMix64

pytestmark = pytest.mark.gpu
MAX_KEYS = 4194304


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


def _call(lib, fn, handle, keys, vals, skip, bits, n_dev, ok, ov):
    _lib.check(fn(handle, C.c_void_p(keys.data_ptr()), C.c_void_p(vals.data_ptr()), keys.numel(),
                  None if n_dev is None else C.c_void_p(n_dev.data_ptr()), skip, bits,
                  C.c_void_p(ok.data_ptr()), C.c_void_p(ov.data_ptr())))


def _both(ctx, keys, vals, skip, bits, n_dev=None):
    lib = ctx.lib
    outs = []
    for fn in (lib.vs_radix_argsort_u32, lib.vs_radix_argsort_u32_noalloc):
        ok, ov = torch.zeros_like(keys), torch.zeros_like(vals)
        _call(lib, fn, ctx.handle, keys, vals, skip, bits, n_dev, ok, ov)
        torch.cuda.synchronize()
        outs.append((ok.cpu().numpy().view(np.uint32), ov.cpu().numpy().view(np.uint32)))
    return outs


@pytest.mark.parametrize("cases", [
    [(3_000_000, 0, 32, None), (50_000, 0, 32, None), (1_000_000, 4, 13, 700_000)],
    [(200_000, 0, 32, None), (3000, 0, 32, None), (3000, 0, 16, 2222), (1000, 0, 0, None)],
], ids=["one-sweep", "three-kernel-and-copy"])
def test_noalloc_sort_matches_the_allocating_sort(cases):
    ctx = va.Context.get(torch.device("cuda"))
    rng = SplitMix64(0xA110C)
    for n, skip, bits, active in cases:
        print(f"[case] noalloc sort n={n} skip={skip} bits={bits} active={active}", flush=True)
        keys = _t(rng.next_u64(n).astype(np.uint32))
        vals = _t(np.arange(n, dtype=np.uint32))
        n_dev = None if active is None else torch.tensor([active], dtype=torch.int32, device="cuda")
        (ak, av), (bk, bv) = _both(ctx, keys, vals, skip, bits, n_dev)
        m = n if active is None else active
        np.testing.assert_array_equal(ak[:m], bk[:m])
        np.testing.assert_array_equal(av[:m], bv[:m])
        if bits == 0:
            np.testing.assert_array_equal(bk, keys.cpu().numpy().view(np.uint32))
            np.testing.assert_array_equal(bv, np.arange(n, dtype=np.uint32))
        field = (ak[:m].astype(np.uint64) >> skip) & ((1 << (8 * ((bits + 7) // 8))) - 1)
        assert (np.diff(field.astype(np.int64)) >= 0).all()


def test_noalloc_sorts_on_two_streams_do_not_overlap():
    """A second context on its own stream sorts right after the first, with no
    host wait between them: its stream waits for the first sort's event."""
    ctx = va.Context.get(torch.device("cuda"))
    lib = ctx.lib
    s2 = torch.cuda.Stream()
    h2 = C.c_void_p()
    _lib.check(lib.vs_ctx_create(torch.cuda.current_device(), C.c_void_p(s2.cuda_stream), C.byref(h2)))
    try:
        rng = SplitMix64(0x57EA)
        n1, n2 = 4_000_000, 1_500_000
        k1, v1 = _t(rng.next_u64(n1).astype(np.uint32)), _t(np.arange(n1, dtype=np.uint32))
        k2, v2 = _t(rng.next_u64(n2).astype(np.uint32)), _t(np.arange(n2, dtype=np.uint32))
        o1k, o1v = torch.zeros_like(k1), torch.zeros_like(v1)
        o2k, o2v = torch.zeros_like(k2), torch.zeros_like(v2)
        torch.cuda.synchronize()
        print("[case] noalloc sorts back to back on two streams", flush=True)
        for _ in range(3):
            _call(lib, lib.vs_radix_argsort_u32_noalloc, ctx.handle, k1, v1, 0, 32, None, o1k, o1v)
            _call(lib, lib.vs_radix_argsort_u32_noalloc, h2, k2, v2, 0, 32, None, o2k, o2v)
        torch.cuda.synchronize()
        for keys, ok, ov in ((k1, o1k, o1v), (k2, o2k, o2v)):
            kk = keys.cpu().numpy().view(np.uint32)
            idx = np.argsort(kk, kind="stable")
            np.testing.assert_array_equal(ok.cpu().numpy().view(np.uint32), kk[idx])
            np.testing.assert_array_equal(ov.cpu().numpy().view(np.uint32), idx.astype(np.uint32))
    finally:
        torch.cuda.synchronize()
        lib.vs_ctx_destroy(h2)


def test_noalloc_sort_refuses_sizes_past_its_scratch():
    ctx = va.Context.get(torch.device("cuda"))
    dummy = torch.zeros(1, dtype=torch.int32, device="cuda")
    p = C.c_void_p(dummy.data_ptr())
    st = ctx.lib.vs_radix_argsort_u32_noalloc(ctx.handle, p, p, MAX_KEYS + 1, None, 0, 32, p, p)
    assert st == _lib.VS_ERR_CAPACITY
    assert b"4194304" in ctx.lib.vs_last_error()
