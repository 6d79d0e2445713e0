"""The allocation-free sort entry point, through the C ABI.

vs_radix_argsort_u32_noalloc sorts in a per-GPU static scratch array instead
of allocating; its output must equal vs_radix_argsort_u32's bit for bit.  Two
calls in a row share the array (the second, smaller one must not see the
first's leftovers): a one-sweep sort of 3M keys, then a 50k-key sort on the
three-kernel schedule, then one with a device count; sizes past the array's
maximum are refused before any GPU work."""
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


def _both(ctx, keys, vals, skip, bits, n_dev=None):
    lib = ctx.lib
    n = keys.numel()
    outs = []
    for fn in (lib.vs_radix_argsort_u32, lib.vs_radix_argsort_u32_noalloc):
        ok, ov = torch.zeros_like(keys), torch.zeros_like(vals)
        _lib.check(fn(ctx.handle, C.c_void_p(keys.data_ptr()), C.c_void_p(vals.data_ptr()), n,
                      None if n_dev is None else C.c_void_p(n_dev.data_ptr()), skip, bits,
                      C.c_void_p(ok.data_ptr()), C.c_void_p(ov.data_ptr())))
        torch.cuda.synchronize()
        outs.append((ok.cpu().numpy().view(np.uint32), ov.cpu().numpy().view(np.uint32)))
    return outs


def test_noalloc_sort_matches_the_allocating_sort():
    ctx = va.Context.get(torch.device("cuda"))
    rng = SplitMix64(0xA110C)
    cases = [(3_000_000, 0, 32, None), (50_000, 0, 32, None), (1_000_000, 4, 13, 700_000)]
    for n, skip, bits, active in cases:
        print(f"[case] noalloc sort n={n} skip={skip} bits={bits} active={active}", flush=True)
        keys = _t(rng.next_u64(n).astype(np.uint32))
        vals = _t(np.arange(n, dtype=np.uint32))
        n_dev = None if active is None else torch.tensor([active], dtype=torch.int32, device="cuda")
        (ak, av), (bk, bv) = _both(ctx, keys, vals, skip, bits, n_dev)
        m = n if active is None else active
        np.testing.assert_array_equal(ak[:m], bk[:m])
        np.testing.assert_array_equal(av[:m], bv[:m])
        field = (ak[:m].astype(np.uint64) >> skip) & ((1 << (8 * ((bits + 7) // 8))) - 1)
        assert (np.diff(field.astype(np.int64)) >= 0).all()


def test_noalloc_sort_refuses_sizes_past_its_scratch():
    ctx = va.Context.get(torch.device("cuda"))
    dummy = torch.zeros(1, dtype=torch.int32, device="cuda")
    p = C.c_void_p(dummy.data_ptr())
    st = ctx.lib.vs_radix_argsort_u32_noalloc(ctx.handle, p, p, MAX_KEYS + 1, None, 0, 32, p, p)
    assert st == _lib.VS_ERR_CAPACITY
    assert b"4194304" in ctx.lib.vs_last_error()
