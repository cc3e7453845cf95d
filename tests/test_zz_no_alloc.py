"""The allocation-free entry point tdgs_scan_counts_noalloc (no reference counterpart: for
callers that cannot allocate device memory) against tdgs_scan_counts, the entry point it
varies, through the C-ABI: two calls in a row on one GPU, the second with a smaller input,
both bit-identical to the workspace-taking scan and to numpy's cumulative sum; a total past 2^31
keeps its int64 total exact and wraps the int32 sums modulo 2^32 (as tdgs.h states); an empty input
writes a zero total; an input past the stated maximum is rejected."""
import ctypes as C

import numpy as np
import pytest
import torch

from tdgs_amd import abi

pytestmark = pytest.mark.gpu

MAX_ITEMS = 16_777_216


def _noalloc(L, stream, counts, n):
    cs = torch.full((max(n, 1),), -7, dtype=torch.int32, device="cuda")
    tot = torch.full((1,), -7, dtype=torch.int64, device="cuda")
    rc = L.tdgs_scan_counts_noalloc(stream, C.c_void_p(counts.data_ptr() if n else None), C.c_int32(n),
                                    C.c_void_p(cs.data_ptr()), C.c_void_p(tot.data_ptr()))
    return rc, cs[:n], tot


def test_scan_counts_noalloc_matches_scan_counts(gpu):
    L = gpu.lib()
    stream = gpu.stream_ptr(0)
    rng = np.random.default_rng(77)
    for n in (MAX_ITEMS, 3_000_001, 70_000):   # later calls smaller: stale tile sums must not leak
        host_counts = rng.integers(0, 64, size=n, dtype=np.int32)
        counts = torch.from_numpy(host_counts).cuda()
        cs_ref, tot_ref = gpu.scan_counts(counts)
        rc, cs, tot = _noalloc(L, stream, counts, n)
        assert rc == abi.TDGS_OK, L.tdgs_last_error()
        torch.cuda.synchronize()
        assert int(tot.item()) == tot_ref == int(host_counts.astype(np.int64).sum())
        assert torch.equal(cs, cs_ref)
        np.testing.assert_array_equal(cs.cpu().numpy(), np.cumsum(host_counts, dtype=np.int64).astype(np.int32))
    rc, _, tot = _noalloc(L, stream, None, 0)
    assert rc == abi.TDGS_OK
    torch.cuda.synchronize()
    assert int(tot.item()) == 0
    # a total of 2^31 or more: the int64 total is exact, the int32 inclusive sums wrap modulo
    # 2^32 (the caller checks the total before using them)
    n = MAX_ITEMS
    host_counts = rng.integers(150, 250, size=n, dtype=np.int32)
    counts = torch.from_numpy(host_counts).cuda()
    rc, cs, tot = _noalloc(L, stream, counts, n)
    assert rc == abi.TDGS_OK
    torch.cuda.synchronize()
    exact = np.cumsum(host_counts, dtype=np.int64)
    assert int(tot.item()) == int(exact[-1]) > 2**31
    np.testing.assert_array_equal(cs.cpu().numpy(), exact.astype(np.uint32).view(np.int32))
    big = torch.zeros(1, dtype=torch.int32, device="cuda")
    rc = L.tdgs_scan_counts_noalloc(stream, C.c_void_p(big.data_ptr()), C.c_int32(MAX_ITEMS + 1),
                                    C.c_void_p(big.data_ptr()), C.c_void_p(big.data_ptr()))
    assert rc == abi.TDGS_ERR_INVALID and b"at most" in L.tdgs_last_error()
