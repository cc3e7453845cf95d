"""The render pipeline's radix passes in both table layouts, through the C-ABI.

The depth presort and the coarse emission pass take their offsets from grouped count tables
(per-tile histogram rows plus 16-tile group sums, no scan launch) while the buffers' capacity
allows it: at most 4096 radix tiles of depth keys (capacity <= 8,388,608 Gaussians) and of
coarse entries (key capacity <= 16,777,216). Past that they take the row-scan path of
radix_sort_pairs. Buffers sized past both limits for a small scene run the row-scan path on
the same frame; both must equal the oracle bit for bit (sorted keys, values, tiles_end, last,
rgb, T, depth), with host counts and with device counts."""
import numpy as np
import pytest
import torch

from tdgs_amd import abi, host, synthetic
from test_gpu_forward import _assert_forward_equal

pytestmark = pytest.mark.gpu

BIG_CAPACITY = 8 * 1024 * 1024 + 4096        # 4099 depth-key tiles of 2048
BIG_KEYS = 16 * 1024 * 1024 + 8192           # 4098 coarse tiles of 4096


@pytest.mark.parametrize("big", [False, True])
@pytest.mark.parametrize("device_counts", [False, True])
def test_grouped_and_row_scan_radix_paths(gpu, oracle, big, device_counts):
    w = synthetic.config(1, n=20_000)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, w.gaussians.sh_degree, background_color=(0.2, 0.1, 0.3))
    r = oracle.render(w.gaussians, cam, t, opts)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    cap = BIG_CAPACITY if big else len(g)
    keys = BIG_KEYS if big else r["nb_keys"] + 1024
    buf = gpu.RenderBuffers(cap, t, 0, keys, keep_flags=True)
    out = gpu.RenderOutputs.for_camera(cam, 0, include_depth=True)
    gpu.render_(out, g, cam, t, opts, buf, device_counts=device_counts)
    torch.cuda.synchronize()
    if device_counts:
        nbf, m, _, status = buf.frame_counts()
        assert status == abi.TDGS_FRAME_OK
    _assert_forward_equal(r, out, buf)
    del buf, out
    torch.cuda.empty_cache()


def test_sort_pairs_at_cfg4_scale_properties(gpu):
    """tdgs_sort_pairs, the drop-in of the reference's only native call (sort_pairs,
    cub_sort_pairs_wrapper.cu:31-43, called from forward_core.jl:618-660 with M > 100M keys at
    cfg4), on 120M (tile, depth bits) keys with end_bit 46 (cfg4's 16320 tiles need 14 tile
    bits) and many ties, values the 1-based input positions. A stable sort is characterised by
    size-independent properties, checked in chunks: keys non-decreasing, values increasing
    within equal keys (stability), every output key equal to the input key its value names,
    and the values a permutation."""
    dev = torch.device("cuda", 0)
    n = 120_000_000
    gen = torch.Generator(device="cuda").manual_seed(0x5047)
    tile = torch.randint(1, 16321, (n,), generator=gen, device=dev, dtype=torch.int64)
    depth = torch.randint(0x3c000000, 0x42000000, (n,), generator=gen, device=dev, dtype=torch.int64)
    keys = (tile << 32) | (depth & ~0xFFF)   # 24576 depths per tile for ~7350 keys: ~14% ties
    del tile, depth
    vals = torch.arange(1, n + 1, dtype=torch.int32, device=dev)
    sk, sv = gpu.sort_pairs(keys, vals, 46)
    torch.cuda.synchronize()
    del vals
    seen = torch.zeros(n + 1, dtype=torch.int32, device=dev)
    chunk = 20_000_000
    ties = 0
    for c0 in range(0, n, chunk):
        c1 = min(n, c0 + chunk + 1)
        k = sk[c0:c1]
        v = sv[c0:c1].to(torch.int64)
        dk = k[1:] - k[:-1]
        assert bool((dk >= 0).all()), c0
        eq = dk == 0
        ties += int(eq.sum())
        assert bool((v[1:][eq] > v[:-1][eq]).all()), c0
        m = min(chunk, n - c0)
        assert bool((keys[v[:m] - 1] == k[:m]).all()), c0
        seen.index_add_(0, v[:m], torch.ones(m, dtype=torch.int32, device=dev))
        del k, v, dk, eq
    assert ties > n // 10
    assert int(seen[0]) == 0 and bool((seen[1:] == 1).all())
