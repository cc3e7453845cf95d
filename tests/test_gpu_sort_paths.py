"""The render pipeline's radix passes in both table layouts and the depth presort's buckets,
through the C-ABI.

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


def test_depth_presort_bucket_past_capacity(gpu, oracle):
    """The bucketed depth presort (dsort.hpp) takes its splitters from a sample of 8192 slots;
    a bucket of more than 8192 Gaussians is sorted chunk by chunk through global memory. Here
    the sampled slots keep the scene's depths while every other Gaussian lies in a narrow depth
    band (relative width 1e-5) that no sampled key falls in: that band (~42k Gaussians, distinct
    depths) lands in at most two buckets. The frame must equal the oracle bit for bit (tile lists,
    images, last contributors), with host and with device counts."""
    from tdgs_amd import synthetic
    n = 50_000
    w = synthetic.config(0, n=n)
    cam = w.cameras[0]
    g_host = w.gaussians
    sampled = np.zeros(n, bool)
    sampled[(np.arange(8192, dtype=np.int64) * n) // 8192] = True   # ds_sample_store's slots
    rng = np.random.default_rng(11)
    mo = g_host.means_opacity
    fwd = cam.R_c2w[:, 2].astype(np.float64)
    pos = np.asarray(cam.t_c2w, np.float64)
    # every Gaussian inside the view (all kept: filtered index = index): the sampled ones at
    # depths 2-4.8 or 5.2-8, the others in the band 5 .. 5 + 5e-5
    d = np.where(sampled, np.where(rng.random(n) < 0.5, rng.uniform(2.0, 4.8, n), rng.uniform(5.2, 8.0, n)),
                 5.0 + rng.uniform(0, 5e-5, n))
    mo[:, :3] = (pos + d[:, None] * fwd + rng.uniform(-0.5, 0.5, (n, 1)) * cam.R_c2w[:, 0]
                 + rng.uniform(-0.5, 0.5, (n, 1)) * cam.R_c2w[:, 1]).astype(np.float32)
    mo[:, 3] = np.abs(mo[:, 3])   # opacities >= 1/2: none culled for its alpha
    opts = host.RenderOptions.for_camera(cam, 0)
    t = host.Tiling.for_camera(cam, 16, 16)
    r = oracle.render(g_host, cam, t, opts)
    nf = r["nb_fgaussians"]
    assert nf == n
    keys = r["depths"][:nf].view(np.uint32)[r["counts"][:nf] > 0]
    lo, hi = np.float32(5.0).view(np.uint32), np.float32(5.00006).view(np.uint32)
    in_band = (keys >= lo) & (keys <= hi)
    assert in_band.sum() > 2 * 8192 + 100, in_band.sum()
    samp_keys = r["depths"][:nf][sampled].view(np.uint32)
    assert not bool(((samp_keys >= lo) & (samp_keys <= hi)).any())
    g = gpu.TrainableGaussiansVector.from_host(g_host, 0)
    for device_counts in (False, True):
        buf = gpu.RenderBuffers(len(g), t, 0, r["nb_keys"] + 1024, keep_flags=True)
        out = gpu.RenderOutputs.for_camera(cam, 0, include_depth=True)
        gpu.render_(out, g, cam, t, opts, buf, device_counts=device_counts)
        torch.cuda.synchronize()
        if device_counts:
            assert buf.frame_counts()[3] == abi.TDGS_FRAME_OK
        _assert_forward_equal(r, out, buf)
