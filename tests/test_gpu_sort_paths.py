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
