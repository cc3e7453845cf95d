"""GPU parity of the forward path (render!) against the CPU oracle, through the C-ABI.

Integer outputs (compaction, tile rectangles, counts, sorted keys and lists, tile ranges,
last contributors) and, because the kernels run the oracle's exact single-precision
operation sequence, the images themselves must match bit for bit.
"""
import numpy as np
import pytest
import torch

from conftest import golden, stacked_faint_gaussians
from tdgs_amd import host, synthetic

pytestmark = pytest.mark.gpu


def _gpu_render(core, g_host, cam, t, opts, depth=True):
    g = core.TrainableGaussiansVector.from_host(g_host, 0)
    out = core.RenderOutputs.for_camera(cam, 0, include_depth=depth)
    buf = core.RenderBuffers(len(g), t, 0, keep_flags=True)
    core.render_(out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    return out, buf


def _assert_forward_equal(orc_r, out, buf):
    nf, m = orc_r["nb_fgaussians"], orc_r["nb_keys"]
    assert buf.nb_fgaussians == nf
    assert buf.nb_keys == m
    np.testing.assert_array_equal(buf.keep.cpu().numpy()[: len(orc_r["keep"])], orc_r["keep"])
    np.testing.assert_array_equal(buf.fgidx_to_gidx[:nf].cpu().numpy(), orc_r["fgidx_to_gidx"][:nf])
    counts = buf.counts[:nf].cpu().numpy()
    np.testing.assert_array_equal(counts, orc_r["counts"][:nf])
    ne = counts > 0
    np.testing.assert_array_equal(buf.tile_ranges[:nf].cpu().numpy()[ne], orc_r["tile_ranges"][:nf][ne])
    np.testing.assert_array_equal(buf.depths[:nf].cpu().numpy()[ne], orc_r["depths"][:nf][ne])
    np.testing.assert_array_equal(buf.f2d[:nf].cpu().numpy()[ne], orc_r["f2d"][:nf][ne])
    if m > 0:
        np.testing.assert_array_equal(buf.sorted_keys[:m].cpu().numpy(), orc_r["sorted_keys"])
        np.testing.assert_array_equal(buf.sorted_values[:m].cpu().numpy(), orc_r["sorted_values"])
        np.testing.assert_array_equal(buf.tiles_end.cpu().numpy(), orc_r["tiles_end"])
    np.testing.assert_array_equal(out.last.cpu().numpy(), orc_r["last"])
    np.testing.assert_array_equal(out.T.cpu().numpy(), orc_r["T"])
    np.testing.assert_array_equal(out.rgb.cpu().numpy(), orc_r["rgb"])
    if out.depth is not None:
        np.testing.assert_array_equal(out.depth.cpu().numpy(), orc_r["depth"])


def test_render_helpers_known_answers(gpu):
    gold = golden("render_helpers.json")
    dev = torch.device("cuda", 0)
    cs, f2g, nf = gpu.fill_fgidx_to_gidx(torch.tensor(gold["keep"], dtype=torch.uint8, device=dev))
    assert nf == 3 and f2g.cpu().tolist() == gold["fgidx_to_gidx"]
    t = host.Tiling.for_screen(2, 2, 1, 1)
    counts = torch.tensor(gold["counts"], dtype=torch.int32, device=dev)
    ccs, m = gpu.scan_counts(counts)
    assert m == 6
    keys, vals = gpu.emit_keys(torch.tensor(gold["depths"], dtype=torch.float32, device=dev),
                               torch.tensor(gold["tile_ranges"], dtype=torch.int32, device=dev), ccs, m, t)
    assert vals.cpu().tolist() == gold["dfgidx_to_fgidx"]
    sk, sv = gpu.sort_pairs(keys, vals, t.end_bit())
    assert sv.cpu().tolist() == gold["sdfgidx_to_fgidx"]
    te = gpu.tile_ranges(sk, t.nb_tiles)
    assert te.cpu().tolist() == gold["tiles_end"]


@pytest.mark.parametrize("n,end_bit,spread", [(1, 41, 4), (1000, 41, 8), (4097, 45, 16), (100_000, 45, 64),
                                              (300_000, 64, 1 << 40), (70_000, 20, 1000),
                                              (2_000_000, 46, 5000), (600_000, 40, 1)])
def test_sort_pairs_matches_stable_sort(gpu, oracle, n, end_bit, spread):
    rng = np.random.default_rng(n + end_bit)
    hi = rng.integers(0, spread, size=n).astype(np.int64)
    lo = rng.integers(0, 1 << 31, size=n).astype(np.int64) & ~np.int64(0xFF)  # many ties
    keys = (hi << 32) | lo if end_bit > 32 else hi
    vals = np.arange(1, n + 1, dtype=np.int32)
    ko, vo = oracle.sort_pairs(keys, vals, end_bit)
    dev = torch.device("cuda", 0)
    gk, gv = gpu.sort_pairs(torch.from_numpy(keys).to(dev), torch.from_numpy(vals).to(dev), end_bit)
    np.testing.assert_array_equal(gk.cpu().numpy(), ko)
    np.testing.assert_array_equal(gv.cpu().numpy(), vo)


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_render_test_scene_bit_exact(gpu, oracle, deg):
    g, cams = host.create_test_scene(sh_degree=deg)
    cam = cams[0]
    opts = host.RenderOptions.for_camera(cam, deg)
    t = host.Tiling.for_camera(cam, 16, 16)
    r = oracle.render(g, cam, t, opts)
    out, buf = _gpu_render(gpu, g, cam, t, opts)
    _assert_forward_equal(r, out, buf)


@pytest.mark.parametrize("cfg,n,tile", [(0, None, (16, 16)), (1, 20_000, (16, 16)), (2, 60_000, (16, 16)),
                                        (2, 60_000, (16, 32))])
def test_render_synthetic_bit_exact(gpu, oracle, cfg, n, tile):
    w = synthetic.config(cfg, n=n, cameras=3)
    cam = w.cameras[min(1, len(w.cameras) - 1)]
    t = host.Tiling.for_camera(cam, *tile)
    opts = host.RenderOptions.for_camera(cam, w.gaussians.sh_degree, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(w.gaussians, cam, t, opts)
    out, buf = _gpu_render(gpu, w.gaussians, cam, t, opts)
    assert r["nb_keys"] > 1000
    _assert_forward_equal(r, out, buf)


@pytest.mark.parametrize("deg", [0, 1, 2])
def test_render_sh3_storage_at_lower_degrees(gpu, oracle, deg):
    """16-coefficient storage rendered at SH degrees 0-2 (training's degree schedule): the
    colours use only the first (deg + 1)^2 coefficients of each channel."""
    w = synthetic.config(1, n=20_000, cameras=2)
    assert w.gaussians.sh_degree == 3
    cam = w.cameras[-1]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, deg, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(w.gaussians, cam, t, opts)
    out, buf = _gpu_render(gpu, w.gaussians, cam, t, opts)
    assert r["nb_keys"] > 1000
    _assert_forward_equal(r, out, buf)


@pytest.mark.parametrize("w,h,tile", [(37, 23, (32, 32)), (301, 173, (8, 8)), (64, 64, (64, 16)), (1, 1, (16, 16))])
def test_render_odd_sizes_and_tiles(gpu, oracle, w, h, tile):
    """Partial tiles at the right and bottom edges, 1024-thread (32x32) and 64-pixel tiles,
    and a one-pixel image."""
    from tdgs_amd.host import look_at_camera
    wl = synthetic.config(0, n=2000)
    cam = look_at_camera(w, h, 60.0, (0.0, 0.0, -4.0))
    t = host.Tiling.for_camera(cam, *tile)
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(wl.gaussians, cam, t, opts)
    out, buf = _gpu_render(gpu, wl.gaussians, cam, t, opts)
    _assert_forward_equal(r, out, buf)


@pytest.mark.parametrize("size,tile", [(8, (8, 8)), (16, (16, 16)), (16, (32, 32))])
def test_render_list_lengths_at_group_and_batch_ends(gpu, oracle, size, tile):
    """One-tile images whose list holds 1 to 5 records, or 1 to 3 records past a full group of
    four and past a full batch (64, 256 and 1024 records: one per thread of 8x8, 16x16 and 32x32
    tiles; the 32x32 tile lies mostly outside its 16 x 16 image). No pixel stops early and the
    list's last record contributes, so every record is stepped, including the padding after
    the list's last group."""
    from tdgs_amd.host import look_at_camera
    cam = look_at_camera(size, size, 60.0, (0.0, 0.0, -4.0))
    t = host.Tiling.for_camera(cam, *tile)
    assert t.nb_tiles == 1
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.1, 0.2, 0.3))
    for k in (1, 2, 3, 4, 5, 63, 64, 65, 66, 67, 255, 256, 257, 258, 259, 1023, 1024, 1025, 1026, 1027):
        g = stacked_faint_gaussians(k)
        r = oracle.render(g, cam, t, opts)
        assert r["nb_keys"] == k and r["last"].max() == k and r["T"].min() > 1e-3, k
        out, buf = _gpu_render(gpu, g, cam, t, opts)
        _assert_forward_equal(r, out, buf)


@pytest.mark.parametrize("width", [2040, 2048])
def test_render_tile_id_width_boundary(gpu, oracle, width):
    """8x8 tiles on width x 2056 pixels: 255 x 257 = 65535 tiles (the largest tiling whose
    tile ids the sort moves as 16-bit values, keys assembled on request) and 256 x 257 = 65792
    (64-bit keys sorted). Both must give the oracle's keys, lists, tile ranges and images."""
    from tdgs_amd.host import look_at_camera
    w = synthetic.config(0, n=4000)
    cam = look_at_camera(width, 2056, 60.0, (0.0, 0.0, -4.0))
    t = host.Tiling.for_camera(cam, 8, 8)
    assert (t.nb_tiles <= 65535) == (width == 2040)
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(w.gaussians, cam, t, opts)
    out, buf = _gpu_render(gpu, w.gaussians, cam, t, opts, depth=False)
    assert r["nb_keys"] > 10_000 and r["sorted_keys"].max() >> 32 > 60_000
    _assert_forward_equal(r, out, buf)


def test_render_large_footprints_bit_exact(gpu, oracle):
    """Gaussians covering tens of tiles each (M > 32 N_f): tiles_end then comes from the tile
    rectangles (difference array) instead of the sorted keys; it must be the same."""
    w = synthetic.config(0, n=3000)
    g = w.gaussians
    g.scaling[...] = g.scaling + np.float32(2.0)   # log-scales ~ N(-1.5, 0.4)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.3, 0.2, 0.1))
    r = oracle.render(g, cam, t, opts)
    out, buf = _gpu_render(gpu, g, cam, t, opts)
    assert r["nb_keys"] > 32 * r["nb_fgaussians"]
    _assert_forward_equal(r, out, buf)


def test_render_needle_gaussians_without_dilation(gpu, oracle):
    """Needle-thin Gaussians with no dilation: within one wavefront's 8x8 pixels the exponent
    falls from above the cut to below -1000, where the branch-free exponential core is not
    exp_f; such lanes must neither contribute nor stop."""
    w = synthetic.config(0, n=4000)
    g = w.gaussians
    g.scaling[:, 0] = np.float32(-7.0)   # sub-pixel width along one axis
    g.scaling[:, 1] = np.float32(-1.0)
    g.means_opacity[:, 3] = np.float32(4.0)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 0, dilation_x_px=0.0, dilation_y_px=0.0)
    r = oracle.render(g, cam, t, opts)
    out, buf = _gpu_render(gpu, g, cam, t, opts)
    assert r["nb_keys"] > 1000
    _assert_forward_equal(r, out, buf)


@pytest.mark.parametrize("depth", [False, True])
def test_render_without_last_contributors(gpu, oracle, depth):
    """The blending variants that do not track the last contributor (its output not requested)
    give the same images."""
    w = synthetic.config(1, n=20_000, cameras=2)
    cam = w.cameras[-1]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, w.gaussians.sh_degree, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(w.gaussians, cam, t, opts)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    out = gpu.RenderOutputs.for_camera(cam, 0, include_depth=depth, include_last_contributing_indices=False)
    buf = gpu.RenderBuffers(len(g), t, 0)
    gpu.render_(out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    assert out.last is None
    np.testing.assert_array_equal(out.rgb.cpu().numpy(), r["rgb"])
    np.testing.assert_array_equal(out.T.cpu().numpy(), r["T"])
    if depth:
        np.testing.assert_array_equal(out.depth.cpu().numpy(), r["depth"])


def test_render_tiny_min_alpha_takes_range_checked_path(gpu, oracle):
    """min_alpha = 1e-38 puts the exponent cut below -87: every batch then leaves the
    hand-scheduled blending steps for the loop that evaluates exp_f with its range handling."""
    w = synthetic.config(0, n=3000)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 0, min_alpha=1e-38, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(w.gaussians, cam, t, opts)
    out, buf = _gpu_render(gpu, w.gaussians, cam, t, opts)
    assert r["nb_keys"] > 1000
    _assert_forward_equal(r, out, buf)


def test_render_only_huge_opacities_take_range_checked_path(gpu, oracle):
    """Render-only opacities above 1e38 make live exponents exceed 88 in their batches, which
    then use the range-checked loop; the other batches the fast steps."""
    from tdgs_amd import ply
    w = synthetic.config(0, n=3000)
    ro = ply.to_render_only(w.gaussians)
    ro.means_opacity[::97, 3] = np.float32(3e38)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(ro, cam, t, opts)
    out = gpu.RenderOutputs.for_camera(cam, 0, include_depth=True)
    buf = gpu.RenderBuffers(len(ro.means_opacity), t, 0, keep_flags=True)
    gpu.render_(out, gpu.RenderOnlyGaussiansVector.from_host(ro, 0), cam, t, opts, buf)
    torch.cuda.synchronize()
    assert r["nb_keys"] > 1000
    _assert_forward_equal(r, out, buf)


def test_render_filter_mode_and_antialiasing(gpu, oracle):
    w = synthetic.config(0, n=5000)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    from tdgs_amd import abi
    opts = host.RenderOptions.for_camera(cam, 0, clip_mode=abi.TDGS_CLIP_FILTER, use_antialiasing=True)
    r = oracle.render(w.gaussians, cam, t, opts)
    out, buf = _gpu_render(gpu, w.gaussians, cam, t, opts)
    _assert_forward_equal(r, out, buf)


def test_render_void_when_nothing_visible(gpu, oracle):
    g, cams = host.create_test_scene(sh_degree=0)
    g.means_opacity[:, 2] = -5.0  # everything behind the camera
    cam = cams[0]
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.25, 0.5, 0.75))
    t = host.Tiling.for_camera(cam, 16, 16)
    out, buf = _gpu_render(gpu, g, cam, t, opts)
    assert buf.nb_fgaussians == 0
    rgb = out.rgb.cpu().numpy()
    np.testing.assert_array_equal(rgb[..., 0], 0.25)
    np.testing.assert_array_equal(rgb[..., 2], 0.75)
    assert np.all(out.T.cpu().numpy() == 1) and np.all(out.last.cpu().numpy() == 0)
    assert np.all(np.isinf(out.depth.cpu().numpy()))


def test_blend_evaluation_counts(gpu):
    """The instrumentation replay (roofline FLOP counts) on the cfg0 scene: evaluations >=
    those past the exponent cut >= contributing ones >= pixels with a last contributor."""
    import ctypes as C
    w = synthetic.config(0, n=5000)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 0)
    out, buf = _gpu_render(gpu, w.gaussians, cam, t, opts)
    ev = torch.zeros(3, dtype=torch.int64, device="cuda")
    gpu.check(gpu.lib().tdgs_blend_evaluations(gpu.stream_ptr(0), C.byref(cam.to_c()), C.byref(t.to_c()),
                                               C.byref(opts.to_c()), C.byref(buf.struct()),
                                               C.c_int64(buf.nb_keys), C.c_void_p(ev.data_ptr())))
    e, live, contrib = ev.cpu().tolist()
    covered = int((out.last.cpu().numpy() > 0).sum())
    assert e >= live >= contrib >= covered > 0
