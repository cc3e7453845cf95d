"""GPU parity of backward! against the CPU oracle, through the C-ABI.

The forward pass is bit-exact, so both sides replay identical lists; only the order of the
float atomics differs, hence the tolerance: relative L2 error <= 1e-3 per gradient array
The reference goldens are also checked directly on the GPU
result (rtol 1e-2 per component, test/backward_core.jl:149-155).
"""
import numpy as np
import pytest
import torch

from conftest import golden, stacked_faint_gaussians
from tdgs_amd import host, synthetic

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3
ARRAYS = ["mean3d", "opacity_feature", "scaling_features", "rotation_features", "sh"]


def rel_l2(a, b):
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    nb = np.linalg.norm(b)
    return np.linalg.norm(a - b) / nb if nb > 0 else np.linalg.norm(a)


def _run(core, orc, g_host, cam, t, opts, rgb_grad_fn):
    ref = orc.render(g_host, cam, t, opts)
    g = core.TrainableGaussiansVector.from_host(g_host, 0)
    out = core.RenderOutputs.for_camera(cam, 0)
    buf = core.RenderBuffers(len(g), t, 0)
    core.render_(out, g, cam, t, opts, buf)
    rgb = out.rgb
    grad = rgb_grad_fn(rgb).float().contiguous()
    fg = core.FilteredGaussiansGradientsVector(buf.capacity, g.sh_degree, 0)
    core.backward_(fg, grad, out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    b = orc.backward(g_host, cam, t, opts, ref, grad.cpu().numpy())
    nf = buf.nb_fgaussians
    assert nf == ref["nb_fgaussians"]
    got = {"grads2d": fg.grads2d[:nf], "mean3d": fg.mean3d[:nf], "opacity_feature": fg.opacity_feature[:nf],
           "scaling_features": fg.scaling_features[:nf], "rotation_features": fg.rotation_features[:nf],
           "sh": fg.sh[:nf]}
    return {k: v.cpu().numpy() for k, v in got.items()}, b


def _l1_grad(rgb):
    return torch.where(rgb > 0.5, 1.0, -1.0) / rgb.numel()


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_backward_test_scene(gpu, oracle, deg):
    g, cams = host.create_test_scene(sh_degree=deg)
    cam = cams[0]
    opts = host.RenderOptions.for_camera(cam, deg)
    t = host.Tiling.for_camera(cam, 16, 16)
    got, ref = _run(gpu, oracle, g, cam, t, opts, _l1_grad)
    for k in ["grads2d"] + ARRAYS:
        assert rel_l2(got[k], ref[k]) <= REL_L2, k
    if deg in (0, 3):
        gold = golden("backward_test_scene.json")["grads"][str(deg)]
        for i in range(3):
            for name, key, sl in (("means2d", "grads2d", slice(0, 2)), ("scaling_features", "scaling_features", None),
                                  ("opacity_features", "opacity_feature", None)):
                v = got[key][i] if sl is None else got[key][i, sl]
                r = np.asarray(gold[name][i], np.float64)
                np.testing.assert_allclose(np.atleast_1d(v), np.atleast_1d(r), rtol=1e-2)


AA = {"use_antialiasing": True}
FILTER = {"clip_mode": 1}   # TDGS_CLIP_FILTER (BoundaryFilter)


@pytest.mark.parametrize("cfg,n,tile,exact,extra", [
    (1, 20_000, (16, 16), False, {}), (1, 20_000, (16, 16), True, {}),
    (2, 60_000, (16, 32), False, {}), (0, None, (16, 16), False, {}),
    (0, None, (32, 32), False, {}), (0, None, (8, 8), False, {}),
    # 192 pixels: one wavefront of four-pixel lanes whose fourth pixel slot lies past the tile
    (0, None, (24, 8), False, {}), (0, None, (8, 24), False, {}),
    # antialiasing (forward_core.jl:450-462, backward_core.jl:331-341, 480) and the
    # BoundaryFilter clip mode (forward_core.jl:343, backward_core.jl:373-381)
    (1, 20_000, (16, 16), False, AA), (2, 60_000, (16, 16), False, AA),
    (1, 20_000, (16, 16), False, FILTER), (2, 60_000, (16, 16), False, FILTER),
    (2, 60_000, (16, 16), True, {**AA, **FILTER}),
    (2, 60_000, (16, 16), False, {**AA, "exact_aa_gradient": True})])
def test_backward_synthetic(gpu, oracle, cfg, n, tile, exact, extra):
    w = synthetic.config(cfg, n=n, cameras=2)
    cam = w.cameras[-1]
    t = host.Tiling.for_camera(cam, *tile)
    opts = host.RenderOptions.for_camera(cam, w.gaussians.sh_degree, background_color=(0.2, 0.1, 0.3),
                                         exact_sh_jacobian=exact, **extra)
    gen = torch.Generator(device="cuda").manual_seed(7)

    def rand_grad(rgb):
        return (torch.rand(rgb.shape, generator=gen, device=rgb.device) - 0.5) * 1e-3

    got, ref = _run(gpu, oracle, w.gaussians, cam, t, opts, rand_grad)
    for k in ["grads2d"] + ARRAYS:
        assert rel_l2(got[k], ref[k]) <= REL_L2, (k, rel_l2(got[k], ref[k]))


@pytest.mark.parametrize("deg", [0, 1, 2])
def test_backward_sh3_storage_at_lower_degrees(gpu, oracle, deg):
    """16-coefficient storage rendered at SH degrees 0-2 (training's degree schedule): the
    gradients match the oracle's, and the coefficients above the render degree get exactly 0."""
    w = synthetic.config(1, n=20_000, cameras=2)
    cam = w.cameras[-1]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, deg, background_color=(0.2, 0.1, 0.3))
    gen = torch.Generator(device="cuda").manual_seed(13)

    def rand_grad(rgb):
        return (torch.rand(rgb.shape, generator=gen, device=rgb.device) - 0.5) * 1e-3

    got, ref = _run(gpu, oracle, w.gaussians, cam, t, opts, rand_grad)
    for k in ["grads2d"] + ARRAYS:
        assert rel_l2(got[k], ref[k]) <= REL_L2, (k, rel_l2(got[k], ref[k]))
    hr = (deg + 1) ** 2
    assert got["sh"].shape[-1] == 16 and np.abs(got["sh"][..., :hr]).max() > 0
    assert np.all(got["sh"][..., hr:] == 0)


@pytest.mark.parametrize("size,tile", [(8, (8, 8)), (16, (16, 16)), (16, (32, 32))])
def test_backward_list_lengths_at_group_and_batch_ends(gpu, oracle, size, tile):
    """One-tile images whose list holds 1 to 5 records, or 1 to 3 records past a full group of
    four and past a full batch of 64, 256 or 1024 records; no pixel stops early, so the walk
    back from each pixel's last contributor visits every record."""
    from tdgs_amd.host import look_at_camera
    cam = look_at_camera(size, size, 60.0, (0.0, 0.0, -4.0))
    t = host.Tiling.for_camera(cam, *tile)
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.2, 0.1, 0.3))
    gen = torch.Generator(device="cuda").manual_seed(5)

    def rand_grad(rgb):
        return (torch.rand(rgb.shape, generator=gen, device=rgb.device) - 0.5) * 1e-3

    for k in (1, 2, 3, 5, 63, 65, 67, 255, 257, 259, 1023, 1025, 1027):
        got, ref = _run(gpu, oracle, stacked_faint_gaussians(k), cam, t, opts, rand_grad)
        for name in ["grads2d"] + ARRAYS:
            assert rel_l2(got[name], ref[name]) <= REL_L2, (k, name, rel_l2(got[name], ref[name]))


def test_backward_tiny_min_alpha_takes_range_checked_path(gpu, oracle):
    """min_alpha = 1e-38 gives per-record cuts below -87, so every batch of the backward
    blending uses the range-checked loop."""
    w = synthetic.config(0, n=3000)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 0, min_alpha=1e-38, background_color=(0.2, 0.1, 0.3))
    gen = torch.Generator(device="cuda").manual_seed(11)

    def rand_grad(rgb):
        return (torch.rand(rgb.shape, generator=gen, device=rgb.device) - 0.5) * 1e-3

    got, ref = _run(gpu, oracle, w.gaussians, cam, t, opts, rand_grad)
    for k in ["grads2d"] + ARRAYS:
        assert rel_l2(got[k], ref[k]) <= REL_L2, (k, rel_l2(got[k], ref[k]))
