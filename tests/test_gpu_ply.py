"""GPU rendering of models read from 3DGS .ply files (RenderOnlyGaussiansVector(ply_path),
src/gaussians.jl:741-762) against the CPU oracle, through the C-ABI."""
import numpy as np
import pytest
import torch

from tdgs_amd import host, ply, synthetic
from test_gpu_forward import _assert_forward_equal

pytestmark = pytest.mark.gpu


def _render(core, g, cam, t, opts):
    out = core.RenderOutputs.for_camera(cam, 0, include_depth=True)
    buf = core.RenderBuffers(len(g), t, 0, keep_flags=True)
    core.render_(out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    return out, buf


@pytest.mark.parametrize("cfg,n,aa", [(0, None, False), (1, 20_000, False), (1, 20_000, True)])
def test_render_only_from_ply_bit_exact(gpu, oracle, tmp_path, cfg, n, aa):
    w = synthetic.config(cfg, n=n, cameras=2)
    p = tmp_path / "model.ply"
    ply.save_3dgs_ply(p, w.gaussians)
    ro = ply.read_render_only_ply(p)
    cam = w.cameras[-1]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, ro.sh_degree, background_color=(0.1, 0.2, 0.3),
                                         use_antialiasing=aa)
    r = oracle.render(ro, cam, t, opts)
    out, buf = _render(gpu, gpu.RenderOnlyGaussiansVector.from_host(ro, 0), cam, t, opts)
    assert r["nb_keys"] > 1000
    _assert_forward_equal(r, out, buf)


def test_render_only_close_to_trainable(gpu, tmp_path):
    """The same model rendered from its features and from the activated opacities and 3D
    covariances: the two projections differ only in float32 rounding."""
    w = synthetic.config(1, n=20_000, cameras=2)
    p = tmp_path / "model.ply"
    ply.save_3dgs_ply(p, w.gaussians)
    g = ply.read_3dgs_ply(p)
    cam = w.cameras[-1]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, g.sh_degree)
    a, _ = _render(gpu, gpu.TrainableGaussiansVector.from_host(g, 0), cam, t, opts)
    b, _ = _render(gpu, gpu.RenderOnlyGaussiansVector.from_host(ply.to_render_only(g), 0), cam, t, opts)
    d = np.abs(a.rgb.cpu().numpy() - b.rgb.cpu().numpy())
    assert d.mean() < 1e-5 and np.quantile(d, 0.999) < 1e-4
