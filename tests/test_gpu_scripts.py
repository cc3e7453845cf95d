"""Scripts.train and Scripts.render (scripts/train.jl:43-197, scripts/render.jl:17-58) end to
end on the GPU, through the C-ABI.

A small scene is rendered from 8 orbit cameras into 8-bit PNG ground-truth images, written
with its camera poses and a noisy colored point cloud as an undistorted COLMAP text model.
train() then initialises Gaussians from the point cloud and trains 300 iterations with a
25% validation split, losses every 100 iterations and snapshots at 100 and 300. Checked: the
output layout (cameras.json with the input poses, point_cloud/iteration_<n>/point_cloud.ply),
the loop's iteration count, finite losses that fall on both splits, and render() of the
output directory: the model the last snapshot holds and the first camera of cameras.json,
bit-exact against the oracle's render of the same render-only model."""
import numpy as np
import pytest
import torch

from tdgs_amd import host, ply, scripts, synthetic, training

pytestmark = pytest.mark.gpu

f32 = np.float32


def _quat_wxyz(R):
    from scipy.spatial.transform import Rotation
    x, y, z, w = Rotation.from_matrix(np.asarray(R, dtype=np.float64)).as_quat()
    return w, x, y, z


def _write_colmap(gpu, d, w=160, h=120, ncam=8, seed=5):
    from PIL import Image
    rng = np.random.default_rng(seed)
    truth = synthetic.config(0).gaussians            # the reference test scene's size class
    (d / "sparse-txt").mkdir(parents=True)
    (d / "images").mkdir()
    g = gpu.TrainableGaussiansVector.from_host(truth, 0)
    lines = ["# Image list", "# IMAGE_ID, QW, QX, QY, QZ, TX, TY, TZ, CAMERA_ID, NAME", "# POINTS2D", "# n"]
    cams = []
    for k in range(ncam):
        a = 2 * np.pi * k / ncam
        cam = host.look_at_camera(w, h, 60.0, (3.5 * np.sin(a), -0.8, -3.5 * np.cos(a)))
        cams.append(cam)
        t = host.Tiling.for_camera(cam, 16, 16)
        opts = host.RenderOptions.for_camera(cam, truth.sh_degree)
        out = gpu.RenderOutputs.for_camera(cam, 0)
        gpu.render_(out, g, cam, t, opts, gpu.RenderBuffers(len(g), t, 0))
        px = np.clip(np.rint(out.rgb.cpu().numpy() * 255), 0, 255).astype(np.uint8).transpose(1, 0, 2)
        Image.fromarray(px, mode="RGB").save(d / "images" / f"img{k:02d}.png")
        R_w2c = cam.R_c2w.T.astype(np.float64)
        t_w2c = -R_w2c @ cam.t_c2w.astype(np.float64)
        vals = " ".join(repr(float(v)) for v in (*_quat_wxyz(R_w2c), *t_w2c))
        lines.append(f"{k + 1} {vals} 1 img{k:02d}.png")
        lines.append("")
    (d / "sparse-txt" / "images.txt").write_text("\n".join(lines) + "\n")
    c0 = cams[0]
    (d / "sparse-txt" / "cameras.txt").write_text(
        f"# cameras\n1 PINHOLE {w} {h} {float(c0.fx)!r} {float(c0.fy)!r} {float(c0.ppx)!r} {float(c0.ppy)!r}\n")
    npts = 4000
    idx = rng.choice(len(truth.means_opacity), npts, replace=False)
    pts = truth.means_opacity[idx, :3] + rng.normal(0, 0.02, (npts, 3)).astype(f32)
    cols = np.clip(truth.sh[idx, :, 0] * host.SH_C0 + 0.5, 0, 1)
    body = "".join(f"{i + 1} {p[0]!r} {p[1]!r} {p[2]!r} {int(round(c[0] * 255))} {int(round(c[1] * 255))} "
                   f"{int(round(c[2] * 255))} 0.1 1 0\n" for i, (p, c) in enumerate(zip(pts.tolist(), cols.tolist())))
    (d / "sparse-txt" / "points3D.txt").write_text(f"# points\n# format\n# Number of points: {npts}, mean\n" + body)
    return cams


def test_train_then_render_output_dir(gpu, oracle, tmp_path):
    inp, outd = tmp_path / "undistorted", tmp_path / "out"
    cams = _write_colmap(gpu, inp)
    logs = []
    res = scripts.train(str(inp), str(outd),
                        training_options_from_scene=lambda r: training.TrainingOptions.for_scene(r, nb_iterations=300),
                        evaluation_iterations=100, save_iterations=(100, 300), validation_ratio=0.25,
                        log=logs.append)
    tr = res.trainer
    assert tr.iteration_nb == 301                    # while iteration_nb <= nb_iterations
    assert [it for it, _ in res.saved] == [100, 300]
    for it in (100, 300):
        assert (outd / "point_cloud" / f"iteration_{it}" / "point_cloud.ply").exists()
    # cameras.json holds every input camera (training and validation)
    saved = ply.load_cameras_from_json(str(outd / "cameras.json"))
    assert len(saved) == len(cams)
    for a, b in zip(saved, cams):
        np.testing.assert_allclose(a.t_c2w, b.t_c2w, atol=1e-5)
        np.testing.assert_allclose(a.R_c2w, b.R_c2w, atol=1e-5)
    # losses at iterations 0, 100, 200, 300 on both splits (validation: cameras 4 and 8)
    assert len(tr.cameras) == 6
    by = {(it, kind): (mse, mae, dssim) for it, kind, mse, mae, dssim in res.losses}
    assert sorted(by) == sorted((it, k) for it in (0, 100, 200, 300) for k in ("Training", "Validation"))
    assert all(np.isfinite(v).all() for v in by.values())
    for kind in ("Training", "Validation"):
        assert by[(300, kind)][0] < 0.9 * by[(0, kind)][0], (kind, by)   # MSE falls
    assert any("Saved Gaussians model after 300 iterations" in s for s in logs)

    # render(output_dir): the last snapshot from the first camera of cameras.json
    out = scripts.render(str(outd), output_png=str(tmp_path / "view.png"))
    torch.cuda.synchronize()
    ro = ply.read_render_only_ply(str(outd / "point_cloud" / "iteration_300" / "point_cloud.ply"))
    cam = saved[0]
    t = host.Tiling.for_camera(cam)
    r = oracle.render(ro, cam, t, host.RenderOptions.for_camera(cam, ro.sh_degree), depth=False, last=False)
    np.testing.assert_array_equal(out.rgb.cpu().numpy(), r["rgb"])
    np.testing.assert_array_equal(out.T.cpu().numpy(), r["T"])
    from PIL import Image
    with Image.open(tmp_path / "view.png") as im:
        assert im.size == (cam.width, cam.height)
