"""Scripts.render / Scripts.train host logic (scripts/render.jl, scripts/train.jl), on the CPU:
reading an undistorted COLMAP text model (cameras, poses, images, point cloud), the initial
Gaussians of MutableTrainableGaussiansVector(points, colours) (gaussians.jl:596-633) against
closed forms, the validation split of scripts/train.jl:72-84, the model and camera render.jl
picks for an output directory, and the error for an input without sparse-txt."""
import math
import os

import numpy as np
import pytest

from tdgs_amd import host, ply, scripts

f32 = np.float32


def _write_png(path, rgb_hw3):
    from PIL import Image
    Image.fromarray(rgb_hw3.astype(np.uint8), mode="RGB").save(path)


def _colmap_dir(tmp_path, w=8, h=6):
    d = tmp_path / "undistorted"
    (d / "sparse-txt").mkdir(parents=True)
    (d / "images").mkdir()
    (d / "sparse-txt" / "cameras.txt").write_text(
        "# Camera list with one line of data per camera:\n"
        "#   CAMERA_ID, MODEL, WIDTH, HEIGHT, PARAMS[]\n"
        "# Number of cameras: 1\n"
        f"1 PINHOLE {w} {h} 10.5 11.25 4.0 2.5\n")
    # two images: the identity pose at t = (1, 2, 3), and a quarter turn about z
    c, s = math.cos(math.pi / 4), math.sin(math.pi / 4)
    (d / "sparse-txt" / "images.txt").write_text(
        "# Image list with two lines of data per image:\n"
        "#   IMAGE_ID, QW, QX, QY, QZ, TX, TY, TZ, CAMERA_ID, NAME\n"
        "#   POINTS2D[] as (X, Y, POINT3D_ID)\n"
        "# Number of images: 2, mean observations per image: 1\n"
        "1 1 0 0 0 1 2 3 1 a.png\n"
        "1.0 2.0 -1\n"
        f"2 {c} 0 0 {s} 0 0 4 1 b.png\n"
        "3.0 4.0 -1\n")
    (d / "sparse-txt" / "points3D.txt").write_text(
        "# 3D point list with one line of data per point:\n"
        "#   POINT3D_ID, X, Y, Z, R, G, B, ERROR, TRACK[] as (IMAGE_ID, POINT2D_IDX)\n"
        "# Number of points: 5, mean track length: 1\n"
        + "".join(f"{k + 1} {float(k)} 0 0 {10 * k} {255 - k} {k} 0.5 1 0\n" for k in range(5)))
    rng = np.random.default_rng(1)
    imgs = {}
    for name in ("a.png", "b.png"):
        px = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
        _write_png(d / "images" / name, px)
        imgs[name] = px
    return d, imgs


def test_read_colmap_text_model(tmp_path):
    d, imgs = _colmap_dir(tmp_path)
    cwis, points, colors = scripts.read_colmap_text_model(str(d))
    assert [c.name for c in cwis] == ["a.png", "b.png"]
    cam = cwis[0].camera
    assert (cam.width, cam.height) == (8, 6)
    assert (float(cam.fx), float(cam.fy), float(cam.ppx), float(cam.ppy), float(cam.skew)) == (10.5, 11.25, 4.0, 2.5, 0.0)
    assert float(cam.near_z) == float(f32(host.DEFAULT_NEAR)) and math.isinf(float(cam.far_z))
    # world-to-camera (I, t): the camera sits at -t
    np.testing.assert_array_equal(cam.R_c2w, np.eye(3, dtype=f32))
    np.testing.assert_array_equal(cam.t_c2w, f32([-1, -2, -3]))
    # a quarter turn about z (world to camera): R_c2w is its transpose, the position -R_c2w t
    cam2 = cwis[1].camera
    np.testing.assert_allclose(cam2.R_c2w, [[0, 1, 0], [-1, 0, 0], [0, 0, 1]], atol=1e-6)
    np.testing.assert_allclose(cam2.t_c2w, [0, 0, -4], atol=1e-6)
    # images: (w, h, 3) = the reference's 3 x h x w, values byte / 255
    for cwi in cwis:
        px = imgs[cwi.name]
        assert cwi.image.shape == (8, 6, 3) and cwi.image.dtype == np.float32
        np.testing.assert_array_equal(cwi.image, (px.astype(f32) / f32(255)).transpose(1, 0, 2))
    np.testing.assert_array_equal(points, f32([[k, 0, 0] for k in range(5)]))
    np.testing.assert_array_equal(colors, f32([[10 * k, 255 - k, k] for k in range(5)]) / f32(255))


def test_gaussians_from_point_cloud_closed_form():
    # points on a line, 1 apart: the 3 nearest other points of x = 0 are at 1, 2, 3 (mean 2),
    # of x = 2 at 1, 1, 2 (mean 4/3)
    pts = f32([[k, 0, 0] for k in range(5)])
    cols = f32([[0.5, 0.0, 1.0]] * 5)
    g = scripts.gaussians_from_point_cloud(pts, cols)
    want = np.log(f32([2, 4 / 3, 4 / 3, 4 / 3, 2]))
    np.testing.assert_allclose(g.scaling, np.repeat(want[:, None], 3, axis=1), rtol=1e-6)
    np.testing.assert_array_equal(g.means_opacity[:, :3], pts)
    sig = 1 / (1 + np.exp(-g.means_opacity[:, 3].astype(np.float64)))
    np.testing.assert_allclose(sig, 0.1, rtol=1e-6)
    np.testing.assert_array_equal(g.rotation, np.tile(f32([1, 0, 0, 0]), (5, 1)))
    assert g.sh.shape == (5, 3, 1) and g.sh_degree == 0
    # colour = C0 * dc + 0.5 (sh.jl:38-44 at degree 0) gives back the point colours
    np.testing.assert_allclose(g.sh[:, :, 0] * host.SH_C0 + 0.5, cols, atol=1e-6)


@pytest.mark.parametrize("n,ratio,want", [(10, 0.0, []), (10, 0.2, [5, 10]), (10, 0.25, [5, 10]),
                                          (7, 0.3, [4]), (9, 1 / 3, [3, 6, 9]), (4, 1.0, [1, 2, 3, 4])])
def test_validation_camera_ids(n, ratio, want):
    assert scripts.validation_camera_ids(n, ratio) == want


def test_random_validation_camera_ids():
    ids = scripts.validation_camera_ids(20, 0.25, random_validation_cameras=True, rng=np.random.default_rng(3))
    assert len(ids) == 5 and len(set(ids)) == 5 and all(1 <= i <= 20 for i in ids)


def test_resolve_model(tmp_path):
    out = tmp_path / "out"
    for it in (7000, 30000, 500):
        (out / "point_cloud" / f"iteration_{it}").mkdir(parents=True)
    cam = host.look_at_camera(64, 48, 60.0, (0.0, 1.0, -3.0))
    ply.save_cameras_json(str(out / "cameras.json"), [cam])
    path, c = scripts.resolve_model(str(out))
    assert path.endswith(os.path.join("iteration_30000", "point_cloud.ply"))
    assert (c.width, c.height) == (64, 48)
    np.testing.assert_array_equal(c.t_c2w, cam.t_c2w)
    path, _ = scripts.resolve_model(str(out), iterations=500)
    assert path.endswith(os.path.join("iteration_500", "point_cloud.ply"))
    # a .ply path: the default camera of render.jl, 1280 x 720 with a 90 degree field of view
    path, c = scripts.resolve_model(str(tmp_path / "model.ply"))
    assert path.endswith("model.ply") and (c.width, c.height) == (1280, 720)
    assert float(c.fx) == float(host.fov_deg_to_focal_length(90.0, 1280))
    np.testing.assert_array_equal(c.R_c2w, np.eye(3, dtype=f32))


def test_train_needs_sparse_txt(tmp_path):
    with pytest.raises(FileNotFoundError, match="sparse-txt"):
        scripts.train(str(tmp_path), str(tmp_path / "out"))


def test_image_npy_and_png_agree(tmp_path):
    rng = np.random.default_rng(2)
    px = rng.integers(0, 256, (5, 7, 3), dtype=np.uint8)
    _write_png(tmp_path / "x.png", px)
    a = scripts.load_image(str(tmp_path / "x.png"))
    np.save(tmp_path / "x.npy", a)
    np.testing.assert_array_equal(scripts.load_image(str(tmp_path / "x.npy")), a)
    assert a.shape == (7, 5, 3)
