"""Scripts.render and Scripts.train (scripts/render.jl, scripts/train.jl) over libtdgs.so.

render(path) loads a 3DGS model (a .ply file, or a training output directory) and renders it
from the first camera of the output directory's cameras.json, or from the reference's default
camera; the interactive viewer loop of scripts/render.jl:52-56 is replaced by returning the
image and optionally writing it as a PNG (the viewer is not part of this library).

train(input_dir, output_dir) is the training loop of scripts/train.jl:43-197 on a COLMAP
directory that has been undistorted and converted to text (sparse-txt/{cameras,images,
points3D}.txt and images/): cameras and ground-truth images, a Gaussian model initialised from
the sparse point cloud, an optional validation split, losses every `evaluation_iterations`
iterations and PLY snapshots at `save_iterations`, in the reference's output layout
(cameras.json, point_cloud/iteration_<n>/point_cloud.ply). Running COLMAP itself
(process_colmap, scripts/train.jl:200-318) needs the colmap program and is not done here: a
directory without sparse-txt is rejected with an error that says so.
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass, field

import numpy as np
import torch

from . import host, ply
from .core import RenderBuffers, RenderOnlyGaussiansVector, RenderOutputs, TrainableGaussiansVector, render_
from .core import image_to_rgb8
from .host import DEFAULT_FAR, DEFAULT_NEAR, HostGaussians, PinholeCamera, RenderOptions, Tiling
from .training import Trainer, TrainingOptions, loss_grad_

f32 = np.float32


# ------------------------------------------------------------------------------------
# Images
# ------------------------------------------------------------------------------------

def load_image(path) -> np.ndarray:
    """EagerImageLoader's array (cameras.jl:845-852, 1023-1080): the image as float32 values
    in [0, 1], in the reference's 3 x h x w layout, i.e. a (w, h, 3) array here. PNG, JPEG and
    the other formats Pillow reads, or a .npy file holding such an array."""
    if str(path).endswith(".npy"):
        a = np.load(path, allow_pickle=False)
        if a.ndim != 3 or a.shape[2] != 3:
            raise ValueError(f"{path}: expected a (w, h, 3) array, got {a.shape}")
        return np.ascontiguousarray(a.astype(f32))
    from PIL import Image
    with Image.open(path) as im:
        rgb = np.asarray(im.convert("RGB"), dtype=np.uint8)   # (h, w, 3)
    return np.ascontiguousarray((rgb.astype(f32) / f32(255)).transpose(1, 0, 2))


def save_image_png(path, rgb8: np.ndarray):
    """Write an (h, w, 3) uint8 image as a PNG."""
    from PIL import Image
    Image.fromarray(np.ascontiguousarray(rgb8), mode="RGB").save(path)


# ------------------------------------------------------------------------------------
# render
# ------------------------------------------------------------------------------------

def default_camera(width=1280, height=720, fov_deg=90.0) -> PinholeCamera:
    """The camera of scripts/render.jl:40-46: 1280 x 720, 90 degrees horizontal field of view,
    at the origin with the identity rotation."""
    f = host.fov_deg_to_focal_length(fov_deg, width)
    return PinholeCamera.from_focal(width, height, f, np.eye(3, dtype=f32), np.zeros(3, dtype=f32))


def resolve_model(path, iterations=None):
    """The .ply file and camera scripts/render.jl:17-39 use for `path`: a .ply file with the
    default camera, or a training output directory's point_cloud/iteration_<n>/point_cloud.ply
    (n = `iterations`, else the largest saved) with the first camera of its cameras.json."""
    if os.path.isdir(path):
        if iterations is None:
            its = [int(d[len("iteration_"):]) for d in os.listdir(os.path.join(path, "point_cloud"))
                   if d.startswith("iteration_")]
            if not its:
                raise FileNotFoundError(f"{path}/point_cloud holds no iteration_<n> directory")
            iterations = max(its)
        ply_path = os.path.join(path, "point_cloud", f"iteration_{iterations}", "point_cloud.ply")
        camera = ply.load_cameras_from_json(os.path.join(path, "cameras.json"))[0]
        return ply_path, camera
    return path, default_camera()


def render(path, iterations=None, camera: PinholeCamera | None = None, output_png: str | None = None,
           tile_size=None, device=0) -> RenderOutputs:
    """scripts/render.jl:17-58 without the viewer: renders the render-only model of `path`
    (RenderOnlyGaussiansVector(ply_path), gaussians.jl:741-762) once, from `camera` or the
    camera resolve_model picks, at the model's SH degree, and writes the viewer's UInt8 image
    to `output_png` when given. Returns the RenderOutputs (rgb and transmittance)."""
    ply_path, cam = resolve_model(path, iterations)
    if camera is not None:
        cam = camera
    g = RenderOnlyGaussiansVector.from_host(ply.read_render_only_ply(ply_path), device)
    tiling = Tiling.for_camera(cam, *(tile_size or (None, None)))
    opts = RenderOptions.for_camera(cam, g.sh_degree)
    out = RenderOutputs.for_camera(cam, device, include_rgb=True, include_transmittance=True,
                                   include_depth=False, include_last_contributing_indices=False)
    buf = RenderBuffers(len(g), tiling, device)
    render_(out, g, cam, tiling, opts, buf)
    if output_png:
        save_image_png(output_png, image_to_rgb8(out.rgb).cpu().numpy())
    return out


# ------------------------------------------------------------------------------------
# COLMAP text model -> cameras, images, initial Gaussians
# ------------------------------------------------------------------------------------

@dataclass
class CameraWithImage:
    """CameraWithImage (cameras.jl:1090-1120) with an eagerly loaded image."""
    camera: PinholeCamera
    image: np.ndarray          # (w, h, 3) float32
    name: str = ""


def _colmap_camera(width, height, fx, fy, cx, cy, q_w2c, t_w2c) -> PinholeCamera:
    """PinholeCamera(width, height, fx, fy, 0, cx, cy, near, far, R_w2c, t_w2c; world-to-camera
    orders) (cameras.jl:120-178): R_c2w = R_w2c^T and position = -R_w2c^T t_w2c, in float32."""
    R_w2c = ply.quaternion_to_rotation_matrix(np.asarray([q_w2c], dtype=f32))[0]
    R_c2w = np.ascontiguousarray(R_w2c.T).astype(f32)
    t_c2w = (-host._mm(R_c2w, np.asarray(t_w2c, dtype=f32).reshape(3, 1))).reshape(3).astype(f32)
    return PinholeCamera(int(width), int(height), f32(fx), f32(fy), f32(0), f32(cx), f32(cy), f32(DEFAULT_NEAR),
                         f32(DEFAULT_FAR), R_c2w, t_c2w)


def read_colmap_text_model(undistorted_dir):
    """processed_colmap_to_cameras_with_images_and_gaussians_model (scripts/train.jl:330-396),
    reading part: the PINHOLE intrinsics of the last line of sparse-txt/cameras.txt, one camera
    per image line of images.txt (odd lines after the four header lines: id, qw qx qy qz,
    tx ty tz, camera id, file name) with its image from images/, and the points and colours of
    points3D.txt. Returns (cameras_with_images, points (n, 3) float32, colours (n, 3) float32
    in [0, 1])."""
    txt = os.path.join(undistorted_dir, "sparse-txt")
    with open(os.path.join(txt, "cameras.txt")) as fh:
        lines = [ln for ln in fh.read().splitlines() if ln.strip()]
    cam_line = lines[-1].split()
    width, height = int(cam_line[2]), int(cam_line[3])
    fx, fy, cx, cy = (float(f32(v)) for v in cam_line[4:8])
    cwis = []
    with open(os.path.join(txt, "images.txt")) as fh:
        for idx, line in enumerate(fh.read().splitlines(), start=1):
            if idx < 5 or idx % 2 == 0:
                continue
            parts = line.split()
            if len(parts) < 10:
                continue
            q = [float(f32(v)) for v in parts[1:5]]
            t = [float(f32(v)) for v in parts[5:8]]
            name = parts[9]
            cam = _colmap_camera(width, height, fx, fy, cx, cy, q, t)
            cwis.append(CameraWithImage(cam, load_image(os.path.join(undistorted_dir, "images", name)), name))
    pts, cols = [], []
    with open(os.path.join(txt, "points3D.txt")) as fh:
        for idx, line in enumerate(fh.read().splitlines(), start=1):
            if idx < 4 or not line.strip():
                continue
            parts = line.split()
            pts.append([float(v) for v in parts[1:4]])
            cols.append([int(v) for v in parts[4:7]])
    points = np.asarray(pts, dtype=f32).reshape(-1, 3)
    colors = (np.asarray(cols, dtype=np.uint8).reshape(-1, 3).astype(f32) / f32(255)).astype(f32)
    return cwis, points, colors


def gaussians_from_point_cloud(points: np.ndarray, colors: np.ndarray) -> HostGaussians:
    """MutableTrainableGaussiansVector(points, rgb_colors) (gaussians.jl:596-633): means at the
    points, opacity logit(0.1), SH degree 0 with the DC coefficient (rgb - 0.5) / C0, identity
    rotations and isotropic log-scales log(mean distance to the 3 nearest other points) (the 4
    nearest neighbours including the point itself, summed and divided by 3)."""
    from scipy.spatial import cKDTree
    points = np.ascontiguousarray(points, dtype=f32)
    n = points.shape[0]
    k = min(4, n)
    d, _ = cKDTree(points.astype(np.float64)).query(points.astype(np.float64), k=k)
    d = np.asarray(d, dtype=np.float64).reshape(n, k)
    mean_d = (d.sum(axis=1) / 3).astype(f32)
    log_s = np.log(mean_d).astype(f32)
    mo = np.empty((n, 4), dtype=f32)
    mo[:, :3] = points
    mo[:, 3] = host.logit32(f32(0.1))
    scaling = np.repeat(log_s[:, None], 3, axis=1).astype(f32)
    rotation = np.zeros((n, 4), dtype=f32)
    rotation[:, 0] = 1
    sh = host.color_to_sh_coeffs_dc(np.asarray(colors, dtype=f32)).astype(f32).reshape(n, 3, 1)
    return HostGaussians(mo, scaling, rotation, sh)


def validation_camera_ids(nb_cameras, validation_ratio, random_validation_cameras=False, rng=None):
    """The 1-based validation camera ids of scripts/train.jl:72-84: floor(n ratio) cameras,
    every cld(n, k)-th one (step, 2 step, ...), or a random selection."""
    k = int(math.floor(nb_cameras * validation_ratio))
    if k == 0:
        return []
    if random_validation_cameras:
        rng = rng or np.random.default_rng()
        return sorted(int(i) + 1 for i in rng.permutation(nb_cameras)[:k])
    step = -(-nb_cameras // k)
    return list(range(step, nb_cameras + 1, step))


# ------------------------------------------------------------------------------------
# train
# ------------------------------------------------------------------------------------

@dataclass
class TrainResult:
    trainer: Trainer
    losses: list = field(default_factory=list)     # (iteration, split, mse, mae, dssim)
    saved: list = field(default_factory=list)      # (iteration, ply path)


def _should(iteration_nb, spec):
    if isinstance(spec, int):
        return spec > 0 and iteration_nb % spec == 0
    return iteration_nb in spec


def evaluate_losses(trainer: Trainer, cameras_with_images, tiling):
    """compute_losses of scripts/train.jl:119-130 averaged over the cameras: MSE, MAE and
    DSSIM (1 - mean SSIM, the training loss's SSIM) of the current model's renders."""
    if not cameras_with_images:
        return None
    out, buf = trainer.render_outputs, trainer.render_buffers
    sums = torch.zeros(2, dtype=torch.float64, device=trainer.device)
    grad = torch.empty_like(out.rgb)
    acc = np.zeros(3)
    for cwi in cameras_with_images:
        gt = torch.from_numpy(cwi.image).to(trainer.device)
        render_(out, trainer.gaussians, cwi.camera, tiling, trainer.render_options, buf)
        sums.zero_()
        loss_grad_(out.rgb, gt, grad, 1.0, sums, trainer.loss_temp)
        n = out.rgb.numel()
        s = sums.cpu().numpy()
        mse = float(((out.rgb - gt) ** 2).sum().item()) / n
        acc += (mse, s[0] / n, 1.0 - s[1] / n)
    return tuple(acc / len(cameras_with_images))


def train(input_dir, output_dir, render_options_from_camera=None, training_options_from_scene=None,
          evaluation_iterations=1000, save_iterations=(7000, 30_000), validation_ratio=0.0,
          random_validation_cameras=False, seed=0, device=0, log=print) -> TrainResult:
    """train (scripts/train.jl:43-197) without the viewer.

    render_options_from_camera(camera) -> RenderOptions (default: SH degree 0, the trainer
    raises it) and training_options_from_scene(scene_radius) -> TrainingOptions (default:
    TrainingOptions.for_scene) play the roles of the reference's keyword functions (the scene
    is represented by its radius, scene.jl:64-73, which is all TrainingOptions(scene) uses).
    As in the reference, losses are evaluated before the step whenever iteration_nb is a
    multiple of evaluation_iterations (or in it, for a collection), the model is saved after
    the step whose iteration_nb is in save_iterations (or a multiple of it), and the loop runs
    while iteration_nb <= nb_iterations (nb_iterations + 1 steps)."""
    if not os.path.isdir(os.path.join(input_dir, "sparse-txt")):
        raise FileNotFoundError(
            f"{input_dir} has no sparse-txt directory: pass an undistorted COLMAP model converted to text "
            "(running COLMAP, process_colmap of scripts/train.jl, is not part of this library)")
    cwis, points, colors = read_colmap_text_model(input_dir)
    if not cwis:
        raise ValueError(f"{input_dir}: images.txt lists no images")
    os.makedirs(output_dir, exist_ok=True)
    ply.save_cameras_json(os.path.join(output_dir, "cameras.json"), [c.camera for c in cwis])

    rng = np.random.default_rng(seed)
    val_ids = validation_camera_ids(len(cwis), validation_ratio, random_validation_cameras, rng)
    train_ids = [i for i in range(1, len(cwis) + 1) if i not in set(val_ids)]
    train_cwis = [cwis[i - 1] for i in train_ids]
    val_cwis = [cwis[i - 1] for i in val_ids]
    train_cams = [c.camera for c in train_cwis]

    radius = host.scene_radius(train_cams)
    first = train_cams[0]
    render_options = (render_options_from_camera or (lambda c: RenderOptions.for_camera(c, 0)))(first)
    tiling = Tiling.for_camera(first)
    options = (training_options_from_scene or TrainingOptions.for_scene)(radius)
    g = TrainableGaussiansVector.from_host(gaussians_from_point_cloud(points, colors), device)
    trainer = Trainer(g, train_cams, [c.image for c in train_cwis], render_options, tiling, options, seed=seed,
                      device=device)
    result = TrainResult(trainer)
    while trainer.iteration_nb <= options.nb_iterations:
        if _should(trainer.iteration_nb, evaluation_iterations):
            trainer.finish_()   # the last step complete (re-run if its keys did not fit), errors raised
            log(f"Losses after iteration {trainer.iteration_nb}:")
            for kind, group in (("Training", train_cwis), ("Validation", val_cwis)):
                ev = evaluate_losses(trainer, group, tiling)
                if ev is None:
                    continue
                result.losses.append((trainer.iteration_nb, kind, *ev))
                log(f"  {kind}:\n    MSE (L2): {ev[0]}\n    MAE (L1): {ev[1]}\n    DSSIM:    {ev[2]}")
        trainer.training_step_()
        if _should(trainer.iteration_nb, save_iterations):
            trainer.finish_()
            d = os.path.join(output_dir, "point_cloud", f"iteration_{trainer.iteration_nb}")
            os.makedirs(d, exist_ok=True)
            path = os.path.join(d, "point_cloud.ply")
            ply.save_3dgs_ply(path, trainer.gaussians.to_host())
            result.saved.append((trainer.iteration_nb, path))
            log(f"Saved Gaussians model after {trainer.iteration_nb} iterations to {path}")
    trainer.finish_()
    if trainer.replayed_steps:
        log(f"{trainer.replayed_steps} device-count steps needed more keys than the key arrays held "
            "and were run again with host counts")
    torch.cuda.synchronize(trainer.device)
    return result
