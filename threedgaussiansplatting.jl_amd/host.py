"""Host-side value types of the render core: cameras, render options, tiling, the test scene.

These mirror the reference's constructors and compute every derived single-precision value
(the cached projection matrix, clip bounds in pixels, default thresholds) on the host with
float32 arithmetic, once, so the GPU library and the CPU oracle receive identical inputs.

Reference: src/cameras.jl (PinholeCamera :50-380, fov :534-562), src/forward_structs.jl
(Tiling :340-424, RenderOptions :579-665), src/image_coordinates.jl:71-76,136-137,
src/scene.jl (radius :49-73, create_test_scene :123-188), src/sh.jl:157-159.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import abi

f32 = np.float32

# src/forward_structs.jl:557-564
DEFAULT_MIN_ALPHA = 1 / 255
DEFAULT_MAX_ALPHA = 0.99
DEFAULT_MIN_TRANSMITTANCE = 0.0001
DEFAULT_DILATION_PX = 0.3
DEFAULT_CLIPPING_MARGIN_NC = 0.3
DEFAULT_MIN_AA_FACTOR = 0.0005
# src/cameras.jl:345-346
DEFAULT_NEAR = 0.2
DEFAULT_FAR = math.inf

SH_C0 = 0.28209479177387814


def _mm(A, B):
    """float32 matrix product summed left to right (StaticArrays' unrolled order)."""
    A = np.asarray(A, dtype=f32)
    B = np.asarray(B, dtype=f32)
    out = np.zeros((A.shape[0], B.shape[1]), dtype=f32)
    for i in range(A.shape[0]):
        for j in range(B.shape[1]):
            acc = f32(A[i, 0] * B[0, j])
            for k in range(1, A.shape[1]):
                acc = f32(acc + f32(A[i, k] * B[k, j]))
            out[i, j] = acc
    return out


def fov_to_focal_length(fov_rad, axis_size):
    """src/cameras.jl:534."""
    return axis_size / (2 * math.tan(fov_rad / 2))


def fov_deg_to_focal_length(fov_deg, axis_size, float32: bool = True):
    """src/cameras.jl:541-542; in float32 arithmetic as the reference does for Float32."""
    if float32:
        rad = f32(f32(fov_deg) * f32(math.pi / 180))
        t = f32(np.tan(f32(rad / f32(2))))
        return f32(f32(axis_size) / f32(f32(2) * t))
    return fov_to_focal_length(math.radians(fov_deg), axis_size)


@dataclass
class PinholeCamera:
    """PinholeCamera (src/cameras.jl:50-106): pose given camera-to-world."""
    width: int
    height: int
    fx: float
    fy: float
    skew: float
    ppx: float
    ppy: float
    near_z: float
    far_z: float
    R_c2w: np.ndarray
    t_c2w: np.ndarray
    P: np.ndarray = field(init=False)

    def __post_init__(self):
        self.R_c2w = np.asarray(self.R_c2w, dtype=f32).reshape(3, 3)
        self.t_c2w = np.asarray(self.t_c2w, dtype=f32).reshape(3)
        K = np.array([[self.fx, self.skew, self.ppx], [0, self.fy, self.ppy], [0, 0, 1]], dtype=f32)
        Rw = self.R_c2w.T.copy()
        tw = _mm(-Rw, self.t_c2w.reshape(3, 1)).reshape(3)
        self.P = _mm(K, np.concatenate([Rw, tw.reshape(3, 1)], axis=1))

    @classmethod
    def from_focal(cls, width, height, focal, R_c2w, t_c2w):
        """src/cameras.jl:363-380: square pixels, centred principal point, 3DGS clip planes."""
        return cls(width, height, f32(focal), f32(focal), f32(0), f32(width) / f32(2),
                   f32(height) / f32(2), f32(DEFAULT_NEAR), f32(DEFAULT_FAR), R_c2w, t_c2w)

    @property
    def position(self):
        return self.t_c2w

    def size(self):
        return (self.height, self.width)

    def to_c(self) -> abi.Camera:
        c = abi.Camera()
        c.width = int(self.width)
        c.height = int(self.height)
        for i, v in enumerate(self.P.reshape(-1)):
            c.P[i] = float(v)
        c.near_z = float(f32(self.near_z))
        c.far_z = float(f32(self.far_z))
        for i in range(3):
            c.position[i] = float(self.t_c2w[i])
        return c


def look_at_camera(width, height, fov_x_deg, position, target=(0.0, 0.0, 0.0),
                   world_up=(0.0, -1.0, 0.0)):
    """Orbit camera: forward = normalize(target - position), right = normalize(forward x up),
    down = forward x right, R_c2w = [right down forward] (x right, y down, z forward,
    src/cameras.jl:626-627; a camera at (0, 0, -r) gets the identity rotation);
    horizontal-FoV focal length as scripts/render.jl:41."""
    p = np.asarray(position, dtype=np.float64)
    fwd = np.asarray(target, dtype=np.float64) - p
    fwd /= np.linalg.norm(fwd)
    right = np.cross(fwd, np.asarray(world_up, dtype=np.float64))
    right /= np.linalg.norm(right)
    down = np.cross(fwd, right)
    R = np.stack([right, down, fwd], axis=1).astype(f32)
    f = fov_deg_to_focal_length(fov_x_deg, width)
    return PinholeCamera.from_focal(width, height, f, R, p.astype(f32))


@dataclass
class Tiling:
    """Tiling{I, TW, TH} (src/forward_structs.jl:340-380)."""
    tile_width: int
    tile_height: int
    nb_tiles_x: int
    nb_tiles_y: int

    @classmethod
    def for_screen(cls, width, height, tile_width, tile_height):
        return cls(int(tile_width), int(tile_height), -(-int(width) // int(tile_width)),
                   -(-int(height) // int(tile_height)))

    @classmethod
    def for_camera(cls, cam: PinholeCamera, tile_width=None, tile_height=None):
        if tile_width is None:
            tile_width, tile_height = get_default_tile_size(cam.width, cam.height)
        return cls.for_screen(cam.width, cam.height, tile_width, tile_height)

    @property
    def nb_tiles(self):
        return self.nb_tiles_x * self.nb_tiles_y

    def end_bit(self):
        """Sort bit range of forward_core.jl:623: 33 + floor(log2(nb_tiles))."""
        return 33 + int(math.floor(math.log2(self.nb_tiles)))

    def to_c(self) -> abi.TilingC:
        return abi.TilingC(self.tile_width, self.tile_height, self.nb_tiles_x, self.nb_tiles_y)


def get_default_tile_size(width, height):
    """src/forward_structs.jl:419-424."""
    return 16, (32 if width * height > 1_500_000 else 16)


def _n2p(size, coord):
    """NormalizedToPixelConverter (image_coordinates.jl:71-76, 136-137) in float32."""
    factor = f32(f32(size) / f32(2))
    return f32(factor * f32(f32(coord) + f32(1)))


@dataclass
class RenderOptions:
    """RenderOptions (src/forward_structs.jl:579-665)."""
    width: int
    height: int
    sh_degree: int
    clip_mode: int = abi.TDGS_CLIP_CLAMP
    background_color: tuple = (0.0, 0.0, 0.0)
    use_antialiasing: bool = False
    min_alpha: float = DEFAULT_MIN_ALPHA
    max_alpha: float = DEFAULT_MAX_ALPHA
    min_transmittance: float = DEFAULT_MIN_TRANSMITTANCE
    dilation_x_px: float = DEFAULT_DILATION_PX
    dilation_y_px: float = DEFAULT_DILATION_PX
    clip_x_min_nc: float = -1 - DEFAULT_CLIPPING_MARGIN_NC
    clip_x_max_nc: float = 1 + DEFAULT_CLIPPING_MARGIN_NC
    clip_y_min_nc: float = -1 - DEFAULT_CLIPPING_MARGIN_NC
    clip_y_max_nc: float = 1 + DEFAULT_CLIPPING_MARGIN_NC
    exact_sh_jacobian: bool = False
    exact_aa_gradient: bool = False

    @classmethod
    def for_camera(cls, cam: PinholeCamera, sh_degree, **kw):
        return cls(cam.width, cam.height, sh_degree, **kw)

    def with_sh_degree(self, sh_degree):
        """set_sh_degree (forward_structs.jl:711-719)."""
        d = dict(self.__dict__)
        d["sh_degree"] = int(sh_degree)
        return RenderOptions(**d)

    def to_c(self) -> abi.RenderOptionsC:
        o = abi.RenderOptionsC()
        for i in range(3):
            o.background[i] = float(f32(self.background_color[i]))
        o.aa_min_factor = float(f32(DEFAULT_MIN_AA_FACTOR))
        o.min_alpha = float(f32(self.min_alpha))
        o.max_alpha = float(f32(self.max_alpha))
        o.min_transmittance = float(f32(self.min_transmittance))
        o.dilation_x = float(f32(self.dilation_x_px))
        o.dilation_y = float(f32(self.dilation_y_px))
        o.clip_x_min = float(_n2p(self.width, self.clip_x_min_nc))
        o.clip_x_max = float(_n2p(self.width, self.clip_x_max_nc))
        o.clip_y_min = float(_n2p(self.height, self.clip_y_min_nc))
        o.clip_y_max = float(_n2p(self.height, self.clip_y_max_nc))
        o.sh_degree = int(self.sh_degree)
        o.clip_mode = int(self.clip_mode)
        o.antialiasing = 1 if self.use_antialiasing else 0
        o.flags = ((abi.TDGS_FLAG_EXACT_SH_JACOBIAN if self.exact_sh_jacobian else 0)
                   | (abi.TDGS_FLAG_EXACT_AA_GRADIENT if self.exact_aa_gradient else 0))
        return o


def logit32(x):
    """logit (src/misc.jl:244-246) in float32: -log(1/x - 1)."""
    x = f32(x)
    return f32(-np.log(f32(f32(f32(1) / x) - f32(1))))


def color_to_sh_coeffs_dc(rgb):
    """src/sh.jl:157-159."""
    return ((np.asarray(rgb, dtype=f32) - f32(0.5)) / f32(SH_C0)).astype(f32)


@dataclass
class HostGaussians:
    """TrainableGaussiansVector contents as host arrays in the reference's memory layout:
    means_opacity (n, 4) == Julia 4 x n, scaling (n, 3), rotation (n, 4), sh (n, 3, h)
    == Julia (h, 3, n)."""
    means_opacity: np.ndarray
    scaling: np.ndarray
    rotation: np.ndarray
    sh: np.ndarray

    @property
    def n(self):
        return self.means_opacity.shape[0]

    @property
    def sh_degree(self):
        return int(round(math.sqrt(self.sh.shape[2]))) - 1


@dataclass
class HostRenderOnlyGaussians:
    """RenderOnlyGaussiansVector contents (src/gaussians.jl:342-392) as host arrays: means with
    activated opacities (n, 4), covariance lower halves [V11, V21, V31, V22, V32, V33] (n, 6),
    sh (n, 3, h)."""
    means_opacity: np.ndarray
    covariances: np.ndarray
    sh: np.ndarray

    @property
    def n(self):
        return self.means_opacity.shape[0]

    @property
    def sh_degree(self):
        return int(round(math.sqrt(self.sh.shape[2]))) - 1


def create_test_scene(sh_degree=0, two_cameras=False):
    """create_test_scene (src/scene.jl:123-188): four Gaussians (red, white behind the camera,
    green, purple) and a 320 x 240 camera with a 90 degree horizontal field of view."""
    w, h = 320, 240
    f = fov_deg_to_focal_length(90, w)
    cam = PinholeCamera.from_focal(w, h, f, np.eye(3, dtype=f32), np.zeros(3, dtype=f32))
    K = np.array([[cam.fx, cam.skew, cam.ppx], [0, cam.fy, cam.ppy], [0, 0, 1]], dtype=np.float64)
    K_inv = np.linalg.inv(K).astype(f32)
    means2d = np.array([[w / 3, w / 2 - 0.1, w / 2 + 0.1, 2 * w / 3],
                        [2 * h / 3, h / 2 + 0.1, h / 3, 2 * h / 3]], dtype=f32)
    depths = np.array([1, -1, 2, 3], dtype=f32)
    hom = np.concatenate([means2d * depths[None, :], depths[None, :]], axis=0).astype(f32)
    means = _mm(K_inv, hom)  # 3 x 4
    opacity_features = np.array([logit32(v) for v in (0.75, 0.99, 0.5, 0.99)], dtype=f32)
    scaling = np.log(np.array([[0.25, 10, 0.5, 1.0], [0.25, 20, 0.5, 0.75],
                               [0.25, 30, 0.5, 0.5]], dtype=f32)).astype(f32)
    rotation = np.array([[math.sqrt(2) / 2, 1.0, 1.0, math.sqrt(3)], [0.0, 0.0, 0.0, 1.0],
                         [0.0, 0.0, 0.0, 0.0], [math.sqrt(2) / 2, 0.0, 0.0, 0.0]], dtype=f32)
    hh = (sh_degree + 1) ** 2
    dcs = [color_to_sh_coeffs_dc(c) for c in ([0.796, 0.235, 0.2], [1.0, 1.0, 1.0],
                                               [0.22, 0.596, 0.149], [0.584, 0.345, 0.698])]
    rest = [0.01, -0.01, 0.01, 0.01]
    sh = np.zeros((4, 3, hh), dtype=f32)
    for g in range(4):
        sh[g, :, 0] = dcs[g]
        sh[g, :, 1:] = f32(rest[g])
    mo = np.concatenate([means.T, opacity_features[:, None]], axis=1).astype(f32)
    gaussians = HostGaussians(np.ascontiguousarray(mo), np.ascontiguousarray(scaling.T),
                              np.ascontiguousarray(rotation.T), sh)
    cams = [cam]
    if two_cameras:
        cams.append(PinholeCamera(cam.width, cam.height, cam.fx, cam.fy, cam.skew, cam.ppx, cam.ppy,
                                  cam.near_z, cam.far_z, cam.R_c2w,
                                  (cam.t_c2w + cam.R_c2w @ np.array([1, 0, 0], dtype=f32)).astype(f32)))
    return gaussians, cams


def scene_radius(cameras, enlargement_factor=1.1):
    """_compute_scene_radius (src/scene.jl:64-73)."""
    pos = np.stack([np.asarray(c.position, dtype=np.float64) for c in cameras])
    center = pos.mean(axis=0)
    return float(enlargement_factor * max(np.linalg.norm(p - center) for p in pos))
