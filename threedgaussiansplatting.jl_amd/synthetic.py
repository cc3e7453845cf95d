"""Seeded synthetic scenes of the benchmark configurations.

Random numbers come from numpy's PCG64 generator seeded with 0x3D6500 + config (draws in
float64, rounded to float32), so the GPU path and the CPU oracle see identical inputs.
Quaternions are normalised N(0, 1) draws stored [r, x, y, z]; cameras look at the origin
from an orbit (world up = -y, x right / y down / z forward camera axes).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .host import HostGaussians, PinholeCamera, Tiling, look_at_camera

SEED_BASE = 0x3D6500


@dataclass
class Workload:
    name: str
    gaussians: HostGaussians
    cameras: list
    tile: tuple


def _gaussians(rng, n, sh_degree, means, log_scale_mu, log_scale_sigma, logit_sigma=1.5,
               dc_sigma=0.3, rest_sigma=0.05):
    h = (sh_degree + 1) ** 2
    logits = rng.normal(0.0, logit_sigma, size=(n, 1))
    log_s = rng.normal(log_scale_mu, log_scale_sigma, size=(n, 3))
    q = rng.normal(0.0, 1.0, size=(n, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    sh = np.zeros((n, 3, h))
    sh[:, :, 0] = rng.normal(0.0, dc_sigma, size=(n, 3))
    if h > 1:
        sh[:, :, 1:] = rng.normal(0.0, rest_sigma, size=(n, 3, h - 1))
    mo = np.concatenate([means, logits], axis=1)
    f = np.float32
    return HostGaussians(np.ascontiguousarray(mo, f), np.ascontiguousarray(log_s, f),
                         np.ascontiguousarray(q, f), np.ascontiguousarray(sh, f))


def _mixed_means(rng, n):
    half = n // 2
    a = rng.uniform(-10.0, 10.0, size=(half, 3))
    b = rng.normal(0.0, 1.5, size=(n - half, 3))
    m = np.concatenate([a, b], axis=0)
    return m[rng.permutation(n)]


def orbit_cameras(rng, count, width, height, radius, fov_deg, elevation_deg=20.0):
    cams = []
    for k in range(count):
        az = 2 * math.pi * k / count
        el = math.radians(rng.uniform(-elevation_deg, elevation_deg)) if count > 1 else 0.0
        pos = radius * np.array([math.cos(el) * math.sin(az), -math.sin(el),
                                 -math.cos(el) * math.cos(az)])
        cams.append(look_at_camera(width, height, fov_deg, pos))
    return cams


def config(idx: int, n: int | None = None, cameras: int | None = None) -> Workload:
    """Workload of BASELINE.json configs[idx]; n / cameras override the sizes (tests use
    reduced sizes of the same distributions)."""
    rng = np.random.Generator(np.random.PCG64(SEED_BASE + idx))
    if idx == 0:
        n = n or 10_000
        g = _gaussians(rng, n, 0, rng.normal(0.0, 1.0, size=(n, 3)), -3.5, 0.4)
        cams = [look_at_camera(256, 256, 60.0, (0.0, 0.0, -4.0))]
        return Workload("cfg0: 10k Gaussians, 256x256, SH0", g, cams, (16, 16))
    if idx == 1:
        n = n or 200_000
        g = _gaussians(rng, n, 3, rng.normal(0.0, 1.0, size=(n, 3)), -3.5, 0.4)
        cams = [look_at_camera(800, 800, 60.0, (0.0, 0.0, -4.0))]
        return Workload("cfg1: 200k Gaussians, 800x800, SH3", g, cams, (16, 16))
    if idx == 2:
        n = n or 1_000_000
        g = _gaussians(rng, n, 3, _mixed_means(rng, n), -4.0, 0.6)
        cams = orbit_cameras(rng, cameras or 120, 1920, 1080, 6.0, 50.0)
        return Workload("cfg2: 1M Gaussians, 1920x1080, SH3, orbit cameras", g, cams, (16, 16))
    if idx == 3:
        n = n or 500_000
        g = _gaussians(rng, n, 3, _mixed_means(rng, n), -4.0, 0.6)
        cams = orbit_cameras(rng, cameras or 100, 1297, 840, 6.0, 50.0)
        return Workload("cfg3: 500k Gaussians, 1297x840, SH3, training", g, cams, (16, 16))
    if idx == 4:
        n = n or 3_000_000
        g = _gaussians(rng, n, 3, _mixed_means(rng, n), -2.5, 0.8)
        cams = orbit_cameras(rng, cameras or 1, 3840, 2160, 6.0, 50.0)
        return Workload("cfg4: 3M Gaussians, 3840x2160, SH3", g, cams, (16, 32))
    raise ValueError(idx)


def tiling_for(w: Workload, cam: PinholeCamera) -> Tiling:
    return Tiling.for_camera(cam, *w.tile)
