"""Closed forms pinning the oracle's functions that the reference's tests leave open:

- the antialiasing factor of an isotropic Gaussian facing the camera: sqrt(det0 / det) =
  sigma^2 / (sigma^2 + 0.3) for a 2D variance sigma^2 (forward_core.jl:450-462);
- the BoundaryFilter keep test at the clip bounds: clip_min < mu <= clip_max on each axis
  (forward_structs.jl:730-733, forward_core.jl:343), with means placed exactly on the bounds;
- the ADC statistic sqrt(gx^2 w^2 / 4 + gy^2 h^2 / 4), accumulated with a count only for
  non-zero mean gradients, on a non-square image (training.jl:478-492);
- the split offsets R (z * s), z ~ N(0, I) (gaussians.jl:1615-1626): their sample covariance
  for a rotated anisotropic parent is R diag(s^2) R^T, and not R^T diag(s^2) R;
- exp_f and log_f, the exponential and logarithm shared by the kernels and the oracle,
  against float64: at most 1 ulp for exp over its normal range (results below FLT_MIN flush
  to 0, above FLT_MAX give +inf) and 2 ulp for log over all positive normal floats.
"""
import math

import numpy as np
import pytest

from tdgs_amd import host

f32 = np.float32


def _axis_camera(w, h, fx, centred=True):
    """A camera at the origin looking along +z with focal length fx (a power of two, so that
    projections of chosen points are exact) and the principal point at the centre of the
    image, or at the pixel origin (then a point at depth 1 projects to exactly fx x)."""
    ppx, ppy = (w / 2, h / 2) if centred else (0.0, 0.0)
    return host.PinholeCamera(w, h, f32(fx), f32(fx), f32(0), f32(ppx), f32(ppy), f32(0.2), f32(np.inf),
                              np.eye(3, dtype=f32), np.zeros(3, dtype=f32))


@pytest.mark.parametrize("z,log_s", [(2.0, -2.0), (5.0, -3.0), (3.0, -4.5), (8.0, -5.0)])
def test_antialiasing_factor_isotropic(oracle, z, log_s):
    w, h = 320, 240
    cam = _axis_camera(w, h, 128.0)
    logit = 1.2
    g = host.HostGaussians(np.array([[0, 0, z, logit]], f32), np.full((1, 3), log_s, f32),
                           np.array([[0.3, -0.5, 0.7, 0.1]], f32), np.full((1, 3, 1), 0.5, f32))
    opts = host.RenderOptions.for_camera(cam, 0, use_antialiasing=True)
    r = oracle.render(g, cam, host.Tiling.for_camera(cam, 16, 16), opts)
    sigma2 = (128.0 * math.exp(log_s) / z) ** 2
    factor = sigma2 / (sigma2 + host.DEFAULT_DILATION_PX)
    a0 = 1 / (1 + math.exp(-logit))
    np.testing.assert_allclose(float(r["f2d"][0, 2]), a0 * max(factor, host.DEFAULT_MIN_AA_FACTOR), rtol=2e-5)
    np.testing.assert_allclose(float(r["f2d"][0, 3]), 1 / (sigma2 + host.DEFAULT_DILATION_PX), rtol=2e-5)


def test_filter_mode_keep_at_clip_bounds(oracle):
    w, h = 64, 48
    cam = _axis_camera(w, h, 32.0, centred=False)
    opts = host.RenderOptions.for_camera(cam, 0, clip_mode=1)
    c = opts.to_c()
    xmin, xmax, ymin, ymax = (f32(v) for v in (c.clip_x_min, c.clip_x_max, c.clip_y_min, c.clip_y_max))
    mid_y, mid_x = f32(h / 2), f32(w / 2)
    pts = [  # (mu_x, mu_y, kept)
        (xmax, mid_y, True), (np.nextafter(xmax, f32(np.inf)), mid_y, False),
        (xmin, mid_y, False), (np.nextafter(xmin, f32(np.inf)), mid_y, True),
        (mid_x, ymax, True), (mid_x, np.nextafter(ymax, f32(np.inf)), False),
        (mid_x, ymin, False), (mid_x, np.nextafter(ymin, f32(np.inf)), True),
        (xmax, ymax, True), (xmin, ymax, False), (mid_x, mid_y, True),
    ]
    # at depth 1 the projection of (mu / fx, ...) is exactly mu (fx a power of two, ppx = 0)
    means = np.array([[mx / f32(32), my / f32(32), 1.0, 2.0] for mx, my, _ in pts], f32)
    n = len(pts)
    g = host.HostGaussians(means, np.full((n, 3), -3.0, f32), np.tile(np.array([1, 0, 0, 0], f32), (n, 1)),
                           np.full((n, 3, 1), 0.5, f32))
    r = oracle.render(g, cam, host.Tiling.for_camera(cam, 16, 16), opts)
    nf = r["nb_fgaussians"]
    np.testing.assert_array_equal(r["keep"].astype(bool), [k for _, _, k in pts])
    kept = r["fgidx_to_gidx"][:nf] - 1
    ne = r["counts"][:nf] > 0      # records are written for non-empty bounding boxes only
    assert ne.sum() >= 3
    np.testing.assert_array_equal(r["f2d"][:nf, 0][ne], [pts[i][0] for i in kept[ne]])   # exact projections
    np.testing.assert_array_equal(r["f2d"][:nf, 1][ne], [pts[i][1] for i in kept[ne]])
    # the clamp mode keeps all of them (only the depth and opacity tests apply)
    r2 = oracle.render(g, cam, host.Tiling.for_camera(cam, 16, 16), host.RenderOptions.for_camera(cam, 0))
    assert r2["keep"].all()
    # opacity exactly min_alpha: kept by the clamp mode (>=), not by the filter mode (also >)
    g.means_opacity[:, 3] = host.logit32(f32(1 / 255))
    a = float(oracle.sigmoid(float(g.means_opacity[0, 3])))
    if a == float(f32(1 / 255)):
        assert not oracle.render(g, cam, host.Tiling.for_camera(cam, 16, 16), opts)["keep"].any()


def test_adc_statistic_non_square_image(oracle):
    W, H = 640, 360
    g2 = np.zeros((5, 9), f32)
    g2[0, :2] = (1e-3, 0.0)
    g2[1, :2] = (0.0, 1e-3)
    g2[2, :2] = (3e-4, -4e-4)
    g2[3, :2] = (0.0, 0.0)          # no contribution: neither accumulated nor counted
    g2[3, 2:] = 1.0                 # (other components do not matter)
    g2[4, :2] = (-2e-5, 7e-6)
    f2g = np.array([4, 2, 7, 1, 3], np.int32)   # fgidx -> gidx (1-based)
    adc = oracle.AdcHost(8)
    oracle.adc_stats(adc, g2, f2g, W, H)
    oracle.adc_stats(adc, g2, f2g, W, H)        # accumulates
    expect = np.zeros(8)
    count = np.zeros(8, np.int32)
    for f in range(5):
        gx, gy = (float(v) for v in g2[f, :2])
        if gx != 0 or gy != 0:
            expect[f2g[f] - 1] += 2 * math.sqrt((gx * W / 2) ** 2 + (gy * H / 2) ** 2)
            count[f2g[f] - 1] += 2
    np.testing.assert_allclose(adc.accum, expect, rtol=1e-6)
    np.testing.assert_array_equal(adc.counts, count)
    # x goes with the width: the swapped statistic differs by far more than the tolerance
    swapped = 2 * math.sqrt((1e-3 * H / 2) ** 2)
    assert abs(adc.accum[3] - swapped) > 0.1 * swapped


@pytest.mark.parametrize("q", [(0.9, 0.2, -0.3, 0.25), (0.3, -0.8, 0.4, 0.35)])
def test_split_offsets_covariance(oracle, q):
    n = 40_000
    s = np.array([0.5, 0.05, 0.15], f32)     # anisotropic
    rot = np.tile(np.array(q, f32), (n, 1))
    g = host.HostGaussians(np.tile(np.array([1.0, -2.0, 3.0, 0.5], f32), (n, 1)), np.tile(np.log(s), (n, 1)),
                           rot, np.zeros((n, 3, 1), f32))
    adc = oracle.AdcHost(n)
    adc.densify[:] = 1                      # every parent splits (densify, not clone)
    adc.cs[:] = 2 * np.arange(1, n + 1)
    adam = oracle.AdamHost(n, 0, [1] * 6)
    new, _ = oracle.adc_apply(adc, g, adam, float(np.log(f32(1 / 1.6))), seed=12345)
    off = new.means_opacity[:, :3].astype(np.float64) - np.array([1.0, -2.0, 3.0])
    R = oracle.quat_to_rot(np.array(q, f32)).astype(np.float64)
    want = R @ np.diag(s.astype(np.float64) ** 2) @ R.T
    cov = np.cov(off.T)
    scale = np.max(s.astype(np.float64)) ** 2
    assert np.max(np.abs(cov - want)) < 0.02 * scale, (cov, want)
    wrong = R.T @ np.diag(s.astype(np.float64) ** 2) @ R
    assert np.max(np.abs(cov - wrong)) > 0.1 * scale
    assert np.max(np.abs(off.mean(0))) < 0.02 * np.max(s)
    # both children of a parent get independent draws, and the log-scales shrink by log(1.6)
    assert not np.allclose(off[0::2], off[1::2])
    np.testing.assert_array_equal(new.scaling, np.tile(np.log(s) + f32(np.log(f32(1 / 1.6))), (2 * n, 1)))


def _ulps(got, ref):
    spacing = np.spacing(np.abs(ref).astype(f32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - ref) / spacing


def test_exp_f_within_one_ulp(oracle):
    x = np.concatenate([np.linspace(-87.33, 88.72, 2_000_001, dtype=f32),
                        f32([0.0, -0.0, 1e-30, -1e-30, 1.0, -1.0, 88.72283, -87.3365])])
    got = oracle.exp_array(x)
    ref = np.exp(x.astype(np.float64))
    assert ref.min() >= np.finfo(f32).tiny
    assert _ulps(got, ref).max() <= 1.0
    # results below FLT_MIN flush to 0 (alpha = a exp(e) is then far below min_alpha), past
    # FLT_MAX +inf, NaN propagates
    assert (oracle.exp_array(f32([-87.34, -90.0, -104.5, -1e30])) == 0).all()
    assert np.isinf(oracle.exp_array(f32([88.7229, 89.0, 1e30]))).all()
    assert np.isnan(oracle.exp_array(f32([np.nan]))).all()


def test_log_f_within_two_ulp(oracle):
    rng = np.random.default_rng(5)
    bits = rng.integers(0x00800000, 0x7F7FFFFF, 2_000_000, dtype=np.int64).astype(np.uint32)   # positive normals
    x = np.concatenate([bits.view(f32), np.linspace(0.5, 2.0, 1_000_001, dtype=f32),
                        f32([1.0, 2.0, 0.5, 1 / 255, 255.0, 3.4e38, 1.2e-38])])
    got = oracle.log_array(x)
    ref = np.log(x.astype(np.float64))
    nz = ref != 0
    assert _ulps(got[nz], ref[nz]).max() <= 2.0
    assert got[~nz].max() == 0.0 and got[~nz].min() == 0.0
    assert np.abs(got - ref).max() < 6e-8 * np.maximum(1.0, np.abs(ref)).max()
