"""Writes tests/golden/float64_autograd.npz: images and gradients of small scenes from an
independent float64 restatement of the render core, differentiated by torch autograd.

Run in the build container only (CPU torch, float64); the committed .npz is the fixture that
tests/test_oracle_float64.py compares the CPU oracle against. The restatement is written from
the mathematics of docs/src/math.md and the reference's semantics, not from the oracle's code:

- projection (cameras.jl:714-774): mu = (P[1:2, 1:3] m + P[1:2, 4]) / r, r = P[3, 1:3] m + P[3, 4];
  J = (1/r) [1 0 -mu_x; 0 1 -mu_y] P[:, 1:3], mu clamped to the extended screen first in
  CovarianceBoundaryClamp mode (forward_structs.jl:737-739), not in BoundaryFilter mode;
- Sigma = J R S S^T R^T J^T (R from the normalised quaternion, S = diag(exp(log s))), plus the
  0.3 px dilation; antialiasing multiplies the opacity by max(5e-4, sqrt(det / det_dilated))
  (forward_core.jl:450-462);
- culling (forward_core.jl:326-355): opacity >= min_alpha and near < depth <= far; BoundaryFilter
  also requires clip_min < mu <= clip_max on both axes and opacity > min_alpha;
- colour: real spherical harmonics up to degree 3 with the normalisation constants of
  sh.jl:1-18, evaluated at normalize(m - camera position), + 1/2, clamped below at 0;
- blending (forward_core.jl:756-993) per pixel centre (u - 1/2, v - 1/2), all kept Gaussians in
  depth order: alpha = min(0.99, a exp(-d^T M d / 2)), M = Sigma^-1; skipped if alpha < 1/255;
  the walk stops (that Gaussian excluded) once T (1 - alpha) < 1e-4; rgb = sum T alpha c + T bg.
The loss is sum(g * rgb) for a fixed random g. With antialiasing the fixture holds the
gradients twice: of this forward pass (d_*), and with the antialiasing factor's derivative taken
as that of f^2 = det0 / det while its value stays f (dref_*), which is what the reference's
backward pass computes. Gradients with respect to mu, a, the lower
vector (M11, M21, M22) of M and the colour are the 2D gradients; those with respect to the
means, opacity logits, log-scales, quaternions and SH coefficients are the 3D gradients.

Scenes are redrawn until no evaluated pair lies within 1e-6 (relative) of the min_alpha or min_T
thresholds or within 1e-4 of the max alpha, and no two kept depths are closer than 1e-5
(relative), so that the float32 oracle (relative errors of a few 1e-7 in alpha) takes the same
discrete decisions; no colour is clamped at 0 and no mean lies
outside the clip bounds of the clamp mode (where the reference's backward pass deliberately
differs from the derivative: sh.jl:106-108 gate, backward_core.jl:812-817).
"""
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
import __graft_entry__  # noqa: E402

__graft_entry__.load_package()
from tdgs_amd import host  # noqa: E402

torch.set_default_dtype(torch.float64)
f32 = np.float32

SH_CONST = [0.28209479177387814, 0.4886025119029199, 0.4886025119029199, 0.4886025119029199,
            1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792,
            0.5462742152960396, -0.5900435899266435, 2.890611442640554, -0.4570457994644658,
            0.3731763325901154, -0.4570457994644658, 1.445305721320277, -0.5900435899266435]


def sh_basis(d, degree):
    x, y, z = d.unbind(1)
    c = SH_CONST
    b = [torch.full_like(x, c[0])]
    if degree >= 1:
        b += [-c[1] * y, c[2] * z, -c[3] * x]
    if degree >= 2:
        b += [c[4] * x * y, c[5] * y * z, c[6] * (2 * z * z - x * x - y * y), c[7] * x * z, c[8] * (x * x - y * y)]
    if degree >= 3:
        b += [c[9] * y * (3 * x * x - y * y), c[10] * x * y * z, c[11] * y * (4 * z * z - x * x - y * y),
              c[12] * z * (2 * z * z - 3 * x * x - 3 * y * y), c[13] * x * (4 * z * z - x * x - y * y),
              c[14] * z * (x * x - y * y), c[15] * x * (x * x - 3 * y * y)]
    return torch.stack(b, 1)


def rotation(q):
    q = q / q.norm(dim=1, keepdim=True)
    r, x, y, z = q.unbind(1)
    return torch.stack([
        torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - r * z), 2 * (x * z + r * y)], 1),
        torch.stack([2 * (x * y + r * z), 1 - 2 * (x * x + z * z), 2 * (y * z - r * x)], 1),
        torch.stack([2 * (x * z - r * y), 2 * (y * z + r * x), 1 - 2 * (x * x + y * y)], 1)], 1)


def restated_render(g, cam, o, g_rgb, reference_aa_gradient=False):
    """Returns (results, margins): rgb (W, H, 3), T (W, H), the keep mask and the gradients.
    reference_aa_gradient: the antialiasing factor keeps its value f = sqrt(det0 / det) but
    propagates the gradient of f^2 = det0 / det, as the reference's backward pass does
    (backward_core.jl:480-490, docs/src/math.md:194-197)."""
    W, H = cam.width, cam.height
    P = torch.tensor(cam.P, dtype=torch.float64)
    pos = torch.tensor(cam.position, dtype=torch.float64)
    c = o.to_c()
    m = torch.tensor(g.means_opacity[:, :3], dtype=torch.float64, requires_grad=True)
    logit = torch.tensor(g.means_opacity[:, 3], dtype=torch.float64, requires_grad=True)
    logs = torch.tensor(g.scaling, dtype=torch.float64, requires_grad=True)
    q = torch.tensor(g.rotation, dtype=torch.float64, requires_grad=True)
    sh = torch.tensor(g.sh, dtype=torch.float64, requires_grad=True)
    a0 = torch.sigmoid(logit)
    ph = m @ P[:, :3].T + P[:, 3]
    depth = ph[:, 2]
    mu = ph[:, :2] / depth[:, None]
    lo = torch.tensor([c.clip_x_min, c.clip_y_min])
    hi = torch.tensor([c.clip_x_max, c.clip_y_max])
    keep = (a0 >= c.min_alpha) & (depth > float(np.float32(cam.near_z))) & (depth <= float(np.float32(cam.far_z)))
    if c.clip_mode == 1:
        keep &= ((mu > lo) & (mu <= hi)).all(1) & (a0 > c.min_alpha)
        muc = mu
    else:
        muc = torch.minimum(torch.maximum(mu, lo), hi)
    n = len(a0)
    zero, one = torch.zeros(n), torch.ones(n)
    A = torch.stack([torch.stack([one, zero, -muc[:, 0]], 1), torch.stack([zero, one, -muc[:, 1]], 1)], 1)
    J = A @ P[:, :3] / depth[:, None, None]
    RS = rotation(q) * torch.exp(logs)[:, None, :]
    S2 = J @ RS @ RS.transpose(1, 2) @ J.transpose(1, 2)
    c11, c21, c22 = S2[:, 0, 0], S2[:, 1, 0], S2[:, 1, 1]
    det0 = c11 * c22 - c21 * c21
    c11 = c11 + c.dilation_x
    c22 = c22 + c.dilation_y
    det = c11 * c22 - c21 * c21
    a = a0
    if c.antialiasing:
        f = torch.clamp(torch.sqrt(torch.clamp(det0, min=0) / det), min=c.aa_min_factor)
        if reference_aa_gradient:
            f2 = torch.clamp(det0, min=0) / det
            f = f.detach() + (f2 - f2.detach())
        a = a0 * f
    M = torch.stack([c22 / det, -c21 / det, c11 / det], 1)
    h = sh.shape[2]
    dirs = m - pos
    dirs = dirs / dirs.norm(dim=1, keepdim=True)
    raw = (sh[:, :, :h] * sh_basis(dirs, int(round(math.sqrt(h))) - 1)[:, None, :]).sum(2) + 0.5
    color = torch.clamp(raw, min=0.0)
    # the 2D gradients are those of the blending stage: the mean as blending sees it is its own
    # node (the mean also enters J, whose derivative belongs to the 3D chain)
    mu_b = mu + 0.0
    for t in (mu_b, a, M, color):
        t.retain_grad()
    u = torch.arange(1, W + 1, dtype=torch.float64) - 0.5
    v = torch.arange(1, H + 1, dtype=torch.float64) - 0.5
    pu, pv = torch.meshgrid(u, v, indexing="ij")   # (W, H): pixel (u, v) at [u - 1, v - 1]
    pu, pv = pu.reshape(-1), pv.reshape(-1)
    T = torch.ones(W * H)
    C = torch.zeros(W * H, 3)
    alive = torch.ones(W * H, dtype=torch.bool)
    order = [int(i) for i in np.argsort(depth.detach().numpy(), kind="stable") if bool(keep[i])]
    margins = {"alpha_min": math.inf, "alpha_max": math.inf, "stop": math.inf, "depth": math.inf}
    kd = depth.detach().numpy()[order]
    if len(kd) > 1:
        margins["depth"] = float(np.min(np.diff(kd) / np.abs(kd[1:])))
    for i in order:
        du, dv = pu - mu_b[i, 0], pv - mu_b[i, 1]
        e = -0.5 * (M[i, 0] * du * du + 2 * M[i, 1] * du * dv + M[i, 2] * dv * dv)
        ag = a[i] * torch.exp(e)
        alpha = torch.clamp(ag, max=c.max_alpha)
        contrib = alive & (alpha >= c.min_alpha)
        Tn = T * (1 - alpha)
        stop = contrib & (Tn < c.min_transmittance)
        use = contrib & ~stop
        al = alpha.detach()
        live = alive & (al > 0.5 * c.min_alpha)
        if bool(live.any()):
            margins["alpha_min"] = min(margins["alpha_min"],
                                       float((torch.abs(al[live] / c.min_alpha - 1)).min()))
        if bool(contrib.any()):
            margins["alpha_max"] = min(margins["alpha_max"],
                                       float((c.max_alpha - ag.detach()[contrib]).min()) / c.max_alpha)
            margins["stop"] = min(margins["stop"],
                                  float((torch.abs(Tn.detach()[contrib] / c.min_transmittance - 1)).min()))
        C = C + torch.where(use[:, None], (T * alpha)[:, None] * color[i][None, :], torch.zeros(1, 3))
        T = torch.where(use, Tn, T)
        alive = alive & ~stop
    bg = torch.tensor([c.background[0], c.background[1], c.background[2]])
    rgb = C + T[:, None] * bg[None, :]
    loss = (rgb * torch.tensor(g_rgb.reshape(-1, 3), dtype=torch.float64)).sum()
    loss.backward()
    kept = keep.numpy()
    margins["color"] = float(raw.detach()[kept].min()) if kept.any() else math.inf
    inside = ((mu >= lo) & (mu <= hi)).all(1).detach().numpy()
    margins["outside_clip"] = int((~inside & kept).sum()) if c.clip_mode == 0 else 0
    res = {
        "rgb": rgb.detach().numpy().reshape(W, H, 3), "T": T.detach().numpy().reshape(W, H), "keep": kept,
        "grads2d": np.concatenate([mu_b.grad.numpy(), a.grad.numpy()[:, None], M.grad.numpy(), color.grad.numpy()], 1),
        "mean3d": m.grad.numpy(), "opacity_feature": logit.grad.numpy(), "scaling_features": logs.grad.numpy(),
        "rotation_features": q.grad.numpy(), "sh": sh.grad.numpy(),
    }
    for k in ("grads2d", "mean3d", "opacity_feature", "scaling_features", "rotation_features", "sh"):
        res[k][~kept] = 0.0
    return res, margins


def rgb_grad(seed, W, H):
    """The fixed dL/d(rgb) of a case, (W, H, 3) float32 in [-1, 1), from its seed."""
    return np.random.default_rng(seed).uniform(-1.0, 1.0, (W, H, 3)).astype(f32)


def random_scene(rng, n, degree, W, H, outside=0):
    """n Gaussians in front of a camera at the origin looking along +z (64 x 48, 60 degrees),
    plus `outside` ones projecting beyond the extended screen."""
    f = host.fov_deg_to_focal_length(60, W)
    cam = host.PinholeCamera.from_focal(W, H, f, np.eye(3, dtype=f32), np.zeros(3, dtype=f32))
    z = rng.uniform(2.0, 6.0, n + outside)
    px = np.concatenate([rng.uniform(0.1 * W, 0.9 * W, n), rng.choice([-0.6, 1.6], outside) * W])
    py = np.concatenate([rng.uniform(0.1 * H, 0.9 * H, n), rng.uniform(0.2 * H, 0.8 * H, outside)])
    x = (px - W / 2) / f * z
    y = (py - H / 2) / f * z
    h = (degree + 1) ** 2
    m = np.stack([x, y, z], 1)
    N = n + outside
    logit = rng.uniform(-1.5, 2.0, N)
    logs = rng.normal(np.log(0.06), 0.35, (N, 3))
    q = rng.normal(0, 1, (N, 4))
    q *= rng.uniform(0.5, 2.0, (N, 1))            # unnormalised quaternions
    sh = np.zeros((N, 3, h))
    sh[:, :, 0] = rng.uniform(-0.6, 1.2, (N, 3))
    if h > 1:
        sh[:, :, 1:] = rng.normal(0, 0.08, (N, 3, h - 1))
    g = host.HostGaussians(np.concatenate([m, logit[:, None]], 1).astype(f32), logs.astype(f32),
                           q.astype(f32), sh.astype(f32))
    return g, cam


def test_scene(degree):
    """create_test_scene (scene.jl:123-188) with opacities 0.75, 0.9, 0.5, 0.9 (the original 0.99
    sits exactly at the 0.99 alpha clamp, where the reference's backward pass ignores the clamp)."""
    g, cams = host.create_test_scene(sh_degree=degree)
    g.means_opacity[:, 3] = np.array([host.logit32(v) for v in (0.75, 0.9, 0.5, 0.9)], dtype=f32)
    return g, cams[0]


CASES = [
    # name, scene builder, options
    ("test_scene_sh3", lambda rng: test_scene(3), {}),
    ("test_scene_sh3_aa", lambda rng: test_scene(3), {"use_antialiasing": True}),
    ("test_scene_sh1_filter", lambda rng: test_scene(1), {"clip_mode": 1}),
    ("random_sh3", lambda rng: random_scene(rng, 24, 3, 64, 48), {}),
    ("random_sh3_aa", lambda rng: random_scene(rng, 24, 3, 64, 48), {"use_antialiasing": True}),
    ("random_sh2_filter", lambda rng: random_scene(rng, 24, 2, 64, 48, outside=4), {"clip_mode": 1}),
    ("random_sh1_aa_filter", lambda rng: random_scene(rng, 24, 1, 64, 48, outside=4),
     {"clip_mode": 1, "use_antialiasing": True}),
    ("random_sh0_bg", lambda rng: random_scene(rng, 30, 0, 64, 48), {"background_color": (0.3, 0.6, 0.9)}),
]


def main():
    out = {}
    for ci, (name, build, kw) in enumerate(CASES):
        rng = np.random.default_rng(0xF64 + ci)
        for attempt in range(200):
            g, cam = build(rng)
            opts = host.RenderOptions.for_camera(cam, g.sh_degree, exact_sh_jacobian=True, **kw)
            grad_seed = int(rng.integers(1 << 31))
            g_rgb = rgb_grad(grad_seed, cam.width, cam.height)
            res, mg = restated_render(g, cam, opts, g_rgb)
            ref = restated_render(g, cam, opts, g_rgb, reference_aa_gradient=True)[0] if opts.use_antialiasing else res
            ok = (mg["alpha_min"] > 1e-6 and mg["alpha_max"] > 1e-4 and mg["stop"] > 1e-6 and mg["depth"] > 1e-5
                  and mg["color"] > 1e-3 and mg["outside_clip"] == 0)
            if ok:
                break
        else:
            raise RuntimeError(f"{name}: no scene without near-threshold pairs")
        print(name, "attempts", attempt + 1, {k: (round(v, 6) if isinstance(v, float) else v) for k, v in mg.items()},
              "kept", int(res["keep"].sum()), "of", g.n)
        p = f"{name}/"
        out[p + "means_opacity"] = g.means_opacity
        out[p + "scaling"] = g.scaling
        out[p + "rotation"] = g.rotation
        out[p + "sh"] = g.sh
        out[p + "camera"] = np.array([cam.width, cam.height], np.int32)
        out[p + "P"] = cam.P.astype(f32)
        out[p + "position"] = np.asarray(cam.position, f32)
        out[p + "options"] = np.array([opts.clip_mode, int(opts.use_antialiasing), *opts.background_color],
                                      np.float64)
        out[p + "rgb_grad_seed"] = np.array([grad_seed], np.int64)
        # the images at (up to) 4096 pixels: all of a 64 x 48 image, a sample of a larger one
        npx = cam.width * cam.height
        px = np.arange(npx) if npx <= 4096 else np.sort(rng.choice(npx, 4096, replace=False))
        out[p + "pixels"] = px.astype(np.int64)
        out[p + "rgb"] = res.pop("rgb").reshape(npx, 3)[px]
        out[p + "T"] = res.pop("T").reshape(npx)[px]
        out[p + "keep"] = res.pop("keep")
        for k, v in res.items():   # gradients; with antialiasing also those of the reference's convention
            out[p + "d_" + k] = v.astype(np.float64)
            out[p + "dref_" + k] = ref[k].astype(np.float64)
    np.savez_compressed(os.path.join(HERE, "float64_autograd.npz"), **out)


if __name__ == "__main__":
    main()
