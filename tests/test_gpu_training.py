"""GPU parity of the optimiser, densification and loss, through the C-ABI.

Adam and adaptive density control run the oracle's per-element arithmetic (shared with the
CPU restatement, including the counter-based split sampler), so they must match bit for
bit. The fused L1 + DSSIM loss is a floating-point reduction and is compared with a float64
torch restatement of the textbook SSIM (Wang et al. 2004; conv2d, zero padding) and its
autograd gradient.
"""
import ctypes as C
import math

import numpy as np
import pytest
import torch

from conftest import golden
from tdgs_amd import host

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _random_scene(n, deg, seed):
    rng = np.random.default_rng(seed)
    h = (deg + 1) ** 2
    q = rng.normal(size=(n, 4))
    return host.HostGaussians(
        np.concatenate([rng.normal(size=(n, 3)), rng.normal(0, 2, size=(n, 1))], 1).astype(np.float32),
        rng.normal(-3, 1, size=(n, 3)).astype(np.float32), q.astype(np.float32),
        rng.normal(0, 0.3, size=(n, 3, h)).astype(np.float32))


def _grads(nf, deg, seed):
    rng = np.random.default_rng(seed)
    h = (deg + 1) ** 2
    return {"mean3d": rng.normal(size=(nf, 3)).astype(np.float32),
            "opacity_feature": rng.normal(size=nf).astype(np.float32),
            "scaling_features": rng.normal(size=(nf, 3)).astype(np.float32),
            "rotation_features": rng.normal(size=(nf, 4)).astype(np.float32),
            "sh": rng.normal(size=(nf, 3, h)).astype(np.float32)}


@pytest.mark.parametrize("deg,render_deg", [(3, 3), (3, 1), (0, 0)])
def test_adam_bit_exact(gpu, oracle, deg, render_deg):
    from tdgs_amd import training
    n, nf = 5000, 3000
    g = _random_scene(n, deg, 1)
    rng = np.random.default_rng(2)
    f2g = np.sort(rng.choice(n, nf, replace=False)).astype(np.int32) + 1
    f2g[::7] = 0  # skipped entries (ADC sets them to 0)
    grads = _grads(nf, deg, 3)
    lrs = [1.6e-4, 0.05, 0.005, 0.001, 0.0025, 0.000125]
    adam_h = oracle.AdamHost(n, deg, lrs, update_count=4)
    for arr in (adam_h.means, adam_h.opacity, adam_h.scaling, adam_h.rotation, adam_h.sh):
        arr[...] = np.abs(rng.normal(size=arr.shape)).astype(np.float32) * 1e-3
    gd = gpu.TrainableGaussiansVector.from_host(g, 0)
    opt = training.AdamOptimizer(gd, training.TrainingOptions())
    m = opt.moments
    m.means_lr, m.opacity_lr, m.scaling_lr, m.rotation_lr, m.sh_dc_lr, m.sh_rest_lr = lrs
    for dst, src in ((m.means, adam_h.means), (m.opacity, adam_h.opacity), (m.scaling, adam_h.scaling),
                     (m.rotation, adam_h.rotation), (m.sh, adam_h.sh)):
        dst.copy_(torch.from_numpy(src))
    opt.update_count = 4
    fg = gpu.FilteredGaussiansGradientsVector(nf, deg, 0)
    for k, v in grads.items():
        getattr(fg, k).copy_(torch.from_numpy(v))
    opt.update_(fg, torch.from_numpy(f2g).to(DEV), nf, render_deg)
    oracle.adam_step(g, adam_h, grads, f2g, render_deg)
    torch.cuda.synchronize()
    assert opt.update_count == adam_h.update_count == 5
    got = gd.to_host()
    for a, b in ((got.means_opacity, g.means_opacity), (got.scaling, g.scaling), (got.rotation, g.rotation),
                 (got.sh, g.sh)):
        np.testing.assert_array_equal(a, b)
    for dst, src in ((m.means, adam_h.means), (m.opacity, adam_h.opacity), (m.scaling, adam_h.scaling),
                     (m.rotation, adam_h.rotation), (m.sh, adam_h.sh)):
        np.testing.assert_array_equal(dst.cpu().numpy(), src)


def test_adc_bit_exact(gpu, oracle):
    from tdgs_amd import training
    n, deg = 20000, 3
    g = _random_scene(n, deg, 5)
    rng = np.random.default_rng(6)
    adc_h = oracle.AdcHost(n)
    adc_h.accum[:] = np.abs(rng.normal(0, 3e-4, n)).astype(np.float32)
    adc_h.counts[:] = rng.integers(0, 3, n).astype(np.int32)
    args = (float(host.logit32(0.005)), True, float(np.log(np.float32(0.5))), 2e-4, float(np.log(np.float32(0.06))))
    nn_h = oracle.adc_plan(adc_h, g, *args)
    gd = gpu.TrainableGaussiansVector.from_host(g, 0)
    adc = training.AdaptiveDensityControlBuffers(n, 0)
    adc.accum.copy_(torch.from_numpy(adc_h.accum))
    adc.counts.copy_(torch.from_numpy(adc_h.counts))
    nn = training.adc_plan_(adc, gd, *args)
    assert nn == nn_h
    for a, b in ((adc.prune, adc_h.prune), (adc.densify, adc_h.densify), (adc.clone, adc_h.clone),
                 (adc.cs, adc_h.cs)):
        np.testing.assert_array_equal(a.cpu().numpy(), b)
    np.testing.assert_array_equal(adc.ngidx[:nn].cpu().numpy(), adc_h.ngidx[:nn])
    assert adc_h.densify.sum() > 100 and adc_h.clone.sum() > 10 and adc_h.prune.sum() > 100
    lrs = [1.6e-4, 0.05, 0.005, 0.001, 0.0025, 0.000125]
    adam_h = oracle.AdamHost(n, deg, lrs)
    for arr in (adam_h.means, adam_h.opacity, adam_h.scaling, adam_h.rotation, adam_h.sh):
        arr[...] = rng.normal(size=arr.shape).astype(np.float32)
    opt = training.AdamOptimizer(gd, training.TrainingOptions())
    for dst, src in ((opt.moments.means, adam_h.means), (opt.moments.opacity, adam_h.opacity),
                     (opt.moments.scaling, adam_h.scaling), (opt.moments.rotation, adam_h.rotation),
                     (opt.moments.sh, adam_h.sh)):
        dst.copy_(torch.from_numpy(src))
    log_split = float(np.log(np.float32(1 / 1.6)))
    new = training.adaptive_density_control_(adc, gd, opt, nn, log_split, 99)
    ng_h, nm_h = oracle.adc_apply(adc_h, g, adam_h, log_split, 99)
    got = new.to_host()
    for a, b in ((got.means_opacity, ng_h.means_opacity), (got.scaling, ng_h.scaling),
                 (got.rotation, ng_h.rotation), (got.sh, ng_h.sh)):
        np.testing.assert_array_equal(a, b)
    for dst, src in ((opt.moments.means, nm_h.means), (opt.moments.opacity, nm_h.opacity),
                     (opt.moments.scaling, nm_h.scaling), (opt.moments.rotation, nm_h.rotation),
                     (opt.moments.sh, nm_h.sh)):
        np.testing.assert_array_equal(dst.cpu().numpy(), src)
    f2g = np.sort(rng.choice(n, 7000, replace=False)).astype(np.int32) + 1
    f2g_d = torch.from_numpy(f2g).to(DEV)
    training.adc_remap_fgidx_(adc, f2g_d, len(f2g))
    np.testing.assert_array_equal(f2g_d.cpu().numpy(), oracle.adc_remap_fgidx(adc_h, f2g))


def test_adc_stats_bit_exact(gpu, oracle):
    from tdgs_amd import training
    n, nf = 3000, 2000
    rng = np.random.default_rng(8)
    f2g = np.sort(rng.choice(n, nf, replace=False)).astype(np.int32) + 1
    g2 = rng.normal(0, 1e-4, size=(nf, 9)).astype(np.float32)
    g2[::5, :2] = 0
    adc_h = oracle.AdcHost(n)
    oracle.adc_stats(adc_h, g2, f2g, 1920, 1080)
    oracle.adc_stats(adc_h, g2, f2g, 1920, 1080)
    adc = training.AdaptiveDensityControlBuffers(n, 0)
    fg = gpu.FilteredGaussiansGradientsVector(nf, 0, 0)
    fg.grads2d.copy_(torch.from_numpy(g2))

    class Cam:
        width, height = 1920, 1080
    f2g_d = torch.from_numpy(f2g).to(DEV)
    training.adc_stats_(adc, fg, f2g_d, nf, Cam)
    training.adc_stats_(adc, fg, f2g_d, nf, Cam)
    np.testing.assert_array_equal(adc.accum.cpu().numpy(), adc_h.accum)
    np.testing.assert_array_equal(adc.counts.cpu().numpy(), adc_h.counts)


def _ssim_torch(x, y):
    """Textbook SSIM map (Wang et al. 2004) on (3, H, W) float64 tensors, zero padding."""
    k = torch.arange(11, dtype=torch.float64) - 5
    g = torch.exp(-k ** 2 / (2 * 1.5 ** 2))
    g = g / g.sum()
    w = (g[:, None] * g[None, :]).expand(3, 1, 11, 11).contiguous()

    def f(a):
        return torch.nn.functional.conv2d(a[None], w, padding=5, groups=3)[0]
    mx, my = f(x), f(y)
    sxx, syy, sxy = f(x * x) - mx ** 2, f(y * y) - my ** 2, f(x * y) - mx * my
    c1, c2 = 0.01 ** 2, 0.03 ** 2
    return ((2 * mx * my + c1) * (2 * sxy + c2)) / ((mx ** 2 + my ** 2 + c1) * (sxx + syy + c2))


@pytest.mark.parametrize("W,H,w", [(64, 48, 0.2), (123, 77, 0.2), (320, 240, 0.5), (1297, 840, 0.2),
                                   (1920, 1080, 0.2)])
def test_loss_grad_against_textbook_ssim(gpu, W, H, w):
    from tdgs_amd import training
    gen = torch.Generator().manual_seed(W * H)
    img = torch.rand((W, H, 3), generator=gen, dtype=torch.float32)
    gt = (img + 0.2 * torch.rand((W, H, 3), generator=gen)).clamp(0, 1).float()
    x = img.double().permute(2, 1, 0).contiguous().requires_grad_(True)  # (3, H, W)
    y = gt.double().permute(2, 1, 0).contiguous()
    n = x.numel()
    ssim = _ssim_torch(x, y).sum()
    loss = (1 - w) * (x - y).abs().sum() / n + w * (1 - ssim / n)
    loss.backward()
    ref_grad = x.grad.permute(2, 1, 0).contiguous().numpy()
    grad = torch.empty((W, H, 3), dtype=torch.float32, device=DEV)
    sums = torch.zeros(2, dtype=torch.float64, device=DEV)
    temp = torch.empty(int(gpu.lib().tdgs_loss_temp_bytes(W, H)), dtype=torch.uint8, device=DEV)
    training.loss_grad_(img.to(DEV), gt.to(DEV), grad, w, sums, temp)
    torch.cuda.synchronize()
    s = sums.cpu().numpy()
    assert abs(s[0] - float((x - y).abs().sum())) <= 1e-4 * abs(s[0])
    assert abs(s[1] - float(ssim)) <= 1e-4 * abs(float(ssim))
    got = grad.cpu().numpy()
    assert np.linalg.norm(got - ref_grad) <= 1e-3 * np.linalg.norm(ref_grad)


@pytest.mark.parametrize("with_dssim", [False, True])
def test_l1_loss_grad_against_oracle(gpu, oracle, with_dssim):
    """tdgs_l1_loss_grad (training.jl:206-215) bit for bit against the oracle, on an image with
    a quarter of its values tied (a tie takes -w), and its L1 sum."""
    from tdgs_amd import training
    W, H = 257, 131
    rng = np.random.default_rng(21 + with_dssim)
    r = rng.random((W, H, 3), dtype=np.float32)
    gt = np.where(rng.random((W, H, 3)) < 0.25, r, rng.random((W, H, 3), dtype=np.float32)).astype(np.float32)
    dg = (rng.standard_normal((W, H, 3)) * 1e-3).astype(np.float32) if with_dssim else None
    weight = 0.2
    l1_w = float(np.float32(1) - np.float32(weight))
    s_ref, ref = oracle.l1_loss_grad(r, gt, l1_w, weight if with_dssim else 0.0, dg)
    out = torch.empty((W, H, 3), dtype=torch.float32, device=DEV)
    l1 = torch.zeros(1, dtype=torch.float64, device=DEV)
    training.l1_loss_grad_(torch.from_numpy(r).to(DEV), torch.from_numpy(gt).to(DEV), out, l1_w,
                           weight if with_dssim else 0.0, None if dg is None else torch.from_numpy(dg).to(DEV), l1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    assert abs(float(l1) - s_ref) <= 1e-12 * s_ref
    ties = r == gt
    assert ties.sum() > 0.2 * r.size
    if not with_dssim:
        w = np.float32(np.float32(l1_w) / np.float32(r.size))
        assert bool((out.cpu().numpy()[ties] == -w).all())


def test_opacity_reset_and_sh_resize(gpu):
    from tdgs_amd import training
    g = _random_scene(1000, 1, 11)
    gd = gpu.TrainableGaussiansVector.from_host(g, 0)
    mom = torch.ones((1000, 2), dtype=torch.float32, device=DEV)
    training.opacity_reset_(gd, 0.01, mom)
    lim = host.logit32(0.01)
    np.testing.assert_array_equal(gd.means_opacity[:, 3].cpu().numpy(), np.minimum(g.means_opacity[:, 3], lim))
    assert float(mom.abs().sum()) == 0
    sh2 = training.sh_resize(gd.sh, 2, 1).cpu().numpy()
    np.testing.assert_array_equal(sh2[:, :, :4], g.sh)
    assert np.all(sh2[:, :, 4:] == 0)
    m = torch.arange(1000 * 3 * 4 * 2, dtype=torch.float32, device=DEV).reshape(1000, 3, 4, 2)
    m3 = training.sh_resize(m, 3, 2).cpu().numpy()
    np.testing.assert_array_equal(m3[:, :, :4, :], m.cpu().numpy())
    assert np.all(m3[:, :, 4:, :] == 0)
    m0 = training.sh_resize(m, 0, 2).cpu().numpy()
    np.testing.assert_array_equal(m0[:, :, 0, :], m.cpu().numpy()[:, :, 0, :])


def test_reference_adc_case_on_gpu(gpu):
    """test/training.jl:40-255 through the GPU entry points."""
    from tdgs_amd import training
    gold = golden("training_adc_adam.json")
    n, deg = 8, 1
    k = np.arange(1, n + 1, dtype=np.float32)
    g = host.HostGaussians(np.repeat(k[:, None], 4, 1).astype(np.float32), np.repeat(k[:, None], 3, 1).astype(np.float32),
                           np.repeat(k[:, None], 4, 1).astype(np.float32),
                           np.repeat(k[:, None], 12, 1).reshape(n, 3, 4).astype(np.float32))
    gd = gpu.TrainableGaussiansVector.from_host(g, 0)
    opt = training.AdamOptimizer(gd, training.TrainingOptions())
    for t in (opt.moments.means, opt.moments.opacity, opt.moments.scaling, opt.moments.rotation, opt.moments.sh):
        t.copy_(torch.from_numpy(k).to(DEV).reshape((n,) + (1,) * (t.dim() - 1)).expand_as(t))
    adc = training.AdaptiveDensityControlBuffers(n, 0)
    adc.prune.copy_(torch.tensor(gold["should_prune"], dtype=torch.uint8))
    adc.densify.copy_(torch.tensor(gold["should_densify"], dtype=torch.uint8))
    adc.clone.copy_(torch.tensor(gold["should_clone"], dtype=torch.uint8))
    adc.cs.copy_(torch.tensor(gold["new_gaussian_counts_cs"], dtype=torch.int32))
    new = training.adaptive_density_control_(adc, gd, opt, 10, gold["split_scale_factor_log"], 3)
    ngidx = np.array(gold["ngidx_to_gidx"], np.float32)
    got = new.to_host()
    np.testing.assert_array_equal(got.means_opacity[:, 3], ngidx)
    np.testing.assert_allclose(got.scaling[:, 0], np.array(gold["scaling_features_after"], np.float32), rtol=1e-6)
    np.testing.assert_array_equal(opt.moments.means[:, 0, 0].cpu().numpy(), np.array(gold["moments_after"], np.float32))
    f2g = torch.tensor(gold["fgidx_to_gidx_before"], dtype=torch.int32, device=DEV)
    training.adc_remap_fgidx_(adc, f2g, 3)
    assert f2g.cpu().tolist() == gold["fgidx_to_gidx_after"]


@pytest.mark.parametrize("cfg,render_deg", [(1, 3), (1, 1), (0, 0)])
def test_backward_project_adam_equals_separate_steps(gpu, cfg, render_deg):
    """tdgs_backward_project_adam (the trainer's fused step) against tdgs_backward_project
    followed by tdgs_adam_step on the same 2D gradients: parameters and moments bit for bit
    (SH3 float4 items, a render degree below the stored one, SH0); and
    tdgs_backward_project_adam_adc against tdgs_adc_stats before the separate steps: the same,
    and the density-control accumulators (started from nonzero values) bit for bit."""
    from tdgs_amd import synthetic, training
    w = synthetic.config(cfg, n=20_000 if cfg else None, cameras=2)
    cam = w.cameras[-1]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, render_deg)
    deg = w.gaussians.sh_degree
    runs = []
    stats = []
    gen = torch.Generator(device="cuda").manual_seed(5)
    grads2d = None
    for fused in (False, True, "adc"):
        gd = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
        out = gpu.RenderOutputs.for_camera(cam, 0)
        buf = gpu.RenderBuffers(len(gd), t, 0)
        gpu.render_(out, gd, cam, t, opts, buf)
        opt = training.AdamOptimizer(gd, training.TrainingOptions())
        rng = np.random.default_rng(9)
        m = opt.moments
        for arr in (m.means, m.opacity, m.scaling, m.rotation, m.sh):
            arr.copy_(torch.from_numpy((np.abs(rng.normal(size=tuple(arr.shape))) * 1e-3).astype(np.float32)))
        opt.update_count = 7
        fg = gpu.FilteredGaussiansGradientsVector(len(gd), deg, 0)
        nbf = buf.nb_fgaussians
        if grads2d is None:   # one set of 2D gradients for both (the blending atomics are unordered)
            rgb_grad = (torch.rand(out.rgb.shape, generator=gen, device="cuda") - 0.5) * 1e-3
            gpu.backward_render_tiles_(fg, rgb_grad.contiguous(), out, cam, t, opts, buf)
            grads2d = fg.grads2d[:nbf].clone()
        fg.grads2d[:nbf].copy_(grads2d)
        adc = training.AdaptiveDensityControlBuffers(len(gd), 0)
        adc.accum.copy_(torch.from_numpy(rng.uniform(0, 1e-3, len(gd)).astype(np.float32)))
        adc.counts.copy_(torch.from_numpy(rng.integers(0, 5, len(gd)).astype(np.int32)))
        if fused == "adc":
            opt.backward_project_update_(fg, cam, opts, buf, adc=adc)
        elif fused:
            opt.backward_project_update_(fg, cam, opts, buf)
        else:
            training.adc_stats_(adc, fg, buf.fgidx_to_gidx, nbf, cam)
            gpu.check(gpu.lib().tdgs_backward_project(gpu.stream_ptr(0), C.byref(fg.struct()), C.byref(gd.struct()),
                                                      C.byref(cam.to_c()), C.byref(opts.to_c()),
                                                      C.byref(buf.struct()), C.c_int32(nbf)))
            opt.update_(fg, buf.fgidx_to_gidx, nbf, render_deg)
        torch.cuda.synchronize()
        assert opt.update_count == 8
        runs.append((gd.to_host(), [x.cpu().numpy() for x in (m.means, m.opacity, m.scaling, m.rotation, m.sh)]))
        stats.append((adc.accum.cpu().numpy(), adc.counts.cpu().numpy()))
    (ga, ma) = runs[0]
    for gb, mb in runs[1:]:
        for x, y in ((ga.means_opacity, gb.means_opacity), (ga.scaling, gb.scaling), (ga.rotation, gb.rotation),
                     (ga.sh, gb.sh)):
            np.testing.assert_array_equal(x, y)
        for x, y in zip(ma, mb):
            np.testing.assert_array_equal(x, y)
    assert not np.array_equal(ga.means_opacity, w.gaussians.means_opacity)
    np.testing.assert_array_equal(stats[2][0], stats[0][0])
    np.testing.assert_array_equal(stats[2][1], stats[0][1])
    assert (stats[0][1] != stats[1][1]).sum() > 100   # the separate statistics counted Gaussians
