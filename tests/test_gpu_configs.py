"""GPU runs of the BASELINE.json configurations at their full sizes.

- cfg1 (200k Gaussians, 800x800, SH3) and cfg2 (1M Gaussians, 1920x1080, SH3, one orbit
  camera): the forward pass bit-exact against the oracle (keys, lists, tile ranges, last
  contributors, images), the backward pass within relative L2 1e-3.
- cfg4 (3M Gaussians, 3840x2160, SH3, 16x32 tiles, > 100M duplicated keys), too large for the
  oracle's sort: size-independent properties of every key (sorted by (tile, depth bits, fgidx),
  each inside its Gaussian's tile rectangle with its depth bits, every Gaussian's rectangle
  emitted exactly once), tiles_end against the histogram of tile ids, last == 0 exactly where
  T == 1, the oracle's blending replayed on 16 tiles from the GPU's own lists, and finite
  gradients.
- cfg3 (500k Gaussians, 1297x840, SH3, 100 cameras, the reference's TrainingOptions): all 3000
  training iterations, across the 25 density-control steps (600, 700, ..., 3000) and the
  opacity reset at 3000, once with the reference's thresholds and once growing past 1M
  Gaussians, with the invariants of
  adaptive_density_control! (training.jl:313-459, gaussians.jl:1526-1694,
  optimizer.jl:1304-1378) checked at each: N' = sum(!prune + densify), carried Gaussians and
  clones equal their parents bit for bit, split log-scales equal the parent's + log(1/1.6),
  second clones and splits start with zero moments, split offsets distributed as R (z * s)
  with z ~ N(0, I); losses finite.
"""
import math

import numpy as np
import pytest
import torch

from tdgs_amd import host, synthetic, training
from test_gpu_backward import ARRAYS, REL_L2, rel_l2
from test_gpu_forward import _assert_forward_equal

pytestmark = pytest.mark.gpu


def _forward_backward_against_oracle(gpu, oracle, w, cam, tile):
    t = host.Tiling.for_camera(cam, *tile)
    opts = host.RenderOptions.for_camera(cam, w.gaussians.sh_degree, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(w.gaussians, cam, t, opts)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    out = gpu.RenderOutputs.for_camera(cam, 0, include_depth=True)
    buf = gpu.RenderBuffers(len(g), t, 0, keep_flags=True)
    gpu.render_(out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    _assert_forward_equal(r, out, buf)
    gen = torch.Generator(device="cuda").manual_seed(17)
    grad = ((torch.rand(out.rgb.shape, generator=gen, device="cuda") - 0.5) * 1e-3).contiguous()
    fg = gpu.FilteredGaussiansGradientsVector(buf.capacity, g.sh_degree, 0)
    gpu.backward_(fg, grad, out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    ref = oracle.backward(w.gaussians, cam, t, opts, r, grad.cpu().numpy())
    nf = buf.nb_fgaussians
    got = {"grads2d": fg.grads2d[:nf], **{k: getattr(fg, k)[:nf] for k in ARRAYS}}
    for k, v in got.items():
        e = rel_l2(v.cpu().numpy(), ref[k])
        assert e <= REL_L2, (k, e)
    return r


def test_cfg1_full_size_forward_backward(gpu, oracle):
    w = synthetic.config(1)
    assert len(w.gaussians.means_opacity) == 200_000
    r = _forward_backward_against_oracle(gpu, oracle, w, w.cameras[0], (16, 16))
    assert r["nb_keys"] > 1_000_000


@pytest.mark.parametrize("tile", [(16, 16), (16, 32)])
def test_cfg2_full_size_forward_backward(gpu, oracle, tile):
    w = synthetic.config(2, cameras=4)
    assert len(w.gaussians.means_opacity) == 1_000_000
    r = _forward_backward_against_oracle(gpu, oracle, w, w.cameras[1], tile)
    assert r["nb_keys"] > 3_000_000


def test_cfg4_full_size_properties(gpu, oracle):
    w = synthetic.config(4)
    cam = w.cameras[0]
    t = synthetic.tiling_for(w, cam)
    assert (t.tile_width, t.tile_height) == (16, 32)
    opts = host.RenderOptions.for_camera(cam, 3)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    out = gpu.RenderOutputs.for_camera(cam, 0, include_depth=True)
    buf = gpu.RenderBuffers(len(g), t, 0)
    gpu.render_(out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    nf, m = buf.nb_fgaussians, buf.nb_keys
    counts = buf.counts[:nf].to(torch.int64)
    assert int(counts.sum()) == m
    assert 100_000_000 < m < 2**31 - 1
    sk = buf.sorted_keys[:m]
    sv = buf.sorted_values[:m]
    ntx, ntiles = t.nb_tiles_x, t.nb_tiles
    ranges = buf.tile_ranges[:nf].to(torch.int64)
    depth_bits = buf.depths[:nf].view(torch.int32).to(torch.int64)
    tile_hist = torch.zeros(ntiles + 1, dtype=torch.int64, device="cuda")
    per_f = torch.zeros(nf + 1, dtype=torch.int64, device="cuda")
    chunk = 50_000_000
    for c0 in range(0, m, chunk):
        n_c = min(chunk, m - c0)
        k = sk[c0:c0 + n_c + 1]
        v = sv[c0:c0 + n_c + 1].to(torch.int64)
        # strictly increasing (tile, depth bits, fgidx): sorted, and no (Gaussian, tile) twice
        dk = k[1:] - k[:-1]
        assert bool(((dk > 0) | ((dk == 0) & (v[1:] > v[:-1]))).all()), c0
        kk, vv = k[:n_c], v[:n_c]
        tile = kk >> 32
        f = vv - 1
        assert bool(((tile >= 1) & (tile <= ntiles)).all()) and bool(((f >= 0) & (f < nf)).all())
        assert bool(((kk & 0xFFFFFFFF) == depth_bits[f]).all())
        tx = (tile - 1) % ntx + 1
        ty = (tile - 1) // ntx + 1
        r = ranges[f]
        assert bool(((tx >= r[:, 0]) & (tx <= r[:, 2]) & (ty >= r[:, 1]) & (ty <= r[:, 3])).all())
        tile_hist += torch.bincount(tile, minlength=ntiles + 1)
        per_f += torch.bincount(vv, minlength=nf + 1)
        del k, v, dk, kk, vv, tile, f, tx, ty, r
    # each Gaussian emitted as many keys as its rectangle has tiles (all inside it, none twice)
    assert torch.equal(per_f[1:], counts)
    area = (ranges[:, 2] - ranges[:, 0] + 1) * (ranges[:, 3] - ranges[:, 1] + 1)
    assert torch.equal(area[counts > 0], counts[counts > 0])
    assert torch.equal(torch.cumsum(tile_hist[1:], 0).to(torch.int32), buf.tiles_end)
    T, last = out.T, out.last
    assert torch.equal(last == 0, T == 1)
    # the oracle's blending on 16 tiles (the 8 longest lists and 8 random ones), replayed on
    # the GPU's sorted lists
    te = buf.tiles_end.cpu().numpy().astype(np.int64)
    lengths = np.diff(np.concatenate([[0], te]))
    rng = np.random.default_rng(4)
    chosen = list(np.argsort(lengths)[-8:] + 1) + list(rng.choice(ntiles, 8, replace=False) + 1)
    f2d = buf.f2d[:nf].cpu().numpy()
    depths = buf.depths[:nf].cpu().numpy()
    W, H, TW, TH = cam.width, cam.height, t.tile_width, t.tile_height
    rgb = np.zeros((W, H, 3), np.float32)
    Ti = np.zeros((W, H), np.float32)
    Di = np.zeros((W, H), np.float32)
    Li = np.zeros((W, H), np.int32)
    got_rgb, got_T, got_D, got_L = (x.cpu().numpy() for x in (out.rgb, out.T, out.depth, out.last))
    for tile in chosen:
        tile = int(tile)
        beg = int(te[tile - 2]) if tile > 1 else 0
        end = int(te[tile - 1])
        tx, ty = (tile - 1) % ntx + 1, (tile - 1) // ntx + 1
        oracle.blend_tile(cam, t, opts, f2d, depths, sv[beg:end].cpu().numpy(), beg, tx, ty, rgb, Ti, Di, Li)
        us = slice((tx - 1) * TW, min(tx * TW, W))
        vs = slice((ty - 1) * TH, min(ty * TH, H))
        np.testing.assert_array_equal(got_rgb[us, vs], rgb[us, vs], err_msg=f"tile {tile}")
        np.testing.assert_array_equal(got_T[us, vs], Ti[us, vs])
        np.testing.assert_array_equal(got_D[us, vs], Di[us, vs])
        np.testing.assert_array_equal(got_L[us, vs], Li[us, vs])
    assert lengths.max() > 10_000
    # backward: finite gradients everywhere
    gen = torch.Generator(device="cuda").manual_seed(0x3D6504)
    grad = ((torch.rand(out.rgb.shape, generator=gen, device="cuda") - 0.5) * 1e-4).contiguous()
    fg = gpu.FilteredGaussiansGradientsVector(buf.capacity, 3, 0)
    gpu.backward_(fg, grad, out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    for k in ["grads2d"] + ARRAYS:
        a = getattr(fg, k)[:nf]
        assert bool(torch.isfinite(a).all()), k
    assert float(fg.grads2d[:nf].abs().sum()) > 0
    del fg
    # backward parity on the 16 tiles (backward_core.jl:96-293 over lists of > 10,000 entries):
    # the image gradient kept on those tiles only, the GPU's 2D gradients against the oracle's
    # per-tile replay on the GPU's own lists, T and last contributors, then the 3D gradients
    # through the oracle's backward projection
    mask = torch.zeros((W, H, 1), dtype=torch.float32, device="cuda")
    for tile in chosen:
        tx, ty = (int(tile) - 1) % ntx + 1, (int(tile) - 1) // ntx + 1
        mask[(tx - 1) * TW:min(tx * TW, W), (ty - 1) * TH:min(ty * TH, H)] = 1.0
    grad16 = (grad * mask).contiguous()
    fg = gpu.FilteredGaussiansGradientsVector(buf.capacity, 3, 0)
    gpu.backward_(fg, grad16, out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    grad16_h = grad16.cpu().numpy()
    acc = np.zeros((nf, 9), np.float64)
    for tile in chosen:
        tile = int(tile)
        beg = int(te[tile - 2]) if tile > 1 else 0
        end = int(te[tile - 1])
        tx, ty = (tile - 1) % ntx + 1, (tile - 1) // ntx + 1
        oracle.backward_tile(cam, t, opts, f2d, sv[beg:end].cpu().numpy(), beg, tx, ty, grad16_h, got_T, got_L, acc)
    g2_ref = acc.astype(np.float32)
    touched = np.abs(g2_ref).sum(axis=1) > 0
    # (the large Gaussians of cfg4 saturate T within the first entries of a list: a few hundred
    # Gaussians reach the 16 tiles' pixels)
    assert touched.sum() > 100
    got2 = fg.grads2d[:nf].cpu().numpy()
    assert rel_l2(got2, g2_ref) <= REL_L2, rel_l2(got2, g2_ref)
    assert not np.abs(got2[~touched]).any()
    fwd = {"nb_fgaussians": nf, "fgidx_to_gidx": buf.fgidx_to_gidx[:nf].cpu().numpy(), "f2d": f2d,
           "counts": buf.counts[:nf].cpu().numpy()}
    ref3 = oracle.backward_project(w.gaussians, cam, opts, fwd, g2_ref)
    for k in ARRAYS:
        e = rel_l2(getattr(fg, k)[:nf].cpu().numpy(), ref3[k])
        assert e <= REL_L2, (k, e)


def test_cfg2_timed_variant_bit_exact(gpu, oracle):
    """The render the bench times, at full cfg2 size: device-side counts, rgb and T without
    depth or last contributors, 16x16 tiles, key arrays sized by host-count renders first, two
    frames back to back without a host synchronisation; the second frame bit for bit against
    the oracle (images, counts, tile lists)."""
    from tdgs_amd import abi
    w = synthetic.config(2, cameras=4)
    assert len(w.gaussians.means_opacity) == 1_000_000
    cams = w.cameras
    t = synthetic.tiling_for(w, cams[0])
    assert (t.tile_width, t.tile_height) == (16, 16)
    opts = host.RenderOptions.for_camera(cams[0], 3)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    out = gpu.RenderOutputs.for_camera(cams[0], 0, include_rgb=True, include_transmittance=True,
                                       include_depth=False, include_last_contributing_indices=False)
    buf = gpu.RenderBuffers(len(g), t, 0)
    for c in cams[2:4]:
        gpu.render_(out, g, c, t, opts, buf)
    out.rgb.fill_(-1.0)
    out.T.fill_(-1.0)
    gpu.render_(out, g, cams[2], t, opts, buf, device_counts=True)
    gpu.render_(out, g, cams[3], t, opts, buf, device_counts=True)
    torch.cuda.synchronize()
    r = oracle.render(w.gaussians, cams[3], t, opts)
    nbf, m, nb, status = buf.frame_counts()
    assert status == abi.TDGS_FRAME_OK
    assert (nbf, m) == (r["nb_fgaussians"], r["nb_keys"]) and m > 3_000_000
    np.testing.assert_array_equal(out.rgb.cpu().numpy(), r["rgb"])
    np.testing.assert_array_equal(out.T.cpu().numpy(), r["T"])
    np.testing.assert_array_equal(buf.tiles_end.cpu().numpy(), r["tiles_end"])
    np.testing.assert_array_equal(buf.sorted_values[:m].cpu().numpy(), r["sorted_values"][:m])


def _check_adc_step(adc, parents, moments, n_new, new, new_moments, log_split):
    """The invariants of one adaptive_density_control! step, on the device. Returns the
    numbers of pruned, cloned and split Gaussians."""
    n = parents["means_opacity"].shape[0]
    prune = adc.prune[:n].bool()
    dens = adc.densify[:n].bool()
    clone = adc.clone[:n].bool() & dens
    split = dens & ~adc.clone[:n].bool()
    cnt = (~prune).to(torch.int64) + dens.to(torch.int64)
    assert int(cnt.sum()) == n_new == len(new)
    parent = torch.repeat_interleave(torch.arange(n, device="cuda"), cnt)
    assert torch.equal(adc.ngidx[:n_new].to(torch.int64) - 1, parent)
    first = torch.cumsum(cnt, 0) - cnt            # new slot of each kept parent's first copy
    carried, cl, sp = ~prune & ~dens, clone, split
    for key in ("means_opacity", "scaling", "rotation", "sh"):
        old, cur = parents[key], getattr(new, key)
        assert torch.equal(cur[first[carried]], old[carried]), key
        assert torch.equal(cur[first[cl]], old[cl]), key
        assert torch.equal(cur[first[cl] + 1], old[cl]), key
    for key in ("rotation", "sh"):
        old, cur = parents[key], getattr(new, key)
        assert torch.equal(cur[first[sp]], old[sp]) and torch.equal(cur[first[sp] + 1], old[sp]), key
    old_mo, cur_mo = parents["means_opacity"], new.means_opacity
    for j in (0, 1):
        assert torch.equal(cur_mo[first[sp] + j, 3], old_mo[sp, 3])
        expect = parents["scaling"][sp] + torch.tensor(np.float32(log_split), device="cuda")
        assert torch.equal(new.scaling[first[sp] + j], expect)
    for key in ("means", "opacity", "scaling", "rotation", "sh"):
        old, cur = moments[key], getattr(new_moments, key)
        assert torch.equal(cur[first[carried]], old[carried]), key
        assert torch.equal(cur[first[cl]], old[cl]), key
        assert not bool(cur[first[cl] + 1].any()), key
        assert not bool(cur[first[sp]].any()) and not bool(cur[first[sp] + 1].any()), key
    if int(sp.sum()) >= 2000:
        # split means: parent + R (z * s), z ~ N(0, I) (gaussians.jl:1617): z recovered as
        # R^T (new - parent) / s has mean ~0 and covariance ~I
        q = parents["rotation"][sp].double()
        q = q / q.norm(dim=1, keepdim=True)
        r_, x, y, z = q.unbind(1)
        R = torch.stack([
            torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - r_ * z), 2 * (x * z + r_ * y)], 1),
            torch.stack([2 * (x * y + r_ * z), 1 - 2 * (x * x + z * z), 2 * (y * z - r_ * x)], 1),
            torch.stack([2 * (x * z - r_ * y), 2 * (y * z + r_ * x), 1 - 2 * (x * x + y * y)], 1)], 1)
        s = torch.exp(parents["scaling"][sp].double())
        zs = []
        for j in (0, 1):
            d = cur_mo[first[sp] + j, :3].double() - old_mo[sp, :3].double()
            zs.append(torch.einsum("nji,nj->ni", R, d) / s)
        zz = torch.cat(zs).cpu().numpy()
        assert np.all(np.abs(zz.mean(0)) < 0.06), zz.mean(0)
        cov = np.cov(zz.T)
        assert np.allclose(cov, np.eye(3), atol=0.1), cov
    return int(prune.sum()), int(cl.sum()), int(sp.sum())


@pytest.mark.parametrize("grad_threshold", [2e-4, 3.5e-5])
def test_cfg3_training_loop(gpu, monkeypatch, grad_threshold):
    """All 3000 iterations of cfg3: 25 density-control steps (600, 700, ..., 3000) and the
    opacity reset at 3000. With the reference's gradient threshold (2e-4) the count stays near
    500k; with 3.5e-5 it grows past 1M (the config's "up to ~1.5M"), which also grows the
    per-Gaussian and key arrays between steps."""
    w = synthetic.config(3)
    cams = w.cameras
    tiling = synthetic.tiling_for(w, cams[0])
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    gen = torch.Generator(device="cuda").manual_seed(0x3D6503)
    images = [torch.rand((c.width, c.height, 3), generator=gen, device="cuda") for c in cams]
    opts = host.RenderOptions.for_camera(cams[0], 3)
    to = training.TrainingOptions.for_scene(host.scene_radius(cams), nb_iterations=3000,
                                            densification_mean2d_grad_norm_threshold_ndc=grad_threshold)
    tr = training.Trainer(g, cams, images, opts, tiling, to, seed=3)
    log_split = float(np.log(np.float32(to.splitting_scale_factor)))
    records = []
    orig = training.adaptive_density_control_

    def checked(adc, gaussians, optimizer, n_new, log_split_factor, seed):
        assert log_split_factor == log_split
        parents = {k: getattr(gaussians, k).clone() for k in ("means_opacity", "scaling", "rotation", "sh")}
        om = optimizer.moments
        moments = {k: getattr(om, k).clone() for k in ("means", "opacity", "scaling", "rotation", "sh")}
        n_old = len(gaussians)
        new = orig(adc, gaussians, optimizer, n_new, log_split_factor, seed)
        pruned, cloned, split = _check_adc_step(adc, parents, moments, n_new, new, optimizer.moments, log_split)
        records.append({"iteration": tr.iteration_nb, "before": n_old, "after": n_new, "pruned": pruned,
                        "cloned": cloned, "split": split})
        return new

    monkeypatch.setattr(training, "adaptive_density_control_", checked)
    losses = []
    key_capacity0 = tr.render_buffers.key_capacity
    nmax = len(tr.gaussians)
    for it in range(3000):
        tr.training_step_()
        nmax = max(nmax, len(tr.gaussians))
        if (it + 1) % 100 == 0 or it + 1 in (601, 701):
            losses.append(tr.current_loss())
        if tr.iteration_nb == 2999:
            big = (tr.gaussians.means_opacity[:, 3] > host.logit32(to.opacity_reset_max_value)).sum()
            assert int(big) > 1000
    tr.finish_()
    torch.cuda.synchronize()
    print(records)
    assert [r["iteration"] for r in records] == list(range(600, 3001, 100))
    assert all(math.isfinite(x) for x in losses)
    # every step applied once (a device-count step whose keys did not fit is run again)
    assert tr.optimizer.update_count == tr.iteration_nb == 3000
    # the opacity reset of iteration 3000 (after that step's density control): every opacity
    # logit at most logit(0.01), the opacity moments zero
    lim = torch.tensor(host.logit32(to.opacity_reset_max_value), device="cuda")
    assert bool((tr.gaussians.means_opacity[:, 3] <= lim).all())
    assert not bool(tr.optimizer.moments.opacity.any())
    for name in ("means_opacity", "scaling", "rotation", "sh"):
        assert bool(torch.isfinite(getattr(tr.gaussians, name)).all()), name
    if grad_threshold < 2e-4:
        assert nmax > 1_000_000, records
        assert tr.render_buffers.capacity >= nmax and tr.render_buffers.key_capacity > key_capacity0
    else:
        assert max(r["after"] for r in records) < 550_000
