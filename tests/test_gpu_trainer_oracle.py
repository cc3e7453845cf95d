"""training_step! on the GPU against the same steps driven through the CPU oracle.

The Trainer (training.jl:173-244) runs eight iterations across a density-control step with
the optimiser fused into the backward projection and without (fused, the steps without density
control render with device-side counts: no host synchronisation): the ADC at iteration 600
(the first), at 3000 (also the opacity reset, training.jl:272-280, whose iteration does not yet
prune by size) and at 3100 (the first that also prunes Gaussians larger than
pruning_3d_max_scale, training.jl:337-349; the threshold is set so that some are).
Each iteration is replayed on the CPU with the oracle's functions in the reference's order:
render! (checked bit for bit against the GPU's image), the backward projection from the GPU's
2D gradients of that iteration, the ADC statistics, at iteration 600 the masks, compaction
(same split sampler and seed) and fgidx remap, the annealed means learning rate, and update!.
The Gaussians, the Adam moments and the update count must then equal the GPU's bit for bit
after every iteration: this pins the step's orchestration (what runs, in which order, on which
index maps). The 2D gradients are the GPU's own because the float atomics of backward blending
sum in a different order than the oracle (that kernel is checked at relative L2 1e-3
elsewhere); everything downstream of them is deterministic.
"""
import numpy as np
import pytest
import torch

from tdgs_amd import host, synthetic, training

pytestmark = pytest.mark.gpu


def _host_state(tr):
    g = tr.gaussians.to_host()
    m = tr.optimizer.moments
    adam = {k: getattr(m, k).cpu().numpy() for k in ("means", "opacity", "scaling", "rotation", "sh")}
    return g, adam


@pytest.mark.parametrize("fuse,start", [(True, 595), (False, 595), (True, 2995), (True, 3095), (False, 3095)])
def test_trainer_steps_match_oracle_driven_steps(gpu, oracle, monkeypatch, fuse, start):
    w = synthetic.config(3, n=20_000, cameras=4)
    cams = w.cameras
    tiling = synthetic.tiling_for(w, cams[0])
    g0 = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    gen = torch.Generator(device="cuda").manual_seed(5)
    images = [torch.rand((c.width, c.height, 3), generator=gen, device="cuda") for c in cams]
    ropts = host.RenderOptions.for_camera(cams[0], 3)
    radius = host.scene_radius(cams)
    # a max-scale prune threshold that ~4% of the Gaussians exceed
    smax = w.gaussians.scaling.max(axis=1)
    base_max_scale = float(np.exp(np.quantile(smax, 0.96)) / radius)
    # thresholds that make the ADC prune, clone and split some of 20k Gaussians
    to = training.TrainingOptions.for_scene(radius, nb_iterations=30_000,
                                            densification_mean2d_grad_norm_threshold_ndc=1e-6,
                                            base_densification_size_threshold=0.003, pruning_min_opacity=0.1,
                                            base_pruning_3d_max_scale=base_max_scale)
    tr = training.Trainer(g0, cams, images, ropts, tiling, to, seed=9, fuse_optimizer=fuse)
    tr.iteration_nb = start
    tr.optimizer.update_count = start

    captured = []
    orig_b2, orig_b = training.backward_render_tiles_, training.backward_

    def nbf_of(buf):
        if buf.nb_fgaussians >= 0:
            return buf.nb_fgaussians
        # a device-count step: read the count (a synchronisation the trainer does not make)
        # and leave the buffers as the step left them, so that the rest of the step still
        # takes the count from the device
        n = buf.frame_counts()[0]
        buf.nb_fgaussians = buf.nb_keys = -1
        return n

    def cap_b2(fg, grad, out, cam, t, o, buf):
        r = orig_b2(fg, grad, out, cam, t, o, buf)
        captured.append(fg.grads2d_matrix(nbf_of(buf)).cpu().numpy().copy())
        return r

    def cap_b(fg, grad, out, g, cam, t, o, buf):
        r = orig_b(fg, grad, out, g, cam, t, o, buf)
        captured.append(fg.grads2d_matrix(nbf_of(buf)).cpu().numpy().copy())
        return r

    monkeypatch.setattr(training, "backward_render_tiles_", cap_b2)
    monkeypatch.setattr(training, "backward_", cap_b)

    g, moments = _host_state(tr)
    adam = oracle.AdamHost(len(g.means_opacity), 3, tr.optimizer.moments.lrs(), update_count=start)
    for k, v in moments.items():
        getattr(adam, k)[...] = v
    adc = oracle.AdcHost(len(g.means_opacity))
    f32 = np.float32
    adc_steps = 0
    resets = 0
    for step in range(8):
        tr.training_step_()
        torch.cuda.synchronize()
        it = tr.iteration_nb
        cam = tr.last_camera
        # fused steps without density control render with device-side counts
        is_adc = it % to.adc_interval == 0 and to.adc_start_iteration_nb <= it <= to.adc_final_iteration_nb
        assert (tr.render_buffers.nb_fgaussians == -1) == (fuse and not is_adc)
        assert len(captured) == step + 1
        g2 = captured[-1]
        fwd = oracle.render(g, cam, tiling, ropts)
        nf = fwd["nb_fgaussians"]
        assert g2.shape[0] == nf
        np.testing.assert_array_equal(tr.render_outputs.rgb.cpu().numpy(), fwd["rgb"])
        grads = oracle.backward_project(g, cam, ropts, fwd, g2)
        f2g = fwd["fgidx_to_gidx"][:nf]
        oracle.adc_stats(adc, g2, f2g, cam.width, cam.height)
        if it % to.adc_interval == 0 and to.adc_start_iteration_nb <= it <= to.adc_final_iteration_nb:
            prune_logit = float(host.logit32(to.pruning_min_opacity))
            log_max_scale = float(np.log(f32(to.pruning_3d_max_scale)))
            n_new = oracle.adc_plan(adc, g, prune_logit, it > to.opacity_reset_interval, log_max_scale,
                                    to.densification_mean2d_grad_norm_threshold_ndc,
                                    float(np.log(f32(to.densification_size_threshold))))
            n_old = len(g.means_opacity)
            assert int(adc.prune.sum()) > 0 and int((adc.densify & adc.clone).sum()) > 0
            assert int((adc.densify & ~adc.clone.astype(bool)).sum()) > 0
            # Gaussians pruned for their size alone, exactly from iteration 3100 on
            by_size = adc.prune.astype(bool) & (g.means_opacity[:, 3] >= f32(prune_logit))
            big = g.scaling.max(axis=1) > f32(log_max_scale)
            assert big.sum() > 100
            assert (by_size.sum() > 0) == (it > to.opacity_reset_interval), (it, by_size.sum())
            g, adam = oracle.adc_apply(adc, g, adam, float(np.log(f32(to.splitting_scale_factor))),
                                       tr.seed * 1_000_003 + it)
            f2g = oracle.adc_remap_fgidx(adc, f2g)
            adc = oracle.AdcHost(n_new)
            adc_steps += 1
            assert len(g.means_opacity) == n_new != n_old
        adam.lrs[0] = training.annealed_means_lr(it, to)
        oracle.adam_step(g, adam, grads, f2g, ropts.sh_degree)
        if it % to.opacity_reset_interval == 0 and \
                to.opacity_reset_start_iteration_nb <= it <= to.opacity_reset_final_iteration_nb:
            # reset_opacities! + zero_opacity_features_adam_moments! (gaussians.jl:1093-1101)
            lim = f32(host.logit32(to.opacity_reset_max_value))
            assert (g.means_opacity[:, 3] > lim).sum() > 100
            g.means_opacity[:, 3] = np.minimum(g.means_opacity[:, 3], lim)
            adam.opacity[...] = 0
            resets += 1
        got_g, got_m = _host_state(tr)
        for k in ("means_opacity", "scaling", "rotation", "sh"):
            np.testing.assert_array_equal(getattr(got_g, k), getattr(g, k), err_msg=f"iteration {it}: {k}")
        for k in ("means", "opacity", "scaling", "rotation", "sh"):
            np.testing.assert_array_equal(got_m[k], getattr(adam, k), err_msg=f"iteration {it}: moments {k}")
        assert tr.optimizer.update_count == adam.update_count == it
        assert tr.optimizer.moments.means_lr == adam.lrs[0]
    assert adc_steps == 1
    assert resets == (1 if start == 2995 else 0)
    assert tr.replayed_steps == 0
