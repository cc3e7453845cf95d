"""The Trainer (training_step!, training.jl:173-244) end to end on the GPU: SH ramp, loss,
backward, statistics, densification, learning-rate annealing, Adam and opacity reset, with
the iteration schedule shortened so every branch runs within a few steps."""
import numpy as np
import pytest
import torch

from tdgs_amd import host, synthetic

pytestmark = pytest.mark.gpu


def test_training_steps_exercise_every_branch(gpu):
    from tdgs_amd import training
    w = synthetic.config(1, n=20_000)
    cams = synthetic.orbit_cameras(np.random.default_rng(0), 4, 320, 240, 4.0, 60.0)
    g_host = w.gaussians
    g_host = host.HostGaussians(g_host.means_opacity, g_host.scaling, g_host.rotation,
                                np.ascontiguousarray(g_host.sh[:, :, :1]))  # start at SH degree 0
    g = gpu.TrainableGaussiansVector.from_host(g_host, 0)
    gen = torch.Generator(device="cuda").manual_seed(1)
    images = [torch.rand((320, 240, 3), generator=gen, device="cuda") for _ in cams]
    opts = host.RenderOptions.for_camera(cams[0], 0)
    tiling = host.Tiling.for_camera(cams[0], 16, 16)
    to = training.TrainingOptions.for_scene(host.scene_radius(cams), nb_iterations=40,
                                            sh_degree_increase_interval=5, adc_start_iteration_nb=10,
                                            adc_interval=10, opacity_reset_interval=15,
                                            densification_mean2d_grad_norm_threshold_ndc=1e-6)
    tr = training.Trainer(g, cams, images, opts, tiling, to, seed=3)
    sizes, losses = [], []
    for _ in range(40):
        tr.training_step_()
        sizes.append(len(tr.gaussians))
        losses.append(tr.current_loss())
    torch.cuda.synchronize()
    assert tr.gaussians.sh_degree == 3 and tr.render_options.sh_degree == 3
    assert tr.optimizer.update_count == 40
    assert sizes[8] == 20_000 and sizes[-1] != 20_000  # densification changed the count
    assert np.all(np.isfinite(losses))
    for t in (tr.gaussians.means_opacity, tr.gaussians.scaling, tr.gaussians.rotation, tr.gaussians.sh):
        assert torch.isfinite(t).all()
    assert len(tr.optimizer.moments) == len(tr.gaussians)
    assert tr.optimizer.moments.sh.shape[2] == 16


def test_host_images_upload_ahead(gpu):
    """GroundTruthImages with host images: uploads run one step ahead on the copy stream and
    every acquire sees exactly its image, also when a camera repeats at once."""
    from tdgs_amd import training
    rng = np.random.default_rng(4)
    imgs = [rng.random((64, 48, 3), dtype=np.float32) for _ in range(3)]
    ref = [torch.from_numpy(im).cuda() for im in imgs]
    gt = training.GroundTruthImages(imgs, torch.device("cuda", 0))
    assert not gt.on_device
    seq = [0, 1, 2, 2, 1, 0, 0, 0, 1, 2, 1]
    scratch = torch.empty((2048, 2048), device="cuda")
    for i, k in enumerate(seq):
        gt.prefetch(k)
        if i + 1 < len(seq):
            gt.prefetch(seq[i + 1])
        scratch.normal_()          # unrelated work on the compute stream
        img = gt.acquire(k)
        assert torch.equal(img, ref[k])
        gt.release(k)


def test_host_images_match_device_images(gpu):
    """Training on host images (pinned, uploaded one step ahead) follows training on the same
    images on the device: the same camera order across permutation boundaries and the same
    losses (up to the order of the gradient atomics, which differs from run to run)."""
    from tdgs_amd import training
    w = synthetic.config(1, n=20_000)
    cams = synthetic.orbit_cameras(np.random.default_rng(0), 3, 320, 240, 4.0, 60.0)
    rng = np.random.default_rng(5)
    host_imgs = [rng.random((320, 240, 3), dtype=np.float32) for _ in cams]
    opts = host.RenderOptions.for_camera(cams[0], 3)
    tiling = host.Tiling.for_camera(cams[0], 16, 16)
    to = training.TrainingOptions.for_scene(host.scene_radius(cams), nb_iterations=100)
    runs = []
    for images in (host_imgs, [torch.from_numpy(im).cuda() for im in host_imgs]):
        g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
        tr = training.Trainer(g, cams, images, opts, tiling, to, seed=7)
        assert tr.images.on_device == (images is not host_imgs)
        order, losses = [], []
        for _ in range(10):
            tr.training_step_()
            order.append(next(i for i, c in enumerate(tr.cameras) if c is tr.last_camera))
            losses.append(tr.current_loss())
        torch.cuda.synchronize()
        runs.append((order, losses))
    (o1, l1), (o2, l2) = runs
    assert o1 == o2 and sorted(o1[:3]) == [0, 1, 2] and sorted(o1[3:6]) == [0, 1, 2]
    assert l1[0] == l2[0]
    np.testing.assert_allclose(l1, l2, rtol=1e-5)
