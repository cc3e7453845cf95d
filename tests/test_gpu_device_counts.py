"""render! without host synchronisation (TDGS_FLAG_DEVICE_COUNTS), through the C-ABI.

The launches after the count scan are sized by the key capacity and read N_f, M and the
non-empty count on the device (the reference reads them on the host every frame,
forward_core.jl:231-233, 259-264). Checked here:
- the render is bit-exact against the oracle (lists, tile ranges, images), with one and with
  two radix passes over the tile ids; tdgs_render_counts returns the counts and the frame
  monitor records the frame;
- a frame whose keys do not fit the key arrays renders as render_void! with status
  TDGS_FRAME_KEY_CAPACITY and the needed key count; the fused backward projection + Adam and
  the ADC statistics then leave everything untouched;
- nothing visible: render_void!'s outputs and zero counts;
- backward! with nb_fgaussians = -1 against the oracle, and the fused Adam step with the device
  count equal to the one with the host count, bit for bit;
- the trainer: a step whose keys did not fit is skipped on the device and counted, and the
  key arrays grow from the frame monitor before the next step.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from tdgs_amd import abi, host, synthetic, training
from test_gpu_backward import ARRAYS, REL_L2, rel_l2
from test_gpu_forward import _assert_forward_equal

pytestmark = pytest.mark.gpu


def _monitor(gpu):
    p = C.POINTER(C.c_int64)()
    gpu.check(gpu.lib().tdgs_ctx_frame_monitor(gpu.context(0), C.byref(p)))
    return [int(p[i]) for i in range(4)]


def _device_render(gpu, g, cam, t, opts, key_capacity=None, depth=True):
    out = gpu.RenderOutputs.for_camera(cam, 0, include_depth=depth)
    buf = gpu.RenderBuffers(len(g), t, 0, key_capacity, keep_flags=True)
    gpu.render_(out, g, cam, t, opts, buf, device_counts=True)
    assert buf.nb_fgaussians == -1 and buf.nb_keys == -1
    torch.cuda.synchronize()
    return out, buf


@pytest.mark.parametrize("cfg,n,size", [(0, None, None), (1, 20_000, None), (0, None, (200, 150))])
def test_device_counts_render_matches_oracle(gpu, oracle, cfg, n, size):
    w = synthetic.config(cfg, n=n)
    cam = w.cameras[0]
    if size is not None:   # <= 256 tiles: the tile sort is the fused emission pass alone
        cam = host.look_at_camera(size[0], size[1], 60.0, (0.0, 0.0, -4.0))
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, w.gaussians.sh_degree, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(w.gaussians, cam, t, opts)
    assert r["nb_keys"] > 1000
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    before = _monitor(gpu)
    out, buf = _device_render(gpu, g, cam, t, opts, key_capacity=r["nb_keys"])   # (exactly enough)
    nbf, m, nb, status = buf.frame_counts()
    assert (nbf, m, status) == (r["nb_fgaussians"], r["nb_keys"], abi.TDGS_FRAME_OK)
    assert nb == int((r["counts"][:nbf] > 0).sum())
    assert (buf.nb_fgaussians, buf.nb_keys) == (nbf, m)
    _assert_forward_equal(r, out, buf)
    after = _monitor(gpu)
    assert after[0] == before[0] + 1 and after[2] == before[2]
    assert after[3] == m and after[1] >= m


def test_device_counts_key_overflow(gpu):
    w = synthetic.config(1, n=20_000)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 3, background_color=(0.25, 0.5, 0.75))
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    out0 = gpu.RenderOutputs.for_camera(cam, 0)
    buf0 = gpu.RenderBuffers(len(g), t, 0)
    gpu.render_(out0, g, cam, t, opts, buf0)
    m_true = buf0.nb_keys
    assert m_true > 10_000
    before = _monitor(gpu)
    out, buf = _device_render(gpu, g, cam, t, opts, key_capacity=m_true // 2)
    nbf, m, nb, status = buf.frame_counts()
    assert status == abi.TDGS_FRAME_KEY_CAPACITY and m == m_true and nbf == buf0.nb_fgaussians
    after = _monitor(gpu)
    assert after[2] == before[2] + 1 and after[3] == m_true
    rgb = out.rgb.cpu().numpy()
    for c, v in enumerate((0.25, 0.5, 0.75)):
        np.testing.assert_array_equal(rgb[..., c], np.float32(v))
    assert np.all(out.T.cpu().numpy() == 1) and np.all(out.last.cpu().numpy() == 0)
    assert np.all(np.isinf(out.depth.cpu().numpy()))
    # the step on that frame leaves the parameters, moments and ADC statistics untouched
    buf.nb_fgaussians = buf.nb_keys = -1
    fg = gpu.FilteredGaussiansGradientsVector(buf.capacity, 3, 0)
    gen = torch.Generator(device="cuda").manual_seed(4)
    fg.grads2d.copy_(torch.rand(fg.grads2d.shape, generator=gen, device="cuda"))
    to = training.TrainingOptions.for_scene(4.4)
    opt = training.AdamOptimizer(g, to)
    p0 = [x.clone() for x in (g.means_opacity, g.scaling, g.rotation, g.sh, opt.moments.sh)]
    opt.backward_project_update_(fg, cam, opts, buf)
    adc = training.AdaptiveDensityControlBuffers(len(g), 0)
    training.adc_stats_(adc, fg, buf.fgidx_to_gidx, -1, cam, buf)
    adc_fused = training.AdaptiveDensityControlBuffers(len(g), 0)   # (tdgs_backward_project_adam_adc)
    opt.backward_project_update_(fg, cam, opts, buf, adc=adc_fused)
    torch.cuda.synchronize()
    for a, b in zip(p0, (g.means_opacity, g.scaling, g.rotation, g.sh, opt.moments.sh)):
        assert torch.equal(a, b)
    for st in (adc, adc_fused):
        assert int(st.counts.sum()) == 0 and float(st.accum.abs().sum()) == 0.0


def test_device_counts_nothing_visible(gpu):
    g_host, cams = host.create_test_scene(sh_degree=0)
    g_host.means_opacity[:, 2] = -5.0  # everything behind the camera
    cam = cams[0]
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.25, 0.5, 0.75))
    t = host.Tiling.for_camera(cam, 16, 16)
    g = gpu.TrainableGaussiansVector.from_host(g_host, 0)
    out, buf = _device_render(gpu, g, cam, t, opts)
    assert buf.frame_counts() == (0, 0, 0, abi.TDGS_FRAME_OK)
    rgb = out.rgb.cpu().numpy()
    np.testing.assert_array_equal(rgb[..., 0], np.float32(0.25))
    np.testing.assert_array_equal(rgb[..., 2], np.float32(0.75))
    assert np.all(out.T.cpu().numpy() == 1) and np.all(out.last.cpu().numpy() == 0)
    assert np.all(np.isinf(out.depth.cpu().numpy()))


def test_device_counts_backward(gpu, oracle):
    w = synthetic.config(1, n=20_000)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 3)
    r = oracle.render(w.gaussians, cam, t, opts)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    out, buf = _device_render(gpu, g, cam, t, opts, key_capacity=2 * r["nb_keys"], depth=False)
    gen = torch.Generator(device="cuda").manual_seed(2)
    grad = ((torch.rand(out.rgb.shape, generator=gen, device="cuda") - 0.5) * 1e-3).contiguous()
    fg = gpu.FilteredGaussiansGradientsVector(buf.capacity, 3, 0)
    gpu.backward_(fg, grad, out, g, cam, t, opts, buf)   # nb_fgaussians = -1
    torch.cuda.synchronize()
    nf = r["nb_fgaussians"]
    ref = oracle.backward(w.gaussians, cam, t, opts, r, grad.cpu().numpy())
    assert rel_l2(fg.grads2d[:nf].cpu().numpy(), ref["grads2d"]) <= REL_L2
    for k in ARRAYS:
        assert rel_l2(getattr(fg, k)[:nf].cpu().numpy(), ref[k]) <= REL_L2, k
    assert float(fg.grads2d[nf:].abs().sum()) == 0.0   # zeroed over the whole capacity
    # fused backward projection + Adam: device count and host count, same 2D gradients
    results = []
    for count in (-1, nf):
        gg = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
        opt = training.AdamOptimizer(gg, training.TrainingOptions.for_scene(4.4))
        buf.nb_fgaussians = count
        opt.backward_project_update_(fg, cam, opts, buf)
        torch.cuda.synchronize()
        results.append([x.cpu() for x in (gg.means_opacity, gg.scaling, gg.rotation, gg.sh, opt.moments.sh)])
    for a, b in zip(*results):
        assert torch.equal(a, b)


def _trainer(gpu, device_counts):
    w = synthetic.config(1, n=20_000, cameras=2)
    cams = w.cameras
    tiling = synthetic.tiling_for(w, cams[0])
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    gen = torch.Generator(device="cuda").manual_seed(3)
    images = [torch.rand((c.width, c.height, 3), generator=gen, device="cuda") for c in cams]
    opts = host.RenderOptions.for_camera(cams[0], 3)
    to = training.TrainingOptions.for_scene(4.4)
    return training.Trainer(g, cams, images, opts, tiling, to, seed=1, device_counts=device_counts)


def test_trainer_reruns_overflowing_step_and_grows_keys(gpu):
    """A device-count step whose keys do not fit is left undone by the device and run again
    with host counts before the next step: every step is applied once, in order, as a trainer
    with host counts applies it (the Adam moments would differ by a whole step otherwise)."""
    tr = _trainer(gpu, True)
    g = tr.gaussians
    tr.render_buffers._alloc_keys(1000)   # far too small: the first step's keys do not fit
    before = [x.clone() for x in (g.means_opacity, g.sh)]
    tr.training_step_()
    torch.cuda.synchronize()
    assert tr.render_buffers.nb_fgaussians == -1   # a device-count step
    for a, b in zip(before, (g.means_opacity, g.sh)):
        assert torch.equal(a, b)                   # left undone on the device
    assert tr.render_buffers.frame_counts()[3] == abi.TDGS_FRAME_KEY_CAPACITY
    tr.render_buffers.nb_fgaussians = tr.render_buffers.nb_keys = -1   # as the step left them
    tr.confirm_device_count_step_()                # runs the step again with host counts
    torch.cuda.synchronize()
    assert tr.replayed_steps == 1
    assert tr.render_buffers.key_capacity > 1000 and tr.render_buffers.nb_keys > 1000
    assert not torch.equal(before[0], g.means_opacity)
    assert tr.optimizer.update_count == tr.iteration_nb == 1
    for _ in range(3):
        tr.training_step_()
    tr.finish_()
    assert tr.replayed_steps == 1 and tr.optimizer.update_count == tr.iteration_nb == 4
    nbf, m, _, status = tr.render_buffers.frame_counts()
    assert status == abi.TDGS_FRAME_OK and m <= tr.render_buffers.key_capacity
    assert np.isfinite(tr.current_loss())
    # the same four steps with host counts: the same state up to the order of the float
    # atomics of backward blending (which can flip the sign of an Adam step where a gradient
    # is near 0: ~2.5e-5 of the parameters' norm; a step left out would be ~1e-2)
    ref = _trainer(gpu, False)
    for _ in range(4):
        ref.training_step_()
    ref.finish_()
    assert ref.replayed_steps == 0 and ref.optimizer.update_count == 4
    for name in ("means", "opacity", "scaling", "rotation", "sh"):
        a = getattr(tr.optimizer.moments, name).double()
        b = getattr(ref.optimizer.moments, name).double()
        assert float((a - b).norm()) <= 1e-4 * float(b.norm()), name
    for name in ("means_opacity", "scaling", "rotation"):
        a = getattr(tr.gaussians, name).double()
        b = getattr(ref.gaussians, name).double()
        assert float((a - b).norm()) <= 3e-4 * float(b.norm()), name
    # the density-control statistics (accumulated inside the fused backward projection + Adam
    # in these steps) count the replayed step once: the left-undone launch added nothing (a
    # second count would change every Gaussian seen in that step; the two trainers' slightly
    # different parameters may move a few across a visibility boundary)
    assert tr.fuse_optimizer and tr.iteration_nb <= tr.options.adc_final_iteration_nb
    seen = int((ref.adc.counts > 0).sum())
    assert seen > 1000
    assert int((tr.adc.counts != ref.adc.counts).sum()) <= max(2, seen // 1000)
    a, b = tr.adc.accum.double(), ref.adc.accum.double()
    assert float((a - b).norm()) <= 1e-3 * float(b.norm())


@pytest.mark.parametrize("device_counts", [False, True])
def test_kept_but_nothing_on_screen(gpu, oracle, device_counts):
    """Gaussians in front of the camera but far to its side: all kept (clamp mode keeps by
    depth alone, forward_core.jl:326-355), none with a tile rectangle on the screen, so the
    depth presort keeps no pair, M = 0 and the frame is the background."""
    import copy
    w = synthetic.config(0, n=5000)
    cam = w.cameras[0]
    g_host = copy.deepcopy(w.gaussians)
    g_host.means_opacity[:, :3] += np.float32(1000.0) * cam.R_c2w[:, 0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.25, 0.5, 0.75))
    r = oracle.render(g_host, cam, t, opts)
    assert r["nb_fgaussians"] > 0 and r["nb_keys"] == 0
    g = gpu.TrainableGaussiansVector.from_host(g_host, 0)
    if device_counts:
        out, buf = _device_render(gpu, g, cam, t, opts, key_capacity=1024)
        assert buf.frame_counts() == (r["nb_fgaussians"], 0, 0, abi.TDGS_FRAME_OK)
    else:
        out = gpu.RenderOutputs.for_camera(cam, 0, include_depth=True)
        buf = gpu.RenderBuffers(len(g), t, 0)
        gpu.render_(out, g, cam, t, opts, buf)
        torch.cuda.synchronize()
        assert (buf.nb_fgaussians, buf.nb_keys) == (r["nb_fgaussians"], 0)
    np.testing.assert_array_equal(out.rgb.cpu().numpy(), r["rgb"])
    np.testing.assert_array_equal(out.T.cpu().numpy(), r["T"])
    assert np.all(out.T.cpu().numpy() == 1) and np.all(out.last.cpu().numpy() == 0)
