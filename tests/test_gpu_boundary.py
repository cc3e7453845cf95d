"""The C-ABI entry points a reference-side caller binds beyond render!/backward!:

- tdgs_project (the cull + compaction + projection half of render!, forward_core.jl:222-254)
  against the oracle, bit for bit;
- the reference's four-array layout of the 2D gradients (backward_structs.jl:17-22) through
  backward!, the fused backward projection + Adam and the ADC statistics, against the
  oracle and against the interleaved layout;
- streams, events and pinned host memory (the overlapped upload of training.jl:196-201);
- tdgs_ctx_check after a clean render;
- tile shapes whose pixel count is not a multiple of 64 (any TW x TH up to 1024 pixels, as
  forward_structs.jl:340-424 accepts), forward bit-exact and backward within rel. L2 1e-3.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from tdgs_amd import abi, host, synthetic, training
from test_gpu_backward import ARRAYS, REL_L2, rel_l2
from test_gpu_forward import _assert_forward_equal

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg,n", [(0, None), (1, 20_000)])
def test_project_matches_oracle(gpu, oracle, cfg, n):
    w = synthetic.config(cfg, n=n)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, w.gaussians.sh_degree)
    r = oracle.render(w.gaussians, cam, t, opts)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    buf = gpu.RenderBuffers(len(g), t, 0, keep_flags=True)
    nf = gpu.project_(g, cam, t, opts, buf)
    torch.cuda.synchronize()
    assert nf == r["nb_fgaussians"] > 0
    np.testing.assert_array_equal(buf.keep.cpu().numpy()[:len(g)], r["keep"])
    np.testing.assert_array_equal(buf.fgidx_to_gidx[:nf].cpu().numpy(), r["fgidx_to_gidx"][:nf])
    counts = buf.counts[:nf].cpu().numpy()
    np.testing.assert_array_equal(counts, r["counts"][:nf])
    ne = counts > 0
    for k in ("depths", "f2d", "tile_ranges"):
        np.testing.assert_array_equal(getattr(buf, k)[:nf].cpu().numpy()[ne], r[k][:nf][ne], err_msg=k)


def _backward(gpu, g, out, cam, t, opts, buf, grad, layout):
    fg = gpu.FilteredGaussiansGradientsVector(buf.capacity, g.sh_degree, 0, layout=layout)
    gpu.backward_(fg, grad, out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    return fg


def test_reference_gradient_layout(gpu, oracle):
    w = synthetic.config(1, n=20_000, cameras=2)
    cam = w.cameras[-1]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 3, background_color=(0.2, 0.1, 0.3))
    r = oracle.render(w.gaussians, cam, t, opts)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    out = gpu.RenderOutputs.for_camera(cam, 0)
    buf = gpu.RenderBuffers(len(g), t, 0)
    gpu.render_(out, g, cam, t, opts, buf)
    gen = torch.Generator(device="cuda").manual_seed(3)
    grad = ((torch.rand(out.rgb.shape, generator=gen, device="cuda") - 0.5) * 1e-3).contiguous()
    fi = _backward(gpu, g, out, cam, t, opts, buf, grad, "interleaved")
    fr = _backward(gpu, g, out, cam, t, opts, buf, grad, "reference")
    assert fr.grads2d is None and fr.mean2d.shape == (buf.capacity, 2) and fr.licov2d.shape == (buf.capacity, 3)
    nf = buf.nb_fgaussians
    ref = oracle.backward(w.gaussians, cam, t, opts, r, grad.cpu().numpy())
    got = fr.grads2d_matrix(nf).cpu().numpy()
    assert rel_l2(got, ref["grads2d"]) <= REL_L2
    assert rel_l2(got, fi.grads2d[:nf].cpu().numpy()) <= REL_L2
    for k in ARRAYS:
        assert rel_l2(getattr(fr, k)[:nf].cpu().numpy(), ref[k]) <= REL_L2, k
    # with the same 2D gradients in both layouts, the backward projection + Adam and the ADC
    # statistics are bit-identical
    fr.mean2d[:nf].copy_(fi.grads2d[:nf, 0:2])
    fr.opacity[:nf].copy_(fi.grads2d[:nf, 2])
    fr.licov2d[:nf].copy_(fi.grads2d[:nf, 3:6])
    fr.color[:nf].copy_(fi.grads2d[:nf, 6:9])
    results = []
    for fg in (fi, fr):
        gg = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
        to = training.TrainingOptions.for_scene(4.4)
        opt = training.AdamOptimizer(gg, to)
        opt.backward_project_update_(fg, cam, opts, buf)
        adc = training.AdaptiveDensityControlBuffers(len(gg), 0)
        training.adc_stats_(adc, fg, buf.fgidx_to_gidx, nf, cam)
        torch.cuda.synchronize()
        results.append([gg.means_opacity.cpu(), gg.scaling.cpu(), gg.rotation.cpu(), gg.sh.cpu(),
                        opt.moments.sh.cpu(), adc.accum.cpu(), adc.counts.cpu()])
    for a, b in zip(*results):
        assert torch.equal(a, b)
    assert int(results[0][-1].sum()) > 0


def test_streams_events_and_pinned_memory(gpu):
    """A pinned host buffer uploaded on a library-created stream; a second stream waits on
    the recorded event before reading the device copy back."""
    L = gpu.lib()
    n = 1 << 20
    s1, s2, ev, e0, e1 = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
    for s in (s1, s2):
        gpu.check(L.tdgs_stream_create(C.byref(s)))
    for e in (ev, e0, e1):
        gpu.check(L.tdgs_event_create(C.byref(e)))
    src, back = C.c_void_p(), C.c_void_p()
    gpu.check(L.tdgs_host_malloc(C.byref(src), C.c_size_t(4 * n)))
    gpu.check(L.tdgs_host_malloc(C.byref(back), C.c_size_t(4 * n)))
    dev = torch.empty(n, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    a = np.ctypeslib.as_array(C.cast(src, C.POINTER(C.c_float)), shape=(n,))
    a[:] = np.arange(n, dtype=np.float32) * 0.5
    gpu.check(L.tdgs_event_record(e0, s1))
    gpu.check(L.tdgs_memcpy_h2d(C.c_void_p(dev.data_ptr()), src, C.c_size_t(4 * n), s1))
    gpu.check(L.tdgs_event_record(ev, s1))
    gpu.check(L.tdgs_event_record(e1, s1))
    gpu.check(L.tdgs_stream_wait_event(s2, ev))
    gpu.check(L.tdgs_memcpy_d2h(back, C.c_void_p(dev.data_ptr()), C.c_size_t(4 * n), s2))
    gpu.check(L.tdgs_stream_synchronize(s2))
    gpu.check(L.tdgs_event_synchronize(e1))
    b = np.ctypeslib.as_array(C.cast(back, C.POINTER(C.c_float)), shape=(n,))
    np.testing.assert_array_equal(b, a)
    ms = C.c_float(-1.0)
    gpu.check(L.tdgs_event_elapsed_ms(e0, e1, C.byref(ms)))
    assert ms.value >= 0.0
    for p in (src, back):
        gpu.check(L.tdgs_host_free(p))
    for e in (ev, e0, e1):
        gpu.check(L.tdgs_event_destroy(e))
    for s in (s1, s2):
        gpu.check(L.tdgs_stream_destroy(s))


def test_ctx_check_after_render(gpu):
    w = synthetic.config(0, n=2000)
    cam = w.cameras[0]
    t = host.Tiling.for_camera(cam, 16, 16)
    opts = host.RenderOptions.for_camera(cam, 0)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    out = gpu.RenderOutputs.for_camera(cam, 0)
    buf = gpu.RenderBuffers(len(g), t, 0)
    gpu.render_(out, g, cam, t, opts, buf)
    gpu.ctx_check(0)


def test_ctx_create_destroy_keep_current_device(gpu):
    """tdgs_ctx_create / tdgs_ctx_destroy work on the context's device and leave the caller's
    current device as it was; a device beyond the count is rejected with TDGS_ERR_INVALID."""
    L = gpu.lib()
    before = torch.cuda.current_device()
    h = C.c_void_p()
    assert L.tdgs_ctx_create(torch.cuda.device_count(), C.byref(h)) == abi.TDGS_ERR_INVALID and not h
    assert L.tdgs_ctx_create(before, C.byref(h)) == abi.TDGS_OK and h
    assert torch.cuda.current_device() == before
    assert L.tdgs_ctx_destroy(h) == abi.TDGS_OK
    assert torch.cuda.current_device() == before


@pytest.mark.parametrize("w,h,tile", [(64, 48, (10, 10)), (100, 70, (12, 20)), (33, 29, (5, 7)), (2, 2, (1, 1)),
                                      (40, 40, (40, 25))])
def test_tiles_of_any_pixel_count(gpu, oracle, w, h, tile):
    from tdgs_amd.host import look_at_camera
    wl = synthetic.config(0, n=1500)
    cam = look_at_camera(w, h, 60.0, (0.0, 0.0, -4.0))
    t = host.Tiling.for_camera(cam, *tile)
    opts = host.RenderOptions.for_camera(cam, 0, background_color=(0.1, 0.2, 0.3))
    r = oracle.render(wl.gaussians, cam, t, opts)
    g = gpu.TrainableGaussiansVector.from_host(wl.gaussians, 0)
    out = gpu.RenderOutputs.for_camera(cam, 0, include_depth=True)
    buf = gpu.RenderBuffers(len(g), t, 0, keep_flags=True)
    gpu.render_(out, g, cam, t, opts, buf)
    torch.cuda.synchronize()
    _assert_forward_equal(r, out, buf)
    gen = torch.Generator(device="cuda").manual_seed(2)
    grad = ((torch.rand(out.rgb.shape, generator=gen, device="cuda") - 0.5) * 1e-3).contiguous()
    fg = _backward(gpu, g, out, cam, t, opts, buf, grad, "interleaved")
    ref = oracle.backward(wl.gaussians, cam, t, opts, r, grad.cpu().numpy())
    nf = buf.nb_fgaussians
    assert rel_l2(fg.grads2d[:nf].cpu().numpy(), ref["grads2d"]) <= REL_L2
    for k in ARRAYS:
        assert rel_l2(getattr(fg, k)[:nf].cpu().numpy(), ref[k]) <= REL_L2, k
