"""Frames in flight: render! calls on two streams at once, each with its own library context
(tdgs_ctx_create) and render buffers, without host synchronisation (TDGS_FLAG_DEVICE_COUNTS),
sharing one Gaussian array. Every frame must equal the same camera rendered alone with the
default context, bit for bit, and each context's frame monitor must count its own frames.
(The reference renders one frame at a time, forward_core.jl:196-314; this checks that the
library keeps no per-frame state outside a context and its buffers.)"""
import ctypes as C

import numpy as np
import pytest
import torch

from tdgs_amd import abi, host, synthetic

pytestmark = pytest.mark.gpu


def _monitor(gpu, handle):
    p = C.POINTER(C.c_int64)()
    gpu.check(gpu.lib().tdgs_ctx_frame_monitor(handle, C.byref(p)))
    return [int(p[i]) for i in range(4)]


def test_two_streams_two_contexts_bit_exact(gpu):
    w = synthetic.config(2, n=150_000)
    cams = w.cameras[:6]
    t = host.Tiling.for_camera(cams[0], 16, 16)
    opts = host.RenderOptions.for_camera(cams[0], w.gaussians.sh_degree)
    g = gpu.TrainableGaussiansVector.from_host(w.gaussians, 0)
    kw = dict(include_rgb=True, include_transmittance=True, include_depth=True, include_last_contributing_indices=True)

    # each camera alone, default context, host-read counts
    ref, counts = [], []
    buf = gpu.RenderBuffers(len(g), t, 0)
    for cam in cams:
        out = gpu.RenderOutputs.for_camera(cam, 0, **kw)
        gpu.render_(out, g, cam, t, opts, buf)
        torch.cuda.synchronize()
        ref.append({k: getattr(out, k).cpu().numpy() for k in ("rgb", "T", "depth", "last")})
        counts.append((buf.nb_fgaussians, buf.nb_keys))
    kcap = max(m for _, m in counts) + 1024

    ctxs = [gpu.Context(0), gpu.Context(0)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    bufs = [gpu.RenderBuffers(len(g), t, 0, kcap) for _ in range(2)]
    rounds = 3
    outs = [gpu.RenderOutputs.for_camera(cams[0], 0, **kw) for _ in range(rounds * len(cams))]
    torch.cuda.synchronize()
    for k in range(len(outs)):
        s = k % 2
        with torch.cuda.stream(streams[s]):
            gpu.render_(outs[k], g, cams[k % len(cams)], t, opts, bufs[s], device_counts=True, ctx=ctxs[s])
    torch.cuda.synchronize()
    for k, out in enumerate(outs):
        r = ref[k % len(cams)]
        for name in ("rgb", "T", "depth", "last"):
            np.testing.assert_array_equal(getattr(out, name).cpu().numpy(), r[name], err_msg=f"frame {k} {name}")
    # the last frame of each stream: its counts; each context's monitor counted its frames
    for s in range(2):
        k_last = len(outs) - 2 + s
        with torch.cuda.stream(streams[s]):
            nbf, m, _, status = bufs[s].frame_counts()
        assert (nbf, m) == counts[k_last % len(cams)] and status == abi.TDGS_FRAME_OK
        mon = _monitor(gpu, ctxs[s].handle)
        assert mon[0] == len(outs) // 2 and mon[2] == 0
    for c in ctxs:
        c.close()
