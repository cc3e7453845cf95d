"""ctypes wrapper of the CPU oracle (oracle/liboracle.so). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module; it is
the checker, never the measured or shipped path. Arrays are numpy arrays in the reference's
memory layouts (see threedgaussiansplatting.jl_amd/host.py): per-Gaussian k x n Julia arrays
are (n, k) C-order arrays here, images 3 x h x w are (w, h, 3).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def _abi():
    import importlib
    return importlib.import_module(__package_root__() + ".abi")


def __package_root__():
    import sys
    for name in ("tdgs_amd",):
        if name in sys.modules:
            return name
    raise RuntimeError("load the package first (__graft_entry__.load_package())")


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            from . import build as _b  # type: ignore
            _b.build()
        _LIB = C.CDLL(path)
        _LIB.oracle_fill_fgidx_to_gidx.restype = C.c_int32
        _LIB.oracle_scan_counts.restype = C.c_int64
        _LIB.oracle_render.restype = C.c_int64
        _LIB.oracle_adc_plan.restype = C.c_int32
        _LIB.oracle_l1_loss_grad.restype = C.c_double
        for fn in ("oracle_exp", "oracle_log", "oracle_sigmoid"):
            getattr(_LIB, fn).restype = C.c_float
            getattr(_LIB, fn).argtypes = [C.c_float]
        _LIB.oracle_normal_pair.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32, C.c_void_p]
        _LIB.oracle_sort_pairs.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                           C.c_int64, C.c_int32]
        _LIB.oracle_tile_ranges.argtypes = [C.c_int64, C.c_void_p, C.c_int32, C.c_void_p]
        _LIB.oracle_set_threads.argtypes = [C.c_int32]
    return _LIB


def set_threads(n):
    """Threads of the oracle's per-tile loops (forward images are identical for any count;
    backward sums in double precision, per thread, added in thread order)."""
    lib().oracle_set_threads(int(n))


def ptr(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def gaussians_struct(g):
    abi = _abi()
    s = abi.Gaussians()
    s.n = g.n
    s.sh_degree = g.sh_degree
    s.means_opacity = g.means_opacity.ctypes.data
    s.sh = g.sh.ctypes.data
    if hasattr(g, "covariances"):  # render-only: activated opacities, 3D covariances
        s.kind = abi.TDGS_RENDER_ONLY
        s.scaling = None
        s.rotation = None
        s.covariances = g.covariances.ctypes.data
    else:
        s.kind = abi.TDGS_TRAINABLE
        s.scaling = g.scaling.ctypes.data
        s.rotation = g.rotation.ctypes.data
        s.covariances = None
    return s


def render(g, cam, tiling, opts, *, rgb=True, T=True, depth=True, last=True):
    """render! (forward_core.jl:196-314) on the CPU; returns a dict of every intermediate."""
    abi = _abi()
    L = lib()
    n = g.n
    W, H = cam.width, cam.height
    gs = gaussians_struct(g)
    c_cam = cam.to_c()
    c_t = tiling.to_c()
    c_o = opts.to_c()
    res = {
        "keep": np.zeros(n, np.uint8),
        "fgidx_to_gidx": np.zeros(n, np.int32),
        "depths": np.zeros(n, np.float32),
        "f2d": np.zeros((n, 9), np.float32),
        "tile_ranges": np.zeros((n, 4), np.int32),
        "counts": np.zeros(n, np.int32),
        "tiles_end": np.zeros(tiling.nb_tiles, np.int32),
    }
    out = {
        "rgb": np.zeros((W, H, 3), np.float32) if rgb else None,
        "T": np.zeros((W, H), np.float32) if T else None,
        "depth": np.zeros((W, H), np.float32) if depth else None,
        "last": np.zeros((W, H), np.int32) if last else None,
    }
    b = abi.RenderBuffersC()
    b.capacity = n
    b.key_capacity = 0
    b.keep = res["keep"].ctypes.data
    b.fgidx_to_gidx = res["fgidx_to_gidx"].ctypes.data
    b.depths = res["depths"].ctypes.data
    b.f2d = res["f2d"].ctypes.data
    b.tile_ranges = res["tile_ranges"].ctypes.data
    b.counts = res["counts"].ctypes.data
    b.tiles_end = res["tiles_end"].ctypes.data
    o = abi.RenderOutputsC(*(None if out[k] is None else out[k].ctypes.data
                             for k in ("rgb", "T", "depth", "last")))
    nbf = C.c_int32(0)
    m = L.oracle_render(C.byref(gs), C.byref(c_cam), C.byref(c_t), C.byref(c_o), C.byref(b),
                        C.byref(o), C.byref(nbf))
    if m > 0:
        for k, dt in (("keys", np.int64), ("values", np.int32), ("sorted_keys", np.int64),
                      ("sorted_values", np.int32)):
            res[k] = np.zeros(m, dt)
        b.key_capacity = m
        b.keys = res["keys"].ctypes.data
        b.values = res["values"].ctypes.data
        b.sorted_keys = res["sorted_keys"].ctypes.data
        b.sorted_values = res["sorted_values"].ctypes.data
        m2 = L.oracle_render(C.byref(gs), C.byref(c_cam), C.byref(c_t), C.byref(c_o), C.byref(b),
                             C.byref(o), C.byref(nbf))
        assert m2 == m
    res["nb_fgaussians"] = int(nbf.value)
    res["nb_keys"] = int(m)
    res.update(out)
    return res


def blend_tile(cam, tiling, opts, f2d, depths, entries, beg, tx, ty, rgb, T, depth, last):
    """render_tiles_kernel! (forward_core.jl:756-993) for tile (tx, ty) alone: its sorted
    entries beg, beg + 1, ... are `entries` (1-based fgidx values); writes that tile's pixels
    of the given full-size images (any may be None)."""
    entries = np.ascontiguousarray(entries, np.int32)
    f2d = np.ascontiguousarray(f2d, np.float32)
    depths = np.ascontiguousarray(depths, np.float32)
    c_cam, c_t, c_o = cam.to_c(), tiling.to_c(), opts.to_c()
    lib().oracle_blend_tile(C.byref(c_cam), C.byref(c_t), C.byref(c_o), ptr(f2d), ptr(depths), ptr(entries),
                            C.c_int64(beg), C.c_int64(beg + entries.size), C.c_int32(tx), C.c_int32(ty),
                            ptr(rgb), ptr(T), ptr(depth), ptr(last))


def backward_tile(cam, tiling, opts, f2d, entries, beg, tx, ty, rgb_grad, T, last, acc):
    """backward_render_tiles_kernel! (backward_core.jl:96-293) for tile (tx, ty) alone: its
    sorted entries beg + 1, beg + 2, ... (1-based) are `entries` (1-based fgidx values); adds the
    tile's 2D gradients into acc ((nb_f, 9) float64)."""
    entries = np.ascontiguousarray(entries, np.int32)
    f2d = np.ascontiguousarray(f2d, np.float32)
    assert acc.dtype == np.float64 and acc.flags.c_contiguous and acc.shape[1] == 9
    c_cam, c_t, c_o = cam.to_c(), tiling.to_c(), opts.to_c()
    lib().oracle_backward_tile(C.byref(c_cam), C.byref(c_t), C.byref(c_o), ptr(f2d), ptr(entries),
                               C.c_int64(beg), C.c_int64(beg + entries.size), C.c_int32(tx), C.c_int32(ty),
                               ptr(np.ascontiguousarray(rgb_grad, np.float32)),
                               ptr(np.ascontiguousarray(T, np.float32)), ptr(np.ascontiguousarray(last, np.int32)),
                               ptr(acc))


def fill_fgidx_to_gidx(keep):
    keep = np.ascontiguousarray(keep, dtype=np.uint8)
    n = keep.size
    cs = np.zeros(n, np.int32)
    f2g = np.zeros(n, np.int32)
    nf = lib().oracle_fill_fgidx_to_gidx(ptr(keep), C.c_int32(n), ptr(cs), ptr(f2g))
    return cs, f2g[:nf], nf


def emit_keys(depths, tile_ranges, counts, tiling):
    counts = np.ascontiguousarray(counts, dtype=np.int32)
    nf = counts.size
    cs = np.zeros(nf, np.int32)
    m = lib().oracle_scan_counts(ptr(counts), C.c_int32(nf), ptr(cs))
    keys = np.zeros(m, np.int64)
    vals = np.zeros(m, np.int32)
    c_t = tiling.to_c()
    lib().oracle_emit_keys(C.c_int32(nf), ptr(np.ascontiguousarray(depths, np.float32)),
                           ptr(np.ascontiguousarray(tile_ranges, np.int32)), ptr(cs),
                           C.byref(c_t), ptr(keys), ptr(vals))
    return cs, keys, vals


def sort_pairs(keys, values, end_bit):
    keys = np.ascontiguousarray(keys, np.int64)
    values = np.ascontiguousarray(values, np.int32)
    ko = np.zeros_like(keys)
    vo = np.zeros_like(values)
    lib().oracle_sort_pairs(ptr(keys), ptr(ko), ptr(values), ptr(vo), keys.size, end_bit)
    return ko, vo


def tile_ranges(sorted_keys, nb_tiles):
    te = np.zeros(nb_tiles, np.int32)
    sk = np.ascontiguousarray(sorted_keys, np.int64)
    lib().oracle_tile_ranges(sk.size, ptr(sk), nb_tiles, ptr(te))
    return te


def backward(g, cam, tiling, opts, fwd, rgb_grad):
    """backward! (backward_core.jl:37-72) on the CPU from the intermediates of render()."""
    abi = _abi()
    L = lib()
    nf = fwd["nb_fgaussians"]
    hg = (g.sh_degree + 1) ** 2
    acc = np.zeros((max(nf, 1), 9), np.float64)
    c_cam, c_t, c_o = cam.to_c(), tiling.to_c(), opts.to_c()
    if fwd["nb_keys"] > 0:
        L.oracle_backward_render_tiles(C.byref(c_cam), C.byref(c_t), C.byref(c_o), ptr(fwd["f2d"]),
                                       ptr(fwd["sorted_values"]), ptr(fwd["tiles_end"]),
                                       ptr(np.ascontiguousarray(rgb_grad, np.float32)),
                                       ptr(fwd["T"]), ptr(fwd["last"]), ptr(acc))
    grads2d = acc.astype(np.float32)
    out = {
        "grads2d": grads2d[:nf],
        "mean3d": np.zeros((nf, 3), np.float32),
        "opacity_feature": np.zeros(nf, np.float32),
        "scaling_features": np.zeros((nf, 3), np.float32),
        "rotation_features": np.zeros((nf, 4), np.float32),
        "sh": np.zeros((nf, 3, hg), np.float32),
    }
    gr = abi.GradientsC()
    gr.capacity = nf
    gr.sh_degree = g.sh_degree
    for k in ("mean3d", "opacity_feature", "scaling_features", "rotation_features", "sh"):
        setattr(gr, k, out[k].ctypes.data if nf > 0 else None)
    if nf > 0:
        L.oracle_backward_project(C.byref(gaussians_struct(g)), C.byref(c_cam), C.byref(c_o),
                                  C.c_int32(nf), ptr(fwd["fgidx_to_gidx"]), ptr(fwd["f2d"]),
                                  ptr(fwd["counts"]), ptr(grads2d), C.byref(gr))
    return out


def backward_project(g, cam, opts, fwd, grads2d, grads_sh_degree=None):
    """backward_project_fgaussians_kernel! (backward_core.jl:309-452) alone, from given 2D
    gradients ((nf, 9) interleaved) and the intermediates of render(); returns the 3D
    gradients by fgidx."""
    abi = _abi()
    nf = fwd["nb_fgaussians"]
    hg = ((g.sh_degree if grads_sh_degree is None else grads_sh_degree) + 1) ** 2
    out = {
        "mean3d": np.zeros((nf, 3), np.float32),
        "opacity_feature": np.zeros(nf, np.float32),
        "scaling_features": np.zeros((nf, 3), np.float32),
        "rotation_features": np.zeros((nf, 4), np.float32),
        "sh": np.zeros((nf, 3, hg), np.float32),
    }
    if nf == 0:
        return out
    gr = abi.GradientsC()
    gr.capacity = nf
    gr.sh_degree = int(round(hg ** 0.5)) - 1
    for k in out:
        setattr(gr, k, out[k].ctypes.data)
    g2 = np.ascontiguousarray(grads2d[:nf], np.float32)
    lib().oracle_backward_project(C.byref(gaussians_struct(g)), C.byref(cam.to_c()), C.byref(opts.to_c()),
                                  C.c_int32(nf), ptr(fwd["fgidx_to_gidx"]), ptr(fwd["f2d"]), ptr(fwd["counts"]),
                                  ptr(g2), C.byref(gr))
    return out


class AdamHost:
    """Adam moments + learning rates (optimizer.jl:9-195) as host arrays."""

    def __init__(self, n, sh_degree, lrs, beta1=0.9, beta2=0.999, epsilon=1e-15, update_count=0):
        h = (sh_degree + 1) ** 2
        self.means = np.zeros((n, 3, 2), np.float32)
        self.opacity = np.zeros((n, 2), np.float32)
        self.scaling = np.zeros((n, 3, 2), np.float32)
        self.rotation = np.zeros((n, 4, 2), np.float32)
        self.sh = np.zeros((n, 3, h, 2), np.float32)
        self.lrs = list(lrs)
        self.beta1, self.beta2, self.epsilon = beta1, beta2, epsilon
        self.update_count = update_count

    def struct(self):
        abi = _abi()
        s = abi.AdamStateC()
        s.means_moments = self.means.ctypes.data
        s.opacity_moments = self.opacity.ctypes.data
        s.scaling_moments = self.scaling.ctypes.data
        s.rotation_moments = self.rotation.ctypes.data
        s.sh_moments = self.sh.ctypes.data
        (s.lr_means, s.lr_opacity, s.lr_scaling, s.lr_rotation, s.lr_sh_dc,
         s.lr_sh_rest) = [float(v) for v in self.lrs]
        s.beta1, s.beta2, s.epsilon = float(self.beta1), float(self.beta2), float(self.epsilon)
        s.update_count = int(self.update_count)
        return s


def adam_step(g, adam: AdamHost, grads, fgidx_to_gidx, sh_degree):
    abi = _abi()
    nf = len(fgidx_to_gidx)
    gr = abi.GradientsC()
    gr.capacity = nf
    gr.sh_degree = (grads["sh"].shape[2] ** 0.5) - 1 if False else int(round(grads["sh"].shape[2] ** 0.5)) - 1
    for k in ("mean3d", "opacity_feature", "scaling_features", "rotation_features", "sh"):
        grads[k] = np.ascontiguousarray(grads[k], np.float32)
        setattr(gr, k, grads[k].ctypes.data)
    st = adam.struct()
    f2g = np.ascontiguousarray(fgidx_to_gidx, np.int32)
    lib().oracle_adam_step(C.byref(gaussians_struct(g)), C.byref(st), C.byref(gr), ptr(f2g),
                           C.c_int32(nf), C.c_int32(sh_degree))
    adam.update_count = st.update_count


def cpu_render_reference(g, cam, opts, threads=1):
    """render! for CPU arrays (forward_core.jl:25-177): the reference's own CPU renderer."""
    W, H = cam.width, cam.height
    rgb = np.zeros((W, H, 3), np.float32)
    T = np.zeros((W, H), np.float32)
    c_cam, c_o = cam.to_c(), opts.to_c()
    lib().cpu_render_reference(C.byref(gaussians_struct(g)), C.byref(c_cam), C.byref(c_o),
                               C.c_int32(threads), ptr(rgb), ptr(T))
    return rgb, T


def cpu_render_reference_timed(g, cam, opts, threads=1, column_step=1, first_column=1):
    """Times the reference's CPU renderer: returns (seconds of the per-Gaussian part,
    seconds of splatting the image columns u = first_column (mod column_step)) measured with
    std::chrono::steady_clock."""
    W, H = cam.width, cam.height
    u_lo, u_hi = first_column, column_step
    rgb = np.zeros((W, H, 3), np.float32)
    T = np.zeros((W, H), np.float32)
    sec = np.zeros(2, np.float64)
    c_cam, c_o = cam.to_c(), opts.to_c()
    lib().cpu_render_reference_timed(C.byref(gaussians_struct(g)), C.byref(c_cam), C.byref(c_o),
                                     C.c_int32(threads), C.c_int32(u_lo), C.c_int32(u_hi), ptr(rgb), ptr(T),
                                     ptr(sec))
    return float(sec[0]), float(sec[1])


def exp(x):
    return lib().oracle_exp(float(x))


def exp_array(x):
    """exp_f of every element of a float32 array."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().oracle_exp_array(ptr(x), ptr(y), C.c_int64(x.size))
    return y


def log_array(x):
    """log_f of every element of a float32 array."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().oracle_log_array(ptr(x), ptr(y), C.c_int64(x.size))
    return y


def log(x):
    return lib().oracle_log(float(x))


def sigmoid(x):
    return lib().oracle_sigmoid(float(x))


def quat_to_rot(q):
    q = np.ascontiguousarray(q, np.float32)
    R = np.zeros(9, np.float32)
    lib().oracle_quat_to_rot(ptr(q), ptr(R))
    return R.reshape(3, 3)


def normal_pair(seed, stream, pair):
    out = np.zeros(2, np.float32)
    lib().oracle_normal_pair(seed, stream, pair, ptr(out))
    return out


class AdcHost:
    """AdaptiveDensityControlBuffers (training_structs.jl:265-331) as host arrays."""

    def __init__(self, n, new_capacity=None):
        self.n = n
        self.accum = np.zeros(n, np.float32)
        self.counts = np.zeros(n, np.int32)
        self.prune = np.zeros(n, np.uint8)
        self.densify = np.zeros(n, np.uint8)
        self.clone = np.zeros(n, np.uint8)
        self.cs = np.zeros(n, np.int32)
        self.new_capacity = new_capacity or 2 * n
        self.ngidx = np.zeros(self.new_capacity, np.int32)

    def struct(self):
        abi = _abi()
        s = abi.AdcBuffersC()
        s.capacity = self.n
        s.new_capacity = self.new_capacity
        s.accum_grad_norms = self.accum.ctypes.data
        s.contribution_counts = self.counts.ctypes.data
        s.prune = self.prune.ctypes.data
        s.densify = self.densify.ctypes.data
        s.clone = self.clone.ctypes.data
        s.new_counts_cs = self.cs.ctypes.data
        s.ngidx_to_gidx = self.ngidx.ctypes.data
        return s


def adc_stats(adc: AdcHost, grads2d, fgidx_to_gidx, width, height):
    s = adc.struct()
    g2 = np.ascontiguousarray(grads2d, np.float32)
    f2g = np.ascontiguousarray(fgidx_to_gidx, np.int32)
    lib().oracle_adc_stats(C.byref(s), ptr(g2), ptr(f2g), C.c_int32(len(f2g)), C.c_int32(width),
                           C.c_int32(height))


def adc_plan(adc: AdcHost, g, prune_logit, use_max_scale, log_max_scale, grad_threshold, log_size_threshold):
    s = adc.struct()
    return lib().oracle_adc_plan(C.byref(s), C.byref(gaussians_struct(g)), C.c_float(prune_logit),
                                 C.c_int32(int(use_max_scale)), C.c_float(log_max_scale),
                                 C.c_float(grad_threshold), C.c_float(log_size_threshold))


def adc_apply(adc: AdcHost, g, adam: AdamHost, log_split_factor, seed):
    """Returns (new HostGaussians, new AdamHost)."""
    from importlib import import_module
    host = import_module(__package_root__() + ".host")
    n_new = int(adc.cs[g.n - 1]) if g.n else 0
    h = (g.sh_degree + 1) ** 2
    ng = host.HostGaussians(np.zeros((n_new, 4), np.float32), np.zeros((n_new, 3), np.float32),
                            np.zeros((n_new, 4), np.float32), np.zeros((n_new, 3, h), np.float32))
    nm = AdamHost(n_new, g.sh_degree, adam.lrs, adam.beta1, adam.beta2, adam.epsilon, adam.update_count)
    s = adc.struct()
    lib().oracle_adc_apply(C.byref(s), C.byref(gaussians_struct(g)), C.byref(gaussians_struct(ng)),
                           C.byref(adam.struct()), C.byref(nm.struct()), C.c_float(log_split_factor),
                           C.c_uint64(seed))
    return ng, nm


def adc_remap_fgidx(adc: AdcHost, fgidx_to_gidx):
    f2g = np.ascontiguousarray(fgidx_to_gidx, np.int32).copy()
    lib().oracle_adc_remap_fgidx(C.byref(adc.struct()), ptr(f2g), C.c_int32(len(f2g)))
    return f2g


def l1_loss_grad(rendered, gt, l1_weight, dssim_weight=0.0, dssim_grad=None):
    r = np.ascontiguousarray(rendered, np.float32)
    g = np.ascontiguousarray(gt, np.float32)
    out = np.zeros_like(r)
    dg = None if dssim_grad is None else np.ascontiguousarray(dssim_grad, np.float32)
    L = lib()
    L.oracle_l1_loss_grad.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_float, C.c_float, C.c_void_p,
                                      C.c_void_p]
    s = L.oracle_l1_loss_grad(ptr(r), ptr(g), r.size, l1_weight, dssim_weight, ptr(dg), ptr(out))
    return s, out
