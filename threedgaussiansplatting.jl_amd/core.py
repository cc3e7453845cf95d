"""Host-side mirror of the reference's render/train entry points over libtdgs.so.

Device memory is torch tensors (plumbing only); every computation runs in the HIP kernels
of libtdgs.so through its C-ABI (include/tdgs.h). There is no CPU or torch fallback: if the
library is missing or fails to load, the calls raise.

Layouts follow the reference (Julia column-major): a k x n reference array is a (n, k)
contiguous tensor here, sh (h, 3, n) is (n, 3, h), rgb images 3 x h x w are (w, h, 3) and
h x w images are (w, h).
"""
from __future__ import annotations

import ctypes as C
import math
import os
from dataclasses import dataclass

import numpy as np
import torch

from . import abi
from .host import HostGaussians, HostRenderOnlyGaussians, PinholeCamera, RenderOptions, Tiling

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtdgs.so")


class TdgsError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"libtdgs error {code}: {msg}")
        self.code = code


class CapacityError(TdgsError):
    pass


_LIB = None


def lib():
    """Load libtdgs.so; raises if it is not built (build with __graft_entry__.build())."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        L.tdgs_last_error.restype = C.c_char_p
        for name in ("tdgs_scan_temp_bytes", "tdgs_sort_pairs_temp_bytes", "tdgs_render_temp_bytes",
                     "tdgs_loss_temp_bytes"):
            getattr(L, name).restype = C.c_size_t
        L.tdgs_loss_temp_bytes.argtypes = [C.c_int32, C.c_int32]
        L.tdgs_scan_temp_bytes.argtypes = [C.c_int64]
        L.tdgs_sort_pairs_temp_bytes.argtypes = [C.c_int32, C.c_int32]
        L.tdgs_render_temp_bytes.argtypes = [C.c_int32, C.c_int64, C.c_void_p]
        L.tdgs_sort_pairs.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_int32, C.c_int32, C.c_void_p]
        L.tdgs_tile_ranges.argtypes = [C.c_void_p, C.c_int64, C.c_void_p, C.c_int32, C.c_void_p]
        L.tdgs_render_sorted_keys.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64]
        L.tdgs_fill_fgidx_to_gidx.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                              C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        L.tdgs_scan_counts.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                       C.c_void_p, C.c_size_t, C.c_void_p]
        L.tdgs_emit_keys.argtypes = [C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_void_p, C.c_void_p]
        _LIB = L
    return _LIB


def check(rc):
    if rc != abi.TDGS_OK:
        msg = lib().tdgs_last_error().decode(errors="replace")
        cls = CapacityError if rc == abi.TDGS_ERR_CAPACITY else TdgsError
        raise cls(rc, msg)


def stream_ptr(device=None):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dptr(t):
    return None if t is None else t.data_ptr()


_CTX = {}


def context(device=0):
    """Per-device library context (pinned readback buffer + device counters)."""
    device = int(device)
    if device not in _CTX:
        h = C.c_void_p()
        check(lib().tdgs_ctx_create(device, C.byref(h)))
        _CTX[device] = h
    return _CTX[device]


class Context:
    """A library context of its own (tdgs_ctx_create / tdgs_ctx_destroy). The context holds
    the device counters of the frame in progress, so frames rendered concurrently on several
    streams each need their own context (and their own RenderBuffers and RenderOutputs);
    the Gaussians may be shared. context(device) is the default one per device."""

    def __init__(self, device=0):
        self.device = int(device)
        self.handle = C.c_void_p()
        check(lib().tdgs_ctx_create(self.device, C.byref(self.handle)))

    def close(self):
        if self.handle:
            check(lib().tdgs_ctx_destroy(self.handle))
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _handle(ctx, device):
    return context(device) if ctx is None else ctx.handle


def _dev(device):
    return torch.device("cuda", int(device))


# ------------------------------------------------------------------------------------
# Containers
# ------------------------------------------------------------------------------------

class TrainableGaussiansVector:
    """MutableTrainableGaussiansVector (src/gaussians.jl:29-98) in device memory."""

    def __init__(self, means_opacity, scaling, rotation, sh):
        self.means_opacity = means_opacity.contiguous()
        self.scaling = scaling.contiguous()
        self.rotation = rotation.contiguous()
        self.sh = sh.contiguous()
        assert self.means_opacity.dtype == torch.float32 and self.means_opacity.shape[1] == 4

    kind = abi.TDGS_TRAINABLE

    @classmethod
    def from_host(cls, g: HostGaussians, device=0):
        d = _dev(device)
        return cls(*(torch.from_numpy(np.ascontiguousarray(a)).to(d)
                     for a in (g.means_opacity, g.scaling, g.rotation, g.sh)))

    def to_host(self) -> HostGaussians:
        return HostGaussians(*(t.cpu().numpy() for t in (self.means_opacity, self.scaling,
                                                         self.rotation, self.sh)))

    def __len__(self):
        return self.means_opacity.shape[0]

    @property
    def device(self):
        return self.means_opacity.device

    @property
    def sh_degree(self):
        return int(round(math.sqrt(self.sh.shape[2]))) - 1

    def struct(self):
        s = abi.Gaussians()
        s.kind = abi.TDGS_TRAINABLE
        s.n = len(self)
        s.sh_degree = self.sh_degree
        s.means_opacity = dptr(self.means_opacity)
        s.scaling = dptr(self.scaling)
        s.rotation = dptr(self.rotation)
        s.covariances = None
        s.sh = dptr(self.sh)
        return s


class RenderOnlyGaussiansVector:
    """RenderOnlyGaussiansVector (src/gaussians.jl:342-392): opacities already activated and
    3D covariances as lower halves."""

    kind = abi.TDGS_RENDER_ONLY

    def __init__(self, means_opacities, covariances, sh):
        self.means_opacity = means_opacities.contiguous()
        self.covariances = covariances.contiguous()
        self.sh = sh.contiguous()

    @classmethod
    def from_host(cls, g: HostRenderOnlyGaussians, device=0):
        d = _dev(device)
        return cls(*(torch.from_numpy(np.ascontiguousarray(a)).to(d)
                     for a in (g.means_opacity, g.covariances, g.sh)))

    def __len__(self):
        return self.means_opacity.shape[0]

    @property
    def device(self):
        return self.means_opacity.device

    @property
    def sh_degree(self):
        return int(round(math.sqrt(self.sh.shape[2]))) - 1

    def struct(self):
        s = abi.Gaussians()
        s.kind = abi.TDGS_RENDER_ONLY
        s.n = len(self)
        s.sh_degree = self.sh_degree
        s.means_opacity = dptr(self.means_opacity)
        s.scaling = None
        s.rotation = None
        s.covariances = dptr(self.covariances)
        s.sh = dptr(self.sh)
        return s


class RenderOutputs:
    """RenderOutputs (src/forward_structs.jl:1-129)."""

    def __init__(self, width, height, device=0, include_rgb=True, include_transmittance=True,
                 include_depth=False, include_last_contributing_indices=True):
        d = _dev(device)
        self.width, self.height = int(width), int(height)
        self.rgb = torch.empty((width, height, 3), dtype=torch.float32, device=d) if include_rgb else None
        self.T = torch.empty((width, height), dtype=torch.float32, device=d) if include_transmittance else None
        self.depth = torch.empty((width, height), dtype=torch.float32, device=d) if include_depth else None
        self.last = (torch.empty((width, height), dtype=torch.int32, device=d)
                     if include_last_contributing_indices else None)

    @classmethod
    def for_camera(cls, cam: PinholeCamera, device=0, **kw):
        return cls(cam.width, cam.height, device, **kw)

    def struct(self):
        return abi.RenderOutputsC(dptr(self.rgb), dptr(self.T), dptr(self.depth), dptr(self.last))


class RenderBuffers:
    """RenderBuffers + Filtered2DGaussiansVector (src/forward_structs.jl:762-833, 1541-1677).
    Per-Gaussian arrays hold `capacity` entries; key arrays grow on demand."""

    def __init__(self, capacity, tiling: Tiling, device=0, key_capacity=None, keep_flags=False):
        d = _dev(device)
        self.device = d
        self.capacity = int(capacity)
        self.tiling = tiling
        cap = max(self.capacity, 1)
        self.keep = torch.empty(cap, dtype=torch.uint8, device=d) if keep_flags else None
        self.fgidx_to_gidx = torch.empty(cap, dtype=torch.int32, device=d)
        self.depths = torch.empty(cap, dtype=torch.float32, device=d)
        self.f2d = torch.empty((cap, 9), dtype=torch.float32, device=d)
        self.tile_ranges = torch.empty((cap, 4), dtype=torch.int32, device=d)
        self.counts = torch.empty(cap, dtype=torch.int32, device=d)
        self.tiles_end = torch.empty(tiling.nb_tiles, dtype=torch.int32, device=d)
        self.nb_fgaussians = 0
        self.nb_keys = 0
        self.key_capacity = 0
        self.keys = self.values = self._sorted_keys = self.sorted_values = None
        self._keys_pending = None   # the C tiling of a render whose keys are not assembled yet
        self._alloc_keys(key_capacity if key_capacity is not None else 8 * cap)

    @property
    def sorted_keys(self):
        """The sorted 64-bit keys of the last render (int64, key_capacity entries, the first
        nb_keys valid). The render sorts 16-bit tile ids when the tiling has at most 65535 tiles;
        the keys are then assembled here on first access (on the current stream)."""
        if self._keys_pending and self.nb_keys < 0:
            self.frame_counts()
        if self._keys_pending and self.nb_keys > 0:
            check(lib().tdgs_render_sorted_keys(stream_ptr(self.device.index), C.byref(self._keys_pending),
                                                C.byref(self.struct()), self.nb_keys))
            self._keys_pending = None
        return self._sorted_keys

    def _alloc_keys(self, key_capacity):
        d = self.device
        kc = max(int(key_capacity), 1)
        self.key_capacity = kc
        self.keys = torch.empty(kc, dtype=torch.int64, device=d)
        self.values = torch.empty(kc, dtype=torch.int32, device=d)
        self._sorted_keys = torch.empty(kc, dtype=torch.int64, device=d)
        self._keys_pending = None   # new key arrays hold no render's keys
        self.sorted_values = torch.empty(kc, dtype=torch.int32, device=d)
        tb = lib().tdgs_render_temp_bytes(self.capacity, kc, C.byref(self.tiling.to_c()))
        self.temp = torch.empty(int(tb), dtype=torch.uint8, device=d)

    def frame_counts(self):
        """The counts of the last render with device_counts=True (tdgs_render_counts;
        synchronises): sets nb_fgaussians and nb_keys, returns (nb_fgaussians, nb_keys,
        non-empty count, frame status)."""
        c = (C.c_int64 * 4)()
        check(lib().tdgs_render_counts(stream_ptr(self.device.index), C.byref(self.struct()), c))
        self.nb_fgaussians, self.nb_keys = int(c[0]), int(c[1])
        return int(c[0]), int(c[1]), int(c[2]), int(c[3])

    def frame_counts_view(self):
        """The device-side frame counts (int64 x 4: nb_fgaussians, nb_keys, non-empty count,
        status) of a device-count render, as a view of temp (for an asynchronous copy)."""
        return self.temp[:32].view(torch.int64)

    def ensure_capacity(self, n):
        """Grows the per-Gaussian arrays to n entries; the key arrays grow in proportion (a
        frame of n Gaussians duplicates about n / capacity times as many keys)."""
        if n > self.capacity:
            keys = int(self.key_capacity * (n / max(self.capacity, 1))) + 1024
            self.__init__(n, self.tiling, self.device.index, keys, self.keep is not None)

    def struct(self):
        b = abi.RenderBuffersC()
        b.capacity = self.capacity
        b.key_capacity = self.key_capacity
        b.keep = dptr(self.keep)
        b.fgidx_to_gidx = dptr(self.fgidx_to_gidx)
        b.depths = dptr(self.depths)
        b.f2d = dptr(self.f2d)
        b.tile_ranges = dptr(self.tile_ranges)
        b.counts = dptr(self.counts)
        b.keys = dptr(self.keys)
        b.values = dptr(self.values)
        b.sorted_keys = dptr(self._sorted_keys)
        b.sorted_values = dptr(self.sorted_values)
        b.tiles_end = dptr(self.tiles_end)
        b.temp = dptr(self.temp)
        b.temp_bytes = self.temp.numel()
        return b


# ------------------------------------------------------------------------------------
# render!
# ------------------------------------------------------------------------------------

def render_(outputs: RenderOutputs, gaussians, camera: PinholeCamera, tiling: Tiling,
            options: RenderOptions, buffers: RenderBuffers, device_counts: bool = False, ctx: Context = None):
    """render! (src/forward_core.jl:196-314). Grows the key buffers when needed.

    device_counts=True renders without synchronising with the host (TDGS_FLAG_DEVICE_COUNTS):
    buffers.nb_fgaussians and nb_keys become -1 and the counts stay on the device
    (buffers.frame_counts() reads them); the key arrays are not grown, and a frame whose keys
    do not fit renders as render_void! with the status TDGS_FRAME_KEY_CAPACITY.

    ctx (a Context, default: the device's) and torch's current stream order the call: frames
    in flight on several streams each use a Context of their own."""
    dev = gaussians.device.index
    h = _handle(ctx, dev)
    buffers.ensure_capacity(len(gaussians))
    g = gaussians.struct()
    cam, t, o = camera.to_c(), tiling.to_c(), options.to_c()
    out = outputs.struct()
    if device_counts:
        o.flags |= abi.TDGS_FLAG_DEVICE_COUNTS
        nbf, m = C.c_int32(0), C.c_int64(0)
        check(lib().tdgs_render(h, stream_ptr(dev), C.byref(g), C.byref(cam), C.byref(t), C.byref(o),
                                C.byref(buffers.struct()), C.byref(out), C.byref(nbf), C.byref(m)))
        buffers.nb_fgaussians = -1
        buffers.nb_keys = -1
        buffers._keys_pending = t
        return outputs
    nbf = C.c_int32(0)
    m = C.c_int64(0)
    for _ in range(2):
        b = buffers.struct()
        rc = lib().tdgs_render(h, stream_ptr(dev), C.byref(g), C.byref(cam), C.byref(t),
                               C.byref(o), C.byref(b), C.byref(out), C.byref(nbf), C.byref(m))
        if rc == abi.TDGS_ERR_CAPACITY and m.value > buffers.key_capacity and m.value < 2**31 - 1:
            buffers._alloc_keys(int(m.value * 1.25) + 1024)
            continue
        check(rc)
        break
    buffers.nb_fgaussians = int(nbf.value)
    buffers.nb_keys = int(m.value)
    buffers._keys_pending = t if buffers.nb_keys > 0 else None
    return outputs


def project_(gaussians, camera: PinholeCamera, tiling: Tiling, options: RenderOptions, buffers: RenderBuffers):
    """The cull, compaction and projection half of render! (forward_core.jl:222-254, kernels
    :326-355, 371-386, 411-517) as one call (tdgs_project): fills buffers' keep flags (when
    allocated), fgidx_to_gidx, depths, f2d, tile_ranges and counts; returns N_f."""
    dev = gaussians.device.index
    buffers.ensure_capacity(len(gaussians))
    nbf = C.c_int32(0)
    check(lib().tdgs_project(context(dev), stream_ptr(dev), C.byref(gaussians.struct()), C.byref(camera.to_c()),
                             C.byref(tiling.to_c()), C.byref(options.to_c()), C.byref(buffers.struct()),
                             C.byref(nbf)))
    buffers.nb_fgaussians = int(nbf.value)
    return buffers.nb_fgaussians


def ctx_check(device=0, ctx: Context = None):
    """tdgs_ctx_check: synchronise and raise on a device-side error flag of the context."""
    check(lib().tdgs_ctx_check(_handle(ctx, device), stream_ptr(device)))


# ------------------------------------------------------------------------------------
# Building blocks (one reference kernel each)
# ------------------------------------------------------------------------------------

def fill_fgidx_to_gidx(keep: torch.Tensor):
    """accumulate!(+) + fill_fgidx_to_gidx_kernel! (forward_core.jl:231-244, 371-386)."""
    dev = keep.device.index
    n = keep.numel()
    cs = torch.empty(n, dtype=torch.int32, device=keep.device)
    f2g = torch.empty(n, dtype=torch.int32, device=keep.device)
    temp = torch.empty(int(lib().tdgs_scan_temp_bytes(n)), dtype=torch.uint8, device=keep.device)
    nf = C.c_int32(0)
    check(lib().tdgs_fill_fgidx_to_gidx(context(dev), stream_ptr(dev), dptr(keep.to(torch.uint8)), n,
                                        dptr(cs), dptr(f2g), dptr(temp), temp.numel(), C.byref(nf)))
    return cs, f2g[: nf.value], nf.value


def scan_counts(counts: torch.Tensor):
    dev = counts.device.index
    n = counts.numel()
    cs = torch.empty(n, dtype=torch.int32, device=counts.device)
    temp = torch.empty(int(lib().tdgs_scan_temp_bytes(n)), dtype=torch.uint8, device=counts.device)
    tot = C.c_int64(0)
    check(lib().tdgs_scan_counts(context(dev), stream_ptr(dev), dptr(counts), n, dptr(cs), dptr(temp),
                                 temp.numel(), C.byref(tot)))
    return cs, tot.value


def emit_keys(depths, tile_ranges, counts_cs, total, tiling: Tiling):
    dev = depths.device.index
    nf = depths.numel()
    keys = torch.empty(max(total, 1), dtype=torch.int64, device=depths.device)
    vals = torch.empty(max(total, 1), dtype=torch.int32, device=depths.device)
    check(lib().tdgs_emit_keys(stream_ptr(dev), nf, dptr(depths), dptr(tile_ranges), dptr(counts_cs),
                               C.byref(tiling.to_c()), dptr(keys), dptr(vals)))
    return keys[:total], vals[:total]


def sort_pairs(keys: torch.Tensor, values: torch.Tensor, end_bit: int):
    """sort_pairs (cub_sort_pairs_wrapper.cu:31-43): stable radix sort on bits [0, end_bit)."""
    dev = keys.device.index
    n = keys.numel()
    tb = int(lib().tdgs_sort_pairs_temp_bytes(n, end_bit))
    temp = torch.empty(tb, dtype=torch.uint8, device=keys.device)
    ko = torch.empty_like(keys)
    vo = torch.empty_like(values)
    check(lib().tdgs_sort_pairs(dptr(temp), tb, dptr(keys), dptr(ko), dptr(values), dptr(vo), n, end_bit,
                                stream_ptr(dev)))
    return ko, vo


def tile_ranges(sorted_keys: torch.Tensor, nb_tiles: int):
    dev = sorted_keys.device.index
    te = torch.empty(nb_tiles, dtype=torch.int32, device=sorted_keys.device)
    check(lib().tdgs_tile_ranges(stream_ptr(dev), sorted_keys.numel(), dptr(sorted_keys), nb_tiles, dptr(te)))
    return te


def image_to_rgb8(image: torch.Tensor, kind=abi.TDGS_IMAGE_RGB, min_depth=0.0, max_depth=1.0,
                  out: torch.Tensor | None = None):
    """The viewer's UInt8 image (gui.jl:958-1067) of a rendered rgb (w, h, 3), T or depth
    (w, h) image: a (h, w, 3) uint8 tensor, i.e. Julia's 3 x w x h."""
    w, h = int(image.shape[0]), int(image.shape[1])
    expect = (w, h, 3) if kind == abi.TDGS_IMAGE_RGB else (w, h)
    if tuple(image.shape) != expect or image.dtype != torch.float32 or not image.is_contiguous():
        raise ValueError(f"image must be contiguous float32 {expect}, got {tuple(image.shape)} {image.dtype}")
    if out is None:
        out = torch.empty((h, w, 3), dtype=torch.uint8, device=image.device)
    check(lib().tdgs_image_to_rgb8(stream_ptr(image.device.index), C.c_int32(kind), C.c_void_p(dptr(image)),
                                   C.c_int32(w), C.c_int32(h), C.c_float(min_depth), C.c_float(max_depth),
                                   C.c_void_p(dptr(out))))
    return out


# ------------------------------------------------------------------------------------
# backward!
# ------------------------------------------------------------------------------------

class FilteredGaussiansGradientsVector:
    """FilteredGaussiansGradientsVector (src/backward_structs.jl:1-156): per filtered Gaussian
    2D gradients and 3D gradients in the reference layouts.

    The 2D gradients are either interleaved (layout="interleaved", the default: one (n, 9)
    array [mean2d 2, opacity 1, inverse covariance lower 3, colour 3], the faster layout) or
    the reference's four arrays (layout="reference": mean2d_grads 2 x n, opacity_grads n,
    licov2d_grads 3 x n, color_grads 3 x n, backward_structs.jl:17-22)."""

    def __init__(self, capacity, sh_degree, device=0, layout="interleaved"):
        d = _dev(device)
        cap = max(int(capacity), 1)
        h = (int(sh_degree) + 1) ** 2
        if layout not in ("interleaved", "reference"):
            raise ValueError(f"unknown 2D gradient layout {layout!r}")
        self.layout = layout
        self.capacity = cap
        self.sh_degree = int(sh_degree)
        if layout == "interleaved":
            self.grads2d = torch.zeros((cap, 9), dtype=torch.float32, device=d)
            self.mean2d = self.grads2d[:, 0:2]
            self.opacity = self.grads2d[:, 2]
            self.licov2d = self.grads2d[:, 3:6]
            self.color = self.grads2d[:, 6:9]
        else:
            self.grads2d = None
            self.mean2d = torch.zeros((cap, 2), dtype=torch.float32, device=d)
            self.opacity = torch.zeros(cap, dtype=torch.float32, device=d)
            self.licov2d = torch.zeros((cap, 3), dtype=torch.float32, device=d)
            self.color = torch.zeros((cap, 3), dtype=torch.float32, device=d)
        self.mean3d = torch.zeros((cap, 3), dtype=torch.float32, device=d)
        self.opacity_feature = torch.zeros(cap, dtype=torch.float32, device=d)
        self.scaling_features = torch.zeros((cap, 3), dtype=torch.float32, device=d)
        self.rotation_features = torch.zeros((cap, 4), dtype=torch.float32, device=d)
        self.sh = torch.zeros((cap, 3, h), dtype=torch.float32, device=d)

    def grads2d_matrix(self, n=None):
        """The 2D gradients of the first n filtered Gaussians as one (n, 9) tensor (a copy for
        the reference layout)."""
        n = self.capacity if n is None else n
        if self.grads2d is not None:
            return self.grads2d[:n]
        return torch.cat([self.mean2d[:n], self.opacity[:n, None], self.licov2d[:n], self.color[:n]], dim=1)

    def zero_2d_(self, n):
        """zero_2d_grads! (backward_structs.jl:250-257) on the first n entries."""
        if self.grads2d is not None:
            self.grads2d[:n].zero_()
        else:
            for t in (self.mean2d, self.opacity, self.licov2d, self.color):
                t[:n].zero_()

    def struct(self):
        s = abi.GradientsC()
        s.capacity = self.capacity
        s.sh_degree = self.sh_degree
        if self.grads2d is not None:
            s.grads2d = dptr(self.grads2d)
        else:
            s.grads2d = None
            s.mean2d_grads = dptr(self.mean2d)
            s.opacity_grads = dptr(self.opacity)
            s.licov2d_grads = dptr(self.licov2d)
            s.color_grads = dptr(self.color)
        s.mean3d = dptr(self.mean3d)
        s.opacity_feature = dptr(self.opacity_feature)
        s.scaling_features = dptr(self.scaling_features)
        s.rotation_features = dptr(self.rotation_features)
        s.sh = dptr(self.sh)
        return s


def backward_render_tiles_(fgradients: FilteredGaussiansGradientsVector, rgb_image_grad: torch.Tensor,
                           outputs: RenderOutputs, camera: PinholeCamera, tiling: Tiling, options: RenderOptions,
                           buffers: RenderBuffers):
    """zero_2d_grads! + backward_render_tiles_kernel! (backward_core.jl:37-58, 96-293): the 2D
    gradients only, for a caller that runs the backward projection itself."""
    dev = rgb_image_grad.device.index
    assert rgb_image_grad.dtype == torch.float32 and rgb_image_grad.is_contiguous()
    nbf = buffers.nb_fgaussians
    if nbf == 0:
        return fgradients
    # (a device-count render: the count is not known here, zero the whole capacity)
    fgradients.zero_2d_(nbf if nbf > 0 else None)
    check(lib().tdgs_backward_render_tiles(stream_ptr(dev), C.byref(fgradients.struct()),
                                           C.c_void_p(dptr(rgb_image_grad)), C.byref(outputs.struct()),
                                           C.byref(camera.to_c()), C.byref(tiling.to_c()), C.byref(options.to_c()),
                                           C.byref(buffers.struct())))
    return fgradients


def backward_(fgradients: FilteredGaussiansGradientsVector, rgb_image_grad: torch.Tensor,
              outputs: RenderOutputs, gaussians: TrainableGaussiansVector, camera: PinholeCamera,
              tiling: Tiling, options: RenderOptions, buffers: RenderBuffers):
    """backward! (src/backward_core.jl:37-72); uses the buffers of the preceding render_."""
    dev = gaussians.device.index
    assert rgb_image_grad.dtype == torch.float32 and rgb_image_grad.is_contiguous()
    gr = fgradients.struct()
    check(lib().tdgs_backward(stream_ptr(dev), C.byref(gr), C.c_void_p(dptr(rgb_image_grad)),
                              C.byref(outputs.struct()), C.byref(gaussians.struct()),
                              C.byref(camera.to_c()), C.byref(tiling.to_c()), C.byref(options.to_c()),
                              C.byref(buffers.struct()), C.c_int32(buffers.nb_fgaussians)))
    return fgradients
