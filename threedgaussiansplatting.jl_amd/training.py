"""Host-side mirror of the reference's optimiser, densification and trainer over libtdgs.so.

Reference: src/optimizer.jl (GaussianAdamMomentsLearningRatesVector :9-195, AdamOptimizer
:761-854, update! :964-1009, ADC of moments :1304-1378), src/training_structs.jl
(TrainingOptions :10-228, ADC buffers :265-468), src/training.jl (Trainer :40-151,
training_step! :173-244, ADC :313-580), src/gaussians.jl:1070-1101, 1526-1694.
"""
from __future__ import annotations

import ctypes as C
import math
import time
from dataclasses import dataclass

import numpy as np
import torch

from . import abi
from .core import (Context, FilteredGaussiansGradientsVector, RenderBuffers, RenderOutputs,
                   TrainableGaussiansVector, _dev, backward_, backward_render_tiles_, check, context, ctx_check, dptr,
                   lib, render_, stream_ptr)
from .host import PinholeCamera, RenderOptions, Tiling, logit32

f32 = np.float32

# src/optimizer.jl:831-833
DEFAULT_BETA1 = 0.9
DEFAULT_BETA2 = 0.999
DEFAULT_EPSILON = 1e-15


@dataclass
class TrainingOptions:
    """TrainingOptions with the 3DGS defaults (training_structs.jl:43-85, 139-228); the
    'base' learning rate and size thresholds are scaled by the scene radius."""
    nb_iterations: int = 30_000
    loss_dssim_vs_L1_weight: float = 0.2
    initial_means_lr: float = 0.00016
    final_means_lr: float = 0.0000016
    opacity_features_lr: float = 0.05
    scaling_features_lr: float = 0.005
    rotation_features_lr: float = 0.001
    sh_coeffs_dc_lr: float = 0.0025
    sh_coeffs_rest_lr: float = 0.0025 / 20
    nb_lr_annealing_steps: int = 30_000
    sh_degree_increase_interval: int = 1_000
    opacity_reset_interval: int = 3_000
    opacity_reset_start_iteration_nb: int = 0
    opacity_reset_final_iteration_nb: int = 12_000
    opacity_reset_max_value: float = 0.01
    adc_interval: int = 100
    adc_start_iteration_nb: int = 600
    adc_final_iteration_nb: int = 14_900
    densification_mean2d_grad_norm_threshold_ndc: float = 0.0002
    densification_size_threshold: float = 0.01
    splitting_scale_factor: float = 1 / (0.8 * 2)
    pruning_min_opacity: float = 0.005
    pruning_3d_max_scale: float = 0.1

    @classmethod
    def for_scene(cls, scene_radius: float, **kw):
        nb = kw.get("nb_iterations", 30_000)
        base_lr = kw.pop("base_initial_means_lr", 0.00016)
        base_final = kw.pop("base_final_means_lr", base_lr / 100.0)
        dc = kw.get("sh_coeffs_dc_lr", 0.0025)
        kw.setdefault("sh_coeffs_rest_lr", dc / 20.0)
        kw.setdefault("nb_lr_annealing_steps", nb)
        size = kw.pop("base_densification_size_threshold", 0.01)
        prune_scale = kw.pop("base_pruning_3d_max_scale", 0.1)
        R = float(f32(scene_radius))
        return cls(initial_means_lr=float(f32(base_lr) * f32(R)), final_means_lr=float(f32(base_final) * f32(R)),
                   densification_size_threshold=float(f32(size) * f32(R)),
                   pruning_3d_max_scale=float(f32(prune_scale) * f32(R)), **kw)


def annealed_means_lr(iteration_nb: int, options: TrainingOptions) -> float:
    """The means learning rate update_learning_rates! (training.jl:287-302) sets at iteration
    iteration_nb (1-based), in float32 as the reference computes it:
    x = clamp((it - 1) / (nb_lr_annealing_steps - 1), 0, 1), lr = exp((1 - x) log lr0 + x log lr1)."""
    x = f32(min(max(f32(iteration_nb - 1) / f32(options.nb_lr_annealing_steps - 1), f32(0)), f32(1)))
    lr = np.exp(f32(f32(f32(1) - x) * np.log(f32(options.initial_means_lr)))
                + f32(x * np.log(f32(options.final_means_lr))))
    return float(f32(lr))


class GaussianAdamMomentsLearningRatesVector:
    """Adam moments (m1, m2 interleaved) and learning rates (optimizer.jl:9-195)."""

    def __init__(self, n, sh_degree, lrs, device=0):
        d = _dev(device)
        h = (sh_degree + 1) ** 2
        self.sh_degree = int(sh_degree)
        self.means = torch.zeros((n, 3, 2), dtype=torch.float32, device=d)
        self.opacity = torch.zeros((n, 2), dtype=torch.float32, device=d)
        self.scaling = torch.zeros((n, 3, 2), dtype=torch.float32, device=d)
        self.rotation = torch.zeros((n, 4, 2), dtype=torch.float32, device=d)
        self.sh = torch.zeros((n, 3, h, 2), dtype=torch.float32, device=d)
        (self.means_lr, self.opacity_lr, self.scaling_lr, self.rotation_lr, self.sh_dc_lr,
         self.sh_rest_lr) = [float(v) for v in lrs]

    def __len__(self):
        return self.means.shape[0]

    def lrs(self):
        return [self.means_lr, self.opacity_lr, self.scaling_lr, self.rotation_lr, self.sh_dc_lr, self.sh_rest_lr]


class AdamOptimizer:
    """MutableAdamOptimizer (optimizer.jl:761-854)."""

    def __init__(self, gaussians: TrainableGaussiansVector, options: TrainingOptions, beta1=DEFAULT_BETA1,
                 beta2=DEFAULT_BETA2, epsilon=DEFAULT_EPSILON, update_count=0):
        self.gaussians = gaussians
        lrs = [options.initial_means_lr, options.opacity_features_lr, options.scaling_features_lr,
               options.rotation_features_lr, options.sh_coeffs_dc_lr, options.sh_coeffs_rest_lr]
        self.moments = GaussianAdamMomentsLearningRatesVector(len(gaussians), gaussians.sh_degree, lrs,
                                                              gaussians.device.index)
        self.beta1, self.beta2, self.epsilon = float(f32(beta1)), float(f32(beta2)), float(f32(epsilon))
        self.update_count = int(update_count)

    def struct(self):
        m = self.moments
        s = abi.AdamStateC()
        s.means_moments = dptr(m.means)
        s.opacity_moments = dptr(m.opacity)
        s.scaling_moments = dptr(m.scaling)
        s.rotation_moments = dptr(m.rotation)
        s.sh_moments = dptr(m.sh)
        (s.lr_means, s.lr_opacity, s.lr_scaling, s.lr_rotation, s.lr_sh_dc, s.lr_sh_rest) = m.lrs()
        s.beta1, s.beta2, s.epsilon = self.beta1, self.beta2, self.epsilon
        s.update_count = self.update_count
        return s

    def backward_project_update_(self, fgradients: FilteredGaussiansGradientsVector, camera, options,
                                 buffers, adc=None):
        """The backward projection with update! applied in place of the 3D gradients
        (tdgs_backward_project_adam); the same parameters and moments as backward_project
        followed by update_, bit for bit. fgradients.grads2d must hold the 2D gradients. With
        adc (an AdaptiveDensityControlBuffers), the density-control statistics of the same
        gradients are accumulated in the same launch, as adc_stats_ would
        (tdgs_backward_project_adam_adc)."""
        g = self.gaussians
        st = self.struct()
        args = (stream_ptr(g.device.index), C.byref(fgradients.struct()), C.byref(g.struct()), C.byref(st),
                C.byref(camera.to_c()), C.byref(options.to_c()), C.byref(buffers.struct()),
                C.c_int32(buffers.nb_fgaussians))
        if adc is None:
            check(lib().tdgs_backward_project_adam(*args))
        else:
            check(lib().tdgs_backward_project_adam_adc(*args, C.byref(adc.struct())))
        self.update_count = st.update_count
        return g

    def update_(self, fgradients: FilteredGaussiansGradientsVector, fgidx_to_gidx: torch.Tensor,
                nb_fgaussians: int, sh_degree: int):
        """update!(opt, fgradients, Val(sh_degree)) (optimizer.jl:964-1009)."""
        g = self.gaussians
        st = self.struct()
        check(lib().tdgs_adam_step(stream_ptr(g.device.index), C.byref(g.struct()), C.byref(st),
                                   C.byref(fgradients.struct()), C.c_void_p(dptr(fgidx_to_gidx)),
                                   C.c_int32(nb_fgaussians), C.c_int32(sh_degree)))
        self.update_count = st.update_count
        return g


class AdaptiveDensityControlBuffers:
    """AdaptiveDensityControlBuffers (training_structs.jl:265-331)."""

    def __init__(self, n, device=0):
        d = _dev(device)
        cap = max(int(n), 1)
        self.capacity = cap
        self.accum = torch.zeros(cap, dtype=torch.float32, device=d)
        self.counts = torch.zeros(cap, dtype=torch.int32, device=d)
        self.prune = torch.zeros(cap, dtype=torch.uint8, device=d)
        self.densify = torch.zeros(cap, dtype=torch.uint8, device=d)
        self.clone = torch.zeros(cap, dtype=torch.uint8, device=d)
        self.cs = torch.zeros(cap, dtype=torch.int32, device=d)
        self.new_capacity = 2 * cap
        self.ngidx = torch.zeros(self.new_capacity, dtype=torch.int32, device=d)
        self.temp = torch.empty(int(lib().tdgs_scan_temp_bytes(cap)), dtype=torch.uint8, device=d)

    def struct(self):
        s = abi.AdcBuffersC()
        s.capacity = self.capacity
        s.new_capacity = self.new_capacity
        s.accum_grad_norms = dptr(self.accum)
        s.contribution_counts = dptr(self.counts)
        s.prune = dptr(self.prune)
        s.densify = dptr(self.densify)
        s.clone = dptr(self.clone)
        s.new_counts_cs = dptr(self.cs)
        s.ngidx_to_gidx = dptr(self.ngidx)
        s.temp = dptr(self.temp)
        s.temp_bytes = self.temp.numel()
        return s


def adc_stats_(adc: AdaptiveDensityControlBuffers, fgradients, fgidx_to_gidx, nb_fgaussians, camera, buffers=None):
    """update_adc_stats_kernel! (training.jl:472-497). nb_fgaussians < 0: the counts of a
    device-count render, read on the device from `buffers` (tdgs_adc_stats_frame)."""
    dev = adc.accum.device.index
    if nb_fgaussians < 0:
        check(lib().tdgs_adc_stats_frame(stream_ptr(dev), C.byref(adc.struct()), C.byref(fgradients.struct()),
                                         C.byref(buffers.struct()), C.c_int32(camera.width),
                                         C.c_int32(camera.height)))
        return
    check(lib().tdgs_adc_stats(stream_ptr(dev), C.byref(adc.struct()), C.byref(fgradients.struct()),
                               C.c_void_p(dptr(fgidx_to_gidx)), C.c_int32(nb_fgaussians),
                               C.c_int32(camera.width), C.c_int32(camera.height)))


def adc_plan_(adc, gaussians, prune_logit, use_max_scale, log_max_scale, grad_threshold, log_size_threshold,
              ctx=None):
    """Masks, counts scan and ngidx_to_gidx (training.jl:325-397); returns the new count.
    Synchronises and reports the device error flags of ctx (default: the device's context)."""
    dev = gaussians.device.index
    nn = C.c_int32(0)
    check(lib().tdgs_adc_plan(context(dev) if ctx is None else ctx.handle, stream_ptr(dev), C.byref(adc.struct()), C.byref(gaussians.struct()),
                              C.c_float(prune_logit), C.c_int32(int(use_max_scale)), C.c_float(log_max_scale),
                              C.c_float(grad_threshold), C.c_float(log_size_threshold), C.byref(nn)))
    return int(nn.value)


def adc_plan_thresholds(iteration_nb: int, options: TrainingOptions):
    """The arguments of adc_plan_ after the Gaussians at an ADC step (training.jl:327-350):
    (logit(pruning_min_opacity), whether the max-scale prune applies, log(pruning_3d_max_scale),
    the gradient threshold, log(densification_size_threshold)), in float32 as the reference
    computes them. The max-scale prune applies only once iteration_nb > opacity_reset_interval
    (:337-349)."""
    o = options
    return (float(logit32(o.pruning_min_opacity)), iteration_nb > o.opacity_reset_interval,
            float(np.log(f32(o.pruning_3d_max_scale))), o.densification_mean2d_grad_norm_threshold_ndc,
            float(np.log(f32(o.densification_size_threshold))))


def adaptive_density_control_(adc, gaussians: TrainableGaussiansVector, optimizer: AdamOptimizer, n_new,
                              log_split_factor, seed):
    """adaptive_density_control! on parameters and moments (gaussians.jl:1526-1694,
    optimizer.jl:1304-1378): returns the new Gaussians; the optimizer is updated in place."""
    dev = gaussians.device
    h = (gaussians.sh_degree + 1) ** 2
    new = TrainableGaussiansVector(torch.empty((n_new, 4), dtype=torch.float32, device=dev),
                                   torch.empty((n_new, 3), dtype=torch.float32, device=dev),
                                   torch.empty((n_new, 4), dtype=torch.float32, device=dev),
                                   torch.empty((n_new, 3, h), dtype=torch.float32, device=dev))
    old_m = optimizer.moments
    new_m = GaussianAdamMomentsLearningRatesVector(n_new, gaussians.sh_degree, old_m.lrs(), dev.index)
    src_m, dst_m = optimizer.struct(), None
    optimizer.moments = new_m
    dst_m = optimizer.struct()
    check(lib().tdgs_adc_apply(stream_ptr(dev.index), C.byref(adc.struct()), C.byref(gaussians.struct()),
                               C.byref(new.struct()), C.byref(src_m), C.byref(dst_m), C.c_float(log_split_factor),
                               C.c_uint64(seed)))
    torch.cuda.current_stream(dev).synchronize()  # old arrays may be released after this point
    del old_m
    optimizer.gaussians = new
    return new


def adc_remap_fgidx_(adc, fgidx_to_gidx, nb_fgaussians):
    """adjust_fgidx_to_gidx_adc_kernel! (training.jl:514-541)."""
    dev = fgidx_to_gidx.device.index
    check(lib().tdgs_adc_remap_fgidx(stream_ptr(dev), C.byref(adc.struct()), C.c_void_p(dptr(fgidx_to_gidx)),
                                     C.c_int32(nb_fgaussians)))


def l1_loss_grad_(rendered, gt, grad_out, l1_weight, dssim_weight=0.0, dssim_grad=None, l1_sum=None):
    """L1 part of training_step!'s loss and its gradient (training.jl:206-215)."""
    dev = rendered.device.index
    check(lib().tdgs_l1_loss_grad(stream_ptr(dev), C.c_void_p(dptr(rendered)), C.c_void_p(dptr(gt)),
                                  C.c_int64(rendered.numel()), C.c_float(l1_weight), C.c_float(dssim_weight),
                                  C.c_void_p(dptr(dssim_grad)), C.c_void_p(dptr(grad_out)),
                                  C.c_void_p(dptr(l1_sum))))


def opacity_reset_(gaussians, max_value, opacity_moments):
    """reset_opacities! + zero_opacity_features_adam_moments! (gaussians.jl:1093-1101)."""
    check(lib().tdgs_opacity_reset(stream_ptr(gaussians.device.index), C.byref(gaussians.struct()),
                                   C.c_float(float(logit32(max_value))), C.c_void_p(dptr(opacity_moments))))


def sh_resize(src: torch.Tensor, new_degree: int, interleave: int):
    """resize_array for a new SH degree (misc.jl:100-125): src is (n, 3, h[, 2])."""
    n = src.shape[0]
    hs = src.shape[2]
    hd = (int(new_degree) + 1) ** 2
    shape = (n, 3, hd) + ((2,) if interleave == 2 else ())
    dst = torch.empty(shape, dtype=torch.float32, device=src.device)
    check(lib().tdgs_sh_resize(stream_ptr(src.device.index), C.c_void_p(dptr(src)), C.c_int32(hs),
                               C.c_void_p(dptr(dst)), C.c_int32(hd), C.c_int64(n), C.c_int32(interleave)))
    return dst


def loss_grad_(rendered, gt, grad_out, dssim_weight, sums, temp):
    """L1 + DSSIM loss gradient (training.jl:196-217); sums (2 doubles) must be zeroed."""
    W, H = rendered.shape[0], rendered.shape[1]
    check(lib().tdgs_loss_grad(stream_ptr(rendered.device.index), C.c_void_p(dptr(rendered)),
                               C.c_void_p(dptr(gt)), C.c_int32(W), C.c_int32(H), C.c_float(dssim_weight),
                               C.c_void_p(dptr(grad_out)), C.c_void_p(dptr(sums)), C.c_void_p(dptr(temp)),
                               C.c_size_t(temp.numel())))


class GroundTruthImages:
    """The ground-truth images of a trainer, on the device or on the host.

    Device images (torch tensors on the GPU) are used in place. Host images (numpy arrays or
    CPU tensors) are copied once into pinned memory; each step's image is then uploaded on a
    copy stream of its own into one of two device buffers, one step ahead, so the transfer
    overlaps the previous step's kernels instead of stalling the step as the blocking
    copyto! of training.jl:196-201 does. Events order the copy after the last read of the
    buffer it overwrites and the loss after the copy it reads."""

    def __init__(self, images, device):
        self.device = device
        imgs = list(images)
        self.on_device = all(isinstance(im, torch.Tensor) and im.is_cuda for im in imgs)
        if self.on_device:
            self.images = imgs
            return
        self.pinned = []
        for im in imgs:
            t = im if isinstance(im, torch.Tensor) else torch.from_numpy(np.asarray(im))
            if t.is_cuda:
                raise ValueError("images must be all on the device or all on the host")
            if t.dtype != torch.float32 or t.dim() != 3 or t.shape[2] != 3:
                raise ValueError(f"host images must be float32 (w, h, 3), got {tuple(t.shape)} {t.dtype}")
            self.pinned.append(t.contiguous().pin_memory())
        shapes = {tuple(t.shape) for t in self.pinned}
        if len(shapes) != 1:
            raise ValueError(f"host images of different sizes: {sorted(shapes)}")
        shape = shapes.pop()
        self.buffers = [torch.empty(shape, dtype=torch.float32, device=device) for _ in range(2)]
        self.copy_stream = torch.cuda.Stream(device=device)   # default priority
        self.uploaded = [torch.cuda.Event() for _ in range(2)]
        self.released = [torch.cuda.Event() for _ in range(2)]
        for e in self.released:
            e.record(torch.cuda.current_stream(device))
        self.slot_image = [None, None]
        self.next_slot = 0

    def prefetch(self, k):
        """Start the upload of image k into the next buffer (host images only)."""
        if self.on_device or k in self.slot_image:
            return
        slot = self.next_slot
        self.next_slot ^= 1
        # the host waits until the device has released the buffer the copy overwrites (the
        # loss of the step before the current one): that keeps it one step ahead of the
        # device. Left to run ahead without bound, the copies and events it queues made the
        # runtime stall the host for 8-10 ms at a time (measured at cfg2), after which the
        # device ran dry: 750-790 it/s instead of 868, against 877 with device images.
        self.released[slot].synchronize()
        with torch.cuda.stream(self.copy_stream):
            self.copy_stream.wait_event(self.released[slot])
            self.buffers[slot].copy_(self.pinned[k], non_blocking=True)
            self.uploaded[slot].record(self.copy_stream)
        self.slot_image[slot] = k

    def acquire(self, k):
        """Image k on the device, ordered on the current stream; pair with release(k)."""
        if self.on_device:
            return self.images[k]
        if k not in self.slot_image:
            self.prefetch(k)
        slot = self.slot_image.index(k)
        torch.cuda.current_stream(self.device).wait_event(self.uploaded[slot])
        return self.buffers[slot]

    def release(self, k):
        """The current stream has issued its last read of image k's buffer."""
        if self.on_device:
            return
        slot = self.slot_image.index(k)
        self.released[slot].record(torch.cuda.current_stream(self.device))
        self.slot_image[slot] = None


class Trainer:
    """Trainer (training.jl:40-151) with training_step_ = training_step! (:173-244).

    images[k] is the ground-truth image of cameras[k], (w, h, 3) float32 (the reference's
    3 x h x w layout), either all device tensors or all host arrays (GroundTruthImages). The
    camera order is a seeded permutation, redrawn after every pass over the cameras (the
    reference uses an unseeded randperm!); the next step's camera is known one step ahead,
    so its host image uploads while the current step runs."""

    def __init__(self, gaussians: TrainableGaussiansVector, cameras, images, render_options: RenderOptions,
                 tiling: Tiling, training_options: TrainingOptions, optimizer: AdamOptimizer | None = None,
                 seed: int = 0, device=0, fuse_optimizer: bool = True, record_adc: bool = False,
                 device_counts: bool = True):
        self.device = _dev(device)
        # the trainer's own library context: its frame monitor counts this trainer's
        # device-count frames only, and its error flags are this trainer's
        self.ctx = Context(self.device.index)
        # device_counts: steps without density control or opacity reset (with the fused
        # optimiser) render with TDGS_FLAG_DEVICE_COUNTS, so they wait for no count on the host.
        # Before the next step is issued, the host waits until the context's frame monitor
        # (pinned memory the device writes when the frame's blending starts, with a whole
        # step of kernels still queued behind it) shows that frame. A frame whose keys did not
        # fit rendered as render_void! and left the parameters and moments untouched; it is
        # then run again with host counts (which grow the key arrays), from the same state, so
        # no step is dropped (replayed_steps counts them). The key arrays are also grown ahead
        # of need from the monitor's key counts.
        self.device_counts = device_counts
        self.replayed_steps = 0
        self._monitor = None
        self._monitor_frames0 = 0      # a new context: no frame before this trainer's
        self._monitor_seen = 0         # overflow frames already handled
        self._dc_frames = 0            # device-count frames issued
        self._unconfirmed = None       # (camera index, camera) of the last device-count step
        self._largest_keys = 0   # largest key count of this trainer's frames seen on the monitor
        # record_adc: keep per density-control step the counts of pruned, cloned and split
        # Gaussians in adc_history (three reductions and a synchronisation per ADC step)
        self.record_adc = record_adc
        self.adc_history = []
        # apply update! inside the backward projection when no density control intervenes
        self.fuse_optimizer = fuse_optimizer
        self.gaussians = gaussians
        self.cameras = list(cameras)
        self.images = GroundTruthImages(images, self.device)
        self.render_options = render_options
        self.tiling = tiling
        self.options = training_options
        self.optimizer = optimizer or AdamOptimizer(gaussians, training_options)
        self.rng = np.random.Generator(np.random.PCG64(seed))
        self.seed = seed
        self.iteration_nb = 0
        self.cameras_order = self.rng.permutation(len(self.cameras))
        self.cameras_order_idx = -1
        self.next_order = None   # the permutation after cameras_order, once drawn
        cam0 = self.cameras[0]
        self.render_outputs = RenderOutputs.for_camera(cam0, device, include_rgb=True, include_transmittance=True,
                                                       include_depth=False, include_last_contributing_indices=True)
        self.render_buffers = RenderBuffers(len(gaussians), tiling, device)
        self.fgradients = FilteredGaussiansGradientsVector(len(gaussians), gaussians.sh_degree, device)
        self.adc = AdaptiveDensityControlBuffers(len(gaussians), device)
        self.rgb_image_grad = torch.empty_like(self.render_outputs.rgb)
        self.loss_sums = torch.zeros(2, dtype=torch.float64, device=self.device)
        self.loss_temp = torch.empty(int(lib().tdgs_loss_temp_bytes(cam0.width, cam0.height)), dtype=torch.uint8,
                                     device=self.device)
        self.last_camera = None

    def current_loss(self):
        """Loss of the last step (synchronises): (1-w) mean L1 + w (1 - mean SSIM)."""
        s = self.loss_sums.cpu().numpy()
        n = self.render_outputs.rgb.numel()
        w = self.options.loss_dssim_vs_L1_weight
        return (1 - w) * s[0] / n + w * (1 - s[1] / n)

    def training_step_(self):
        """training_step! (training.jl:173-244)."""
        self.confirm_device_count_step_()
        self.iteration_nb += 1
        self.cameras_order_idx += 1
        if self.cameras_order_idx >= len(self.cameras_order):
            self.cameras_order = self.next_order if self.next_order is not None else \
                self.rng.permutation(len(self.cameras))
            self.next_order = None
            self.cameras_order_idx = 0
        self.maybe_increase_sh_degree_()
        k = int(self.cameras_order[self.cameras_order_idx])
        self.images.prefetch(k)
        self.images.prefetch(self.peek_next_camera())
        cam = self.cameras[k]
        self.last_camera = cam
        dev_counts = (self.device_counts and self.fuse_optimizer and not self.adc_step_due()
                      and not self.opacity_reset_due()
                      and self.fgradients.capacity >= self.render_buffers.capacity
                      and self.tiling.nb_tiles <= 65535)
        in_adc = self._render_to_update_(k, cam, dev_counts)
        if in_adc:
            self.complete_adc_step_()
        self.maybe_opacity_reset_()

    def _render_to_update_(self, k, cam, dev_counts):
        """The part of training_step! from render! to update! (training.jl:186-236) with
        camera k; True when density control ran."""
        if dev_counts:
            self._grow_keys_from_monitor()
        render_(self.render_outputs, self.gaussians, cam, self.tiling, self.render_options, self.render_buffers,
                device_counts=dev_counts, ctx=self.ctx)
        if dev_counts:
            self._dc_frames += 1
            self._unconfirmed = (k, cam)
        self.loss_sums.zero_()
        gt = self.images.acquire(k)
        w = self.options.loss_dssim_vs_L1_weight
        if w == 0:
            # L1 only: the reference still evaluates D-SSIM with weight 0 (training.jl:202-215)
            l1_loss_grad_(self.render_outputs.rgb, gt, self.rgb_image_grad, 1.0, 0.0, None, self.loss_sums[0:1])
        else:
            loss_grad_(self.render_outputs.rgb, gt, self.rgb_image_grad, w, self.loss_sums, self.loss_temp)
        self.images.release(k)
        if self.fuse_optimizer and not self.adc_step_due():
            # no density control between the backward pass and update!: the backward
            # projection applies the optimiser step itself (the 3D gradients are not stored),
            # and accumulates the density-control statistics (maybe_densify_and_prune!'s only
            # work in such an iteration) in the same launch
            backward_render_tiles_(self.fgradients, self.rgb_image_grad, self.render_outputs, cam, self.tiling,
                                   self.render_options, self.render_buffers)
            stats = self.iteration_nb <= self.options.adc_final_iteration_nb
            self.update_learning_rates_()
            self.optimizer.backward_project_update_(self.fgradients, cam, self.render_options, self.render_buffers,
                                                    adc=self.adc if stats else None)
            in_adc = False
        else:
            backward_(self.fgradients, self.rgb_image_grad, self.render_outputs, self.gaussians, cam, self.tiling,
                      self.render_options, self.render_buffers)
            in_adc = self.maybe_densify_and_prune_()
            self.update_learning_rates_()
            self.optimizer.update_(self.fgradients, self.render_buffers.fgidx_to_gidx,
                                   self.render_buffers.nb_fgaussians, self.render_options.sh_degree)
        return in_adc

    def confirm_device_count_step_(self, timeout_s: float = 60.0):
        """Waits until the frame monitor shows the last device-count step's frame (its
        blending has started, so the rest of that step is still queued on the device), raises
        on device error flags, and re-runs that step with host counts when its keys did not
        fit (the device left the parameters and moments untouched; update! counted the step,
        so the count is taken back first). Every step is thereby applied exactly once, in
        order. training_step_ calls it first; call it after the last step (finish_)."""
        if self._unconfirmed is None:
            return
        k, cam = self._unconfirmed
        self._unconfirmed = None
        target = self._monitor_frames0 + self._dc_frames
        mon = self.frame_monitor()
        if mon[0] < target:
            t0 = time.monotonic()
            while mon[0] < target:
                if time.monotonic() - t0 > timeout_s:
                    ctx_check(self.device.index, self.ctx)   # raises on a device-side error
                    raise RuntimeError(f"frame {target} of the trainer's context did not start blending "
                                       f"within {timeout_s} s (monitor {mon})")
                time.sleep(0)
                mon = self.frame_monitor()
        if mon[4]:
            ctx_check(self.device.index, self.ctx)   # reports and clears the flags
            raise RuntimeError(f"device error flags {mon[4]:#x} at training iteration {self.iteration_nb}")
        if mon[2] > self._monitor_seen:
            self._monitor_seen = mon[2]
            self._largest_keys = max(self._largest_keys, mon[3])
            self.replayed_steps += 1
            self.optimizer.update_count -= 1
            self._render_to_update_(k, cam, False)

    def finish_(self):
        """Confirms the last step (see confirm_device_count_step_) and checks the context's
        device error flags (synchronises)."""
        self.confirm_device_count_step_()
        ctx_check(self.device.index, self.ctx)

    def frame_monitor(self):
        """The trainer context's frame monitor (tdgs_ctx_frame_monitor): [frames, largest key
        count, frames whose keys did not fit, last key count, pending device error flags] of
        its device-count renders so far, read without synchronisation."""
        if self._monitor is None:
            p = C.POINTER(C.c_int64)()
            check(lib().tdgs_ctx_frame_monitor(self.ctx.handle, C.byref(p)))
            self._monitor = p
        return [int(self._monitor[i]) for i in range(5)]

    def _grow_keys_from_monitor(self):
        """Grows the key arrays to 1.5x the largest key count seen once it passes 80% of the
        capacity (the monitor shows the frames whose blending has started)."""
        frames, _, _, last, _ = self.frame_monitor()
        if frames > self._monitor_frames0:
            self._largest_keys = max(self._largest_keys, last)
        b = self.render_buffers
        want = int(1.5 * self._largest_keys) + 1024 if self._largest_keys > 0.8 * b.key_capacity else 0
        if want > b.key_capacity:
            b._alloc_keys(want)

    def adc_step_due(self):
        """Whether maybe_densify_and_prune! densifies and prunes at this iteration."""
        o = self.options
        it = self.iteration_nb
        return it <= o.adc_final_iteration_nb and it >= o.adc_start_iteration_nb and it % o.adc_interval == 0

    def peek_next_camera(self):
        """Camera index of the next step (draws the next permutation early if needed; the
        sequence of permutations is the same as drawing it when it is reached)."""
        i = self.cameras_order_idx + 1
        if i < len(self.cameras_order):
            return int(self.cameras_order[i])
        if self.next_order is None:
            self.next_order = self.rng.permutation(len(self.cameras))
        return int(self.next_order[0])

    def maybe_increase_sh_degree_(self):
        """maybe_increase_sh_degree! (training.jl:253-263)."""
        if self.iteration_nb % self.options.sh_degree_increase_interval != 0:
            return
        d = self.gaussians.sh_degree
        if d >= 3:
            return
        d += 1
        self.render_options = self.render_options.with_sh_degree(d)
        self.gaussians.sh = sh_resize(self.gaussians.sh, d, 1)
        self.fgradients.sh = sh_resize(self.fgradients.sh, d, 1)
        self.fgradients.sh_degree = d
        m = self.optimizer.moments
        m.sh = sh_resize(m.sh, d, 2)
        m.sh_degree = d

    def opacity_reset_due(self):
        """Whether maybe_opacity_reset! resets the opacities at this iteration."""
        o = self.options
        it = self.iteration_nb
        return o.opacity_reset_start_iteration_nb <= it <= o.opacity_reset_final_iteration_nb and \
            it % o.opacity_reset_interval == 0

    def maybe_opacity_reset_(self):
        """maybe_opacity_reset! (training.jl:272-280)."""
        if self.opacity_reset_due():
            o = self.options
            opacity_reset_(self.gaussians, o.opacity_reset_max_value, self.optimizer.moments.opacity)

    def update_learning_rates_(self):
        """update_learning_rates! (training.jl:287-302)."""
        self.optimizer.moments.means_lr = annealed_means_lr(self.iteration_nb, self.options)

    def maybe_densify_and_prune_(self):
        """maybe_densify_and_prune! (training.jl:313-444); True when an ADC step ran."""
        o = self.options
        it = self.iteration_nb
        if it > o.adc_final_iteration_nb:
            return False
        nbf = self.render_buffers.nb_fgaussians
        adc_stats_(self.adc, self.fgradients, self.render_buffers.fgidx_to_gidx, nbf, self.last_camera,
                   self.render_buffers)
        if not (it >= o.adc_start_iteration_nb and it % o.adc_interval == 0):
            return False
        n_new = adc_plan_(self.adc, self.gaussians, *adc_plan_thresholds(it, o), ctx=self.ctx)
        if self.record_adc:
            n = len(self.gaussians)
            a = self.adc
            dens = a.densify[:n].bool()
            cl = dens & a.clone[:n].bool()
            self.adc_history.append({"iteration": it, "before": n, "after": n_new,
                                     "pruned": int(a.prune[:n].sum().item()), "cloned": int(cl.sum().item()),
                                     "split": int((dens & ~cl).sum().item())})
        new = adaptive_density_control_(self.adc, self.gaussians, self.optimizer, n_new,
                                        float(np.log(f32(o.splitting_scale_factor))), self.seed * 1_000_003 + it)
        adc_remap_fgidx_(self.adc, self.render_buffers.fgidx_to_gidx, nbf)
        self.gaussians = new
        self.adc = AdaptiveDensityControlBuffers(n_new, self.device.index)
        return True

    def complete_adc_step_(self):
        """complete_adc_step! (training.jl:455-459): resize gradients and render buffers."""
        n = len(self.gaussians)
        self.render_buffers.ensure_capacity(n)
        # (at least the render buffers' capacity, which device-count steps need)
        self.fgradients = FilteredGaussiansGradientsVector(max(n, self.render_buffers.capacity),
                                                           self.gaussians.sh_degree, self.device.index)
