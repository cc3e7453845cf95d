"""Benchmark of the render core on one MI355X: BASELINE.json's headline metric.

Workload: 1,000,000 Gaussians, 1920x1080, SH degree 3, 120
seeded orbit cameras, 16x16 tiles; synthetic seeded data. A step renders one camera (frame
k uses camera k mod 120) with the full render! pipeline: cull, compaction, projection,
duplication, sort, ranges and blending, with the counts kept on the device (no host
synchronisation per frame; frames_per_s_host_counts repeats the frames with the reference's
per-frame readback).

Prints one JSON line. `value` is frames/s over the timed steps (render! calls only: the
per-frame events and the stage profiler run on separate passes over the cameras);
`roofline` describes the stage that takes the most time, with its algorithmic bytes (or
FLOP) per launch divided by its mean duration measured live with HIP events on the rendering
stream; `cpu_baseline`
times the reference's own CPU renderer (render! for CPU arrays, forward_core.jl:25-177,
restated in C++ in oracle/) on one frame of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
import __graft_entry__  # noqa: E402

__graft_entry__.load_package()

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP32_PEAK_TFLOPS = 157.3       # MI355X vector FP32 (published)
# Gaussians up to which the depth presort is the bucket sort (kDsMaxSlots in csrc/dsort.hpp)
DS_MAX_SLOTS = 1_400_000

# FLOP of blending under the metric's accounting: 20 per (pixel, sorted entry) evaluation made
# before the pixel's early exit (E_f) plus one exponential per evaluation; backward blending
# ~60 per (pixel, entry) evaluation of the reverse walk (E_b).
BLEND_FLOP_PER_EVAL, BLEND_EXP_PER_EVAL = 20, 1
BACKWARD_BLEND_FLOP_PER_EVAL = 60
# The same loop's FLOP as this build executes it (reported beside, labelled "detailed"): the
# exponent, 5 FMA (10), for every evaluation; for one that passes the exponent cut also the
# exponential (1 mul, 2 + 6 FMA, 1 mul: 18) and 1 - alpha, T (1 - alpha) (2); for a
# contributing one also the weight T alpha (1) and the colour, 3 FMA (6).
BLEND_FLOP_EVAL, BLEND_FLOP_LIVE, BLEND_FLOP_CONTRIB = 10, 20, 7

STAGES = ["cull_compact", "project", "depth_sort", "count_scan", "emit", "tile_sort", "tile_ranges",
          "blend", "backward_blend", "backward_project", "adam", "adc", "loss"]


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=600)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", type=int, default=2)
    p.add_argument("--train-steps", type=int, default=100)
    p.add_argument("--train-warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra-configs", action="store_true",
                   help="skip the config 1 / 3 training and config 4 stress legs")
    p.add_argument("--cfg3-iterations", type=int, default=3000)
    p.add_argument("--no-in-flight", action="store_true",
                   help="skip the frames-in-flight legs (kernel profiles: their concurrent launches "
                        "would mix into the single-stream kernel durations)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run 10 device-to-device copies of 1 GiB (HBM counter calibration)")
    p.add_argument("--only", choices=["stress_cfg4", "sort_pairs", "train_cfg3", "train_cfg3_growth"],
                   help="only run one of the extra legs and print its JSON (kernel profiles of that leg)")
    p.add_argument("--traffic-summary", nargs=4, metavar=("FETCH_DB", "WRITE_DB", "COPY_FETCH_DB", "COPY_WRITE_DB"),
                   help="print the HBM traffic summary (profiles/hbm_traffic.json) from the rocpd databases "
                        "of rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this script and of --copy-calibration")
    return p.parse_args()


def copy_calibration():
    """Known-size traffic for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE: each copy reads and
    writes exactly 1 GiB."""
    import torch
    src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_each": 1 << 30, "copies": 10}))


# rocprofv3 kernel names -> the counter summary's keys (the first match wins; the blend is the
# timed render's variant, without last-contributor output)
TRAFFIC_KERNELS = [
    ("k_render_tiles<true, false, false, false>", "blend"),
    ("k_backward_blend<", "backward_blend"),
    ("k_project<", "project"),
    ("k_keep_counts", "keep_counts"),
    ("k_adam(", "adam"),
    ("k_emit_count<", "emit_count"),
    ("k_emit_scatter<", "coarse_sort_scatter"),
    ("k_backward_project<false>", "backward_project"),
    ("k_backward_project<true>", "backward_project_adam"),
    ("k_rs_scatter_grouped<unsigned int>", "depth_sort_scatter"),
    ("k_rs_count_grouped<unsigned int>", "depth_sort_count"),
    ("k_ds_count", "depth_sort_bucket_count"),
    ("k_ds_scatter", "depth_sort_bucket_scatter"),
    ("k_ds_buckets", "depth_sort_buckets"),
    ("k_ssim_forward", "loss_ssim_forward"),
    ("k_ssim_backward", "loss_ssim_backward"),
    ("k_bin_tiles<3, false>", "bin_count"),
    ("k_bin_tiles<3, true>", "bin_write"),
    ("k_bin_tiles<4, false>", "bin_count_16x"),
    ("k_bin_tiles<4, true>", "bin_write_16x"),
    ("k_bin_scan", "bin_scan"),
    ("k_scan_apply<tdgs::SortedTileBlockCounts", "count_scan_apply"),
]


def _pmc_means(db, counter):
    """Mean value per dispatch of one counter, by kernel name, from a rocpd database."""
    import sqlite3
    con = sqlite3.connect(db)
    per = {}
    for name, value, did in con.execute(
            "select name, counter_value, dispatch_id from pmc_events where counter_name = ?", (counter,)):
        d = per.setdefault(name, {})
        d[did] = d.get(did, 0.0) + value   # (summed over the counter's instances)
    con.close()
    return {k: (sum(v.values()) / len(v), len(v)) for k, v in per.items()}


def traffic_summary(fetch_db, write_db, cfetch_db, cwrite_db):
    """HBM bytes per launch of each kernel: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) scaled
    by what they read for one device-to-device copy of 1 GiB (--copy-calibration)."""
    fetch, write = _pmc_means(fetch_db, "FETCH_SIZE"), _pmc_means(write_db, "WRITE_SIZE")

    def calib(db, counter):
        m = {k: v for k, v in _pmc_means(db, counter).items() if "copy" in k.lower()}
        name = max(m, key=lambda k: m[k][1])   # the copy run ten times
        return (1 << 30) / (m[name][0] * 1024.0)

    ff, wf = calib(cfetch_db, "FETCH_SIZE"), calib(cwrite_db, "WRITE_SIZE")
    kernels = {}
    for name in sorted(set(fetch) | set(write)):
        key = next((k for pat, k in TRAFFIC_KERNELS if pat in name), None)
        if key is None or key in kernels or name not in fetch or name not in write:
            continue
        fb, wb = fetch[name][0] * 1024.0 * ff, write[name][0] * 1024.0 * wf
        kernels[key] = {"kernel": name, "dispatches": fetch[name][1], "fetch_bytes": int(fb),
                        "write_bytes": int(wb), "bytes_per_launch": int(fb + wb)}
    return {"calibration": {"fetch_factor": ff, "write_factor": wf}, "kernels": kernels}


def hbm_practical():
    """What a streaming kernel reaches on this part (context for the HBM fractions, which are
    quoted against the 8 TB/s peak): torch's copy of 1 GiB (read + write), timed with HIP events
    over 5 repetitions after 2."""
    import torch
    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    out = {}
    for name, fn, moved in (("copy", lambda: dst.copy_(src), 2 * 4 * n),):
        for _ in range(2):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(5 * moved / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    del src, dst
    torch.cuda.empty_cache()
    return out


def traffic_from_profiles(kernel):
    """HBM bytes per launch of a kernel from the committed rocprofv3 counter summary
    (profiles/hbm_traffic.json, written from two --pmc runs), or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    k = t.get("kernels", {}).get(kernel)
    return None if k is None else k.get("bytes_per_launch")


def backward_evaluations(last, tiles_end, tiling):
    """E_b: the (pixel, sorted entry) evaluations of backward blending's reverse walk, each
    pixel from its last contributor back to its tile's first entry (backward_core.jl:212-224):
    sum over pixels with last > 0 of last - (index before the tile's first entry)."""
    import torch
    W, H = last.shape
    u = torch.arange(W, device=last.device)[:, None] // tiling.tile_width
    v = torch.arange(H, device=last.device)[None, :] // tiling.tile_height
    tile0 = u + v * tiling.nb_tiles_x                         # 0-based tile of each pixel
    te = tiles_end.to(torch.int64)
    beg = torch.where(tile0 > 0, te[(tile0 - 1).clamp(min=0)], torch.zeros_like(tile0))
    lst = last.to(torch.int64)
    return int(torch.where(lst > 0, lst - beg, torch.zeros_like(lst)).sum().item())


def bin_geometry(tiling):
    """The coarse blocks of the tile lists (forward.hip bin_geom): log2 of the block size in tiles
    (x, y), the smallest of 8x8, 16x8, 16x16 tiles that leaves at most 255 blocks."""
    for sx, sy in ((3, 3), (4, 3), (4, 4)):
        nbx, nby = -(-tiling.nb_tiles_x // (1 << sx)), -(-tiling.nb_tiles_y // (1 << sy))
        if nbx * nby <= 255:
            break
    return sx, sy


def coarse_entries(ranges, counts, tiling):
    """M_c: (Gaussian, coarse block) pairs of the non-empty Gaussians (the binning's entries);
    ranges holds each Gaussian's 1-based inclusive tile rectangle (x0, y0, x1, y1)."""
    if tiling.nb_tiles > 65535:
        return 0
    sx, sy = bin_geometry(tiling)
    r = ranges[counts > 0].astype(np.int64)
    bx = ((r[:, 2] - 1) >> sx) - ((r[:, 0] - 1) >> sx) + 1
    by = ((r[:, 3] - 1) >> sy) - ((r[:, 1] - 1) >> sy) + 1
    return int(bx.dot(by))


def frame_stats(core, g, cams, tiling, opts, buffers, idx):
    """N_f, N_b, M, blending evaluations E_f (all, past the exponent cut, contributing), the
    backward walk's evaluations E_b and the binning's coarse entries M_c, for the given cameras
    (untimed pass)."""
    import torch
    L = core.lib()
    outputs = core.RenderOutputs.for_camera(cams[0], 0, include_rgb=True, include_transmittance=True,
                                            include_depth=False, include_last_contributing_indices=True)
    ev = torch.zeros(3, dtype=torch.int64, device="cuda")
    st = []
    for k in idx:
        core.render_(outputs, g, cams[k], tiling, opts, buffers)
        nf = buffers.nb_fgaussians
        counts = buffers.counts[:nf].cpu().numpy()
        nb = int((counts > 0).sum())
        mc = coarse_entries(buffers.tile_ranges[:nf].cpu().numpy(), counts, tiling)
        ev.zero_()
        core.check(L.tdgs_blend_evaluations(core.stream_ptr(0), C.byref(cams[k].to_c()), C.byref(tiling.to_c()),
                                            C.byref(opts.to_c()), C.byref(buffers.struct()),
                                            C.c_int64(buffers.nb_keys), C.c_void_p(ev.data_ptr())))
        e = ev.cpu().tolist()
        eb = backward_evaluations(outputs.last, buffers.tiles_end, tiling)
        st.append((nf, nb, buffers.nb_keys, e[0], e[1], e[2], eb, mc))
    torch.cuda.synchronize()
    return np.array(st, dtype=np.float64)


def train_bench(core, w, cams, tiling, deg, steps, warmup):
    """Training steps (training_step!: render, L1 + DSSIM loss, backward, ADC statistics,
    learning-rate annealing, Adam) on the same workload, at iterations before the first
    densification (iteration 600), against seeded uniform-noise target images."""
    import torch
    from tdgs_amd import host, training
    g = core.TrainableGaussiansVector.from_host(w.gaussians, 0)
    gen = torch.Generator(device="cuda").manual_seed(0x3D6501)
    images = [torch.rand((c.width, c.height, 3), generator=gen, device="cuda") for c in cams]
    opts = host.RenderOptions.for_camera(cams[0], deg)
    to = training.TrainingOptions.for_scene(host.scene_radius(cams), sh_degree_increase_interval=10**9)
    tr = training.Trainer(g, cams, images, opts, tiling, to, seed=1)
    # key arrays sized on every camera (synchronous renders grow them): the steps without
    # density control then run without host synchronisation and none is skipped
    for c in cams:
        core.render_(tr.render_outputs, g, c, tiling, opts, tr.render_buffers)
    for _ in range(warmup):
        tr.training_step_()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tr.training_step_()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    loss = tr.current_loss()
    tr.finish_()
    assert tr.replayed_steps == 0, "a timed step's keys did not fit the key arrays"
    # stage times from further steps with the stage profiler on (its events are not in the
    # timed loop above)
    L = core.lib()
    psteps = max(10, steps // 4)
    core.check(L.tdgs_profile_begin(C.c_int32(16 * psteps + 64)))
    for _ in range(psteps):
        tr.training_step_()
    torch.cuda.synchronize()
    ms = (C.c_double * 13)()
    cnt = (C.c_int64 * 13)()
    core.check(L.tdgs_profile_end(ms, cnt))
    stage = {STAGES[i]: round(ms[i] / psteps, 4) for i in range(13) if cnt[i] > 0}
    # the backward projection and Adam as separate launches (what the trainer runs at density
    # control iterations), for their per-kernel times
    tr.fuse_optimizer = False
    core.check(L.tdgs_profile_begin(C.c_int32(16 * psteps + 64)))
    for _ in range(psteps):
        tr.training_step_()
    torch.cuda.synchronize()
    core.check(L.tdgs_profile_end(ms, cnt))
    assert tr.iteration_nb < to.adc_start_iteration_nb
    stage["unfused"] = {}
    for name in ("backward_project", "adam"):
        i = STAGES.index(name)
        if cnt[i] > 0:
            stage["unfused"][name] = round(ms[i] / psteps, 4)
    return steps / (t1 - t0), (t1 - t0) * 1000.0 / steps, stage, loss


def train_host_images(core, w, tiling, deg, steps=60, warmup=5, ncams=16):
    """Training steps of the main workload with the ground truth on the host (pinned,
    uploaded one step ahead on a copy stream) beside the same steps with it on the device:
    the difference is what the host-to-device traffic costs once overlapped."""
    import torch
    from tdgs_amd import host, training
    cams = w.cameras[:ncams]
    rng = np.random.Generator(np.random.PCG64(0x3D6501))
    host_imgs = [rng.random((c.width, c.height, 3), dtype=np.float32) for c in cams]
    out = {"cameras": ncams, "steps": steps, "image_MB": round(host_imgs[0].nbytes / 1e6, 2)}
    for name, images in (("device", [torch.from_numpy(im).cuda() for im in host_imgs]), ("host", host_imgs)):
        g = core.TrainableGaussiansVector.from_host(w.gaussians, 0)
        opts = host.RenderOptions.for_camera(cams[0], deg)
        to = training.TrainingOptions.for_scene(host.scene_radius(w.cameras), sh_degree_increase_interval=10**9)
        tr = training.Trainer(g, cams, images, opts, tiling, to, seed=1)
        for _ in range(warmup):
            tr.training_step_()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            tr.training_step_()
        torch.cuda.synchronize()
        out[f"{name}_images_it_per_s"] = round(steps / (time.perf_counter() - t0), 2)
        del tr, g
        torch.cuda.empty_cache()
    return out


def train_cfg1(core, steps=100, warmup=5):
    """Config 1: one training step (200k Gaussians, 800x800, SH3, L1 + 0.2 DSSIM against a seeded
    uniform target) repeated `steps` times on its single camera."""
    import torch
    from tdgs_amd import host, synthetic, training
    w = synthetic.config(1)
    cam = w.cameras[0]
    tiling = synthetic.tiling_for(w, cam)
    g = core.TrainableGaussiansVector.from_host(w.gaussians, 0)
    gen = torch.Generator(device="cuda").manual_seed(0x3D6501)
    images = [torch.rand((cam.width, cam.height, 3), generator=gen, device="cuda")]
    opts = host.RenderOptions.for_camera(cam, 3)
    # one camera: scene_radius (spread of the camera centres, scene.jl:64-73) would be 0 and
    # the annealed means learning rate log-linear in 0; use 1.1 x the camera's distance to the
    # point it looks at (the origin) instead
    radius = 1.1 * float(np.linalg.norm(cam.position))
    to = training.TrainingOptions.for_scene(radius, sh_degree_increase_interval=10**9)
    tr = training.Trainer(g, w.cameras, images, opts, tiling, to, seed=1)
    for _ in range(warmup):
        tr.training_step_()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tr.training_step_()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return {"workload": w.name, "train_it_per_s": round(steps / dt, 2), "ms_per_iteration": round(dt * 1e3 / steps, 4),
            "steps": steps, "loss_last": round(float(tr.current_loss()), 6)}


def train_cfg3(core, iterations, grad_threshold=None):
    """Config 3: the full training loop from 500k Gaussians (1297x840, SH3, 100 orbit cameras,
    seeded uniform-noise targets) with the reference TrainingOptions defaults for
    `iterations` iterations: density control every 100 iterations from 600, opacity reset at
    3000. Wall time of all iterations, densification and pruning included. grad_threshold
    replaces the densification threshold (2e-4): with uniform-noise targets the default keeps
    the count near 500k, a lower one grows it past 1M as the config's "up to ~1.5M" says."""
    import torch
    from tdgs_amd import host, synthetic, training
    w = synthetic.config(3)
    cams = w.cameras
    tiling = synthetic.tiling_for(w, cams[0])
    g = core.TrainableGaussiansVector.from_host(w.gaussians, 0)
    gen = torch.Generator(device="cuda").manual_seed(0x3D6503)
    images = [torch.rand((c.width, c.height, 3), generator=gen, device="cuda") for c in cams]
    opts = host.RenderOptions.for_camera(cams[0], 3)
    kw = {} if grad_threshold is None else {"densification_mean2d_grad_norm_threshold_ndc": grad_threshold}
    to = training.TrainingOptions.for_scene(host.scene_radius(cams), nb_iterations=iterations, **kw)
    tr = training.Trainer(g, cams, images, opts, tiling, to, seed=3, record_adc=True)
    n0 = len(tr.gaussians)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    nmax = n0
    for _ in range(iterations):
        tr.training_step_()
        nmax = max(nmax, len(tr.gaussians))
    tr.finish_()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    assert tr.optimizer.update_count == iterations
    return {"workload": w.name + f", {iterations} iterations with density control",
            "densification_threshold": to.densification_mean2d_grad_norm_threshold_ndc,
            "train_it_per_s": round(iterations / dt, 2), "seconds": round(dt, 3), "iterations": iterations,
            "gaussians_initial": n0, "gaussians_final": len(tr.gaussians), "gaussians_max": nmax,
            "steps_rerun_with_host_counts": tr.replayed_steps,
            "density_control": tr.adc_history, "loss_last": round(float(tr.current_loss()), 6)}


def sort_pairs_bench(core, n=120_000_000, end_bit=46, repeats=5):
    """tdgs_sort_pairs (the drop-in of cub_sort_pairs_wrapper.cu:31-43) on n random (tile, depth
    bits) keys with end_bit 46 (cfg4's 16320 tiles), as forward_core.jl:618-660 calls it at
    cfg4's scale: HIP events around each call, median. Bytes: this build's passes (8-bit
    digits: per pass a count reading the keys, a scatter reading and writing keys and values,
    8 + 2 (8 + 4) = 32 B per key) and CUB's onesweep passes over the same bits (reading and
    writing keys and values, 2 (8 + 4) = 24 B per key and pass, plus one read of the keys for
    its histograms)."""
    import torch
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device="cuda").manual_seed(0x5047)
    tile = torch.randint(1, 16321, (n,), generator=gen, device=dev, dtype=torch.int64)
    depth = torch.randint(0x3c000000, 0x42000000, (n,), generator=gen, device=dev, dtype=torch.int64)
    keys = (tile << 32) | depth
    del tile, depth
    vals = torch.arange(1, n + 1, dtype=torch.int32, device=dev)
    L = core.lib()
    tb = int(L.tdgs_sort_pairs_temp_bytes(n, end_bit))
    temp = torch.empty(tb, dtype=torch.uint8, device=dev)
    ko = torch.empty_like(keys)
    vo = torch.empty_like(vals)
    stream = core.stream_ptr(0)
    times = []
    for r in range(repeats + 1):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        core.check(L.tdgs_sort_pairs(core.dptr(temp), tb, core.dptr(keys), core.dptr(ko), core.dptr(vals),
                                     core.dptr(vo), n, end_bit, stream))
        e1.record()
        torch.cuda.synchronize()
        if r > 0:
            times.append(e0.elapsed_time(e1))
    ms = float(np.median(times))
    assert bool((ko[1:] >= ko[:-1]).all())
    passes = -(-end_bit // 8)
    impl = passes * 32 * n
    cub = passes * 24 * n + 8 * n
    del keys, vals, ko, vo, temp
    torch.cuda.empty_cache()
    return {"keys": n, "end_bit": end_bit, "passes": passes, "ms": round(ms, 3),
            "keys_per_s": round(n / (ms * 1e-3), 1),
            "impl_bytes": impl, "impl_GBs": round(impl / (ms * 1e-3) / 1e9, 1),
            "impl_hbm_frac": round(impl / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "cub_equivalent_bytes": cub, "cub_equivalent_GBs": round(cub / (ms * 1e-3) / 1e9, 1)}


def render_other_tiling(core, w, g, tile, frames=240, warmup=10):
    """The headline render with another tile size (the reference's default at 1080p is 16x32,
    forward_structs.jl:419-424): wall-clock frames/s and the blending stage time."""
    import torch
    from tdgs_amd import host
    cams = w.cameras
    t = host.Tiling.for_camera(cams[0], *tile)
    opts = host.RenderOptions.for_camera(cams[0], w.gaussians.sh_degree)
    out = core.RenderOutputs.for_camera(cams[0], 0, include_rgb=True, include_transmittance=True,
                                        include_depth=False, include_last_contributing_indices=False)
    buf = core.RenderBuffers(len(g), t, 0)
    for k in range(warmup):
        core.render_(out, g, cams[k % len(cams)], t, opts, buf)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(frames):
        core.render_(out, g, cams[k % len(cams)], t, opts, buf)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    L = core.lib()
    core.check(L.tdgs_profile_begin(C.c_int32(16 * len(cams) + 64)))
    for k in range(len(cams)):
        core.render_(out, g, cams[k], t, opts, buf)
    torch.cuda.synchronize()
    ms = (C.c_double * 13)()
    cnt = (C.c_int64 * 13)()
    core.check(L.tdgs_profile_end(ms, cnt))
    return {"tile": list(tile), "tiles": t.nb_tiles, "frames": frames,
            "frames_per_s": round(frames / (t1 - t0), 2),
            "stage_ms": {STAGES[i]: round(ms[i] / cnt[i], 4) for i in range(13) if cnt[i] > 0}}


def render_in_flight(core, g, cams, tiling, opts, key_capacity, frames, streams):
    """The headline frames with `streams` frames in flight: frame k is rendered on stream
    k % streams with that stream's own library context, render buffers and outputs (a
    context holds the device counters of one frame at a time), without host synchronisation.
    While one frame's sort chain (short, latency-bound launches) runs, another frame's
    blending fills the rest of the GPU. Wall-clock frames/s over all streams."""
    import torch
    ncam = len(cams)
    ctxs = [core.Context(0) for _ in range(streams)]
    strs = [torch.cuda.Stream() for _ in range(streams)]
    outs = [core.RenderOutputs.for_camera(cams[0], 0, include_rgb=True, include_transmittance=True,
                                          include_depth=False, include_last_contributing_indices=False)
            for _ in range(streams)]
    bufs = [core.RenderBuffers(len(g), tiling, 0, key_capacity) for _ in range(streams)]
    mons = []
    for c in ctxs:
        p = C.POINTER(C.c_int64)()
        core.check(core.lib().tdgs_ctx_frame_monitor(c.handle, C.byref(p)))
        mons.append(p)
    torch.cuda.synchronize()

    def run(k0, k1):
        for k in range(k0, k1):
            s = k % streams
            with torch.cuda.stream(strs[s]):
                core.render_(outs[s], g, cams[k % ncam], tiling, opts, bufs[s], device_counts=True, ctx=ctxs[s])

    run(0, 4 * streams)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(0, frames)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    assert all(int(p[2]) == 0 for p in mons), "a frame's keys did not fit the key arrays"
    assert sum(int(p[0]) for p in mons) == frames + 4 * streams
    for c in ctxs:
        c.close()
    return {"streams": streams, "frames": frames, "frames_per_s": round(frames / dt, 2),
            "ms_per_frame": round(dt * 1000.0 / frames, 4)}


def stress_cfg4(core, repeats=5):
    """Config 4: 3M Gaussians at 3840x2160 (SH3, 16x32 tiles), forward and backward of one
    camera against a seeded uniform target; more than 100M duplicated keys."""
    import torch
    from tdgs_amd import host, synthetic, training
    w = synthetic.config(4)
    cam = w.cameras[0]
    tiling = synthetic.tiling_for(w, cam)
    g = core.TrainableGaussiansVector.from_host(w.gaussians, 0)
    opts = host.RenderOptions.for_camera(cam, 3)
    out = core.RenderOutputs.for_camera(cam, 0, include_rgb=True, include_transmittance=True, include_depth=False,
                                        include_last_contributing_indices=True)
    buf = core.RenderBuffers(len(g), tiling, 0)
    fg = core.FilteredGaussiansGradientsVector(len(g), 3, 0)
    gen = torch.Generator(device="cuda").manual_seed(0x3D6504)
    gt = torch.rand((cam.width, cam.height, 3), generator=gen, device="cuda")
    grad = torch.empty_like(out.rgb)
    sums = torch.zeros(2, dtype=torch.float64, device="cuda")
    temp = torch.empty(int(core.lib().tdgs_loss_temp_bytes(cam.width, cam.height)), dtype=torch.uint8, device="cuda")
    core.render_(out, g, cam, tiling, opts, buf)
    training.loss_grad_(out.rgb, gt, grad, 0.2, sums, temp)
    core.backward_(fg, grad, out, g, cam, tiling, opts, buf)
    torch.cuda.synchronize()
    L = core.lib()
    core.check(L.tdgs_profile_begin(C.c_int32(16 * repeats + 64)))
    fw, bw = [], []
    for _ in range(repeats):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        core.render_(out, g, cam, tiling, opts, buf)
        e[1].record()
        core.backward_(fg, grad, out, g, cam, tiling, opts, buf)
        e[2].record()
        torch.cuda.synchronize()
        fw.append(e[0].elapsed_time(e[1]))
        bw.append(e[1].elapsed_time(e[2]))
    ms = (C.c_double * 13)()
    cnt = (C.c_int64 * 13)()
    core.check(L.tdgs_profile_end(ms, cnt))
    stage = {STAGES[i]: round(ms[i] / cnt[i], 4) for i in range(13) if cnt[i] > 0}
    m, nf = buf.nb_keys, buf.nb_fgaussians
    counts = buf.counts[:nf].cpu().numpy()
    nb = int((counts > 0).sum())
    mc = coarse_entries(buf.tile_ranges[:nf].cpu().numpy(), counts, tiling)
    # the sort and ranges (the depth presort, the coarse sort and the binning) priced as the
    # metric does (CUB's 8-bit LSD passes over the 64-bit keys, then the ranges) and as this
    # build's kernels move them
    t_sort = sum(stage.get(s_, 0.0) for s_ in ("depth_sort", "tile_sort", "tile_ranges"))
    conv_b = 8 * m + 24 * m * math.ceil(tiling.end_bit() / 8) + 8 * m + 4 * tiling.nb_tiles
    impl_b = sum(algorithmic_bytes(s_, len(g), nf, nb, m, 0, 16, tiling.nb_tiles, mc)
                 for s_ in ("depth_sort", "tile_sort", "tile_ranges"))
    gbs = lambda b: b / (t_sort * 1e-3) / 1e9
    return {"workload": w.name, "keys": m, "filtered": nf, "nonempty": nb, "coarse_entries": mc,
            "forward_ms": round(float(np.median(fw)), 3),
            "backward_ms": round(float(np.median(bw)), 3), "stage_ms": stage,
            "sort_ranges_ms": round(t_sort, 4),
            "sort_ranges_convention_bytes": int(conv_b),
            # the rate a 64-bit key sort would need to finish in the same time (above the HBM
            # peak here: the binning moves far fewer bytes than a sort of the M keys)
            "sort_ranges_convention_equivalent_GBs": round(gbs(conv_b), 1),
            "sort_ranges_impl_bytes": int(impl_b), "sort_ranges_impl_GBs": round(gbs(impl_b), 1),
            "sort_ranges_impl_hbm_frac": round(gbs(impl_b) / HBM_PEAK_GBS, 4)}


def algorithmic_bytes(stage, n, nf, nb, m, npx, h, ntiles, mc=0):
    """Bytes one launch of a stage moves as this build's kernels do it (per frame averages),
    each input read once and each output written once. With at most 65535 tiles the tile lists
    come from coarse binning over mc (Gaussian, block) entries: emit counts the block ids,
    tile_sort is their one radix pass, tile_ranges the lists themselves (count, scan, write)."""
    if stage == "cull_compact":          # keep test: means + opacity in; per-block counts out
        return 16 * n
    if stage == "project":               # parameters of every Gaussian, SH of the non-empty ones;
        # fgidx, counts, record (36), depth key + value of the kept; depth and rectangle of the
        # non-empty; depth key + value slots of the culled
        return 44 * n + 12 * h * nb + (4 + 4 + 36 + 8) * nf + 20 * nb + 8 * (n - nf)
    if stage == "depth_sort" and n <= DS_MAX_SLOTS:   # the bucket presort: bucket ids counted
        # (4 per key in, 1 per slot out), the kept scattered to their buckets (4 + 1 in, 12 out
        # per kept: 64-bit key, 32-bit fgidx), each bucket sorted (12 in, the 4-byte fgidx out)
        # and the rectangles gathered into depth order (16 in + 16 out)
        return 5 * n + 5 * n + 12 * nb + 12 * nb + 4 * nb + 32 * nb
    if stage == "depth_sort":            # first pass over all N depth keys (count + scatter of the
        # kept), three more over the N_b non-empty ones: count 4, scatter 8 in + 8 out; the last
        # pass gathers each rectangle into depth order (16 in + 16 out; it also sums the count
        # scan's tiles)
        return 4 * n + 8 * n + 8 * nb + 3 * (4 + 16) * nb + 32 * nb
    if stage == "count_scan":            # one pass: the rectangles in depth order in (tiles and
        # blocks per Gaussian), the scan out
        return (16 + 4) * nb
    if stage == "emit":                  # scan, fgidx, rectangle of the non-empty in (block ids counted)
        return (8 + 4 + 16) * nb
    if stage == "tile_sort":             # the same in again; (16-bit block id, 32-bit value, 32-bit
        # block tile masks) per entry out
        return (8 + 4 + 16) * nb + 10 * mc
    if stage == "tile_ranges":           # count pass: masks in; write pass: masks + values in;
        # per-(segment, tile) counts scanned; the M list entries out
        return 4 * mc + 8 * mc + 8 * ntiles + 4 * m
    if stage == "blend":                 # metric's K5: 40 per key, 20 per pixel
        return 40 * m + 20 * npx
    return None


def measured_traffic():
    """HBM bytes per launch from the committed rocprofv3 counter summary (FETCH_SIZE +
    WRITE_SIZE, profiles/hbm_traffic.json), keyed by stage name, or {}."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        t = json.load(f)
    return {k: v.get("bytes_per_launch") for k, v in t.get("kernels", {}).items()}


# the counter-summary kernels of each survey row with their launches per frame (or step): the
# row's bytes are the sum of per-launch bytes times launches (up to DS_MAX_SLOTS Gaussians the
# depth presort is the bucket sort, three launches; above, the radix passes run their count and
# scatter kernels once per 8-bit pass, four passes over the 32-bit depth keys)
MEASURED_KERNELS = {
    "K1_project": [("keep_counts", 1), ("project", 1)],
    "K2_scan_keys": [("count_scan_apply", 1), ("emit_count", 1)],
    "K3_K4_sort_ranges": [("depth_sort_bucket_count", 1), ("depth_sort_bucket_scatter", 1), ("depth_sort_buckets", 1),
                          ("coarse_sort_scatter", 1), ("bin_count", 1), ("bin_scan", 1), ("bin_write", 1)],
    "K3_K4_sort_ranges_radix": [("depth_sort_count", 4), ("depth_sort_scatter", 4), ("coarse_sort_scatter", 1),
                                ("bin_count", 1), ("bin_scan", 1), ("bin_write", 1)],
    "K5_blend": [("blend", 1)],
    "K6_backward_blend": [("backward_blend", 1)],
    "K7_backward_project": [("backward_project", 1)],
    "K8_adam": [("adam", 1)],
    "K7_K8_fused": [("backward_project_adam", 1)],
}


def cold_stages(core, out, g, cams, tiling, opts, buf, frames, write=False):
    """Stage times with the caches flushed before every frame, outside the profiled stages:
    1 GiB (more than the 256 MB Infinity Cache and the 8 x 4 MB L2) read between frames, so
    the frame's data is not resident and the caches hold clean lines. write=True flushes by
    writing the 1 GiB instead: the caches then hold the flush's dirty lines, whose write-back
    the next kernels pay for as they evict them."""
    import torch
    flush = torch.zeros(1 << 28, dtype=torch.float32, device="cuda")
    acc = torch.zeros((), dtype=torch.float32, device="cuda")
    L = core.lib()
    core.check(L.tdgs_profile_begin(C.c_int32(16 * frames + 64)))
    for k in range(frames):
        if write:
            flush.fill_(float(k))
        else:
            acc += flush.sum()
        core.render_(out, g, cams[k % len(cams)], tiling, opts, buf, device_counts=True)
    torch.cuda.synchronize()
    ms = (C.c_double * 13)()
    cnt = (C.c_int64 * 13)()
    core.check(L.tdgs_profile_end(ms, cnt))
    del flush
    torch.cuda.empty_cache()
    return {STAGES[i]: ms[i] / cnt[i] for i in range(13) if cnt[i] > 0}


def survey_kernels(stage_ms, train_stage, n, nf, nb, m, npx, h, ntiles, end_bit, e_f, e_b, mc=0, cold_ms=None):
    """Per-kernel roofline fractions. `bytes` follow the metric's accounting (K1 = cull,
    compaction and projection: 16 N + (28 + 12h) N_f read, 8 N_f + 56 N_b written; K1_project_cold
    = the same with the caches flushed before every frame (cold_ms, cold_stages); K2 = count
    scan and key emission: 8 N_f + 24 N_b + 12 M; K3 + K4 = the sort, priced as CUB's 8-bit-digit
    LSD sort of the 64-bit keys: 8 M + 24 M ceil(end_bit / 8), and the ranges: 8 M + 4 T, whose
    results this build obtains together from the depth presort and the coarse binning (stages
    depth_sort, tile_sort, tile_ranges; reported as one row, K3_K4); K5 = blend:
    40 M + 20 P, FLOP 20 E_f + E_f exponentials; K6 = backward blend: 40 M + 20 P + 36 A with A the
    per-(tile, Gaussian) atomic flushes (<= M), FLOP 60 E_b; K7 = backward projection
    (160 + 24h) N_f; K8 = Adam 28 (11 + 3h) N_f + 4 N_f; K7_K8_fused = the trainer's fused launch,
    K7 + K8 without the 3D gradients K7 writes and K8 reads back: (160 + 24h + 28 (11 + 3h) + 4 -
    8 (11 + 3h)) N_f, 1728 B at SH3). `impl_bytes` are what this build's kernels move
    (algorithmic_bytes) and `measured_bytes` the counter summary's HBM traffic; each comes with
    its fraction of the 8 TB/s peak."""
    g3 = 11 + 3 * h
    k7, k8 = (160 + 24 * h) * nf, 28 * g3 * nf + 4 * nf
    rows = {
        "K1_project": (16 * n + (28 + 12 * h) * nf + 8 * nf + 56 * nb, ["cull_compact", "project"], stage_ms, None),
        # the same with the caches flushed before every frame (cold_stages)
        "K1_project_cold": (16 * n + (28 + 12 * h) * nf + 8 * nf + 56 * nb, ["cull_compact", "project"],
                            cold_ms or {}, None),
        "K2_scan_keys": (8 * nf + 24 * nb + 12 * m, ["count_scan", "emit"], stage_ms, None),
        "K3_K4_sort_ranges": (8 * m + 24 * m * math.ceil(end_bit / 8) + 8 * m + 4 * ntiles,
                              ["depth_sort", "tile_sort", "tile_ranges"], stage_ms, None),
        "K5_blend": (40 * m + 20 * npx, ["blend"], stage_ms, (BLEND_FLOP_PER_EVAL + BLEND_EXP_PER_EVAL) * e_f),
    }
    if train_stage:
        sep = train_stage.get("unfused", {})
        rows["K6_backward_blend"] = (40 * m + 20 * npx + 36 * m, ["backward_blend"], train_stage,
                                     BACKWARD_BLEND_FLOP_PER_EVAL * e_b)
        rows["K7_backward_project"] = (k7, ["backward_project"], sep, None)
        rows["K8_adam"] = (k8, ["adam"], sep, None)
        if "adam" not in train_stage:   # the trainer's fused launch
            rows["K7_K8_fused"] = (k7 + k8 - 2 * 4 * g3 * nf, ["backward_project"], train_stage, None)
    impl = {s_: algorithmic_bytes(s_, n, nf, nb, m, npx, h, ntiles, mc) for s_ in stage_ms}
    measured = measured_traffic()
    out = {}
    for k, (b, stages, src, flop) in rows.items():
        if not all(s_ in src for s_ in stages):
            continue
        t = sum(src[s_] for s_ in stages)
        gbs = b / (t * 1e-3) / 1e9
        row = {"stages": stages, "ms": round(t, 4), "bytes": int(b), "GBs": round(gbs, 1),
               "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        ib = [impl.get(s_) for s_ in stages]
        if all(v is not None for v in ib) and (src is stage_ms or src is cold_ms):
            row["impl_bytes"] = int(sum(ib))
            row["impl_hbm_frac"] = round(sum(ib) / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        mk = MEASURED_KERNELS.get({"K3_K4_sort_ranges": "K3_K4_sort_ranges_radix" if n > DS_MAX_SLOTS else k,
                                   "K1_project_cold": "K1_project"}.get(k, k))
        if mk and all(measured.get(x) for x, _ in mk):
            mb = sum(measured[x] * c for x, c in mk)
            row["measured_bytes"] = int(mb)
            row["measured_hbm_frac"] = round(mb / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        if flop:
            tf = flop / (t * 1e-3) / 1e12
            row.update({"flop": int(flop), "TFLOPs": round(tf, 2), "valu_frac": round(tf / FP32_PEAK_TFLOPS, 4)})
        out[k] = row
    return out


def cpu_reference_baseline(orc, g, cam, opts, repeats=5, sample_step=16):
    """The reference's own CPU renderer (render! for CPU arrays, forward_core.jl:25-177,
    restated in C++ in oracle/) on one frame of the workload, std::chrono::steady_clock, median
    of `repeats` runs after one warm-up:
    - banded: all the box's threads (up to 16), each splatting every threads-th image column of
      the full frame (identical output to one thread);
    - faithful (single thread, as the reference runs): on a bounded sample, every
      sample_step-th image column, with the per-Gaussian cull/projection/colour/depth sort in
      full; the frame time is t(per-Gaussian part) + sample_step x t(sampled columns)."""
    nproc = os.cpu_count() or 1
    threads = min(16, nproc)
    band = [orc.cpu_render_reference_timed(g, cam, opts, threads) for _ in range(repeats + 1)][1:]
    t_band = float(np.median([a + b for a, b in band]))
    single = [orc.cpu_render_reference_timed(g, cam, opts, 1, sample_step, 1) for _ in range(repeats + 1)][1:]
    t_prep = float(np.median([a for a, _ in single]))
    t_cols = float(np.median([b for _, b in single]))
    t_single = t_prep + sample_step * t_cols
    return {"value": round(1.0 / t_band, 4), "unit": "frames/s", "cores": threads, "nproc": nproc, "kind": "port",
            "sample": f"1 frame (camera 0) of the same workload with the reference CPU renderer "
                      f"(forward_core.jl:25-177) restated in C++, {threads} threads dealt image columns; "
                      f"median of {repeats} after 1 warm-up",
            "frame_s": round(t_band, 4),
            "single_thread": {"value": round(1.0 / t_single, 5), "unit": "frames/s", "cores": 1,
                              "frame_s_estimate": round(t_single, 3),
                              "per_gaussian_s": round(t_prep, 4), "sampled_columns_s": round(t_cols, 4),
                              "sample": f"one thread, every {sample_step}th image column of the same frame "
                                        f"plus the full per-Gaussian part, median of {repeats} after 1 "
                                        f"warm-up; frame = per-Gaussian + {sample_step} x sampled columns"}}


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.traffic_summary:
        print(json.dumps(traffic_summary(*args.traffic_summary), indent=1))
        return
    if args.only:
        import torch
        from tdgs_amd import core
        torch.cuda.set_device(0)
        legs = {"stress_cfg4": lambda: stress_cfg4(core), "sort_pairs": lambda: sort_pairs_bench(core),
                "train_cfg3": lambda: train_cfg3(core, args.cfg3_iterations),
                "train_cfg3_growth": lambda: train_cfg3(core, args.cfg3_iterations, grad_threshold=3.5e-5)}
        print(json.dumps({args.only: legs[args.only]()}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the path would shard "
              "by camera views or by image bands of tiles; no multi-GPU path is built)", file=sys.stderr)
        sys.exit(2)
    import torch
    from tdgs_amd import core, host, synthetic

    torch.cuda.set_device(0)
    w = synthetic.config(args.config)
    cams = w.cameras
    cam0 = cams[0]
    tiling = synthetic.tiling_for(w, cam0)
    deg = w.gaussians.sh_degree
    opts = host.RenderOptions.for_camera(cam0, deg)
    g = core.TrainableGaussiansVector.from_host(w.gaussians, 0)
    out = core.RenderOutputs.for_camera(cam0, 0, include_rgb=True, include_transmittance=True,
                                        include_depth=False, include_last_contributing_indices=False)
    buf = core.RenderBuffers(len(g), tiling, 0)
    ncam = len(cams)

    # size the key arrays on every camera the timed frames use (synchronous renders, which grow
    # them), then warm up
    used = sorted({k % ncam for k in range(args.steps)})
    for k in used:
        core.render_(out, g, cams[k], tiling, opts, buf)
    for k in range(args.warmup):
        core.render_(out, g, cams[k % ncam], tiling, opts, buf, device_counts=True)
    torch.cuda.synchronize()

    # the timed frames: nothing but render! calls (no events, no stage profiler), without host
    # synchronisation (device-side counts); the frame monitor confirms afterwards that every
    # frame's keys fit
    mon = C.POINTER(C.c_int64)()
    core.check(core.lib().tdgs_ctx_frame_monitor(core.context(0), C.byref(mon)))
    overflows0 = int(mon[2])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        core.render_(out, g, cams[k % ncam], tiling, opts, buf, device_counts=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    assert int(mon[2]) == overflows0, "a timed frame's keys did not fit the key arrays"
    wall_ms = (t1 - t0) * 1000.0 / args.steps
    fps = 1000.0 / wall_ms
    # the same frames with the counts read on the host every frame (the reference's flow)
    t0 = time.perf_counter()
    for k in range(args.steps):
        core.render_(out, g, cams[k % ncam], tiling, opts, buf)
    torch.cuda.synchronize()
    fps_sync = args.steps / (time.perf_counter() - t0)
    # per-frame times (HIP events around each frame) and stage times (the library's stage
    # profiler), each over one more pass of the cameras
    nextra = min(args.steps, ncam)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(nextra)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(nextra)]
    for k in range(nextra):
        starts[k].record()
        core.render_(out, g, cams[k % ncam], tiling, opts, buf, device_counts=True)
        ends[k].record()
    torch.cuda.synchronize()
    frame_ms = np.array([s.elapsed_time(e) for s, e in zip(starts, ends)])
    L = core.lib()
    core.check(L.tdgs_profile_begin(C.c_int32(16 * nextra + 64)))
    for k in range(nextra):
        core.render_(out, g, cams[k % ncam], tiling, opts, buf, device_counts=True)
    torch.cuda.synchronize()
    ms = (C.c_double * 13)()
    cnt = (C.c_int64 * 13)()
    core.check(L.tdgs_profile_end(ms, cnt))
    assert int(mon[2]) == overflows0, "a frame's keys did not fit the key arrays"
    cold_stage_ms = cold_stages(core, out, g, cams, tiling, opts, buf, nextra)
    cold_dirty_ms = cold_stages(core, out, g, cams, tiling, opts, buf, nextra, write=True)

    in_flight = None
    if not args.no_in_flight:
        in_flight = [render_in_flight(core, g, cams, tiling, opts, buf.key_capacity, args.steps, s) for s in (2, 3)]

    st = frame_stats(core, g, cams, tiling, opts, buf, used)
    n = len(g)
    nf, nb, m, evals, evals_live, evals_contrib, evals_back, mc = st.mean(axis=0)
    npx = cam0.width * cam0.height
    h = (deg + 1) ** 2
    stage_ms = {STAGES[i]: ms[i] / cnt[i] for i in range(13) if cnt[i] > 0}
    dom = max(stage_ms, key=stage_ms.get)
    stage_gbs = {}
    for s_, t_ in stage_ms.items():
        b = algorithmic_bytes(s_, n, nf, nb, m, npx, h, tiling.nb_tiles, mc)
        if b is not None:
            stage_gbs[s_] = b / (t_ * 1e-3) / 1e9
    b_dom = algorithmic_bytes(dom, n, nf, nb, m, npx, h, tiling.nb_tiles, mc)
    achieved = b_dom / (stage_ms[dom] * 1e-3) / 1e9
    roofline = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(dom),
                "algorithmic_bytes_per_launch": int(b_dom), "mean_launch_ms": round(stage_ms[dom], 4)}
    if dom == "blend":
        # the metric's FLOP of blending: 20 per evaluation before the early exit plus its
        # exponential; the loop as this build executes it is reported beside ("detailed")
        flop = (BLEND_FLOP_PER_EVAL + BLEND_EXP_PER_EVAL) * evals
        flop_detailed = BLEND_FLOP_EVAL * evals + BLEND_FLOP_LIVE * evals_live + BLEND_FLOP_CONTRIB * evals_contrib
        tflops = flop / (stage_ms[dom] * 1e-3) / 1e12
        if tflops / FP32_PEAK_TFLOPS > roofline["frac"]:
            roofline.update({"bound": "valu", "achieved": round(tflops, 2), "peak": FP32_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(tflops / FP32_PEAK_TFLOPS, 4),
                             "algorithmic_flop_per_launch": int(flop),
                             "flop_accounting": "20 E_f + E_f exponentials, E_f = (pixel, entry) evaluations "
                                                "before each pixel's early exit (counted by a replay)",
                             "detailed_flop_per_launch": int(flop_detailed),
                             "detailed_frac": round(flop_detailed / (stage_ms[dom] * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 4),
                             "hbm_frac": round(achieved / HBM_PEAK_GBS, 4)})

    hbm_ref = hbm_practical()

    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import build as oracle_build
        oracle_build.build(force=False)
        import oracle as orc
        cpu = cpu_reference_baseline(orc, w.gaussians, cam0, opts)

    train = None
    if args.train_steps > 0:
        its, ms_it, tstage, loss = train_bench(core, w, cams, tiling, deg, args.train_steps, args.train_warmup)
        train = {"train_it_per_s": round(its, 2), "ms_per_iteration": round(ms_it, 4), "steps": args.train_steps,
                 "stage_ms": tstage, "loss_last": round(float(loss), 6)}

    extra = None
    if not args.no_extra_configs:
        torch.cuda.empty_cache()
        extra = {"render_cfg2_tile16x32": render_other_tiling(core, w, g, (16, 32))}
        torch.cuda.empty_cache()
        extra["train_cfg2_host_images"] = train_host_images(core, w, tiling, deg)
        torch.cuda.empty_cache()
        extra["train_cfg1"] = train_cfg1(core)
        torch.cuda.empty_cache()
        extra["train_cfg3"] = train_cfg3(core, args.cfg3_iterations)
        torch.cuda.empty_cache()
        extra["train_cfg3_growth"] = train_cfg3(core, args.cfg3_iterations, grad_threshold=3.5e-5)
        torch.cuda.empty_cache()
        extra["stress_cfg4"] = stress_cfg4(core)
        torch.cuda.empty_cache()
        extra["sort_pairs_cfg4_scale"] = sort_pairs_bench(core)

    res = {
        "metric": "render fps + train it/s at 1M Gaussians 1080p SH3 (1 GPU); % HBM roofline",
        "value": round(fps, 2), "unit": "frames/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall_ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": w.name, "gaussians": n, "width": cam0.width, "height": cam0.height,
                   "sh_degree": deg, "tile": list(w.tile), "cameras": ncam, "outputs": "rgb+T"},
        "host_sync_per_frame": False,
        "frames_per_s_host_counts": round(fps_sync, 2),
        "frame_ms_p50": round(float(np.percentile(frame_ms, 50)), 4),
        "frame_ms_p99": round(float(np.percentile(frame_ms, 99)), 4),
        "frames_in_flight": in_flight,
        "mean_counts": {"filtered": round(nf), "nonempty": round(nb), "keys": round(m),
                        "blend_evaluations": round(evals), "blend_evaluations_live": round(evals_live),
                        "blend_evaluations_contributing": round(evals_contrib),
                        "backward_blend_evaluations": round(evals_back), "coarse_entries": round(mc)},
        "train": train,
        "stage_ms": {k: round(v, 4) for k, v in stage_ms.items()},
        "stage_algorithmic_GBs": {k: round(v, 1) for k, v in stage_gbs.items()},
        "roofline": roofline,
        "hbm_practical_GBs": hbm_ref,
        "survey_kernels": survey_kernels(stage_ms, train["stage_ms"] if train else None, n, nf, nb, m, npx, h,
                                         tiling.nb_tiles, tiling.end_bit(), evals, evals_back, mc,
                                         cold_ms=cold_stage_ms),
        "stage_ms_cold_cache": {k: round(v, 4) for k, v in cold_stage_ms.items()},
        "stage_ms_cold_cache_after_1GiB_write": {k: round(v, 4) for k, v in cold_dirty_ms.items()},
        "cpu_baseline": cpu,
        "extra_configs": extra,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
