"""Benchmark of the render core on one MI355X: BASELINE.json's headline metric.

Workload: 1,000,000 Gaussians, 1920x1080, SH degree 3, 120
seeded orbit cameras, 16x16 tiles; synthetic seeded data. A step renders one camera (frame
k uses camera k mod 120) with the full render! pipeline: cull, compaction, projection,
duplication, sort, ranges and blending, including its host synchronisation.

Prints one JSON line. `value` is frames/s over the timed steps; `roofline` describes the
stage that takes the most time, with its algorithmic bytes (or FLOP) per launch divided by
its mean duration measured live with HIP events on the rendering stream; `cpu_baseline`
times the reference's own CPU renderer (render! for CPU arrays, forward_core.jl:25-177,
restated in C++ in oracle/) on one frame of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
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

STAGES = ["cull_compact", "project", "depth_sort", "count_scan", "emit", "tile_sort", "tile_ranges",
          "blend", "backward_blend", "backward_project", "adam", "adc", "loss"]


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=600)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", type=int, default=2)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-threads", type=int, default=0)
    return p.parse_args()


def frame_stats(core, g, cams, tiling, opts, outputs, buffers, idx):
    """N_f, N_b, M for the given cameras (untimed pass)."""
    import torch
    st = []
    for k in idx:
        core.render_(outputs, g, cams[k], tiling, opts, buffers)
        nf = buffers.nb_fgaussians
        nb = int((buffers.counts[:nf] > 0).sum().item())
        st.append((nf, nb, buffers.nb_keys))
    torch.cuda.synchronize()
    return np.array(st, dtype=np.float64)


def algorithmic_bytes(stage, n, nf, nb, m, npx, h, ntiles):
    """Bytes one launch of a stage must move (per frame averages)."""
    if stage == "cull_compact":
        return 16 * n + 2 * n + 4 * nf
    if stage == "project":
        return (4 + 16 + 12 + 16 + 4) * nf + 8 * n + (56 + 12 * h) * nb
    if stage == "depth_sort":
        return 4 * 16 * n
    if stage == "count_scan":
        return 12 * n
    if stage == "emit":
        return 32 * nb + 12 * m
    if stage == "tile_sort":
        return 2 * 24 * m
    if stage == "tile_ranges":
        return 8 * m + 4 * ntiles
    if stage == "blend":
        return 40 * m + 16 * npx
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the path shards by "
              "views or image bands, see DESIGN.md)", file=sys.stderr)
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

    for k in range(args.warmup):
        core.render_(out, g, cams[k % ncam], tiling, opts, buf)
    torch.cuda.synchronize()

    L = core.lib()
    core.check(L.tdgs_profile_begin(C.c_int32(16 * args.steps + 64)))
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        starts[k].record()
        core.render_(out, g, cams[k % ncam], tiling, opts, buf)
        ends[k].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (C.c_double * 13)()
    cnt = (C.c_int64 * 13)()
    core.check(L.tdgs_profile_end(ms, cnt))
    frame_ms = np.array([s.elapsed_time(e) for s, e in zip(starts, ends)])
    wall_ms = (t1 - t0) * 1000.0 / args.steps
    fps = 1000.0 / wall_ms

    used = sorted({k % ncam for k in range(args.steps)})
    st = frame_stats(core, g, cams, tiling, opts, out, buf, used)
    n = len(g)
    nf, nb, m = st.mean(axis=0)
    npx = cam0.width * cam0.height
    h = (deg + 1) ** 2
    stage_ms = {STAGES[i]: ms[i] / cnt[i] for i in range(13) if cnt[i] > 0}
    dom = max(stage_ms, key=stage_ms.get)
    stage_gbs = {}
    for s_, t_ in stage_ms.items():
        b = algorithmic_bytes(s_, n, nf, nb, m, npx, h, tiling.nb_tiles)
        if b is not None:
            stage_gbs[s_] = b / (t_ * 1e-3) / 1e9
    b_dom = algorithmic_bytes(dom, n, nf, nb, m, npx, h, tiling.nb_tiles)
    achieved = b_dom / (stage_ms[dom] * 1e-3) / 1e9
    roofline = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "algorithmic_bytes_per_launch": int(b_dom), "mean_launch_ms": round(stage_ms[dom], 4)}

    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import build as oracle_build
        oracle_build.build(force=False)
        import oracle as orc
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        c0 = time.perf_counter()
        orc.cpu_render_reference(w.gaussians, cam0, opts, threads=threads)
        c1 = time.perf_counter()
        cpu = {"value": round(1.0 / (c1 - c0), 4), "unit": "frames/s", "cores": threads, "kind": "port",
               "sample": f"1 frame (camera 0) of the same workload with the reference CPU renderer "
                         f"(forward_core.jl:25-177) restated in C++, {threads} threads by image columns"}

    res = {
        "metric": "render fps + train it/s at 1M Gaussians 1080p SH3 (1 GPU); % HBM roofline",
        "value": round(fps, 2), "unit": "frames/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall_ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": w.name, "gaussians": n, "width": cam0.width, "height": cam0.height,
                   "sh_degree": deg, "tile": list(w.tile), "cameras": ncam, "outputs": "rgb+T"},
        "frame_ms_p50": round(float(np.percentile(frame_ms, 50)), 4),
        "frame_ms_p99": round(float(np.percentile(frame_ms, 99)), 4),
        "mean_counts": {"filtered": round(nf), "nonempty": round(nb), "keys": round(m)},
        "stage_ms": {k: round(v, 4) for k, v in stage_ms.items()},
        "stage_algorithmic_GBs": {k: round(v, 1) for k, v in stage_gbs.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
