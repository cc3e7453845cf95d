"""bench.py's host-side contract and accounting, on the CPU: more than one GPU is refused with
a message; every stage's algorithmic bytes are positive and grow with the counts; every kernel
the survey rows price by measured traffic has a line in the committed counter summary
(profiles/hbm_traffic.json), so no row silently loses its measured bytes."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


CFG2 = dict(n=1_000_000, nf=906_688, nb=379_884, m=6_147_727, npx=1920 * 1080, h=16, ntiles=8160, mc=690_584)


@pytest.mark.parametrize("stage", ["cull_compact", "project", "depth_sort", "count_scan", "emit", "tile_sort",
                                   "tile_ranges", "blend"])
def test_algorithmic_bytes_positive_and_monotone(stage):
    b = bench.algorithmic_bytes(stage, **CFG2)
    assert b is not None and b > 0
    bigger = dict(CFG2, nf=CFG2["nf"] + 1000, nb=CFG2["nb"] + 1000, m=CFG2["m"] + 1000, mc=CFG2["mc"] + 1000)
    assert bench.algorithmic_bytes(stage, **bigger) >= b
    assert bench.algorithmic_bytes("no_such_stage", **CFG2) is None


def test_measured_rows_have_profile_lines():
    with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
        kernels = json.load(f)["kernels"]
    for row, parts in bench.MEASURED_KERNELS.items():
        for name, launches in parts:
            assert name in kernels, (row, name)
            assert kernels[name]["bytes_per_launch"] > 0 and launches >= 1
    assert bench.traffic_from_profiles("blend") == kernels["blend"]["bytes_per_launch"]


def test_traffic_summary_scales_by_the_copy(tmp_path):
    """--traffic-summary: per-kernel means of FETCH_SIZE / WRITE_SIZE (KiB per dispatch, summed
    over a dispatch's instances) times 1 GiB over the 1 GiB copy's counter value."""
    import sqlite3

    def db(name, rows):
        p = str(tmp_path / name)
        con = sqlite3.connect(p)
        con.execute("create table pmc_events (name text, counter_name text, counter_value real, dispatch_id int)")
        con.executemany("insert into pmc_events values (?, ?, ?, ?)", rows)
        con.commit()
        con.close()
        return p

    blend = "void tdgs::k_render_tiles<true, false, false, false>(tdgs::BlendArgs)"
    other = "some_library_kernel"
    # two dispatches of the blend, the second counted by two instances
    fetch = db("f.db", [(blend, "FETCH_SIZE", 100.0, 1), (blend, "FETCH_SIZE", 150.0, 2),
                        (blend, "FETCH_SIZE", 50.0, 2), (other, "FETCH_SIZE", 7.0, 3)])
    write = db("w.db", [(blend, "WRITE_SIZE", 40.0, 1), (blend, "WRITE_SIZE", 60.0, 2)])
    gib_kib = (1 << 30) / 1024.0
    copy = "__amd_rocclr_copyBuffer"
    cf = db("cf.db", [(copy, "FETCH_SIZE", gib_kib / 2, d) for d in range(10)] + [("fill", "FETCH_SIZE", 1.0, 11)])
    cw = db("cw.db", [(copy, "WRITE_SIZE", gib_kib, d) for d in range(10)])
    s = bench.traffic_summary(fetch, write, cf, cw)
    assert s["calibration"] == {"fetch_factor": 2.0, "write_factor": 1.0}
    k = s["kernels"]
    assert set(k) == {"blend"}
    assert k["blend"]["dispatches"] == 2
    assert k["blend"]["fetch_bytes"] == int(150.0 * 1024 * 2.0)   # mean of 100 and 200 KiB, doubled
    assert k["blend"]["write_bytes"] == int(50.0 * 1024)
    assert k["blend"]["bytes_per_launch"] == k["blend"]["fetch_bytes"] + k["blend"]["write_bytes"]
