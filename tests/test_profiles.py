"""CPU: the committed HBM-traffic records bench.py reads, and bench.py's one-GPU contract.

bench.py copies `hbm_bytes_per_launch` of profiles/traffic_<workload>[_scores_only].json
into its line's `roofline.traffic`.  Each record must say which kernel and source
commit its counters come from, and its byte figure must follow from its own
counters: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) times their calibration
factors (measured on a copy kernel of known size, 2 and 1 to within 1e-5).
"""
import glob
import json
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RECORDS = sorted(glob.glob(os.path.join(ROOT, "profiles", "traffic_*.json")))
WORKLOADS = {"c2", "c3", "c3d768", "c3f32", "c3bwd", "c4", "c4d1024", "c4mq", "c5"}


def test_records_exist_for_the_headline_workloads():
    names = {os.path.basename(p) for p in RECORDS}
    for w in ("c2", "c2_scores_only", "c3", "c3_scores_only", "c5"):
        assert f"traffic_{w}.json" in names


@pytest.mark.parametrize("path", RECORDS, ids=[os.path.basename(p) for p in RECORDS])
def test_record_is_self_consistent(path):
    with open(path) as f:
        t = json.load(f)
    name = os.path.basename(path)[len("traffic_"):-len(".json")]
    assert t["workload"] in WORKLOADS
    assert name in (t["workload"], t["workload"] + "_scores_only")
    assert t["kernel"]
    assert re.fullmatch(r"[0-9a-f]{7,40}", t["commit"])
    assert abs(t["fetch_scale"] - 2.0) < 1e-5 and abs(t["write_scale"] - 1.0) < 1e-5
    counted = 1024 * (t["fetch_size_kib_per_dispatch"] * t["fetch_scale"]
                      + t["write_size_kib_per_dispatch"] * t["write_scale"])
    # Older records applied the calibration's exact factor (8 GiB read / 4,194,319 KiB).
    assert abs(t["hbm_bytes_per_launch"] - counted) <= 1e-4 * counted
    assert t["algorithmic_bytes_per_launch"] > 0


def test_scores_only_records_move_fewer_bytes():
    for w in ("c2", "c3", "c4mq"):
        with open(os.path.join(ROOT, "profiles", f"traffic_{w}.json")) as f:
            tape = json.load(f)
        with open(os.path.join(ROOT, "profiles", f"traffic_{w}_scores_only.json")) as f:
            so = json.load(f)
        assert so["write_size_kib_per_dispatch"] < tape["write_size_kib_per_dispatch"]
        assert so["hbm_bytes_per_launch"] < tape["hbm_bytes_per_launch"]


def test_bench_refuses_more_than_one_gpu():
    """One GPU per box: --gpus 2 prints one JSON line saying so and exits 2, before
    anything touches a device."""
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]
