"""The committed inputs bench.py reads at run time: the HBM traffic summary
under profiles/ carries every key the roofline section uses, and its figure is
consistent with the per-kernel rows it summarises."""
import json
import os

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_traffic_summary_has_the_keys_bench_reads():
    tr = bench.load_traffic(ROOT)
    assert tr is not None, "profiles/decode_linear_hbm_traffic.json is missing or unreadable"
    for key in ("hbm_bytes_per_launch", "source", "fetch_bytes_per_launch",
                "write_bytes_per_launch", "linear_calls", "per_kernel"):
        assert key in tr, key
    # each total is truncated to whole bytes on its own
    assert abs(tr["hbm_bytes_per_launch"]
               - (tr["fetch_bytes_per_launch"] + tr["write_bytes_per_launch"])) <= 1


def test_traffic_summary_matches_its_per_kernel_rows():
    with open(os.path.join(ROOT, "profiles", "decode_linear_hbm_traffic.json")) as f:
        tr = json.load(f)
    fetch = sum(k["dispatches"] * k["fetch_bytes_per_dispatch"] for k in tr["per_kernel"])
    write = sum(k["dispatches"] * k["write_bytes_per_dispatch"] for k in tr["per_kernel"])
    n = tr["linear_calls"]
    # per-kernel rows are rounded down per dispatch: agree to a few bytes per call
    assert abs(fetch / n - tr["fetch_bytes_per_launch"]) < 64
    assert abs(write / n - tr["write_bytes_per_launch"]) < 64
