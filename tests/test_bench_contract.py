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


def test_prefill_figures_are_flat_scalars_of_the_roofline():
    """The decode roofline object carries the prefill target's figures as scalar
    keys within its first 24 keys, and the nested tables come after them."""
    names = ["qkv", "o", "gate_up", "down"]
    rl = {"kernel": "k", "bound": "hbm", "achieved": 1.0, "peak": 8000.0, "unit": "GB/s",
          "frac": 0.5, "traffic": 1, "avg_launch_us": 1.0, "algorithmic_bytes_per_launch": 1,
          "launches": 1, "frac_M1": 0.6, "frac_M4": 0.5, "frac_M16": 0.4,
          "launch_floor_us": 1.5, "per_shape_GBps": {"o_M1": 1.0},
          "per_shape_us": {"o_M1": 1.0}, "traffic_source": "s"}
    rp = {"frac": 0.45, "achieved": 2250.0, "with_quant_TOPS": 2100.0,
          **{f"frac_{n}": 0.4 for n in names}}
    out = bench.flatten_prefill(rl, rp, names)
    keys = list(out)
    scalars = [k for k in keys if not isinstance(out[k], dict)]
    assert keys[:len(scalars)] == scalars
    for k in ("frac", "frac_M1", "frac_M4", "frac_M16", "prefill_frac", "prefill_achieved_TOPS",
              "prefill_with_quant_TOPS", *[f"prefill_frac_{n}" for n in names]):
        assert k in keys[:24], k
    assert out["prefill_frac"] == 0.45 and out["prefill_frac_down"] == 0.4
