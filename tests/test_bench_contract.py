"""bench.py's output contract, checked on the CPU (no GPU work).

The driver parses one JSON line from `python bench.py`; these tests pin the
pieces that do not need a device: the single-GPU refusal, the roofline
object's arithmetic and units, and the CPU-baseline helpers' fields."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


@pytest.mark.parametrize("bound,peak_key,unit", [("mfma", "bf16", "TFLOP/s"), ("mfma", "int8", "TOP/s"),
                                                 ("mfma", "fp32", "TFLOP/s"), ("hbm", "hbm", "GB/s")])
def test_roofline_fields(bound, peak_key, unit):
    work, ms = 1.0995e12, 0.75
    r = bench.roofline(bound, work, ms, peak_key, "no_such_workload")
    assert set(r) >= {"bound", "achieved", "peak", "unit", "frac", "traffic"}
    assert r["bound"] == bound and r["unit"] == unit
    scale = 1e9 if bound == "hbm" else 1e12
    assert r["achieved"] == pytest.approx(work / (ms * 1e-3) / scale, rel=1e-4)
    assert r["peak"] == bench.PEAK[peak_key]
    assert r["frac"] == pytest.approx(r["achieved"] / r["peak"], abs=1e-4)
    assert r["traffic"] is None and r["traffic_source"] is None


def test_peaks_are_the_published_dense_figures():
    assert bench.PEAK == {"bf16": 2500.0, "int8": 5000.0, "fp32": 157.3, "hbm": 8000.0}


def test_committed_traffic_figures_are_per_launch_bytes():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    data = json.load(open(path))
    names = [k for k in data if not k.startswith("_")]
    assert {"gemm_bf16_8192", "gemm_int8_dequant", "rmsnorm", "layernorm", "attention"} <= set(names)
    for name in names:
        b = bench.traffic_from_profiles(name)
        assert b == data[name]["bytes_per_launch"] and b > 0
    # the streaming kernels move their algorithmic bytes (268 MB in, 268 MB out)
    for name in ("rmsnorm", "softmax", "gelu"):
        assert bench.traffic_from_profiles(name) == pytest.approx(536.9e6, rel=0.01)


def test_host_fields():
    d = bench.with_host({"value": 1.0})
    assert d["cpu_model"] and d["host_cpus"] >= 1
    assert 1 <= bench.cpu_threads() <= (os.cpu_count() or 1)


@pytest.mark.parametrize("layer", [False, True])
def test_norm_cpu_baseline_runs_every_row_it_is_given(layer):
    from grxcp_amd import synth
    rows, hidden = 64, 256
    x = synth.normal_bf16(rows * hidden, 7)
    g = synth.normal_bf16(hidden, 8, 1.0, 0.02)
    b = synth.normal_bf16(hidden, 9, 0.0, 0.02)
    d = bench.cpu_norm_baseline(x, g, b, rows, hidden, layer)
    assert d["value"] > 0 and d["unit"] == "GB/s" and d["kind"] == "port"
    assert d["sample"].startswith(f"{rows} of {rows} rows")
