"""bench.py's host side on the CPU: the one-GPU refusal, the device-source
digest and the counter file the roofline's traffic comes from."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU only" in r.stdout + r.stderr


def test_source_digest_covers_every_device_source(tmp_path, monkeypatch):
    d = bench.csrc_digest()
    assert len(d) == 16 and int(d, 16) >= 0
    assert bench.csrc_digest() == d
    # the same recipe over a copy, then one byte changed in one file: another digest
    src = tmp_path / "fleet-mi300x_amd" / "csrc"
    src.mkdir(parents=True)
    (tmp_path / "include").mkdir()
    for f in sorted((ROOT / "fleet-mi300x_amd" / "csrc").iterdir()):
        if f.is_file():
            (src / f.name).write_bytes(f.read_bytes())
    (tmp_path / "include" / "fleet_moe.h").write_bytes((ROOT / "include" / "fleet_moe.h").read_bytes())
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    assert bench.csrc_digest() == d
    target = src / "moe_common.h"
    target.write_bytes(target.read_bytes() + b"\n")
    assert bench.csrc_digest() != d


def test_counter_file_has_the_roofline_rows():
    data = bench.load_counter_file()
    assert len(data.get("csrc_sha16", "")) == 16
    kernels = data["kernels"]
    for name in ("moe_layer", "moe_layer_cold", "attention", "lm_head", "dense", "column",
                 "grouped_T4", "grouped_T16", "grouped_T64"):
        row = kernels[name]
        assert row["hbm_bytes"] > 0 and row["algorithmic_bytes"] > 0 and row["us"] > 0
        ratio = row["hbm_bytes"] / row["algorithmic_bytes"]
        assert row["traffic_over_algorithmic"] == pytest.approx(ratio, rel=1e-3)
        assert 0.99 < ratio < 1.5, (name, ratio)
    # config 1's algorithmic bytes: six routed experts and the shared expert
    h, i, si = 2048, 1408, 2816
    assert kernels["moe_layer"]["algorithmic_bytes"] == 6 * 3 * h * i * 2 + 3 * h * si * 2
    src = bench.counters_source()
    assert src["measured_csrc_sha16"] == data["csrc_sha16"]
    assert src["matches_current_sources"] == (data["csrc_sha16"] == bench.csrc_digest())


def test_counter_view_divides_profiled_bytes_by_this_runs_time():
    profiled = {"moe_layer": {"hbm_bytes": 142_000_000, "traffic_over_algorithmic": 1.026}}
    v = bench.counter_view({"roofline": {"kernel_us_mean": 28.4}}, profiled)
    e = v["moe_layer"]
    assert e["counter_gbs"] == pytest.approx(142e6 / 28.4e-6 / 1e9, rel=1e-3)
    assert e["counter_frac"] == pytest.approx(e["counter_gbs"] / bench.HBM_PEAK_GBS, rel=1e-3)
    assert "attention" not in v                    # no time for it in this result

