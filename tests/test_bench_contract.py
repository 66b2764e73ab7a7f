"""bench.py's output contract on the CPU: the single-GPU refusal, the
committed profile summaries behind every timed workload's roofline and VALU
objects, and the arithmetic of those objects."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

# every (profile key, envs, frameskip) the default run times: the headline
# and the workloads timed beside it
TIMED = [("c2", 16_384, 24)] + [(key, n, fs) for _, key, n, fs, _, _ in bench.EXTRA]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, cwd=ROOT, timeout=300)  # fmt: skip
    assert r.returncode == 2
    assert "--gpus must be 1" in r.stderr
    assert r.stdout.strip() == ""  # no JSON line


@pytest.mark.parametrize("key,n,fs", TIMED)
def test_timed_workloads_have_profile_summaries(key, n, fs):
    prof = bench.profile_file(key, n, fs)
    assert prof is not None, f"no traffic summary for {key} at {n} envs, frameskip {fs}"
    assert prof["num_envs"] == n and prof["frameskip"] == fs
    # HBM traffic per launch: FETCH_SIZE and WRITE_SIZE (KiB) scaled by the
    # copy calibration of the same runs
    want = prof["fetch_kib"] * 1024 * prof["fetch_scale"] + prof["write_kib"] * 1024 * prof["write_scale"]
    assert prof["bytes_per_launch"] == pytest.approx(want, rel=1e-6)
    assert 0.0 < prof["active_lane_frac"] <= 1.0 and 0.0 < prof["valu_busy"] <= 1.0
    assert prof["valu_peak_lane_ops_per_s"] == pytest.approx(256 * 64 * 2.4e9)
    src = ROOT / prof["source"]
    assert src.exists(), src
    # the summary it came from names the same workload shape and the counters
    text = src.read_text()
    assert f"{n:,}" in text and "FETCH_SIZE" in text and "WRITE_SIZE" in text


def test_roofline_and_valu_objects():
    res = {"num_envs": 131_072, "frameskip": 24, "step_kernel_ms": 2.0}
    data_b = 10_000.0
    r = bench.roofline("c5", res, data_b, 1.0)
    bytes_per_env_step = bench.STATE_BYTES + data_b
    assert r["bytes_per_env_step"] == bytes_per_env_step
    assert r["achieved"] == pytest.approx(131_072 * bytes_per_env_step / 2.0e-3 / 1e9)
    assert r["frac"] == pytest.approx(r["achieved"] / bench.HBM_PEAK_GBS)
    assert r["peak"] == 8000.0 and r["unit"] == "GB/s" and r["bound"] == "hbm"
    prof = json.loads((ROOT / "profiles" / "traffic_c5_131072.json").read_text())
    assert r["traffic"] == prof["bytes_per_launch"]
    v = bench.valu_object("c5", res)
    assert v["achieved"] == pytest.approx(prof["valu_wave_insts_per_launch"] * 64 / 2.0e-3)
    assert v["frac"] == pytest.approx(v["achieved"] / v["peak"])
    # a shape without a summary: no traffic, no VALU object
    other = {"num_envs": 1_000, "frameskip": 24, "step_kernel_ms": 1.0}
    assert bench.roofline("c5", other, data_b, 1.0)["traffic"] is None
    assert bench.valu_object("c5", other) is None
