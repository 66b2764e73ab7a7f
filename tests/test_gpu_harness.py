"""Lockstep verify of the HIP backend against the oracle through the harness
(the reference's ``--verify`` flow), and the benchmark mode's artifact."""

from __future__ import annotations

import json

import pytest

from gbxcule_amd import harness as H
from gbxcule_amd.carts.synth import CARTS

from ._oracle_backend import OracleBackend
from .conftest import require_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cart,fs,steps", [("c3", 1, 60), ("c4m3", 4, 30), ("c1", 2, 40)])
def test_verify_hip_against_oracle(tmp_path, bootstub, cart, fs, steps):
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    rom = tmp_path / f"{cart}.gb"
    rom.write_bytes(CARTS[cart]())
    ref = OracleBackend(rom, frames_per_step=fs, render_bg=True)
    dut = HipVecBackend(str(rom), num_envs=1, frames_per_step=fs, stage="emulate_only",
                        render_bg=True, bootrom=bootstub)  # fmt: skip
    try:
        rc, bundle = H.run_verify(
            ref, dut, rom_path=rom, ref_name="oracle", dut_name="hip_vec", verify_steps=steps,
            frames_per_step=fs, mem_regions=[(0xC000, 0xE000), (0xFF00, 0x10000), (0x8000, 0xA000)],
            compare_frame=True, output_dir=tmp_path, log=lambda s: None,
        )  # fmt: skip
        assert rc == 0, f"mismatch bundle at {bundle}"
    finally:
        ref.close()
        dut.close()


def test_benchmark_artifact(tmp_path):
    require_gpu()
    rom = tmp_path / "c2.gb"
    rom.write_bytes(CARTS["c2"]())
    rc = H.main(["--rom", str(rom), "--backend", "hip_vec", "--num-envs", "256", "--steps", "4",
                 "--warmup-steps", "2", "--action-gen", "seeded_random", "--actions-seed", "100",
                 "--output-dir", str(tmp_path / "runs")])  # fmt: skip
    assert rc == 0
    (art,) = list((tmp_path / "runs").rglob("*.json"))
    a = json.loads(art.read_text())
    assert a["schema_version"] == 1
    r = a["results"]
    assert r["measured_steps"] == 4 and r["num_envs"] == 256 and r["total_sps"] > 0
    assert r["frames_per_sec"] == pytest.approx(r["total_sps"] * 24)
    assert a["config"]["action_generator"]["name"] == "seeded_random"
    assert a["config"]["sync_every"] == 64
    assert 1 <= r["divergence"]["unique_pc_count"] <= 256
