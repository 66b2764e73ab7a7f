"""The benchmark / lockstep-verify harness on the CPU: pure helpers against
the reference harness's rules (bench/harness.py), artifact and mismatch
bundle formats, and verify runs between two oracle-backed backends -- one
with a planted register fault -- including replay of a bundle's actions."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from gbxcule_amd import harness as H
from gbxcule_amd.carts.synth import CARTS

from ._oracle_backend import OracleBackend


@pytest.fixture(scope="module")
def rom_file(tmp_path_factory):
    p = tmp_path_factory.mktemp("roms") / "c3.gb"
    p.write_bytes(CARTS["c3"]())
    return p


def test_generate_actions():
    a = H.generate_actions(5, 16, 7, "seeded_random", 8)
    assert np.array_equal(a, np.random.default_rng(12).integers(0, 8, 16, dtype=np.int32))
    assert a.dtype == np.int32
    assert not H.generate_actions(0, 4, None, "noop", 8).any()
    names = ["NOOP", "A", "B", "START", "UP", "DOWN", "LEFT", "RIGHT"]
    assert H.generate_actions(0, 6, None, "striped", 8, names).tolist() == [4, 5, 6, 7, 4, 5]
    assert H.generate_actions(0, 5, None, "striped", 6).tolist() == [0, 1, 2, 3, 0]
    assert H.get_action_gen_metadata("striped", None, action_names=names, num_actions=8)[
        "pattern_action_names"] == ["UP", "DOWN", "LEFT", "RIGHT"]  # fmt: skip
    with pytest.raises(ValueError):
        H.generate_actions(0, 4, None, "seeded_random", 8)
    with pytest.raises(ValueError):
        H.generate_actions(0, 4, 1, "bogus", 8)
    sched = H.get_action_schedule_metadata(24, 8)
    assert sched["tick_split"] == [23, 1]


def test_state_normalize_and_diff():
    st = {"pc": 0x150, "sp": 0xFFFE, "a": 1, "f": 0xB0, "b": 2, "c": 3, "d": 4, "e": 5, "h": 6,
          "l": 7, "flags": {"z": 1, "n": 0, "h": 1, "c": 1}, "instr_count": 10}  # fmt: skip
    n = H.normalize_cpu_state(st)
    assert list(n)[:10] == list(H.CANONICAL_REGISTER_KEYS)
    assert n["cycle_count"] is None and n["trap_kind"] is None
    assert H.diff_states(n, dict(n)) is None
    m = dict(n, a=9, flags=dict(n["flags"], z=0), instr_count=11)
    d = H.diff_states(n, m)
    assert d == {"a": {"ref": 1, "dut": 9}, "flags": {"z": {"ref": 1, "dut": 0}},
                 "instr_count": {"ref": 10, "dut": 11}}  # fmt: skip
    # counters compared only when both sides report them
    assert H.diff_states(n, dict(n, cycle_count=5)) is None


def test_mem_regions_and_hash():
    assert H.parse_mem_region("C000:C100") == (0xC000, 0xC100)
    assert H.parse_mem_region("0xff80:0x10000") == (0xFF80, 0x10000)
    for bad in ("C000", "C100:C000", ":10", "0:10001"):
        with pytest.raises(ValueError):
            H.parse_mem_region(bad)
    assert H.hash_memory(b"abc") == __import__("hashlib").blake2b(b"abc", digest_size=16).hexdigest()


def test_artifact_and_trace(tmp_path):
    p = H.write_artifact(tmp_path / "runs", run_id="r1", system_info={"x": 1},
                         config={"c": 2}, results={"total_sps": 3.0})  # fmt: skip
    art = json.loads(p.read_text())
    assert art["schema_version"] == 1 and art["run_id"] == "r1" and art["results"]["total_sps"] == 3.0
    assert set(art) == {"schema_version", "run_id", "timestamp_utc", "system", "config", "results"}
    assert [x.name for x in p.parent.iterdir()] == ["r1.json"]  # no temp files left
    H.write_actions_trace([[1, 2], [3, 4]], tmp_path / "a.jsonl")
    back = H.load_actions_trace(tmp_path / "a.jsonl")
    assert [x.tolist() for x in back] == [[1, 2], [3, 4]]
    (tmp_path / "bad.jsonl").write_text("[1]\nnot json\n")
    with pytest.raises(ValueError, match="line 2"):
        H.load_actions_trace(tmp_path / "bad.jsonl")


def _verify(rom_file, tmp_path, plant=None, **kw):
    ref = OracleBackend(rom_file, frames_per_step=1, render_bg=True)
    dut = OracleBackend(rom_file, frames_per_step=1, render_bg=True, plant=plant)
    try:
        return H.run_verify(ref, dut, rom_path=rom_file, ref_name="oracle", dut_name="oracle_planted",
                            frames_per_step=1, output_dir=tmp_path, log=lambda s: None, **kw)  # fmt: skip
    finally:
        ref.close()
        dut.close()


def test_verify_pass(rom_file, tmp_path):
    rc, bundle = _verify(rom_file, tmp_path, verify_steps=40, mem_regions=[(0xC000, 0xC100)],
                         compare_frame=True)  # fmt: skip
    assert (rc, bundle) == (0, None)
    assert not (tmp_path / "mismatch").exists()


def test_verify_mismatch_bundle_and_replay(rom_file, tmp_path):
    rc, bundle = _verify(rom_file, tmp_path, plant=(12, "a"), verify_steps=40, compare_every=2,
                         mem_regions=[(0xC000, 0xC040), (0x8000, 0xA000)], compare_frame=True)  # fmt: skip
    assert rc == 1
    meta = json.loads((bundle / "metadata.json").read_text())
    assert meta["schema_version"] == 2 and meta["mismatch_step"] == 12
    assert meta["ref_backend"] == "oracle" and meta["dut_backend"] == "oracle_planted"
    assert meta["mem_hash_version"] == "blake2b-128-v1"
    assert meta["rom_sha256"] == H.compute_rom_sha256(rom_file)
    diff = json.loads((bundle / "diff.json").read_text())
    assert diff["a"]["ref"] ^ diff["a"]["dut"] == 1
    assert "ppu_regs" in diff and "LCDC" in diff["ppu_regs"]["ref"]
    ref_state = json.loads((bundle / "ref_state.json").read_text())
    assert ref_state["a"] == diff["a"]["ref"]
    assert len((bundle / "actions.jsonl").read_text().splitlines()) == 13
    assert (bundle / "rom.gb").read_bytes() == rom_file.read_bytes()
    assert os.access(bundle / "repro.sh", os.X_OK)
    script = (bundle / "repro.sh").read_text()
    assert "--verify" in script and "--mem-region C000:C040" in script and "--compare-frame" in script
    assert (bundle / "oam_ref_FE00_FEA0.bin").stat().st_size == 160
    assert (bundle / "vram_ref_8000_8400.bin").stat().st_size == 1024  # truncated dump
    assert (bundle / "ref_cart_state.json").exists()
    # replaying the bundle's actions reproduces the same mismatch step
    replay = H.load_actions_trace(bundle / "actions.jsonl")
    rc2, b2 = _verify(rom_file, tmp_path / "again", plant=(12, "a"), verify_steps=40,
                      compare_every=2, replay_actions=replay)  # fmt: skip
    assert rc2 == 1 and json.loads((b2 / "metadata.json").read_text())["mismatch_step"] == 12


def test_cli_verify_with_registered_backends(rom_file, tmp_path):
    H.register_backend("oracle_cli", lambda rom, **kw: OracleBackend(rom, **kw))
    H.register_backend("oracle_cli_bad", lambda rom, **kw: OracleBackend(rom, plant=(3, "b"), **kw))
    args = ["--rom", str(rom_file), "--verify", "--ref-backend", "oracle_cli", "--verify-steps", "8",
            "--frames-per-step", "1", "--output-dir", str(tmp_path)]  # fmt: skip
    assert H.main(args + ["--dut-backend", "oracle_cli"]) == 0
    assert H.main(args + ["--dut-backend", "oracle_cli_bad"]) == 1
    (bundle,) = (tmp_path / "mismatch").iterdir()
    assert json.loads((bundle / "metadata.json").read_text())["mismatch_step"] == 3
    with pytest.raises(ValueError, match="Unknown backend"):
        H.create_backend("nope", str(rom_file))
