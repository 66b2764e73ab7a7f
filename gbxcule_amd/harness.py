"""Benchmark and lockstep-verify harness over the gbxcule backend protocol.

Restates the reference's ``bench/harness.py`` for this build: the same action
generators (``generate_actions``, :205-249), canonical CPU-state
normalisation and diff (:516-611), memory-region hashing (blake2b-128),
benchmark timing (:808-889), the version-1 run artifact written atomically
(:938-998; schema in ``ARCHITECTURE.md`` 8.3) and the version-2 mismatch
bundle (``metadata.json``, ``ref_state.json``, ``dut_state.json``,
``diff.json``, ``actions.jsonl``, memory / PPU dumps, the ROM and a
``repro.sh``; :1562-1790).

Backends are looked up by name in ``BACKEND_REGISTRY``; ``hip_vec`` (the
MI355X backend) is registered here and callers register their own reference
backends (PyBoy, a CPU emulator) with ``register_backend``.  ``run_verify``
also accepts backend objects directly.  Any object with the ``VecBackend``
surface works: ``reset``, ``step``, ``get_cpu_state``, and optionally
``read_memory``, ``get_cart_state``, ``read_frame_bg_shade_env0``,
``get_pc_snapshot``, ``close``.

Run ``python -m gbxcule_amd.harness --help``.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import platform
import shutil
import sys
import time
import uuid
from collections.abc import Callable, Mapping
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import numpy as np

from .abi import ACTION_CODEC_ID, ACTION_NAMES, NUM_ACTIONS

RESULT_SCHEMA_VERSION = 1
MISMATCH_SCHEMA_VERSION = 2
ACTION_GEN_VERSION = "1.0"
MEM_HASH_VERSION = "blake2b-128-v1"
MAX_MEM_DUMP_BYTES = 1024
FRAME_HASH_HISTORY_LEN = 4
PPU_DUMP_REGIONS = (("oam", 0xFE00, 0xFEA0), ("vram", 0x8000, 0xA000))
CANONICAL_REGISTER_KEYS = ("pc", "sp", "a", "f", "b", "c", "d", "e", "h", "l")
CANONICAL_FLAG_KEYS = ("z", "n", "h", "c")
CANONICAL_TRAP_KEYS = ("trap_flag", "trap_pc", "trap_opcode", "trap_kind")
PPU_REGS = (("LCDC", 0xFF40), ("STAT", 0xFF41), ("SCY", 0xFF42), ("SCX", 0xFF43),
            ("LY", 0xFF44), ("LYC", 0xFF45), ("WY", 0xFF4A), ("WX", 0xFF4B),
            ("BGP", 0xFF47), ("OBP0", 0xFF48), ("OBP1", 0xFF49), ("IF", 0xFF0F))  # fmt: skip


def _utc_now() -> datetime:
    return datetime.now(timezone.utc)


# -- backends ------------------------------------------------------------------
def _make_hip_vec(rom_path: str, **kw: Any) -> Any:
    from .backend import HipVecBackend

    return HipVecBackend(rom_path, **kw)


BACKEND_REGISTRY: dict[str, Callable[..., Any]] = {"hip_vec": _make_hip_vec}


def register_backend(name: str, factory: Callable[..., Any]) -> None:
    """``factory(rom_path, **create_backend keywords)`` -> backend."""
    BACKEND_REGISTRY[name] = factory


def create_backend(
    name: str,
    rom_path: str,
    *,
    num_envs: int = 1,
    frames_per_step: int = 24,
    release_after_frames: int = 8,
    stage: str = "emulate_only",
    obs_dim: int = 32,
    base_seed: int | None = None,
    action_codec: str = ACTION_CODEC_ID,
    render_bg: bool = False,
) -> Any:
    if name not in BACKEND_REGISTRY:
        raise ValueError(f"Unknown backend: {name}. Available: {list(BACKEND_REGISTRY)}")
    return BACKEND_REGISTRY[name](
        rom_path, num_envs=num_envs, frames_per_step=frames_per_step,
        release_after_frames=release_after_frames, stage=stage, obs_dim=obs_dim,
        base_seed=base_seed, action_codec=action_codec, render_bg=render_bg,
    )  # fmt: skip


# -- actions ---------------------------------------------------------------------
def _striped_pattern(action_names: list[str] | None, num_actions: int) -> np.ndarray:
    """UP, DOWN, LEFT, RIGHT when the codec names them, else the first four
    non-NOOP actions (harness.py:170-202)."""
    if num_actions < 4:
        raise ValueError("striped generator requires at least 4 actions")
    names = [str(n).upper() for n in action_names] if action_names else None
    if names and all(t in names for t in ("UP", "DOWN", "LEFT", "RIGHT")):
        return np.array([names.index(t) for t in ("UP", "DOWN", "LEFT", "RIGHT")], np.int32)
    cand = [i for i, n in enumerate(names) if n not in {"NOOP", "NO-OP", "NONE"}] if names else []
    if len(cand) < 4:
        cand = list(range(num_actions))
    return np.array(cand[:4], dtype=np.int32)


def generate_actions(
    step_idx: int,
    num_envs: int,
    seed: int | None,
    gen_name: str,
    num_actions: int,
    action_names: list[str] | None = None,
) -> np.ndarray:
    """int32 actions of one step: ``noop``; ``seeded_random`` =
    ``default_rng(seed + step_idx).integers(0, num_actions, num_envs)``;
    ``striped`` = a 4-action pattern by env index."""
    if num_actions < 1:
        raise ValueError("num_actions must be >= 1")
    if gen_name == "noop":
        return np.zeros((num_envs,), dtype=np.int32)
    if gen_name == "seeded_random":
        if seed is None:
            raise ValueError("seeded_random generator requires a seed")
        rng = np.random.default_rng(seed + step_idx)
        return rng.integers(0, num_actions, size=(num_envs,), dtype=np.int32)
    if gen_name == "striped":
        pat = _striped_pattern(action_names, num_actions)
        return pat[np.arange(num_envs) % len(pat)].astype(np.int32)
    raise ValueError(f"Unknown action generator: {gen_name}")


def get_action_gen_metadata(gen_name: str, seed: int | None, *, action_names=None,
                            num_actions: int | None = None) -> dict[str, Any]:  # fmt: skip
    meta: dict[str, Any] = {"name": gen_name, "version": ACTION_GEN_VERSION, "seed": seed}
    if gen_name == "striped":
        if num_actions is None:
            raise ValueError("striped metadata requires num_actions")
        pat = _striped_pattern(action_names, num_actions).tolist()
        meta["pattern"] = pat
        if action_names:
            meta["pattern_action_names"] = [action_names[i] for i in pat]
    return meta


def get_action_codec_metadata(codec_id: str = ACTION_CODEC_ID) -> dict[str, Any]:
    if codec_id != ACTION_CODEC_ID:
        raise ValueError(f"Unknown action codec: {codec_id}")
    return {"id": codec_id, "name": codec_id, "version": "1", "num_actions": NUM_ACTIONS,
            "action_names": list(ACTION_NAMES)}  # fmt: skip


def get_action_schedule_metadata(frames_per_step: int, release_after_frames: int) -> dict[str, Any]:
    return {
        "frames_per_step": frames_per_step,
        "release_after_frames": release_after_frames,
        "tick_split": [max(frames_per_step - 1, 0), 1 if frames_per_step > 0 else 0],
    }


def load_actions_trace(actions_file: str | Path) -> list[np.ndarray]:
    """One JSON list of ints per line (blank lines skipped)."""
    out = []
    for num, line in enumerate(Path(actions_file).read_text().splitlines(), 1):
        line = line.strip()
        if not line:
            continue
        try:
            out.append(np.array(json.loads(line), dtype=np.int32))
        except (json.JSONDecodeError, TypeError) as e:
            raise ValueError(f"Invalid action trace at line {num}: {e}") from e
    return out


def write_actions_trace(actions_trace: list[list[int]], output_path: Path) -> None:
    output_path.parent.mkdir(parents=True, exist_ok=True)
    output_path.write_text("".join(json.dumps(a) + "\n" for a in actions_trace))


# -- state comparison --------------------------------------------------------------
def parse_mem_region(region: str) -> tuple[int, int]:
    """``LO:HI`` in hex, HI exclusive, within [0, 0x10000]."""
    if ":" not in region:
        raise ValueError("mem region must be in LO:HI form")

    def h(text: str) -> int:
        t = text.strip().lower()
        t = t[2:] if t.startswith("0x") else t
        if not t:
            raise ValueError("empty hex value")
        v = int(t, 16)
        if not 0 <= v <= 0x10000:
            raise ValueError(f"hex value out of range: {text}")
        return v

    lo_s, hi_s = region.split(":", 1)
    lo, hi = h(lo_s), h(hi_s)
    if lo >= hi:
        raise ValueError(f"invalid memory range: {region}")
    return lo, hi


def parse_mem_regions(regions: list[str] | None) -> list[tuple[int, int]]:
    return [parse_mem_region(r) for r in regions or []]


def hash_memory(data: bytes) -> str:
    return hashlib.blake2b(data, digest_size=16).hexdigest()


def normalize_cpu_state(state: Mapping[str, Any]) -> dict[str, Any]:
    """Canonical key order and plain ints (``None`` where a backend has no value)."""
    out: dict[str, Any] = {k: (int(state[k]) if k in state else None) for k in CANONICAL_REGISTER_KEYS}
    flags = state.get("flags") or {}
    out["flags"] = {k: int(flags.get(k, 0)) for k in CANONICAL_FLAG_KEYS}
    for k in ("instr_count", "cycle_count", *CANONICAL_TRAP_KEYS):
        out[k] = int(state[k]) if state.get(k) is not None else None
    return out


def diff_states(ref_state: dict[str, Any], dut_state: dict[str, Any]) -> dict[str, Any] | None:
    """Field-level differences; counters and trap fields only when both sides have them."""
    diffs: dict[str, Any] = {}
    for k in CANONICAL_REGISTER_KEYS:
        if ref_state.get(k) != dut_state.get(k):
            diffs[k] = {"ref": ref_state.get(k), "dut": dut_state.get(k)}
    rf, df = ref_state.get("flags", {}), dut_state.get("flags", {})
    fd = {k: {"ref": rf.get(k), "dut": df.get(k)} for k in CANONICAL_FLAG_KEYS if rf.get(k) != df.get(k)}
    if fd:
        diffs["flags"] = fd
    for k in ("instr_count", "cycle_count", *CANONICAL_TRAP_KEYS):
        r, d = ref_state.get(k), dut_state.get(k)
        if r is not None and d is not None and r != d:
            diffs[k] = {"ref": r, "dut": d}
    return diffs or None


# -- system info, benchmark, artifacts ------------------------------------------------
def get_system_info() -> dict[str, Any]:
    info: dict[str, Any] = {
        "platform": platform.system(),
        "python": platform.python_version(),
        "numpy": np.__version__,
        "cpu": platform.processor() or None,
        "cpu_count": os.cpu_count(),
        "gpu": None,
        "gpu_names": [],
        "torch": None,
        "hip_version": None,
        "hip_visible_devices": os.environ.get("HIP_VISIBLE_DEVICES"),
    }
    try:
        import torch

        info["torch"] = torch.__version__
        info["hip_version"] = getattr(torch.version, "hip", None)
        if torch.cuda.is_available():
            names = [torch.cuda.get_device_name(i) for i in range(torch.cuda.device_count())]
            info["gpu_names"] = names
            info["gpu"] = names[0] if names else None
    except Exception:  # best effort, like the reference
        pass
    return info


def compute_rom_sha256(rom_path: str | Path) -> str:
    return hashlib.sha256(Path(rom_path).read_bytes()).hexdigest()


def synchronize_backend(backend: Any) -> None:
    if getattr(backend, "device", "cpu") != "cuda":
        return
    fn = getattr(backend, "synchronize", None)
    if callable(fn):
        fn()
        return
    import torch

    torch.cuda.synchronize()


def run_benchmark(backend: Any, *, steps: int, warmup_steps: int, action_gen: str,
                  actions_seed: int | None, frames_per_step: int, sync_every: int | None,
                  num_actions: int, action_names: list[str] | None = None) -> dict[str, Any]:  # fmt: skip
    """Warmup steps (negative step indices), then ``steps`` timed numpy steps
    with a sync every ``sync_every`` steps and at the end (harness.py:808-889)."""
    n = backend.num_envs
    backend.reset(seed=actions_seed)
    for i in range(warmup_steps):
        backend.step(generate_actions(-(warmup_steps - i), n, actions_seed, action_gen,
                                      num_actions, action_names))  # fmt: skip
    synchronize_backend(backend)
    t0 = time.perf_counter()
    for i in range(steps):
        backend.step(generate_actions(i, n, actions_seed, action_gen, num_actions, action_names))
        if sync_every and (i + 1) % sync_every == 0:
            synchronize_backend(backend)
    synchronize_backend(backend)
    dt = time.perf_counter() - t0
    total = steps * n
    sps = total / dt if dt > 0 else 0.0
    return {
        "warmup_steps": warmup_steps,
        "measured_steps": steps,
        "num_envs": n,
        "seconds": dt,
        "total_env_steps": total,
        "total_sps": sps,
        "per_env_sps": steps / dt if dt > 0 else 0.0,
        "frames_per_step": frames_per_step,
        "frames_per_sec": sps * frames_per_step,
    }


def get_divergence_receipt(backend: Any) -> dict[str, Any] | None:
    fn = getattr(backend, "get_pc_snapshot", None)
    if not callable(fn):
        return None
    pcs = np.asarray(fn(), dtype=np.int32).reshape(-1)
    u = int(np.unique(pcs).size)
    return {"metric": "unique_pc_count", "unique_pc_count": u, "num_envs": int(pcs.size),
            "unique_pc_ratio": (u / float(pcs.size)) if pcs.size else None}  # fmt: skip


def _write_json_atomic(path: Path, data: dict) -> None:
    """Temp file in the target directory, then rename: a reader never sees a
    partial artifact."""
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.parent / f".{path.name}.{uuid.uuid4().hex}.tmp"
    try:
        tmp.write_text(json.dumps(data, indent=2))
        os.replace(tmp, path)
    except Exception:
        tmp.unlink(missing_ok=True)
        raise


def write_artifact(output_dir: Path, *, run_id: str, system_info: dict[str, Any],
                   config: dict[str, Any], results: dict[str, Any]) -> Path:  # fmt: skip
    artifact = {
        "schema_version": RESULT_SCHEMA_VERSION,
        "run_id": run_id,
        "timestamp_utc": _utc_now().isoformat(),
        "system": system_info,
        "config": config,
        "results": results,
    }
    path = Path(output_dir) / f"{run_id}.json"
    _write_json_atomic(path, artifact)
    return path


# -- verify ------------------------------------------------------------------------
def _read_ppu_regs(backend: Any) -> dict[str, int] | None:
    reader = getattr(backend, "read_memory", None)
    if not callable(reader):
        return None
    try:
        return {name: reader(0, a, a + 1)[0] for name, a in PPU_REGS}
    except Exception:
        return None


def _read_ppu_dumps(ref: Any, dut: Any):
    rr, dr = getattr(ref, "read_memory", None), getattr(dut, "read_memory", None)
    if not callable(rr) or not callable(dr):
        return None
    meta, blobs = [], []
    for name, lo, hi in PPU_DUMP_REGIONS:
        top = min(hi, lo + MAX_MEM_DUMP_BYTES)
        try:
            rb, db = bytes(rr(0, lo, top)), bytes(dr(0, lo, top))
        except Exception:
            continue
        meta.append({"name": name, "lo": lo, "hi": hi, "dump_hi": top, "truncated": top < hi})
        blobs.append((name, lo, top, rb, db))
    return (meta, blobs) if meta else None


def _read_cart_state(backend: Any) -> dict[str, int] | None:
    fn = getattr(backend, "get_cart_state", None)
    if not callable(fn):
        return None
    try:
        return dict(fn(0))
    except Exception:
        return None


def _frame_shades(backend: Any) -> np.ndarray:
    reader = getattr(backend, "read_frame_bg_shade_env0", None)
    if not callable(reader):
        raise ValueError(f"Backend '{getattr(backend, 'name', 'unknown')}' does not support frame reads")
    return np.frombuffer(reader(), dtype=np.uint8).reshape(144, 160)


def write_mismatch_bundle(
    output_dir: Path,
    *,
    timestamp: str,
    rom_path: Path,
    rom_sha256: str,
    ref_backend: str,
    dut_backend: str,
    mismatch_step: int,
    env_idx: int,
    ref_state: dict[str, Any],
    dut_state: dict[str, Any],
    diff: dict[str, Any],
    action_codec: dict[str, Any],
    actions_trace: list[list[int]],
    system_info: dict[str, Any],
    action_gen_name: str,
    action_gen_seed: int | None,
    frames_per_step: int,
    release_after_frames: int,
    compare_every: int,
    verify_steps: int,
    mem_regions: list[tuple[int, int]] | None = None,
    mem_dumps: list[tuple[int, int, bytes, bytes]] | None = None,
    compare_frame: bool = False,
    frame_warmup: int = 0,
    ref_cart_state: dict[str, Any] | None = None,
    dut_cart_state: dict[str, Any] | None = None,
    ppu_regs: dict[str, dict[str, int]] | None = None,
    frame_hash_history: list[dict[str, Any]] | None = None,
    ppu_dumps=None,
) -> Path:
    """``<output_dir>/mismatch/<timestamp>_<rom>_<ref>_vs_<dut>/``, written in
    a temp directory and renamed into place."""
    final = Path(output_dir) / "mismatch" / f"{timestamp}_{Path(rom_path).stem}_{ref_backend}_vs_{dut_backend}"
    tmp = Path(output_dir) / "mismatch" / f".tmp_{uuid.uuid4()}"
    try:
        tmp.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(rom_path, tmp / "rom.gb")
        meta: dict[str, Any] = {
            "schema_version": MISMATCH_SCHEMA_VERSION,
            "timestamp_utc": _utc_now().isoformat(),
            "rom_path": str(rom_path),
            "rom_filename": "rom.gb",
            "rom_size": (tmp / "rom.gb").stat().st_size,
            "rom_sha256": rom_sha256,
            "ref_backend": ref_backend,
            "dut_backend": dut_backend,
            "mismatch_step": mismatch_step,
            "env_idx": env_idx,
            "verify_steps": verify_steps,
            "compare_every": compare_every,
            "frames_per_step": frames_per_step,
            "release_after_frames": release_after_frames,
            "compare_frame": compare_frame,
            "frame_warmup": frame_warmup,
            "action_generator": {"name": action_gen_name, "version": ACTION_GEN_VERSION,
                                 "seed": action_gen_seed},  # fmt: skip
            "action_codec": action_codec,
            "system": system_info,
        }
        if ppu_regs is not None:
            meta["ppu_regs"] = ppu_regs
        if frame_hash_history is not None:
            meta["frame_hash_history"] = frame_hash_history
        if ppu_dumps is not None:
            meta["ppu_mem_dumps"] = ppu_dumps[0]
        if mem_regions:
            meta["mem_regions"] = [{"lo": lo, "hi": hi} for lo, hi in mem_regions]
            meta["mem_hash_version"] = MEM_HASH_VERSION
        files: dict[str, Any] = {"metadata.json": meta, "ref_state.json": ref_state,
                                 "dut_state.json": dut_state, "diff.json": diff}  # fmt: skip
        if ref_cart_state is not None:
            files["ref_cart_state.json"] = ref_cart_state
        if dut_cart_state is not None:
            files["dut_cart_state.json"] = dut_cart_state
        for name, obj in files.items():
            (tmp / name).write_text(json.dumps(obj, indent=2))
        for lo, hi, rb, db in mem_dumps or []:
            (tmp / f"mem_ref_{lo:04X}_{hi:04X}.bin").write_bytes(rb)
            (tmp / f"mem_dut_{lo:04X}_{hi:04X}.bin").write_bytes(db)
        for name, lo, hi, rb, db in (ppu_dumps[1] if ppu_dumps else []):
            (tmp / f"{name}_ref_{lo:04X}_{hi:04X}.bin").write_bytes(rb)
            (tmp / f"{name}_dut_{lo:04X}_{hi:04X}.bin").write_bytes(db)
        write_actions_trace(actions_trace, tmp / "actions.jsonl")
        flags = "".join(f"    --mem-region {lo:04X}:{hi:04X} \\\n" for lo, hi in mem_regions or [])
        if compare_frame:
            flags += "    --compare-frame \\\n"
            if frame_warmup:
                flags += f"    --frame-warmup {frame_warmup} \\\n"
        script = (
            "#!/bin/bash\n"
            f"# Reproduces the mismatch at step {mismatch_step} (written {_utc_now().isoformat()})\n"
            "set -e\n"
            'HERE="$(cd "$(dirname "$0")" && pwd)"\n'
            "python -m gbxcule_amd.harness \\\n"
            "    --verify \\\n"
            f"    --ref-backend {ref_backend} \\\n"
            f"    --dut-backend {dut_backend} \\\n"
            '    --rom "$HERE/rom.gb" \\\n'
            f"    --verify-steps {verify_steps} \\\n"
            f"    --compare-every {compare_every} \\\n"
            f"    --frames-per-step {frames_per_step} \\\n"
            f"    --release-after-frames {release_after_frames} \\\n"
            f"    --action-codec {action_codec['id']} \\\n"
            f"{flags}"
            '    --actions-file "$HERE/actions.jsonl"\n'
        )
        (tmp / "repro.sh").write_text(script)
        os.chmod(tmp / "repro.sh", 0o755)
        if final.exists():
            shutil.rmtree(final)
        shutil.move(str(tmp), str(final))
        return final
    except Exception:
        if tmp.exists():
            shutil.rmtree(tmp)
        raise


def run_verify(
    ref: Any,
    dut: Any,
    *,
    rom_path: str | Path,
    ref_name: str = "ref",
    dut_name: str = "dut",
    verify_steps: int = 512,
    compare_every: int = 1,
    frames_per_step: int = 1,
    release_after_frames: int = 8,
    action_gen: str = "seeded_random",
    actions_seed: int | None = 0,
    action_codec: str = ACTION_CODEC_ID,
    mem_regions: list[tuple[int, int]] | None = None,
    compare_frame: bool = False,
    frame_warmup: int = 0,
    replay_actions: list[np.ndarray] | None = None,
    output_dir: str | Path = "bench/runs",
    log: Callable[[str], None] = print,
) -> tuple[int, Path | None]:
    """Step ``ref`` and ``dut`` (env 0) in lockstep and compare the canonical
    CPU state every ``compare_every`` steps, plus memory-region hashes and the
    env-0 frame hash when asked (harness.py:1793-2096).  On the first
    mismatch write a bundle and return ``(1, bundle_dir)``; else ``(0, None)``.
    Both backends must already be constructed with the same settings."""
    mem_regions = list(mem_regions or [])
    seed = actions_seed if action_gen == "seeded_random" else None
    codec = get_action_codec_metadata(action_codec)
    if replay_actions is not None and len(replay_actions) < verify_steps:
        verify_steps = len(replay_actions)
    ref.reset(seed=seed)
    dut.reset(seed=seed)
    if mem_regions:
        for b, name in ((ref, ref_name), (dut, dut_name)):
            if not callable(getattr(b, "read_memory", None)):
                raise ValueError(f"backend '{name}' does not support memory reads required by mem regions")
    if compare_frame:
        _frame_shades(ref)
        _frame_shades(dut)
    trace: list[list[int]] = []
    history: list[dict[str, Any]] = []
    for step in range(verify_steps):
        if replay_actions is not None:
            actions = np.asarray(replay_actions[step], dtype=np.int32)
        else:
            actions = generate_actions(step, 1, seed, action_gen, codec["num_actions"], codec["action_names"])
        trace.append(actions.tolist())
        ref.step(actions)
        dut.step(actions)
        if step % compare_every:
            continue
        rs = normalize_cpu_state(ref.get_cpu_state(0))
        ds = normalize_cpu_state(dut.get_cpu_state(0))
        diff = diff_states(rs, ds)
        dumps: list[tuple[int, int, bytes, bytes]] = []
        mem_diffs = []
        for lo, hi in mem_regions:
            rb, db = bytes(ref.read_memory(0, lo, hi)), bytes(dut.read_memory(0, lo, hi))
            if len(rb) != hi - lo or len(db) != hi - lo:
                raise ValueError(f"memory slice length mismatch for {lo:04X}:{hi:04X}")
            rh, dh = hash_memory(rb), hash_memory(db)
            if rh != dh:
                mem_diffs.append({"lo": lo, "hi": hi, "ref_hash": rh, "dut_hash": dh})
                if hi - lo <= MAX_MEM_DUMP_BYTES:
                    dumps.append((lo, hi, rb, db))
        if mem_diffs:
            diff = dict(diff or {}, memory=mem_diffs)
        if compare_frame and step >= frame_warmup:
            rh, dh = hash_memory(_frame_shades(ref).tobytes()), hash_memory(_frame_shades(dut).tobytes())
            history = (history + [{"step": step, "ref_hash": rh, "dut_hash": dh}])[-FRAME_HASH_HISTORY_LEN:]
            if rh != dh:
                diff = dict(diff or {}, frame_hash={"ref_hash": rh, "dut_hash": dh})
        if diff is None:
            continue
        ppu_ref, ppu_dut = _read_ppu_regs(ref), _read_ppu_regs(dut)
        ppu = {"ref": ppu_ref, "dut": ppu_dut} if ppu_ref is not None and ppu_dut is not None else None
        if ppu is not None:
            diff["ppu_regs"] = ppu
        log(f"MISMATCH at step {step}")
        log(f"First differing fields: {list(diff)[:5]}")
        bundle = write_mismatch_bundle(
            Path(output_dir), timestamp=_utc_now().strftime("%Y%m%d_%H%M%S"),
            rom_path=Path(rom_path), rom_sha256=compute_rom_sha256(rom_path),
            ref_backend=ref_name, dut_backend=dut_name, mismatch_step=step, env_idx=0,
            ref_state=rs, dut_state=ds, diff=diff, action_codec=codec, actions_trace=trace,
            system_info=get_system_info(), action_gen_name=action_gen, action_gen_seed=seed,
            frames_per_step=frames_per_step, release_after_frames=release_after_frames,
            compare_every=compare_every, verify_steps=verify_steps, mem_regions=mem_regions,
            mem_dumps=dumps or None, compare_frame=compare_frame, frame_warmup=frame_warmup,
            ref_cart_state=_read_cart_state(ref), dut_cart_state=_read_cart_state(dut),
            ppu_regs=ppu, frame_hash_history=history if compare_frame else None,
            ppu_dumps=_read_ppu_dumps(ref, dut),
        )  # fmt: skip
        log(f"Bundle: {bundle}")
        log(f"Repro: {bundle / 'repro.sh'}")
        return 1, bundle
    log(f"PASS: No mismatches in {verify_steps} steps")
    return 0, None


# -- CLI -----------------------------------------------------------------------------
def parse_args(argv: list[str] | None = None) -> argparse.Namespace:
    ap = argparse.ArgumentParser(description="gbxcule benchmark / lockstep verify harness")
    ap.add_argument("--rom", required=True)
    ap.add_argument("--backend", default="hip_vec")
    ap.add_argument("--num-envs", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup-steps", type=int, default=10)
    ap.add_argument("--sync-every", type=int, default=None,
                    help="sync every K steps (default 64 on the GPU; 0 = end only)")
    ap.add_argument("--stage", default="emulate_only")
    ap.add_argument("--frames-per-step", type=int, default=24)
    ap.add_argument("--release-after-frames", type=int, default=8)
    ap.add_argument("--action-gen", default="noop", choices=["noop", "seeded_random", "striped"])
    ap.add_argument("--actions-seed", type=int, default=None,
                    help="seed of seeded_random; warmup steps use seed - warmup .. seed - 1")
    ap.add_argument("--action-codec", default=ACTION_CODEC_ID)
    ap.add_argument("--output-dir", default="bench/runs")
    ap.add_argument("--verify", action="store_true")
    ap.add_argument("--ref-backend", default="hip_vec")
    ap.add_argument("--dut-backend", default="hip_vec")
    ap.add_argument("--verify-steps", type=int, default=512)
    ap.add_argument("--compare-every", type=int, default=1)
    ap.add_argument("--mem-region", action="append", default=[])
    ap.add_argument("--compare-frame", action="store_true")
    ap.add_argument("--frame-warmup", type=int, default=0)
    ap.add_argument("--actions-file", default=None)
    return ap.parse_args(argv)


def main(argv: list[str] | None = None) -> int:
    args = parse_args(argv)
    rom = Path(args.rom)
    if args.verify:
        try:
            regions = parse_mem_regions(args.mem_region)
            replay = load_actions_trace(args.actions_file) if args.actions_file else None
        except (ValueError, FileNotFoundError) as e:
            print(f"Error: {e}", file=sys.stderr)
            return 1
        kw = dict(num_envs=1, frames_per_step=args.frames_per_step,
                  release_after_frames=args.release_after_frames, stage=args.stage,
                  action_codec=args.action_codec, render_bg=args.compare_frame)  # fmt: skip
        ref = create_backend(args.ref_backend, str(rom), **kw)
        try:
            dut = create_backend(args.dut_backend, str(rom), **kw)
        except Exception:
            getattr(ref, "close", lambda: None)()
            raise
        try:
            rc, _ = run_verify(
                ref, dut, rom_path=rom, ref_name=args.ref_backend, dut_name=args.dut_backend,
                verify_steps=args.verify_steps, compare_every=args.compare_every,
                frames_per_step=args.frames_per_step, release_after_frames=args.release_after_frames,
                action_gen=args.action_gen, actions_seed=args.actions_seed,
                action_codec=args.action_codec, mem_regions=regions,
                compare_frame=args.compare_frame, frame_warmup=args.frame_warmup,
                replay_actions=replay, output_dir=args.output_dir,
            )  # fmt: skip
        finally:
            for b in (ref, dut):
                getattr(b, "close", lambda: None)()
        return rc
    backend = create_backend(args.backend, str(rom), num_envs=args.num_envs,
                             frames_per_step=args.frames_per_step,
                             release_after_frames=args.release_after_frames, stage=args.stage,
                             action_codec=args.action_codec)  # fmt: skip
    sync_every = args.sync_every
    if sync_every is None:
        sync_every = 64 if getattr(backend, "device", "cpu") == "cuda" else None
    try:
        codec = get_action_codec_metadata(args.action_codec)
        results = run_benchmark(
            backend, steps=args.steps, warmup_steps=args.warmup_steps, action_gen=args.action_gen,
            actions_seed=args.actions_seed, frames_per_step=args.frames_per_step,
            sync_every=sync_every, num_actions=codec["num_actions"],
            action_names=codec["action_names"],
        )  # fmt: skip
        receipt = get_divergence_receipt(backend)
    finally:
        getattr(backend, "close", lambda: None)()
    if receipt is not None:
        results["divergence"] = receipt
    stamp = _utc_now().strftime("%Y%m%dT%H%M%SZ")
    run_id = f"{stamp}__{args.backend}__rom_{rom.stem}__envs_{args.num_envs}"
    config = {
        "backend": args.backend,
        "rom_path": str(rom),
        "rom_sha256": compute_rom_sha256(rom),
        "stage": args.stage,
        "num_envs": args.num_envs,
        "steps": args.steps,
        "warmup_steps": args.warmup_steps,
        "sync_every": sync_every,
        "action_generator": get_action_gen_metadata(args.action_gen, args.actions_seed,
                                                    action_names=codec["action_names"],
                                                    num_actions=codec["num_actions"]),  # fmt: skip
        "action_codec": codec,
        "action_schedule": get_action_schedule_metadata(args.frames_per_step, args.release_after_frames),
    }
    path = write_artifact(Path(args.output_dir) / stamp, run_id=run_id,
                          system_info=get_system_info(), config=config, results=results)  # fmt: skip
    print(json.dumps(results))
    print(f"Artifact: {path}")
    return 0


if __name__ == "__main__":  # pragma: no cover
    sys.exit(main())
