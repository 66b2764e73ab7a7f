"""Throughput of the HIP Game Boy core on one MI355X.

A step is one launch of the SM83 step kernel over every env (plus, for the
PPU/RL workloads, the snapshot render, the masked reset and the RAM-sense
gather), on synthetic seeded cartridges with a seeded 8-way action trace that
is uploaded to the device before timing.  Metric: env-steps/s (whole job) and
emulated frames/s = env-steps/s * frameskip.

The headline ``value`` is the CPU-step workload at 16,384 envs, frameskip 24
(``--workload`` selects another).  The same JSON line carries measured
sub-objects for the 128K-env half of the metric (``workloads``): the banked
cart with interrupts at 131,072 envs, frameskip 24 and 1, and the RL rollout
shape at 131,072 envs, each timed the same way in this run.

``roofline`` is computed for the step kernel from its algorithmic bytes per
env-step (922 B of per-env state read+written plus the emulated data-memory
bytes the oracle counts on the same trace) and its average duration measured
with HIP events on the stream it is launched on.  ``cpu_baseline`` times the
oracle (a C++ restatement of the reference Warp CPU backend) on a bounded
sample of the same workload on the host cores allotted to this process, and
on one thread.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from dataclasses import replace
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "env-steps/sec @ frameskip 24 (16K & 128K envs); emulated frames/sec"
STATE_BYTES = 922  # per-env scalar state + FF00-FFFF page, read and written once
HBM_PEAK_GBS = 8000.0
# the 128K-env workloads timed beside the headline: (key, workload, envs,
# frameskip, steps, warmup steps).  The rollout is timed once it has settled:
# after 200 steps about 87% of its envs have been restored at least once, so
# envs of one wavefront run their frames out of phase as in a long rollout
# (the first steps after power-on are about 13% faster).
EXTRA = (
    ("c3_ppu_packed_16k_fs24", "c3", 16_384, 24, 20, 20),
    ("c4_mbc1_irq_131k_fs24", "c4", 131_072, 24, 10, 2),
    ("c4_mbc1_irq_131k_fs1", "c4", 131_072, 1, 50, 2),
    ("c4_mbc3_ram_irq_131k_fs24", "c4m3", 131_072, 24, 10, 2),
    ("c4_mbc3_ram_irq_131k_fs1", "c4m3", 131_072, 1, 50, 2),
    ("c5_rl_rollout_131k_fs24", "c5", 131_072, 24, 20, 200),
)
TARGETS = {  # env-steps/s the banked-cart 131K target names, per frameskip
    ("c4", 131_072, 24): 400_000,
    ("c4", 131_072, 1): 10_000_000,
    ("c4m3", 131_072, 24): 400_000,
    ("c4m3", 131_072, 1): 10_000_000,
}
# Untimed steps that bring a workload to its steady state before the warmup
# and timed steps.  The CPU-step cart's lanes drift apart over its first
# launches (each lane's program follows its own joypad-keyed branches), and a
# launch lengthens as they do; after 100 steps the launch time has settled.
SETTLE = {"c2": 100}



def wl_label(wl, default) -> str:
    """The registry name of a workload, with the env count and frameskip it
    ran at when they differ from the registry's."""
    name = wl.name
    if wl.num_envs != default.num_envs:
        name = name.rsplit("_", 1)[0] + f"_{wl.num_envs}envs"
    if wl.frames_per_step != default.frames_per_step:
        name += f"_fs{wl.frames_per_step}"
    return name

def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--settle", type=int, default=None,
                    help="untimed steps before the warmup (default: the workload's settle count)")
    ap.add_argument("--workload", default="c2", help="c1, c2, c3, c4, c4m3, c5")
    ap.add_argument("--envs", type=int, default=None, help="override the env count")
    ap.add_argument("--frameskip", type=int, default=None, help="override the frameskip")
    ap.add_argument("--reset-prob", type=float, default=None,
                    help="override the per-step masked-reset probability")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="time only the headline workload")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 256 MiB device copy (PMC scaling reference)")
    return ap.parse_args()


def cpu_threads() -> tuple[int, int]:
    """(threads to use, CPUs this process may run on).  The pool of the GPU
    host is shared per GPU; OMP_NUM_THREADS states this process's share."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        avail = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    return max(1, min(avail, share)), avail


def oracle_sample(wl, rom, boot, n_env, seconds, threads, max_steps=200):
    """Time the oracle on envs [0, n_env) of the workload's own trace: up to
    ``max_steps`` steps, stopping early once ``seconds`` (if > 0) have passed."""
    from gbxcule_amd.carts.synth import seeded_actions
    from oracle.ref import RefMachine

    ref = RefMachine(n_env, rom, boot)
    ref.step(None, 0, 0, wl.stage)
    steps = 0
    t0 = time.perf_counter()
    while steps < max_steps:
        act = seeded_actions(wl.actions_seed, steps, wl.num_envs)[:n_env]
        ref.step(act, wl.frames_per_step, wl.release_after_frames, wl.stage, threads=threads)
        if wl.render:
            ref.render(packed=wl.render == "packed", threads=threads)
        steps += 1
        if seconds > 0 and time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    data_per_env_step = float(ref.data_bytes.sum()) / (n_env * steps)
    instr_per_env_step = float(ref.field("instr_count").sum()) / (n_env * steps)
    ref.close()
    return steps, dt, data_per_env_step, instr_per_env_step


def profile_file(key: str, n: int, fs: int):
    """A committed rocprof summary for this workload shape, if any."""
    f = ROOT / "profiles" / f"traffic_{key}_{n}{'' if fs == 24 else f'_fs{fs}'}.json"
    return json.loads(f.read_text()) if f.exists() else None


def time_workload(wl, steps: int, warmup: int, settle: int = 0) -> dict:
    """Run ``settle`` + ``warmup`` + ``steps`` steps of ``wl`` and time the
    last ``steps``."""
    import torch

    from gbxcule_amd.backend import HipVecBackend
    from gbxcule_amd.carts.bootstub import build_bootstub
    from gbxcule_amd.carts.synth import seeded_actions
    from gbxcule_amd.reset_cache import ResetCache

    n, fs = wl.num_envs, wl.frames_per_step
    dev = torch.device("cuda", 0)
    be = HipVecBackend(
        wl.rom(),
        num_envs=n,
        frames_per_step=fs,
        release_after_frames=wl.release_after_frames,
        stage=wl.stage,
        render_pixels=wl.render == "unpacked",
        render_pixels_packed=wl.render == "packed",
        render_on_step=False,
        bootrom=build_bootstub(),
    )
    try:
        be.reset(seed=wl.actions_seed)
        warmup += settle
        total = warmup + steps
        # timed steps use step indices 0..steps-1 of the seeded trace; settle
        # and warmup steps draw from indices past 10**6 so they never overlap
        idx = [10**6 + k for k in range(warmup)] + list(range(steps))
        trace = np.stack([seeded_actions(wl.actions_seed, k, n) for k in idx]).astype(np.int32)
        actions = torch.from_numpy(trace).to(dev)
        masks = cache = senses_out = packed_out = None
        if wl.reset_prob > 0:
            rng = np.random.default_rng(wl.actions_seed + 1000)
            masks = torch.from_numpy((rng.random((total, n)) < wl.reset_prob).astype(np.uint8)).to(dev)
            cache = ResetCache.from_backend(be, env_idx=0)
        if wl.senses:
            rng = np.random.default_rng(wl.actions_seed + 2000)
            addrs = np.sort(rng.choice(np.arange(0xC000, 0xE000), wl.senses, replace=False))
            senses_out = torch.empty((n, wl.senses), dtype=torch.uint8, device=dev)
        if wl.render == "packed":
            packed_out = torch.empty((n, 72, 20), dtype=torch.uint8, device=dev)

        def one_step(k, ev=None):
            if ev is not None:
                ev[0].record()
            be.step_torch(actions[k])
            if ev is not None:
                ev[1].record()
            if wl.render == "packed":
                be.render_pixels_snapshot_packed_to_torch(packed_out, 0)
            elif wl.render == "unpacked":
                be.render_pixels_snapshot()
            if cache is not None:
                cache.apply_mask_torch(masks[k])
            if senses_out is not None:
                be.ram_senses_torch(addrs, out=senses_out)

        for k in range(warmup):
            one_step(k)
        torch.cuda.synchronize()
        instr0 = int(be.export_field("instr_count").sum()) if cache is None else 0
        # the kernel runs on torch's current stream, where these events record
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(steps)]
        t0 = time.perf_counter()
        for i in range(steps):
            one_step(warmup + i, events[i])
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        kernel_ms = float(np.mean([a.elapsed_time(b) for a, b in events]))
        value = n * steps / elapsed
        # emulated instructions per env-step from the device counters: over
        # the timed steps, or, where a masked reset sets restored envs'
        # counters back to the snapshot's, over one more (untimed) step read
        # before its reset
        if cache is None:
            instr_per_env_step = (int(be.export_field("instr_count").sum()) - instr0) / (n * steps)
        else:
            i0 = int(be.export_field("instr_count").sum())
            be.step_torch(actions[total - 1])
            torch.cuda.synchronize()
            instr_per_env_step = (int(be.export_field("instr_count").sum()) - i0) / n
        return {
            "value": value,
            "unit": "env-steps/s",
            "num_envs": n,
            "frameskip": fs,
            "steps": steps,
            "warmup": warmup - settle,
            "settle": settle,
            "ms_per_step": elapsed / steps * 1e3,
            "step_kernel_ms": kernel_ms,
            "frames_per_sec": value * fs,
            "emulated_instr_per_sec": instr_per_env_step * value,
            "emulated_instr_per_env_step": instr_per_env_step,
            "traps": int(be.export_field("trap_flag").sum()),
            "step_lanes": be.step_lanes,
        }
    finally:
        be.close()


def roofline(key: str, res: dict, data_b: float, instr_b: float) -> dict:
    """Step-kernel roofline: algorithmic bytes per launch over its measured
    duration; rocprof traffic per launch where a committed summary exists."""
    n, fs, kernel_ms = res["num_envs"], res["frameskip"], res["step_kernel_ms"]
    bytes_per_env_step = STATE_BYTES + data_b
    achieved = n * bytes_per_env_step / (kernel_ms * 1e-3) / 1e9
    prof = profile_file(key, n, fs)
    out = {
        "bound": "hbm",
        "achieved": achieved,
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": achieved / HBM_PEAK_GBS,
        "traffic": prof.get("bytes_per_launch") if prof else None,
        "kernel": "gbx::step_kernel",
        "bytes_per_env_step": bytes_per_env_step,
        "instr_per_env_step": instr_b,
        "achieved_counts": "emulated accesses: the step kernel batches poll and copy loops and "
        "keeps hot registers in VGPRs, so it moves far fewer bytes than it emulates",
    }
    if prof:
        out["traffic_source"] = prof.get("source")
    return out


def valu_object(key: str, res: dict):
    """VALU issue against the chip's peak: profiled wave-instructions per
    launch (committed rocprof summary of the same workload) x 64 lanes over
    this run's measured kernel time, plus the profiled active-lane fraction."""
    prof = profile_file(key, res["num_envs"], res["frameskip"])
    if not prof or not prof.get("valu_wave_insts_per_launch"):
        return None
    lane_ops = prof["valu_wave_insts_per_launch"] * 64 / (res["step_kernel_ms"] * 1e-3)
    peak = prof["valu_peak_lane_ops_per_s"]
    out = {
        "achieved": lane_ops,
        "peak": peak,
        "unit": "lane-op/s (issue slots)",
        "frac": lane_ops / peak,
        "source": prof.get("source"),
    }
    for k in ("active_lane_frac", "valu_busy", "useful_lane_frac"):
        if k in prof:
            out[k] = prof[k]
    return out


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: the emulator has no cross-env communication and "
            "this build runs on a single MI355X; --gpus must be 1",
            file=sys.stderr,
        )
        return 2
    import torch

    from gbxcule_amd.carts.bootstub import build_bootstub
    from gbxcule_amd.carts.synth import WORKLOADS

    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    wl = WORKLOADS[args.workload]
    if args.envs or args.frameskip or args.reset_prob is not None:
        wl = replace(
            wl,
            num_envs=args.envs or wl.num_envs,
            frames_per_step=args.frameskip or wl.frames_per_step,
            reset_prob=wl.reset_prob if args.reset_prob is None else args.reset_prob,
        )
    n, fs = wl.num_envs, wl.frames_per_step
    steps = args.steps if args.steps is not None else (20 if n <= 20000 else 10)
    settle = SETTLE.get(args.workload, 0) if args.settle is None else args.settle
    res = time_workload(wl, steps, args.warmup, settle)
    rom, boot = wl.rom(), build_bootstub()

    # the 128K-env workloads, each timed the same way
    extra = {}
    if not args.no_extra:
        for key, wname, en, efs, esteps, ewarm in EXTRA:
            ewl = replace(WORKLOADS[wname], num_envs=en, frames_per_step=efs)
            r = time_workload(ewl, esteps, max(ewarm, args.warmup))
            # the same 24 emulated frames as one frameskip-24 step
            _, _, db, ib = oracle_sample(ewl, ewl.rom(), boot, 64, 0.0, cpu_threads()[0],
                                         max_steps=max(1, 24 // efs))
            r["roofline"] = roofline(wname, r, db, ib)
            r["valu"] = valu_object(wname, r)
            r["workload"] = key
            tgt = TARGETS.get((wname, en, efs))
            if tgt:
                r["target"] = tgt
            extra[key] = r

    # CPU baseline on a bounded sample of the same trace; also yields the
    # per-env-step emulated data bytes for the roofline.
    threads, avail = cpu_threads()
    cpu = None
    if args.no_cpu_baseline:
        _, _, data_b, instr_b = oracle_sample(wl, rom, boot, 64, 0.0, threads, max_steps=max(1, 24 // fs))
    else:
        n_cpu = min(n, 64 * threads)
        c_steps, c_dt, data_b, instr_b = oracle_sample(wl, rom, boot, n_cpu, args.cpu_seconds, threads)
        n1 = min(n, 32)
        s1, dt1, _, _ = oracle_sample(wl, rom, boot, n1, args.cpu_seconds / 2, 1)
        cpu = {
            "value": n_cpu * c_steps / c_dt,
            "unit": "env-steps/s",
            "cores": threads,
            "kind": "port",
            "host_cpus": avail,
            "single_thread_value": n1 * s1 / dt1,
            "sample": f"oracle (C++ restatement of the reference Warp CPU step, g++ -O3 "
            f"-march=x86-64-v3) on envs 0..{n_cpu - 1} of the same cart and action trace, "
            f"{c_steps} steps of frameskip {fs}, {threads} OpenMP threads ({avail} CPUs "
            f"available), {c_dt:.1f} s; single thread: envs 0..{n1 - 1}, {s1} steps, {dt1:.1f} s",
        }
    out = {
        "metric": METRIC,
        "value": res["value"],
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {
            "workload": wl_label(wl, WORKLOADS[args.workload]),
            "num_envs": n,
            "frameskip": fs,
            "release_after_frames": wl.release_after_frames,
            "cart": wl.cart,
            "cart_seed": wl.cart_seed,
            "actions_seed": wl.actions_seed,
            "stage": wl.stage,
            "render": wl.render,
            "reset_prob": wl.reset_prob,
            "senses": wl.senses,
            "step_lanes": res["step_lanes"],
            "settle_steps": settle,
        },
        "frames_per_sec": res["frames_per_sec"],
        "emulated_instr_per_sec": res["emulated_instr_per_sec"],
        "emulated_instr_per_env_step": res["emulated_instr_per_env_step"],
        "step_kernel_ms": res["step_kernel_ms"],
        "traps": res["traps"],
        "roofline": roofline(args.workload, res, data_b, instr_b),
        "valu": valu_object(args.workload, res) if fs == WORKLOADS[args.workload].frames_per_step else None,
        "cpu_baseline": cpu,
        "workloads": extra,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
