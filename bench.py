"""Throughput of the HIP Game Boy core on one MI355X.

A step is one launch of the SM83 step kernel over every env (plus, for the
PPU/RL workloads, the snapshot render, the masked reset and the RAM-sense
gather), on synthetic seeded cartridges with a seeded 8-way action trace that
is uploaded to the device before timing.  Metric: env-steps/s (whole job) and
emulated frames/s = env-steps/s * frameskip.

Default workload: 16,384 envs, frameskip 24, CPU-step only (the config the
headline metric is quoted on).  ``--workload`` selects the others.

Prints one JSON line.  ``roofline`` is computed for the step kernel from its
algorithmic bytes per env-step (922 B of per-env state read+written plus the
emulated data-memory bytes the oracle counts on the same trace) and its
average duration measured with HIP events; ``cpu_baseline`` times the oracle
(a C++ restatement of the reference Warp CPU backend) on a bounded prefix of
the same workload on the host cores.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "env-steps/sec @ frameskip 24 (16K & 128K envs); emulated frames/sec"
STATE_BYTES = 922  # per-env scalar state + FF00-FFFF page, read and written once
HBM_PEAK_GBS = 8000.0


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="c2", help="c1, c2, c3, c4, c4m3, c5")
    ap.add_argument("--envs", type=int, default=None, help="override the env count")
    ap.add_argument("--frameskip", type=int, default=None, help="override the frameskip")
    ap.add_argument("--reset-prob", type=float, default=None,
                    help="override the per-step masked-reset probability")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 256 MiB device copy (PMC scaling reference)")
    return ap.parse_args()


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def oracle_sample(wl, rom, boot, n_env, seconds, threads, max_steps=200):
    """Time the oracle on envs [0, n_env) of the workload's own trace."""
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
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    data_per_env_step = float(ref.data_bytes.sum()) / (n_env * steps)
    instr_per_env_step = float(ref.field("instr_count").sum()) / (n_env * steps)
    ref.close()
    return steps, dt, data_per_env_step, instr_per_env_step


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

    from gbxcule_amd.backend import HipVecBackend
    from gbxcule_amd.carts.bootstub import build_bootstub
    from gbxcule_amd.carts.synth import WORKLOADS, seeded_actions
    from gbxcule_amd.reset_cache import ResetCache

    wl = WORKLOADS[args.workload]
    if args.envs or args.frameskip or args.reset_prob is not None:
        from dataclasses import replace

        wl = replace(
            wl,
            num_envs=args.envs or wl.num_envs,
            frames_per_step=args.frameskip or wl.frames_per_step,
            reset_prob=wl.reset_prob if args.reset_prob is None else args.reset_prob,
        )
    n, fs = wl.num_envs, wl.frames_per_step
    steps = args.steps if args.steps is not None else (20 if n <= 20000 else 10)
    warmup = args.warmup
    rom, boot = wl.rom(), build_bootstub()
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)

    be = HipVecBackend(
        rom,
        num_envs=n,
        frames_per_step=fs,
        release_after_frames=wl.release_after_frames,
        stage=wl.stage,
        render_pixels=wl.render == "unpacked",
        render_pixels_packed=wl.render == "packed",
        render_on_step=False,
        bootrom=boot,
    )
    be.reset(seed=wl.actions_seed)
    total = warmup + steps
    # timed steps use step indices 0..steps-1 of the seeded trace; warmup
    # steps draw from indices past 10**6 so they never overlap
    idx = [10**6 + k for k in range(warmup)] + list(range(steps))
    trace = np.stack([seeded_actions(wl.actions_seed, k, n) for k in idx]).astype(np.int32)
    actions = torch.from_numpy(trace).to(dev)
    masks = None
    senses_out = None
    cache = None
    if wl.reset_prob > 0:
        rng = np.random.default_rng(wl.actions_seed + 1000)
        masks = torch.from_numpy((rng.random((total, n)) < wl.reset_prob).astype(np.uint8)).to(dev)
        cache = ResetCache.from_backend(be, env_idx=0)
    if wl.senses:
        rng = np.random.default_rng(wl.actions_seed + 2000)
        addrs = np.sort(rng.choice(np.arange(0xC000, 0xE000), wl.senses, replace=False))
        senses_out = torch.empty((n, wl.senses), dtype=torch.uint8, device=dev)
    packed_out = None
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

    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for k in range(warmup):
        one_step(k)
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        one_step(warmup + i, events[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_ms = [a.elapsed_time(b) for a, b in events]
    kernel_ms = float(np.mean(step_ms))
    value = n * steps / elapsed
    traps = int(be.export_field("trap_flag").sum())
    lanes = be.step_lanes
    instr_gpu = float(be.export_field("instr_count").sum())

    # CPU baseline on a bounded prefix of the same trace; also yields the
    # per-env-step emulated data bytes for the roofline.
    threads = cpu_threads()
    cpu = None
    if args.no_cpu_baseline:
        _, _, data_b, instr_b = oracle_sample(wl, rom, boot, 64, 0.0, threads, max_steps=1)
    else:
        n_cpu = min(n, 32 * threads)
        c_steps, c_dt, data_b, instr_b = oracle_sample(
            wl, rom, boot, n_cpu, args.cpu_seconds, threads
        )
        cpu = {
            "value": n_cpu * c_steps / c_dt,
            "unit": "env-steps/s",
            "cores": threads,
            "kind": "port",
            "sample": f"oracle (C++ restatement of the reference Warp CPU step) on envs "
            f"0..{n_cpu - 1} of the same cart and action trace, {c_steps} steps of "
            f"frameskip {fs}, {threads} OpenMP threads, {c_dt:.1f} s",
        }
    bytes_per_env_step = STATE_BYTES + data_b
    achieved = n * bytes_per_env_step / (kernel_ms * 1e-3) / 1e9
    traffic = None
    valu = None
    tfile = ROOT / "profiles" / f"traffic_{args.workload}_{n}.json"
    if tfile.exists() and fs == WORKLOADS[args.workload].frames_per_step:
        t = json.loads(tfile.read_text())
        traffic = t.get("bytes_per_launch")
        if t.get("valu_wave_insts_per_launch"):
            # VALU issue slots: profiled wave-instructions per launch x 64 lanes
            # over this run's measured kernel time
            lane_ops = t["valu_wave_insts_per_launch"] * 64 / (kernel_ms * 1e-3)
            peak = t["valu_peak_lane_ops_per_s"]
            valu = {
                "achieved": lane_ops,
                "peak": peak,
                "unit": "lane-op/s",
                "frac": lane_ops / peak,
                "source": t.get("source"),
            }
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": elapsed / steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {
            "workload": wl.name,
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
            "step_lanes": lanes,
        },
        "frames_per_sec": value * fs,
        "emulated_instr_per_sec": instr_gpu / max(warmup + steps, 1) / (elapsed / steps),
        "step_kernel_ms": kernel_ms,
        "traps": traps,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": "gbx::step_kernel",
            "bytes_per_env_step": bytes_per_env_step,
            "instr_per_env_step": instr_b,
        },
        "valu": valu,
        "cpu_baseline": cpu,
    }
    be.close()
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
