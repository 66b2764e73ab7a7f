"""Parity over long traces: the configurations' stated lengths.

* C1 (64 envs, frameskip 4): all 256 steps, the full state of every env
  compared with the oracle after every step.
* C2 (16,384 envs, frameskip 24) and C5 (131,072 envs, 1% masked restores,
  unpacked render and RAM senses every step; 2,000 steps): the GPU runs every
  env.  A sample of envs (env 0, env N-1, random envs, and in C5 envs restored
  several times) is replayed on the oracle from power-on on its own action
  and restore columns and compared in full at checkpoints.  At every
  checkpoint every env is also held to two invariants of the reference's
  frame loop: with the LCD on, cycle_in_frame = LY * 456 + scanline cycle
  (both restart together when the LCD is switched on and advance by the same
  cycles), and cycle_count - cycle_in_frame grows by exactly frameskip *
  70,224 per step while the LCD is not switched.  C2 runs all 1,000 steps,
  as five tests of 200 steps that continue one run (about 0.14 s per
  launch).  C5 runs all 2,000: its 256-entry SCX/SCY walk wraps many times.
* C3 (16,384 envs, packed render every step) for 240 steps, sampled the
  same way, the sample's packed observation included.
* C4 (512 KiB MBC1 cart, timer/VBlank/STAT interrupts, HALT wake loops) at
  its target shape, 131,072 envs, for 200 steps, sampled the same way.
* The MBC3 cart (C4's variant, 32 KiB cart RAM, RTC) for 200 steps at 8,192
  envs: 80 emulated seconds, so the RTC carries into minutes; every env's
  clock must equal the closed form of its cycle count.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.synth import seeded_actions
from oracle.ref import RefMachine

from ._parity import assert_same_state, ref_export_env
from .conftest import require_gpu

pytestmark = pytest.mark.gpu

CS_RTC_SECONDS, CS_RTC_MINUTES, CS_RTC_LAST_CYCLE = 9, 10, 14


def _backend(rom, boot, n, fs, render):
    from gbxcule_amd.backend import HipVecBackend

    return HipVecBackend(
        rom, num_envs=n, frames_per_step=fs, release_after_frames=8, stage="full_step",
        render_pixels=render == "unpacked", render_pixels_packed=render == "packed", bootrom=boot,
    )  # fmt: skip


class FrameInvariants:
    """The two frame-loop invariants above, over every env."""

    def __init__(self, fs: int):
        self.fs = fs
        self.prev = None

    def check(self, dut, k: int, tag: str) -> None:
        cf = dut.export_field("cycle_in_frame")
        ly, sc = dut.export_field("ppu_ly"), dut.export_field("ppu_scanline_cycle")
        lcd_on = (dut.memory_torch()[:, 0xFF40].cpu().numpy() & 0x80) != 0
        bad = np.nonzero(lcd_on & (cf != (ly * 456 + sc) % 70224))[0]
        assert bad.size == 0, f"[{tag} step {k}] {bad.size} envs: cycle_in_frame != LY*456+scanline, env {bad[0]}"
        cur = (dut.export_field("cycle_count") - cf, k)
        if self.prev is not None:
            steps = cur[1] - self.prev[1]
            bad = np.nonzero(cur[0] - self.prev[0] != steps * self.fs * 70224)[0]
            assert bad.size == 0, f"[{tag} step {k}] {bad.size} envs ran other than {steps * self.fs} frames"
        self.prev = cur
        assert int(dut.export_field("trap_flag").sum()) == 0, f"[{tag} step {k}] trapped envs"


def _step_async(dut, act) -> None:
    """One step from device actions (no host sync, so the oracle's replay of
    the sample runs while the GPU steps)."""
    import torch

    dut.step_torch(torch.from_numpy(act).cuda())


def _compare_sample(dut, ref, sample, tag, render=None) -> None:
    """Full state of the sampled envs against the oracle.  The action slot is
    left out: step_torch runs on the caller's device actions and, like the
    reference's (backends/warp_vec.py:1266-1269), leaves the backend's own
    action buffer as it was, while the oracle's step stores each action."""
    import torch

    from gbxcule_amd.state_io import FIELDS

    for j, e in enumerate(sample.tolist()):
        got, want = dut.export_env(e), ref_export_env(ref, j)
        bad = [FIELDS[i] for i in range(len(FIELDS))
               if got.scalars[i] != want.scalars[i] and FIELDS[i] != "actions"]  # fmt: skip
        assert not bad, f"[{tag}] env {e}: fields {bad[:5]} differ"
        np.testing.assert_array_equal(got.cart_state, want.cart_state, err_msg=f"{tag} env {e} cart state")
        if not np.array_equal(got.mem, want.mem):
            a = int(np.nonzero(got.mem != want.mem)[0][0])
            raise AssertionError(f"[{tag}] env {e} memory differs first at {a:#06x}")
        np.testing.assert_array_equal(got.cart_ram, want.cart_ram, err_msg=f"{tag} env {e} cart RAM")
    idx = torch.from_numpy(sample).cuda()
    np.testing.assert_array_equal(dut.obs_torch()[idx].cpu().numpy().view(np.uint32), ref.obs.view(np.uint32))
    np.testing.assert_array_equal(dut.reward_torch()[idx].cpu().numpy().view(np.uint32), ref.reward.view(np.uint32))
    np.testing.assert_array_equal(dut.export_serial()[sample], ref.serial_buf, err_msg=f"{tag} serial")
    if render == "unpacked":
        np.testing.assert_array_equal(dut.pixels_torch()[idx].cpu().numpy(), ref.pix, err_msg=f"{tag} pixels")
    if render == "packed":
        np.testing.assert_array_equal(
            dut.pixels_packed_torch()[idx].cpu().numpy(), ref.pix_packed, err_msg=f"{tag} packed pixels"
        )


def test_c1_every_step_of_the_full_trace(carts, bootstub):
    require_gpu()
    n, fs, steps, seed = 64, 4, 256, 0
    rom = carts["c1"]
    dut = _backend(rom, bootstub, n, fs, None)
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=seed)
        ref.step(None, 0, 0, "full_step")
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            obs, *_ = dut.step(act)
            ref.step(act, fs, 8, "full_step", threads=8)
            assert_same_state(dut, ref, step=k, tag="c1-256")
            np.testing.assert_array_equal(obs.view(np.uint32), ref.obs.view(np.uint32))
        assert int(ref.field("trap_flag").sum()) == 0
    finally:
        dut.close()
        ref.close()


class SampledRun:
    """A workload on the GPU at full size with a sample of its envs replayed
    on the oracle, advanced in parts so that a long trace reports as it
    goes.  Checkpoints every ``every`` steps: the frame invariants over every
    env and the sample's full state."""

    def __init__(self, rom, boot, n, fs, seed, tag, every, sample_size=6, render=None):
        rng = np.random.default_rng(seed)
        self.sample = np.unique(
            np.concatenate([[0, n - 1], rng.choice(n, sample_size, replace=False)])
        ).astype(np.int64)
        self.n, self.fs, self.seed, self.tag, self.every = n, fs, seed, tag, every
        self.render = render
        self.dut = _backend(rom, boot, n, fs, render)
        self.ref = RefMachine(self.sample.size, rom, boot)
        self.inv = FrameInvariants(fs)
        self.k = 0
        self.dut.reset(seed=seed)
        self.ref.step(None, 0, 0, "full_step")

    def advance_to(self, steps: int) -> None:
        while self.k < steps:
            act = seeded_actions(self.seed, self.k, self.n)
            _step_async(self.dut, act)
            self.ref.step(act[self.sample], self.fs, 8, "full_step", threads=8)
            if self.render:
                self.ref.render(packed=self.render == "packed", threads=8)
            self.k += 1
            if self.k % self.every == 0 or self.k == 1:
                self.inv.check(self.dut, self.k, self.tag)
                _compare_sample(self.dut, self.ref, self.sample, f"{self.tag} step {self.k}", self.render)

    def close(self) -> None:
        self.dut.close()
        self.ref.close()


@pytest.fixture(scope="module")
def c2_run(carts, bootstub):
    require_gpu()
    run = SampledRun(carts["c2"], bootstub, 16384, 24, 1, "c2-long", every=50)
    yield run
    run.close()


@pytest.mark.parametrize("part", range(5))
def test_c2_long_trace(c2_run, part):
    """C2's 1,000 steps at 16,384 envs, 200 per test."""
    c2_run.advance_to(200 * (part + 1))


def test_c4_mbc1_long_trace_at_target_shape(carts, bootstub):
    """C4 at 131,072 envs, frameskip 24, 200 steps (4,800 frames)."""
    require_gpu()
    run = SampledRun(carts["c4"], bootstub, 131072, 24, 3, "c4-long", every=25, sample_size=8)
    try:
        run.advance_to(200)
    finally:
        run.close()


def test_c3_packed_render_long_trace(carts, bootstub):
    """C3 at 16,384 envs, frameskip 24, packed 72x80 render every step, 240
    steps: the SCX/SCY walk table wraps (256 entries, one per frame)."""
    require_gpu()
    run = SampledRun(carts["c3"], bootstub, 16384, 24, 2, "c3-long", every=40, render="packed")
    try:
        run.advance_to(240)
    finally:
        run.close()


def test_c5_full_trace_with_restores(carts, bootstub):
    """2,000 steps at 131,072 envs: step, unpacked render, ~1% masked restore
    from the step-0 snapshot of env 0, 32-byte RAM-sense gather."""
    require_gpu()
    import torch

    from gbxcule_amd.reset_cache import ResetCache

    n, fs, seed, steps, every = 131072, 24, 5, 2000, 250
    rom = carts["c5"]
    rng = np.random.default_rng(seed)
    masks = np.zeros((steps, n), dtype=bool)  # 262 MB; drawn a row at a time
    for k in range(1, steps):
        masks[k] = rng.random(n) < 0.01
    counts = masks.sum(0)
    addrs = np.sort(rng.choice(np.arange(0xC000, 0xE000), 32, replace=False)).astype(np.int32)
    addrs[:4] = (0xFF40, 0xFF44, 0xFF0F, 0xFFFF)
    many = np.nonzero(counts >= 3)[0]
    pick = [0, n - 1] + rng.choice(many, 3, replace=False).tolist() + rng.choice(n, 3, replace=False).tolist()
    sample = np.unique(np.array(pick, dtype=np.int64))
    dut = _backend(rom, bootstub, n, fs, "unpacked")
    ref = RefMachine(sample.size, rom, bootstub)
    inv = FrameInvariants(fs)
    try:
        dut.reset(seed=0)
        ref.step(None, 0, 0, "full_step")
        cache = None
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            if k > 0:
                cache.apply_mask_torch(torch.from_numpy(masks[k].astype(np.uint8)).cuda())
                ref.masked_reset(masks[k][sample].astype(np.uint8))
            _step_async(dut, act)
            ref.step(act[sample], fs, 8, "full_step", threads=8)
            ref.render(packed=False, threads=8)
            senses = dut.ram_senses_torch(addrs)
            if k == 0:
                cache = ResetCache.from_backend(dut, env_idx=0)
                ref.snapshot(0, with_pix=True)  # sample index 0 is env 0
            if (k + 1) % every == 0:
                print(f"c5 full trace: step {k + 1}/{steps}", flush=True)
                inv.prev = None  # restores rewrite the counters: the LY invariant only
                inv.check(dut, k + 1, "c5")
                _compare_sample(dut, ref, sample, f"c5 step {k + 1}", "unpacked")
                np.testing.assert_array_equal(senses.cpu().numpy()[sample], ref.mem[:, addrs])
        assert int(counts[sample].max()) >= 3
    finally:
        dut.close()
        ref.close()


def test_mbc3_rtc_carries_minutes(carts, bootstub):
    require_gpu()
    n, fs, seed, steps, every = 8192, 24, 4, 200, 50
    rom = carts["c4m3"]
    rng = np.random.default_rng(seed)
    sample = np.unique(np.concatenate([[0, n - 1], rng.choice(n, 6, replace=False)])).astype(np.int64)
    dut = _backend(rom, bootstub, n, fs, None)
    ref = RefMachine(sample.size, rom, bootstub)
    inv = FrameInvariants(fs)
    try:
        dut.reset(seed=seed)
        ref.step(None, 0, 0, "full_step")
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            _step_async(dut, act)
            ref.step(act[sample], fs, 8, "full_step", threads=8)
            if (k + 1) % every == 0:
                print(f"mbc3 rtc: step {k + 1}/{steps}", flush=True)
                inv.check(dut, k + 1, "mbc3")
                _compare_sample(dut, ref, sample, f"mbc3 step {k + 1}")
        cs = dut.export_cart_state()
        assert int(cs[:, CS_RTC_MINUTES].min()) >= 1, "the RTC never carried into minutes"
        assert (cs[sample] == ref.cart_state).all()
        # nothing writes the clock here: every env's clock is its cycle count
        # since power-on in whole seconds (4,194,304 cycles), taken apart
        cyc = dut.export_field("cycle_count").astype(np.int64)
        secs = cyc // 4194304
        np.testing.assert_array_equal(cs[:, CS_RTC_SECONDS], secs % 60)
        np.testing.assert_array_equal(cs[:, CS_RTC_MINUTES], secs // 60 % 60)
        np.testing.assert_array_equal(cs[:, CS_RTC_LAST_CYCLE], cyc % 4194304)
    finally:
        dut.close()
        ref.close()


def serial_cart() -> bytes:
    """Sends 8 bytes over the serial port every frame, more than the
    1,024-byte capture buffer holds after 128 frames."""
    from gbxcule_amd.carts.asm import Asm
    from gbxcule_amd.carts.synth import PROGRAM_ORIGIN, _vectors, finalize_rom

    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)
    a.ld_r_d8("B", 0)
    a.label("loop")
    a.label("w1")
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", 144)
    a.jr("w1", "NZ")
    a.ld_r_d8("C", 8)
    a.label("send")
    a.ld_r_r("A", "B")
    a.ldh_a8_a(0x01)  # SB
    a.ld_r_d8("A", 0x81)
    a.ldh_a8_a(0x02)  # SC: start, internal clock
    a.inc_r("B")
    a.dec_r("C")
    a.jr("send", "NZ")
    a.label("w2")
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", 145)
    a.jr("w2", "NZ")
    a.jp("loop")
    rom = bytearray(0x8000)
    _vectors(rom)
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD SERIAL", 0x00, 0x00, 0x00)


def test_serial_buffer_overflow(bootstub):
    require_gpu()
    n, fs, steps = 64, 24, 8
    rom = serial_cart()
    dut = _backend(rom, bootstub, n, fs, None)
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=0)
        ref.step(None, 0, 0, "full_step")
        for k in range(steps):
            act = seeded_actions(9, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "full_step", threads=8)
            assert_same_state(dut, ref, step=k, tag="serial")
        assert int(ref.field("serial_len").min()) == 1024
        assert int(ref.field("serial_overflow").min()) == 1
    finally:
        dut.close()
        ref.close()
