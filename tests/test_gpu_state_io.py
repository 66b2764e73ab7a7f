"""Savestates on the device: the one-env image entry points of the C ABI
(``gbx_export_env`` / ``gbx_import_env``) and the backend's
save_state / load_state / *_file methods, against the oracle.

Mirrors the reference's ``tests/test_state_io.py``: save, run on, restore
and compare; file round trips; state transfer between two backends that then
stay in step.  Beyond it, the loaded env is stepped on the HIP backend and on
the oracle from the same loaded state and compared bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.synth import seeded_actions
from oracle.ref import RefMachine

from ._parity import assert_same_state, ref_export_env, ref_import_env
from .conftest import require_gpu

pytestmark = pytest.mark.gpu


def _backend(rom, boot, n, fs=24):
    from gbxcule_amd.backend import HipVecBackend

    return HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=8,
                         stage="full_step", bootrom=boot)  # fmt: skip


def _same_image(a, b, tag):
    np.testing.assert_array_equal(a.scalars, b.scalars, err_msg=f"{tag} scalars")
    np.testing.assert_array_equal(a.cart_state, b.cart_state, err_msg=f"{tag} cart state")
    np.testing.assert_array_equal(a.mem, b.mem, err_msg=f"{tag} memory")
    np.testing.assert_array_equal(a.cart_ram, b.cart_ram, err_msg=f"{tag} cart RAM")


@pytest.mark.parametrize("cart", ["c4m3", "c3"])
def test_env_image_roundtrip(carts, bootstub, cart):
    """export_env reads exactly env k; import_env writes exactly env k (and
    the latches when given), leaving every other env untouched."""
    require_gpu()
    from gbxcule_amd.state_io import FIELDS

    n = 130  # three 64-env blocks, the last one partial
    dut = _backend(carts[cart], bootstub, n)
    ref = RefMachine(n, carts[cart], bootstub)
    rng = np.random.default_rng(7)
    try:
        dut.reset(seed=0)
        ref.step(None, 0, 0, "full_step")
        act = seeded_actions(3, 0, n)
        dut.step(act)
        ref.step(act, 24, 8, "full_step", threads=8)
        for k in (0, 70, 129):
            _same_image(dut.export_env(k), ref_export_env(ref, k), f"export env {k}")
        before_mem = dut.export_memory()
        before_f = {f: dut.export_field(f) for f in FIELDS}
        before_cs = dut.export_cart_state()
        before_cr = dut.export_cart_ram()
        k = 70
        img = dut.export_env(k)
        img.scalars[:] = rng.integers(0, 1 << 16, img.scalars.size)
        img.cart_state[:] = rng.integers(0, 4, img.cart_state.size)
        img.mem[:] = rng.integers(0, 256, img.mem.size, dtype=np.uint8)
        img.cart_ram[:] = rng.integers(0, 256, img.cart_ram.size, dtype=np.uint8)
        img.latches = rng.integers(0, 256, (9, 144), dtype=np.uint8)
        dut.import_env(k, img)
        back = dut.export_env(k)
        _same_image(back, img, "import")
        np.testing.assert_array_equal(dut.export_latches(), img.latches)
        others = np.arange(n) != k
        np.testing.assert_array_equal(dut.export_memory()[others], before_mem[others])
        np.testing.assert_array_equal(dut.export_cart_state()[others], before_cs[others])
        if img.cart_ram.size:
            np.testing.assert_array_equal(dut.export_cart_ram()[others], before_cr[others])
        for f in FIELDS:
            np.testing.assert_array_equal(dut.export_field(f)[others], before_f[f][others], f)
    finally:
        dut.close()
        ref.close()


@pytest.mark.parametrize("cart", ["c4m3", "c3", "c2"])
def test_savestate_load_then_step_parity(carts, bootstub, tmp_path, cart):
    """Save env 5 after two steps, write it to a file, load the file into
    env 9 on both machines, then keep stepping: identical state throughout."""
    require_gpu()
    from gbxcule_amd.abi import parse_cartridge_header
    from gbxcule_amd.state_io import (
        apply_state_to_image,
        load_pyboy_state,
        state_from_image,
    )

    n, fs = 64, 24
    rom = carts[cart]
    dut = _backend(rom, bootstub, n, fs)
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=0)
        ref.step(None, 0, 0, "full_step")
        for s in range(2):
            act = seeded_actions(11, s, n)
            dut.step(act)
            ref.step(act, fs, 8, "full_step", threads=8)
        st = dut.save_state(5)
        assert st == state_from_image(ref_export_env(ref, 5))
        path = tmp_path / f"{cart}.state"
        dut.save_state_file(str(path), env_idx=5)
        dut.load_state_file(str(path), env_idx=9)
        ram = parse_cartridge_header(rom).ram_byte_length
        loaded = load_pyboy_state(path, expected_cart_ram_size=ram)
        img = ref_export_env(ref, 9)
        apply_state_to_image(loaded, img)
        ref_import_env(ref, 9, img)
        assert_same_state(dut, ref, step=-1, tag=f"{cart} loaded")
        np.testing.assert_array_equal(dut.export_latches(), ref.latches)
        for s in range(2, 5):
            act = seeded_actions(11, s, n)
            dut.step(act)
            ref.step(act, fs, 8, "full_step", threads=8)
            assert_same_state(dut, ref, step=s, tag=f"{cart} after load")
            np.testing.assert_array_equal(dut.export_latches(), ref.latches)
        assert int(ref.field("instr_count")[9]) > 0
    finally:
        dut.close()
        ref.close()


def test_save_run_restore_and_transfer(carts, bootstub, tmp_path):
    """The reference's method tests: restore after running on, file round
    trip, and two backends kept in step after a state transfer."""
    require_gpu()
    rom = carts["c4"]
    a = _backend(rom, bootstub, 4, fs=1)
    b = _backend(rom, bootstub, 4, fs=1)
    try:
        a.reset(seed=0)
        b.reset(seed=0)
        zeros = np.zeros(4, dtype=np.int32)
        for _ in range(10):
            a.step(zeros)
        saved = a.save_state(0)
        assert saved.version == 9 and len(saved.vram) == 8192 and len(saved.hram) == 127
        for _ in range(50):
            a.step(zeros)
        assert a.save_state(0).div_counter != saved.div_counter or a.save_state(0).pc != saved.pc
        a.load_state(saved, env_idx=0)
        back = a.save_state(0)
        for f in ("a", "f", "sp", "pc", "ime", "halted", "vram", "wram", "hram"):
            assert getattr(back, f) == getattr(saved, f), f
        path = tmp_path / "a.state"
        a.save_state_file(str(path), env_idx=0)
        assert path.stat().st_size > 130000
        for _ in range(20):
            a.step(zeros)
        a.load_state_file(str(path), env_idx=0)
        assert a.save_state(0).pc == saved.pc
        # transfer env 0 of a into env 2 of b; both then run in step
        b.load_state(a.save_state(0), env_idx=2)
        s1, s2 = a.save_state(0), b.save_state(2)
        for f in ("a", "f", "pc", "sp", "vram", "wram"):
            assert getattr(s1, f) == getattr(s2, f), f
        for _ in range(10):
            a.step(zeros)
            b.step(zeros)
        s1, s2 = a.save_state(0), b.save_state(2)
        assert (s1.pc, s1.a, s1.wram) == (s2.pc, s2.a, s2.wram)
        with pytest.raises(ValueError):
            a.save_state(4)
    finally:
        a.close()
        b.close()
