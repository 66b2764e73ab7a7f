"""Host-side pieces that need no GPU: cartridge header parsing, the synthetic
carts, the action trace generator, the boot stub and backend argument checks."""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.abi import (
    ACTION_BUTTON_MASK,
    ACTION_DPAD_MASK,
    MBC_KIND_MBC1,
    MBC_KIND_MBC3,
    MBC_KIND_ROM_ONLY,
    parse_cartridge_header,
)
from gbxcule_amd.carts.synth import (
    CARTS,
    WORKLOADS,
    global_checksum,
    header_checksum,
    seeded_actions,
)


def _hdr(t, r, ram):
    rom = bytearray(0x8000 << r)
    rom[0x147], rom[0x148], rom[0x149] = t, r, ram
    return bytes(rom)


@pytest.mark.parametrize(
    "t,r,ram,kind,banks,mask,ram_banks",
    [
        (0x00, 0x00, 0x00, MBC_KIND_ROM_ONLY, 2, 1, 0),
        (0x01, 0x04, 0x00, MBC_KIND_MBC1, 32, 31, 0),
        (0x03, 0x05, 0x03, MBC_KIND_MBC1, 64, 63, 4),
        (0x13, 0x06, 0x03, MBC_KIND_MBC3, 128, 127, 4),
        (0x0F, 0x01, 0x02, MBC_KIND_MBC3, 4, 3, 1),
    ],
)
def test_header_parse(t, r, ram, kind, banks, mask, ram_banks):
    """Reference core/cartridge.py:139-187 size tables."""
    spec = parse_cartridge_header(_hdr(t, r, ram))
    assert (spec.mbc_kind, spec.rom_bank_count, spec.rom_bank_mask, spec.ram_bank_count) == (
        kind,
        banks,
        mask,
        ram_banks,
    )


@pytest.mark.parametrize("rom,msg", [(b"\0" * 0x100, "too small"), (_hdr(0x05, 0, 0), "type")])
def test_header_rejects(rom, msg):
    with pytest.raises(ValueError, match=msg):
        parse_cartridge_header(rom)


def test_synthetic_carts_have_valid_checksums(carts):
    for name, rom in carts.items():
        assert rom[0x14D] == header_checksum(rom), name
        assert (rom[0x14E] << 8 | rom[0x14F]) == global_checksum(rom), name
        assert rom[0x100:0x104] == bytes([0x00, 0xC3, 0x50, 0x01])
        parse_cartridge_header(rom)


def test_carts_are_deterministic():
    for name, fn in CARTS.items():
        assert fn() == fn(), name


def test_seeded_actions_is_default_rng_trace():
    """bench/harness.py:236-243: default_rng(seed + step).integers(0, 8, N)."""
    a = seeded_actions(3, 5, 100)
    b = np.random.default_rng(8).integers(0, 8, size=(100,), dtype=np.int32)
    np.testing.assert_array_equal(a, b)
    assert a.dtype == np.int32


def test_action_codec_table():
    """Reference core/action_codec.py:81-134 (NOOP, A, B, START, UP, DOWN,
    LEFT, RIGHT) and JOYP bit positions."""
    assert ACTION_DPAD_MASK == (0, 0, 0, 0, 4, 8, 2, 1)
    assert ACTION_BUTTON_MASK == (0, 1, 2, 8, 0, 0, 0, 0)


def test_workload_sizes_match_configs():
    assert WORKLOADS["c1"].num_envs == 64 and WORKLOADS["c1"].frames_per_step == 4
    assert WORKLOADS["c2"].num_envs == 16_384 and WORKLOADS["c2"].frames_per_step == 24
    assert WORKLOADS["c5"].num_envs == 131_072 and WORKLOADS["c5"].reset_prob == 0.01


def test_backend_rejects_bad_arguments_before_any_gpu_call(carts):
    from gbxcule_amd.backend import HipVecBackend

    with pytest.raises(ValueError, match="obs_dim"):
        HipVecBackend(carts["c1"], num_envs=4, obs_dim=16)
    with pytest.raises(ValueError, match="stage"):
        HipVecBackend(carts["c1"], num_envs=4, stage="bogus")
    be = HipVecBackend(carts["c1"], num_envs=4)
    with pytest.raises(RuntimeError, match="reset"):
        be.step(np.zeros(4, np.int32))
    with pytest.raises(RuntimeError, match="reset"):
        be.get_cpu_state(0)


def test_boot_stub_ends_with_boot_rom_disable(bootstub):
    assert len(bootstub) == 256
    assert bootstub[0xFE:] == bytes([0xE0, 0x50])
