"""Layout constants, cartridge header parsing and the action codec.

These are the values the emulator core and its callers agree on.  They mirror
the reference's pure-core modules:

* ``src/gbxcule/core/abi.py:33-56`` (memory size, screen, downsample, packed
  bytes, scanline length),
* ``src/gbxcule/core/cartridge.py:9-76, 139-187`` (cart types, ROM/RAM size
  codes, ``CART_STATE_*`` slot indices, header parsing),
* ``src/gbxcule/core/action_codec.py:39-134`` (8-action codec).

The device-side layout of this build differs from the reference (memory is
interleaved in blocks of 64 envs); the constants below describe the logical
Game Boy state, which is identical.
"""

from __future__ import annotations

from dataclasses import dataclass

MEM_SIZE = 65_536
OBS_DIM_DEFAULT = 32
SERIAL_MAX = 1024
SCREEN_W = 160
SCREEN_H = 144
DOWNSAMPLE_W = SCREEN_W // 2
DOWNSAMPLE_H = SCREEN_H // 2
DOWNSAMPLE_W_BYTES = DOWNSAMPLE_W // 4
PACKED_FRAME_BYTES = DOWNSAMPLE_H * DOWNSAMPLE_W_BYTES
CYCLES_PER_SCANLINE = 456
CYCLES_PER_FRAME = 70_224
LINES_PER_FRAME = 154
ROM_LIMIT = 0x8000
BOOTROM_SIZE = 0x100
CART_ROM_BANK_SIZE = 0x4000
CART_RAM_BANK_SIZE = 0x2000

# Envs per interleave block of the device memory image (one wavefront).
ENV_BLOCK = 64

MBC_KIND_ROM_ONLY = 0
MBC_KIND_MBC1 = 1
MBC_KIND_MBC3 = 2

# Per-env cartridge state slots (reference core/cartridge.py:55-76).
CART_STATE_STRIDE = 20
CART_STATE_FIELDS = (
    "mbc_kind",
    "ram_enable",
    "rom_bank_lo",
    "rom_bank_hi",
    "ram_bank",
    "bank_mode",
    "bootrom_enabled",
    "rtc_select",
    "rtc_latch",
    "rtc_seconds",
    "rtc_minutes",
    "rtc_hours",
    "rtc_days_low",
    "rtc_days_high",
    "rtc_last_cycle",
    "rtc_latched_seconds",
    "rtc_latched_minutes",
    "rtc_latched_hours",
    "rtc_latched_days_low",
    "rtc_latched_days_high",
)
CART_STATE_INDEX = {name: i for i, name in enumerate(CART_STATE_FIELDS)}

ROM_SIZE_MAP = {
    0x00: 32 * 1024,
    0x01: 64 * 1024,
    0x02: 128 * 1024,
    0x03: 256 * 1024,
    0x04: 512 * 1024,
    0x05: 1024 * 1024,
    0x06: 2 * 1024 * 1024,
    0x07: 4 * 1024 * 1024,
    0x08: 8 * 1024 * 1024,
    0x52: int(1.1 * 1024 * 1024),
    0x53: int(1.2 * 1024 * 1024),
    0x54: int(1.5 * 1024 * 1024),
}
RAM_SIZE_MAP = {
    0x00: 0,
    0x01: 2 * 1024,
    0x02: 8 * 1024,
    0x03: 32 * 1024,
    0x04: 128 * 1024,
    0x05: 64 * 1024,
}
MBC1_TYPES = (0x01, 0x02, 0x03)
MBC3_TYPES = (0x0F, 0x10, 0x11, 0x12, 0x13)
SUPPORTED_TYPES = (0x00,) + MBC1_TYPES + MBC3_TYPES


@dataclass(frozen=True)
class CartridgeSpec:
    """Header fields and derived sizes (reference core/cartridge.py:79-93)."""

    cart_type: int
    mbc_kind: int
    rom_size_code: int
    rom_byte_length: int
    rom_bank_count: int
    rom_bank_mask: int  # -1 when the bank count is not a power of two
    ram_size_code: int
    ram_byte_length: int
    ram_bank_count: int


def parse_cartridge_header(rom: bytes) -> CartridgeSpec:
    """Parse type/size codes at 0x147-0x149 (reference core/cartridge.py:139-187).

    Raises ``ValueError`` for short ROMs and unsupported codes, like the
    reference.
    """
    if len(rom) < 0x150:
        raise ValueError(f"ROM too small for header: {len(rom)} bytes")
    cart_type = rom[0x0147]
    if cart_type not in SUPPORTED_TYPES:
        raise ValueError(f"Unsupported cartridge type: 0x{cart_type:02X}")
    rom_code = rom[0x0148]
    ram_code = rom[0x0149]
    if rom_code not in ROM_SIZE_MAP:
        raise ValueError(f"Unsupported ROM size code: 0x{rom_code:02X}")
    if ram_code not in RAM_SIZE_MAP:
        raise ValueError(f"Unsupported RAM size code: 0x{ram_code:02X}")
    rom_bytes = ROM_SIZE_MAP[rom_code]
    ram_bytes = RAM_SIZE_MAP[ram_code]
    if rom_bytes % CART_ROM_BANK_SIZE:
        raise ValueError(f"Invalid ROM byte length: {rom_bytes}")
    if ram_bytes % CART_RAM_BANK_SIZE:
        raise ValueError(f"Invalid RAM byte length: {ram_bytes}")
    rom_banks = rom_bytes // CART_ROM_BANK_SIZE
    ram_banks = ram_bytes // CART_RAM_BANK_SIZE
    mask = rom_banks - 1 if rom_banks & (rom_banks - 1) == 0 else -1
    if cart_type in MBC1_TYPES:
        kind = MBC_KIND_MBC1
    elif cart_type in MBC3_TYPES:
        kind = MBC_KIND_MBC3
    else:
        kind = MBC_KIND_ROM_ONLY
    return CartridgeSpec(
        cart_type=cart_type,
        mbc_kind=kind,
        rom_size_code=rom_code,
        rom_byte_length=rom_bytes,
        rom_bank_count=rom_banks,
        rom_bank_mask=mask,
        ram_size_code=ram_code,
        ram_byte_length=ram_bytes,
        ram_bank_count=ram_banks,
    )


# Action codec "pokemonred_puffer_v1" (reference core/action_codec.py:81-134).
ACTION_CODEC_ID = "pokemonred_puffer_v1"
ACTION_NAMES = ("NOOP", "A", "B", "START", "UP", "DOWN", "LEFT", "RIGHT")
NUM_ACTIONS = len(ACTION_NAMES)
DPAD_RIGHT, DPAD_LEFT, DPAD_UP, DPAD_DOWN = 1, 2, 4, 8
BUTTON_A, BUTTON_B, BUTTON_SELECT, BUTTON_START = 1, 2, 4, 8
ACTION_DPAD_MASK = (0, 0, 0, 0, DPAD_UP, DPAD_DOWN, DPAD_LEFT, DPAD_RIGHT)
ACTION_BUTTON_MASK = (0, BUTTON_A, BUTTON_B, BUTTON_START, 0, 0, 0, 0)

STAGES = ("emulate_only", "reward_only", "obs_only", "full_step")
STAGE_ID = {name: i for i, name in enumerate(STAGES)}
