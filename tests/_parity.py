"""Comparison helpers: HIP backend state vs the oracle, field by field."""

from __future__ import annotations

import numpy as np

from oracle.ref import SCALAR_FIELDS


def assert_same_state(dut, ref, *, step: int, tag: str, mem: bool = True) -> None:
    """Every per-env scalar, the cart state, cart RAM, serial bytes and
    (optionally) the full 64 KiB memory image must be identical."""
    for name in SCALAR_FIELDS:
        got = dut.export_field(name)
        want = ref.field(name).astype(np.int64)
        if not np.array_equal(got, want):
            bad = np.nonzero(got != want)[0]
            i = int(bad[0])
            raise AssertionError(
                f"[{tag} step {step}] field {name}: {len(bad)} envs differ; "
                f"env {i}: hip={got[i]} oracle={want[i]} "
                f"(pc hip={dut.export_field('pc')[i]:#x} oracle={ref.field('pc')[i]:#x})"
            )
    cs = dut.export_cart_state()
    if not np.array_equal(cs, ref.cart_state):
        bad = np.argwhere(cs != ref.cart_state)
        e = int(bad[0][0])
        raise AssertionError(
            f"[{tag} step {step}] cart_state differs in {len(bad)} slots, first at "
            f"{bad[:5].tolist()}; env {e}: hip={cs[e].tolist()} oracle={ref.cart_state[e].tolist()}"
        )
    cr = dut.export_cart_ram()
    if not np.array_equal(cr, ref.cart_ram):
        bad = np.argwhere(cr != ref.cart_ram)
        raise AssertionError(f"[{tag} step {step}] cart_ram differs at {bad[:5].tolist()}")
    if not np.array_equal(dut.export_serial(), ref.serial_buf):
        raise AssertionError(f"[{tag} step {step}] serial buffer differs")
    if mem:
        got = dut.export_memory()
        if not np.array_equal(got, ref.mem):
            bad = np.argwhere(got != ref.mem)
            e, a = (int(x) for x in bad[0])
            raise AssertionError(
                f"[{tag} step {step}] memory differs in {len(bad)} bytes; first env {e} "
                f"addr {a:#06x}: hip={got[e, a]:#04x} oracle={ref.mem[e, a]:#04x}"
            )


def ref_export_env(ref, env: int):
    """The oracle's env ``env`` as an ``EnvImage`` (what ``gbx_export_env``
    returns for the HIP backend)."""
    from gbxcule_amd.abi import parse_cartridge_header
    from gbxcule_amd.state_io import FIELDS, EnvImage

    # a cart without RAM still has a 1-byte dummy slot per env in the oracle
    ram = parse_cartridge_header(ref._rom.tobytes()).ram_byte_length
    return EnvImage(
        scalars=np.array([int(ref.field(n)[env]) for n in FIELDS], dtype=np.int64),
        cart_state=ref.cart_state[env].copy(),
        mem=ref.mem[env].copy(),
        cart_ram=ref.cart_ram[env, :ram].copy() if ram else np.zeros(0, np.uint8),
    )


def ref_import_env(ref, env: int, img) -> None:
    """Write an ``EnvImage`` into the oracle, as ``gbx_import_env`` does on the
    device (cart RAM and latches only when the image carries them)."""
    from gbxcule_amd.state_io import FIELDS

    for i, n in enumerate(FIELDS):
        v = ref.field(n)
        v[env] = np.array(img.scalars[i]).astype(v.dtype)
    ref.cart_state[env] = img.cart_state
    ref.mem[env] = img.mem
    if img.cart_ram.size:
        ref.cart_ram[env, : img.cart_ram.size] = img.cart_ram
    if img.latches is not None:
        ref.latches[:] = img.latches
