"""``gbx_export_env_noalloc`` (the export entry point that allocates nothing)
against ``gbx_export_env``, through the C ABI.

Two calls in a row share the static device scratch: the first exports an env
of a cart with 32 KiB of cart RAM, the second an env of a ROM-only cart,
whose image is smaller, so bytes the first call left in the scratch must not
reach the second call's outputs.  A third call returns to the first context
with another env.  A cart with 128 KiB of cart RAM is rejected with a clear
error instead.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from gbxcule_amd.carts.synth import seeded_actions

from ._isa import flat_rom
from .conftest import require_gpu

pytestmark = pytest.mark.gpu


def _export(backend, fn: str, env: int):
    from gbxcule_amd import _lib

    lib = _lib.load()
    ram = backend._info(_lib.INFO_RAM_BYTES)
    scalars = np.full(len(_lib.FIELDS), -7, np.int64)
    cart = np.full(20, -7, np.int32)
    mem = np.full(65536, 0xEE, np.uint8)
    cram = np.full(max(ram, 1), 0xEE, np.uint8)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    rc = getattr(lib, fn)(backend.ctx, env, p(scalars), p(cart), p(mem), p(cram) if ram else None)
    _lib.check(rc)
    return scalars, cart, mem, cram[:ram]


def _backend(rom, boot, n):
    from gbxcule_amd.backend import HipVecBackend

    b = HipVecBackend(rom, num_envs=n, frames_per_step=6, release_after_frames=8,
                      stage="emulate_only", bootrom=boot)  # fmt: skip
    b.reset(seed=0)
    return b


def _same(a, b, tag):
    for x, y, name in zip(a, b, ("scalars", "cart_state", "mem", "cart_ram")):
        np.testing.assert_array_equal(x, y, err_msg=f"{tag}: {name}")


def test_noalloc_export_matches_export_twice_then_smaller(carts, bootstub):
    require_gpu()
    big = _backend(carts["c4m3"], bootstub, 200)  # MBC3, 32 KiB cart RAM
    small = _backend(carts["c2"], bootstub, 64)  # ROM-only: no cart RAM
    try:
        for k in range(3):
            big.step(seeded_actions(4, k, 200))
            small.step(seeded_actions(1, k, 64))
        want = _export(big, "gbx_export_env", 137)
        got = _export(big, "gbx_export_env_noalloc", 137)
        _same(got, want, "first call (32 KiB cart RAM)")
        assert want[3].size == 32768 and int(want[0][10]) > 0  # instructions ran
        want = _export(small, "gbx_export_env", 5)
        got = _export(small, "gbx_export_env_noalloc", 5)
        _same(got, want, "second call (smaller image)")
        assert want[3].size == 0
        want = _export(big, "gbx_export_env", 199)
        got = _export(big, "gbx_export_env_noalloc", 199)
        _same(got, want, "third call")
    finally:
        big.close()
        small.close()


def test_noalloc_export_rejects_images_over_the_scratch(bootstub):
    require_gpu()
    from gbxcule_amd import _lib

    rom = flat_rom({0x150: bytes([0x18, 0xFE])}, cart_type=0x13, ram_code=0x04)  # 128 KiB RAM
    b = _backend(rom, bootstub, 2)
    try:
        with pytest.raises(ValueError, match="static scratch"):
            _export(b, "gbx_export_env_noalloc", 1)
        lib = _lib.load()
        assert b"exceeds" in lib.gbx_last_error()
        _export(b, "gbx_export_env", 1)  # the allocating entry point still serves it
    finally:
        b.close()
