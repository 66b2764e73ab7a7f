"""ctypes binding of ``libgbx_hip.so`` (the C ABI in ``include/gbx_hip.h``).

The library is loaded from ``gbxcule_amd/lib/``.  There is no fallback: if it
is missing or fails to load, every entry point raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libgbx_hip.so"

GBX_OK, GBX_E_INVALID, GBX_E_STATE, GBX_E_HIP, GBX_E_UNSUPPORTED = 0, -1, -2, -3, -4

FIELDS = (
    "pc", "sp", "a", "b", "c", "d", "e", "h", "l", "f",
    "instr_count", "cycle_count", "cycle_in_frame", "trap_flag", "trap_pc",
    "trap_opcode", "trap_kind", "actions", "joyp_select", "serial_len",
    "serial_overflow", "ime", "ime_delay", "halted", "div_counter",
    "timer_prev_in", "tima_reload_pending", "tima_reload_delay",
    "ppu_scanline_cycle", "ppu_ly", "ppu_window_line", "ppu_stat_prev",
)  # fmt: skip
FIELD_ID = {name: i for i, name in enumerate(FIELDS)}

BUF_MEM, BUF_PIX, BUF_PIX_PACKED, BUF_OBS, BUF_REWARD, BUF_ACTIONS, BUF_CART_RAM, BUF_FRAME_BG = range(8)
(
    INFO_NUM_ENVS,
    INFO_PADDED_ENVS,
    INFO_ROM_BANKS,
    INFO_ROM_BANK_MASK,
    INFO_RAM_BANKS,
    INFO_RAM_BYTES,
    INFO_MBC_KIND,
    INFO_OBS_DIM,
    INFO_CART_RAM_STRIDE,
    INFO_STEP_LANES,
) = range(10)

# Every symbol the header declares, with its ctypes signature.
_vp, _i32, _i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
_P64 = ctypes.POINTER(ctypes.c_int64)
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "gbx_last_error": (ctypes.c_char_p, []),
    "gbx_version": (ctypes.c_int, []),
    "gbx_create": (ctypes.c_int, [_i32, _vp, _i64, _vp, _i32, _i32, ctypes.POINTER(_vp)]),
    "gbx_destroy": (ctypes.c_int, [_vp]),
    "gbx_reset": (ctypes.c_int, [_vp, _vp]),
    "gbx_upload_actions": (ctypes.c_int, [_vp, _vp, _vp]),
    "gbx_step": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, _vp]),
    "gbx_render": (ctypes.c_int, [_vp, _vp, _i64, _i32, _vp]),
    "gbx_render_bg_env0": (ctypes.c_int, [_vp, _vp, _vp]),
    "gbx_snapshot": (ctypes.c_int, [_vp, _i32, _i32, _vp]),
    "gbx_masked_reset": (ctypes.c_int, [_vp, _vp, _vp]),
    "gbx_gather_mem": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp]),
    "gbx_read_mem": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "gbx_write_mem": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "gbx_state_hash": (ctypes.c_int, [_vp, _vp, _vp]),
    "gbx_export_scalar": (ctypes.c_int, [_vp, _i32, _vp]),
    "gbx_import_scalar": (ctypes.c_int, [_vp, _i32, _vp]),
    "gbx_export_mem": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _vp]),
    "gbx_import_mem": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i32]),
    "gbx_export_cart_state": (ctypes.c_int, [_vp, _vp]),
    "gbx_import_cart_state": (ctypes.c_int, [_vp, _vp]),
    "gbx_export_cart_ram": (ctypes.c_int, [_vp, _i32, _i32, _vp]),
    "gbx_export_serial": (ctypes.c_int, [_vp, _vp]),
    "gbx_export_latches": (ctypes.c_int, [_vp, _vp]),
    "gbx_export_env": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _vp]),
    "gbx_export_env_noalloc": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _vp]),
    "gbx_import_env": (ctypes.c_int, [_vp, _i32, _vp, _vp, _vp, _vp, _vp]),
    "gbx_buffer": (ctypes.c_int, [_vp, _i32, ctypes.POINTER(_vp), _P64]),
    "gbx_info": (ctypes.c_int, [_vp, _i32, _P64]),
    "gbx_set_debug": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32]),
}

_lib: ctypes.CDLL | None = None


class GbxError(RuntimeError):
    """A HIP runtime failure inside the library."""


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it is absent."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with gbxcule_amd.build.build() "
                "(hipcc --offload-arch=gfx950)"
            )
        # torch bundles its own HIP runtime under the same soname as ROCm's.
        # Loading torch first makes the library bind to that runtime, so the
        # process holds one HIP runtime and device pointers are shared with
        # torch; loading the library first would put ROCm's runtime in place
        # and torch would then find no GPU.
        import torch  # noqa: F401

        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    """Map a library status code to the reference's Python exception types."""
    if rc == GBX_OK:
        return
    msg = (load().gbx_last_error() or b"").decode(errors="replace")
    if rc == GBX_E_INVALID:
        raise ValueError(msg)
    if rc == GBX_E_STATE:
        raise RuntimeError(msg)
    if rc == GBX_E_UNSUPPORTED:
        raise ValueError(msg)
    raise GbxError(msg or f"libgbx_hip error {rc}")
