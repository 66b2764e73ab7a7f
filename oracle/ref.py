"""ctypes driver for the parity oracle (``oracle/lib/libgbx_ref.so``).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``.  The product backend never imports
this module.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "lib" / "libgbx_ref.so"

# Scalar field ids (gbx_ref.h REF_*; identical to gbx_hip.h GBX_FIELD_*).
SCALAR_FIELDS = (
    "pc", "sp", "a", "b", "c", "d", "e", "h", "l", "f",
    "instr_count", "cycle_count", "cycle_in_frame", "trap_flag", "trap_pc",
    "trap_opcode", "trap_kind", "actions", "joyp_select", "serial_len",
    "serial_overflow", "ime", "ime_delay", "halted", "div_counter",
    "timer_prev_in", "tima_reload_pending", "tima_reload_delay",
    "ppu_scanline_cycle", "ppu_ly", "ppu_window_line", "ppu_stat_prev",
)  # fmt: skip
FIELD_ID = {name: i for i, name in enumerate(SCALAR_FIELDS)}
REF_MEM, REF_CART_STATE, REF_CART_RAM, REF_SERIAL_BUF = 100, 101, 102, 103
REF_OBS, REF_REWARD, REF_LATCHES, REF_PIX, REF_PIX_PACKED, REF_DATA_BYTES = (
    104, 105, 106, 107, 108, 109,
)  # fmt: skip
STAGE_ID = {"emulate_only": 0, "reward_only": 1, "obs_only": 2, "full_step": 3}

_lib = None


def build() -> Path:
    """Compile the oracle with ``make`` (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        lib.ref_create.restype = vp
        lib.ref_create.argtypes = [i32, vp, i64, vp, i32, i32]
        lib.ref_destroy.argtypes = [vp]
        lib.ref_reset.argtypes = [vp]
        lib.ref_step.argtypes = [vp, vp, i32, i32, i32, i32, i32, i32]
        lib.ref_render.argtypes = [vp, i32, i32]
        lib.ref_render_bg_env0.argtypes = [vp, vp]
        lib.ref_snapshot_ex.argtypes = [vp, i32, i32]
        lib.ref_masked_reset.argtypes = [vp, vp]
        lib.ref_set_debug.argtypes = [vp, i32, i32, i32, i32]
        lib.ref_field_ptr.restype = vp
        lib.ref_field_ptr.argtypes = [vp, i32, ctypes.POINTER(i64), ctypes.POINTER(i32)]
        _lib = lib
    return _lib


_DTYPES = {1: np.uint8, 4: np.int32, 8: np.int64}


class RefMachine:
    """N Game Boys stepped by the oracle; arrays are live numpy views."""

    def __init__(self, num_envs: int, rom: bytes, boot: bytes, obs_dim: int = 32):
        self._lib = load()
        self._rom = np.frombuffer(rom, dtype=np.uint8).copy()
        self._boot = np.frombuffer(boot, dtype=np.uint8).copy()
        h = self._lib.ref_create(
            num_envs,
            self._rom.ctypes.data,
            len(self._rom),
            self._boot.ctypes.data,
            len(self._boot),
            obs_dim,
        )
        if not h:
            raise ValueError("oracle rejected the cartridge or arguments")
        self._h = ctypes.c_void_p(h)
        self.num_envs = num_envs
        self.obs_dim = obs_dim

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.ref_destroy(self._h)
            self._h = None

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    # -- raw views -----------------------------------------------------------
    def _view(self, field: int, dtype=None) -> np.ndarray:
        nb = ctypes.c_int64()
        es = ctypes.c_int32()
        p = self._lib.ref_field_ptr(self._h, field, ctypes.byref(nb), ctypes.byref(es))
        if not p:
            raise KeyError(field)
        dt = dtype or _DTYPES[es.value]
        count = nb.value // np.dtype(dt).itemsize
        buf = (ctypes.c_char * nb.value).from_address(p)
        return np.frombuffer(buf, dtype=dt, count=count)

    def field(self, name: str) -> np.ndarray:
        return self._view(FIELD_ID[name])

    @property
    def mem(self) -> np.ndarray:
        return self._view(REF_MEM).reshape(self.num_envs, 65536)

    @property
    def cart_state(self) -> np.ndarray:
        return self._view(REF_CART_STATE).reshape(self.num_envs, 20)

    @property
    def cart_ram(self) -> np.ndarray:
        return self._view(REF_CART_RAM).reshape(self.num_envs, -1)

    @property
    def serial_buf(self) -> np.ndarray:
        return self._view(REF_SERIAL_BUF).reshape(self.num_envs, 1024)

    @property
    def obs(self) -> np.ndarray:
        return self._view(REF_OBS, np.float32).reshape(self.num_envs, self.obs_dim)

    @property
    def reward(self) -> np.ndarray:
        return self._view(REF_REWARD, np.float32)

    @property
    def latches(self) -> np.ndarray:
        return self._view(REF_LATCHES).reshape(9, 144)

    @property
    def pix(self) -> np.ndarray:
        return self._view(REF_PIX).reshape(self.num_envs, 72, 80)

    @property
    def pix_packed(self) -> np.ndarray:
        return self._view(REF_PIX_PACKED).reshape(self.num_envs, 72, 20)

    @property
    def data_bytes(self) -> np.ndarray:
        return self._view(REF_DATA_BYTES)

    def scalars(self) -> dict[str, np.ndarray]:
        return {name: self.field(name).copy() for name in SCALAR_FIELDS}

    # -- operations ------------------------------------------------------------
    def reset(self) -> None:
        self._lib.ref_reset(self._h)

    def step(
        self,
        actions: np.ndarray | None,
        frames: int,
        release: int = 8,
        stage: str = "emulate_only",
        env_lo: int = 0,
        env_hi: int | None = None,
        threads: int | None = None,
    ) -> None:
        ptr = None
        if actions is not None:
            actions = np.ascontiguousarray(actions, dtype=np.int32)
            if actions.shape != (self.num_envs,):
                raise ValueError("actions must have shape (num_envs,)")
            ptr = actions.ctypes.data
        if threads is None:
            threads = int(os.environ.get("GBX_REF_THREADS", "1"))
        hi = self.num_envs if env_hi is None else env_hi
        rc = self._lib.ref_step(
            self._h, ptr, frames, release, STAGE_ID[stage], env_lo, hi, threads
        )
        if rc != 0:
            raise RuntimeError("ref_step failed")

    def render(self, packed: bool, threads: int = 1) -> None:
        self._lib.ref_render(self._h, 1 if packed else 0, threads)

    def render_bg_env0(self) -> np.ndarray:
        """Env 0's 160x144 shade frame from its scanline latches."""
        out = np.zeros((144, 160), dtype=np.uint8)
        if self._lib.ref_render_bg_env0(self._h, out.ctypes.data) != 0:
            raise RuntimeError("ref_render_bg_env0 failed")
        return out

    def snapshot(self, env_idx: int = 0, with_pix: bool = False) -> None:
        if self._lib.ref_snapshot_ex(self._h, env_idx, 1 if with_pix else 0) != 0:
            raise ValueError("bad snapshot env")

    def masked_reset(self, mask: np.ndarray) -> None:
        mask = np.ascontiguousarray(mask, dtype=np.uint8)
        if self._lib.ref_masked_reset(self._h, mask.ctypes.data) != 0:
            raise RuntimeError("masked reset without snapshot")

    def set_debug(self, rst38=0, trap_pc=0, max_instr=0, watch_addr=0) -> None:
        self._lib.ref_set_debug(self._h, rst38, trap_pc, max_instr, watch_addr)
