"""The C ABI library loads and exports every function include/gbx_hip.h
declares (no GPU calls)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    text = (ROOT / "include" / "gbx_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gbx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "gbx_step" in names and "gbx_masked_reset" in names
    assert len(names) >= 20


def test_library_exports_every_declared_symbol():
    from gbxcule_amd import _lib

    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"libgbx_hip.so does not export {name}"
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_error_path_without_gpu():
    """Argument checks run before any HIP call and report ValueError text."""
    from gbxcule_amd import _lib

    lib = _lib.load()
    out = ctypes.c_void_p()
    rc = lib.gbx_create(0, None, 0, None, 0, 32, ctypes.byref(out))
    assert rc == _lib.GBX_E_INVALID
    assert b"num_envs" in lib.gbx_last_error()
    assert lib.gbx_step(None, None, 1, 0, 0, None) == _lib.GBX_E_INVALID
