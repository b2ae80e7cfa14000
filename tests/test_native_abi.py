"""The HIP library loads (no GPU needed) and exports every entry point that
include/m2r.h declares; the Python binding knows each of them."""
import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "m2r.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+(m2r_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "m2r_state_step_ridge" in names and "m2r_fp4_decode_g16" in names
    assert len(names) >= 13


def test_library_exports_every_declared_symbol():
    from mamba2_recall import _native
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    from mamba2_recall import _native
    assert set(declared_symbols()) <= set(_native._SIGNATURES)


def test_error_reporting_without_device():
    """Rejected geometry returns nonzero with a message, before any launch."""
    from mamba2_recall import _native
    lib = _native.lib()
    rc = lib.m2r_fp4_decode_g16(None, None, None, None, 0, 16, None, None)
    assert rc != 0
    assert b"non-positive" in lib.m2r_last_error()
