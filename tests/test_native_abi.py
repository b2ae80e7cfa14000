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


def test_step_shape_hook_accepts_documented_shapes_only():
    """m2r_set_step_shape takes the documented shapes, including (4, 0) (two
    waves per head slot) and (4, -4) (four), rejects the others with a message, and (0, 0)
    restores the automatic choice (no launch, no device)."""
    from mamba2_recall import _native
    lib = _native.lib()
    try:
        for shape in [(1, 1), (4, 1), (4, 2), (4, 4), (8, 2), (4, 0), (4, -2), (4, -4), (0, 0)]:
            assert lib.m2r_set_step_shape(*shape) == 0, shape
        for shape in [(8, 0), (2, 2), (8, 4), (1, 0), (16, 1), (4, -3), (8, -4), (4, -1)]:
            assert lib.m2r_set_step_shape(*shape) != 0, shape
            assert b"step shape" in lib.m2r_last_error()
    finally:
        lib.m2r_set_step_shape(0, 0)
