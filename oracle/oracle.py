"""ctypes bindings and numpy helpers for the C oracle (test infrastructure).

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg
use this module.  Arrays are numpy; binary16 tensors travel as uint16 bit
patterns.  Each function names the reference code it restates (see the C
file's header for the line ranges).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libm2r_oracle.so"
_lib = None

MODE_LEGACY, MODE_STORED, MODE_RIDGE = 0, 1, 2


def build(force: bool = False) -> Path:
    src = HERE / "m2r_oracle.c"
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < src.stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE), "-B" if force else "libm2r_oracle.so"],
                       check=True, capture_output=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        P, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        _lib.orc_state_step.argtypes = [I, I, I, I] + [P] * 5 + [P, I, P, I] + [P] * 4 + [P] * 7 + [I64] * 5
        _lib.orc_state_step.restype = I
        _lib.orc_dense3_step.argtypes = [I] + [P] * 5 + [P, I, P, I, P, P, P, P] + [I64] * 5
        _lib.orc_dense3_step.restype = I
        _lib.orc_s16_step.argtypes = [P] * 5 + [P, I, P, I] + [P] * 3 + [I64] * 5
        _lib.orc_s16_step.restype = I
        _lib.orc_fp4_decode.argtypes = [I, P, P, F, P, I64, I64]
        _lib.orc_fp4_decode.restype = ctypes.c_uint32
        _lib.orc_unary.argtypes = [P, P, I64, I]
        _lib.orc_stored_quantize_n.argtypes = [P, P, P, I64, I]
        _lib.orc_check_round_identity.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        _lib.orc_check_round_identity.restype = I64
        _lib.orc_check_markstein.argtypes = [ctypes.c_uint64, I64, I, P]
        _lib.orc_check_markstein.restype = I64
        _lib.orc_encode_legacy.argtypes = [P] * 6 + [I64]
        _lib.orc_check_residual_round.argtypes = [ctypes.c_uint64, I64, I, ctypes.c_float, ctypes.c_float, P]
        _lib.orc_check_residual_round.restype = I64
        _lib.orc_check_two_sided_round.argtypes = [ctypes.c_uint64, I64, I, ctypes.c_float, P]
        _lib.orc_check_two_sided_round.restype = I64
        _lib.orc_check_latent_division.argtypes = [ctypes.c_uint64, I]
        _lib.orc_check_latent_division.restype = I64
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def unary(values: np.ndarray, op: int) -> np.ndarray:
    """Elementwise primitive `op` (same numbering as the device probe)."""
    v = np.ascontiguousarray(values, dtype=np.uint32)
    out = np.empty_like(v)
    lib().orc_unary(_p(v), _p(out), v.size, op)
    return out


def stored_quantize(values: np.ndarray, scales_f16_bits: np.ndarray, limit: int) -> np.ndarray:
    """scripts/state_ppl_codec_v6.py:52-61 on CPU."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    s = np.ascontiguousarray(scales_f16_bits, dtype=np.uint16)
    q = np.empty(v.shape, dtype=np.int32)
    lib().orc_stored_quantize_n(_p(v), _p(s), _p(q), v.size, limit)
    return q


def state_step(mode, n8, n4, nz, x, dt, A, B, C, D, dt_bias, perm, basis, lscale, pred, state, L=None):
    """One call of the packed-row scan; mutates `state` (dict of numpy arrays
    lo/hi/q4/latent/s8/s4, f16 as uint16) and returns y (uint16 f16 bits).
    x [B,L,H,P], dt [B,L,H], B/C [B,L,G,128] as uint16; A f32 [H]; D and
    dt_bias either uint16 (f16) or float32 [H]."""
    batch, length, heads, dim = x.shape
    groups = B.shape[2]
    y = np.zeros_like(x)
    d_f32 = int(D.dtype == np.float32)
    db_f32 = int(dt_bias.dtype == np.float32)
    lat = state.get("latent")
    rc = lib().orc_state_step(mode, n8, n4, nz, _p(x), _p(dt), _p(A), _p(B), _p(C), _p(D), d_f32, _p(dt_bias),
                              db_f32, _p(perm), _p(basis), _p(lscale), _p(pred), _p(state["lo"]), _p(state["hi"]),
                              _p(state["q4"]), _p(lat), _p(state["s8"]), _p(state["s4"]), _p(y), batch, length,
                              heads, dim, groups)
    if rc:
        raise ValueError(f"oracle state step rejected the geometry (rc={rc})")
    return y


def dense3_step(table_kind, x, dt, A, B, C, D, dt_bias, table, state):
    """mamba2_recall/state_codec_dense3.py:82-148 on CPU; mutates state
    (codes [B,H,P,3,16] u8, scales [B,H,P,2] uint16)."""
    batch, length, heads, dim = x.shape
    groups = B.shape[2]
    y = np.zeros_like(x)
    rc = lib().orc_dense3_step(table_kind, _p(x), _p(dt), _p(A), _p(B), _p(C), _p(D), int(D.dtype == np.float32),
                               _p(dt_bias), int(dt_bias.dtype == np.float32), _p(table), _p(state["codes"]),
                               _p(state["scales"]), _p(y), batch, length, heads, dim, groups)
    if rc:
        raise ValueError(f"oracle dense3 step rejected the geometry (rc={rc})")
    return y


def s16_step(x, dt, A, B, C, D, dt_bias, state, collect_stats=False):
    """mamba2_recall/state_codec.py:65-102 on CPU; mutates `state` (uint16
    f16 bits [B,H,P,128]) and returns (y uint16 bits, stats f32 or None)."""
    batch, length, heads, dim = x.shape
    groups = B.shape[2]
    y = np.zeros_like(x)
    stats = np.zeros((batch, heads, (dim + 15) // 16, 128), np.float32) if collect_stats else None
    rc = lib().orc_s16_step(_p(x), _p(dt), _p(A), _p(B), _p(C), _p(D), int(D.dtype == np.float32), _p(dt_bias),
                            int(dt_bias.dtype == np.float32), _p(state), _p(y), _p(stats), batch, length, heads,
                            dim, groups)
    if rc:
        raise ValueError(f"oracle s16 step rejected the geometry (rc={rc})")
    return y, stats


def fp4_decode(group, packed, scales, global_scale, rows, cols):
    """mamba2_recall/fp4.py:151-154 plus decode_packet's checks; returns
    (uint16 f16 bits [rows, cols], error bits)."""
    out = np.zeros((rows, cols), dtype=np.uint16)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales)
    err = lib().orc_fp4_decode(group, _p(packed), _p(scales), float(global_scale), _p(out), rows, cols)
    return out, int(err)


def check_round_identity(lo_bits: int, hi_bits: int) -> int:
    return int(lib().orc_check_round_identity(lo_bits, hi_bits))


def check_markstein(seed: int, n_random: int, n_boundary_scales: int):
    """Returns (differing integer codes, differing nonzero normal quotients)."""
    div_bad = ctypes.c_int64(0)
    bad = lib().orc_check_markstein(seed, n_random, n_boundary_scales, ctypes.byref(div_bad))
    return int(bad), int(div_bad.value)


def check_residual_round(seed: int, n_random: int, n_boundary_scales: int, thr8: float, thr4: float):
    """Returns (fast codes that differ from roundf(v / d), pairs sent to the
    exact path)."""
    flagged = ctypes.c_int64(0)
    bad = lib().orc_check_residual_round(seed, n_random, n_boundary_scales, thr8, thr4, ctypes.byref(flagged))
    return int(bad), int(flagged.value)


def check_two_sided_round(seed: int, n_random: int, n_boundary_scales: int, rel: float):
    """Returns (kept two-sided codes that differ from roundf(v / d), cases sent
    to the exact path)."""
    flagged = ctypes.c_int64(0)
    bad = lib().orc_check_two_sided_round(seed, n_random, n_boundary_scales, rel, ctypes.byref(flagged))
    return int(bad), int(flagged.value)


def threads():
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def check_latent_division(seed: int, n_random_per_scale: int) -> int:
    return int(lib().orc_check_latent_division(seed, n_random_per_scale))


def encode_legacy(v):
    """state_codec.py:299-331 (encode_state_, sq3p25) on FP32 rows [..., 128]
    in packed order; returns dict lo, hi [..., 8], q4 [..., 32] (uint8) and
    s8, s4 [...] (binary16 bits)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    lead = v.shape[:-1]
    rows = int(np.prod(lead))
    out = dict(lo=np.zeros(lead + (8,), np.uint8), hi=np.zeros(lead + (8,), np.uint8),
               q4=np.zeros(lead + (32,), np.uint8), s8=np.zeros(lead, np.uint16), s4=np.zeros(lead, np.uint16))
    lib().orc_encode_legacy(_p(v), _p(out["lo"]), _p(out["hi"]), _p(out["q4"]), _p(out["s8"]), _p(out["s4"]), rows)
    return out
