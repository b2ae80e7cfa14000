"""Loader for the gfx950 HIP library (`lib/libm2r_hip.so`) and thin helpers
for calling its C-ABI with torch device tensors.

The library must be present: every codec entry point in this package calls
into it and raises if it is missing.  There is no CPU or Triton fallback.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

PKG_ROOT = Path(__file__).resolve().parents[1]
LIB_PATH = PKG_ROOT / "lib" / "libm2r_hip.so"

_lib = None

P, I, I64, U32P = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
F32 = ctypes.c_float

_SIGNATURES = {
    "m2r_abi_version": ([], I),
    "m2r_last_error": ([], ctypes.c_char_p),
    "m2r_state_step_ridge": ([P] * 5 + [P, I, P, I] + [P] * 4 + [P] * 7 + [I64] * 5 + [I] * 3 + [P], I),
    "m2r_state_step_ridge_ws": ([P] * 5 + [P, I, P, I] + [P] * 4 + [P] * 7 + [I64] * 5 + [I] * 3 + [P, I64, P], I),
    "m2r_ridge_records_bytes": ([I64] * 3, I64),
    "m2r_state_step_tier": ([P] * 5 + [P, I, P, I] + [P] + [P] * 6 + [I64] * 5 + [I] * 3 + [P], I),
    "m2r_state_step_legacy": ([P] * 5 + [P, I, P, I] + [P] + [P] * 6 + [I64] * 5 + [P], I),
    "m2r_state_step_dense3": ([P] * 5 + [P, I, P, I] + [P, I] + [P] * 3 + [I64] * 5 + [P], I),
    "m2r_state_step_s16": ([P] * 5 + [P, I, P, I] + [P] * 3 + [I64] * 5 + [P], I),
    "m2r_state_decode": ([I, I, I, I] + [P] * 7 + [P] + [I64] * 4 + [P], I),
    "m2r_state_encode_legacy": ([P] * 6 + [I64, P], I),
    "m2r_fp4_decode_g16": ([P, P, P, P, I64, I64, P, P], I),
    "m2r_fp4_decode_g64": ([P, P, P, I64, I64, P, P], I),
    "m2r_probe_stored_quantize": ([P, P, P, I64, I, P], I),
    "m2r_probe_unary": ([P, P, I64, I, P], I),
    "m2r_probe_div": ([P, P, P, I64, P], I),
    "m2r_set_fp4_decode_shape": ([I, I, I], I),
    "m2r_stream_probe": ([P, P, I64, I, I, I, I, I, P], I),
    "m2r_stream_probe_phased": ([P, P, I64, I, I, I, I, I, P], I),
    "m2r_probe_butterfly": ([P, P, P], I),
    "m2r_set_step_shape": ([I, I], I),
    "m2r_causal_conv_update": ([P, I64, I64, I64, P, I64, P, P, P, I64, I64, I, I, P], I),
    "m2r_gated_rmsnorm": ([P, I64, P, I64, P, P, I64, I64, I64, I64, F32, P], I),
    "m2r_fp4_gemv_g16": ([P, P, P, P, I64, P, I64, I64, I64, I64, P], I),
    "m2r_state_step_ridge_layers_workspace": ([I], I64),
    "m2r_state_step_ridge_layers": ([P, I, I64, I64, I64, I64, P, I64, P], I),
    "m2r_state_step_ridge_layers_noalloc": ([P, I, I64, I64, I64, I64, P], I),
}


class RidgeLayer(ctypes.Structure):
    """m2r_ridge_layer of include/m2r.h: one layer of the multi-layer step."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("x", "dt", "A", "B", "C", "D", "dt_bias", "perm", "basis", "lscale",
                                                "pred", "lo", "hi", "q4", "latent", "s8", "s4", "y")] + \
               [(n, ctypes.c_int32) for n in ("n8", "n4", "nz", "d_is_f32", "db_is_f32", "reserved")]


class NativeLibraryMissing(RuntimeError):
    pass


def lib():
    """The loaded HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise NativeLibraryMissing(
                f"HIP library {LIB_PATH} is missing; run __graft_entry__.build() "
                "(or python build_lib.py in the package directory) first")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name, None)
            if fn is None:
                continue
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def exported_symbols():
    return [name for name in _SIGNATURES if hasattr(lib(), name)]


def call(name: str, *args):
    """Invoke a C-ABI entry point; nonzero status raises RuntimeError."""
    fn = getattr(lib(), name)
    rc = fn(*args)
    if rc != 0:
        msg = lib().m2r_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """The current HIP stream of `t`'s device, as the C-ABI expects it."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_device(t: torch.Tensor, what: str = "tensor"):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{what} must be a CUDA (HIP) tensor")
