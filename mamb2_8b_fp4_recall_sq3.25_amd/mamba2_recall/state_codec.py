"""Packed recurrent StateQuant cache (sq3p25) and the FP16-carry control (s16).

Drop-in for the reference's mamba2_recall/state_codec.py: same names,
signatures, in-place semantics and exceptions.  The scans run the gfx950
HIP kernels of libm2r_hip.so:
  sq3p25 -> m2r_state_step_legacy (reference _sq_scan, state_codec.py:105-176)
  s16    -> m2r_state_step_s16    (reference _s16_scan, state_codec.py:65-102)
Every token reads out its FP32 update before the carry is quantized (sq3p25)
or rounded to FP16 (s16).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native, _packed

MODES = ("s16", "sq3p25")
RP = 16
S16_TILE = 4
N = 128


@dataclass
class PackedState:
    """Named device buffers of one layer's carry (state_codec.py:29-48)."""
    mode: str
    tensors: dict
    shape: tuple

    @property
    def nbytes(self):
        storages = {(t.device, t.untyped_storage().data_ptr()): t.untyped_storage().nbytes()
                    for t in self.tensors.values()}
        return sum(storages.values())

    def clone(self):
        return PackedState(self.mode, {k: v.clone() for k, v in self.tensors.items()}, self.shape)

    def zero_(self):
        for value in self.tensors.values():
            value.zero_()
        return self


def allocate_state(batch, heads, dim, dstate, mode, device):
    """state_codec.py:51-62: zeroed, exact-size buffers."""
    if mode not in MODES or dstate != N or min(batch, heads, dim) <= 0:
        raise ValueError("Require s16/sq3p25, dstate=128, and positive geometry")
    shape = (batch, heads, dim, dstate)
    if mode == "s16":
        tensors = {"state": torch.zeros(shape, dtype=torch.float16, device=device)}
    else:
        tensors = {key: torch.zeros((batch, heads, dim, size), dtype=torch.uint8, device=device)
                   for key, size in (("lo", 8), ("hi", 8), ("q4", 32))}
        tensors.update({key: torch.zeros((batch, heads, dim), dtype=torch.float16, device=device)
                        for key in ("s8", "s4")})
    return PackedState(mode, tensors, shape)


def validate_permutation(permutation, groups):
    """state_codec.py:179-184."""
    if permutation is None or permutation.dtype != torch.uint8 or tuple(permutation.shape) != (groups, N):
        raise ValueError("Permutation must be uint8[groups,128]")
    expected = torch.arange(N, device=permutation.device).expand(groups, N)
    if not torch.equal(permutation.long().sort(-1).values, expected):
        raise ValueError("Each permutation row must contain 0..127 exactly once")


def _validate_state(state, device):
    """state_codec.py:187-200."""
    if not isinstance(state, PackedState) or state.mode not in MODES:
        raise ValueError("Invalid packed state")
    b, h, p, n = state.shape
    spec = ({"state": (state.shape, torch.float16)} if state.mode == "s16" else {
        "lo": ((b, h, p, 8), torch.uint8), "hi": ((b, h, p, 8), torch.uint8),
        "q4": ((b, h, p, 32), torch.uint8), "s8": ((b, h, p), torch.float16),
        "s4": ((b, h, p), torch.float16)})
    if n != N or set(state.tensors) != set(spec):
        raise ValueError("State keys or geometry differ")
    for key, (shape, dtype) in spec.items():
        t = state.tensors[key]
        if tuple(t.shape) != tuple(shape) or t.dtype != dtype or t.device != device or not t.is_contiguous():
            raise ValueError(f"Invalid state buffer {key}")


@torch.no_grad()
def scan(x, dt, A, B, C, D, dt_bias, state, permutation=None, collect_stats=False):
    """Mutate the carry for every token; return (FP16 readouts, statistics).

    Inputs: x[B,L,H,P], dt[B,L,H], B/C[B,L,G,128] in FP16; A[H] FP32,
    D[H] and dt_bias[H] FP16/FP32.  Inputs may be views (copied contiguous).
    Statistics (s16 only) are sums of |FP16 carry| over tokens and the 16
    rows of each P tile, shape [B,H,ceil(P/16),128] (state_codec.py:242-261).
    """
    if not isinstance(x, torch.Tensor) or x.ndim != 4 or x.dtype != torch.float16 or not x.is_cuda:
        raise ValueError("x must be CUDA FP16[batch,tokens,heads,dim]")
    b, length, h, p = x.shape
    if length < 1 or state.shape != (b, h, p, N):
        raise ValueError("Positive sequence length and matching state required")
    _validate_state(state, x.device)
    _packed.check_inputs(x, dt, A, B, C, D, dt_bias, state.shape)
    g = B.shape[2]
    if collect_stats and state.mode != "s16":
        raise ValueError("Calibration statistics require s16")
    if state.mode == "sq3p25":
        if (permutation is None or permutation.dtype != torch.uint8 or tuple(permutation.shape) != (g, N)
                or permutation.device != x.device):
            raise ValueError("SQ requires CUDA uint8[groups,128] permutation")
        y = _packed.launch_packed("legacy", x, dt, A, B, C, D, dt_bias, permutation, state.tensors,
                                  n8=16, n4=64, nz=48)
        return y, None
    if permutation is not None:
        raise ValueError("s16 does not accept a permutation")
    x, dt, A, B, C, D, dt_bias = (v.contiguous() for v in (x, dt, A, B, C, D, dt_bias))
    y = torch.empty_like(x)
    tiles = (p + RP - 1) // RP
    stats = torch.zeros((b, h, tiles, N), device=x.device, dtype=torch.float32) if collect_stats else None
    ptr = _native.ptr
    with torch.cuda.device(x.device):
        _native.call("m2r_state_step_s16", ptr(x), ptr(dt), ptr(A), ptr(B), ptr(C), ptr(D),
                     int(D.dtype == torch.float32), ptr(dt_bias), int(dt_bias.dtype == torch.float32),
                     ptr(state.tensors["state"]), ptr(y), ptr(stats), b, length, h, p, g, _native.stream_of(x))
    return y, stats


@torch.no_grad()
def decode_state(state, permutation=None):
    """Diagnostic full FP32 decode (state_codec.py:269-296).

    sq3p25 returns packed-order coordinates (last 48 zero) unless a [G,128]
    permutation is supplied, in which case original coordinates.
    """
    if state.mode == "s16":
        return state.tensors["state"].float()
    if state.mode != "sq3p25":
        raise ValueError("Unsupported mode")
    values = _packed.decode_rows(state.tensors, 16, 64, shape=state.shape)
    if permutation is None:
        return values
    g = permutation.shape[0]
    validate_permutation(permutation, g)
    if state.shape[1] % g:
        raise ValueError("Invalid grouping")
    return _packed.scatter_permutation(values, permutation)


@torch.no_grad()
def encode_state_(state, dense_permuted):
    """Diagnostic initialization (state_codec.py:299-331): FP32 denominators
    amax/127 and amax/7 floored at 1e-8, codes sign(z)*floor(|z|+0.5) with
    z = v/den, clamped; stored scales are half(den)."""
    if tuple(dense_permuted.shape) != state.shape or not bool(torch.isfinite(dense_permuted).all()):
        raise ValueError("Diagnostic input must be finite and match state shape")
    if state.mode == "s16":
        state.tensors["state"].copy_(dense_permuted)
        return state
    if state.mode != "sq3p25":
        raise ValueError("Unsupported mode")
    v = dense_permuted.float().contiguous()
    _native.require_device(v, "dense state")
    # the reference rejects FP16-overflowing scales before writing anything
    s8 = (v[..., :16].abs().amax(-1) / 127.).clamp_min(1e-8)
    s4 = (v[..., 16:80].abs().amax(-1) / 7.).clamp_min(1e-8)
    if not bool(torch.isfinite(s8.half()).all() & torch.isfinite(s4.half()).all()):
        raise ValueError("Scale exceeds FP16 range")
    b, h, p, _ = state.shape
    t = state.tensors
    ptr = _native.ptr
    with torch.cuda.device(v.device):
        _native.call("m2r_state_encode_legacy", ptr(v), ptr(t["lo"]), ptr(t["hi"]), ptr(t["q4"]), ptr(t["s8"]),
                     ptr(t["s4"]), b * h * p, _native.stream_of(v))
    return state
