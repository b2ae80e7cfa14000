"""Dense Q3.25 carry: all 128 coordinates as signed 3-bit codes (-3..3) in
three bit planes (48 B) plus two FP16 half-row scales (4 B).

Drop-in for the reference's mamba2_recall/state_codec_dense3.py.  The scan
runs the gfx950 HIP kernel m2r_state_step_dense3; the table is a per-group
permutation (uint8) or a power-of-two equalizer (int8 exponents in [-8, 8]).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native, _packed

N = 128
TILE = 16
TABLE_KINDS = ("permutation", "equalizer")
MIN_EXPONENT, MAX_EXPONENT = -8, 8


@dataclass
class Dense3State:
    tensors: dict
    shape: tuple
    mode: str = "dense3"

    @property
    def nbytes(self):
        storages = {(v.device, v.untyped_storage().data_ptr()): v.untyped_storage().nbytes()
                    for v in self.tensors.values()}
        return sum(storages.values())

    def clone(self):
        return Dense3State({k: v.clone() for k, v in self.tensors.items()}, self.shape)

    def zero_(self):
        for value in self.tensors.values():
            value.zero_()
        return self


def allocate_state(batch, heads, dim, dstate, device):
    """state_codec_dense3.py:43-50."""
    if dstate != N or min(batch, heads, dim) <= 0:
        raise ValueError("Dense Q3 requires positive geometry and dstate128")
    return Dense3State({"codes": torch.zeros((batch, heads, dim, 3, 16), dtype=torch.uint8, device=device),
                        "scales": torch.zeros((batch, heads, dim, 2), dtype=torch.float16, device=device)},
                       (batch, heads, dim, dstate))


def validate_table(table, groups, kind):
    """state_codec_dense3.py:53-64."""
    if kind not in TABLE_KINDS or not isinstance(table, torch.Tensor):
        raise ValueError("Dense Q3 table kind must be permutation or equalizer")
    dtype = torch.uint8 if kind == "permutation" else torch.int8
    if table.dtype != dtype or tuple(table.shape) != (groups, N):
        raise ValueError("Dense Q3 table dtype or shape differs")
    if kind == "permutation":
        expected = torch.arange(N, device=table.device).expand(groups, N)
        if not torch.equal(table.long().sort(-1).values, expected):
            raise ValueError("Each permutation must contain0..127 exactly")
    elif not bool(((table >= MIN_EXPONENT) & (table <= MAX_EXPONENT)).all()):
        raise ValueError("Power2 exponents must lie in[-8,8]")


def validate_state(state, device):
    """state_codec_dense3.py:67-79."""
    if not isinstance(state, Dense3State) or state.mode != "dense3":
        raise ValueError("Expected a dense Q3 packed state")
    b, h, p, n = state.shape
    spec = {"codes": ((b, h, p, 3, 16), torch.uint8), "scales": ((b, h, p, 2), torch.float16)}
    if n != N or set(state.tensors) != set(spec):
        raise ValueError("Dense Q3 state geometry/keys differ")
    for key, (shape, dtype) in spec.items():
        value = state.tensors[key]
        if (tuple(value.shape) != shape or value.dtype != dtype or value.device != device
                or not value.is_contiguous()):
            raise ValueError("Invalid packed state tensor: " + key)


@torch.no_grad()
def scan(x, dt, A, B, C, D, dt_bias, state, table, table_kind="permutation"):
    """Mutate the packed carry after every token; return the FP16 readout.

    x[B,L,H,P], dt[B,L,H], B/C[B,L,G,128] are FP16; A[H] is FP32.  Equalizer
    mode keeps original coordinates and applies B*2^-k, C*2^k
    (state_codec_dense3.py:151-186).  Table contents are validated once by the
    controller, not here.
    """
    if not isinstance(x, torch.Tensor) or x.ndim != 4 or x.dtype != torch.float16 or not x.is_cuda:
        raise ValueError("x must be CUDA FP16[batch,tokens,heads,dim]")
    b, length, h, p = x.shape
    if length < 1 or state.shape != (b, h, p, N):
        raise ValueError("Positive sequence length and matching state required")
    validate_state(state, x.device)
    if B.ndim != 4 or B.shape[2] < 1 or h % B.shape[2]:
        raise ValueError("Invalid B/C head grouping")
    g = B.shape[2]
    for tensor, shape in ((dt, (b, length, h)), (A, (h,)), (B, (b, length, g, N)), (C, (b, length, g, N)),
                          (D, (h,)), (dt_bias, (h,))):
        if tensor.device != x.device or tuple(tensor.shape) != shape:
            raise ValueError("Input shape/device mismatch")
    if A.dtype != torch.float32 or any(v.dtype != torch.float16 for v in (dt, B, C)):
        raise ValueError("A must be FP32; dt/B/C must be FP16")
    if any(v.dtype not in (torch.float16, torch.float32) for v in (D, dt_bias)):
        raise ValueError("D and dt_bias must be FP16/FP32")
    expected_dtype = torch.uint8 if table_kind == "permutation" else torch.int8
    if (table_kind not in TABLE_KINDS or table.dtype != expected_dtype or tuple(table.shape) != (g, N)
            or table.device != x.device):
        raise ValueError("Dense Q3 table differs")
    x, dt, A, B, C, D, dt_bias, table = (v.contiguous() for v in (x, dt, A, B, C, D, dt_bias, table))
    out = torch.empty_like(x)
    ptr = _native.ptr
    with torch.cuda.device(x.device):
        _native.call("m2r_state_step_dense3", ptr(x), ptr(dt), ptr(A), ptr(B), ptr(C), ptr(D),
                     int(D.dtype == torch.float32), ptr(dt_bias), int(dt_bias.dtype == torch.float32), ptr(table),
                     int(table_kind == "equalizer"), ptr(state.tensors["codes"]), ptr(state.tensors["scales"]),
                     ptr(out), b, length, h, p, g, _native.stream_of(x))
    return out


@torch.no_grad()
def decode_state(state, table=None, table_kind="permutation"):
    """Diagnostic FP32 decode (state_codec_dense3.py:189-212)."""
    validate_state(state, state.tensors["codes"].device)
    codes = state.tensors["codes"]
    b, h, p, _ = state.shape
    value = torch.empty(state.shape, dtype=torch.float32, device=codes.device)
    ptr = _native.ptr
    with torch.cuda.device(codes.device):
        _native.call("m2r_state_decode", 1, 0, 0, 0, ptr(codes), None, None, None, ptr(state.tensors["scales"]),
                     None, None, ptr(value), b, h, p, 0, _native.stream_of(codes))
    if table is None:
        return value
    g = table.shape[0]
    validate_table(table, g, table_kind)
    if h % g or table.device != value.device:
        raise ValueError("Table grouping/device differs")
    expanded = table.repeat_interleave(h // g, 0)[None, :, None, :]
    if table_kind == "equalizer":
        return torch.ldexp(value, expanded.to(torch.int32))
    return _packed.scatter_permutation(value, table)


@torch.no_grad()
def validate_finite_result(state, output=None):
    """state_codec_dense3.py:215-228."""
    validate_state(state, state.tensors["codes"].device)
    if not bool(torch.isfinite(state.tensors["scales"]).all()):
        raise FloatingPointError("Dense Q3 FP16 scale overflow/nonfinite carry")
    if output is not None and not bool(torch.isfinite(output).all()):
        raise FloatingPointError("Dense Q3 nonfinite readout")
    return True
