"""Shared validation and launch plumbing for the packed 52-byte state rows.

The three same-byte formats (legacy sq3p25, stored-scale tiers, ridge latent)
run one HIP kernel template; this module turns the reference's tensor
arguments into the C-ABI call.  Validation order and exception types follow
the reference scan() functions:
  mamba2_recall/state_codec.py:212-240, scripts/state_ppl_codec_v10.py:163-184,
  scripts/w4_state_repair_codec_v2.py:108-129,
  scripts/fp4_zero_predictor_codec_v1.py:186-220.
"""
from __future__ import annotations

import torch

from . import _native


def check_inputs(x, dt, A, B, C, D, dt_bias, state_shape):
    """Geometry/dtype checks shared by every packed scan; returns
    (batch, length, heads, dim, groups)."""
    if not isinstance(x, torch.Tensor) or x.ndim != 4 or x.dtype != torch.float16 or not x.is_cuda:
        raise ValueError("x must be CUDA FP16[batch,tokens,heads,dim]")
    batch, length, heads, dim = x.shape
    if length < 1 or tuple(state_shape) != (batch, heads, dim, 128):
        raise ValueError("Positive sequence length and matching state required")
    if B.ndim != 4:
        raise ValueError("B must have four axes")
    groups = B.shape[2]
    if groups < 1 or heads % groups:
        raise ValueError("heads must be divisible by B/C groups")
    shapes = ((dt, (batch, length, heads)), (A, (heads,)), (B, (batch, length, groups, 128)),
              (C, (batch, length, groups, 128)), (D, (heads,)), (dt_bias, (heads,)))
    for t, shape in shapes:
        if tuple(t.shape) != shape or t.device != x.device:
            raise ValueError("Input device/geometry mismatch")
    if A.dtype != torch.float32 or any(t.dtype != torch.float16 for t in (dt, B, C)):
        raise ValueError("A must be FP32; dt/B/C must be FP16")
    if any(t.dtype not in (torch.float16, torch.float32) for t in (D, dt_bias)):
        raise ValueError("D and dt_bias must be FP16 or FP32")
    return batch, length, heads, dim, groups


def launch_packed(kind, x, dt, A, B, C, D, dt_bias, perm, tensors, *, n8, n4, nz,
                  basis=None, lscale=None, pred=None):
    """Run the fused step over all tokens of x; mutates `tensors` in place and
    returns the FP16 readout y (same shape as x).  kind: 'legacy' | 'tier' |
    'ridge'."""
    batch, length, heads, dim = x.shape
    groups = B.shape[2]
    x, dt, A, B, C, D, dt_bias, perm = (v.contiguous() for v in (x, dt, A, B, C, D, dt_bias, perm))
    y = torch.empty_like(x)
    d_f32 = int(D.dtype == torch.float32)
    db_f32 = int(dt_bias.dtype == torch.float32)
    p = _native.ptr
    stream = _native.stream_of(x)
    with torch.cuda.device(x.device):
        common = (p(x), p(dt), p(A), p(B), p(C), p(D), d_f32, p(dt_bias), db_f32, p(perm))
        geo = (batch, length, heads, dim, groups)
        if kind == "ridge":
            # multi-token calls on the small-batch shapes (at most 1024 64-row
            # slots) take a token-record workspace (results identical without)
            ws, ws_bytes = None, 0
            if length > 1 and batch * heads * -(-dim // 64) <= 1024:
                ws_bytes = int(_native.lib().m2r_ridge_records_bytes(batch, length, groups))
                ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=x.device)
            _native.call("m2r_state_step_ridge_ws", *common, p(basis.contiguous()), p(lscale.contiguous()),
                         p(pred.contiguous()), p(tensors["lo"]), p(tensors["hi"]), p(tensors["q4"]),
                         p(tensors["latent"]), p(tensors["s8"]), p(tensors["s4"]), p(y), *geo, n8, n4, nz,
                         p(ws) if ws is not None else None, ws_bytes, stream)
        elif kind == "tier":
            _native.call("m2r_state_step_tier", *common, p(tensors["lo"]), p(tensors["hi"]), p(tensors["q4"]),
                         p(tensors["s8"]), p(tensors["s4"]), p(y), *geo, n8, n4, nz, stream)
        elif kind == "legacy":
            _native.call("m2r_state_step_legacy", *common, p(tensors["lo"]), p(tensors["hi"]),
                         p(tensors["q4"]), p(tensors["s8"]), p(tensors["s4"]), p(y), *geo, stream)
        else:
            raise ValueError("unknown packed kind " + repr(kind))
    return y


def decode_rows(tensors, n8, n4, *, shape):
    """Packed rows -> FP32 [B,H,P,128] in packed lane order (dead tier 0),
    via the HIP decode kernel."""
    lo, hi, q4, s8, s4 = (tensors[k] for k in ("lo", "hi", "q4", "s8", "s4"))
    out = torch.empty(shape, dtype=torch.float32, device=lo.device)
    batch, heads, dim, _ = shape
    p = _native.ptr
    with torch.cuda.device(lo.device):
        _native.call("m2r_state_decode", 0, n8, n4, 128 - n8 - n4, p(lo), p(hi), p(q4), None, p(s8), p(s4),
                     None, p(out), batch, heads, dim, 0, _native.stream_of(lo))
    return out


def scatter_permutation(values, permutation):
    """Packed lane order -> original coordinates: out[..., perm[g, n]] = v[..., n]
    (state_codec.py:290-296)."""
    groups = permutation.shape[0]
    batch, heads, dim, n = values.shape
    if heads % groups:
        raise ValueError("Invalid grouping")
    indices = permutation.long().repeat_interleave(heads // groups, 0)[None, :, None, :].expand(batch, heads, dim, n)
    return torch.zeros_like(values).scatter_(-1, indices, values)
