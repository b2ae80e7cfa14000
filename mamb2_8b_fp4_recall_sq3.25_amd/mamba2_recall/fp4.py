"""FP4 (E2M1) weight decode to resident FP16: drop-in for the decode side of
the reference's mamba2_recall/fp4.py.

E2M1 codes 0..7 are [0, .5, 1, 1.5, 2, 3, 4, 6]; bit 3 is the sign; the low
nibble of byte i is column 2i.  G16 stores one E4M3FN block scale per 16
weights and one FP32 whole-matrix scale; decode is
FP16(FP32(FP32(code*block)*global)).  G64 stores one FP16 scale per 64
weights; decode is FP16(FP32(code*scale)).  decode_packet runs the gfx950
HIP kernels (m2r_fp4_decode_g16 / _g64), which also evaluate the
reference's validity conditions in the same pass, so a call costs one
device synchronization instead of four.
"""
from __future__ import annotations

import torch

from . import _native

FORMATS = ("fp4_g64_f16", "fp4_g16_e4m3")
GROUP_SIZES = dict(zip(FORMATS, (64, 16)))
E2M1_MAGNITUDES = (0., .5, 1., 1.5, 2., 3., 4., 6.)
DEFAULT_CHUNK_ROWS = 512
MAX_CHUNK_ELEMENTS = 4_194_304
PARAMETER_COUNT = 8_236_999_680
TENSOR_COUNT = 507
FP4_TENSOR_COUNT = 114

# device error bits of the decode kernels, in the reference's check order
ERR_SCALE = 1 | 2
ERR_GLOBAL = 32
ERR_PADDING = 16
ERR_ZERO_SCALE = 4
ERR_DECODED = 8


def _need(condition, message):
    if not condition:
        raise ValueError(message)


def _format(format_name):
    _need(format_name in FORMATS, "Unknown frozen FP4 format")
    return GROUP_SIZES[format_name]


def _decode_e2m1_codes(codes):
    """fp4.py:100-103 (format helper; not the weight-decode path)."""
    levels = torch.tensor(E2M1_MAGNITUDES, device=codes.device, dtype=torch.float32)
    sign = (1 - 2 * ((codes & 8) != 0).to(torch.int8)).float()
    return levels[(codes & 7).long()] * sign


def decode_e2m1(codes):
    _need(isinstance(codes, torch.Tensor) and codes.dtype == torch.uint8, "E2M1 codes must be uint8")
    _need(bool((codes <= 15).all()), "E2M1 nibble outside [0,15]")
    return _decode_e2m1_codes(codes)


def pack_nibbles(codes):
    """fp4.py:118-122."""
    _need(codes.dtype == torch.uint8 and codes.ndim == 2, "Codes must be uint8 matrix")
    _need(bool((codes <= 15).all()), "Code outside nibble range")
    if codes.shape[1] % 2:
        codes = torch.nn.functional.pad(codes, (0, 1))
    return (codes[:, 0::2] | (codes[:, 1::2] << 4)).contiguous()


def unpack_nibbles(packed, columns):
    """fp4.py:125-130."""
    _need(packed.dtype == torch.uint8 and packed.ndim == 2, "Packed values must be uint8 matrix")
    _need(type(columns) is int and columns > 0 and packed.shape[1] == (columns + 1) // 2, "Packed width differs")
    if columns % 2:
        _need(bool(((packed[:, -1] & 0xf0) == 0).all()), "Nonzero high-nibble padding")
    result = torch.stack((packed & 15, packed >> 4), dim=-1).flatten(-2)
    return result[:, :columns].contiguous()


def _global_checked(value, device):
    _need(isinstance(value, torch.Tensor) and value.dtype == torch.float32 and value.numel() == 1,
          "A stored whole-tensor FP32 scale is required")
    return value.to(device=device).reshape(())


def _scales_valid(scales):
    f = scales.float()
    return bool(torch.isfinite(f).all()) and bool((f >= 0).all())


def decode_into(packed, scales, global_scale, out, *, rows, columns, group, err_flag=None):
    """Raw decode of one packet into `out` (FP16 [rows, columns], contiguous)
    on the current stream, no host synchronization.  `global_scale` is a
    device FP32 scalar tensor (G16) or None (G64); `err_flag`, if given, is a
    device int32[1] that accumulates the violation bits."""
    p = _native.ptr
    stream = _native.stream_of(packed)
    with torch.cuda.device(packed.device):
        if group == 16:
            _native.call("m2r_fp4_decode_g16", p(packed), p(scales), p(global_scale), p(out), rows, columns,
                         p(err_flag), stream)
        else:
            _native.call("m2r_fp4_decode_g64", p(packed), p(scales), p(out), rows, columns, p(err_flag), stream)
    return out


GEMV_ROWS = (1, 2, 4)


GEMV_COLUMNS = (2048, 4096, 8192)


def gemv_supported(rows, columns):
    """Whether gemv_g16 takes `rows` activation rows against a matrix of
    `columns` inputs (1, 2 or 4 rows; 2048, 4096 or 8192 columns)."""
    return rows in GEMV_ROWS and columns in GEMV_COLUMNS


def gemv_g16(packed, scales, global_scale, u, *, out=None):
    """y = u @ W.T for the FP4 G16 matrix W [N, K] kept packed (codes u8
    [N, K/2], E4M3 block bytes u8 [N, K/16], device FP32 global scalar) and
    FP16 activations u [M, K] (M in 1, 2, 4): the HIP kernel reads the packed
    format directly and uses, for every weight, the binary16 value
    decode_packet gives; products accumulate in binary32 and y is FP16
    [M, N].  The packet must satisfy decode_packet's checks.  No host
    synchronization."""
    _need(isinstance(u, torch.Tensor) and u.dtype == torch.float16 and u.ndim == 2, "u must be FP16 [rows, K]")
    rows, columns = u.shape
    _need(packed.dtype == torch.uint8 and packed.ndim == 2 and packed.shape[1] * 2 == columns,
          "packed codes must be uint8 [N, K/2]")
    n = packed.shape[0]
    sb = scales.view(torch.uint8) if scales.dtype == torch.float8_e4m3fn else scales
    _need(sb.dtype == torch.uint8 and tuple(sb.shape) == (n, columns // 16), "block scales must be [N, K/16]")
    _need(gemv_supported(rows, columns), "gemv_g16 supports 1, 2 or 4 rows and K of 2048, 4096 or 8192")
    for t in (packed, sb, u, global_scale):
        _native.require_device(t, "gemv operand")
    packed, sb = packed.contiguous(), sb.contiguous()
    if u.stride(1) != 1 or u.stride(0) % 8 or u.data_ptr() % 16:
        u = u.contiguous()
    if out is None:
        out = torch.empty((rows, n), dtype=torch.float16, device=u.device)
    _need(out.dtype == torch.float16 and tuple(out.shape) == (rows, n) and out.stride(1) == 1, "out must be FP16 [M, N]")
    with torch.cuda.device(u.device):
        _native.call("m2r_fp4_gemv_g16", _native.ptr(packed), _native.ptr(sb), _native.ptr(global_scale),
                     _native.ptr(u), u.stride(0), _native.ptr(out), out.stride(0), rows, n, columns,
                     _native.stream_of(u))
    return out


@torch.no_grad()
def decode_packet(packet):
    """fp4.py:225-250: validate a packet and return its FP16 [rows, columns]
    decode.  Raises ValueError with the reference's message for the first
    violated condition in the reference's order."""
    format_name = packet["format"]
    group = _format(format_name)
    shape = packet["shape"]
    _need(isinstance(shape, (tuple, list)) and len(shape) == 2 and all(type(v) is int and v > 0 for v in shape),
          "Invalid packet shape")
    rows, columns = shape
    groups = (columns + group - 1) // group
    padded = groups * group
    _need(packet["group_size"] == group, "Group size differs from fixed format")
    packed, scales = packet["packed"], packet["scales"]
    _need(packed.dtype == torch.uint8 and tuple(packed.shape) == (rows, padded // 2), "Packed geometry differs")
    dtype = torch.float16 if group == 64 else torch.float8_e4m3fn
    _need(scales.dtype == dtype and tuple(scales.shape) == (rows, groups) and scales.device == packed.device,
          "Stored scale geometry/dtype differs")
    _native.require_device(packed, "packed FP4 codes")
    canonical = (packed.is_contiguous() and scales.is_contiguous()
                 and all(v.storage_offset() == 0 and v.untyped_storage().nbytes() == v.numel() * v.element_size()
                         for v in (packed, scales)))
    global_ok = True
    if group == 16:
        g = packet["global_scale"]
        global_ok = isinstance(g, torch.Tensor) and g.dtype == torch.float32 and g.numel() == 1
    elif packet["global_scale"] is not None:
        global_ok = False
    if not canonical or not global_ok:
        # host-side failures: report them after the scale-validity check that
        # precedes them in the reference
        _need(_scales_valid(scales), "Invalid stored scale")
        _need(packed.is_contiguous() and scales.is_contiguous(), "Exact contiguous packed buffers required")
        for value in (packed, scales):
            _need(value.storage_offset() == 0 and value.untyped_storage().nbytes() == value.numel() * value.element_size(),
                  "Padded/aliased backing storage is not a canonical packet")
        if group == 16:
            _global_checked(packet["global_scale"], packed.device)
        _need(packet["global_scale"] is None, "Unexpected global scale for G64")
    global_scale = _global_checked(packet["global_scale"], packed.device) if group == 16 else None
    out = torch.empty((rows, columns), dtype=torch.float16, device=packed.device)
    flag = torch.zeros(1, dtype=torch.int32, device=packed.device)
    decode_into(packed, scales.view(torch.uint8) if group == 16 else scales, global_scale, out,
                rows=rows, columns=columns, group=group, err_flag=flag)
    raise_decode_errors(int(flag.item()))
    return out


def raise_decode_errors(err):
    """Raises the reference's ValueError for the first condition (in the
    reference's check order) whose bit is set in the kernels' error word."""
    if err:
        _need(not err & ERR_SCALE, "Invalid stored scale")
        _need(not err & ERR_GLOBAL, "Global scale must be finite and positive")
        _need(not err & ERR_PADDING, "Nonzero final-group padding")
        _need(not err & ERR_ZERO_SCALE, "Nonzero code in a zero-scale group")
        _need(not err & ERR_DECODED, "Nonfinite decoded FP16 weights")


def expected_payload_bytes(format_name):
    """fp4.py:385: exact packed payload of the full 8B weight set."""
    group = _format(format_name)
    return 8_233_418_752 * 17 // 32 + 7_161_856 if group == 64 else 8_233_418_752 * 9 // 16 + 114 * 4 + 7_161_856
