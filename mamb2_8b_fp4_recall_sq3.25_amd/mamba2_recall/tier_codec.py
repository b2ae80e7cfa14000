"""Same-52-byte stored-scale tier codecs (INT8 / INT4 / zero-carry tiers).

Drop-in for the reference's scripts/state_ppl_codec_v10.py (layouts
16_64_48, 8_80_40, 24_48_56, 32_32_64; 16_64_48 is the v6 stored_scale path
of scripts/state_ppl_codec_v6.py) and scripts/w4_state_repair_codec_v2.py
(adds 36_24_68, 40_16_72, 44_8_76).  Layout 'A_B_C' carries A INT8
coordinates, B INT4 coordinates and C zero-carry coordinates, in permuted
order.  The scan runs the HIP kernel m2r_state_step_tier: stored-scale
requantization after every token (state_ppl_codec_v6.py:52-61).
"""
from __future__ import annotations

import torch

from . import _packed
from .state_codec import PackedState, validate_permutation
from .state_quant import _MixerController

V10_LAYOUTS = ("16_64_48", "8_80_40", "24_48_56", "32_32_64")
BASELINE = "32_32_64"
NEW_LAYOUTS = ("36_24_68", "40_16_72", "44_8_76")
LAYOUT_ORDER = (BASELINE, "16_64_48", "8_80_40", "24_48_56", *NEW_LAYOUTS)
LAYOUTS = LAYOUT_ORDER
COUNTS = {"16_64_48": (16, 64, 48), "8_80_40": (8, 80, 40), "24_48_56": (24, 48, 56),
          "32_32_64": (32, 32, 64), "36_24_68": (36, 24, 68), "40_16_72": (40, 16, 72),
          "44_8_76": (44, 8, 76)}
RP = 16
CACHE_BYTES = 28499968
TABLE_BYTES = 57344


def layout_descriptor(layout=BASELINE):
    """w4_state_repair_codec_v2.py:34-44 / state_ppl_codec_v10.py:31-37."""
    if layout not in COUNTS:
        raise ValueError("Unknown fixed W4 state repair tier layout")
    n8, n4, nzero = COUNTS[layout]
    if n8 + n4 + nzero != 128 or n8 + n4 // 2 != 48 or n8 % 2 or n4 % 2:
        raise RuntimeError("Internal repair layout violates the 52-byte row")
    return dict(layout=layout, n8=n8, n4=n4, nzero=nzero, payload_bytes=48, scale_bytes=4, row_bytes=52,
                resident_layout_metadata_bytes=0, tensor_widths=dict(lo=n8 // 2, hi=n8 // 2, q4=n4 // 2))


def state_mode(layout):
    """The reference's PackedState.mode string for a tier layout."""
    if layout == "16_64_48":
        return "sq3p25"
    if layout in V10_LAYOUTS:
        return "v10_" + layout
    return "w4_repair_v2_" + layout


def validate_layouts(layouts):
    if not isinstance(layouts, (tuple, list)) or len(layouts) != 56:
        raise ValueError("Exactly 56 per-layer layout names are required")
    result = tuple(layouts)
    for layout in result:
        if not isinstance(layout, str):
            raise ValueError("Layout IDs must be strings on the CPU")
        layout_descriptor(layout)
    return result


def uniform_layouts(layout=BASELINE):
    layout_descriptor(layout)
    return (layout,) * 56


def allocate_state(batch, heads, dim, dstate, device, *, layout=BASELINE):
    descriptor = layout_descriptor(layout)
    if dstate != 128 or any(type(v) is not int or v <= 0 for v in (batch, heads, dim)):
        raise ValueError("Positive integer geometry and 128 state coordinates required")
    shape = (batch, heads, dim, 128)
    tensors = {key: torch.zeros((batch, heads, dim, width), dtype=torch.uint8, device=device)
               for key, width in descriptor["tensor_widths"].items()}
    tensors.update({key: torch.zeros((batch, heads, dim), dtype=torch.float16, device=device)
                    for key in ("s8", "s4")})
    return PackedState(state_mode(layout), tensors, shape)


def validate_state(state, device, layout):
    """w4_state_repair_codec_v2.py:77-100: exact, unaliased, contiguous."""
    descriptor = layout_descriptor(layout)
    batch, heads, dim, dstate = state.shape
    if dstate != 128 or min(batch, heads, dim) <= 0:
        raise ValueError("Invalid packed state geometry")
    if state.mode != state_mode(layout) or set(state.tensors) != {"lo", "hi", "q4", "s8", "s4"}:
        raise ValueError("Packed state layout or tensor inventory differs")
    storages = set()
    for key, value in state.tensors.items():
        shape = (batch, heads, dim)
        dtype = torch.float16 if key in ("s8", "s4") else torch.uint8
        if key in descriptor["tensor_widths"]:
            shape += (descriptor["tensor_widths"][key],)
        if (tuple(value.shape) != shape or value.dtype != dtype or value.device != torch.device(device)
                or not value.is_contiguous() or value.storage_offset() != 0
                or value.untyped_storage().nbytes() != value.numel() * value.element_size()):
            raise ValueError("State must use exact unpadded physical tensor allocations")
        storages.add(value.untyped_storage().data_ptr())
    if len(storages) != 5 or state.nbytes != batch * heads * dim * 52:
        raise ValueError("State tensors alias or exceed the52-byte budget")
    return True


@torch.no_grad()
def scan(x, dt, A, B, C, D, dt_bias, state, permutation, *, layout=BASELINE):
    """Return (FP16 readout, None), mutating the packed carry after every token
    (state_ppl_codec_v10.py:157-192; w4_state_repair_codec_v2.py:103-137)."""
    descriptor = layout_descriptor(layout)
    if not isinstance(x, torch.Tensor) or x.ndim != 4 or x.dtype != torch.float16 or not x.is_cuda:
        raise ValueError("x must be CUDA FP16[batch,tokens,heads,dim]")
    batch, length, heads, dim = x.shape
    if length < 1 or state.shape != (batch, heads, dim, 128):
        raise ValueError("Positive sequence and matching packed geometry required")
    validate_state(state, x.device, layout)
    groups = _packed.check_inputs(x, dt, A, B, C, D, dt_bias, state.shape)[4]
    if (permutation.dtype != torch.uint8 or tuple(permutation.shape) != (groups, 128)
            or permutation.device != x.device):
        raise ValueError("Permutation must be CUDA uint8[groups,128]")
    y = _packed.launch_packed("tier", x, dt, A, B, C, D, dt_bias, permutation, state.tensors,
                              n8=descriptor["n8"], n4=descriptor["n4"], nz=descriptor["nzero"])
    return y, None


@torch.no_grad()
def decode_state(state, permutation=None, *, layout=BASELINE):
    """FP32 carry in packed order (zero-carry tier 0) or, with a permutation,
    original coordinates (state_ppl_codec_v10.py:195-217)."""
    descriptor = layout_descriptor(layout)
    validate_state(state, state.tensors["lo"].device, layout)
    values = _packed.decode_rows(state.tensors, descriptor["n8"], descriptor["n4"], shape=state.shape)
    if permutation is None:
        return values
    validate_permutation(permutation, permutation.shape[0])
    return _packed.scatter_permutation(values, permutation)


def validate_finite_result(state, output=None):
    """state_ppl_codec_v6.py:273-278."""
    values = [v for v in state.tensors.values() if v.is_floating_point()]
    if output is not None:
        values.append(output)
    if values and not bool(torch.stack([torch.isfinite(v).all() for v in values]).all()):
        raise FloatingPointError("Nonfinite state scale, diagnostic carry or readout")
    return True


class StateRepairV2(_MixerController):
    """Per-layer stored-scale tier carry with one [56,8,128] coordinate table
    (w4_state_repair_codec_v2.py:168-260): each layer uses its own layout,
    all rows are 52 bytes, and a batch-one request cache (convolution windows
    + packed rows + table) is exactly 28,499,968 bytes."""

    scale_mode, int4_clip, diagnostic = "stored_scale", 1.0, None

    def __init__(self, model, table, layouts):
        self._layouts = validate_layouts(layouts)
        super().__init__(model, "sq3p25", table, False)
        if (self.permutations.numel() != TABLE_BYTES
                or self.permutations.untyped_storage().nbytes() != TABLE_BYTES):
            raise ValueError("The one coordinate table must occupy exactly 57,344 bytes")

    @property
    def layouts(self):
        return self._layouts

    def _new_state(self, batch_size, index):
        layout = self.layouts[index]
        state = allocate_state(batch_size, self.HEADS, self.HEADDIM, self.D_STATE, self.device, layout=layout)
        validate_state(state, self.device, layout)
        return state

    def _after_reset(self, batch_size):
        if self.cache_breakdown()["total_bytes"] != batch_size * (CACHE_BYTES - TABLE_BYTES) + TABLE_BYTES:
            raise RuntimeError("Per-layer repair cache exceeds the fixed physical budget")

    def _scan_layer(self, index, mx, x, dt, aa, bm, cm, entry):
        return scan(x, dt, aa, bm, cm, mx.D, mx.dt_bias, entry.state, self.permutations[index],
                    layout=self.layouts[index])

    def assert_finite_cache(self):
        """state_ppl_codec_v6.py:362-367."""
        values = [v.conv for v in self._cache]
        values += [t for v in self._cache for t in v.state.tensors.values() if t.is_floating_point()]
        if values and not bool(torch.stack([torch.isfinite(t.float()).all() for t in values]).all()):
            raise FloatingPointError("Nonfinite persistent scale, convolution or diagnostic carry")
        return True

    def cache_breakdown(self):
        """state_ppl_codec_v6.py:369-384 (stored-scale, no diagnostic)."""
        conv = sum(v.conv.untyped_storage().nbytes() for v in self._cache)
        state = sum(v.state.nbytes for v in self._cache)
        scales = sum(v.state.tensors[k].untyped_storage().nbytes() for v in self._cache for k in ("s8", "s4"))
        table = self.permutations.untyped_storage().nbytes()
        return {"mode": self.mode, "scale_mode": self.scale_mode, "int4_clip": self.int4_clip,
                "diagnostic": self.diagnostic, "is_3p25_candidate": True, "batch_size": self._batch_size,
                "allocated_layers": len(self._cache), "conv_fp16_bytes": conv, "ssm_payload_bytes": state - scales,
                "ssm_scale_bytes": scales, "ssm_total_bytes": state, "permutation_bytes": table,
                "total_bytes": conv + state + table, "calibration_workspace_bytes": 0,
                "diagnostic_dense_fp32_bytes": 0, "row_bytes": 52,
                "tokens_per_layer": [v.tokens for v in self._cache],
                "scope": "Actual persistent request cache and permutation table. Weights, activations, registers "
                         "and allocator reserve excluded."}

    def storage_descriptor(self):
        """w4_state_repair_codec_v2.py:203-224."""
        layers = []
        for index, entry in enumerate(self._cache):
            layout = self.layouts[index]
            validate_state(entry.state, self.device, layout)
            layers.append(dict(**layout_descriptor(layout), state_shape=list(entry.state.shape),
                               state_bytes=entry.state.nbytes,
                               tensors={k: dict(shape=list(v.shape), dtype=str(v.dtype),
                                                storage_bytes=v.untyped_storage().nbytes())
                                        for k, v in entry.state.tensors.items()},
                               conv_shape=list(entry.conv.shape),
                               conv_storage_bytes=entry.conv.untyped_storage().nbytes()))
        return dict(format="W4_STATE_REPAIR_STORAGE_V2", layouts=list(self.layouts), row_bytes=52, payload_bytes=48,
                    scale_bytes=4, resident_layout_metadata_bytes=0,
                    cpu_layout_metadata=dict(kind="tuple[str,...]", entries=56,
                                             scope="Host orchestration only; Python heap is not GPU recurrent storage"),
                    permutation_shape=list(self.permutations.shape), permutation_dtype=str(self.permutations.dtype),
                    permutation_storage_bytes=self.permutations.untyped_storage().nbytes(),
                    total_cache_bytes=self.cache_breakdown()["total_bytes"], layers=layers)
