"""Published group-ridge latent state codec (52-byte rows, 3.25 bit/coord).

Drop-in for the reference's scripts/fp4_zero_predictor_codec_v1.py: INT8 and
INT4 tiers with stored FP16 scales, two E4M3 latent coefficients per row for
the zero-carry tier, and a static per-group ridge predictor whose transient
readout correction is contracted inside the kernel (no FP32 temporary, no
host synchronization).  The scan runs the HIP kernel m2r_state_step_ridge.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native, _packed, tier_codec
from .state_codec import PackedState

RP = 16
CACHE_BYTES = 28499968
TABLE_BYTES = 57344


def layout_descriptor(layout):
    """fp4_zero_predictor_codec_v1.py:28-36: parent 'A_B_C' -> (A, B-4, C+4)."""
    old = tier_codec.layout_descriptor(layout)
    n8, n4, nzero = old["n8"], old["n4"] - 4, old["nzero"] + 4
    if n4 < 4 or n8 + n4 + nzero != 128 or n8 + n4 // 2 + 2 + 4 != 52:
        raise ValueError("Latent tier layout violates same-byte geometry")
    return dict(layout=layout, n8=n8, n4=n4, nzero=nzero, payload_bytes=48, scale_bytes=4, row_bytes=52,
                latent_coefficients=2, latent_dtype="torch.float8_e4m3fn",
                tensor_widths=dict(lo=n8 // 2, hi=n8 // 2, q4=n4 // 2, latent=2))


def allocate_state(batch, heads, dim, dstate, device, *, layout):
    """fp4_zero_predictor_codec_v1.py:39-49."""
    spec = layout_descriptor(layout)
    if dstate != 128 or any(type(v) is not int or v <= 0 for v in (batch, heads, dim)):
        raise ValueError("Positive state geometry and dstate=128 required")
    base = (batch, heads, dim)
    tensors = {name: torch.zeros((*base, width), device=device,
                                 dtype=torch.float8_e4m3fn if name == "latent" else torch.uint8)
               for name, width in spec["tensor_widths"].items()}
    tensors.update({name: torch.zeros(base, device=device, dtype=torch.float16) for name in ("s8", "s4")})
    return PackedState("latent_fp8_" + layout, tensors, (*base, 128))


def validate_state(state, device, layout):
    """fp4_zero_predictor_codec_v1.py:52-73."""
    spec = layout_descriptor(layout)
    if (state.mode != "latent_fp8_" + layout or len(state.shape) != 4 or state.shape[-1] != 128
            or set(state.tensors) != {"lo", "hi", "q4", "latent", "s8", "s4"}):
        raise ValueError("Latent packed state mode/inventory differs")
    base = tuple(state.shape[:3])
    if min(base) <= 0:
        raise ValueError("Invalid latent state geometry")
    storages = set()
    for name, value in state.tensors.items():
        shape = base + ((spec["tensor_widths"][name],) if name in spec["tensor_widths"] else ())
        dtype = (torch.float16 if name in ("s8", "s4") else
                 torch.float8_e4m3fn if name == "latent" else torch.uint8)
        if (tuple(value.shape) != shape or value.dtype != dtype or value.device != torch.device(device)
                or not value.is_contiguous() or value.storage_offset() != 0
                or value.untyped_storage().nbytes() != value.numel() * value.element_size()):
            raise ValueError("Latent packed state backing allocation differs: " + name)
        storages.add(value.untyped_storage().data_ptr())
    if len(storages) != 6 or state.nbytes != base[0] * base[1] * base[2] * 52:
        raise ValueError("Latent state aliases or exceeds 52-byte row")
    return True


def check_static_metadata(permutation, basis, latent_scale, predictor, *, groups, layout, device):
    """Host-only part of scan()'s static-table checks
    (fp4_zero_predictor_codec_v1.py:203-217): dtype, shape and device of the
    permutation, bases, latent scales and predictor.  The kernel indexes these
    tables by the shapes checked here, so every scan runs this, whatever its
    `validate` flag; it reads tensor metadata only and never synchronizes."""
    spec = layout_descriptor(layout)
    if (not all(isinstance(v, torch.Tensor) for v in (permutation, basis, latent_scale, predictor))
            or permutation.dtype != torch.uint8 or tuple(permutation.shape) != (groups, 128)
            or permutation.device != device
            or basis.dtype != torch.float16 or tuple(basis.shape) != (groups, spec["nzero"], 2)
            or basis.device != device
            or latent_scale.dtype != torch.float16 or tuple(latent_scale.shape) != (groups, 2)
            or latent_scale.device != device):
        raise ValueError("Latent static basis/scales differ")
    features = spec["n8"] + spec["n4"] + 2
    if (predictor.dtype != torch.float16 or tuple(predictor.shape) != (groups, features, spec["nzero"])
            or predictor.device != device or not predictor.is_contiguous()):
        raise ValueError("Static zero-tier predictor differs")


def validate_statics(permutation, basis, latent_scale, predictor, *, groups, layout, device):
    """The static-table checks of scan() (fp4_zero_predictor_codec_v1.py:203-217):
    the metadata checks, then the value checks (finite bases, scales and
    predictor, positive latent scales), which synchronize with the device, so
    controllers run them once."""
    check_static_metadata(permutation, basis, latent_scale, predictor, groups=groups, layout=layout,
                          device=device)
    if (not bool(torch.isfinite(basis).all()) or not bool(torch.isfinite(latent_scale).all())
            or not bool((latent_scale > 0).all())):
        raise ValueError("Latent static basis/scales differ")
    if not bool(torch.isfinite(predictor).all()):
        raise ValueError("Static zero-tier predictor differs")


@torch.no_grad()
def scan(x, dt, A, B, C, D, dt_bias, state, permutation, basis, latent_scale, predictor, *, layout,
         validate=True):
    """Return (FP16 readout, None), mutating the packed carry after every token.

    Same contract as fp4_zero_predictor_codec_v1.scan (:184-236).  The ridge
    correction corr[b,t,g,f] = sum_d C[b,t,g,perm[g,n8+n4+d]] * pred[g,f,d]
    is computed inside the kernel.  With validate=True the static tables and
    the finiteness of the correction are checked here exactly as the
    reference does (five device synchronizations); validate=False skips
    only those value checks, for callers that validated the statics once:
    the tables' dtype, shape and device are checked on every call.
    """
    spec = layout_descriptor(layout)
    if not isinstance(x, torch.Tensor) or x.ndim != 4 or x.dtype != torch.float16 or not x.is_cuda:
        raise ValueError("x must be CUDA FP16 [batch,tokens,heads,dim]")
    batch, length, heads, dim = x.shape
    if length < 1 or dim % RP or state.shape != (batch, heads, dim, 128):
        raise ValueError("Positive sequence and matching latent state required")
    validate_state(state, x.device, layout)
    groups = B.shape[2] if B.ndim == 4 else 0
    expected = ((dt, (batch, length, heads)), (A, (heads,)), (B, (batch, length, groups, 128)),
                (C, (batch, length, groups, 128)), (D, (heads,)), (dt_bias, (heads,)))
    for value, shape in expected:
        if tuple(value.shape) != shape or value.device != x.device:
            raise ValueError("Latent scan input geometry/device differs")
    if (groups < 1 or heads % groups or A.dtype != torch.float32
            or any(v.dtype != torch.float16 for v in (dt, B, C))
            or any(v.dtype not in (torch.float16, torch.float32) for v in (D, dt_bias))):
        raise ValueError("Latent scan dtype/grouping differs")
    check_static_metadata(permutation, basis, latent_scale, predictor, groups=groups, layout=layout,
                          device=x.device)
    if validate:
        validate_statics(permutation, basis, latent_scale, predictor, groups=groups, layout=layout,
                         device=x.device)
        # |C| <= 65504, |pred| <= 65504 and nzero <= 124 keep every finite
        # correction below 6e11, so it is finite iff the gathered C entries are.
        dead_ix = permutation[:, spec["n8"] + spec["n4"]:].long()
        dead_c = C.gather(3, dead_ix[None, None, :, :].expand(batch, length, -1, -1))
        if not bool(torch.isfinite(dead_c).all()):
            raise FloatingPointError("Nonfinite transient predictor readout")
    y = _packed.launch_packed("ridge", x, dt, A, B, C, D, dt_bias, permutation, state.tensors,
                              n8=spec["n8"], n4=spec["n4"], nz=spec["nzero"], basis=basis,
                              lscale=latent_scale, pred=predictor)
    return y, None


def layer_table(steps):
    """The C-ABI layer table (an array of m2r_ridge_layer) of `steps`, for
    scan_layers and callers that launch the multi-layer step themselves.
    Each step is a dict with scan()'s tensor arguments (x, dt, A, B, C, D,
    dt_bias, state, permutation, basis, latent_scale, predictor), its
    `layout` and `y`, an FP16 output of x's shape; every layer has one token
    and the same batch, heads, dim and groups.  Shapes, dtypes, devices and
    the statics' metadata are checked here; the statics' values are taken as
    validated (scan's validate=False)."""
    if not steps:
        raise ValueError("At least one layer required")
    x0 = steps[0]["x"]
    # the launch takes one group count for every layer (the kernel indexes
    # each layer's B, C and statics with it): a layer with fewer groups would
    # be read past its tensors' ends
    group_counts = {tuple(st["B"].shape[2:3]) if st["B"].ndim == 4 else None for st in steps}
    if len(group_counts) != 1 or None in group_counts:
        raise ValueError("Every layer needs the same number of B/C groups")
    table = (_native.RidgeLayer * len(steps))()
    for i, st in enumerate(steps):
        x, state, layout = st["x"], st["state"], st["layout"]
        spec = layout_descriptor(layout)
        if (not isinstance(x, torch.Tensor) or x.ndim != 4 or x.dtype != torch.float16 or not x.is_cuda
                or x.shape != x0.shape or x.device != x0.device or x.shape[1] != 1):
            raise ValueError("Every layer needs CUDA FP16 x of one shape [batch,1,heads,dim]")
        batch, _, heads, dim = x.shape
        if dim % RP or state.shape != (batch, heads, dim, 128):
            raise ValueError("Positive sequence and matching latent state required")
        validate_state(state, x.device, layout)
        B, C = st["B"], st["C"]
        groups = B.shape[2] if B.ndim == 4 else 0
        expected = ((st["dt"], (batch, 1, heads)), (st["A"], (heads,)), (B, (batch, 1, groups, 128)),
                    (C, (batch, 1, groups, 128)), (st["D"], (heads,)), (st["dt_bias"], (heads,)),
                    (st["y"], tuple(x.shape)))
        for value, shape in expected:
            if tuple(value.shape) != shape or value.device != x.device or not value.is_contiguous():
                raise ValueError("Latent scan input geometry/device differs")
        if (groups < 1 or heads % groups or st["A"].dtype != torch.float32 or st["y"].dtype != torch.float16
                or any(v.dtype != torch.float16 for v in (st["dt"], B, C))
                or any(v.dtype not in (torch.float16, torch.float32) for v in (st["D"], st["dt_bias"]))):
            raise ValueError("Latent scan dtype/grouping differs")
        check_static_metadata(st["permutation"], st["basis"], st["latent_scale"], st["predictor"], groups=groups,
                              layout=layout, device=x.device)
        t = state.tensors
        e = table[i]
        for name, value in (("x", x), ("dt", st["dt"]), ("A", st["A"]), ("B", B), ("C", C), ("D", st["D"]),
                            ("dt_bias", st["dt_bias"]), ("perm", st["permutation"]), ("basis", st["basis"]),
                            ("lscale", st["latent_scale"]), ("pred", st["predictor"]), ("lo", t["lo"]),
                            ("hi", t["hi"]), ("q4", t["q4"]), ("latent", t["latent"]), ("s8", t["s8"]),
                            ("s4", t["s4"]), ("y", st["y"])):
            setattr(e, name, value.data_ptr())
        e.n8, e.n4, e.nz = spec["n8"], spec["n4"], spec["nzero"]
        e.d_is_f32 = int(st["D"].dtype == torch.float32)
        e.db_is_f32 = int(st["dt_bias"].dtype == torch.float32)
    return table


@torch.no_grad()
def scan_layers(steps, *, workspace=None):
    """One launch of the one-token ridge step over several resident layers,
    each exactly as scan(..., validate=False) with one token would step it
    (its packed carry mutated, its readout written to step["y"]).  No
    counterpart in the reference, whose mixers step one layer per call: this
    is the one-launch variant for independent layers (the synthetic 56-layer
    benchmark, or separate states stepped together).  `workspace`: a uint8
    CUDA tensor of at least layers_workspace_bytes(len(steps)) bytes for the
    device copy of the layer table (allocated here when None)."""
    table = layer_table(steps)
    x = steps[0]["x"]
    batch, _, heads, dim = x.shape
    groups = steps[0]["B"].shape[2]
    need = layers_workspace_bytes(len(steps))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    if workspace.dtype != torch.uint8 or workspace.device != x.device or workspace.numel() < need:
        raise ValueError("Layer-table workspace too small")
    _native.call("m2r_state_step_ridge_layers", ctypes.byref(table), len(steps), batch, heads, dim, groups,
                 _native.ptr(workspace), workspace.numel(), _native.stream_of(x))
    return [st["y"] for st in steps]


def layers_workspace_bytes(nlayers):
    return int(_native.lib().m2r_state_step_ridge_layers_workspace(int(nlayers)))


class PredictorState(tier_codec.StateRepairV2):
    """Mixer controller with ridge-predicted zero-tier history
    (fp4_zero_predictor_codec_v1.py:239-367): the stored-scale tier carry of
    StateRepairV2 plus two E4M3 latent coefficients per row, with per-layer
    static bases [8,nz,2], latent scales [8,2] and predictors [8,F,nz].

    `validate_each_step` (default True, as the reference) repeats the scan's
    static-table and correction-finiteness checks on every call; the statics
    are already checked here at construction, so a caller that accepts
    non-finite activations surfacing later (assert_finite_cache) may turn it
    off to keep the per-token path free of host synchronizations."""

    validate_each_step = True

    def __init__(self, model, table, layouts, bases, scales, predictors):
        super().__init__(model, table, layouts)
        if len(bases) != self.LAYERS or len(scales) != self.LAYERS or len(predictors) != self.LAYERS:
            raise ValueError("Exactly 56 static bases/scales/predictors required")
        self.bases, self.latent_scales, self.predictors = [], [], []
        for layer, layout in enumerate(self.layouts):
            spec = layout_descriptor(layout)
            basis = bases[layer].to(device=self.device, dtype=torch.float16).contiguous()
            scale = scales[layer].to(device=self.device, dtype=torch.float16).contiguous()
            predictor = predictors[layer].to(device=self.device, dtype=torch.float16).contiguous()
            features = spec["n8"] + spec["n4"] + 2
            if (tuple(basis.shape) != (self.GROUPS, spec["nzero"], 2) or tuple(scale.shape) != (self.GROUPS, 2)
                    or tuple(predictor.shape) != (self.GROUPS, features, spec["nzero"])
                    or not bool(torch.isfinite(basis).all()) or not bool(torch.isfinite(scale).all())
                    or not bool(torch.isfinite(predictor).all()) or not bool((scale > 0).all())
                    or any(v.untyped_storage().nbytes() != v.numel() * 2 for v in (basis, scale, predictor))):
                raise ValueError("Static predictor/basis/scale allocation differs")
            self.bases.append(basis)
            self.latent_scales.append(scale)
            self.predictors.append(predictor)

    def _new_state(self, batch_size, index):
        layout = self.layouts[index]
        state = allocate_state(batch_size, self.HEADS, self.HEADDIM, self.D_STATE, self.device, layout=layout)
        validate_state(state, self.device, layout)
        return state

    def _after_reset(self, batch_size):
        if self.cache_breakdown()["total_bytes"] != batch_size * (CACHE_BYTES - TABLE_BYTES) + TABLE_BYTES:
            raise RuntimeError("Latent request cache violates fixed physical budget")

    def _scan_layer(self, index, mx, x, dt, aa, bm, cm, entry):
        return scan(x, dt, aa, bm, cm, mx.D, mx.dt_bias, entry.state, self.permutations[index], self.bases[index],
                    self.latent_scales[index], self.predictors[index], layout=self.layouts[index],
                    validate=self.validate_each_step)

    def assert_finite_cache(self):
        """fp4_zero_predictor_codec_v1.py:306-312."""
        values = [entry.conv for entry in self._cache]
        values.extend(t for entry in self._cache for t in entry.state.tensors.values() if t.is_floating_point())
        if values and not all(bool(torch.isfinite(v.float()).all()) for v in values):
            raise FloatingPointError("Nonfinite persistent latent/scale/convolution cache")
        return True

    def storage_descriptor(self):
        """fp4_zero_predictor_codec_v1.py:282-304."""
        layers = []
        for layer, (entry, layout, basis, scale, predictor) in enumerate(
                zip(self._cache, self.layouts, self.bases, self.latent_scales, self.predictors)):
            validate_state(entry.state, self.device, layout)
            layers.append(dict(**layout_descriptor(layout), layer=layer, state_shape=list(entry.state.shape),
                               state_bytes=entry.state.nbytes,
                               tensors={k: dict(shape=list(v.shape), dtype=str(v.dtype),
                                                storage_bytes=v.untyped_storage().nbytes())
                                        for k, v in entry.state.tensors.items()},
                               conv_shape=list(entry.conv.shape),
                               conv_storage_bytes=entry.conv.untyped_storage().nbytes(),
                               static_basis_bytes=basis.untyped_storage().nbytes(),
                               static_scale_bytes=scale.untyped_storage().nbytes(),
                               static_predictor_bytes=predictor.untyped_storage().nbytes()))
        return dict(format="FP4_LATENT_STATE_STORAGE_V1", layouts=list(self.layouts), row_bytes=52, payload_bytes=48,
                    scale_bytes=4, permutation_storage_bytes=self.permutations.untyped_storage().nbytes(),
                    total_cache_bytes=self.cache_breakdown()["total_bytes"],
                    static_basis_bytes=sum(x.untyped_storage().nbytes() for x in self.bases),
                    static_scale_bytes=sum(x.untyped_storage().nbytes() for x in self.latent_scales),
                    static_predictor_bytes=sum(x.untyped_storage().nbytes() for x in self.predictors),
                    layers=layers)
