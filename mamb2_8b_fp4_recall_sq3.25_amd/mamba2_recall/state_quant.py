"""Per-token state controllers for a frozen Mamba-2 8B model: drop-in for the
reference's mamba2_recall/state_quant.py (StateQuant, PackedStateRuntime,
_LayerCache).

A controller replaces every mixer's forward with: in_proj -> causal conv ->
split -> codec scan (the gfx950 state-step kernel: readout of each token's
FP32 update, then requantization or FP16 rounding of the carry) -> the
mixer's gated norm *called as a module* (so external norm hooks still fire)
-> out_proj.  It owns one request cache (convolution window + packed state
per layer), is single-stream and non-reentrant, and one controller at a time
may own a model.

`_MixerController` holds the orchestration shared by every codec; a codec
supplies `_new_state` (one layer's carry), `_scan_layer` (one layer's codec
call) and its cache accounting.  StateQuant covers the s16 control and the
legacy sq3p25 carry; state_quant_dense3, tier_codec and ridge_codec define
the dense 3-bit, stored-scale tier and ridge-latent controllers.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F

from . import _native, fp4, state_codec

# Installed controllers, keyed by the identity of the model each owns.  Values
# are held weakly; the installed per-layer hooks keep a controller alive until
# close() removes them and the entry.
_CLAIMS: "weakref.WeakValueDictionary[int, _MixerController]" = weakref.WeakValueDictionary()


@dataclass
class _LayerCache:
    conv: torch.Tensor
    state: object
    tokens: int = 0


@dataclass
class _Request:
    """Caches and ordering state of the request in flight: the layer caches,
    the layer the next mixer call must be for, the token count every layer of
    the current backbone call must see, and whether a call failed."""
    batch: int
    layers: list
    next_layer: int = 0
    call_tokens: Optional[int] = None
    failed: bool = False


class _LayerHook:
    """Installed as one mixer's `forward` (an instance attribute shadowing the
    class method), so module hooks registered on the mixer still run around it."""

    __slots__ = ("controller", "index", "module")

    def __init__(self, controller, index, module):
        self.controller, self.index, self.module = controller, index, module

    def __call__(self, u, seqlen=None, seq_idx=None, cu_seqlens=None, inference_params=None):
        return self.controller._forward(self.index, self.module, u, seqlen, seq_idx, cu_seqlens, inference_params)


_MISSING = object()


def conv_update(window, value, weight, bias, *, silu=True):
    """One-token causal convolution update on the device (the arithmetic of
    the reference's PyTorch fallback, state_quant.py:289-297, in one HIP
    kernel): rolls `window` [B,C,4] in place, appends `value` [B,C] and
    returns silu(sum(window * weight) + bias) as a new FP16 [B,C] tensor."""
    if (window.dtype != torch.float16 or value.dtype != torch.float16 or weight.dtype != torch.float16
            or window.ndim != 3 or value.ndim != 2 or weight.ndim != 2 or window.shape[-1] != 4
            or tuple(value.shape) != tuple(window.shape[:2]) or tuple(weight.shape) != tuple(window.shape[1:])
            or value.stride(-1) != 1 or not weight.is_contiguous()
            or (bias is not None and (bias.dtype != torch.float16 or tuple(bias.shape) != (window.shape[1],)
                                      or not bias.is_contiguous()))):
        raise ValueError("Convolution update expects FP16 window [B,C,4], value [B,C], weight [C,4], bias [C]")
    for t in (window, value, weight) + (() if bias is None else (bias,)):
        _native.require_device(t, "convolution operand")
    batch, channels = value.shape
    out = torch.empty((batch, channels), dtype=torch.float16, device=value.device)
    _native.call("m2r_causal_conv_update", _native.ptr(window), window.stride(0), window.stride(1), window.stride(2),
                 _native.ptr(value), value.stride(0), _native.ptr(weight), _native.ptr(bias), _native.ptr(out),
                 batch, channels, 4, 1 if silu else 0, _native.stream_of(value))
    return out


def _row_view(t, channels):
    """(rows, row stride) of `t` [..., channels] when its leading dimensions
    collapse into rows of one stride with unit channel stride, else None."""
    if t.dim() < 1 or t.shape[-1] != channels or t.stride(-1) != 1:
        return None
    lead = [(t.shape[i], t.stride(i)) for i in range(t.dim() - 1) if t.shape[i] > 1]
    if not lead:
        return 1, channels
    for (_, s_outer), (n_inner, s_inner) in zip(lead, lead[1:]):
        if s_outer != s_inner * n_inner:
            return None
    return t.numel() // channels, lead[-1][1]


def gated_rmsnorm(y, z, weight, eps, group_size):
    """The mixer's gated RMS norm (norm_before_gate False) on the device:
    per group of `group_size` channels, v = y * z * sigmoid(z) in FP32,
    out = FP16((v / sqrt(mean(v^2) + eps)) * weight); the computation of
    mamba_ssm's RMSNormGated, which the reference's controllers call as
    mx.norm(y, z) (state_quant.py:298-300), in one HIP kernel (fixed
    reduction tree, deterministic).  y, z: FP16 [..., C] with unit channel
    stride and leading dimensions of one row stride; returns a new FP16
    tensor of y's shape."""
    channels = y.shape[-1]
    if (y.dtype != torch.float16 or z.dtype != torch.float16 or weight.dtype != torch.float16
            or tuple(z.shape) != tuple(y.shape) or tuple(weight.shape) != (channels,) or not weight.is_contiguous()):
        raise ValueError("Gated norm expects FP16 y and z of one shape and an FP16 weight [C]")
    ry, rz = _row_view(y, channels), _row_view(z, channels)
    if ry is None or rz is None:
        raise ValueError("Gated norm operands need unit channel stride and one row stride")
    for t in (y, z, weight):
        _native.require_device(t, "gated norm operand")
    rows = ry[0]
    out = torch.empty(y.shape, dtype=torch.float16, device=y.device)
    stream = _native.stream_of(y)
    for r0 in range(0, rows, 65535):   # the grid's row limit
        n = min(65535, rows - r0)
        _native.call("m2r_gated_rmsnorm", y.data_ptr() + 2 * r0 * ry[1], ry[1], z.data_ptr() + 2 * r0 * rz[1],
                     rz[1], _native.ptr(weight), out.data_ptr() + 2 * r0 * channels, channels, n, channels,
                     group_size, float(eps), stream)
    return out


class _NormHook:
    """Installed as a mixer's gated-norm `forward` while a controller owns the
    model: module hooks on the norm (the Resurface adapter's pre-hook among
    them) still run around it.  Calls the native kernel for a gate z whose
    operands it supports, else the forward it shadows."""

    __slots__ = ("module", "fallback")

    def __init__(self, module, fallback):
        self.module, self.fallback = module, fallback

    def __call__(self, x, z=None):
        m = self.module
        if (z is not None and x.dtype == torch.float16 and z.dtype == torch.float16 and x.shape == z.shape
                and x.data_ptr() % 8 == 0 and z.data_ptr() % 8 == 0
                and _kernel_rows(x) and _kernel_rows(z)):
            return gated_rmsnorm(x, z, m.weight, m.eps, m.group_size)
        return self.fallback(x, z)


def _kernel_rows(t):
    """True when `t` is rows the gated-norm kernel reads: one row stride, a
    multiple of 4 elements, and rows that do not overlap (stride at least the
    channel count, or a single row); a broadcast or overlapping view goes to
    the module's own forward instead."""
    v = _row_view(t, t.shape[-1])
    return v is not None and v[1] % 4 == 0 and (v[0] == 1 or v[1] >= t.shape[-1])


def native_norm_compatible(norm, channels, group_size):
    """True when `norm` is a gated RMS norm the native kernel computes:
    gate applied before the norm, FP16 weight [channels], no bias, groups of
    `group_size` (a multiple of 4, at most 4096)."""
    w = getattr(norm, "weight", None)
    return (isinstance(w, torch.Tensor) and w.dtype == torch.float16 and tuple(w.shape) == (channels,)
            and w.is_contiguous() and w.data_ptr() % 8 == 0 and getattr(norm, "bias", None) is None
            and not getattr(norm, "norm_before_gate", False) and getattr(norm, "group_size", None) == group_size
            and isinstance(getattr(norm, "eps", None), float) and group_size % 4 == 0 and group_size <= 4096)


def _native_conv_ops():
    """mamba_ssm's fused causal-conv kernels when that package is present,
    else (None, None) and the PyTorch arithmetic below is used."""
    try:
        from mamba_ssm.modules import mamba2 as native
    except ImportError:
        return None, None
    return native.causal_conv1d_update, native.causal_conv1d_fn


class _MixerController:
    """Owns the per-token state of a frozen Mamba-2 8B model while installed:
    every mixer call runs in_proj -> causal conv -> split -> one codec call ->
    the mixer's gated norm as a module call -> out_proj, with the request
    ordering the reference enforces (state_quant.py:59-281).  A codec
    subclass supplies `_new_state`, `_scan_layer` and `cache_breakdown`."""

    LAYERS, D_MODEL, HEADS, HEADDIM, D_STATE, GROUPS, D_CONV, D_INNER = 56, 4096, 128, 64, 128, 8, 4, 8192
    # the mixers' gated norms run on the native kernel while installed (their
    # module hooks still run); False keeps the model's own norm computation.
    # The native kernel sums the squares in a fixed tree of its own and agrees
    # with a binary64 restatement of the formula to one binary16 rounding; the
    # reference's norm (mamba_ssm's RMSNormGated, a Triton kernel) reduces in
    # another order, so outputs can differ from it in the last bit of some
    # channels (that kernel's arithmetic is not available here to pin).
    native_norm = True
    PARAMETER_TENSORS, PARAMETER_COUNT = 507, 8_236_999_680
    TABLE_SHAPE = (56, 8, 128)

    def __init__(self, model, mode, permutations, collect_stats):
        self.model = model
        self.mode = mode
        self.collect_stats = bool(collect_stats)
        self._mixers = [layer.mixer for layer in model.backbone.layers]
        self._validate_model()
        self.device = self._mixers[0].in_proj.weight.device
        if self.device.type != "cuda":
            raise ValueError("The packed state codec requires a CUDA model")
        self.permutations = self._validate_permutations(permutations)
        bc = self.GROUPS * self.D_STATE
        # split sizes of the in_proj output (z, x|B|C, dt) and of the
        # convolution output (x, B, C)
        self._in_sizes = (self.D_INNER, self.D_INNER + 2 * bc, self.HEADS)
        self._conv_sizes = (self.D_INNER, bc, bc)
        self._request: Optional[_Request] = None
        self._hooks = {}          # mixer index -> (module, forward it shadowed or _MISSING)
        self._norm_hooks = {}     # mixer index -> (gated norm module, forward it shadowed or _MISSING)
        self._running = False     # inside backbone()
        self._rates = {}
        self._packed = None
        self._stat_sums = {}      # layer index -> FP64 [groups, 128] totals
        self._stat_counts = [0] * len(self._mixers)

    # ------------------------------------------------------------- compatibility
    @property
    def _cache(self):
        """The layer caches of the request in flight (empty when cleared)."""
        return self._request.layers if self._request is not None else []

    @property
    def _batch_size(self):
        return self._request.batch if self._request is not None else None

    @property
    def _installed(self):
        return bool(self._hooks)

    # ---------------------------------------------------------------- geometry
    @property
    def _conv_channels(self):
        return self.D_INNER + 2 * self.GROUPS * self.D_STATE

    def _validate_model(self):
        """state_quant.py:81-119."""
        backbone = self.model.backbone
        if len(self._mixers) != self.LAYERS:
            raise ValueError("This runtime requires the pure 56-layer 8B model")
        if backbone.fused_add_norm or backbone.residual_in_fp32:
            raise ValueError("Native unfused FP16 residual orchestration required")
        params = dict(self.model.named_parameters())
        if len(params) != self.PARAMETER_TENSORS or sum(p.numel() for p in params.values()) != self.PARAMETER_COUNT:
            raise ValueError("Source must have 507 original tensors / 8,236,999,680 parameters")
        if any(p.dtype != torch.float16 or p.requires_grad or p.grad is not None for p in params.values()):
            raise ValueError("Load the frozen FP16 source with no gradients")
        if len({p.device for p in params.values()}) != 1:
            raise ValueError("The frozen model must occupy one CUDA device")
        want = (self.D_MODEL, self.HEADS, self.HEADDIM, self.D_STATE, self.GROUPS, self.D_CONV, self.D_INNER,
                self.D_INNER)
        shapes = ((self.D_INNER * 2 + 2 * self.GROUPS * self.D_STATE + self.HEADS, self.D_MODEL),
                  (self.D_MODEL, self.D_INNER), (self._conv_channels, 1, self.D_CONV))
        for index, (layer, mx) in enumerate(zip(backbone.layers, self._mixers)):
            if layer.fused_add_norm or layer.residual_in_fp32 or layer.mlp is not None:
                raise ValueError(f"Unsupported block orchestration at layer {index}")
            geometry = (mx.d_model, mx.nheads, mx.headdim, mx.d_state, mx.ngroups, mx.d_conv, mx.d_ssm, mx.d_inner)
            if geometry != want:
                raise ValueError(f"Unsupported mixer geometry at layer {index}: {geometry}")
            if mx.use_mem_eff_path or not mx.rmsnorm or mx.D_has_hdim:
                raise ValueError("Explicit gated norm and one D per head required")
            if mx.activation not in ("silu", "swish") or mx.dt_limit != (0.0, float("inf")):
                raise ValueError("Unsupported activation or dt clipping")
            if mx.process_group is not None:
                raise ValueError("Distributed tensor parallel execution is unsupported")
            if mx.norm.group_size != self.D_INNER // self.GROUPS:
                raise ValueError("Expected eight gated RMSNorm groups")
            actual = tuple(tuple(v.shape) for v in (mx.in_proj.weight, mx.out_proj.weight, mx.conv1d.weight))
            if actual != shapes:
                raise ValueError(f"Projection/convolution shapes differ: {actual}")

    def _validate_permutations(self, values):
        """state_quant.py:121-133 (a uint8 permutation per layer and group)."""
        if not isinstance(values, torch.Tensor) or values.dtype != torch.uint8:
            raise ValueError("Packed state requires a uint8 tensor of permutations")
        if tuple(values.shape) != self.TABLE_SHAPE:
            raise ValueError("Expected permutations of shape [56,8,128]")
        cpu = values.detach().cpu().contiguous()
        if not torch.equal(cpu.sort(dim=-1).values, torch.arange(self.D_STATE, dtype=torch.uint8).expand_as(cpu)):
            raise ValueError("Every state group must be a permutation of 0..127")
        return cpu.to(device=self.device, dtype=torch.uint8).contiguous()

    # ---------------------------------------------------------------- lifetime
    def install(self):
        """Put a hook in front of every mixer's forward (the reference's
        install, state_quant.py:135-151: one owner per model)."""
        if self._installed:
            raise RuntimeError("StateQuant controller is already installed")
        key = id(self.model)
        if _CLAIMS.get(key) is not None:
            raise RuntimeError("Another StateQuant controller owns this model")
        _CLAIMS[key] = self
        try:
            for index, mx in enumerate(self._mixers):
                self._hooks[index] = (mx, mx.__dict__.get("forward", _MISSING))
                mx.forward = _LayerHook(self, index, mx)
            if self.native_norm:
                # the gated norm stays a module call (its hooks run); its
                # computation moves to the native kernel while installed
                for index, mx in enumerate(self._mixers):
                    norm = mx.norm
                    if native_norm_compatible(norm, self.D_INNER, self.D_INNER // self.GROUPS):
                        shadowed = norm.__dict__.get("forward", _MISSING)
                        self._norm_hooks[index] = (norm, shadowed)
                        norm.forward = _NormHook(norm, norm.forward)
        except Exception:
            self.close()
            raise
        return self

    def __enter__(self):
        return self.install()

    def __exit__(self, exc_type, exc_value, traceback):
        self.close()
        return False

    def close(self):
        """Remove the hooks (restoring whatever forward each mixer had),
        release the model and drop the request caches."""
        while self._norm_hooks:
            _, (norm, shadowed) = self._norm_hooks.popitem()
            if shadowed is _MISSING:
                norm.__dict__.pop("forward", None)
            else:
                norm.forward = shadowed
        while self._hooks:
            _, (mx, shadowed) = self._hooks.popitem()
            if shadowed is _MISSING:
                mx.__dict__.pop("forward", None)
            else:
                mx.forward = shadowed
        if _CLAIMS.get(id(self.model)) is self:
            del _CLAIMS[id(self.model)]
        self.clear()

    def clear(self):
        """Release all request caches, retaining calibration totals and tables."""
        self._request = None

    @torch.no_grad()
    def reset(self, batch_size=1):
        """Start a request: zero caches for every layer (state_quant.py:177-193)."""
        if not self._installed:
            raise RuntimeError("Install the controller before resetting caches")
        if not isinstance(batch_size, int) or isinstance(batch_size, bool) or batch_size <= 0:
            raise ValueError("batch_size must be a positive integer")
        self.clear()
        layers = []
        for index in range(len(self._mixers)):
            # the window is channels-last in memory (the layout of the
            # native convolution state), viewed as [batch, channels, 4]
            window = torch.zeros(batch_size, self.D_CONV, self._conv_channels, device=self.device,
                                 dtype=torch.float16).permute(0, 2, 1)
            layers.append(_LayerCache(conv=window, state=self._new_state(batch_size, index)))
        self._request = _Request(batch=batch_size, layers=layers)
        self._after_reset(batch_size)
        return self

    def _after_reset(self, batch_size):
        pass

    @torch.no_grad()
    def backbone(self, ids, reset=False):
        """model.backbone(ids) with every mixer going through this controller
        (state_quant.py:195-217): the request's caches are used and advanced."""
        if not self._installed:
            raise RuntimeError("StateQuant controller is not installed")
        if not isinstance(ids, torch.Tensor) or ids.ndim != 2 or ids.shape[1] == 0:
            raise ValueError("Input IDs must be nonempty [batch,tokens]")
        if ids.device != self.device or ids.dtype != torch.long:
            raise ValueError("Input IDs must be CUDA int64 on the model device")
        if self._running:
            raise RuntimeError("Concurrent/reentrant backbone invocation is unsupported")
        if reset or self._request is None:
            self.reset(ids.shape[0])
        self._running = True
        try:
            hidden = self.model.backbone(ids)
            if self._request.next_layer != 0:
                raise RuntimeError("Backbone did not execute every state-quantized layer")
        except Exception:
            if self._request is not None:
                self._request.failed = True
            raise
        finally:
            self._running = False
        return hidden

    # ---------------------------------------------------------------- one layer
    def _admit(self, index, u, extras):
        """The reference's checks before a mixer call (state_quant.py:219-247),
        in its order; returns the layer's cache."""
        if not self._installed or (self._request is not None and self._request.failed):
            raise RuntimeError("Controller is inactive or failed; reset before reusing it")
        if any(value is not None for value in extras):
            raise ValueError("Use controller-owned caches; native InferenceParams/varlen are unsupported")
        well_formed = (isinstance(u, torch.Tensor) and u.ndim == 3 and u.dtype == torch.float16
                       and u.device == self.device and u.shape[-1] == self.D_MODEL and u.shape[1] > 0)
        if not well_formed:
            raise ValueError("Mixer input must be CUDA FP16 [batch,tokens,4096]")
        if self._request is None:
            if index != 0:
                raise RuntimeError("A new request must start with backbone layer zero")
            self.reset(u.shape[0])
        request = self._request
        if u.shape[0] != request.batch or index != request.next_layer:
            raise RuntimeError("Batch shape or backbone layer order changed without a reset")
        tokens = u.shape[1]
        if index == 0:
            positions = {layer.tokens for layer in request.layers}
            if len(positions) != 1:
                raise RuntimeError("Per-layer cache positions disagree; reset the request")
            request.call_tokens = tokens
        elif tokens != request.call_tokens:
            raise RuntimeError("Backbone layers received different token counts")
        return request.layers[index]

    @torch.no_grad()
    def _forward(self, index, mx, u, seqlen, seq_idx, cu_seqlens, inference_params):
        """One mixer call: admission checks, then the mixer around the codec."""
        layer = self._admit(index, u, (seqlen, seq_idx, cu_seqlens, inference_params))
        try:
            out = self._mixer(index, mx, u, layer)
        except Exception:
            self._request.failed = True
            raise
        request = self._request
        request.next_layer = index + 1 if index + 1 < len(self._mixers) else 0
        if request.next_layer == 0:
            request.call_tokens = None
        return out

    def _mixer(self, index, mx, u, layer):
        batch, tokens = u.shape[0], u.shape[1]
        # a one-token continuation runs the projections and the norm on rank-2
        # inputs (the shapes the native step uses, and the ones norm hooks see)
        step = layer.tokens > 0 and tokens == 1
        if step:
            zxbcdt = self._project(index, "in_proj", mx, u[:, 0])[:, None]
        else:
            zxbcdt = mx.in_proj(u)
        z, xbc, dt = torch.split(zxbcdt, self._in_sizes, dim=-1)
        xbc = self._conv_step(mx, xbc[:, 0], layer)[:, None] if step else self._conv_prefill(mx, xbc, layer)
        x, bm, cm = torch.split(xbc, self._conv_sizes, dim=-1)
        y, stats = self._scan_layer(index, mx, x.reshape(batch, tokens, self.HEADS, self.HEADDIM), dt,
                                    self._decay_rates(index, mx),
                                    bm.reshape(batch, tokens, self.GROUPS, self.D_STATE),
                                    cm.reshape(batch, tokens, self.GROUPS, self.D_STATE), layer)
        if y.dtype != torch.float16 or tuple(y.shape) != (batch, tokens, self.HEADS, self.HEADDIM):
            raise RuntimeError("State codec returned unexpected readout dtype/shape")
        if self.collect_stats:
            self._accumulate_statistics(index, stats, batch, tokens)
        # the gated norm is called as a module, so its hooks see (y, z)
        y = y.reshape(batch, tokens, self.D_INNER)
        if step:
            out = self._project(index, "out_proj", mx, mx.norm(y[:, 0], z[:, 0]))[:, None]
        else:
            out = mx.out_proj(mx.norm(y, z))
        layer.tokens += tokens
        return out

    def use_packed_projections(self, packets, verify=False):
        """Run the one-token in_proj and out_proj of every layer as
        packed-resident FP4 G16 GEMVs (fp4.gemv_g16) instead of FP16 GEMMs.
        `packets[i]` is dict(in_proj=(codes, scales, global), out_proj=(...))
        in the checkpoint's G16 format for layer i, or None to keep that
        layer on its modules; `packets=None` turns the mode off.  The weights
        the GEMV uses are the binary16 values of decode_packet, so only the
        summation order of the projections changes; prefill steps and batch
        sizes the GEMV does not take keep the modules.  `verify=True` decodes
        every packet once and requires it to equal the module's weight bit
        for bit."""
        if packets is None:
            self._packed = None
            return self
        if len(packets) != len(self._mixers):
            raise ValueError("One packed-projection entry per layer required")
        checked = []
        for mx, entry in zip(self._mixers, packets):
            if entry is None:
                checked.append(None)
                continue
            pair = {}
            for name in ("in_proj", "out_proj"):
                module = getattr(mx, name)
                codes, scales, global_scale = entry[name]
                rows, cols = module.weight.shape
                if (module.bias is not None or codes.dtype != torch.uint8 or tuple(codes.shape) != (rows, cols // 2)
                        or tuple(scales.shape) != (rows, cols // 16) or codes.device != self.device
                        or scales.device != self.device or global_scale.device != self.device
                        or global_scale.numel() != 1 or global_scale.dtype != torch.float32):
                    raise ValueError(f"Packed {name} does not match the layer's projection")
                sb = scales.view(torch.uint8) if scales.dtype == torch.float8_e4m3fn else scales
                if verify:
                    decoded = fp4.decode_packet(dict(format="fp4_g16_e4m3", shape=[rows, cols], group_size=16,
                                                     packed=codes, scales=sb.view(torch.float8_e4m3fn),
                                                     global_scale=global_scale.reshape(())))
                    if not torch.equal(decoded.view(torch.int16), module.weight.view(torch.int16)):
                        raise ValueError(f"Packed {name} does not decode to the module's weight")
                pair[name] = (codes.contiguous(), sb.contiguous(), global_scale.reshape(1))
            checked.append(pair)
        self._packed = checked
        return self

    def _project(self, index, name, mx, value):
        """One-token projection: the packed GEMV when registered and the batch
        size is supported, else the module."""
        entry = self._packed[index] if self._packed is not None else None
        if entry is not None and fp4.gemv_supported(value.shape[0], value.shape[1]):
            return fp4.gemv_g16(*entry[name], value)
        return getattr(mx, name)(value)

    def _decay_rates(self, index, mx):
        """A = -exp(float(A_log)) of one layer (state_quant.py:256), kept
        between calls while the parameter is unchanged (same storage and
        in-place version counter)."""
        key = (mx.A_log.data_ptr(), mx.A_log._version)
        cached = self._rates.get(index)
        if cached is None or cached[0] != key:
            cached = (key, -torch.exp(mx.A_log.float()))
            self._rates[index] = cached
        return cached[1]

    # ---------------------------------------------------------------- convolution
    # Same arithmetic as the reference's _convolution (state_quant.py:283-317):
    # mamba_ssm's fused kernels when present, otherwise its PyTorch fallback
    # (the one-token update as the HIP kernel conv_update).
    def _conv_step(self, mx, column, layer):
        """One token: shift the cached window, append `column` [B, C], return
        the activated convolution output [B, C]."""
        update_op, _ = _native_conv_ops()
        weight = mx.conv1d.weight[:, 0, :]
        if update_op is not None:
            return update_op(column, layer.conv, weight, mx.conv1d.bias, mx.activation)
        return conv_update(layer.conv, column, weight, mx.conv1d.bias, silu=mx.activation in ("silu", "swish"))

    def _conv_prefill(self, mx, xbc, layer):
        """Several tokens (or the first): the causal convolution over the
        cached history (the window's last D_CONV - 1 raw inputs, after the
        first call) followed by the new inputs; the window then holds the last
        D_CONV raw inputs, zero-padded on the left."""
        _, fused_op = _native_conv_ops()
        tokens = xbc.shape[1]
        fresh = xbc.transpose(1, 2)                              # [B, C, tokens]
        history = self.D_CONV - 1 if layer.tokens > 0 else 0
        series = torch.cat((layer.conv[:, :, 1:], fresh), dim=-1) if history else fresh
        kept = min(self.D_CONV, series.shape[-1])
        if kept < self.D_CONV:
            layer.conv.zero_()
        layer.conv[:, :, self.D_CONV - kept:].copy_(series[:, :, series.shape[-1] - kept:])
        if fused_op is not None:
            out = fused_op(series, mx.conv1d.weight[:, 0, :], bias=mx.conv1d.bias, activation=mx.activation,
                           seq_idx=None).transpose(1, 2)
        else:
            out = mx.act(mx.conv1d(series).transpose(1, 2)[:, :series.shape[-1]])
        return out[:, history:history + tokens]

    # ---------------------------------------------------------------- statistics
    def _accumulate_statistics(self, index, stats, batch, length):
        """Adds one codec call's |FP16 carry| sums to the layer's FP64 totals per
        (group, coordinate) (state_quant.py:319-330)."""
        tiles = (self.HEADDIM + 15) // 16
        expected = (batch, self.HEADS, tiles, self.D_STATE)
        if (not isinstance(stats, torch.Tensor) or stats.dtype != torch.float32 or stats.device != self.device
                or tuple(stats.shape) != expected):
            raise RuntimeError("Expected codec calibration sum [batch,128,4,128] FP32")
        heads_per_group = self.HEADS // self.GROUPS
        by_group = stats.double().reshape(batch, self.GROUPS, heads_per_group, tiles, self.D_STATE).sum(dim=(0, 2, 3))
        total = self._stat_sums.get(index)
        self._stat_sums[index] = by_group if total is None else total.add_(by_group)
        self._stat_counts[index] += batch * length * heads_per_group * self.HEADDIM

    def reset_statistics(self):
        self._stat_sums = {}
        self._stat_counts = [0] * len(self._mixers)

    def statistics(self):
        """CPU FP64 sums/means [56,8,128] and sample counts [56]."""
        layers = range(len(self._mixers))
        if not self.collect_stats or any(i not in self._stat_sums for i in layers):
            raise RuntimeError("Complete S16 calibration is required before collecting statistics")
        counts = torch.tensor(self._stat_counts, dtype=torch.int64)
        if bool((counts <= 0).any()):
            raise RuntimeError("Calibration has empty layers")
        sums = torch.stack([self._stat_sums[i] for i in layers]).detach().cpu()
        return {"sum_abs": sums, "sample_count_per_group": counts, "mean_abs": sums / counts[:, None, None],
                "semantics": "abs(FP16 stored carry), each token; average over batch, heads within each group, "
                             "P and time"}

    @property
    def cache_bytes(self):
        return self.cache_breakdown()["total_bytes"]

    # ---------------------------------------------------------------- codec hooks
    def _new_state(self, batch_size, index):
        raise NotImplementedError

    def _scan_layer(self, index, mx, x, dt, aa, bm, cm, entry):
        raise NotImplementedError

    def cache_breakdown(self):
        raise NotImplementedError


def permutations_from_statistics(statistics):
    """run_statequant.py:81-83: the sq3p25 permutation table of a calibration.

    ``statistics`` is the dict ``StateQuant.statistics()`` returns (or its
    ``mean_abs`` tensor [layers, groups, 128]).  Each (layer, group) row lists
    the coordinates by decreasing mean |FP16 carry|, equal means in coordinate
    order (a stable sort), as uint8: the first 16 become the INT8 tier, the
    next 64 the INT4 tier.  RuntimeError for non-finite statistics, as the
    reference raises before sorting."""
    mean_abs = statistics["mean_abs"] if isinstance(statistics, dict) else statistics
    if not isinstance(mean_abs, torch.Tensor) or mean_abs.ndim != 3 or mean_abs.shape[-1] != state_codec.N:
        raise ValueError("Expected calibration mean_abs [layers,groups,128]")
    if not bool(torch.isfinite(mean_abs).all()):
        raise RuntimeError("Nonfinite calibration statistics")
    return torch.argsort(mean_abs, dim=-1, descending=True, stable=True).to(torch.uint8)


class StateQuant(_MixerController):
    """Sequential s16 control or packed sq3p25 carry (state_quant.py:41-79).

    ``permutations`` is uint8[56,8,128] for sq3p25 (in packed order the first
    16 coordinates use INT8, the next 64 INT4, the last 48 carry nothing) and
    must be None for s16.  ``collect_stats`` (s16 only) accumulates FP64
    group totals of |FP16 carry|; they survive request resets.
    """

    def __init__(self, model, mode="s16", permutations=None, collect_stats=False):
        if mode not in ("s16", "sq3p25"):
            raise ValueError("State mode must be explicitly s16 or sq3p25")
        if collect_stats and mode != "s16":
            raise ValueError("Calibration statistics require the S16 control")
        self._codec_mode = mode
        super().__init__(model, mode, permutations, collect_stats)

    def _validate_permutations(self, values):
        if self._codec_mode == "s16":
            if values is not None:
                raise ValueError("S16 control must use original state coordinates")
            return None
        return super()._validate_permutations(values)

    def _new_state(self, batch_size, index):
        return state_codec.allocate_state(batch_size, self.HEADS, self.HEADDIM, self.D_STATE, self._codec_mode,
                                          self.device)

    def _scan_layer(self, index, mx, x, dt, aa, bm, cm, entry):
        permutation = None if self.permutations is None else self.permutations[index]
        return state_codec.scan(x, dt, aa, bm, cm, mx.D, mx.dt_bias, entry.state, permutation=permutation,
                                collect_stats=self.collect_stats)

    def cache_breakdown(self):
        """Bytes the request holds per kind of tensor, in the reference's
        report format (state_quant.py:347-366): windows, packed payload,
        stored scales, the permutation table and, outside the total, the
        calibration sums."""
        def size(t):
            return t.numel() * t.element_size()

        layers = self._cache
        conv = sum(size(c.conv) for c in layers)
        state = sum(int(c.state.nbytes) for c in layers)
        scales = sum(size(t) for c in layers for k, t in c.state.tensors.items() if k in ("s8", "s4"))
        tables = 0 if self.permutations is None else size(self.permutations)
        report = {"mode": self.mode, "batch_size": self._batch_size, "allocated_layers": len(layers)}
        report.update(conv_fp16_bytes=conv, ssm_payload_bytes=state - scales, ssm_scale_bytes=scales,
                      ssm_total_bytes=state, permutation_bytes=tables, total_bytes=conv + state + tables,
                      calibration_workspace_bytes=sum(size(t) for t in self._stat_sums.values()),
                      tokens_per_layer=[c.tokens for c in layers],
                      scope="Actual persistent request cache plus compact permutation table; weights, activations, "
                            "registers, allocator reserve and calibration workspace excluded from total_bytes")
        return report


PackedStateRuntime = StateQuant
