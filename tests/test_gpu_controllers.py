"""The per-token state controllers on a random-init Mamba-2 8B model (the
real geometry: 56 layers, 507 tensors, 8,236,999,680 parameters, 16.5 GB of
FP16 weights).  Known answer: a batch-one request cache (convolution windows
+ packed rows + one [56,8,128] table) is 28,499,968 bytes (README.md:123).
Wiring check: the controller's layer-0 carry after a prefill equals the codec
scan applied to the Mamba-2 definition of that layer's inputs."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import cases

pytestmark = pytest.mark.gpu

LAYOUTS = ("36_24_68", "16_64_48", "32_32_64", "40_16_72", "16_64_48", "16_64_48", "24_48_56", "32_32_64") * 7
CACHE_B1 = 28_499_968
TABLE = 57_344


def tables(device, seed=3):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randperm(128, generator=g) for _ in range(56 * 8)]).reshape(56, 8, 128).to(torch.uint8)


def ids(device, batch, n, seed=5):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randint(0, 256000, (batch, n), generator=g, device=device)


def layer0_inputs(model, tokens):
    """Mamba-2 definition of layer 0's codec inputs for a prefill from zero."""
    mx = model.backbone.layers[0].mixer
    u = model.backbone.layers[0].norm(model.backbone.embedding(tokens))
    z, xbc, dt = torch.split(mx.in_proj(u), (8192, 8192 + 2048, 128), dim=-1)
    xbc = F.silu(F.conv1d(xbc.transpose(1, 2), mx.conv1d.weight, mx.conv1d.bias, padding=3, groups=10240)[..., :-3])
    xbc = xbc.transpose(1, 2)
    b, n = tokens.shape
    x, bm, cm = torch.split(xbc, (8192, 1024, 1024), dim=-1)
    return (x.reshape(b, n, 128, 64), dt, -torch.exp(mx.A_log.float()), bm.reshape(b, n, 8, 128),
            cm.reshape(b, n, 8, 128), mx.D, mx.dt_bias)


def test_state_quant_sq3p25_cache_wiring_and_guards(model, device):
    from mamba2_recall import state_codec
    from mamba2_recall.state_quant import PackedStateRuntime, StateQuant
    perms = tables(device)
    tok = ids(device, 1, 6)
    with StateQuant(model, mode="sq3p25", permutations=perms) as sq:
        print("[controllers] sq3p25 prefill 4 + 2 steps", flush=True)
        h = sq.backbone(tok[:, :4])
        assert h.shape == (1, 4, 4096) and bool(torch.isfinite(h).all())
        ref = state_codec.allocate_state(1, 128, 64, 128, "sq3p25", device)
        x, dt, A, B, C, D, db = layer0_inputs(model, tok[:, :4])
        state_codec.scan(x, dt, A, B, C, D, db, ref, permutation=perms[0].to(device))
        for k in ref.tensors:
            assert torch.equal(ref.tensors[k], sq._cache[0].state.tensors[k]), k
        for t in (4, 5):
            h = sq.backbone(tok[:, t:t + 1])
            assert h.shape == (1, 1, 4096) and bool(torch.isfinite(h).all())
        br = sq.cache_breakdown()
        assert br["total_bytes"] == CACHE_B1 and sq.cache_bytes == CACHE_B1
        assert br["tokens_per_layer"] == [6] * 56
        with pytest.raises(RuntimeError, match="Another StateQuant controller owns this model"):
            PackedStateRuntime(model, mode="sq3p25", permutations=perms).install()
        with pytest.raises(RuntimeError, match="layer order changed"):
            sq._forward(3, model.backbone.layers[3].mixer, torch.zeros(1, 1, 4096, dtype=torch.float16,
                                                                    device=device), None, None, None, None)
        sq.reset(2)
        assert sq.cache_bytes == 2 * (CACHE_B1 - TABLE) + TABLE
    assert all(isinstance(layer.mixer.forward, type(model.backbone.layers[0].mixer.forward))
               for layer in model.backbone.layers)
    with pytest.raises(RuntimeError, match="native Mamba-2 mixer forward"):
        model.backbone(tok[:, :1])


def test_state_quant_s16_statistics(model, device):
    from mamba2_recall.state_quant import StateQuant
    with pytest.raises(ValueError, match="require the S16 control"):
        StateQuant(model, mode="sq3p25", permutations=tables(device), collect_stats=True)
    with StateQuant(model, mode="s16", collect_stats=True) as sq:
        print("[controllers] s16 prefill 3 + 1 step with statistics", flush=True)
        sq.backbone(ids(device, 2, 3))
        sq.backbone(ids(device, 2, 1, seed=6))
        st = sq.statistics()
        assert st["sum_abs"].shape == (56, 8, 128) and st["sum_abs"].dtype == torch.float64
        assert st["sample_count_per_group"].tolist() == [2 * 4 * 16 * 64] * 56
        assert bool(torch.isfinite(st["mean_abs"]).all())
    # the reference's calibration flow (run_statequant.py:81-83): the table
    # from these statistics drives a packed sq3p25 run
    from mamba2_recall.state_quant import permutations_from_statistics
    table = permutations_from_statistics(st)
    assert table.dtype == torch.uint8 and tuple(table.shape) == (56, 8, 128)
    ordered = torch.gather(st["mean_abs"], -1, table.long())
    assert bool((ordered[..., :-1] >= ordered[..., 1:]).all())
    with StateQuant(model, mode="sq3p25", permutations=table) as sq:
        print("[controllers] sq3p25 with the calibrated table", flush=True)
        h = sq.backbone(ids(device, 2, 3))
        h = sq.backbone(ids(device, 2, 1, seed=6))
        assert bool(torch.isfinite(h).all())


@pytest.mark.parametrize("kind", ["permutation", "equalizer"])
def test_dense3_controller(model, device, kind):
    from mamba2_recall.state_quant_dense3 import DenseStateQuant
    if kind == "permutation":
        table = tables(device)
    else:
        g = torch.Generator().manual_seed(9)
        table = torch.randint(-8, 9, (56, 8, 128), generator=g).to(torch.int8)
    with DenseStateQuant(model, table, table_kind=kind) as dq:
        print(f"[controllers] dense3 {kind}", flush=True)
        h = dq.backbone(ids(device, 1, 3))
        h = dq.backbone(ids(device, 1, 1, seed=7))
        assert bool(torch.isfinite(h).all())
        assert dq.assert_finite_cache()
        assert dq.cache_bytes == CACHE_B1


def test_tier_and_predictor_controllers(model, device):
    from mamba2_recall import ridge_codec
    from mamba2_recall.tier_codec import StateRepairV2
    perms = tables(device)
    with StateRepairV2(model, perms, LAYOUTS) as rq:
        print("[controllers] tier", flush=True)
        h = rq.backbone(ids(device, 1, 3))
        h = rq.backbone(ids(device, 1, 1, seed=8))
        assert bool(torch.isfinite(h).all()) and rq.assert_finite_cache()
        assert rq.cache_bytes == CACHE_B1
        assert rq.storage_descriptor()["total_cache_bytes"] == CACHE_B1
    rng = np.random.default_rng(11)
    bases, scales, preds = [], [], []
    for layout in LAYOUTS:
        n8, n4, nz = cases.ridge_counts(layout)
        s = cases.ridge_statics(rng, 8, n8, n4, nz)
        bases.append(torch.from_numpy(s["basis"].view(np.float16)))
        scales.append(torch.from_numpy(s["lscale"].view(np.float16)))
        preds.append(torch.from_numpy(s["pred"].view(np.float16)))
    with ridge_codec.PredictorState(model, perms, LAYOUTS, bases, scales, preds) as pq:
        print("[controllers] ridge", flush=True)
        h = pq.backbone(ids(device, 2, 3))
        h = pq.backbone(ids(device, 2, 1, seed=9))
        assert bool(torch.isfinite(h).all()) and pq.assert_finite_cache()
        assert pq.cache_bytes == 2 * (CACHE_B1 - TABLE) + TABLE
        d = pq.storage_descriptor()
        assert d["static_predictor_bytes"] == sum(p.numel() * 2 for p in preds)
    bad = list(scales)
    bad[3] = torch.zeros_like(bad[3])
    with pytest.raises(ValueError, match="Static predictor/basis/scale allocation differs"):
        ridge_codec.PredictorState(model, perms, LAYOUTS, bases, bad, preds)


def test_repeated_reset_determinism(model, device):
    """The reference's runtime invariant (run_fp4_ridge_resurface_v3.py:90-99,
    cache_identity run_fp4_latent_state_quality_v1.py:49-61): two identical
    requests after a reset give identical hidden states and identical bytes in
    every cache tensor (convolution windows and packed rows), here for the
    ridge hook with a prefill and two one-token steps."""
    from mamba2_recall import ridge_codec
    perms = tables(device)
    rng = np.random.default_rng(12)
    bases, scales, preds = [], [], []
    for layout in LAYOUTS:
        n8, n4, nz = cases.ridge_counts(layout)
        s = cases.ridge_statics(rng, 8, n8, n4, nz)
        bases.append(torch.from_numpy(s["basis"].view(np.float16)))
        scales.append(torch.from_numpy(s["lscale"].view(np.float16)))
        preds.append(torch.from_numpy(s["pred"].view(np.float16)))
    tok = ids(device, 2, 6, seed=21)
    runs = []
    with ridge_codec.PredictorState(model, perms, LAYOUTS, bases, scales, preds) as pq:
        for attempt in range(2):
            print(f"[controllers] determinism run {attempt}", flush=True)
            hs = [pq.backbone(tok[:, :4], reset=True)]
            hs += [pq.backbone(tok[:, t:t + 1]) for t in (4, 5)]
            cache = [(e.conv.clone(), {k: v.clone() for k, v in e.state.tensors.items()}) for e in pq._cache]
            runs.append((hs, cache))
    (h0, c0), (h1, c1) = runs
    assert all(torch.equal(a, b) for a, b in zip(h0, h1))
    for (conv0, st0), (conv1, st1) in zip(c0, c1):
        assert torch.equal(conv0, conv1)
        assert all(torch.equal(st0[k], st1[k]) for k in st0)


def test_packed_projections(model, device):
    """use_packed_projections: the one-token in_proj/out_proj as packed FP4
    GEMVs.  Packets whose decode equals the module weights pass verify=True
    (the model's projections are first overwritten by the decode of seeded G16
    packets); a packet that decodes differently is rejected.  A 56-layer
    one-token step with the packed projections stays close to the FP16-module
    step: each projection differs only in summation order (within 1e-3,
    test_packed_projection_outputs_per_layer), but every layer requantizes its
    state, so a code that sits on a rounding boundary can move by one step and
    the differences compound over the 56 layers; 2e-2 bounds that drift of
    the final hidden state."""
    import math
    from mamba2_recall import fp4, ridge_codec
    gen = torch.Generator(device=device).manual_seed(31)

    def packet(w):
        rows, cols = w.shape
        packed = torch.randint(0, 256, (rows, cols // 2), generator=gen, device=device, dtype=torch.uint8)
        s = torch.exp(torch.randn((rows, cols // 16), generator=gen, device=device) * 0.5) / math.sqrt(8.5625 * cols)
        g = (s.max() / 448.0).float().reshape(1)
        sb = (s / g).clamp(0, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        fp4.decode_into(packed, sb, g, w.data, rows=rows, columns=cols, group=16)
        return packed, sb, g

    print("[controllers] packed projections: writing decoded packets into the projections", flush=True)
    packets = [dict(in_proj=packet(layer.mixer.in_proj.weight), out_proj=packet(layer.mixer.out_proj.weight))
               for layer in model.backbone.layers]
    perms = tables(device)
    rng = np.random.default_rng(14)
    bases, scales, preds = [], [], []
    for layout in LAYOUTS:
        n8, n4, nz = cases.ridge_counts(layout)
        s = cases.ridge_statics(rng, 8, n8, n4, nz)
        bases.append(torch.from_numpy(s["basis"].view(np.float16)))
        scales.append(torch.from_numpy(s["lscale"].view(np.float16)))
        preds.append(torch.from_numpy(s["pred"].view(np.float16)))
    tok = ids(device, 2, 5, seed=33)
    with ridge_codec.PredictorState(model, perms, LAYOUTS, bases, scales, preds) as pq:
        bad = list(packets)
        bad[5] = dict(in_proj=packets[6]["in_proj"], out_proj=packets[5]["out_proj"])
        with pytest.raises(ValueError, match="does not decode to the module's weight"):
            pq.use_packed_projections(bad, verify=True)
        pq.backbone(tok[:, :4], reset=True)
        snap = [(e.conv.clone(), {k: v.clone() for k, v in e.state.tensors.items()}) for e in pq._cache]
        h16 = pq.backbone(tok[:, 4:5])
        for e, (conv, tensors) in zip(pq._cache, snap):
            e.conv.copy_(conv)
            for k, v in tensors.items():
                e.state.tensors[k].copy_(v)
            e.tokens -= 1
        pq.use_packed_projections(packets, verify=True)
        hp = pq.backbone(tok[:, 4:5])
        pq.use_packed_projections(None)
        torch.cuda.synchronize()
        err = float((hp.float() - h16.float()).norm() / h16.float().norm())
        print(f"[controllers] packed vs FP16 one-token hidden rel L2 {err:.2e}", flush=True)
        assert bool(torch.isfinite(hp).all()) and err < 2e-2


class _AdapterHooks:
    """Hooks shaped like the Resurface adapter's (resurface_native.py:167-170,
    186-231): a mixer forward pre-hook that takes the mixer input, a norm
    forward pre-hook that replaces the norm's y with y + scale * [u, u] and
    marks the input consumed, and an always-call mixer forward hook that
    raises if the mixer returned without the norm hook having run."""

    def __init__(self, model, scale):
        self.scale = scale
        self.calls = [0] * len(model.backbone.layers)
        self.frames = {}
        self.handles = []
        for i, layer in enumerate(model.backbone.layers):
            mx = layer.mixer
            self.handles.append(mx.register_forward_pre_hook(self._input(i), with_kwargs=True))
            self.handles.append(mx.norm.register_forward_pre_hook(self._norm(i), with_kwargs=True))
            self.handles.append(mx.register_forward_hook(self._end(i), with_kwargs=True, always_call=True))

    def _input(self, i):
        def hook(module, args, kwargs):
            u = args[0] if args else kwargs["u"]
            assert i not in self.frames, "reentrant mixer call"
            self.frames[i] = {"u": u, "consumed": False}
        return hook

    def _norm(self, i):
        def hook(module, args, kwargs):
            frame = self.frames.get(i)
            if frame is None or frame["consumed"]:
                raise RuntimeError("Norm hook has no unique corresponding mixer input")
            y = args[0]
            u = frame["u"].reshape(*y.shape[:-1], 4096)
            frame["consumed"] = True
            self.calls[i] += 1
            return (y + self.scale * torch.cat((u, u), dim=-1), *args[1:]), kwargs
        return hook

    def _end(self, i):
        def hook(module, args, kwargs, output):
            frame = self.frames.pop(i, None)
            if frame is not None and output is not None and not frame["consumed"]:
                raise RuntimeError("Native mixer bypassed adapter injection")
        return hook

    def close(self):
        for h in self.handles:
            h.remove()


def _ridge_statics(seed):
    rng = np.random.default_rng(seed)
    bases, scales, preds = [], [], []
    for layout in LAYOUTS:
        n8, n4, nz = cases.ridge_counts(layout)
        s = cases.ridge_statics(rng, 8, n8, n4, nz)
        bases.append(torch.from_numpy(s["basis"].view(np.float16)))
        scales.append(torch.from_numpy(s["lscale"].view(np.float16)))
        preds.append(torch.from_numpy(s["pred"].view(np.float16)))
    return bases, scales, preds


def _g16_packets(model, device, seed):
    """Seeded G16 packets written into every projection (decoded weights), so
    the packed GEMVs and the modules hold the same weights."""
    import math
    from mamba2_recall import fp4
    gen = torch.Generator(device=device).manual_seed(seed)

    def packet(w):
        rows, cols = w.shape
        packed = torch.randint(0, 256, (rows, cols // 2), generator=gen, device=device, dtype=torch.uint8)
        s = torch.exp(torch.randn((rows, cols // 16), generator=gen, device=device) * 0.5) / math.sqrt(8.5625 * cols)
        g = (s.max() / 448.0).float().reshape(1)
        sb = (s / g).clamp(0, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        fp4.decode_into(packed, sb, g, w.data, rows=rows, columns=cols, group=16)
        return packed, sb, g

    return [dict(in_proj=packet(layer.mixer.in_proj.weight), out_proj=packet(layer.mixer.out_proj.weight))
            for layer in model.backbone.layers]


def test_resurface_hooks_under_the_predictor_controller(model, device):
    """The norm stays a module call under the controller: with the adapter's
    three hook kinds registered, the norm pre-hook fires exactly once per
    layer per backbone call (prefill, one-token steps, packed projections),
    its change reaches the hidden states (a zero change leaves them bit for
    bit), the end hook never reports a bypass, and a HIP graph captured with
    the hooks replays the hooked step."""
    from mamba2_recall import ridge_codec
    perms = tables(device)
    bases, scales, preds = _ridge_statics(15)
    tok = ids(device, 2, 6, seed=41)
    packets = _g16_packets(model, device, 43)
    with ridge_codec.PredictorState(model, perms, LAYOUTS, bases, scales, preds) as pq:
        pq.validate_each_step = False

        def run(hooks_scale, packed=False):
            hooks = _AdapterHooks(model, hooks_scale) if hooks_scale is not None else None
            try:
                pq.use_packed_projections(packets if packed else None)
                hs = [pq.backbone(tok[:, :4], reset=True)]
                hs += [pq.backbone(tok[:, t:t + 1]) for t in (4, 5)]
                torch.cuda.synchronize()
                return hs, (list(hooks.calls) if hooks else None)
            finally:
                pq.use_packed_projections(None)
                if hooks:
                    hooks.close()

        print("[controllers] resurface hooks: plain, zero-change and active runs", flush=True)
        plain, _ = run(None)
        zero, calls0 = run(0.0)
        active, calls = run(0.05)
        assert calls0 == [3] * 56 and calls == [3] * 56
        assert all(torch.equal(a, b) for a, b in zip(plain, zero))
        assert all(not torch.equal(a, b) for a, b in zip(plain, active))
        assert all(bool(torch.isfinite(h).all()) for h in active)
        print("[controllers] resurface hooks with packed projections", flush=True)
        packed_plain, _ = run(None, packed=True)
        packed_active, pcalls = run(0.05, packed=True)
        assert pcalls == [3] * 56
        assert torch.equal(packed_active[0], active[0])   # prefill keeps the modules
        assert all(not torch.equal(a, b) for a, b in zip(packed_plain[1:], packed_active[1:]))

        print("[controllers] resurface hooks captured in a HIP graph", flush=True)
        hooks = _AdapterHooks(model, 0.05)
        try:
            pq.backbone(tok[:, :4], reset=True)
            snap = [(e.conv.clone(), {k: v.clone() for k, v in e.state.tensors.items()}) for e in pq._cache]
            static = tok[:, 4:5].clone()
            eager = pq.backbone(static).clone()

            def restore():
                for e, (conv, tensors) in zip(pq._cache, snap):
                    e.conv.copy_(conv)
                    for k, v in tensors.items():
                        e.state.tensors[k].copy_(v)

            restore()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                pq.backbone(static)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            restore()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = pq.backbone(static)
            for _ in range(3):
                restore()
                graph.replay()
                torch.cuda.synchronize()
                assert torch.equal(out, eager)
            assert hooks.calls == [4] * 56   # prefill, eager step, side-stream warm-up, capture
            del graph
        finally:
            hooks.close()


def test_packed_projection_outputs_per_layer(model, device):
    """Each layer's packed FP4 GEMV projections against its FP16 modules on
    the same inputs (the decoded weights are identical; only the summation
    order differs): in_proj and out_proj outputs within 1e-3 relative L2, the
    north-star bar for layer outputs, at batch 1 and 4."""
    from mamba2_recall import fp4
    packets = _g16_packets(model, device, 45)
    gen = torch.Generator(device=device).manual_seed(46)
    worst = 0.0
    for batch in (1, 4):
        for index in (0, 27, 55):
            mx = model.backbone.layers[index].mixer
            for name, width in (("in_proj", 4096), ("out_proj", 8192)):
                u = torch.randn(batch, width, generator=gen, device=device).half()
                want = getattr(mx, name)(u).float()
                got = fp4.gemv_g16(*packets[index][name], u).float()
                err = float((got - want).norm() / want.norm())
                worst = max(worst, err)
                assert err <= 1e-3, (batch, index, name, err)
    print(f"[controllers] packed projections: worst rel L2 {worst:.2e}", flush=True)


def test_native_gated_norm_installed_and_restored(model, device):
    """While a controller owns the model, every mixer's gated norm is still a
    module call whose computation is the native kernel; close() restores the
    module's own forward.  With native_norm False the module keeps it, and
    the one-token output agrees with the native one within the norm's
    binary16 rounding propagated through the stack."""
    from mamba2_recall import state_quant
    from mamba2_recall.state_quant import StateQuant
    mixers = [layer.mixer for layer in model.backbone.layers]
    tok = ids(device, 1, 3, seed=31)
    print("[controllers] native gated norm install / restore", flush=True)
    with StateQuant(model, mode="s16") as sq:
        assert all(isinstance(mx.norm.__dict__.get("forward"), state_quant._NormHook) for mx in mixers)
        h_native = sq.backbone(tok)
    assert all("forward" not in mx.norm.__dict__ for mx in mixers)

    class Plain(StateQuant):
        native_norm = False
    with Plain(model, mode="s16") as sq:
        assert all("forward" not in mx.norm.__dict__ for mx in mixers)
        h_module = sq.backbone(tok)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(h_native).all()) and bool(torch.isfinite(h_module).all())
    rel = float((h_native.float() - h_module.float()).norm() / h_module.float().norm())
    assert rel < 2e-2, rel
