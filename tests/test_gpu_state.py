"""GPU parity of the fused state step against the CPU oracle.

Bar: packed codes, stored scales and latent bytes bit-exact; the FP16
readout y within 1e-3 relative L2 (north_star tolerance, FP32 accumulate).
Every case prints its identity before the device call.
"""
import numpy as np
import pytest
import torch

import cases
from cases import RIDGE_LAYOUTS, TIER_LAYOUTS, ridge_counts, tier_counts

pytestmark = pytest.mark.gpu

Y_TOL = 1e-3


def dev16(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def devp(a, device):
    """f16 params come as uint16 bits, f32 ones as float32."""
    if a.dtype == np.uint16:
        return dev16(a, device)
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def devp_shifted(a, device):
    """devp(a) at an address one element past an allocation's start: f16
    inputs then start on an odd multiple of 2 bytes."""
    t = devp(a, device)
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=device)
    buf[1:].copy_(t.reshape(-1))
    return buf[1:].view(t.shape)


def device_inputs(inp, device, shifted=()):
    return {k: (devp_shifted if k in shifted else devp)(v, device) for k, v in inp.items() if k != "perm"}


def to_state(np_state, state, device):
    for k, v in np_state.items():
        t = state.tensors[k]
        src = torch.from_numpy(np.ascontiguousarray(v))
        t.view(torch.uint8).copy_(src.view(torch.uint8).reshape(t.view(torch.uint8).shape).to(device))


def from_state(state):
    out = {}
    for k, t in state.tensors.items():
        u8 = t.view(torch.uint8).cpu().numpy()
        out[k] = u8.view(np.uint16).reshape(t.shape) if t.element_size() == 2 else u8.reshape(t.shape)
    return out


def assert_state_equal(got, want, what):
    for k in want:
        g, w = got[k], want[k]
        assert g.shape == w.shape, (what, k, g.shape, w.shape)
        bad = int((g.reshape(-1) != w.reshape(-1)).sum())
        assert bad == 0, f"{what}: {bad} mismatched {k} elements of {w.size}"


def assert_y_close(y_dev, y_ref, what):
    got = cases.f16_to_f32(y_dev.cpu().numpy().view(np.uint16))
    want = cases.f16_to_f32(y_ref)
    assert np.isfinite(got).all(), what
    err = cases.rel_l2(got, want)
    assert err <= Y_TOL, f"{what}: y rel L2 {err:.3e} > {Y_TOL}"
    return err


def plant_scales(rng, st0, fields, specials):
    """Writes the binary16 bit patterns `specials` into randomly chosen
    entries of the given scale fields (one field per entry, chosen at random)."""
    for bits in specials:
        f = fields[int(rng.integers(0, len(fields)))]
        flat = st0[f].reshape(-1)
        flat[int(rng.integers(0, flat.size))] = bits


def assert_y_pattern_close(y_dev, y_ref, what):
    """Readouts some of whose rows are not finite on both sides: the NaN and
    infinite positions agree, the finite rows are within the tolerance."""
    got = cases.f16_to_f32(y_dev.cpu().numpy().view(np.uint16))
    want = cases.f16_to_f32(y_ref)
    assert (np.isnan(got) == np.isnan(want)).all(), f"{what}: NaN readout rows differ"
    assert (np.isinf(got) == np.isinf(want)).all(), f"{what}: infinite readout rows differ"
    fin = np.isfinite(want)
    err = cases.rel_l2(got[fin], want[fin])
    assert err <= Y_TOL, f"{what}: y rel L2 {err:.3e} > {Y_TOL}"


NONFINITE_SCALES = [0x7C00, 0xFC00, 0x7E00, 0x7C00, 0xFE00, 0x7C00]


def run_ridge(oracle, device, layout, batch, L, H, P, G, seed, *, random_state=True, d_f32=False, db_f32=False,
              dt_bias_zero=True, x_scale=1.0, scale_mu=-4.0, special_scales=None, shifted=()):
    from mamba2_recall import ridge_codec
    n8, n4, nz = ridge_counts(layout)
    rng = np.random.default_rng(seed)
    inp = cases.step_inputs(rng, batch, L, H, P, G, d_f32=d_f32, db_f32=db_f32, dt_bias_zero=dt_bias_zero,
                            x_scale=x_scale)
    sta = cases.ridge_statics(rng, G, n8, n4, nz)
    st0 = (cases.random_packed_state(rng, batch, H, P, n8, n4, latent=True, scale_mu=scale_mu) if random_state
           else cases.zero_packed_state(batch, H, P, n8, n4, latent=True))
    if special_scales is not None:
        plant_scales(rng, st0, ("s8", "s4"), special_scales)
    print(f"[ridge] layout={layout} B={batch} L={L} H={H} P={P} G={G} seed={seed}", flush=True)
    ref_state = cases.copy_state(st0)
    y_ref = oracle.state_step(oracle.MODE_RIDGE, n8, n4, nz, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"],
                              inp["D"], inp["dt_bias"], inp["perm"], sta["basis"], sta["lscale"], sta["pred"],
                              ref_state)
    state = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
    to_state(st0, state, device)
    t = device_inputs(inp, device, shifted)
    perm = torch.from_numpy(inp["perm"]).to(device)
    basis, ls, pred = (dev16(sta[k], device) for k in ("basis", "lscale", "pred"))
    y, _ = ridge_codec.scan(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], state, perm, basis, ls,
                            pred, layout=layout)
    torch.cuda.synchronize()
    assert_state_equal(from_state(state), ref_state, f"ridge {layout}")
    if special_scales is not None:
        return assert_y_pattern_close(y, y_ref, f"ridge {layout}")
    return assert_y_close(y, y_ref, f"ridge {layout}")


def run_tier(oracle, device, kind, layout, batch, L, H, P, G, seed, *, random_state=True, d_f32=False,
             db_f32=False, dt_bias_zero=True, x_scale=1.0, scale_mu=-4.0, special_scales=None, shifted=()):
    from mamba2_recall import state_codec, tier_codec
    n8, n4, nz = tier_counts(layout)
    rng = np.random.default_rng(seed)
    inp = cases.step_inputs(rng, batch, L, H, P, G, d_f32=d_f32, db_f32=db_f32, dt_bias_zero=dt_bias_zero,
                            x_scale=x_scale)
    st0 = (cases.random_packed_state(rng, batch, H, P, n8, n4, scale_mu=scale_mu) if random_state
           else cases.zero_packed_state(batch, H, P, n8, n4))
    if special_scales is not None:
        plant_scales(rng, st0, ("s8", "s4"), special_scales)
    print(f"[{kind}] layout={layout} B={batch} L={L} H={H} P={P} G={G} seed={seed}", flush=True)
    ref_state = cases.copy_state(st0)
    mode = oracle.MODE_LEGACY if kind == "legacy" else oracle.MODE_STORED
    y_ref = oracle.state_step(mode, n8, n4, nz, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"],
                              inp["dt_bias"], inp["perm"], None, None, None, ref_state)
    t = device_inputs(inp, device, shifted)
    perm = torch.from_numpy(inp["perm"]).to(device)
    if kind == "legacy":
        state = state_codec.allocate_state(batch, H, P, 128, "sq3p25", device)
        to_state(st0, state, device)
        y, _ = state_codec.scan(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], state, perm)
    else:
        state = tier_codec.allocate_state(batch, H, P, 128, device, layout=layout)
        to_state(st0, state, device)
        y, _ = tier_codec.scan(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], state, perm,
                               layout=layout)
    torch.cuda.synchronize()
    assert_state_equal(from_state(state), ref_state, f"{kind} {layout}")
    if special_scales is not None:
        return assert_y_pattern_close(y, y_ref, f"{kind} {layout}")
    return assert_y_close(y, y_ref, f"{kind} {layout}")


@pytest.mark.parametrize("layout", RIDGE_LAYOUTS)
def test_ridge_one_token_model_geometry(oracle, device, layout):
    run_ridge(oracle, device, layout, batch=2, L=1, H=128, P=64, G=8, seed=11)


@pytest.mark.parametrize("layout", RIDGE_LAYOUTS)
def test_ridge_multi_token(oracle, device, layout):
    run_ridge(oracle, device, layout, batch=1, L=5, H=128, P=64, G=8, seed=12)


@pytest.mark.parametrize("L", [1, 17, 65])
def test_ridge_reference_fixture_geometry(oracle, device, L):
    # scripts/check_state_ridge_training_v3.py:28 uses b,h,p,g = 1,8,16,2
    for layout in RIDGE_LAYOUTS:
        run_ridge(oracle, device, layout, batch=1, L=L, H=8, P=16, G=2, seed=13 + L, random_state=False)


@pytest.mark.parametrize("x_scale,scale_mu", [(1e-5, -14.0), (3e-7, -17.0), (1e-9, -24.0)])
def test_tiny_states_subnormal_stored_scales(oracle, device, x_scale, scale_mu):
    """Updates small enough that the new stored scales are binary16
    subnormals or underflow to zero: the rounded quotient can exceed the
    limit there, so these rows take the clamping quantizer."""
    run_ridge(oracle, device, "32_32_64", 2, 3, 32, 64, 2, 71, x_scale=x_scale, scale_mu=scale_mu)
    run_tier(oracle, device, "tier", "16_64_48", 2, 3, 32, 64, 2, 72, x_scale=x_scale, scale_mu=scale_mu)
    run_tier(oracle, device, "legacy", "16_64_48", 2, 3, 32, 64, 2, 73, x_scale=x_scale, scale_mu=scale_mu)


def test_ridge_zero_state_and_f32_params(oracle, device):
    run_ridge(oracle, device, "32_32_64", batch=3, L=2, H=128, P=64, G=8, seed=14, random_state=False,
              d_f32=True, db_f32=True, dt_bias_zero=False)


def test_ridge_wide_batch_four_wave_blocks(oracle, device):
    # batch * heads * p-blocks >= 4096 selects the 4-wave workgroups
    run_ridge(oracle, device, "24_48_56", batch=32, L=1, H=128, P=64, G=8, seed=15)


def test_ridge_ragged_p(oracle, device):
    run_ridge(oracle, device, "36_24_68", batch=2, L=2, H=16, P=80, G=2, seed=16)


@pytest.mark.parametrize("layout", RIDGE_LAYOUTS)
def test_ridge_model_batch_sixteen_head_blocks(oracle, device, layout):
    # the benchmark geometry (batch 64, one token) selects 16 heads per
    # workgroup: every one-token instance the headline benchmark times
    run_ridge(oracle, device, layout, batch=64, L=1, H=128, P=64, G=8, seed=19)


def test_tier_and_legacy_benchmark_geometry(oracle, device):
    # the batch-64 one-token instances of the other packed formats that the
    # benchmark times beside the ridge step
    run_tier(oracle, device, "tier", "32_32_64", batch=64, L=1, H=128, P=64, G=8, seed=24)
    run_tier(oracle, device, "legacy", "16_64_48", batch=64, L=1, H=128, P=64, G=8, seed=33)


def test_ridge_unvalidated_scan_still_checks_table_shapes(device):
    """validate=False skips only the synchronizing value checks: a predictor,
    permutation or basis of the wrong shape or dtype is rejected before the
    kernel would index past it."""
    from mamba2_recall import ridge_codec
    layout = "32_32_64"
    n8, n4, nz = ridge_counts(layout)
    rng = np.random.default_rng(90)
    inp = cases.step_inputs(rng, 1, 1, 128, 64, 8)
    sta = cases.ridge_statics(rng, 8, n8, n4, nz)
    print("[ridge validate=False] mis-shaped statics", flush=True)
    state = ridge_codec.allocate_state(1, 128, 64, 128, device, layout=layout)
    t = {k: devp(v, device) for k, v in inp.items() if k != "perm"}
    perm = torch.from_numpy(inp["perm"]).to(device)
    basis, ls, pred = (dev16(sta[k], device) for k in ("basis", "lscale", "pred"))
    args = (t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], state)
    with pytest.raises(ValueError, match="predictor differs"):
        ridge_codec.scan(*args, perm, basis, ls, pred[:, :-4].contiguous(), layout=layout, validate=False)
    with pytest.raises(ValueError, match="predictor differs"):
        ridge_codec.scan(*args, perm, basis, ls, pred.float(), layout=layout, validate=False)
    with pytest.raises(ValueError, match="basis/scales differ"):
        ridge_codec.scan(*args, perm[:4], basis, ls, pred, layout=layout, validate=False)
    with pytest.raises(ValueError, match="basis/scales differ"):
        ridge_codec.scan(*args, perm, basis[:, :8], ls, pred, layout=layout, validate=False)
    before = {k: v.clone() for k, v in state.tensors.items()}
    torch.cuda.synchronize()
    assert all(torch.equal(before[k], state.tensors[k]) for k in before)


SHAPES = [(1, 1), (4, 1), (4, 2), (4, 4), (8, 2), (4, 0), (4, -4)]


@pytest.fixture
def forced_shape(request):
    from mamba2_recall import _native
    _native.call("m2r_set_step_shape", *request.param)
    yield request.param
    _native.call("m2r_set_step_shape", 0, 0)


@pytest.mark.parametrize("L", [1, 3])
def test_ridge_every_shape_same_bits(device, L):
    """Every workgroup shape of four or eight waves, including the slots on
    two and four waves (whose waves step parts of a tier and share the tier
    maxima and the readout partial sums), gives the same codes, scales and y
    bit for bit: the readout is summed per segment of the carried coordinates
    in one fixed order, and the ridge correction is split the same way.  (The
    one-wave workgroups compute the correction of the readout weights in
    another order: the same codes, y within the oracle tolerance, checked by
    the per-shape tests.)  Layouts whose INT4 tier is split between waves,
    whose INT8 tier is, and neither."""
    from mamba2_recall import _native, ridge_codec
    for layout in ("8_80_40", "24_48_56", "36_24_68", "44_8_76"):
        n8, n4, nz = ridge_counts(layout)
        rng = np.random.default_rng(90 + L)
        B, H, P, G = 2, 16, 64, 1
        inp = cases.step_inputs(rng, B, L, H, P, G)
        sta = cases.ridge_statics(rng, G, n8, n4, nz)
        st0 = cases.random_packed_state(rng, B, H, P, n8, n4, latent=True)
        t = device_inputs(inp, device)
        perm = torch.from_numpy(inp["perm"]).to(device)
        basis, ls, pred = (dev16(sta[k], device) for k in ("basis", "lscale", "pred"))
        results = []
        try:
            for shape in [sh for sh in SHAPES if sh[0] >= 4]:
                print(f"[same bits] layout={layout} L={L} shape={shape}", flush=True)
                _native.call("m2r_set_step_shape", *shape)
                state = ridge_codec.allocate_state(B, H, P, 128, device, layout=layout)
                to_state(st0, state, device)
                y, _ = ridge_codec.scan(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], state, perm,
                                        basis, ls, pred, layout=layout)
                torch.cuda.synchronize()
                results.append((shape, y.view(torch.int16).clone(),
                                {k: v.view(torch.uint8).clone() for k, v in state.tensors.items()}))
        finally:
            _native.call("m2r_set_step_shape", 0, 0)
        shape0, y0, s0 = results[0]
        for shape, y, st in results[1:]:
            assert torch.equal(y, y0), (layout, L, shape, shape0)
            for k in s0:
                assert torch.equal(st[k], s0[k]), (layout, L, shape, k)


def _ridge_step_direct(t, perm, basis, ls, pred, state, layout, ws):
    """One m2r_state_step_ridge_ws call (ws: a workspace tensor or None)."""
    from mamba2_recall import _native
    n8, n4, nz = ridge_counts(layout)
    p = _native.ptr
    batch, L, H, P = t["x"].shape
    G = t["B"].shape[2]
    y = torch.empty_like(t["x"])
    st = state.tensors
    _native.call("m2r_state_step_ridge_ws", p(t["x"]), p(t["dt"]), p(t["A"]), p(t["B"]), p(t["C"]), p(t["D"]),
                 int(t["D"].dtype == torch.float32), p(t["dt_bias"]), int(t["dt_bias"].dtype == torch.float32),
                 p(perm), p(basis), p(ls), p(pred), p(st["lo"]), p(st["hi"]), p(st["q4"]), p(st["latent"]),
                 p(st["s8"]), p(st["s4"]), p(y), batch, L, H, P, G, n8, n4, nz, p(ws),
                 0 if ws is None else ws.numel() * 4, _native.stream_of(t["x"]))
    return y


@pytest.mark.parametrize("layout", RIDGE_LAYOUTS)
def test_ridge_token_records_same_bits_as_in_kernel_build(device, layout):
    """Multi-token launches of the shapes with several waves per slot read
    their tokens' state-independent values from records a first kernel wrote
    (the split token build of four waves, run per token): codes, scales,
    latent bytes and y equal the in-kernel build's bit for bit, with the
    automatic shape (four or two waves per slot) and forced two- and four-wave
    slots, token counts that are and are not multiples of the records
    kernel's 8 tokens per workgroup, batch rows 1 to 3, and a ragged head
    dimension (P = 72: a second, partly filled 64-row block per head)."""
    from mamba2_recall import _native, ridge_codec
    n8, n4, nz = ridge_counts(layout)
    H, G = 128, 8
    try:
        for shape in ((0, 0), (4, 0), (4, -4)):
            for batch, L, P in ((1, 37, 64), (2, 16, 64), (1, 2, 64), (3, 19, 72)):
                print(f"[token records] layout={layout} shape={shape} B={batch} L={L} P={P}", flush=True)
                _native.call("m2r_set_step_shape", *shape)
                rng = np.random.default_rng(700 + batch * 100 + L)
                inp = cases.step_inputs(rng, batch, L, H, P, G)
                sta = cases.ridge_statics(rng, G, n8, n4, nz)
                st0 = cases.random_packed_state(rng, batch, H, P, n8, n4, latent=True)
                t = device_inputs(inp, device)
                perm = torch.from_numpy(inp["perm"]).to(device)
                basis, ls, pred = (dev16(sta[k], device) for k in ("basis", "lscale", "pred"))
                ws_bytes = int(_native.lib().m2r_ridge_records_bytes(batch, L, G))
                assert ws_bytes == batch * L * G * 1024
                # poison the workspace: every record value must come from the records kernel
                ws = torch.full((ws_bytes // 4,), float("nan"), dtype=torch.float32, device=device)
                s_build = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
                s_rec = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
                to_state(st0, s_build, device)
                to_state(st0, s_rec, device)
                y_build = _ridge_step_direct(t, perm, basis, ls, pred, s_build, layout, None)
                y_rec = _ridge_step_direct(t, perm, basis, ls, pred, s_rec, layout, ws)
                torch.cuda.synchronize()
                assert torch.equal(y_rec.view(torch.int16), y_build.view(torch.int16)), (layout, shape, batch, L, P)
                for k in s_build.tensors:
                    assert torch.equal(s_rec.tensors[k].view(torch.uint8), s_build.tensors[k].view(torch.uint8)), \
                        (layout, shape, batch, L, P, k)
                assert not torch.isnan(ws).all()   # the records path ran
    finally:
        _native.call("m2r_set_step_shape", 0, 0)


def test_ridge_token_records_graph_replays_match_eager(device):
    """The records kernel and the record-fed step captured in a HIP graph
    (one workspace, static inputs): three replays, each from the same
    starting state (reset eagerly in between), give the eager call's codes,
    scales, latent bytes and y bit for bit."""
    from mamba2_recall import _native, ridge_codec
    layout = "24_48_56"
    n8, n4, nz = ridge_counts(layout)
    batch, L, H, P, G = 1, 37, 128, 64, 8
    print(f"[token records graph] layout={layout} B={batch} L={L}", flush=True)
    rng = np.random.default_rng(4242)
    inp = cases.step_inputs(rng, batch, L, H, P, G)
    sta = cases.ridge_statics(rng, G, n8, n4, nz)
    st0 = cases.random_packed_state(rng, batch, H, P, n8, n4, latent=True)
    t = device_inputs(inp, device)
    perm = torch.from_numpy(inp["perm"]).to(device)
    basis, ls, pred = (dev16(sta[k], device) for k in ("basis", "lscale", "pred"))
    ws = torch.empty(int(_native.lib().m2r_ridge_records_bytes(batch, L, G)) // 4, dtype=torch.float32, device=device)
    s_eager = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
    to_state(st0, s_eager, device)
    y_eager = _ridge_step_direct(t, perm, basis, ls, pred, s_eager, layout, ws)
    torch.cuda.synchronize()
    s_graph = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
    to_state(st0, s_graph, device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # warm-up outside the capture
        _ridge_step_direct(t, perm, basis, ls, pred, s_graph, layout, ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_graph = _ridge_step_direct(t, perm, basis, ls, pred, s_graph, layout, ws)
    for rep in range(3):
        to_state(st0, s_graph, device)
        ws.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph.view(torch.int16), y_eager.view(torch.int16)), rep
        for k in s_eager.tensors:
            assert torch.equal(s_graph.tensors[k].view(torch.uint8), s_eager.tensors[k].view(torch.uint8)), (rep, k)


@pytest.mark.parametrize("forced_shape", SHAPES, indirect=True, ids=lambda s: f"w{s[0]}h{s[1]}")
def test_ridge_every_workgroup_shape(oracle, device, forced_shape):
    """Each (waves, head slots per wave) variant: multi-token, ragged P, one
    group and several (the ridge format needs P % 16 == 0)."""
    run_ridge(oracle, device, "32_32_64", batch=2, L=3, H=32, P=80, G=2, seed=61)
    run_ridge(oracle, device, "8_80_40", batch=1, L=2, H=16, P=48, G=1, seed=62)
    run_ridge(oracle, device, "44_8_76", batch=3, L=1, H=16, P=64, G=1, seed=63, random_state=False)


@pytest.mark.parametrize("forced_shape", SHAPES, indirect=True, ids=lambda s: f"w{s[0]}h{s[1]}")
def test_one_token_staged_inputs_every_workgroup_shape(oracle, device, forced_shape):
    """One-token steps, whose instances with an even number of heads per
    workgroup stage x, dt, dt_bias, A, D, B, C and the statics in LDS by
    dword transfers: f16 and f32 D and dt_bias (nonzero), ragged P (second
    P block of 16 rows), one group and several, every packed format."""
    run_ridge(oracle, device, "32_32_64", batch=2, L=1, H=32, P=80, G=2, seed=66, d_f32=True, db_f32=True,
              dt_bias_zero=False)
    run_ridge(oracle, device, "8_80_40", batch=3, L=1, H=16, P=64, G=1, seed=67, dt_bias_zero=False)
    run_tier(oracle, device, "tier", "40_16_72", batch=2, L=1, H=32, P=80, G=2, seed=68, d_f32=True,
             dt_bias_zero=False)
    run_tier(oracle, device, "legacy", "16_64_48", batch=2, L=1, H=16, P=64, G=1, seed=69, db_f32=True,
             dt_bias_zero=False)


@pytest.mark.parametrize("kind", ["ridge", "tier"])
def test_one_token_unaligned_inputs_take_the_register_prologue(oracle, device, kind):
    """f16 inputs that start 2 bytes past a dword (views one element into
    their allocations) cannot be staged by dword transfers: the one-token
    step then loads them into registers, with the same results."""
    shifted = ("x", "dt", "D", "dt_bias")
    if kind == "ridge":
        run_ridge(oracle, device, "24_48_56", batch=64, L=1, H=128, P=64, G=8, seed=70, dt_bias_zero=False,
                  shifted=shifted)
    else:
        run_tier(oracle, device, "tier", "32_32_64", batch=64, L=1, H=128, P=64, G=8, seed=71,
                 dt_bias_zero=False, shifted=shifted)


@pytest.mark.parametrize("forced_shape", SHAPES, indirect=True, ids=lambda s: f"w{s[0]}h{s[1]}")
def test_tier_and_legacy_every_workgroup_shape(oracle, device, forced_shape):
    # odd P exercises the 16-bit row staging
    run_tier(oracle, device, "tier", "36_24_68", batch=2, L=3, H=32, P=80, G=2, seed=64)
    run_tier(oracle, device, "legacy", "16_64_48", batch=1, L=2, H=16, P=33, G=1, seed=65)


@pytest.mark.parametrize("layout", TIER_LAYOUTS)
def test_tier_one_token(oracle, device, layout):
    run_tier(oracle, device, "tier", layout, batch=2, L=1, H=128, P=64, G=8, seed=21)


@pytest.mark.parametrize("layout", TIER_LAYOUTS)
def test_tier_multi_token_small(oracle, device, layout):
    run_tier(oracle, device, "tier", layout, batch=1, L=17, H=8, P=16, G=2, seed=22, random_state=False)


def test_tier_wide_batch(oracle, device):
    run_tier(oracle, device, "tier", "8_80_40", batch=32, L=1, H=128, P=64, G=8, seed=23)


def test_legacy_one_and_multi_token(oracle, device):
    run_tier(oracle, device, "legacy", "16_64_48", batch=2, L=1, H=128, P=64, G=8, seed=31)
    run_tier(oracle, device, "legacy", "16_64_48", batch=1, L=9, H=128, P=64, G=8, seed=32, random_state=False,
             d_f32=True, dt_bias_zero=False)


def test_sequential_tokens_equal_one_call(oracle, device):
    """L tokens in one call == L calls of one token (the carry between tokens
    is exactly the dequantized codes)."""
    from mamba2_recall import ridge_codec
    layout = "40_16_72"
    n8, n4, nz = ridge_counts(layout)
    rng = np.random.default_rng(41)
    batch, L, H, P, G = 2, 6, 128, 64, 8
    inp = cases.step_inputs(rng, batch, L, H, P, G)
    sta = cases.ridge_statics(rng, G, n8, n4, nz)
    st0 = cases.random_packed_state(rng, batch, H, P, n8, n4, latent=True)
    t = {k: devp(v, device) for k, v in inp.items() if k != "perm"}
    perm = torch.from_numpy(inp["perm"]).to(device)
    basis, ls, pred = (dev16(sta[k], device) for k in ("basis", "lscale", "pred"))
    s_all = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
    s_seq = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
    to_state(st0, s_all, device)
    to_state(st0, s_seq, device)
    y_all, _ = ridge_codec.scan(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], s_all, perm, basis,
                                ls, pred, layout=layout)
    ys = []
    for i in range(L):
        sl = slice(i, i + 1)
        y1, _ = ridge_codec.scan(t["x"][:, sl], t["dt"][:, sl], t["A"], t["B"][:, sl], t["C"][:, sl], t["D"],
                                 t["dt_bias"], s_seq, perm, basis, ls, pred, layout=layout, validate=False)
        ys.append(y1)
    torch.cuda.synchronize()
    assert_state_equal(from_state(s_seq), from_state(s_all), "sequential vs one call")
    assert torch.equal(torch.cat(ys, 1), y_all)


@pytest.mark.parametrize("layout,L", [("8_80_40", 2048), ("36_24_68", 300), ("44_8_76", 300)])
def test_prefill_window_equals_token_by_token(device, layout, L):
    """The reference's prefill shape (batch 1, 128 heads, 8 groups): one
    multi-token call (four waves per 64-row slot, the dt activation and its
    batches of 64 tokens) leaves the same packed state and y bits as L
    one-token calls (two waves per slot), up to a whole 2048-token window."""
    from mamba2_recall import ridge_codec
    n8, n4, nz = ridge_counts(layout)
    rng = np.random.default_rng(L)
    batch, H, P, G = 1, 128, 64, 8
    print(f"[prefill window] layout={layout} L={L}", flush=True)
    inp = cases.step_inputs(rng, batch, L, H, P, G)
    sta = cases.ridge_statics(rng, G, n8, n4, nz)
    st0 = cases.random_packed_state(rng, batch, H, P, n8, n4, latent=True)
    t = {k: devp(v, device) for k, v in inp.items() if k != "perm"}
    perm = torch.from_numpy(inp["perm"]).to(device)
    basis, ls, pred = (dev16(sta[k], device) for k in ("basis", "lscale", "pred"))
    s_all = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
    s_seq = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
    to_state(st0, s_all, device)
    to_state(st0, s_seq, device)
    y_all, _ = ridge_codec.scan(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], s_all, perm, basis,
                                ls, pred, layout=layout)
    y_seq = torch.empty_like(y_all)
    for i in range(L):
        sl = slice(i, i + 1)
        y1, _ = ridge_codec.scan(t["x"][:, sl], t["dt"][:, sl], t["A"], t["B"][:, sl], t["C"][:, sl], t["D"],
                                 t["dt_bias"], s_seq, perm, basis, ls, pred, layout=layout, validate=False)
        y_seq[:, sl] = y1
    torch.cuda.synchronize()
    assert_state_equal(from_state(s_seq), from_state(s_all), f"prefill window {layout} L={L}")
    assert torch.equal(y_seq.view(torch.int16), y_all.view(torch.int16))
    assert torch.isfinite(y_all).all()


def run_dense3(oracle, device, kind, batch, L, H, P, G, seed, *, random_state=True, x_scale=1.0, scale_mu=-2.0,
               special_scales=None, nonfinite_y=False):
    """`special_scales`: binary16 bit patterns written into the scales of a
    few rows (infinite or NaN stored scales).  Such rows' readout, and that of
    rows whose readout overflows binary16 (`nonfinite_y`), is not finite on
    both sides: y is then compared on the finite rows, plus the pattern of
    NaN and infinite values."""
    from mamba2_recall import state_codec_dense3 as d3
    rng = np.random.default_rng(seed)
    inp = cases.step_inputs(rng, batch, L, H, P, G, x_scale=x_scale)
    if kind == "equalizer":
        table = rng.integers(-8, 9, size=(G, 128)).astype(np.int8)
    else:
        table = inp["perm"]
    rows = (batch, H, P)
    if random_state:
        st0 = dict(codes=rng.integers(0, 256, size=rows + (3, 16), dtype=np.uint16).astype(np.uint8),
                   scales=cases.f16(np.exp(rng.normal(scale_mu, 0.5, size=rows + (2,)))))
    else:
        st0 = dict(codes=np.zeros(rows + (3, 16), np.uint8), scales=np.zeros(rows + (2,), np.uint16))
    if special_scales is not None:
        plant_scales(rng, st0, ("scales",), special_scales)
    print(f"[dense3 {kind}] B={batch} L={L} H={H} P={P} G={G} seed={seed}", flush=True)
    ref = cases.copy_state(st0)
    y_ref = oracle.dense3_step(1 if kind == "equalizer" else 0, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"],
                               inp["D"], inp["dt_bias"], np.ascontiguousarray(table), ref)
    state = d3.allocate_state(batch, H, P, 128, device)
    to_state(st0, state, device)
    t = {k: devp(v, device) for k, v in inp.items() if k != "perm"}
    y = d3.scan(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], state,
                torch.from_numpy(np.ascontiguousarray(table)).to(device), kind)
    torch.cuda.synchronize()
    assert_state_equal(from_state(state), ref, f"dense3 {kind}")
    if special_scales is not None or nonfinite_y:
        return assert_y_pattern_close(y, y_ref, f"dense3 {kind}")
    return assert_y_close(y, y_ref, f"dense3 {kind}")


@pytest.mark.parametrize("kind", ["permutation", "equalizer"])
def test_dense3_one_token(oracle, device, kind):
    run_dense3(oracle, device, kind, batch=2, L=1, H=128, P=64, G=8, seed=51)


@pytest.mark.parametrize("kind", ["permutation", "equalizer"])
def test_dense3_multi_token_small(oracle, device, kind):
    run_dense3(oracle, device, kind, batch=1, L=9, H=8, P=16, G=2, seed=52, random_state=False)


def test_dense3_wide_batch(oracle, device):
    run_dense3(oracle, device, "permutation", batch=32, L=1, H=128, P=64, G=8, seed=53)


def test_dense3_benchmark_geometry(oracle, device):
    # batch 64, one token: 16 heads per workgroup (four waves of four slots)
    run_dense3(oracle, device, "permutation", batch=64, L=1, H=128, P=64, G=8, seed=54)
    run_dense3(oracle, device, "equalizer", batch=64, L=1, H=128, P=64, G=8, seed=55)


D3_SHAPES = [(1, 1), (4, 1), (4, 2), (4, 4)]


@pytest.mark.parametrize("forced_shape", D3_SHAPES, indirect=True, ids=lambda s: f"w{s[0]}h{s[1]}")
def test_dense3_every_workgroup_shape(oracle, device, forced_shape):
    """Each (waves, head slots per wave) variant of the streaming kernel:
    multi-token with ragged P (a 16-row second slot), one group and several,
    one token from a zero state, both table kinds."""
    run_dense3(oracle, device, "permutation", batch=2, L=3, H=32, P=80, G=2, seed=56)
    run_dense3(oracle, device, "equalizer", batch=1, L=2, H=16, P=48, G=1, seed=57)
    run_dense3(oracle, device, "permutation", batch=3, L=1, H=16, P=68, G=1, seed=58, random_state=False)


def test_dense3_unaligned_geometry_staged_kernel(oracle, device):
    # P % 4 != 0: slots cannot move as 16-byte transfers; the staged kernel runs
    run_dense3(oracle, device, "permutation", batch=2, L=3, H=16, P=18, G=2, seed=59)
    run_dense3(oracle, device, "equalizer", batch=1, L=1, H=8, P=33, G=1, seed=60)


@pytest.mark.parametrize("x_scale,scale_mu", [(1e-5, -14.0), (1e-9, -24.0)])
def test_dense3_tiny_states(oracle, device, x_scale, scale_mu):
    """Half-row maxima small enough that den is the 1e-8 floor."""
    run_dense3(oracle, device, "permutation", batch=2, L=3, H=32, P=64, G=2, seed=66, x_scale=x_scale,
               scale_mu=scale_mu)


def test_dense3_large_states(oracle, device):
    """Updates large enough that some new stored scales overflow binary16 (and
    some readouts with them)."""
    run_dense3(oracle, device, "permutation", batch=2, L=1, H=32, P=64, G=2, seed=69, x_scale=1e4, scale_mu=6.0,
               nonfinite_y=True)


def test_dense3_non_finite_scales(oracle, device):
    """Rows whose stored scale is +inf, -inf or NaN: their updates are not
    finite, their maxima infinite, and the clamping quantizer with the
    infinite-den division runs (NaN quotients clamp to -3)."""
    run_dense3(oracle, device, "permutation", batch=2, L=1, H=32, P=64, G=2, seed=67,
               special_scales=NONFINITE_SCALES)
    run_dense3(oracle, device, "equalizer", batch=1, L=2, H=16, P=64, G=1, seed=68,
               special_scales=NONFINITE_SCALES)
    run_dense3(oracle, device, "permutation", batch=1, L=2, H=16, P=18, G=1, seed=70,
               special_scales=NONFINITE_SCALES)   # the staged kernel


def test_packed_rows_non_finite_scales(oracle, device):
    """Packed rows whose INT8 or INT4 stored scale is +inf, -inf or NaN: the
    tier maximum is infinite (den = inf) or the updates NaN, for the ridge,
    stored-scale tier and legacy formats."""
    run_ridge(oracle, device, "32_32_64", batch=2, L=2, H=32, P=64, G=2, seed=74, special_scales=NONFINITE_SCALES)
    run_tier(oracle, device, "tier", "24_48_56", batch=2, L=2, H=32, P=64, G=2, seed=75,
             special_scales=NONFINITE_SCALES)
    run_tier(oracle, device, "legacy", "16_64_48", batch=2, L=2, H=32, P=64, G=2, seed=76,
             special_scales=NONFINITE_SCALES)


def run_s16(oracle, device, batch, L, H, P, G, seed, collect):
    from mamba2_recall import state_codec
    rng = np.random.default_rng(seed)
    inp = cases.step_inputs(rng, batch, L, H, P, G)
    st0 = cases.f16(rng.standard_normal((batch, H, P, 128)) * 0.5)
    print(f"[s16] B={batch} L={L} H={H} P={P} G={G} seed={seed} stats={collect}", flush=True)
    ref = st0.copy()
    y_ref, s_ref = oracle.s16_step(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["dt_bias"], ref,
                                   collect_stats=collect)
    state = state_codec.allocate_state(batch, H, P, 128, "s16", device)
    state.tensors["state"].copy_(dev16(st0, device))
    t = {k: devp(v, device) for k, v in inp.items() if k != "perm"}
    y, stats = state_codec.scan(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], state,
                                collect_stats=collect)
    torch.cuda.synchronize()
    got = state.tensors["state"].cpu().numpy().view(np.uint16)
    assert int((got != ref).sum()) == 0, "s16 carry differs"
    assert_y_close(y, y_ref, "s16")
    if collect:
        s = stats.cpu().numpy()
        assert s.shape == s_ref.shape
        # one fixed summation order on both sides: equal bit for bit
        assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32)), "s16 statistics differ"
    else:
        assert stats is None


def test_s16_control_step(oracle, device):
    run_s16(oracle, device, 2, 3, 128, 64, 8, 81, collect=False)
    run_s16(oracle, device, 1, 5, 16, 40, 2, 82, collect=True)      # ragged statistics tile
    run_s16(oracle, device, 2, 7, 32, 64, 4, 83, collect=True)      # whole tiles, several tokens


def test_s16_statistics_same_on_every_run(oracle, device):
    """The statistics feed a stable argsort of per-coordinate means
    (scripts/run_statequant.py:83): the same data must give the same bits on
    every run, so two runs of one call are compared bit for bit."""
    from mamba2_recall import state_codec
    rng = np.random.default_rng(84)
    batch, L, H, P, G = 2, 9, 64, 64, 4
    inp = cases.step_inputs(rng, batch, L, H, P, G)
    st0 = cases.f16(rng.standard_normal((batch, H, P, 128)) * 0.5)
    t = {k: devp(v, device) for k, v in inp.items() if k != "perm"}
    runs = []
    for _ in range(3):
        state = state_codec.allocate_state(batch, H, P, 128, "s16", device)
        state.tensors["state"].copy_(dev16(st0, device))
        _, stats = state_codec.scan(t["x"], t["dt"], t["A"], t["B"], t["C"], t["D"], t["dt_bias"], state,
                                    collect_stats=True)
        runs.append(stats.cpu().numpy().view(np.uint32).copy())
    assert all(np.array_equal(runs[0], r) for r in runs[1:])


def test_ridge_2048_token_drift_batch64(oracle, device):
    """The batch-64 drift check of the 56-layer benchmark configuration, on one
    layer: independent seeded inputs per sequence, 2048 consecutive tokens in
    blocks of 128 that alternate between 128 one-token calls (the per-token
    requantize hook's pattern) and one 128-token call.  After every block the
    packed state of sequences 0, 13, 37 and 63 equals the CPU oracle's bit for
    bit, and their readout is within the tolerance."""
    from mamba2_recall import ridge_codec
    layout = "8_80_40"
    n8, n4, nz = ridge_counts(layout)
    batch, H, P, G, blocks, blk = 64, 128, 64, 8, 16, 128
    sub = [0, 13, 37, 63]
    rng = np.random.default_rng(2048)
    par = cases.step_inputs(rng, 1, 1, H, P, G)          # A, D, dt_bias, perm
    sta = cases.ridge_statics(rng, G, n8, n4, nz)
    st0 = cases.random_packed_state(rng, batch, H, P, n8, n4, latent=True)

    def rows_of(a):   # packed arrays are [batch, heads, dim, ...]
        return np.ascontiguousarray(a[sub])

    ref_state = {k: rows_of(v) for k, v in st0.items()}
    state = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
    to_state(st0, state, device)
    A = torch.from_numpy(par["A"]).to(device)
    D, db = dev16(par["D"], device), dev16(par["dt_bias"], device)
    perm = torch.from_numpy(par["perm"]).to(device)
    basis, ls, pred = (dev16(sta[k], device) for k in ("basis", "lscale", "pred"))
    for k in range(blocks):
        gen = torch.Generator(device=device).manual_seed(4096 + k)
        x = torch.randn(batch, blk, H, P, generator=gen, device=device).half()
        dt = torch.randn(batch, blk, H, generator=gen, device=device).half()
        Bm = torch.randn(batch, blk, G, 128, generator=gen, device=device).half()
        Cm = torch.randn(batch, blk, G, 128, generator=gen, device=device).half()
        one_token = k % 2 == 0
        print(f"[ridge drift] layout={layout} B={batch} block={k} tokens={k * blk}..{(k + 1) * blk - 1} "
              f"one_token_calls={one_token}", flush=True)
        if one_token:
            ys = []
            for t in range(blk):
                yt, _ = ridge_codec.scan(x[:, t:t + 1].contiguous(), dt[:, t:t + 1].contiguous(), A,
                                         Bm[:, t:t + 1].contiguous(), Cm[:, t:t + 1].contiguous(), D, db, state,
                                         perm, basis, ls, pred, layout=layout, validate=(k == 0 and t == 0))
                ys.append(yt)
            y = torch.cat(ys, dim=1)
        else:
            y, _ = ridge_codec.scan(x, dt, A, Bm, Cm, D, db, state, perm, basis, ls, pred, layout=layout,
                                    validate=False)
        torch.cuda.synchronize()
        host = lambda v: np.ascontiguousarray(v[sub].cpu().numpy().view(np.uint16))
        y_ref = oracle.state_step(oracle.MODE_RIDGE, n8, n4, nz, host(x), host(dt), par["A"], host(Bm), host(Cm),
                                  par["D"], par["dt_bias"], par["perm"], sta["basis"], sta["lscale"], sta["pred"],
                                  ref_state)
        got = {kk: rows_of(v) for kk, v in from_state(state).items()}
        assert_state_equal(got, ref_state, f"ridge drift block {k}")
        assert_y_close(y[sub], y_ref, f"ridge drift block {k}")


def test_legacy_diagnostic_encode_matches_reference_vectors(device):
    """m2r_state_encode_legacy through state_codec.encode_state_ against the
    reference's own encode_state_ outputs (tests/golden/encode_legacy_vectors.npz),
    bit-exact; and an FP16-overflowing row is rejected before the state is written."""
    from pathlib import Path
    from mamba2_recall import state_codec
    g = np.load(Path(__file__).resolve().parent / "golden" / "encode_legacy_vectors.npz")
    print("[legacy encode] golden vectors", g["dense"].shape, flush=True)
    state = state_codec.allocate_state(2, 2, 64, 128, "sq3p25", device)
    state_codec.encode_state_(state, torch.from_numpy(g["dense"]).to(device))
    torch.cuda.synchronize()
    got = from_state(state)
    for k in ("lo", "hi", "q4", "s8", "s4"):
        assert np.array_equal(got[k], g[k]), k
    before = {k: v.clone() for k, v in state.tensors.items()}
    big = torch.from_numpy(g["dense"]).to(device).clone()
    big[0, 0, 0, 0] = 1e8
    with pytest.raises(ValueError, match="Scale exceeds FP16 range"):
        state_codec.encode_state_(state, big)
    assert all(torch.equal(before[k], state.tensors[k]) for k in before)


def test_decode_state_matches_reference_vectors(device):
    """The diagnostic decoders against the reference's own decode_state
    outputs (tests/golden/decode_state_vectors.npz, written by
    tests/golden/make_decode_state_vectors.py), bit for bit as FP32 patterns:
    sq3p25 in packed order and scattered through a permutation; dense 3-bit
    with no table, a permutation table and an equalizer table.  The packed
    bytes are arbitrary and the scales include zero, negative zero, a binary16
    subnormal and a negative value."""
    from pathlib import Path
    from mamba2_recall import state_codec, state_codec_dense3
    g = np.load(Path(__file__).resolve().parent / "golden" / "decode_state_vectors.npz")
    bits = lambda t: t.cpu().numpy().view(np.uint32)
    print("[decode_state] sq3p25 and dense3 golden vectors", flush=True)
    st = state_codec.allocate_state(1, 4, 16, 128, "sq3p25", device)
    for k in ("lo", "hi", "q4"):
        st.tensors[k].copy_(torch.from_numpy(g[f"sq_{k}"]).to(device))
    for k in ("s8", "s4"):
        st.tensors[k].copy_(torch.from_numpy(g[f"sq_{k}"].view(np.float16)).to(device))
    perm = torch.from_numpy(g["perm"]).to(device)
    assert np.array_equal(bits(state_codec.decode_state(st)), g["sq_decode"].view(np.uint32))
    assert np.array_equal(bits(state_codec.decode_state(st, perm)), g["sq_decode_perm"].view(np.uint32))
    ds = state_codec_dense3.allocate_state(1, 4, 16, 128, device)
    ds.tensors["codes"].copy_(torch.from_numpy(g["d3_codes"]).to(device))
    ds.tensors["scales"].copy_(torch.from_numpy(g["d3_scales"].view(np.float16)).to(device))
    eq = torch.from_numpy(g["d3_equalizer"]).to(device)
    assert np.array_equal(bits(state_codec_dense3.decode_state(ds)), g["d3_decode"].view(np.uint32))
    assert np.array_equal(bits(state_codec_dense3.decode_state(ds, perm, "permutation")),
                          g["d3_decode_perm"].view(np.uint32))
    assert np.array_equal(bits(state_codec_dense3.decode_state(ds, eq, "equalizer")),
                          g["d3_decode_eq"].view(np.uint32))


@pytest.mark.parametrize("length", [1, 17, 65])
def test_ridge_reference_fixture_recipe_strided_and_compact(oracle, device, length):
    """The forward half of the reference's own codec fixture
    (scripts/check_state_ridge_training_v3.py:19-49): its seed and input
    recipe (b,h,p,g = 1,8,16,2; one projection split into x*.05, B*.1, C*.1,
    dt*.03; A = -1, D = 1, dt_bias = -3; basis N*.03, latent scale .001,
    predictor N*.01; zero state), for the seven layouts, with projection-strided
    views and compact copies.  The strided and compact scans agree exactly
    (torch.equal, as the fixture requires of its two paths), and both equal
    the oracle: packed state bit-exact, y within the tolerance."""
    from mamba2_recall import ridge_codec
    torch.manual_seed(2026093007)
    b, h, p, g = 1, 8, 16, 2
    for layout in RIDGE_LAYOUTS:
        n8, n4, nz = ridge_counts(layout)
        features = n8 + n4 + 2
        projected = torch.randn(b, length, h * p + 2 * g * 128 + h, device=device).half()
        xv, bv, cv, dv = torch.split(projected, (h * p, g * 128, g * 128, h), dim=-1)
        xv.mul_(.05); bv.mul_(.1); cv.mul_(.1); dv.mul_(.03)
        x, B, C, dt = xv.reshape(b, length, h, p), bv.reshape(b, length, g, 128), cv.reshape(b, length, g, 128), dv
        if length > 1:
            assert not all(t.is_contiguous() for t in (x, dt, B, C))
        A = -torch.ones(h, device=device)
        D = torch.ones(h, device=device).half()
        bias = torch.full((h,), -3., device=device).half()
        table = torch.stack([torch.randperm(128, device=device) for _ in range(g)]).to(torch.uint8)
        basis = (torch.randn(g, nz, 2, device=device) * .03).half()
        scale = torch.full((g, 2), .001, device=device).half()
        predictor = (torch.randn(g, features, nz, device=device) * .01).half()
        print(f"[ridge fixture recipe] layout={layout} L={length}", flush=True)
        s_strided = ridge_codec.allocate_state(b, h, p, 128, device, layout=layout)
        s_compact = ridge_codec.allocate_state(b, h, p, 128, device, layout=layout)
        y_s, _ = ridge_codec.scan(x, dt, A, B, C, D, bias, s_strided, table, basis, scale, predictor, layout=layout)
        xc, dtc, Bc, Cc = (t.contiguous() for t in (x, dt, B, C))
        y_c, _ = ridge_codec.scan(xc, dtc, A, Bc, Cc, D, bias, s_compact, table, basis, scale, predictor,
                                  layout=layout)
        torch.cuda.synchronize()
        assert torch.equal(y_s, y_c)
        assert all(torch.equal(s_strided.tensors[k], s_compact.tensors[k]) for k in s_compact.tensors)
        host = lambda t: np.ascontiguousarray(t.cpu().numpy().view(np.uint16))
        ref_state = cases.zero_packed_state(b, h, p, n8, n4, latent=True)
        y_ref = oracle.state_step(oracle.MODE_RIDGE, n8, n4, nz, host(xc), host(dtc), A.cpu().numpy(), host(Bc),
                                  host(Cc), host(D), host(bias), table.cpu().numpy(), host(basis), host(scale),
                                  host(predictor), ref_state)
        assert_state_equal(from_state(s_compact), ref_state, f"ridge fixture recipe {layout}")
        assert_y_close(y_c, y_ref, f"ridge fixture recipe {layout}")
