"""Host-side checks of the drop-in surface, on CPU tensors (no device work).

The layout mapping is pinned by the layout triples of the reference's codec
fixtures (`docs/evidence/fp_state_diagnostics/v12,v14/codec_fixture.json`:
parent 'A_B_C' -> (A, B-4, C+4)); the allocation checks by the 52-byte row
(`README.md:123`: 425,984 B per layer at batch 1).  Error classes and
messages follow the reference's validators (cited per test).
"""
import pytest
import torch

from mamba2_recall import ridge_codec, state_codec, state_codec_dense3, tier_codec

PUBLISHED = {  # layout: (n8, n4, nz, F)
    "36_24_68": (36, 20, 72, 58), "16_64_48": (16, 60, 52, 78), "32_32_64": (32, 28, 68, 62),
    "40_16_72": (40, 12, 76, 54), "24_48_56": (24, 44, 60, 70), "8_80_40": (8, 76, 44, 86),
    "44_8_76": (44, 4, 80, 50),
}


@pytest.mark.parametrize("layout", sorted(PUBLISHED))
def test_ridge_layout_mapping(layout):
    d = ridge_codec.layout_descriptor(layout)
    n8, n4, nz, features = PUBLISHED[layout]
    assert (d["n8"], d["n4"], d["nzero"]) == (n8, n4, nz)
    assert d["n8"] + d["n4"] + 2 == features
    assert d["row_bytes"] == 52 and sum(d["tensor_widths"].values()) + 4 == 52


def test_tier_layout_rejects_unknown():
    # w4_state_repair_codec_v2.py:34-37
    with pytest.raises(ValueError, match="Unknown fixed W4 state repair tier layout"):
        tier_codec.layout_descriptor("36_24_69")
    with pytest.raises(ValueError):
        ridge_codec.layout_descriptor("not_a_layout")


@pytest.mark.parametrize("layout", ["36_24_68", "8_80_40"])
def test_ridge_state_allocation_and_validation(layout):
    # fp4_zero_predictor_codec_v1.py:39-73
    st = ridge_codec.allocate_state(1, 128, 64, 128, "cpu", layout=layout)
    assert st.nbytes == 425_984
    assert ridge_codec.validate_state(st, "cpu", layout)
    with pytest.raises(ValueError, match="mode/inventory"):
        ridge_codec.validate_state(st, "cpu", "44_8_76" if layout != "44_8_76" else "36_24_68")
    lo = st.tensors["lo"]
    st.tensors["lo"] = torch.zeros(lo.shape[:-1] + (lo.shape[-1] * 2,), dtype=torch.uint8)[..., ::2]
    with pytest.raises(ValueError, match="backing allocation differs: lo"):
        ridge_codec.validate_state(st, "cpu", layout)
    st.tensors["lo"] = st.tensors["hi"]    # same shape and dtype, shared storage
    with pytest.raises(ValueError, match="aliases"):
        ridge_codec.validate_state(st, "cpu", layout)


@pytest.mark.parametrize("args", [(1, 128, 64, 64), (0, 128, 64, 128), (1.0, 128, 64, 128)])
def test_ridge_allocation_rejects_geometry(args):
    with pytest.raises(ValueError, match="dstate=128"):
        ridge_codec.allocate_state(*args, "cpu", layout="32_32_64")


def test_legacy_state_is_52_bytes_per_row():
    # state_codec.py:51-62
    st = state_codec.allocate_state(2, 128, 64, 128, "sq3p25", "cpu")
    assert sum(t.numel() * t.element_size() for t in st.tensors.values()) == 2 * 8192 * 52


def test_permutation_validation():
    # state_codec.py:179-184
    perm = torch.stack([torch.randperm(128) for _ in range(8)]).to(torch.uint8)
    state_codec.validate_permutation(perm, 8)
    bad = perm.clone()
    bad[5, 0] = bad[5, 1]
    with pytest.raises(ValueError, match="exactly once"):
        state_codec.validate_permutation(bad, 8)
    with pytest.raises(ValueError, match="uint8"):
        state_codec.validate_permutation(perm.long(), 8)
    with pytest.raises(ValueError, match="uint8"):
        state_codec.validate_permutation(perm[:7], 8)


def test_dense3_table_validation():
    # state_codec_dense3.py:53-64
    perm = torch.stack([torch.randperm(128) for _ in range(8)]).to(torch.uint8)
    state_codec_dense3.validate_table(perm, 8, "permutation")
    eq = torch.randint(-8, 9, (8, 128), dtype=torch.int8)
    state_codec_dense3.validate_table(eq, 8, "equalizer")
    with pytest.raises(ValueError, match="kind"):
        state_codec_dense3.validate_table(perm, 8, "both")
    with pytest.raises(ValueError, match="dtype or shape"):
        state_codec_dense3.validate_table(eq, 8, "permutation")
    dup = perm.clone()
    dup[2, 7] = dup[2, 9]
    with pytest.raises(ValueError, match="exactly"):
        state_codec_dense3.validate_table(dup, 8, "permutation")
    for v in (-9, 9):
        hot = eq.clone()
        hot[4, 100] = v
        with pytest.raises(ValueError, match=r"\[-8,8\]"):
            state_codec_dense3.validate_table(hot, 8, "equalizer")


def test_dense3_allocation():
    # state_codec_dense3.py:43-50
    st = state_codec_dense3.allocate_state(1, 128, 64, 128, "cpu")
    assert sum(t.numel() * t.element_size() for t in st.tensors.values()) == 425_984
    with pytest.raises(ValueError, match="dstate128"):
        state_codec_dense3.allocate_state(1, 128, 64, 127, "cpu")


def scan_inputs(batch=1, L=1):
    x = torch.zeros(batch, L, 128, 64, dtype=torch.float16)
    dt = torch.zeros(batch, L, 128, dtype=torch.float16)
    A = -torch.ones(128)
    B = torch.zeros(batch, L, 8, 128, dtype=torch.float16)
    return x, dt, A, B, B.clone(), torch.zeros(128, dtype=torch.float16), torch.zeros(128, dtype=torch.float16)


def test_scans_reject_host_tensors():
    # state_codec.py:203-210, state_codec_dense3.py:151-160, fp4_zero_predictor_codec_v1.py:185-195:
    # every scan requires device FP16 x before anything else
    x, dt, A, B, C, D, db = scan_inputs()
    st = state_codec.allocate_state(1, 128, 64, 128, "sq3p25", "cpu")
    perm = torch.stack([torch.randperm(128) for _ in range(8)]).to(torch.uint8)
    with pytest.raises(ValueError, match="x must be CUDA FP16"):
        state_codec.scan(x, dt, A, B, C, D, db, st, permutation=perm)
    d3 = state_codec_dense3.allocate_state(1, 128, 64, 128, "cpu")
    with pytest.raises(ValueError, match="x must be CUDA FP16"):
        state_codec_dense3.scan(x, dt, A, B, C, D, db, d3, perm)
    rs = ridge_codec.allocate_state(1, 128, 64, 128, "cpu", layout="32_32_64")
    with pytest.raises(ValueError, match="x must be CUDA FP16"):
        ridge_codec.scan(x, dt, A, B, C, D, db, rs, perm, None, None, None, layout="32_32_64")


def _ridge_statics(layout, groups=8):
    d = ridge_codec.layout_descriptor(layout)
    features = d["n8"] + d["n4"] + 2
    perm = torch.stack([torch.randperm(128) for _ in range(groups)]).to(torch.uint8)
    basis = torch.zeros(groups, d["nzero"], 2, dtype=torch.float16)
    ls = torch.full((groups, 2), 1e-3, dtype=torch.float16)
    pred = torch.zeros(groups, features, d["nzero"], dtype=torch.float16)
    return perm, basis, ls, pred


@pytest.mark.parametrize("bad", ["pred_shape", "pred_dtype", "pred_strided", "perm_shape", "basis_shape",
                                 "lscale_dtype"])
def test_ridge_static_metadata_checks_never_skipped(bad):
    # fp4_zero_predictor_codec_v1.py:203-217: the kernel indexes the tables by
    # these shapes, so scan(validate=False) still runs this host-only part
    layout = "32_32_64"
    perm, basis, ls, pred = _ridge_statics(layout)
    ridge_codec.check_static_metadata(perm, basis, ls, pred, groups=8, layout=layout, device=torch.device("cpu"))
    if bad == "pred_shape":
        pred = pred[:, :-1].contiguous()
    elif bad == "pred_dtype":
        pred = pred.float()
    elif bad == "pred_strided":
        pred = torch.zeros(pred.shape[:-1] + (2 * pred.shape[-1],), dtype=torch.float16)[..., ::2]
    elif bad == "perm_shape":
        perm = perm[:7]
    elif bad == "basis_shape":
        basis = basis[:, :-1]
    else:
        ls = ls.float()
    msg = "predictor differs" if bad.startswith("pred") else "basis/scales differ"
    with pytest.raises(ValueError, match=msg):
        ridge_codec.check_static_metadata(perm, basis, ls, pred, groups=8, layout=layout,
                                          device=torch.device("cpu"))


def test_ridge_value_checks_reject_nonfinite_and_nonpositive():
    layout = "44_8_76"
    perm, basis, ls, pred = _ridge_statics(layout)
    dev = torch.device("cpu")
    ridge_codec.validate_statics(perm, basis, ls, pred, groups=8, layout=layout, device=dev)
    for which in ("basis", "ls_zero", "ls_inf", "pred"):
        b, l, p = basis.clone(), ls.clone(), pred.clone()
        if which == "basis":
            b[3, 5, 1] = float("nan")
        elif which == "ls_zero":
            l[2, 0] = 0
        elif which == "ls_inf":
            l[2, 1] = float("inf")
        else:
            p[1, 2, 3] = float("-inf")
        with pytest.raises(ValueError):
            ridge_codec.validate_statics(perm, b, l, p, groups=8, layout=layout, device=dev)


def test_layers_step_rejects_bad_calls_before_any_launch():
    """The multi-layer step validates on the host: no layers, an unsupported
    layout, misaligned state arrays and a short workspace are rejected with
    a message, before anything is enqueued (fake, never dereferenced device
    addresses)."""
    import ctypes
    from mamba2_recall import _native
    lib = _native.lib()
    layer = _native.RidgeLayer()
    for i, (name, _) in enumerate(_native.RidgeLayer._fields_[:18]):
        setattr(layer, name, 0x10000 * (i + 1))
    layer.n8, layer.n4, layer.nz = 32, 28, 68
    arr = (_native.RidgeLayer * 1)(layer)

    def err(*args):
        rc = lib.m2r_state_step_ridge_layers(*args)
        assert rc != 0
        return lib.m2r_last_error().decode()

    assert "no layers" in err(ctypes.byref(arr), 0, 1, 128, 64, 8, 0x900000, 1 << 20, None)
    assert "workspace" in err(ctypes.byref(arr), 1, 1, 128, 64, 8, 0x900000, 8, None)
    arr[0].n8 = 30
    assert "layout" in err(ctypes.byref(arr), 1, 1, 128, 64, 8, 0x900000, 1 << 20, None)
    arr[0].n8, arr[0].lo = 32, 0x10008
    assert "16-byte" in err(ctypes.byref(arr), 1, 1, 128, 64, 8, 0x900000, 1 << 20, None)
    arr[0].lo = 0x10000
    assert "multiple of 8" in err(ctypes.byref(arr), 1, 1, 128, 60, 8, 0x900000, 1 << 20, None)
    assert lib.m2r_state_step_ridge_layers_workspace(56) == 56 * lib.m2r_state_step_ridge_layers_workspace(1)


def test_ridge_workspace_step_rejects_bad_workspaces_before_any_launch():
    """The workspace variant of the ridge step checks its workspace on the
    host (fake, never dereferenced device addresses): a size without a
    workspace, a misaligned one and one smaller than the records need are
    rejected with a message; the size query is batch * L * G KiB."""
    from mamba2_recall import _native
    lib = _native.lib()
    assert lib.m2r_ridge_records_bytes(1, 2048, 8) == 2048 * 8 * 1024
    assert lib.m2r_ridge_records_bytes(0, 5, 8) == 0
    fake = [0x10000 * (i + 1) for i in range(20)]

    def err(ws, nbytes):
        args = fake[:6] + [0, fake[6], 0] + fake[7:11] + fake[11:18] + [1, 37, 128, 64, 8, 32, 28, 68, ws, nbytes,
                                                                          None]
        rc = lib.m2r_state_step_ridge_ws(*args)
        assert rc != 0
        return lib.m2r_last_error().decode()

    assert "without a workspace" in err(None, 4096)
    assert "16-byte" in err(0x900008, 1 << 30)
    assert "smaller" in err(0x900000, 37 * 8 * 1024 - 1)


def test_layer_table_rejects_mixed_group_counts():
    """The multi-layer launch takes one group count for all layers and the
    kernel indexes every layer's B, C and statics with it: a table whose
    layers disagree is rejected on the host, before any device check."""
    def step(groups):
        return {"x": torch.zeros(1, 1, 128, 64, dtype=torch.float16),
                "B": torch.zeros(1, 1, groups, 128, dtype=torch.float16)}
    with pytest.raises(ValueError, match="same number of B/C groups"):
        ridge_codec.layer_table([step(8), step(8), step(4)])
    with pytest.raises(ValueError, match="same number of B/C groups"):
        ridge_codec.layer_table([step(8), {"x": step(8)["x"], "B": torch.zeros(8, 128)}])


def test_norm_hook_takes_only_non_overlapping_rows():
    """The gated-norm hook calls the kernel only for operands it reads as
    separate rows; a broadcast gate (row stride 0) or overlapping rows go to
    the module's own forward instead of failing in the kernel's checks."""
    from mamba2_recall import state_quant
    base = torch.zeros(4, 96, dtype=torch.float16)
    assert state_quant._kernel_rows(base)
    assert state_quant._kernel_rows(torch.zeros(4, 128, dtype=torch.float16)[:, :96])   # projection split
    assert state_quant._kernel_rows(torch.zeros(1, 1, 96, dtype=torch.float16))
    assert not state_quant._kernel_rows(torch.zeros(1, 96, dtype=torch.float16).expand(4, 96))
    overlap = torch.zeros(400, dtype=torch.float16).as_strided((4, 96), (8, 1))
    assert not state_quant._kernel_rows(overlap)
    assert not state_quant._kernel_rows(torch.zeros(4, 97, dtype=torch.float16)[:, :96])   # stride not % 4
