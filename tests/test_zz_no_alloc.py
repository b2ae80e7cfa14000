"""The no-allocation multi-layer step (m2r_state_step_ridge_layers_noalloc,
layer table in the library's static device array) against the workspace
entry point m2r_state_step_ridge_layers, both called through the C ABI:
two calls in a row, the second over a smaller input (fewer layers at a
smaller batch); packed states and readouts must be bit-identical."""
import ctypes

import numpy as np
import pytest
import torch

from cases import RIDGE_LAYOUTS
from test_gpu_layers import make_layers

pytestmark = pytest.mark.gpu

H, P, G = 128, 64, 8


def clone_steps(steps):
    from mamba2_recall import ridge_codec
    out = []
    for st in steps:
        c = dict(st)
        state = ridge_codec.allocate_state(st["x"].shape[0], H, P, 128, st["x"].device, layout=st["layout"])
        for k, t in st["state"].tensors.items():
            state.tensors[k].copy_(t)
        c["state"], c["y"] = state, torch.empty_like(st["y"])
        out.append(c)
    return out


def call_both(steps):
    from mamba2_recall import _native, ridge_codec
    ref = clone_steps(steps)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    x = steps[0]["x"]
    batch = x.shape[0]
    t_ref = ridge_codec.layer_table(ref)
    ws = torch.empty(ridge_codec.layers_workspace_bytes(len(ref)), dtype=torch.uint8, device=x.device)
    _native.call("m2r_state_step_ridge_layers", ctypes.byref(t_ref), len(ref), batch, H, P, G, _native.ptr(ws),
                 ws.numel(), stream)
    t_new = ridge_codec.layer_table(steps)
    _native.call("m2r_state_step_ridge_layers_noalloc", ctypes.byref(t_new), len(steps), batch, H, P, G, stream)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(steps, ref)):
        for k, t in a["state"].tensors.items():
            assert torch.equal(t.view(torch.uint8), b["state"].tensors[k].view(torch.uint8)), (i, k)
        assert torch.equal(a["y"].view(torch.int16), b["y"].view(torch.int16)), i


def test_noalloc_layers_step_matches_workspace_entry_point(device):
    rng = np.random.default_rng(7)
    print("[no-alloc] call 1: batch 2, 56 layers", flush=True)
    big, _ = make_layers(rng, 2, (RIDGE_LAYOUTS * 8)[:56], device)
    call_both(big)
    print("[no-alloc] call 2: batch 1, 9 layers", flush=True)
    small, _ = make_layers(rng, 1, (RIDGE_LAYOUTS * 2)[:9], device)
    call_both(small)


def test_noalloc_layers_step_rejects_oversized_table():
    """More layers than the static array holds: a clear error, nothing
    enqueued."""
    from mamba2_recall import _native
    lib = _native.lib()
    arr = (_native.RidgeLayer * 257)()
    rc = lib.m2r_state_step_ridge_layers_noalloc(ctypes.byref(arr), 257, 1, 128, 64, 8, None)
    assert rc != 0 and b"M2R_LAYERS_NOALLOC_MAX" in lib.m2r_last_error()


def test_layers_entry_points_reject_graph_capture(device):
    """Both multi-layer entry points copy their layer table from host memory
    that the next call overwrites, so a captured copy would replay with
    another call's table: on a capturing stream they return an error before
    anything is enqueued, and eager calls still match afterwards."""
    from mamba2_recall import _native, ridge_codec
    rng = np.random.default_rng(11)
    steps, _ = make_layers(rng, 1, RIDGE_LAYOUTS[:2], device)
    table = ridge_codec.layer_table(steps)
    ws = torch.empty(ridge_codec.layers_workspace_bytes(len(steps)), dtype=torch.uint8, device=device)
    lib = _native.lib()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    print("[no-alloc] capture: both entry points on a capturing stream", flush=True)
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            st = ctypes.c_void_p(side.cuda_stream)
            rc_noalloc = lib.m2r_state_step_ridge_layers_noalloc(ctypes.byref(table), len(steps), 1, H, P, G, st)
            err_noalloc = lib.m2r_last_error()
            rc_ws = lib.m2r_state_step_ridge_layers(ctypes.byref(table), len(steps), 1, H, P, G,
                                                    ctypes.c_void_p(ws.data_ptr()), ws.numel(), st)
            err_ws = lib.m2r_last_error()
        finally:
            graph.capture_end()
    assert rc_noalloc != 0 and b"capturing" in err_noalloc, err_noalloc
    assert rc_ws != 0 and b"capturing" in err_ws, err_ws
    torch.cuda.synchronize()
    print("[no-alloc] eager calls after the rejected capture", flush=True)
    call_both(steps)
