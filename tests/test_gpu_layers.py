"""GPU parity of the one-launch multi-layer ridge step (m2r_state_step_ridge_layers):
every layer's packed state and readout must equal, bit for bit, what one
per-layer launch of m2r_state_step_ridge (itself oracle-checked) gives on the
same inputs, over the published layouts and the three workgroup shapes the
batch size selects.  One layer per case is also compared with the C oracle."""
import numpy as np
import pytest
import torch

import cases
from cases import RIDGE_LAYOUTS, ridge_counts

pytestmark = pytest.mark.gpu

H, P, G = 128, 64, 8


def dev16(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)


def make_layers(rng, batch, layouts, device):
    from mamba2_recall import ridge_codec
    steps, np_layers = [], []
    for layout in layouts:
        n8, n4, nz = ridge_counts(layout)
        inp = cases.step_inputs(rng, batch, 1, H, P, G)
        sta = cases.ridge_statics(rng, G, n8, n4, nz)
        st0 = cases.random_packed_state(rng, batch, H, P, n8, n4, latent=True)
        state = ridge_codec.allocate_state(batch, H, P, 128, device, layout=layout)
        for k, v in st0.items():
            t = state.tensors[k].view(torch.uint8)
            t.copy_(torch.from_numpy(np.ascontiguousarray(v)).view(torch.uint8).reshape(t.shape).to(device))
        x = dev16(inp["x"], device)
        steps.append(dict(x=x, dt=dev16(inp["dt"], device), A=torch.from_numpy(inp["A"]).to(device),
                          B=dev16(inp["B"], device), C=dev16(inp["C"], device), D=dev16(inp["D"], device),
                          dt_bias=dev16(inp["dt_bias"], device), state=state,
                          permutation=torch.from_numpy(inp["perm"]).to(device), basis=dev16(sta["basis"], device),
                          latent_scale=dev16(sta["lscale"], device), predictor=dev16(sta["pred"], device),
                          layout=layout, y=torch.empty_like(x)))
        np_layers.append((inp, sta, st0))
    return steps, np_layers


def per_layer_reference(steps):
    """The same steps through one m2r_state_step_ridge launch per layer, on
    copies of the states: (states, readouts)."""
    from mamba2_recall import ridge_codec
    states, ys = [], []
    for st in steps:
        copy = ridge_codec.allocate_state(st["x"].shape[0], H, P, 128, st["x"].device, layout=st["layout"])
        for k, t in st["state"].tensors.items():
            copy.tensors[k].copy_(t)
        y, _ = ridge_codec.scan(st["x"], st["dt"], st["A"], st["B"], st["C"], st["D"], st["dt_bias"], copy,
                                st["permutation"], st["basis"], st["latent_scale"], st["predictor"],
                                layout=st["layout"], validate=False)
        states.append(copy)
        ys.append(y)
    return states, ys


@pytest.mark.parametrize("batch,nlayers", [(1, 9), (2, 7), (48, 7), (64, 7)])
def test_layers_step_equals_per_layer_launches(oracle, device, batch, nlayers):
    """batch 1 and 2: (4 waves, 1 slot) workgroups; 48: (4, 2); 64: (4, 4)."""
    from mamba2_recall import ridge_codec
    rng = np.random.default_rng(batch * 100 + nlayers)
    layouts = [RIDGE_LAYOUTS[i % len(RIDGE_LAYOUTS)] for i in range(nlayers)]
    print(f"[layers] batch={batch} nlayers={nlayers}", flush=True)
    steps, np_layers = make_layers(rng, batch, layouts, device)
    ref_states, ref_ys = per_layer_reference(steps)
    ridge_codec.scan_layers(steps)
    torch.cuda.synchronize()
    for i, st in enumerate(steps):
        for k, t in st["state"].tensors.items():
            assert torch.equal(t.view(torch.uint8), ref_states[i].tensors[k].view(torch.uint8)), (i, k)
        assert torch.equal(st["y"].view(torch.int16), ref_ys[i].view(torch.int16)), i
    # layer 0 against the oracle as well
    inp, sta, st0 = np_layers[0]
    n8, n4, nz = ridge_counts(layouts[0])
    ref = cases.copy_state(st0)
    y_ref = oracle.state_step(oracle.MODE_RIDGE, n8, n4, nz, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"],
                              inp["D"], inp["dt_bias"], inp["perm"], sta["basis"], sta["lscale"], sta["pred"], ref)
    for k in st0:
        got = steps[0]["state"].tensors[k].view(torch.uint8).cpu().numpy().reshape(-1)
        want = np.ascontiguousarray(ref[k]).view(np.uint8).reshape(-1)
        assert (got == want).all(), k
    err = cases.rel_l2(cases.f16_to_f32(steps[0]["y"].cpu().numpy().view(np.uint16)), cases.f16_to_f32(y_ref))
    assert err <= 1e-3


def test_layers_step_repeated_calls_and_reused_workspace(device):
    """Three consecutive one-token launches through one workspace, the second
    over fewer layers, equal the per-layer launches after each call."""
    from mamba2_recall import ridge_codec
    rng = np.random.default_rng(5)
    steps, _ = make_layers(rng, 1, RIDGE_LAYOUTS * 2, device)
    ws = torch.empty(ridge_codec.layers_workspace_bytes(len(steps)), dtype=torch.uint8, device=device)
    for n in (len(steps), 5, len(steps)):
        print(f"[layers repeat] nlayers={n}", flush=True)
        sub = steps[:n]
        ref_states, ref_ys = per_layer_reference(sub)
        ridge_codec.scan_layers(sub, workspace=ws)
        torch.cuda.synchronize()
        for i, st in enumerate(sub):
            for k, t in st["state"].tensors.items():
                assert torch.equal(t.view(torch.uint8), ref_states[i].tensors[k].view(torch.uint8)), (n, i, k)
            assert torch.equal(st["y"].view(torch.int16), ref_ys[i].view(torch.int16)), (n, i)
