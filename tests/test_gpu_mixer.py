"""GPU parity of the one-token convolution update (m2r_causal_conv_update)
against the reference's PyTorch fallback of the same update
(mamba2_recall/state_quant.py:289-297, restated verbatim below), bit for bit
on the rolled window and the FP16 output, and the controller's cached decay
rates.  Every case prints its identity before the device call."""
import numpy as np
import pytest
import torch
from torch import nn

pytestmark = pytest.mark.gpu


def reference_update(window, value, weight, bias, act):
    """state_quant.py:291-297, the update branch with no native kernel."""
    window.copy_(torch.roll(window, shifts=-1, dims=-1))
    window[:, :, -1] = value
    out = torch.sum(window * weight, dim=-1)
    if bias is not None:
        out = out + bias
    return act(out).to(dtype=value.dtype)


def make_window(batch, channels, layout, device, gen, scale):
    if layout == "time_major":   # how the controller keeps it: a transposed [B, 4, C] buffer
        w = torch.empty(batch, 4, channels, device=device, dtype=torch.float16).transpose(1, 2)
    else:
        w = torch.empty(batch, channels, 4, device=device, dtype=torch.float16)
    w.copy_((torch.randn(batch, channels, 4, generator=gen, device=device) * scale).half())
    return w


@pytest.mark.parametrize("batch,layout,with_bias,scale", [
    (1, "time_major", True, 1.0), (16, "time_major", True, 1.0), (3, "contiguous", False, 1.0),
    (16, "time_major", True, 30.0), (2, "time_major", True, 1e-4)])
def test_conv_update_matches_reference_fallback(device, batch, layout, with_bias, scale):
    from mamba2_recall.state_quant import conv_update
    channels = 10240
    gen = torch.Generator(device=device).manual_seed(100 + batch)
    print(f"[conv update] B={batch} C={channels} layout={layout} bias={with_bias} scale={scale}", flush=True)
    win = make_window(batch, channels, layout, device, gen, scale)
    projected = (torch.randn(batch, 1, 18560, generator=gen, device=device) * scale).half()
    value = projected[:, 0, 8192:8192 + channels]          # a strided view, as the split gives
    weight = (torch.randn(channels, 1, 4, generator=gen, device=device) * 0.5).half()[:, 0, :]
    bias = (torch.randn(channels, generator=gen, device=device) * 0.1).half() if with_bias else None
    ref_win = win.clone()
    want = reference_update(ref_win, value, weight, bias, nn.SiLU())
    for step in range(4):   # consecutive tokens roll the window again
        got = conv_update(win, value, weight, bias, silu=True)
        torch.cuda.synchronize()
        assert torch.equal(win, ref_win), f"window after update {step + 1}"
        mism = int((got.view(torch.int16) != want.view(torch.int16)).sum())
        assert mism == 0, f"update {step + 1}: {mism} output values differ from the reference fallback"
        value = (torch.randn(batch, channels, generator=gen, device=device) * scale).half()
        want = reference_update(ref_win, value, weight, bias, nn.SiLU())


def test_conv_update_rejects_bad_shapes(device):
    from mamba2_recall.state_quant import conv_update
    win = torch.zeros(1, 8, 3, device=device, dtype=torch.float16)
    with pytest.raises(ValueError, match="Convolution update"):
        conv_update(win, torch.zeros(1, 8, device=device, dtype=torch.float16),
                    torch.zeros(8, 3, device=device, dtype=torch.float16), None)
