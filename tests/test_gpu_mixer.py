"""GPU parity of the one-token convolution update (m2r_causal_conv_update)
against the reference's PyTorch fallback of the same update
(mamba2_recall/state_quant.py:289-297, restated verbatim below), bit for bit
on the rolled window and the FP16 output, and of the gated RMS norm
(m2r_gated_rmsnorm) against its formula in float64, to one binary16
rounding.  Every case prints its identity before the device call."""
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


def gated_norm_reference(y, z, weight, eps, group_size):
    """The gated RMS norm's formula (mamba_ssm RMSNormGated, norm_before_gate
    False, as the reference's controllers call it: state_quant.py:298-300)
    in float64: v = y * z * sigmoid(z); v / sqrt(mean_group(v^2) + eps) * w."""
    v = y.double() * z.double() * torch.sigmoid(z.double())
    shape = v.shape
    g = v.reshape(*shape[:-1], shape[-1] // group_size, group_size)
    g = g / torch.sqrt(g.pow(2).mean(-1, keepdim=True) + eps)
    return g.reshape(shape) * weight.double()


def f16_ulps(a, b):
    """Distance in binary16 units in the last place between FP16 tensors of
    finite values (sign-magnitude bit patterns mapped to a monotone scale)."""
    def key(t):
        i = t.view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (key(a) - key(b)).abs()


@pytest.mark.parametrize("rows,group_size,eps,scale,strided", [
    (1, 1024, 1e-5, 1.0, True), (3, 1024, 1e-5, 1.0, True), (17, 1024, 1e-6, 4.0, False),
    (2, 512, 1e-5, 1.0, True), (5, 4096, 1e-5, 0.01, False), (4, 256, 1e-5, 30.0, True)])
def test_gated_rmsnorm_matches_formula(device, rows, group_size, eps, scale, strided):
    """The native gated norm against the formula in float64: every output
    within one binary16 rounding of the float64 value's binary16 rounding
    (binary32 arithmetic, a different summation order), most of them equal;
    z read through the in_proj split's row stride when strided."""
    from mamba2_recall.state_quant import gated_rmsnorm
    channels = 8192
    gen = torch.Generator(device=device).manual_seed(rows * 7 + group_size)
    print(f"[gated norm] rows={rows} group={group_size} eps={eps} scale={scale} strided={strided}", flush=True)
    y = (torch.randn(rows, channels, generator=gen, device=device) * scale).half()
    zfull = (torch.randn(rows, 18560, generator=gen, device=device) * 2).half()
    z = zfull[:, :channels] if strided else zfull[:, :channels].contiguous()
    weight = (1 + 0.1 * torch.randn(channels, generator=gen, device=device)).half()
    out = gated_rmsnorm(y, z, weight, eps, group_size)
    torch.cuda.synchronize()
    want = gated_norm_reference(y, z, weight, eps, group_size).half()
    assert out.shape == y.shape and out.dtype == torch.float16 and bool(torch.isfinite(out).all())
    d = f16_ulps(out, want)
    assert int(d.max()) <= 1, int(d.max())
    assert float((d == 0).float().mean()) > 0.95
    # deterministic: a second call gives the same bits
    assert torch.equal(out, gated_rmsnorm(y, z, weight, eps, group_size))


def test_gated_rmsnorm_three_dim_rows_and_rejections(device):
    """[B, L, C] operands (rows of one stride, z a view of the projection
    output) give the rows' results; unsupported operands raise."""
    from mamba2_recall.state_quant import gated_rmsnorm
    gen = torch.Generator(device=device).manual_seed(5)
    print("[gated norm] [2, 3, 8192] rows and rejected operands", flush=True)
    y = torch.randn(2, 3, 8192, generator=gen, device=device).half()
    z = torch.randn(2, 3, 18560, generator=gen, device=device).half()[..., :8192]
    w = torch.ones(8192, device=device, dtype=torch.float16)
    out = gated_rmsnorm(y, z, w, 1e-5, 1024)
    flat = gated_rmsnorm(y.reshape(6, 8192), z.contiguous().reshape(6, 8192), w, 1e-5, 1024)
    torch.cuda.synchronize()
    assert torch.equal(out.reshape(6, 8192), flat)
    with pytest.raises(ValueError, match="Gated norm"):
        gated_rmsnorm(y, z.float(), w, 1e-5, 1024)
    with pytest.raises(ValueError, match="Gated norm"):   # leading dimensions of two row strides
        gated_rmsnorm(y.transpose(0, 1), z.transpose(0, 1), w, 1e-5, 1024)
    with pytest.raises(RuntimeError, match="group size"):
        gated_rmsnorm(y, z, w, 1e-5, 1000)
