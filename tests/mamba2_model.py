"""A random-init Mamba-2 8B language model with the module structure and
attribute names of mamba_ssm's MambaLMHeadModel (unfused FP16 residual path),
for exercising the state controllers on a GPU without mamba_ssm.  Only the
pieces the controllers use are implemented: embedding, per-block RMSNorm,
the mixer's in_proj / depthwise causal conv1d / A_log / D / dt_bias / gated
RMSNorm / out_proj, final norm and lm_head.  The mixer's own forward is never
called: an installed controller replaces it."""
import math

import torch
from torch import nn
import torch.nn.functional as F


def _mean_square(v):
    """Mean of v^2 over the last dimension (a multiple of 64 wide) as two
    reductions of at most 64 elements per output: each output fits one
    workgroup, so no reduction splits across workgroups (which would clear
    semaphores with a memset inside a captured HIP graph)."""
    n = v.shape[-1]
    partial = v.pow(2).reshape(*v.shape[:-1], n // 64, 64).sum(-1)
    return partial.sum(-1, keepdim=True) / n


class RMSNorm(nn.Module):
    def __init__(self, d, eps=1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x):
        v = x.float()
        v = v * torch.rsqrt(_mean_square(v) + self.eps)
        return (v * self.weight.float()).to(x.dtype)


class GatedRMSNorm(nn.Module):
    """norm(y * silu(z)) per group of `group_size` channels, times weight."""

    def __init__(self, d, group_size, eps=1e-5):
        super().__init__()
        self.eps, self.group_size = eps, group_size
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, y, z):
        v = y.float() * F.silu(z.float())
        shape = v.shape
        v = v.reshape(*shape[:-1], shape[-1] // self.group_size, self.group_size)
        v = v * torch.rsqrt(_mean_square(v) + self.eps)
        return (v.reshape(shape) * self.weight.float()).to(y.dtype)


class Mixer(nn.Module):
    def __init__(self, d_model=4096, d_inner=8192, nheads=128, d_state=128, ngroups=8, d_conv=4):
        super().__init__()
        self.d_model, self.d_inner, self.d_ssm, self.nheads = d_model, d_inner, d_inner, nheads
        self.headdim, self.d_state, self.ngroups, self.d_conv = d_inner // nheads, d_state, ngroups, d_conv
        self.use_mem_eff_path, self.rmsnorm, self.D_has_hdim = False, True, False
        self.activation, self.dt_limit, self.process_group = "silu", (0.0, float("inf")), None
        conv_dim = d_inner + 2 * ngroups * d_state
        self.in_proj = nn.Linear(d_model, 2 * d_inner + 2 * ngroups * d_state + nheads, bias=False)
        self.conv1d = nn.Conv1d(conv_dim, conv_dim, d_conv, groups=conv_dim, padding=d_conv - 1, bias=True)
        self.act = nn.SiLU()
        self.A_log = nn.Parameter(torch.empty(nheads))
        self.D = nn.Parameter(torch.empty(nheads))
        self.dt_bias = nn.Parameter(torch.empty(nheads))
        self.norm = GatedRMSNorm(d_inner, d_inner // ngroups)
        self.out_proj = nn.Linear(d_inner, d_model, bias=False)

    def forward(self, u, **kwargs):
        raise RuntimeError("native Mamba-2 mixer forward is not available; install a state controller")


class Block(nn.Module):
    def __init__(self, d_model):
        super().__init__()
        self.mixer = Mixer(d_model)
        self.norm = RMSNorm(d_model)
        self.fused_add_norm, self.residual_in_fp32, self.mlp = False, False, None

    def forward(self, hidden, residual=None):
        residual = hidden if residual is None else hidden + residual
        return self.mixer(self.norm(residual)), residual


class Backbone(nn.Module):
    def __init__(self, layers, d_model, vocab):
        super().__init__()
        self.embedding = nn.Embedding(vocab, d_model)
        self.layers = nn.ModuleList(Block(d_model) for _ in range(layers))
        self.norm_f = RMSNorm(d_model)
        self.fused_add_norm, self.residual_in_fp32 = False, False

    def forward(self, ids):
        hidden, residual = self.embedding(ids), None
        for layer in self.layers:
            hidden, residual = layer(hidden, residual)
        return self.norm_f(hidden + residual)


class Mamba2LM(nn.Module):
    def __init__(self, layers=56, d_model=4096, vocab=256000):
        super().__init__()
        self.backbone = Backbone(layers, d_model, vocab)
        self.lm_head = nn.Linear(d_model, vocab, bias=False)


@torch.no_grad()
def random_model(device, seed=0):
    """Frozen FP16 8B model built directly on `device` with seeded weights."""
    with torch.device("meta"):
        model = Mamba2LM()
    model = model.to_empty(device=device).half()
    gen = torch.Generator(device=device).manual_seed(seed)
    for name, p in model.named_parameters():
        if name.endswith("A_log"):
            p.copy_(torch.log(torch.rand(p.shape, generator=gen, device=device) * 15 + 1))
        elif name.endswith(".D"):
            p.copy_(torch.randn(p.shape, generator=gen, device=device))
        elif name.endswith("dt_bias"):
            p.copy_(torch.log(torch.expm1(torch.rand(p.shape, generator=gen, device=device) * 0.09 + 0.01)))
        elif name.endswith("norm.weight") or name.endswith("norm_f.weight"):
            p.fill_(1.0)
        elif name.endswith("conv1d.bias"):
            p.zero_()
        else:
            fan_in = p.shape[-1] if p.ndim > 1 else 1
            p.normal_(0.0, 1.0 / math.sqrt(fan_in), generator=gen)
    return model.requires_grad_(False).eval()
