"""Benchmark of the MI355X state codec and FP4 weight decode.

Headline (`value`): algorithmic GB/s of one 56-layer token step of the
published ridge-latent state codec (fused selective-state step +
per-token requantization) at batch 64, BASELINE config 4, with the published
per-layer layouts.  One step = 56 per-layer kernel launches replayed as a
HIP graph; inputs and packed states are resident in HBM.  Also reported:
the same step at batch 1 (µs/token, graph of 56 launches), the full 8B FP4
G16 decode, the measured device-to-device copy
bandwidth, a live roofline for the dominant kernel, and the CPU oracle
timed on a bounded sample (state step and FP4 decode) as a baseline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-fp4] [--skip-cpu] [--skip-e2e]
       python bench.py --only step|copy|codecs|layers|ceiling|e2e|loader|prefill|fp4
       (profiling runs: only the step graph at --batch, only a 256 MiB copy
       used to calibrate counters, only the other codecs' batch-64 graphs,
       only the one-launch multi-layer step at --batch, only the HBM
       ceilings, only the end-to-end decode, only the checkpoint loader,
       only the batch-1 prefill, only the FP4 full decode)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "mamb2_8b_fp4_recall_sq3.25_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = "state codec GB/s (frac HBM peak); 56-layer per-token requant µs, batch 1/64"
HBM_PEAK_GBS = 8000.0
# evaluation/wt2_test_v1/comparison.json state_provenance.layouts (per layer)
PUBLISHED_LAYOUTS = (
    "36_24_68", "16_64_48", "32_32_64", "40_16_72", "16_64_48", "16_64_48", "24_48_56", "32_32_64", "32_32_64",
    "32_32_64", "32_32_64", "36_24_68", "40_16_72", "24_48_56", "8_80_40", "32_32_64", "32_32_64", "32_32_64",
    "32_32_64", "24_48_56", "16_64_48", "16_64_48", "24_48_56", "16_64_48", "32_32_64", "24_48_56", "24_48_56",
    "8_80_40", "40_16_72", "32_32_64", "24_48_56", "24_48_56", "40_16_72", "36_24_68", "16_64_48", "8_80_40",
    "16_64_48", "24_48_56", "44_8_76", "36_24_68", "24_48_56", "24_48_56", "16_64_48", "32_32_64", "8_80_40",
    "32_32_64", "8_80_40", "8_80_40", "24_48_56", "8_80_40", "16_64_48", "44_8_76", "44_8_76", "8_80_40",
    "24_48_56", "32_32_64")
H, P, G, NSTATE = 128, 64, 8, 128


def ridge_counts(layout):
    a, b, c = map(int, layout.split("_"))
    return a, b - 4, c + 4


def step_bytes(batch, layouts):
    """Algorithmic HBM bytes of one 56-layer step: per layer
    889,088*B (packed state in+out 2*52*8192, x and y 2*16384, B and C 4096,
    dt 256) plus statics perm 1024 + basis 32*nz + lscale 32 +
    predictor 16*F*nz + A/D/dt_bias 1024."""
    total = 0
    for layout in layouts:
        n8, n4, nz = ridge_counts(layout)
        F = n8 + n4 + 2
        total += 889_088 * batch + 1024 + 32 * nz + 32 + 16 * F * nz + 1024
    return total


class RidgeStack:
    """56 layers of resident inputs, statics and packed states."""

    def __init__(self, batch, device, seed=2026, tokens=1):
        from mamba2_recall import _native, ridge_codec
        self.native = _native
        self.batch = batch
        self.tokens = tokens
        self.device = device
        self.ws = None   # token-record workspace of a multi-token stack (allocated on first launch)
        gen = torch.Generator(device=device).manual_seed(seed)
        f16 = torch.float16
        self.layers = []
        for i, layout in enumerate(PUBLISHED_LAYOUTS):
            n8, n4, nz = ridge_counts(layout)
            F = n8 + n4 + 2
            d = dict(layout=layout, n8=n8, n4=n4, nz=nz)
            d["x"] = torch.randn((batch, tokens, H, P), generator=gen, device=device).to(f16)
            d["dt"] = torch.randn((batch, tokens, H), generator=gen, device=device).to(f16)
            u = torch.rand(H, generator=gen, device=device) * float(np.log(16.0))
            d["A"] = (-torch.exp(u)).float().contiguous()
            d["B"] = torch.randn((batch, tokens, G, NSTATE), generator=gen, device=device).to(f16)
            d["C"] = torch.randn((batch, tokens, G, NSTATE), generator=gen, device=device).to(f16)
            d["D"] = torch.randn(H, generator=gen, device=device).to(f16)
            d["dt_bias"] = torch.zeros(H, device=device, dtype=f16)
            d["perm"] = torch.stack([torch.randperm(NSTATE, generator=gen, device=device)
                                     for _ in range(G)]).to(torch.uint8).contiguous()
            d["basis"] = (torch.randn((G, nz, 2), generator=gen, device=device) * 0.03).to(f16)
            d["lscale"] = torch.full((G, 2), 0.001, device=device, dtype=f16)
            d["pred"] = (torch.randn((G, F, nz), generator=gen, device=device) * 0.05).to(f16)
            d["state"] = ridge_codec.allocate_state(batch, H, P, NSTATE, device, layout=layout)
            d["y"] = torch.empty_like(d["x"])
            self.layers.append(d)
        # warm the carry from zero with 16 tokens per layer,
        # as 16 one-token steps (equal to one 16-token call; keeps every launch
        # of the kernel a one-token launch, as in the timed region); a
        # multi-token stack starts from the carry of one pass over its tokens
        for d in self.layers:
            for t in range(16 if tokens == 1 else 1):
                ridge_codec.scan(d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], d["dt_bias"], d["state"],
                                 d["perm"], d["basis"], d["lscale"], d["pred"], layout=d["layout"], validate=(t == 0))
        torch.cuda.synchronize()

    def launch_all(self, stream_handle):
        """The 56 layers in order; a multi-token stack passes its token-record
        workspace (one buffer: the layers run one after another on one
        stream), as ridge_codec.scan does for multi-token calls."""
        p = self.native.ptr
        if self.tokens > 1 and self.ws is None:
            nbytes = int(self.native.lib().m2r_ridge_records_bytes(self.batch, self.tokens, G))
            self.ws = torch.empty(nbytes // 4, dtype=torch.float32, device=self.device)
        ws, ws_bytes = (p(self.ws), self.ws.numel() * 4) if self.ws is not None else (None, 0)
        for d in self.layers:
            t = d["state"].tensors
            self.native.call("m2r_state_step_ridge_ws", p(d["x"]), p(d["dt"]), p(d["A"]), p(d["B"]), p(d["C"]),
                             p(d["D"]), 0, p(d["dt_bias"]), 0, p(d["perm"]), p(d["basis"]), p(d["lscale"]),
                             p(d["pred"]), p(t["lo"]), p(t["hi"]), p(t["q4"]), p(t["latent"]), p(t["s8"]),
                             p(t["s4"]), p(d["y"]), self.batch, self.tokens, H, P, G, d["n8"], d["n4"], d["nz"],
                             ws, ws_bytes, stream_handle)

    def graph(self):
        import ctypes
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.launch_all(ctypes.c_void_p(s.cuda_stream))   # untimed warm-up on the side stream
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            self.launch_all(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        return g


def prefill_timing(device, tokens=2048, steps=5, warmup=2):
    """The reference's perplexity path runs each ~2047-token window through
    every layer as one multi-token scan (scripts/run_fp4_ridge_resurface_v3.py:
    102): the 56 published layers at batch 1, each one launch of the
    runtime-L ridge instance over `tokens` tokens (the state stays in
    registers and LDS across the tokens), as a graph of 56 launches.
    Algorithmic bytes per layer: packed state in and out once, the statics,
    and per token x, y, B, C and dt.  Returns ms per window, µs per token
    (all 56 layers) and GB/s."""
    stack = RidgeStack(1, device, seed=2028, tokens=tokens)
    g = stack.graph()
    ms, _ = time_graph(g, steps, warmup)
    del g
    per_token = 2 * 16384 + 2 * 2048 + 256
    nbytes = sum(2 * 52 * 8192 + per_token * tokens + (step_bytes(1, (lay,)) - 889_088) for lay in PUBLISHED_LAYOUTS)
    del stack
    torch.cuda.empty_cache()
    return dict(tokens=tokens, ms_per_window=round(ms, 3), us_per_token_56_layers=round(ms * 1e3 / tokens, 3),
                gbs=round(nbytes / (ms * 1e-3) / 1e9, 1),
                note="batch 1, published layouts, one launch per layer of the runtime-L ridge step over the "
                     "whole window (HIP graph of 56 launches)")


def layers_one_launch(stack, steps, warmup):
    """The same 56-layer one-token step as one launch of the multi-layer
    kernel (m2r_state_step_ridge_layers: every workgroup reads its layer's
    arguments from a table in device memory), timed as eager calls, each of
    which copies the table from the host before its launch.  Returns ms per
    56-layer step."""
    import ctypes
    from mamba2_recall import ridge_codec
    steps_ = [dict(x=d["x"], dt=d["dt"], A=d["A"], B=d["B"], C=d["C"], D=d["D"], dt_bias=d["dt_bias"],
                   state=d["state"], permutation=d["perm"], basis=d["basis"], latent_scale=d["lscale"],
                   predictor=d["pred"], layout=d["layout"], y=d["y"]) for d in stack.layers]
    table = ridge_codec.layer_table(steps_)
    n = len(steps_)
    ws = torch.empty(ridge_codec.layers_workspace_bytes(n), dtype=torch.uint8, device=stack.device)
    x = steps_[0]["x"]
    args = (ctypes.byref(table), n, x.shape[0], H, P, G, stack.native.ptr(ws), ws.numel())
    stack.native.call("m2r_state_step_ridge_layers", *args, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(warmup):
        stack.native.call("m2r_state_step_ridge_layers", *args, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(steps):
        stack.native.call("m2r_state_step_ridge_layers", *args, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    ev1.record()
    torch.cuda.synchronize()
    eager_ms = ev0.elapsed_time(ev1) / steps
    return eager_ms


def time_graph(g, steps, warmup):
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return ev0.elapsed_time(ev1) / steps, wall * 1e3 / steps


TRAFFIC_PROFILE = ROOT / "profiles" / "state_step_b64_pmc_traffic.txt"


# the step kernel's sources and the build script (its compiler flags), in the
# package directory
STEP_KERNEL_SOURCES = ("csrc/m2r_state.hip", "csrc/m2r_step.h", "csrc/m2r_device.h", "csrc/m2r_tile.h",
                       "build_lib.py")


def step_kernel_digest():
    """First 16 hex digits of the SHA-256 of the step kernel's sources and
    build script (in STEP_KERNEL_SOURCES order): the key under which a
    traffic profile of that kernel is valid."""
    import hashlib
    h = hashlib.sha256()
    for name in STEP_KERNEL_SOURCES:
        h.update((ROOT / "mamb2_8b_fp4_recall_sq3.25_amd" / name).read_bytes())
    return h.hexdigest()[:16]


def measured_traffic():
    """HBM bytes per launch of the step kernel at batch 64, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), or None when
    the summary is missing or was measured on other kernel sources than the
    ones in this tree (its kernel_source_sha16 line)."""
    try:
        fields = dict(line.split("=", 1) for line in TRAFFIC_PROFILE.read_text().splitlines() if "=" in line)
        if fields.get("kernel_source_sha16", "").strip() != step_kernel_digest():
            return None
        return int(fields["traffic_bytes_per_launch"].strip())
    except (OSError, ValueError, KeyError):
        return None


def copy_bandwidth(device):
    """Device-to-device copy (reads and writes interleaved, 1 GiB each way)
    and a write-only stream (fill of 1 GiB): the two reference rates for the
    HBM-bound kernels.  Returns (copy GB/s counting both directions, fill GB/s)."""
    a = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    b = torch.empty_like(a)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def rate(fn, nbytes):
        fn()
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(10):
            fn()
        ev1.record()
        torch.cuda.synchronize()
        return nbytes * 10 / (ev0.elapsed_time(ev1) * 1e-3) / 1e9

    copy_gbs = rate(lambda: b.copy_(a), 2 * a.numel())
    fill_gbs = rate(lambda: b.fill_(7), b.numel())
    del a, b
    torch.cuda.empty_cache()
    return copy_gbs, fill_gbs


# (bytes read, 16-byte vectors written) per unit
MIXES = {"read_only": (16, 0), "write_only": (0, 1), "copy_1to1": (16, 1), "fp4_mix_22to78": (32, 7),
         "fp4_shape_20to80": (4, 1)}


def stream_ceiling(device, reps=10):
    """HBM ceilings measured by the library's hand-written streaming kernel
    (m2r_stream_probe): read-only, write-only, 1:1 (the state step's mix) and
    22:78 read:write (the FP4 G16 decode's 4.5 bytes read per 16 written),
    and a 4-byte read per 16-byte write (20:80: the decode's access shape,
    256 B read and 1 KiB written per wave instruction).
    Variants: 1 GiB or 4 GiB moved per launch; one unit per lane per step or
    bursts of 8 units' loads before their stores; a grid of 2048 or 16384
    workgroups striding over the buffer, or one step per wave; the default or
    the non-temporal cache policy.  Returns GB/s of bytes moved per variant
    and the best per mix."""
    import ctypes
    from mamba2_recall import _native
    src = torch.empty(2 << 30, dtype=torch.uint8, device=device)
    dst = torch.empty(4 << 30, dtype=torch.uint8, device=device)
    src.fill_(3)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out, best = {}, {}
    for name, (r, w) in MIXES.items():
        per_unit = r + 16 * w
        for size in (1 << 30, 4 << 30):
            units = min((src.numel() // r) if r else 1 << 62, (dst.numel() // (16 * w)) if w else 1 << 62,
                        size // per_unit)
            for burst, blocks, nt in [(b, g, n) for b in ((1, 4) if r == 4 else (1, 8)) for g in (2048, 16384, 0)
                                      for n in (0, 1)]:
                u = units - units % (64 * burst)

                def run():
                    _native.call("m2r_stream_probe", _native.ptr(src), _native.ptr(dst), u, r, w, burst, blocks, nt, h)
                run()
                torch.cuda.synchronize()
                ev0.record()
                for _ in range(reps):
                    run()
                ev1.record()
                torch.cuda.synchronize()
                gbs = u * per_unit * reps / (ev0.elapsed_time(ev1) * 1e-3) / 1e9
                key = f"{name}/{size >> 30}GiB/burst{burst}/{'blocks' + str(blocks) if blocks else 'onestep'}/{'nt' if nt else 'default'}"
                out[key] = round(gbs, 1)
                best[name] = max(best.get(name, 0.0), round(gbs, 1))
    del src, dst
    torch.cuda.empty_cache()
    return dict(best_gbs=best, variants_gbs=out,
                note="m2r_stream_probe: 16-byte loads/stores, contiguous 1 KiB per wave instruction, "
                     "256-thread workgroups; GB/s of bytes read + written")


PHASED_MIXES = {"read_100": (1, 0), "read_0": (0, 1), "read_10": (1, 9), "read_20": (1, 4),
                "read_20_block16k": (4, 16), "read_30": (3, 7), "read_50": (1, 1)}


def stream_sweep(device, reps=10):
    """Read-fraction sweep and time-phased variants of the streaming probe
    (m2r_stream_probe_phased): per 256-thread workgroup step, r 16-byte loads
    then w 16-byte stores per thread (every instruction a contiguous 1 KiB per
    wave), 0/10/20/30/50/100% of the bytes read (20% also with 16 KiB read and
    64 KiB written per workgroup step); phase 0 (a thread stores once its own
    loads land), 1 (a workgroup barrier between the step's loads and stores),
    2 (the stores also complete before the next step's loads); one step per
    workgroup or a grid of 2048 / 8192 workgroups; default or non-temporal
    cache policy.  About 1 GiB moved per launch.  Returns GB/s per variant and
    the best per mix."""
    import ctypes
    from mamba2_recall import _native
    src = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    dst = torch.empty(2 << 30, dtype=torch.uint8, device=device)
    src.fill_(3)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out, best = {}, {}
    for name, (r, w) in PHASED_MIXES.items():
        per_step = 256 * 16 * (r + w)
        steps = min((1 << 30) // per_step, (src.numel() // (256 * 16 * r)) if r else 1 << 62,
                    (dst.numel() // (256 * 16 * max(w, 1))))
        for phase in (0, 1, 2):
            for blocks in (0, 2048, 8192):
                for nt in (0, 1):
                    def run():
                        _native.call("m2r_stream_probe_phased", _native.ptr(src), _native.ptr(dst), steps, r, w,
                                     phase, blocks, nt, h)
                    run()
                    torch.cuda.synchronize()
                    ev0.record()
                    for _ in range(reps):
                        run()
                    ev1.record()
                    torch.cuda.synchronize()
                    gbs = steps * per_step * reps / (ev0.elapsed_time(ev1) * 1e-3) / 1e9
                    key = f"{name}/phase{phase}/{'blocks' + str(blocks) if blocks else 'onestep'}/{'nt' if nt else 'default'}"
                    out[key] = round(gbs, 1)
                    best[name] = max(best.get(name, 0.0), round(gbs, 1))
    del src, dst
    torch.cuda.empty_cache()
    return dict(best_gbs=best, variants_gbs=out,
                note="m2r_stream_probe_phased: GB/s of bytes read + written; read_N = N% of the bytes read")


def fp4_full_decode(device, steps=10):
    """56 x in_proj [18560,4096] + 56 x out_proj [4096,8192]
    + embedding and lm_head [256000,4096]; random nibbles, lognormal(-3,0.5)
    block scales in the reference G16 format (E4M3 of s/global, global =
    max(s)/448)."""
    from mamba2_recall import fp4
    shapes = [(18560, 4096)] * 56 + [(4096, 8192)] * 56 + [(256000, 4096)] * 2
    gen = torch.Generator(device=device).manual_seed(7)
    mats = []
    for rows, cols in shapes:
        packed = torch.randint(0, 256, (rows, cols // 2), generator=gen, device=device, dtype=torch.uint8)
        s = torch.exp(torch.randn((rows, cols // 16), generator=gen, device=device) * 0.5 - 3.0)
        g = (s.max() / 448.0).float().reshape(1)
        sb = (s / g).clamp(0, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        out = torch.empty((rows, cols), dtype=torch.float16, device=device)
        mats.append((packed, sb, g, out, rows, cols))
    nbytes = sum(r * c // 2 + r * c // 16 + 4 + r * c * 2 for r, c in shapes)
    assert nbytes == 21_098_136_008

    def run():
        for packed, sb, g, out, rows, cols in mats:
            fp4.decode_into(packed, sb, g, out, rows=rows, columns=cols, group=16)
    run()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        run()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    del mats
    torch.cuda.empty_cache()
    return ms, nbytes / (ms * 1e-3) / 1e9


def other_codecs(device, batch=64, launches=56, steps=10):
    """Per-launch time of the other state codecs at the benchmark geometry
    (one token, H=128, P=64, G=8), each a graph of `launches` launches of one
    layer with resident inputs: the stored-scale tier codec (layout
    32_32_64), the legacy sq3p25 codec, the dense 3-bit codec (permutation
    table) and the FP16-carry control.  Bytes per launch are algorithmic: the
    packed 52-byte rows in and out (256-byte FP16 rows for the control) plus
    x, y, B, C and dt."""
    import ctypes
    from mamba2_recall import _native
    p = _native.ptr
    gen = torch.Generator(device=device).manual_seed(99)
    f16 = torch.float16
    x = torch.randn(batch, 1, H, P, generator=gen, device=device).to(f16)
    dt = torch.randn(batch, 1, H, generator=gen, device=device).to(f16)
    Bm = torch.randn(batch, 1, G, NSTATE, generator=gen, device=device).to(f16)
    Cm = torch.randn(batch, 1, G, NSTATE, generator=gen, device=device).to(f16)
    A = -torch.exp(torch.rand(H, generator=gen, device=device) * np.log(16.0))
    D = torch.randn(H, generator=gen, device=device).to(f16)
    db = torch.zeros(H, device=device, dtype=f16)
    perm = torch.stack([torch.randperm(NSTATE, generator=gen, device=device) for _ in range(G)]).to(torch.uint8)
    y = torch.empty_like(x)
    rows = batch * H * P
    u8 = lambda n: torch.randint(0, 256, (rows, n), generator=gen, device=device, dtype=torch.uint8)
    sc = lambda n: (torch.rand(rows, n, generator=gen, device=device) * 0.01 + 1e-3).to(f16)
    io = batch * (2 * 16384 + 4096 + 256)
    lo, hi, q4, s8, s4 = u8(16), u8(16), u8(16), sc(1), sc(1)
    codes, scales = u8(48), sc(2)
    state16 = (torch.randn(rows, NSTATE, generator=gen, device=device) * 0.1).to(f16)
    cases = {
        "tier_32_32_64": (lambda h: _native.call(
            "m2r_state_step_tier", p(x), p(dt), p(A), p(Bm), p(Cm), p(D), 0, p(db), 0, p(perm), p(lo), p(hi),
            p(q4), p(s8), p(s4), p(y), batch, 1, H, P, G, 32, 32, 64, h), 2 * 52 * rows + io),
        "legacy_sq3p25": (lambda h: _native.call(
            "m2r_state_step_legacy", p(x), p(dt), p(A), p(Bm), p(Cm), p(D), 0, p(db), 0, p(perm), p(lo), p(hi),
            p(q4), p(s8), p(s4), p(y), batch, 1, H, P, G, h), 2 * 52 * rows + io),
        "dense3": (lambda h: _native.call(
            "m2r_state_step_dense3", p(x), p(dt), p(A), p(Bm), p(Cm), p(D), 0, p(db), 0, p(perm), 0, p(codes),
            p(scales), p(y), batch, 1, H, P, G, h), 2 * 52 * rows + io),
        "s16_control": (lambda h: _native.call(
            "m2r_state_step_s16", p(x), p(dt), p(A), p(Bm), p(Cm), p(D), 0, p(db), 0, p(state16), p(y), None,
            batch, 1, H, P, G, h), 2 * 256 * rows + io),
    }
    out = {}
    for name, (fn, nbytes) in cases.items():
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn(ctypes.c_void_p(s.cuda_stream))
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            h = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for _ in range(launches):
                fn(h)
        ms, _ = time_graph(g, steps, 2)
        us = ms * 1e3 / launches
        out[name] = dict(us_per_launch=round(us, 2), gbs=round(nbytes / (us * 1e-6) / 1e9, 1))
        del g
    return out


def e2e_decode(device, batches=(1, 4, 16), prefill=8, tokens=256, eager_tokens=64):
    """BASELINE config 5, with a shortened continuation: a random-init Mamba-2
    8B model (56 layers, d_model 4096, d_inner 8192, vocab 256000) whose
    in_proj, out_proj, embedding and lm_head weights are decoded on the device
    from seeded FP4 G16 packets (uniform nibbles; lognormal block scales sized
    for unit-variance activations, global = max/448, E4M3 block bytes), with
    the ridge-latent per-token requantize hook installed on every layer
    (published layouts, seeded statics).  Greedy decode: a prefill of
    `prefill` tokens, two untimed steps, then `tokens` timed steps of
    backbone + lm_head + argmax, eager, and with the backbone replayed as one
    captured HIP graph per step (lm_head and argmax stay eager), with the
    projections as FP16 GEMMs and (batch sizes the kernel takes) as
    packed-resident FP4 GEMVs; the hook's per-call host validation
    is off (statics are validated once).  The eager run covers the first
    `eager_tokens` steps (its ids and layer 0's packed state are the
    reference the graph replays are checked against); the graph is timed over
    `tokens` steps.  Returns ms per generated token."""
    import math
    import torch.nn.functional as F
    sys.path.insert(0, str(ROOT / "tests"))
    import cases
    from mamba2_model import random_model
    from mamba2_recall import fp4, ridge_codec
    model = random_model(device, seed=11)
    gen = torch.Generator(device=device).manual_seed(12)

    def packet(w):
        rows, cols = w.shape
        packed = torch.randint(0, 256, (rows, cols // 2), generator=gen, device=device, dtype=torch.uint8)
        # E|level|^2 of a uniform nibble is 68.5/8: scales for weight variance 1/cols
        sc = torch.exp(torch.randn((rows, cols // 16), generator=gen, device=device) * 0.5) / math.sqrt(8.5625 * cols)
        g = (sc.max() / 448.0).float().reshape(1)
        sb = (sc / g).clamp(0, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        fp4.decode_into(packed, sb, g, w.data, rows=rows, columns=cols, group=16)
        return packed, sb, g

    packet(model.backbone.embedding.weight)
    packet(model.lm_head.weight)
    packets = [dict(in_proj=packet(layer.mixer.in_proj.weight), out_proj=packet(layer.mixer.out_proj.weight))
               for layer in model.backbone.layers]
    torch.cuda.synchronize()
    rng = np.random.default_rng(13)
    perms = torch.stack([torch.from_numpy(rng.permutation(128).astype(np.uint8)) for _ in range(56 * 8)])
    perms = perms.reshape(56, 8, 128)
    bases, scales, preds = [], [], []
    for layout in PUBLISHED_LAYOUTS:
        n8, n4, nz = ridge_counts(layout)
        st = cases.ridge_statics(rng, G, n8, n4, nz)
        bases.append(torch.from_numpy(st["basis"].view(np.float16)))
        scales.append(torch.from_numpy(st["lscale"].view(np.float16)))
        preds.append(torch.from_numpy(st["pred"].view(np.float16)))
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(reps):
            fn()
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / reps

    def next_ids(hidden):
        # lm_head and the argmax over 256000 logits run eagerly, outside the
        # captured graphs: that argmax is a multi-workgroup torch reduction
        # that clears its semaphores with hipMemsetAsync, and memset nodes in
        # captured graphs are not reliable on replay
        return model.lm_head(hidden[:, -1:]).float().argmax(-1)

    def snapshot(pq):
        return [(e.conv.clone(), {k: v.clone() for k, v in e.state.tensors.items()}) for e in pq._cache]

    def restore(pq, snap):
        for e, (conv, tensors) in zip(pq._cache, snap):
            e.conv.copy_(conv)
            for k, v in tensors.items():
                e.state.tensors[k].copy_(v)

    def decode_modes(pq, snap, start):
        """Eager run from the snapshot, the same step captured as a HIP graph,
        replays checked token by token and on layer 0's packed state against
        the eager run, then `tokens` replays timed from the snapshot."""
        restore(pq, snap)
        nxt, eager_ids, first_logits = start.clone(), [], None
        torch.cuda.synchronize()
        ev0.record()
        for i in range(eager_tokens):
            logits = model.lm_head(pq.backbone(nxt)[:, -1:]).float()
            first_logits = logits.clone() if i == 0 else first_logits
            nxt = logits.argmax(-1)
            eager_ids.append(nxt)
        ev1.record()
        torch.cuda.synchronize()
        eager_ms = ev0.elapsed_time(ev1) / eager_tokens
        eager_state = {k: v.clone() for k, v in pq._cache[0].state.tensors.items()}
        restore(pq, snap)
        static_ids = start.clone()
        static_hidden = torch.empty(start.shape[0], 1, 4096, dtype=torch.float16, device=device)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):   # capture warm-up, then the snapshot is restored
            static_hidden.copy_(pq.backbone(static_ids))
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        restore(pq, snap)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_hidden.copy_(pq.backbone(static_ids))

        def step():   # one decode step: the backbone graph, then the eager head and feedback
            graph.replay()
            static_ids.copy_(next_ids(static_hidden))

        graph_ids = []
        for _ in range(eager_tokens):
            step()
            graph_ids.append(static_ids.clone())
        torch.cuda.synchronize()
        same = all(torch.equal(a, b) for a, b in zip(eager_ids, graph_ids)) and all(
            torch.equal(pq._cache[0].state.tensors[k], v) for k, v in eager_state.items())
        restore(pq, snap)
        static_ids.copy_(start)
        graph_ms = timed(step, tokens)
        finite = bool(pq.assert_finite_cache())
        del graph
        return dict(eager_ms=eager_ms, graph_ms=graph_ms, same=same, finite=finite, logits=first_logits)

    out = {}
    with torch.no_grad():
        # the projections alone, batch 1: FP16 GEMM (hipBLASLt) vs the packed FP4
        # GEMV, each as a graph of one launch per layer (device time per launch)
        u1 = torch.randn(1, 4096, generator=gen, device=device).half()
        u2 = torch.randn(1, 8192, generator=gen, device=device).half()
        mods = [layer.mixer for layer in model.backbone.layers]

        def graph_us(step):
            step()
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                step()
            us = timed(gr.replay, 20) * 1e3 / len(mods)
            del gr
            return round(us, 2)

        out["projection_us_batch1"] = dict(
            in_proj_fp16=graph_us(lambda: [F.linear(u1, m.in_proj.weight) for m in mods]),
            in_proj_fp4_gemv=graph_us(lambda: [fp4.gemv_g16(*pk["in_proj"], u1) for pk in packets]),
            out_proj_fp16=graph_us(lambda: [F.linear(u2, m.out_proj.weight) for m in mods]),
            out_proj_fp4_gemv=graph_us(lambda: [fp4.gemv_g16(*pk["out_proj"], u2) for pk in packets]),
            note="graph of 56 launches (one per layer's matrix), device time per launch")
        for batch in batches:
            with ridge_codec.PredictorState(model, perms, PUBLISHED_LAYOUTS, bases, scales, preds) as pq:
                pq.validate_each_step = False
                ids = torch.randint(0, 256000, (batch, prefill), generator=gen, device=device)
                nxt = next_ids(pq.backbone(ids, reset=True))
                for _ in range(2):
                    nxt = next_ids(pq.backbone(nxt))
                torch.cuda.synchronize()
                snap, start = snapshot(pq), nxt.clone()
                r16 = decode_modes(pq, snap, start)
                row = dict(eager_ms_per_token=round(r16["eager_ms"], 3), graph_ms_per_token=round(r16["graph_ms"], 3),
                           graph_tokens_per_s=round(batch * 1e3 / r16["graph_ms"], 1),
                           graph_matches_eager=r16["same"], finite_cache=r16["finite"])
                if fp4.gemv_supported(batch, 4096):
                    pq.use_packed_projections(packets, verify=(batch == batches[0]))
                    rp = decode_modes(pq, snap, start)
                    pq.use_packed_projections(None)
                    rel = float((rp["logits"] - r16["logits"]).norm() / r16["logits"].norm())
                    row.update(packed_fp4_graph_ms_per_token=round(rp["graph_ms"], 3),
                               packed_fp4_graph_tokens_per_s=round(batch * 1e3 / rp["graph_ms"], 1),
                               packed_fp4_eager_ms_per_token=round(rp["eager_ms"], 3),
                               packed_fp4_graph_matches_eager=rp["same"], packed_fp4_finite_cache=rp["finite"],
                               packed_fp4_first_logits_rel_l2_vs_fp16=round(rel, 6))
            out[f"batch{batch}"] = row
    del model, packets
    torch.cuda.empty_cache()
    out["note"] = (f"random-init 8B, FP16 weights decoded from seeded FP4 G16; ridge hook on 56 layers; prefill "
                   f"{prefill}; {eager_tokens} eager greedy tokens (the reference the graph replays are checked "
                   f"against, token by token and on layer 0's packed state) and {tokens} timed greedy tokens, each "
                   f"one replay of the captured backbone graph plus the eager lm_head, argmax and token "
                   f"feedback; PyTorch GEMMs around the HIP codec, convolution-update and "
                   f"gated-norm kernels; packed_fp4: the one-token in_proj/out_proj as "
                   f"packed-resident FP4 G16 GEMVs")
    return out


def loader_bench(device, layers=8, shard_limit=256 << 20):
    """The packed-checkpoint loader (fp4_checkpoint.load_packed_tensors) on a
    synthetic checkpoint in the reference's shard format: `layers` layers'
    in_proj [18560, 4096] and out_proj [4096, 8192] as FP4 G16 parts of at
    most `shard_limit` bytes, written to a temporary directory (so read from
    the page cache), then loaded: pinned host buffers, host-to-device copies
    and the device decode into resident FP16.  Returns the rates over packed
    (file) bytes and decoded bytes."""
    import tempfile
    from mamba2_recall import fp4_checkpoint as ck
    ledger = {"tensors": {}}
    for i in range(layers):
        ledger["tensors"][f"backbone.layers.{i}.mixer.in_proj.weight"] = {"kind": "fp4_g16_e4m3", "shape": [18560, 4096]}
        ledger["tensors"][f"backbone.layers.{i}.mixer.out_proj.weight"] = {"kind": "fp4_g16_e4m3", "shape": [4096, 8192]}
    plan = ck.make_plan(ledger, shard_limit)
    rng = np.random.default_rng(21)
    packed_bytes = decoded_bytes = 0
    with tempfile.TemporaryDirectory() as tmp:
        tmp = Path(tmp)
        headers = {f: ck._create_shard(tmp / f, spec) for f, spec in ck._file_specs(plan).items()}

        def write(path, key, data):
            base, header = headers[path]
            begin, end = header[key]["data_offsets"]
            with open(tmp / path, "r+b") as f:
                f.seek(base + begin)
                f.write(data)

        for name, item in sorted(plan.items()):
            rows, cols = item["shape"]
            write(item["global_scale_file"], "global_scale", np.float32(0.01).tobytes())
            for part in item["parts"]:
                n = part["row_stop"] - part["row_start"]
                write(part["file"], "codes", rng.integers(0, 256, (n, cols // 2), dtype=np.uint8).tobytes())
                write(part["file"], "block_scale_bytes", rng.integers(0x20, 0x60, (n, cols // 16), dtype=np.uint8).tobytes())
            packed_bytes += rows * cols // 2 + rows * cols // 16 + 4
            decoded_bytes += rows * cols * 2
        ck.load_packed_tensors(tmp, plan, device=device)   # warm-up: page cache and pinned buffers
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tensors = ck.load_packed_tensors(tmp, plan, device=device)
        torch.cuda.synchronize()
        secs = time.perf_counter() - t0
        del tensors
    torch.cuda.empty_cache()
    return dict(matrices=len(plan), packed_bytes=packed_bytes, seconds=round(secs, 4),
                packed_gbs=round(packed_bytes / secs / 1e9, 2), decoded_gbs=round(decoded_bytes / secs / 1e9, 2),
                note="synthetic checkpoint in the reference shard format, files in the page cache; pinned host "
                     "buffers, host-to-device copies and device decode; wall clock")


def cpu_baseline(budget_s=12.0, fp4_budget_s=3.0):
    """The C oracle (OpenMP over rows) on a bounded sample of the batch-64
    workload: the published layers in order at batch 8, repeated until the
    budget is spent; throughput in algorithmic GB/s.  Beside it, the oracle's
    FP4 G16 decode on a bounded sample of the full-set workload."""
    sys.path.insert(0, str(ROOT / "tests"))
    import cases
    from oracle import oracle
    oracle.build()
    rng = np.random.default_rng(1)
    batch = 8
    done_bytes, elapsed, layers = 0, 0.0, 0
    for layout in PUBLISHED_LAYOUTS * 64:
        n8, n4, nz = ridge_counts(layout)
        inp = cases.step_inputs(rng, batch, 1, H, P, G)
        sta = cases.ridge_statics(rng, G, n8, n4, nz)
        st = cases.random_packed_state(rng, batch, H, P, n8, n4, latent=True)
        t0 = time.perf_counter()
        oracle.state_step(oracle.MODE_RIDGE, n8, n4, nz, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"],
                          inp["D"], inp["dt_bias"], inp["perm"], sta["basis"], sta["lscale"], sta["pred"], st)
        elapsed += time.perf_counter() - t0
        done_bytes += step_bytes(batch, (layout,))
        layers += 1
        if elapsed >= budget_s:
            break
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    # FP4 G16 decode: one in_proj and one out_proj matrix per round (the
    # reference's sample for the full-set rate), algorithmic bytes = codes +
    # block scales + FP16 output
    fp4_bytes, fp4_s, rounds = 0, 0.0, 0
    while fp4_s < fp4_budget_s:
        for rows, cols in ((4096, 4096), (1024, 8192)):   # row slices of one in_proj and one out_proj
            codes = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
            blocks = rng.integers(0x30, 0x48, (rows, cols // 16), dtype=np.uint8)
            t0 = time.perf_counter()
            _, err = oracle.fp4_decode(16, codes, blocks, 1.0 / 448.0, rows, cols)
            fp4_s += time.perf_counter() - t0
            if err:
                raise RuntimeError(f"CPU FP4 baseline: decode rejected a valid packet (bits {err})")
            fp4_bytes += rows * cols // 2 + rows * cols // 16 + 2 * rows * cols
        rounds += 1
    torch_leg = torch_cpu_baseline(cores)
    return dict(value=round(done_bytes / elapsed / 1e9, 4), unit="GB/s", cores=cores, kind="port",
                cpu_model=cpu_model(),
                sample=f"C oracle (OpenMP over rows), {layers} published ridge layer steps in order at batch "
                       f"{batch}, 1 token each, {elapsed:.1f} s",
                fp4_g16_decode=dict(value=round(fp4_bytes / fp4_s / 1e9, 3), unit="GB/s", cores=cores, kind="port",
                                    sample=f"C oracle, {rounds} x (in_proj rows [4096,4096] + out_proj rows "
                                           f"[1024,8192]), {fp4_s:.1f} s"),
                pytorch_cpu=torch_leg)


def cpu_model():
    """The host CPU's model name (first processor in /proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def torch_cpu_baseline(threads, budget_s=2.0):
    """The PyTorch-CPU restatements (oracle/torch_cpu.py) with
    torch.set_num_threads(threads): the FP4 G16 decode of the first 4096 rows
    of an in_proj and the first 1024 rows of an out_proj per round
    (algorithmic bytes: codes + block scales + FP16 output), and the packed-row dequantization of one published-layout layer
    at batch 8 (52-byte rows in, 512 FP32 bytes out per row), each repeated
    for about `budget_s` seconds."""
    from oracle import torch_cpu
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        gen = torch.Generator().manual_seed(5)
        mats = []
        for rows, cols in ((4096, 4096), (1024, 8192)):   # row slices of one in_proj and one out_proj
            codes = torch.randint(0, 256, (rows, cols // 2), generator=gen, dtype=torch.uint8)
            blocks = torch.randint(0x30, 0x48, (rows, cols // 16), generator=gen, dtype=torch.uint8)
            mats.append((codes, blocks, rows * cols // 2 + rows * cols // 16 + 2 * rows * cols))
        fp4_bytes, fp4_s, rounds = 0, 0.0, 0
        while fp4_s < budget_s:
            for codes, blocks, nbytes in mats:
                t0 = time.perf_counter()
                torch_cpu.fp4_g16_decode(codes, blocks, 1.0 / 448.0)
                fp4_s += time.perf_counter() - t0
                fp4_bytes += nbytes
            rounds += 1
        n8, n4, _ = ridge_counts("32_32_64")
        rows = 8 * H * P
        st = dict(lo=torch.randint(0, 256, (rows, n8 // 2), generator=gen, dtype=torch.uint8),
                  hi=torch.randint(0, 256, (rows, n8 // 2), generator=gen, dtype=torch.uint8),
                  q4=torch.randint(0, 256, (rows, n4 // 2), generator=gen, dtype=torch.uint8),
                  s8=(torch.rand(rows, generator=gen) * 0.01).half().view(torch.int16),
                  s4=(torch.rand(rows, generator=gen) * 0.1).half().view(torch.int16))
        dec_bytes, dec_s, calls = 0, 0.0, 0
        while dec_s < budget_s:
            t0 = time.perf_counter()
            torch_cpu.decode_rows(st["lo"], st["hi"], st["q4"], st["s8"], st["s4"], n8, n4)
            dec_s += time.perf_counter() - t0
            dec_bytes += rows * (52 + 512)
            calls += 1
    finally:
        torch.set_num_threads(previous)
    return dict(fp4_g16_decode=dict(value=round(fp4_bytes / fp4_s / 1e9, 3), unit="GB/s", cores=threads,
                                    kind="port", sample=f"oracle/torch_cpu.py, {rounds} x (in_proj rows [4096,4096] + "
                                                        f"out_proj rows [1024,8192]), {fp4_s:.1f} s"),
                decode_state=dict(value=round(dec_bytes / dec_s / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                                  sample=f"oracle/torch_cpu.py packed-row dequantization, layout 32_32_64, batch 8 "
                                         f"({rows} rows), {calls} calls, {dec_s:.1f} s"))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--step-shape", default=None, metavar="WAVES,HEADS",
                    help="with --only step or prefill: force the step kernel's workgroup shape (m2r_set_step_shape), "
                         "for counter runs that compare shapes")
    ap.add_argument("--skip-fp4", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only", choices=("step", "copy", "codecs", "e2e", "loader", "ceiling", "layers", "prefill", "fp4"),
                    default=None)
    ap.add_argument("--skip-e2e", action="store_true", help="skip the end-to-end 8B decode (BASELINE config 5)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the state codec and FP4 decode shard with no communication "
              "(rows by sequence or B/C group; weights by matrix rows), so multi-GPU runs are not part of "
              "this build. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda:0")
    from mamba2_recall import _native
    _native.lib()
    if args.only == "copy":   # counter calibration: the probe's 1:1 copy of 256 MiB, known bytes each way
        import ctypes
        a = torch.full((256 << 20,), 3, dtype=torch.uint8, device=device)
        b = torch.empty_like(a)
        h = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for _ in range(args.steps):
            _native.call("m2r_stream_probe", _native.ptr(a), _native.ptr(b), a.numel() // 16, 16, 1, 1, 2048, 0, h)
        torch.cuda.synchronize()
        print(json.dumps(dict(only="copy", kernel="k_stream_probe<16, 1, 1, false>", bytes_read=a.numel(),
                              bytes_written=a.numel(), launches=args.steps)))
        return

    if args.step_shape:
        if args.only not in ("step", "prefill"):
            raise SystemExit("--step-shape applies to --only step and --only prefill")
        _native.call("m2r_set_step_shape", *(int(v) for v in args.step_shape.split(",")))
    if args.only == "prefill":
        print(json.dumps(dict(only="prefill", step_shape=args.step_shape, prefill_b1_2048=prefill_timing(device))))
        return
    if args.only == "ceiling":
        print(json.dumps(dict(only="ceiling", ceiling=stream_ceiling(device), sweep=stream_sweep(device))))
        return
    if args.only == "loader":
        print(json.dumps(dict(only="loader", loader=loader_bench(device))))
        return
    if args.only == "e2e":
        print(json.dumps(dict(only="e2e", e2e_decode=e2e_decode(device))))
        return
    if args.only == "fp4":   # the FP4 G16 full 8B decode alone (profiling runs)
        fp4_ms, fp4_gbs = fp4_full_decode(device, steps=args.steps)
        print(json.dumps(dict(only="fp4", fp4_g16_full_decode_ms=round(fp4_ms, 3), fp4_g16_full_decode_gbs=round(fp4_gbs, 1))))
        return
    if args.only == "codecs":
        print(json.dumps(dict(only="codecs", other_codecs_b64=other_codecs(device, steps=args.steps))))
        return

    if args.only == "layers":   # the one-launch multi-layer step alone (profiling runs)
        stack = RidgeStack(args.batch, device)
        ms = layers_one_launch(stack, args.steps, args.warmup)
        print(json.dumps(dict(only="layers", batch=args.batch, ms_per_step=round(ms, 5))))
        return
    stack = RidgeStack(args.batch, device)
    g = stack.graph()
    ms, wall_ms = time_graph(g, args.steps, args.warmup)
    nbytes = step_bytes(args.batch, PUBLISHED_LAYOUTS)
    gbs = nbytes / (ms * 1e-3) / 1e9
    # average launch of the step kernel: the timed graph region (HIP events on
    # the replay stream) over its 56 launches per step
    kern_us = ms * 1e3 / len(PUBLISHED_LAYOUTS)
    per_launch = nbytes / len(PUBLISHED_LAYOUTS)
    achieved = per_launch / (kern_us * 1e-6) / 1e9
    del g
    if args.only != "step":   # the same 56 layers as one launch of the multi-layer kernel
        ms_one = layers_one_launch(stack, args.steps, args.warmup)
    del stack
    torch.cuda.empty_cache()
    if args.only == "step":
        print(json.dumps(dict(only="step", batch=args.batch, step_shape=args.step_shape, ms_per_step=round(ms, 5),
                              avg_launch_us=round(kern_us, 3))))
        return

    stack1 = RidgeStack(1, device, seed=2027)
    g1 = stack1.graph()
    ms1, _ = time_graph(g1, max(args.steps, 50), args.warmup)
    ms1_one = layers_one_launch(stack1, max(args.steps, 50), args.warmup)
    del g1, stack1
    torch.cuda.empty_cache()

    copy_gbs, fill_gbs = copy_bandwidth(device)
    ceiling = stream_ceiling(device)
    best = ceiling["best_gbs"]
    extra = dict(batch1_us_per_token=round(ms1 * 1e3, 2), batch1_gbs=round(step_bytes(1, PUBLISHED_LAYOUTS) / (ms1 * 1e-3) / 1e9, 1),
                 batch1_one_launch_us_per_token=round(ms1_one * 1e3, 2),
                 batch1_one_launch_note="the 56 synthetic layers as one launch of the multi-layer kernel "
                                        "(layer table copied from the host every call), not a graph of 56 launches",
                 batch64_us_per_token=round(ms * 1e3, 2), wall_ms_per_step=round(wall_ms, 4),
                 batch64_one_launch_ms_per_step=round(ms_one, 4),
                 batch64_one_launch_gbs=round(nbytes / (ms_one * 1e-3) / 1e9, 1),
                 batch64_one_launch_note="the same 56 layers as one launch of the multi-layer kernel: later "
                                         "workgroups' starts overlap earlier ones' slots; a model cannot use it "
                                         "between its layers (each layer's inputs come from the previous one's "
                                         "projections), so the headline is the graph of 56 per-layer launches",
                 d2d_copy_gbs=round(copy_gbs, 1), write_only_fill_gbs=round(fill_gbs, 1),
                 hbm_frac_of_copy=round(gbs / copy_gbs, 4),
                 hbm_ceiling_best_gbs=best,
                 step_frac_of_1to1_ceiling=round(achieved / best["copy_1to1"], 4))
    if not args.skip_fp4:
        fp4_ms, fp4_gbs = fp4_full_decode(device)
        fp4_ceiling = max(best["fp4_mix_22to78"], best["fp4_shape_20to80"])
        extra.update(fp4_g16_full_decode_ms=round(fp4_ms, 3), fp4_g16_full_decode_gbs=round(fp4_gbs, 1),
                     fp4_g16_full_decode_frac=round(fp4_gbs / HBM_PEAK_GBS, 4),
                     fp4_g16_frac_of_copy=round(fp4_gbs / copy_gbs, 4),
                     fp4_g16_frac_of_mix_ceiling=round(fp4_gbs / fp4_ceiling, 4))
    extra["other_codecs_b64"] = other_codecs(device)
    extra["prefill_b1_2048"] = prefill_timing(device)
    extra["checkpoint_loader"] = loader_bench(device)
    if not args.skip_e2e:
        extra["e2e_decode"] = e2e_decode(device, batches=(1, 16))
    line = dict(
        metric=METRIC, value=round(gbs, 2), unit="GB/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(ms, 5), higher_is_better=True, scaling="weak", vs_baseline=None, dtype="f32",
        data="synthetic",
        config=dict(workload="56-layer ridge-latent state step + per-token requant (BASELINE config 4, one token)",
                    batch=args.batch, layers=56, heads=H, headdim=P, d_state=NSTATE, groups=G,
                    layouts="published per-layer (wt2_test_v1)", launch="HIP graph of 56 per-layer kernels",
                    algorithmic_bytes_per_step=nbytes),
        roofline=dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                      frac=round(achieved / HBM_PEAK_GBS, 4), traffic=measured_traffic(),
                      kernel="k_state_step (ridge)", avg_launch_us=round(kern_us, 3),
                      algorithmic_bytes_per_launch=round(per_launch)),
        extra=extra)
    if not args.skip_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
