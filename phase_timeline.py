"""Phase timeline of one state-step launch, from the instrumented build.

The library proper has no instrumentation.  With M2R_PHASE_TIMELINE defined,
every wave of the ridge step kernel stamps the shader clock at its phase
boundaries (m2r_step.h: ST_* stamps) and writes them to a device buffer.

  python phase_timeline.py build     compiles csrc/timeline/m2r_timeline.hip
                                     (the state-step sources with the flag) and
                                     links lib/libm2r_timeline.so (CPU, hipcc)
  python phase_timeline.py run [--out FILE]
                                     on the GPU: the 56 published layers at
                                     batch 1 and 64 (one token) and the batch-1
                                     2048-token prefill, each layer launched
                                     twice in a row with the stamps (the second
                                     launch kept), and prints (or writes) the
                                     per-phase medians

Times are µs from the wave's own start (the shader clock's rate is taken per
wave from the constant 100 MHz clock), medians over every wave of every
layer; the launch figure is the span from the first wave's start to the last
wave's end, per layer, from the 100 MHz clock (10 ns resolution).
"""
from __future__ import annotations

import argparse
import ctypes
import hashlib
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "mamb2_8b_fp4_recall_sq3.25_amd"
SRC = PKG / "csrc" / "timeline" / "m2r_timeline.hip"
LIB = PKG / "lib" / "libm2r_timeline.so"

# stamp indices (m2r_step.h, enum ST_*)
ST_START, ST_ARGS, ST_ISSUED, ST_SLOT0_ISSUED, ST_ACT, ST_TOKEN, ST_BARRIER, ST_BUILD, ST_SLOT = range(9)
ST_TL, ST_COPYOUT, ST_END, ST_REAL0, ST_REAL1 = 12, 24, 25, 30, 31
ST_TL_TOKEN = 100   # the prefill token whose phases are stamped (m2r_step.h)


def build():
    sys.path.insert(0, str(PKG))
    import build_lib
    objdir = build_lib.LIB_DIR / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    obj = objdir / "m2r_timeline.o"
    probe = objdir / "m2r_probe.o"   # the error-reporting helpers (and probes)
    build_lib._compile(SRC, obj)
    if not probe.exists():
        build_lib._compile(build_lib.CSRC / "m2r_probe.hip", probe)
    subprocess.run([build_lib.HIPCC, f"--offload-arch={build_lib.ARCH}", "-shared", "-fPIC", "-o", str(LIB),
                    str(obj), str(probe)], check=True)
    print(f"built {LIB}", flush=True)


def source_digest():
    h = hashlib.sha256()
    # the same files, in the same order, as the other step profiles' digest
    for name in ("csrc/m2r_state.hip", "csrc/m2r_step.h", "csrc/m2r_device.h", "csrc/m2r_tile.h", "build_lib.py"):
        h.update((PKG / name).read_bytes())
    return h.hexdigest()[:16]


def phase_rows(batch):
    """(label, stamp index) of the phases the instances at `batch` stamp."""
    rows = [("arguments loaded", ST_ARGS), ("token, statics and predictor transfers issued", ST_ISSUED),
            ("first slot's transfers issued", ST_SLOT0_ISSUED), ("dt activation done", ST_ACT),
            ("token inputs landed (own wave)", ST_TOKEN), ("workgroup barrier passed (every wave's inputs)", ST_BARRIER),
            ("token build and ridge correction done", ST_BUILD)]
    if batch == 64:   # four one-wave slots per wave
        for k in range(4):
            rows += [(f"slot {k}: data landed", ST_SLOT + 4 * k), (f"slot {k}: INT8 tier done", ST_SLOT + 4 * k + 1),
                     (f"slot {k}: INT4 tier done", ST_SLOT + 4 * k + 2), (f"slot {k}: done (y stored)", ST_SLOT + 4 * k + 3)]
    else:             # one slot on four waves
        rows += [("slot: data landed", ST_SLOT), ("slot: update half done", ST_SLOT + 1),
                 ("slot: maxima barrier passed", ST_SLOT + 2), ("slot: requantization half and y store done", ST_SLOT + 3)]
    rows += [("state copy-out issued", ST_COPYOUT), ("every store complete (wave end)", ST_END)]
    return rows


TL_ROWS = [("token values ready (record read, or token built)", ST_TL + 1), ("update half done", ST_TL + 2),
           ("maxima barrier passed", ST_TL + 3), ("requantization half and y store done", ST_TL + 4),
           ("token end (next record published)", ST_TL + 5)]


def run(out):
    import numpy as np
    import torch
    sys.path.insert(0, str(ROOT))
    sys.path.insert(0, str(PKG))
    import bench
    from mamba2_recall import _native
    if not LIB.exists():
        raise RuntimeError(f"{LIB} is missing: run `python phase_timeline.py build` first")
    lib = ctypes.CDLL(str(LIB))
    for name in ("m2r_state_step_ridge_ws", "m2r_ridge_records_bytes"):
        argt, rest = _native._SIGNATURES[name]
        getattr(lib, name).argtypes, getattr(lib, name).restype = argt, rest
    lib.m2r_timeline_set.argtypes, lib.m2r_timeline_set.restype = [ctypes.c_void_p], ctypes.c_int
    dev = torch.device("cuda:0")
    lines = [f"# phase timeline of the ridge step (instrumented build, kernel_source_sha16 {source_digest()} "
             "of csrc/{m2r_state.hip, m2r_step.h, m2r_device.h, m2r_tile.h} and build_lib.py)",
             "# command: python phase_timeline.py run --out <this file> (after `python phase_timeline.py build`)",
             "# µs from each wave's start, median [10th-90th percentile] over every wave of the 56 published",
             "# layers, each layer launched twice in a row and the second launch kept; each stamp costs a few",
             "# instructions and an LDS write, so the instrumented launch is slightly slower than the library's"]
    p = _native.ptr
    for batch, tokens in ((64, 1), (1, 1), (1, 2048)):
        print(f"[timeline] batch {batch} tokens {tokens}", flush=True)
        st = bench.RidgeStack(batch, dev, tokens=tokens)
        blocks = batch * 128 // 16 if batch == 64 else batch * 128   # (4,4) or four waves per head slot
        waves = blocks * 4
        buf = torch.zeros((56, waves * 32), dtype=torch.int64, device=dev)
        ws = None
        if tokens > 1:   # the token-record workspace, as bench.py's multi-token stack passes it
            ws = torch.empty(lib.m2r_ridge_records_bytes(batch, tokens, 8) // 4, dtype=torch.float32, device=dev)

        def launch(d, stream):
            t = d["state"].tensors
            rc = lib.m2r_state_step_ridge_ws(p(d["x"]), p(d["dt"]), p(d["A"]), p(d["B"]), p(d["C"]), p(d["D"]), 0,
                                             p(d["dt_bias"]), 0, p(d["perm"]), p(d["basis"]), p(d["lscale"]),
                                             p(d["pred"]), p(t["lo"]), p(t["hi"]), p(t["q4"]), p(t["latent"]),
                                             p(t["s8"]), p(t["s4"]), p(d["y"]), batch, tokens, 128, 64, 8, d["n8"],
                                             d["n4"], d["nz"], p(ws), 0 if ws is None else ws.numel() * 4, stream)
            assert rc == 0, rc

        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert lib.m2r_timeline_set(None) == 0
        for _ in range(3):
            for d in st.layers:
                launch(d, stream)
        torch.cuda.synchronize()
        # stamped pass: one layer at a time into its own buffer (the buffer's
        # address is a device symbol, set with the stream drained); of two
        # launches of a layer the second is kept
        for i, d in enumerate(st.layers):
            assert lib.m2r_timeline_set(ctypes.c_void_p(buf[i].data_ptr())) == 0
            launch(d, stream)
            launch(d, stream)
            torch.cuda.synchronize()
        assert lib.m2r_timeline_set(None) == 0
        s = buf.cpu().numpy().reshape(56, waves, 32).astype(np.int64)
        real = (s[:, :, ST_REAL1] - s[:, :, ST_REAL0]) / 100.0          # µs, 100 MHz clock
        ticks = s[:, :, ST_END] - s[:, :, ST_START]
        ghz = np.median(ticks / np.maximum(real, 1e-3)) / 1e3
        span = [(s[i, :, ST_REAL1].max() - s[i, :, ST_REAL0].min()) / 100.0 for i in range(56)]
        start_spread = [(s[i, :, ST_REAL0].max() - s[i, :, ST_REAL0].min()) / 100.0 for i in range(56)]
        what = "one token" if tokens == 1 else f"{tokens}-token prefill"
        lines += ["", f"## batch {batch}, {what}: {blocks} workgroups x 4 waves per launch; shader clock {ghz:.2f} GHz",
                  f"launch span (first wave start to last wave end), median over layers: {np.median(span):.2f} µs "
                  f"(min {np.min(span):.2f}, max {np.max(span):.2f}); wave start spread {np.median(start_spread):.2f} µs"]
        if tokens > 1:
            lines += [f"per token: {np.median(span) / tokens:.3f} µs (span / tokens); token {ST_TL_TOKEN}, µs from "
                      "that token's start on each wave:", f"{'phase':52s} {'median':>8s}  [p10 - p90] µs"]
            for label, idx in TL_ROWS:
                v = (s[:, :, idx] - s[:, :, ST_TL]) / (ghz * 1e3)
                v = v[(s[:, :, idx] != 0) & (s[:, :, ST_TL] != 0)]
                lines.append(f"{label:52s} {np.median(v):8.3f}  [{np.percentile(v, 10):.3f} - "
                             f"{np.percentile(v, 90):.3f}]")
            # per wave of the slot (wave w of a four-wave workgroup steps readout segment w)
            lines.append(f"by wave of the slot, medians (µs from the token's start): " +
                         ", ".join(label.split(" (")[0] for label, _ in TL_ROWS))
            for w in range(4):
                cells = []
                for _, idx in TL_ROWS:
                    v = (s[:, w::4, idx] - s[:, w::4, ST_TL]) / (ghz * 1e3)
                    cells.append(f"{np.median(v[(s[:, w::4, idx] != 0) & (s[:, w::4, ST_TL] != 0)]):.3f}")
                lines.append(f"  wave {w}: " + "  ".join(cells))
            del st, buf, ws
            torch.cuda.empty_cache()
            continue
        lines.append(f"{'phase':52s} {'median':>8s}  [p10 - p90] µs")
        for label, idx in phase_rows(batch):
            v = (s[:, :, idx] - s[:, :, ST_START]) / (ghz * 1e3)
            v = v[s[:, :, idx] != 0]
            lines.append(f"{label:52s} {np.median(v):8.2f}  [{np.percentile(v, 10):.2f} - {np.percentile(v, 90):.2f}]")
        del st, buf
        torch.cuda.empty_cache()
    text = "\n".join(lines) + "\n"
    print(text, flush=True)
    if out:
        Path(out).parent.mkdir(parents=True, exist_ok=True)
        Path(out).write_text(text)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("what", choices=("build", "run"))
    ap.add_argument("--out", default=None)
    args = ap.parse_args()
    build() if args.what == "build" else run(args.out)
