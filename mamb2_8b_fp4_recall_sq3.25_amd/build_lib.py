"""Build the gfx950 HIP library `lib/libm2r_hip.so` from `csrc/*.hip`.

Every translation unit is compiled with binary32 contraction disabled
(-ffp-contract=off: the codec's bit-exactness relies on separately rounded
products and sums), IEEE denormals kept, and packed-FP32 instruction
selection disabled.  The packed-row and dense3 step kernels (m2r_state.hip,
the instrumented copy that includes it, m2r_dense3.hip) are scheduled for
instruction-level parallelism (SOURCE_FLAGS).  Objects are compiled in
parallel, then linked.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB_DIR = HERE / "lib"
LIB = LIB_DIR / "libm2r_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-source additions.  The packed-row and dense3 step kernels are VALU-bound
# or latency-bound chains with the instruction order pinned where it matters;
# the max-ILP machine scheduler measured 1.3-1.8% faster per launch at batch 4
# to 64, 3% on the 2048-token prefill (batch 16 within 0.2%) and, with the
# tier loops' scheduling barriers dropped, a further 1.3% at batch 64 and
# 2.4% for dense3, while the FP4 decode, the GEMV, the s16 step (its own
# translation unit for that reason) and the multi-layer kernel were 4-19%
# slower with it.
SCHED_ILP_FLAGS = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
SOURCE_FLAGS = {"m2r_state.hip": SCHED_ILP_FLAGS, "m2r_timeline.hip": SCHED_ILP_FLAGS,
                "m2r_dense3.hip": SCHED_ILP_FLAGS}


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, obj: Path):
    cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    return obj


def build(verbose: bool = False) -> Path:
    LIB_DIR.mkdir(exist_ok=True)
    objdir = LIB_DIR / "obj"
    objdir.mkdir(exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(lambda s: _compile(s, objdir / (s.stem + ".o")), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
