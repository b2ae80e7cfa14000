"""Writes tests/golden/encode_legacy_vectors.npz: input rows and the packed
sq3p25 output of the reference's diagnostic encoder
`mamba2_recall/state_codec.py:299-331` (encode_state_, FP32 denominators and
sign(z) * floor(|z| + 0.5) codes), run on the CPU in this container from the
reference checkout.  The fixture is data only (inputs and outputs); nothing
from the reference is copied.  Usage: python make_encode_legacy_vectors.py
[reference root]."""
import importlib.util
import sys

# importing the reference by path must never write bytecode into its checkout
sys.dont_write_bytecode = True
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def load_reference(root):
    spec = importlib.util.spec_from_file_location("ref_state_codec", Path(root) / "mamba2_recall" / "state_codec.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod   # dataclasses resolve annotations through the module
    spec.loader.exec_module(mod)
    return mod


def rows():
    """[2, 2, 64, 128] FP32 rows in packed coordinate order, covering:
    lognormal-scaled Gaussian rows; rows whose INT8 / INT4 tier maxima are
    127 / 7 exactly (scale 1) with codes at and one ulp either side of every
    half-integer; tiny rows (the 1e-8 scale floor); zero rows; signed zeros;
    rows with one dominant coordinate."""
    rng = np.random.default_rng(2026)
    v = np.zeros((256, 128), np.float32)
    v[:96] = rng.standard_normal((96, 128)) * np.exp(rng.normal(0.0, 0.5, (96, 1)))
    for i in range(96, 160):   # exact boundaries: tier maxima 127 and 7 give scale 1
        k = rng.integers(0, 127, 16).astype(np.float32) + 0.5
        k4 = rng.integers(0, 7, 64).astype(np.float32) + 0.5
        j = (i - 96) % 3
        step = {0: 0.0, 1: 1.0, 2: -1.0}[j]
        v8 = np.nextafter(k, k + step) if step else k
        v4 = np.nextafter(k4, k4 + step) if step else k4
        sgn8 = np.where(rng.random(16) < 0.5, -1, 1).astype(np.float32)
        sgn4 = np.where(rng.random(64) < 0.5, -1, 1).astype(np.float32)
        v[i, :16] = v8 * sgn8
        v[i, 16:80] = v4 * sgn4
        v[i, 0], v[i, 16] = 127.0, 7.0
        v[i, 80:] = rng.standard_normal(48)
    v[160:192] = rng.standard_normal((32, 128)) * 1e-9       # below the 1e-8 floor
    v[192:200] = 0.0
    v[200:208] = -0.0
    v[208:240] = rng.standard_normal((32, 128)) * 1e-3
    v[208:240, 3] = 50.0
    v[208:240, 40] = -3.0
    v[240:256] = rng.standard_normal((16, 128)) * 300.0      # large, within FP16 scales
    return v.reshape(2, 2, 64, 128)


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = load_reference(root)
    dense = torch.from_numpy(rows())
    state = ref.allocate_state(2, 2, 64, 128, "sq3p25", "cpu")
    ref.encode_state_(state, dense)
    out = {k: v.numpy() for k, v in state.tensors.items()}
    np.savez_compressed(HERE / "encode_legacy_vectors.npz", dense=dense.numpy(),
                        lo=out["lo"], hi=out["hi"], q4=out["q4"],
                        s8=out["s8"].view(np.uint16), s4=out["s4"].view(np.uint16))
    print("wrote", HERE / "encode_legacy_vectors.npz", {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
