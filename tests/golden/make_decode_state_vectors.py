"""Writes tests/golden/decode_state_vectors.npz: packed states, tables and
the FP32 output of the reference's diagnostic decoders, run on the CPU in
this container from the reference checkout:
  mamba2_recall/state_codec.py:269-296        decode_state (sq3p25), packed
                                              order and with a permutation
  mamba2_recall/state_codec_dense3.py:189-212 decode_state (dense3), no table,
                                              permutation and equalizer tables
The fixture is data only.  Usage: python make_decode_state_vectors.py
[reference root]."""
import importlib.util
import sys

# importing the reference by path must never write bytecode into its checkout
sys.dont_write_bytecode = True
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
B, H, P, G = 1, 4, 16, 2


def load(root, rel, name):
    spec = importlib.util.spec_from_file_location(name, Path(root) / rel)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod   # dataclasses resolve annotations through the module
    spec.loader.exec_module(mod)
    return mod


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sc = load(root, "mamba2_recall/state_codec.py", "ref_state_codec")
    d3 = load(root, "mamba2_recall/state_codec_dense3.py", "ref_state_codec_dense3")
    rng = np.random.default_rng(4242)
    gen = torch.Generator().manual_seed(4242)
    out = {}
    # sq3p25: every byte pattern is a valid carry; scales include subnormal
    # binary16 values, signed zeros and negatives
    st = sc.allocate_state(B, H, P, 128, "sq3p25", "cpu")
    for k, n in (("lo", 8), ("hi", 8), ("q4", 32)):
        st.tensors[k].copy_(torch.randint(0, 256, (B, H, P, n), generator=gen, dtype=torch.uint8))
    s = np.exp(rng.normal(-4.0, 2.0, size=(2, B, H, P))).astype(np.float16)
    s.reshape(2, -1)[:, :4] = np.array([0.0, -0.0, 6e-8, -0.5], np.float16)
    st.tensors["s8"].copy_(torch.from_numpy(s[0]))
    st.tensors["s4"].copy_(torch.from_numpy(s[1]))
    perm = torch.stack([torch.randperm(128, generator=gen) for _ in range(G)]).to(torch.uint8)
    for k in ("lo", "hi", "q4"):
        out[f"sq_{k}"] = st.tensors[k].numpy()
    out["sq_s8"] = st.tensors["s8"].numpy().view(np.uint16)
    out["sq_s4"] = st.tensors["s4"].numpy().view(np.uint16)
    out["perm"] = perm.numpy()
    out["sq_decode"] = sc.decode_state(st).numpy()
    out["sq_decode_perm"] = sc.decode_state(st, perm).numpy()
    # dense3
    ds = d3.allocate_state(B, H, P, 128, "cpu")
    ds.tensors["codes"].copy_(torch.randint(0, 256, (B, H, P, 3, 16), generator=gen, dtype=torch.uint8))
    sd = np.exp(rng.normal(-3.0, 1.5, size=(B, H, P, 2))).astype(np.float16)
    sd.reshape(-1)[:3] = np.array([0.0, -0.0, 6e-8], np.float16)
    ds.tensors["scales"].copy_(torch.from_numpy(sd))
    eq = torch.randint(-8, 9, (G, 128), generator=gen, dtype=torch.int8)
    out["d3_codes"] = ds.tensors["codes"].numpy()
    out["d3_scales"] = ds.tensors["scales"].numpy().view(np.uint16)
    out["d3_equalizer"] = eq.numpy()
    out["d3_decode"] = d3.decode_state(ds).numpy()
    out["d3_decode_perm"] = d3.decode_state(ds, perm, "permutation").numpy()
    out["d3_decode_eq"] = d3.decode_state(ds, eq, "equalizer").numpy()
    np.savez_compressed(HERE / "decode_state_vectors.npz", **out)
    print("wrote", HERE / "decode_state_vectors.npz", sorted(out))


if __name__ == "__main__":
    main()
