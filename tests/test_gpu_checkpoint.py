"""GPU check of the packed-checkpoint loader: synthetic shards in the
reference's container format decode on the device bit-exactly to the CPU
oracle, including a matrix split over several parts."""
import hashlib

import numpy as np
import pytest
import torch

import test_gpu_fp4 as fp4t

pytestmark = pytest.mark.gpu


def write_region(path, base, header, key, data):
    begin, end = header[key]["data_offsets"]
    assert end - begin == len(data)
    with open(path, "r+b") as f:
        f.seek(base + begin)
        f.write(data)


def test_load_packed_tensors_matches_oracle(oracle, device, tmp_path):
    from mamba2_recall import fp4_checkpoint as ck
    ledger = {"tensors": {"a.in_proj.weight": {"kind": "fp4_g16_e4m3", "shape": [1000, 4096]},
                          "a.out_proj.weight": {"kind": "fp4_g16_e4m3", "shape": [64, 512]},
                          "a.D": {"kind": "fp16", "shape": [128]},
                          "a.conv1d.weight": {"kind": "fp16", "shape": [40, 1, 4]}}}
    plan = ck.make_plan(ledger, 1 << 20)
    assert len(plan["a.in_proj.weight"]["parts"]) == 3
    specs = ck._file_specs(plan)
    headers = {f: ck._create_shard(tmp_path / f, s) for f, s in specs.items()}
    rng = np.random.default_rng(5)
    want = {}
    for name, item in sorted(plan.items()):
        if item["kind"] == "fp16":
            v = rng.normal(size=item["shape"]).astype(np.float16)
            base, header = headers[item["file"]]
            write_region(tmp_path / item["file"], base, header, name, v.tobytes())
            want[name] = v.view(np.uint16)
            continue
        rows, cols = item["shape"]
        packed, sb, g = fp4t.g16_packet(rng, rows, cols, device)
        ref, err = oracle.fp4_decode(16, packed, sb, g, rows, cols)
        assert err == 0
        want[name] = ref
        base, header = headers[item["global_scale_file"]]
        write_region(tmp_path / item["global_scale_file"], base, header, "global_scale",
                     np.float32(g).tobytes())
        for part in item["parts"]:
            base, header = headers[part["file"]]
            r0, r1 = part["row_start"], part["row_stop"]
            write_region(tmp_path / part["file"], base, header, "codes", packed[r0:r1].tobytes())
            write_region(tmp_path / part["file"], base, header, "block_scale_bytes", sb[r0:r1].tobytes())
    print("[checkpoint] synthetic shards written", flush=True)
    tensors, hashes = ck.load_packed_tensors(tmp_path, plan, device=device, hash_decoded=True)
    for name in plan:
        got = tensors[name].cpu().numpy().view(np.uint16).reshape(want[name].shape)
        assert int((got != want[name]).sum()) == 0, name
        assert hashes[name] == hashlib.sha256(want[name].tobytes()).hexdigest()


def test_loader_raises_reference_error_for_bad_scale(oracle, device, tmp_path):
    from mamba2_recall import fp4_checkpoint as ck
    plan = ck.make_plan({"tensors": {"w": {"kind": "fp4_g16_e4m3", "shape": [8, 32]}}}, 1 << 20)
    specs = ck._file_specs(plan)
    headers = {f: ck._create_shard(tmp_path / f, s) for f, s in specs.items()}
    part = plan["w"]["parts"][0]
    base, header = headers[part["file"]]
    write_region(tmp_path / part["file"], base, header, "global_scale", np.float32(0.5).tobytes())
    write_region(tmp_path / part["file"], base, header, "codes", bytes([0x11] * 128))
    scales = bytearray([0x38] * 16)
    scales[5] = 0x7F                       # E4M3 NaN
    write_region(tmp_path / part["file"], base, header, "block_scale_bytes", bytes(scales))
    with pytest.raises(ValueError, match="Invalid stored scale"):
        ck.load_packed_tensors(tmp_path, plan, device=device)


@pytest.mark.parametrize("first_bad", ["scale", "global"])
def test_loader_raises_first_failing_matrix_in_plan_order(device, tmp_path, first_bad):
    """Two failing matrices with different errors: the error raised is the
    first one's in plan order (the error words are read after every
    matrix is queued, not after each)."""
    from mamba2_recall import fp4_checkpoint as ck
    plan = ck.make_plan({"tensors": {name: {"kind": "fp4_g16_e4m3", "shape": [8, 32]} for name in ("w0", "w1")}},
                        1 << 20)
    specs = ck._file_specs(plan)
    headers = {f: ck._create_shard(tmp_path / f, s) for f, s in specs.items()}
    kinds = {"w0": first_bad, "w1": "global" if first_bad == "scale" else "scale"}
    for name, kind in kinds.items():
        part = plan[name]["parts"][0]
        base, header = headers[part["file"]]
        scales = bytearray([0x38] * 16)
        if kind == "scale":
            scales[3] = 0x7F                   # E4M3 NaN block scale
        write_region(tmp_path / part["file"], base, header, "global_scale",
                     np.float32(-1.0 if kind == "global" else 0.5).tobytes())
        write_region(tmp_path / part["file"], base, header, "codes", bytes([0x11] * 128))
        write_region(tmp_path / part["file"], base, header, "block_scale_bytes", bytes(scales))
    want = "Invalid stored scale" if first_bad == "scale" else "Global scale must be finite and positive"
    with pytest.raises(ValueError, match=want):
        ck.load_packed_tensors(tmp_path, plan, device=device)
