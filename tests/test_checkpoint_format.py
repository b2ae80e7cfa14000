"""CPU checks of the packed-checkpoint container (no GPU needed).

Known answers from the reference: the full 8B plan's logical payload is
4,638,460,360 B (README.md:120, fp4.py:385-386) and the decoded resident
weights are 16,473,999,360 B (fp4_checkpoint.py:21), with 507 tensors of
which 114 are FP4 matrices (fp4_checkpoint.py:58-61)."""
import json
import struct

import pytest

from mamba2_recall import fp4_checkpoint as ck

LAYERS, D_MODEL, D_INNER, VOCAB = 56, 4096, 8192, 256000


def production_ledger():
    """Tensor inventory of the Mamba-2 8B model (kinds and shapes only)."""
    t = {}
    for i in range(LAYERS):
        p = f"backbone.layers.{i}."
        t[p + "mixer.in_proj.weight"] = {"kind": "fp4_g16_e4m3", "shape": [18560, D_MODEL]}
        t[p + "mixer.out_proj.weight"] = {"kind": "fp4_g16_e4m3", "shape": [D_MODEL, D_INNER]}
        for name, shape in (("mixer.A_log", [128]), ("mixer.D", [128]), ("mixer.dt_bias", [128]),
                            ("mixer.conv1d.weight", [10240, 1, 4]), ("mixer.conv1d.bias", [10240]),
                            ("mixer.norm.weight", [D_INNER]), ("norm.weight", [D_MODEL])):
            t[p + name] = {"kind": "fp16", "shape": shape}
    t["backbone.embedding.weight"] = {"kind": "fp4_g16_e4m3", "shape": [VOCAB, D_MODEL]}
    t["lm_head.weight"] = {"kind": "fp4_g16_e4m3", "shape": [VOCAB, D_MODEL]}
    t["backbone.norm_f.weight"] = {"kind": "fp16", "shape": [D_MODEL]}
    return {"tensors": t}


def payload(spec):
    return ck._header(spec)[2]


def test_production_plan_payload_and_counts():
    plan = ck.make_plan(production_ledger(), 256 * 1024 * 1024)
    assert len(plan) == 507
    assert sum(item["kind"] == "fp4_g16_e4m3" for item in plan.values()) == 114
    specs = ck._file_specs(plan)
    assert sum(payload(s) for s in specs.values()) == ck.PAYLOAD_BYTES
    decoded = sum(2 * __import__("math").prod(item["shape"]) for item in plan.values())
    assert decoded == ck.WEIGHT_BYTES


def test_part_rows_follow_512_row_chunks():
    plan = ck.make_plan(production_ledger(), 256 * 1024 * 1024)
    emb = plan["backbone.embedding.weight"]
    starts = [p["row_start"] for p in emb["parts"]]
    # 2304 B per row -> 116508 rows fit; rounded down to 227 * 512
    assert starts == [0, 116224, 232448] and emb["parts"][-1]["row_stop"] == VOCAB
    assert emb["global_scale_file"] == emb["parts"][0]["file"]
    small = ck.make_plan({"tensors": {"w": {"kind": "fp4_g16_e4m3", "shape": [1000, 4096]}}}, 1 << 20)
    assert [(p["row_start"], p["row_stop"]) for p in small["w"]["parts"]] == [(0, 455), (455, 910), (910, 1000)]


def test_plan_rejects_bad_geometry():
    with pytest.raises(ValueError, match="at least one MiB"):
        ck.make_plan(production_ledger(), 1000)
    with pytest.raises(ValueError, match="divisible by 16"):
        ck.make_plan({"tensors": {"w": {"kind": "fp4_g16_e4m3", "shape": [4, 40]}}}, 1 << 20)


def test_header_is_deterministic_and_aligned():
    spec = {"codes": {"dtype": "U8", "shape": [3, 8]}, "block_scale_bytes": {"dtype": "U8", "shape": [3, 1]},
            "global_scale": {"dtype": "F32", "shape": []}}
    raw, header, size = ck._header(spec)
    assert len(raw) % 8 == 0 and size == 24 + 3 + 4
    parsed = json.loads(raw)
    # tensors packed in name order: block_scale_bytes, codes, global_scale
    assert parsed["block_scale_bytes"]["data_offsets"] == [0, 3]
    assert parsed["codes"]["data_offsets"] == [3, 27]
    assert parsed["global_scale"]["data_offsets"] == [27, 31]
    assert parsed["__metadata__"] == {"format": ck.FORMAT, "scale_bytes": "float8_e4m3fn"}
    assert raw == ck._header(dict(reversed(list(spec.items()))))[0]


def test_inspect_round_trip_and_rejections(tmp_path):
    spec = {"x": {"dtype": "F16", "shape": [5, 3]}}
    base, header = ck._create_shard(tmp_path / "a.safetensors", spec)
    assert ck.inspect_shard(tmp_path / "a.safetensors", spec) == (base, header)
    # wrong inventory
    with pytest.raises(ValueError, match="differs from deterministic plan"):
        ck.inspect_shard(tmp_path / "a.safetensors", {"x": {"dtype": "F16", "shape": [5, 4]}})
    # extra byte
    with open(tmp_path / "a.safetensors", "ab") as f:
        f.write(b"\0")
    with pytest.raises(ValueError, match="truncated or has extra bytes"):
        ck.inspect_shard(tmp_path / "a.safetensors", spec)
    # duplicate header key
    raw = b'{"x":{"dtype":"F16","shape":[1],"data_offsets":[0,2]},"x":{"dtype":"F16","shape":[1],"data_offsets":[0,2]}}'
    raw += b" " * (-len(raw) % 8)
    (tmp_path / "d.safetensors").write_bytes(struct.pack("<Q", len(raw)) + raw + b"\0\0")
    with pytest.raises(ValueError, match="Duplicate safetensors header entry"):
        ck.inspect_shard(tmp_path / "d.safetensors", {"x": {"dtype": "F16", "shape": [1]}})
    # misaligned header size
    (tmp_path / "m.safetensors").write_bytes(struct.pack("<Q", 3) + b"{} ")
    with pytest.raises(ValueError, match="size/alignment"):
        ck.inspect_shard(tmp_path / "m.safetensors", {})


def test_verify_requires_pinned_ledger(tmp_path):
    (tmp_path / "weight_manifest.json").write_text(json.dumps({"format": ck.FORMAT, "complete": True}))
    (tmp_path / "conversion_receipt.json").write_text("{}")
    with pytest.raises(ValueError, match="exact audited FP4 G16 ledger"):
        ck.verify_checkpoint(tmp_path)


def test_export_is_not_part_of_this_package():
    with pytest.raises(NotImplementedError):
        ck.export_checkpoint()


def test_threaded_region_reads_match_the_file(tmp_path):
    """The loader's region reads: pieces read by several threads land in
    their places of the buffer, and a region past the end of the file comes
    back short (the loader then reports truncated data)."""
    import numpy as np
    data = np.random.default_rng(3).integers(0, 256, (1 << 20) + 77, dtype=np.uint8).tobytes()
    path = tmp_path / "region.bin"
    path.write_bytes(data)
    reader = ck._PinnedReader(None, None)
    reader.CHUNK = 1 << 14   # small pieces: every region below of 32 KiB or more is read by the pool
    for position, count in [(0, 0), (5, 100), (0, len(data)), (12345, (1 << 19) + 3), (len(data) - 40, 40)]:
        buf = bytearray(count)
        assert reader._read(path, position, memoryview(buf)) == count
        assert bytes(buf) == data[position:position + count]
    buf = bytearray(1 << 16)
    assert reader._read(path, len(data) - 1000, memoryview(buf)) == 1000
    assert bytes(buf[:1000]) == data[-1000:]
