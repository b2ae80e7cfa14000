"""Packed FP4 G16 checkpoint reader: drop-in for the load side of the
reference's mamba2_recall/fp4_checkpoint.py.

On-disk format (kept byte-identical so checkpoints written by the reference
load here): safetensors-layout shards whose header is a deterministic
function of the tensor plan.  Each FP4 matrix is split by rows into parts;
a part holds `codes` U8[rows, cols/2] (low nibble = even column) and
`block_scale_bytes` U8[rows, cols/16] (E4M3FN bytes); the first part also
holds the whole-matrix `global_scale` F32[].  Retained FP16 tensors live in
`weights-retained-fp16.safetensors`.

Decode path (MI355X): each part is read from the file straight into pinned
host memory, copied to the device asynchronously, and decoded by the gfx950
kernel directly into its rows of the resident FP16 destination.  Validity is
accumulated in a device word and checked once per tensor; hashing the decoded
FP16 bytes (the reference's per-chunk device-to-host hash) is optional.

Verification helpers (`read_ledger`, `make_plan`, `inspect_shard`,
`verify_checkpoint`) use only the standard library.
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import struct
from pathlib import Path

FORMAT = "MAMBA2_FP4_G16_PACKED_CHECKPOINT_V1"
# identities of the audited production conversion (fp4_checkpoint.py:17-21)
LEDGER_SHA = "55de4189a7e04c9564a48b0fbb5f37428d3d1bb5b6274831d878b41ef4686c9b"
SOURCE_SHA = "47c2766f6aad89d73beafbeaecb334aab902d7370906d081764a90bb7a8bbbcb"
PAYLOAD_BYTES = 4_638_460_360
WEIGHT_BYTES = 16_473_999_360
DTYPE_BYTES = {"U8": 1, "F16": 2, "F32": 4}
MAX_HEADER_BYTES = 8 * 1024 * 1024
RETAINED_FILE = "weights-retained-fp16.safetensors"
READ_BLOCK = 8 * 1024 * 1024


def need(condition, message):
    if not condition:
        raise ValueError(message)


def sha_file(path):
    h = hashlib.sha256()
    with Path(path).open("rb") as f:
        while True:
            block = f.read(READ_BLOCK)
            if not block:
                return h.hexdigest()
            h.update(block)


def read_json(path):
    return json.loads(Path(path).read_text())


def write_json(path, value):
    """Creates `path` (never overwrites), sorted keys, no NaN."""
    with Path(path).open("x") as f:
        f.write(json.dumps(value, sort_keys=True, indent=2, allow_nan=False) + "\n")


def read_ledger(path):
    """fp4_checkpoint.py:54-63: the pinned conversion ledger."""
    need(sha_file(path) == LEDGER_SHA, "The exact audited FP4 G16 ledger is required")
    ledger = read_json(path)
    need(ledger["complete"] is True and ledger["format_name"] == "fp4_g16_e4m3"
         and ledger["source_checkpoint_sha256"] == SOURCE_SHA
         and ledger["tensor_count"] == 507 and ledger["fp4_tensor_count"] == 114
         and ledger["parameter_count"] == 8_236_999_680
         and ledger["logical_encoded_payload_bytes"] == PAYLOAD_BYTES,
         "Pinned conversion ledger has unexpected production geometry")
    return ledger


def _rows_per_part(columns, shard_limit_bytes):
    """Largest row count of an FP4 part under the shard limit (4 bytes kept
    for the global scale), rounded down to the 512-row quantization chunks
    when at least one chunk fits."""
    per_row = columns // 2 + columns // 16
    rows = max(1, (shard_limit_bytes - 4) // per_row)
    return rows - rows % 512 if rows >= 512 else rows


def make_plan(ledger, shard_limit_bytes):
    """fp4_checkpoint.py:66-92: deterministic tensor -> shard plan."""
    need(type(shard_limit_bytes) is int and shard_limit_bytes >= 1024 * 1024,
         "Shard limit must be an integer of at least one MiB")
    plan, matrix = {}, 0
    for name in sorted(ledger["tensors"]):
        item = ledger["tensors"][name]
        if item["kind"] == "fp16":
            plan[name] = {"kind": "fp16", "shape": item["shape"], "file": RETAINED_FILE, "key": name}
            continue
        need(item["kind"] == "fp4_g16_e4m3" and len(item["shape"]) == 2, "Unexpected quantized matrix kind/shape")
        rows, columns = item["shape"]
        need(columns % 16 == 0, "Production FP4 width is not divisible by 16")
        step = _rows_per_part(columns, shard_limit_bytes)
        matrix += 1
        parts = [{"file": f"weights-fp4-{matrix:03d}-part-{k + 1:03d}.safetensors", "row_start": start,
                  "row_stop": min(rows, start + step)} for k, start in enumerate(range(0, rows, step))]
        plan[name] = {"kind": "fp4_g16_e4m3", "shape": item["shape"], "parts": parts,
                      "global_scale_file": parts[0]["file"]}
    return plan


def _file_specs(plan):
    """fp4_checkpoint.py:100-114: tensors of every shard file."""
    specs = {RETAINED_FILE: {}}
    for name, item in plan.items():
        if item["kind"] == "fp16":
            specs[item["file"]][name] = {"dtype": "F16", "shape": item["shape"]}
            continue
        columns = item["shape"][1]
        for k, part in enumerate(item["parts"]):
            rows = part["row_stop"] - part["row_start"]
            spec = {"codes": {"dtype": "U8", "shape": [rows, columns // 2]},
                    "block_scale_bytes": {"dtype": "U8", "shape": [rows, columns // 16]}}
            if k == 0:
                spec["global_scale"] = {"dtype": "F32", "shape": []}
            specs[part["file"]] = spec
    return specs


def _header(spec):
    """Deterministic safetensors header of one shard: tensors in name order,
    packed back to back; compact JSON padded with spaces to 8 bytes.
    Returns (raw header bytes, parsed header, payload bytes)."""
    header = {"__metadata__": {"format": FORMAT, "scale_bytes": "float8_e4m3fn"}}
    offset = 0
    for name in sorted(spec):
        item = spec[name]
        size = math.prod(item["shape"]) * DTYPE_BYTES[item["dtype"]]
        header[name] = dict(item, data_offsets=[offset, offset + size])
        offset += size
    raw = json.dumps(header, separators=(",", ":"), allow_nan=False).encode()
    raw += b" " * (-len(raw) % 8)
    return raw, header, offset


def _create_shard(path, spec):
    """Writes the header of a new shard and sizes its payload (zero bytes).
    Returns (payload base offset, parsed header)."""
    raw, header, payload = _header(spec)
    with Path(path).open("xb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        f.truncate(8 + len(raw) + payload)
    return 8 + len(raw), header


def _no_duplicates(pairs):
    out = {}
    for key, value in pairs:
        need(key not in out, "Duplicate safetensors header entry")
        out[key] = value
    return out


def inspect_shard(path, expected_spec):
    """fp4_checkpoint.py:147-164: the shard's header must equal the plan's
    deterministic header byte for byte and its size must be exact.
    Returns (payload base offset, parsed header)."""
    path = Path(path)
    need(path.is_file() and not path.is_symlink(), "Expected regular safetensors shard")
    with path.open("rb") as f:
        prefix = f.read(8)
        need(len(prefix) == 8, "Truncated safetensors header prefix")
        size = struct.unpack("<Q", prefix)[0]
        need(2 <= size <= MAX_HEADER_BYTES and size % 8 == 0, "Invalid safetensors header size/alignment")
        raw = f.read(size)
        need(len(raw) == size, "Truncated safetensors header")
    parsed = json.loads(raw, object_pairs_hook=_no_duplicates)
    want_raw, want_header, payload = _header(expected_spec)
    need(parsed == want_header and raw == want_raw, "Shard tensor inventory/header differs from deterministic plan")
    need(path.stat().st_size == 8 + size + payload, "Shard is truncated or has extra bytes")
    return 8 + size, parsed


def _hash_region(path, start, size, digest):
    with Path(path).open("rb") as f:
        f.seek(start)
        left = size
        while left:
            block = f.read(min(READ_BLOCK, left))
            need(block, "Truncated payload region")
            digest.update(block)
            left -= len(block)


def _region_sha(path, base, header, key):
    begin, end = header[key]["data_offsets"]
    h = hashlib.sha256()
    _hash_region(path, base + begin, end - begin, h)
    return h


def verify_checkpoint(directory, code_root=None):
    """fp4_checkpoint.py:178-238: container, manifest and exact encoded bytes,
    without torch.  `code_root`, when given, also checks the manifest's
    runtime-source hashes against files under it; those hashes pin the
    reference's own Python sources, which this package replaces, so the check
    is opt-in here."""
    directory = Path(directory)
    need(directory.is_dir() and not directory.is_symlink(), "Regular checkpoint directory required")
    manifest = read_json(directory / "weight_manifest.json")
    need(manifest["format"] == FORMAT and manifest["complete"] is True, "Not a complete FP4 G16 checkpoint")
    ledger = read_ledger(directory / "conversion_receipt.json")
    plan = make_plan(ledger, manifest["shard_limit_bytes"])
    need(manifest["layout"] == plan and manifest["logical_weight_payload_bytes"] == PAYLOAD_BYTES
         and manifest["decoded_resident_weight_bytes"] == WEIGHT_BYTES
         and manifest["source_checkpoint_sha256"] == SOURCE_SHA
         and manifest["conversion_receipt_sha256"] == LEDGER_SHA,
         "Manifest differs from pinned checkpoint identities")
    if code_root is not None:
        code_root = Path(code_root)
        for name, digest in manifest["code_sha256"].items():
            need(sha_file(code_root / name) == digest, "Checkpoint runtime source differs: " + name)
        for name, digest in ledger["code_sha256"].items():
            need(sha_file(code_root / name) == digest, "Original measured FP4 source differs: " + name)
    specs = _file_specs(plan)
    need(set(manifest["files"]) == set(specs), "Manifest shard inventory differs")
    headers, file_sha = {}, {}
    for filename in sorted(specs):
        path = directory / filename
        headers[filename] = inspect_shard(path, specs[filename])
        file_sha[filename] = sha_file(path)
        need(manifest["files"][filename] == {"sha256": file_sha[filename], "bytes": path.stat().st_size},
             "Shard file identity differs: " + filename)
    need(manifest["shard_file_bytes"] == sum((directory / f).stat().st_size for f in specs)
         and manifest["format_name"] == "fp4_g16_e4m3"
         and manifest["packed_resident_kernel"] is False and manifest["custom_runtime"] is True,
         "Stored size/runtime claims differ from actual package")
    for name, item in plan.items():
        want = ledger["tensors"][name]
        if item["kind"] == "fp16":
            base, header = headers[item["file"]]
            need(_region_sha(directory / item["file"], base, header, name).hexdigest() == want["decoded_sha256"],
                 "Retained FP16 tensor differs: " + name)
            continue
        for key, hash_key in (("codes", "codes_sha256"), ("block_scale_bytes", "scales_sha256")):
            h = hashlib.sha256()
            for part in item["parts"]:
                base, header = headers[part["file"]]
                begin, end = header[key]["data_offsets"]
                _hash_region(directory / part["file"], base + begin, end - begin, h)
            need(h.hexdigest() == want[hash_key], "Packed tensor bytes differ: " + name + "/" + key)
        base, header = headers[item["global_scale_file"]]
        need(_region_sha(directory / item["global_scale_file"], base, header, "global_scale").hexdigest()
             == want["global_scale_sha256"], "Tensor global scale differs: " + name)
    inventory = set(specs) | {"conversion_receipt.json", "weight_manifest.json", "SHA256SUMS"}
    need(not any(p.is_symlink() for p in directory.rglob("*")), "Checkpoint contains symlink")
    need({str(p.relative_to(directory)) for p in directory.rglob("*") if p.is_file()} == inventory,
         "Unexpected files in checkpoint directory")
    for name in ("conversion_receipt.json", "weight_manifest.json"):
        file_sha[name] = sha_file(directory / name)
    sums = "".join(f"{file_sha[n]}  {n}\n" for n in sorted(inventory - {"SHA256SUMS"}))
    need((directory / "SHA256SUMS").read_text() == sums, "Checkpoint checksum list differs")
    return manifest, ledger


def export_checkpoint(*args, **kwargs):
    """The encoder side (fp4.quantize_chunk and the export recipe) is not part
    of this package; checkpoints are written by the reference."""
    raise NotImplementedError("export_checkpoint: the FP4 encoder is not part of this package")


# ---------------------------------------------------------------------------
# Device loading


class _PinnedReader:
    """Reads file regions into pinned host buffers, reusing a buffer only
    after the host-to-device copy that read it has completed.  Regions of at
    least SMALL bytes (the code bytes of a part) and smaller ones (its block
    scales, the global scales) take turns in separate pairs of buffers, so
    the read of the next part's codes overlaps the copy of this part's.  A
    region of at least two CHUNK-sized pieces is read by a few threads at
    once, each with positioned reads into its own piece of the buffer (the
    reads release the interpreter lock)."""

    CHUNK = 1 << 20
    WORKERS = 8
    SMALL = 1 << 20

    def __init__(self, torch, device, slots=2):
        self.torch, self.device = torch, device
        # per size class: [pinned buffer, copy-done event] slots and the next turn
        self.slots = {big: [[None, None] for _ in range(slots)] for big in (False, True)}
        self.turn = {False: 0, True: 0}
        self.pool = None

    def _read(self, path, position, buf):
        """Reads len(buf) bytes at `position` of `path` into the writable
        memoryview `buf`; returns the number of bytes read (short only at
        the end of the file)."""
        count = len(buf)
        fd = os.open(path, os.O_RDONLY)
        try:
            def piece(span):
                begin, end = span
                at = begin
                while at < end:
                    got = os.preadv(fd, [buf[at:end]], position + at)
                    if got <= 0:
                        break
                    at += got
                return at - begin

            if count < 2 * self.CHUNK:
                return piece((0, count))
            step = max(self.CHUNK, -(-count // self.WORKERS))
            spans = [(a, min(a + step, count)) for a in range(0, count, step)]
            if self.pool is None:
                from concurrent.futures import ThreadPoolExecutor
                self.pool = ThreadPoolExecutor(max_workers=self.WORKERS)
            return sum(self.pool.map(piece, spans))
        finally:
            os.close(fd)

    def to_device(self, path, position, count, dest):
        """Copies `count` file bytes at `position` into the uint8 device tensor
        `dest` (asynchronously, on the current stream)."""
        torch = self.torch
        big = count >= self.SMALL
        slots = self.slots[big]
        slot = slots[self.turn[big]]
        self.turn[big] = (self.turn[big] + 1) % len(slots)
        if slot[1] is not None:
            slot[1].synchronize()
        if slot[0] is None or slot[0].numel() < count:
            slot[0] = torch.empty(max(count, 1 << 20), dtype=torch.uint8, pin_memory=True)
        view = slot[0][:count]
        got = self._read(Path(path), position, memoryview(view.numpy()))
        need(got == count, "Truncated checkpoint data")
        dest.copy_(view, non_blocking=True)
        slot[1] = torch.cuda.Event()
        slot[1].record()


def load_packed_tensors(directory, plan, *, device="cuda", hash_decoded=False, progress=None):
    """Decodes every tensor of `plan` from the shards in `directory` into
    resident FP16 device tensors.  Returns {name: tensor} and, if
    `hash_decoded`, {name: sha256 hex of the decoded FP16 bytes}.  Shard
    headers are checked against the plan (inspect_shard) before any read.
    The decode's error words are read once, after every matrix is queued
    (a read per matrix would drain the copy pipeline each time); the error
    raised is that of the first failing matrix in plan order, as a check
    after each matrix would raise it."""
    import torch

    from . import fp4
    directory = Path(directory)
    device = torch.device(device)
    headers = {f: inspect_shard(directory / f, spec) for f, spec in _file_specs(plan).items()}
    reader = _PinnedReader(torch, device)
    tensors, hashes = {}, {}
    with torch.cuda.device(device):
        flags = torch.zeros(max(len(plan), 1), dtype=torch.int32, device=device)   # per matrix, plan order
        for ordinal, name in enumerate(sorted(plan), 1):
            item = plan[name]
            shape = item["shape"]
            out = torch.empty(shape, dtype=torch.float16, device=device)
            if item["kind"] == "fp16":
                base, header = headers[item["file"]]
                begin, end = header[name]["data_offsets"]
                reader.to_device(directory / item["file"], base + begin, end - begin, out.view(-1).view(torch.uint8))
            else:
                need(item["kind"] == "fp4_g16_e4m3", "Unexpected quantized matrix kind/shape")
                rows, columns = shape
                base, header = headers[item["global_scale_file"]]
                global_scale = torch.empty(1, dtype=torch.float32, device=device)
                reader.to_device(directory / item["global_scale_file"],
                                 base + header["global_scale"]["data_offsets"][0], 4, global_scale.view(torch.uint8))
                flag = flags[ordinal - 1:ordinal]
                for part in item["parts"]:
                    base, header = headers[part["file"]]
                    r0, r1 = part["row_start"], part["row_stop"]
                    n = r1 - r0
                    codes = torch.empty((n, columns // 2), dtype=torch.uint8, device=device)
                    scales = torch.empty((n, columns // 16), dtype=torch.uint8, device=device)
                    reader.to_device(directory / part["file"], base + header["codes"]["data_offsets"][0],
                                     codes.numel(), codes.view(-1))
                    reader.to_device(directory / part["file"], base + header["block_scale_bytes"]["data_offsets"][0],
                                     scales.numel(), scales.view(-1))
                    fp4.decode_into(codes, scales, global_scale, out[r0:r1], rows=n, columns=columns, group=16,
                                    err_flag=flag)
            if hash_decoded:
                h = hashlib.sha256()
                flat = out.view(-1)
                step = fp4.MAX_CHUNK_ELEMENTS
                for start in range(0, flat.numel(), step):
                    h.update(flat[start:start + step].cpu().numpy().tobytes())
                hashes[name] = h.hexdigest()
            tensors[name] = out
            if progress:
                progress({"tensor": name, "index": ordinal, "total": len(plan)})
        for err in flags.cpu().tolist():   # synchronizes with every decode
            fp4.raise_decode_errors(err)
    torch.cuda.synchronize(device)
    return (tensors, hashes) if hash_decoded else tensors


def load_packed_model(directory, *, device="cuda", chunk_rows=512, progress=None, model=None, hash_decoded=True,
                      code_root=None):
    """fp4_checkpoint.py:345-405: verify the checkpoint, decode every tensor
    to resident FP16 on `device` and install it into `model` (by default the
    reference runtime's model built on the meta device, which needs its
    mamba_ssm dependency).  With `hash_decoded` the decoded bytes are hashed
    against the ledger as the reference does."""
    import torch
    from torch import nn
    need(chunk_rows == 512, "Production reload decodes in the measured 512-row chunks")
    manifest, ledger = verify_checkpoint(directory, code_root)
    if model is None:
        try:
            from . import runtime  # noqa: F401  (the reference's model builder)
        except ImportError as exc:
            raise ImportError("load_packed_model needs a model: pass model=... (the reference runtime "
                              "and its mamba_ssm dependency are not part of this package)") from exc
        model = runtime.make_model(device="meta", dtype=torch.float16)
    plan = manifest["layout"]
    expected = {name: list(t.shape) for name, t in model.state_dict().items()}
    need(expected == {name: item["shape"] for name, item in plan.items()}, "Native model geometry differs")
    loaded = load_packed_tensors(directory, plan, device=device, hash_decoded=hash_decoded, progress=progress)
    tensors, hashes = loaded if hash_decoded else (loaded, {})
    for name in sorted(plan):
        if hash_decoded:
            need(hashes[name] == ledger["tensors"][name]["decoded_sha256"], "Reloaded decoded hash differs: " + name)
        module_name, local = name.rsplit(".", 1)
        module = model.get_submodule(module_name)
        if local in module._parameters:
            setattr(module, local, nn.Parameter(tensors[name], requires_grad=False))
        elif local in module._buffers:
            module._buffers[local] = tensors[name]
        else:
            raise ValueError("Unknown native tensor: " + name)
    need(not any(t.is_meta for t in model.state_dict().values()), "Incomplete packed checkpoint reload")
    need(model.backbone.embedding.weight.data_ptr() != model.lm_head.weight.data_ptr(), "Unexpected tied embeddings")
    model._fp4_receipt = dict(ledger, serialization="safetensors_packed_checkpoint",
                              source_checkpoint_required=False,
                              packed_checkpoint_manifest_sha256=sha_file(Path(directory) / "weight_manifest.json"))
    return model.eval().requires_grad_(False)
